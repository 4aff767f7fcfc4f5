// cbx_philox.h -- device Philox4x32-10 and the 53-bit uniform used for draws.
//
// Philox4x32-10 from Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3" (SC'11): per round two 32x32->64 multiplies
// (0xD2511F53 on x0, 0xCD9E8D57 on x2) feed a Feistel-like permutation; the
// two key words advance by the Weyl constants 0x9E3779B9 / 0xBB67AE85 between
// the ten rounds.  A draw is keyed (seed, stream, step): no state is carried,
// so any row of any step can be drawn independently on any lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbx {

struct U32x4 { uint32_t x0, x1, x2, x3; };

__device__ __forceinline__ U32x4 philox4x32_10(U32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        if (round) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint32_t lo0 = 0xD2511F53u * c.x0;
        const uint32_t hi0 = __umulhi(0xD2511F53u, c.x0);
        const uint32_t lo1 = 0xCD9E8D57u * c.x2;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c.x2);
        c = U32x4{hi1 ^ c.x1 ^ k0, lo1, hi0 ^ c.x3 ^ k1, lo0};
    }
    return c;
}

// Counter {step lo, step hi, stream lo, stream hi}, key {seed lo, seed hi};
// 27 + 26 random bits as in Matsumoto & Nishimura's genrand_res53, so u is a
// multiple of 2^-53 in [0, 1).
__device__ __forceinline__ double philox_uniform(uint64_t seed, uint64_t stream, uint64_t step) {
    const U32x4 o = philox4x32_10(
        U32x4{(uint32_t)step, (uint32_t)(step >> 32), (uint32_t)stream, (uint32_t)(stream >> 32)},
        (uint32_t)seed, (uint32_t)(seed >> 32));
    const double a = (double)(o.x0 >> 5), b = (double)(o.x1 >> 6);
    return (a * 67108864.0 + b) * (1.0 / 9007199254740992.0);
}

}  // namespace cbx
