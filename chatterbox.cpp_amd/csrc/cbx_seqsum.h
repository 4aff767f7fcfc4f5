// cbx_seqsum.h -- the exact binary32 value of a left-to-right running sum of
// non-negative terms, evaluated in parallel.
//
// The reference accumulates its top-p and softmax normalisers one float at a
// time (src/main.cpp:759, :763-768, :786-790); rounding makes the result
// depend on the order, so a tree sum does not reproduce it.  This file gives
// the same bits with a scan:
//
// While the running sum P stays inside one binade [2^b, 2^(b+1)), every
// partial sum is an integer multiple N*u of that binade's unit u = 2^(b-23),
// and adding a term t >= 0 gives, with y = t/u (exact: u is a power of two),
// f = floor(y), r = y - f:
//     r < 1/2:  N' = N + f        r > 1/2:  N' = N + f + 1
//     r = 1/2:  N' = whichever of N + f, N + f + 1 is even (ties to even).
// So a term acts on N only through N's parity: parity in -> (increment,
// parity out).  Such steps compose associatively -- a two-row table, one row
// per incoming parity -- and a scan over the tables gives every partial sum
// of the segment exactly.  A segment ends at the first term whose result
// reaches 2^(b+1) (tables are exact up to there, so that term is found
// exactly); its value is one ordinary binary32 add of the exact previous sum,
// and the next segment continues from it with the doubled unit.
//
// The per-term and composition rules below are shared by the device scan and
// the host tests.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define CBX_SEQ_HD __host__ __device__ __forceinline__
#else
#define CBX_SEQ_HD inline
#include <math.h>
#include <string.h>
#endif

namespace cbx {

// Increments saturate here: any partial sum this far past a binade's end is
// already past the segment, and saturation keeps the scan monotone.
constexpr int kSeqSat = 1 << 26;
// Values of y = t/u beyond this are clamped (they end the segment anyway).
constexpr float kSeqClamp = 33554432.0f;  // 2^25

// One term in a binade of unit 2^e: the increment without the tie bit, whether
// it is a tie, and the parity of floor(t/u).
struct SeqStep {
    int inc;
    int tie;
    int fodd;
};

// Composition of steps: for an incoming parity p (row p), the total increment
// d_p and the outgoing parity (bit p of q).
struct SeqTab {
    int d0, d1;
    int q;
};

CBX_SEQ_HD SeqTab seq_identity() { return SeqTab{0, 0, 2}; }

// Exponent of the unit of the binade holding P (P >= 0, finite): 2^(e-150)
// for a normal number with biased exponent e; subnormals and the lowest
// normal binade share 2^-149.
CBX_SEQ_HD int seq_unit_exp(float P) {
#if defined(__HIPCC__)
    const uint32_t bits = __builtin_bit_cast(uint32_t, P);
#else
    uint32_t bits;
    memcpy(&bits, &P, 4);
#endif
    const int e = (int)((bits >> 23) & 0xffu);
    return e == 0 ? -149 : e - 150;
}

CBX_SEQ_HD SeqStep seq_step(float t, int e) {
    float y = ldexpf(t, -e);
    y = y < kSeqClamp ? y : kSeqClamp;
    const int f = (int)y;
    const float r = y - (float)f;  // exact: the fraction of y
    SeqStep s;
    s.inc = f + (r > 0.5f ? 1 : 0);
    s.tie = (r == 0.5f) ? 1 : 0;
    s.fodd = f & 1;
    return s;
}

// Apply one step to a partial increment d with current parity c.
CBX_SEQ_HD void seq_apply(int& d, int& c, const SeqStep& s) {
    const int i = s.inc + (s.tie & (c ^ s.fodd));
    d = d + i < kSeqSat ? d + i : kSeqSat;
    c = s.tie ? 0 : (c ^ (i & 1));
}

CBX_SEQ_HD SeqTab seq_push(SeqTab T, const SeqStep& s) {
    int c0 = T.q & 1, c1 = (T.q >> 1) & 1;
    seq_apply(T.d0, c0, s);
    seq_apply(T.d1, c1, s);
    T.q = c0 | (c1 << 1);
    return T;
}

// A then B.
CBX_SEQ_HD SeqTab seq_compose(const SeqTab& A, const SeqTab& B) {
    const int c0 = A.q & 1, c1 = (A.q >> 1) & 1;
    const int b0 = B.q & 1, b1 = (B.q >> 1) & 1;
    SeqTab R;
    const int e0 = A.d0 + (c0 ? B.d1 : B.d0), e1 = A.d1 + (c1 ? B.d1 : B.d0);
    R.d0 = e0 < kSeqSat ? e0 : kSeqSat;
    R.d1 = e1 < kSeqSat ? e1 : kSeqSat;
    R.q = (c0 ? b1 : b0) | ((c1 ? b1 : b0) << 1);
    return R;
}

}  // namespace cbx
