// Prints rocRAND's Philox4x32-10 block for a counter and key given on the
// command line: an implementation by other authors, used to check ours.
// usage: rocrand_philox_kat c0 c1 c2 c3 k0 k1   (hex or decimal words)
#include <cstdio>
#include <cstdlib>

#include <rocrand/rocrand_philox4x32_10.h>

// ten_rounds() is the engine's raw block function; expose it.
struct RawPhilox : rocrand_device::philox4x32_10_engine {
    uint4 block(uint4 c, uint2 k) { return ten_rounds(c, k); }
};

int main(int argc, char** argv) {
    if (argc != 7) return 2;
    unsigned v[6];
    for (int i = 0; i < 6; ++i) v[i] = (unsigned)strtoul(argv[i + 1], nullptr, 0);
    RawPhilox e;
    const uint4 o = e.block(uint4{v[0], v[1], v[2], v[3]}, uint2{v[4], v[5]});
    printf("%08x %08x %08x %08x\n", o.x, o.y, o.z, o.w);
    return 0;
}
