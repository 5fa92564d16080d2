// ORACLE cross-check (test infrastructure only): drives rocRAND's Philox4x32-10 engine on the host
// (rocrand: rocrand_philox4x32_10.h:124-300), the generator torch-ROCm's device draws use. Reads
// "seed subsequence offset nblocks" lines on stdin (offset in 32-bit words, as hiprand_init takes it) and
// prints next4() blocks, plus the host Box-Muller pair of each block's first two words
// (rocrand_normal.h:53-68, host branch).
#include <cstdio>
#include <rocrand/rocrand_philox4x32_10.h>
#include <rocrand/rocrand_normal.h>

int main() {
    unsigned long long seed, subseq, off, n;
    while (std::scanf("%llu %llu %llu %llu", &seed, &subseq, &off, &n) == 4) {
        rocrand_device::philox4x32_10_engine eng(seed, subseq, off);
        for (unsigned long long i = 0; i < n; ++i) {
            uint4 w = eng.next4();
            float2 bm = rocrand_device::detail::box_muller(w.x, w.y);
            std::printf("%08x %08x %08x %08x %.9e %.9e\n", w.x, w.y, w.z, w.w, bm.x, bm.y);
        }
    }
    return 0;
}
