// ORACLE cross-check (test infrastructure only): drives torch's own host/device Philox engine
// (torch: include/ATen/core/PhiloxRNGEngine.h:67-236) so tests can compare oracle/philox.c against an
// implementation it was not derived from. Reads "seed subsequence block_offset nblocks" lines on stdin and
// prints each 128-bit block as four hex words. torch's engine counts its offset in 128-bit blocks.
#include <ATen/core/PhiloxRNGEngine.h>
#include <cinttypes>
#include <cstdio>

int main() {
    unsigned long long seed, subseq, off, n;
    while (std::scanf("%llu %llu %llu %llu", &seed, &subseq, &off, &n) == 4) {
        at::philox_engine eng(seed, subseq, off);
        for (unsigned long long i = 0; i < n; ++i) {
            uint32_t w[4];
            for (int j = 0; j < 4; ++j) w[j] = eng();
            std::printf("%08x %08x %08x %08x\n", w[0], w[1], w[2], w[3]);
        }
    }
    return 0;
}
