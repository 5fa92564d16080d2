/*
 * ORACLE -- test infrastructure only. Nothing in the product (noise_amd/) may link, load or call this
 * file; tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it to check the product.
 *
 * CPU restatement of the noise that the reference draws from torch's device generator:
 *   - eggroll.py:114   buffer = torch.randn(2**28, generator=Generator('cuda').manual_seed(SEED))
 *   - eggroll.py:117-120 offsets = torch.randint(0, NOISE - sum(p.shape), (P,), generator=g) per parameter
 *   - run.py:216, 221, 233 (DUST noise, signs, orthogonal-draw row offsets)
 * On torch-ROCm these are torch's grid-stride distribution kernel over rocRAND Philox4x32-10:
 *   torch: include/ATen/native/hip/DistributionTemplates.h:52-89 (calc_execution_policy, grid-stride loop),
 *          :126-131 (generator offset bookkeeping), :318-348 (randint 32-bit path), :446-457 (normal4)
 *   torch: include/ATen/core/TransformationHelper.h:42-44 (val % range + base), :97-99 (val*std + mean)
 *   rocrand: rocrand_philox4x32_10.h:124-197 (seed/restart/next4), :199-222 (counter arithmetic),
 *            :275-300 (rounds), rocrand_normal.h:53-68 (Box-Muller), rocrand_common.h:26-30 (constants)
 *   Philox4x32-10 itself: Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11.
 *
 * Element L of a draw of `numel` values with S = 256*G grid threads (G = min(ceil(numel/256),
 * CUs*floor(maxThreadsPerCU/256))) is lane (L mod 4S)/S of the k-th Philox block of thread t = L mod S,
 * k = L / 4S, i.e. Philox4x32-10 of counter (offset/4 + k, 0, t_lo, t_hi) under key (seed_lo, seed_hi).
 *
 * The integer outputs (u32 blocks, randint values) are exact. The float normals use the host libm
 * (logf, sqrtf, sinf, cosf) as rocRAND's host branch does (rocrand_normal.h:62-64); the device branch uses
 * __sincosf, so host floats agree with the device only to a few ulp. Bit-exactness of the device normals
 * is pinned on the GPU against torch.randn itself, not by this file.
 */
#include <math.h>
#include <stdint.h>

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

/* One Philox4x32 round (SC'11, eq. for Philox-4x32: two 32x32->64 products, xor with key). */
static void philox_round(uint32_t c[4], const uint32_t k[2]) {
    uint64_t p0 = (uint64_t)PHILOX_M0 * c[0];
    uint64_t p1 = (uint64_t)PHILOX_M1 * c[2];
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c[1] ^ k[0];
    uint32_t n2 = hi0 ^ c[3] ^ k[1];
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
}

/* Philox4x32 with `rounds` rounds (10 for Philox4x32-10); the key is bumped by the Weyl constants
 * between rounds. */
void oracle_philox4x32(const uint32_t ctr[4], const uint32_t key[2], int rounds, uint32_t out[4]) {
    uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
    uint32_t k[2] = {key[0], key[1]};
    for (int r = 0; r < rounds; ++r) {
        philox_round(c, k);
        k[0] += PHILOX_W0;
        k[1] += PHILOX_W1;
    }
    out[0] = c[0]; out[1] = c[1]; out[2] = c[2]; out[3] = c[3];
}

/* Grid threads S of torch's calc_execution_policy (DistributionTemplates.h:52-65). */
uint64_t oracle_grid_threads(uint64_t numel, uint32_t cus, uint32_t max_threads_per_cu) {
    uint64_t blocks = (numel + 255) / 256;
    uint64_t cap = (uint64_t)cus * (max_threads_per_cu / 256);
    if (blocks > cap) blocks = cap;
    return blocks * 256;
}

/* Generator offset increment of one draw (DistributionTemplates.h:64: counter_offset), unroll 4. */
uint64_t oracle_offset_increment(uint64_t numel, uint64_t grid_threads) {
    return ((numel - 1) / (grid_threads * 4) + 1) * 4;
}

/* Counter arithmetic of rocrand's restart(subsequence, offset) + k next4() calls
 * (rocrand_philox4x32_10.h:165-178, 199-235): counter = (offset/4 + k) in words 0-1 with carry,
 * subsequence added into words 2-3. torch's offsets are multiples of 4, so the substate is 0. */
static void element_counter(uint64_t offset, uint64_t subseq, uint64_t k, uint32_t c[4]) {
    uint64_t lo = offset / 4 + k; /* fits 64 bits for every offset torch produces */
    c[0] = (uint32_t)lo;
    c[1] = (uint32_t)(lo >> 32);
    c[2] = (uint32_t)subseq;
    c[3] = (uint32_t)(subseq >> 32);
}

/* The Philox block and lane that element L of a draw uses. */
static void element_block(uint64_t seed, uint64_t offset, uint64_t S, uint64_t L, uint32_t out[4], int *lane) {
    uint64_t k = L / (4 * S);
    uint64_t r = L % (4 * S);
    uint64_t t = r % S;
    uint32_t c[4], key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    *lane = (int)(r / S);
    element_counter(offset, t, k, c);
    oracle_philox4x32(c, key, 10, out);
}

/* u32 that element L of a 32-bit randint draw sees (DistributionTemplates.h:339-345). */
void oracle_draw_u32(uint64_t seed, uint64_t offset, uint64_t S, const int64_t *idx, int64_t n, uint32_t *out) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t blk[4];
        int lane;
        element_block(seed, offset, S, (uint64_t)idx[i], blk, &lane);
        out[i] = blk[lane];
    }
}

/* torch.randint(base, base+range) for range < 2^28 (32-bit path; TransformationHelper.h:42-44). */
void oracle_randint(uint64_t seed, uint64_t offset, uint64_t S, uint64_t range, int64_t base,
                    const int64_t *idx, int64_t n, int64_t *out) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t blk[4];
        int lane;
        element_block(seed, offset, S, (uint64_t)idx[i], blk, &lane);
        out[i] = (int64_t)(blk[lane] % range) + base;
    }
}

/* Box-Muller of one u32 pair, host branch of rocrand_normal.h:53-68. u lies in (0, 1], v in (0, 2pi]. */
static void box_muller(uint32_t x, uint32_t y, float *r0, float *r1) {
    const float inv = 2.3283064e-10f;        /* 2^-32 */
    const float inv_2pi = 1.46291807e-09f;   /* 2^-32 * 2pi */
    float u = inv + (float)x * inv;
    float v = inv_2pi + (float)y * inv_2pi;
    float s = sqrtf(-2.0f * logf(u));
    *r0 = sinf(v) * s;
    *r1 = cosf(v) * s;
}

/* torch.randn elements (normal4: lanes 0,1 from words (0,1), lanes 2,3 from words (2,3)). */
void oracle_randn(uint64_t seed, uint64_t offset, uint64_t S, const int64_t *idx, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t blk[4];
        int lane;
        float a, b;
        element_block(seed, offset, S, (uint64_t)idx[i], blk, &lane);
        if (lane < 2) box_muller(blk[0], blk[1], &a, &b);
        else box_muller(blk[2], blk[3], &a, &b);
        out[i] = (lane & 1) ? b : a;
    }
}

/* The (u, v) Box-Muller inputs of element L, exposed so tests can bound the device error analytically. */
void oracle_randn_uv(uint64_t seed, uint64_t offset, uint64_t S, const int64_t *idx, int64_t n,
                     uint32_t *ux, uint32_t *vy, int32_t *is_cos) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t blk[4];
        int lane;
        element_block(seed, offset, S, (uint64_t)idx[i], blk, &lane);
        ux[i] = lane < 2 ? blk[0] : blk[2];
        vy[i] = lane < 2 ? blk[1] : blk[3];
        is_cos[i] = lane & 1;
    }
}
