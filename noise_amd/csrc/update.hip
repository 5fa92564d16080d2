// EGGROLL's update reassembly: fitness weights and the rank-1 gradient sum, the noise regenerated from the
// Philox counter inside the kernels (no 1 GiB buffer, no gathered fp32 noise rows).
//
// Replaces eggroll.py:151-163:
//   fitness = losses[1::2] - losses[0::2]; fitness = fitness / (fitness.std() + 1e-8)
//   weight = zeros(pairs).index_add_(0, arange(len(fitness)) % pairs, fitness)
//   gradients[name] -= (w[:, None] * a).t() @ b       per chunk of directions   (2-D parameters)
//   gradients[name] -= w @ eps                                                  (1-D parameters)
//   p.grad = gradients[name] / len(fitness)
// where a = buffer[off_d + 0 .. rows), b = buffer[off_d + rows .. rows + cols) (eggroll.py:122-128).
//
// A 2-D parameter's gradient G = scale * sum_d w_d a_d b_d^T is a GEMM [rows x pairs] x [pairs x cols]. The
// reference runs it in fp32 (TF32 under set_float32_matmul_precision('high'), run.py:676 / eggroll.py main);
// gfx950 has no xf32 MFMA, so each chunk of directions is regenerated into a bf16 table holding the hi and lo
// halves of every value (v = hi + lo to 2^-16; the weights folded into a's rows), in blocks of 32 directions
// per 128 B line: [hi x 32 | lo x 32]. The GEMM reads a line of every row per stage and issues the three bf16
// products hi_a hi_b, hi_a lo_b, lo_a hi_b of each 16 directions from one read of each fragment
// (split-bf16x3, fp32 accumulation). Chunks accumulate into G in order (deterministic). Parameters whose
// sides are not multiples of 256 (ve_gate [8, 32], the 1-D mixing scalars) are small: one workgroup per
// gradient entry sums over all directions.
#include <atomic>

#include "common.hpp"
#include "philox.hpp"
#include "tile.hpp"

namespace noise {
namespace {

constexpr int kMaxParams = 64;
constexpr int kTile = 256;

// The big parameters of one call (kernel argument, ~2.6 KB).
struct UpdateSet {
    int n;
    const int64_t *offsets[kMaxParams];
    __bf16 *table[kMaxParams];        // [rows + cols][2 np]: a rows, then b rows, [hi 32 | lo 32] blocks
    float *grad[kMaxParams];          // [rows][cols]
    int rows[kMaxParams], cols[kMaxParams];
    int row_start[kMaxParams + 1];    // prefix sums of rows + cols
    int tile_start[kMaxParams + 1];   // prefix sums of (rows / 256) (cols / 256)
};

// The small parameters of one call.
struct UpdateSmall {
    int n;
    const int64_t *offsets[kMaxParams];
    float *grad[kMaxParams];
    int rows[kMaxParams], cols[kMaxParams];  // cols = 0: a 1-D parameter of rows entries
    int start[kMaxParams + 1];               // prefix sums of the entry counts
};

__device__ inline float noise_at(const DrawLayout &dl, int64_t L, int64_t numel) {
    return (L >= 0 && L < numel) ? draw_normal(dl, (uint64_t)L, 0.0f, 1.0f) : __builtin_nanf("");
}

// eggroll.py:151-154 in one workgroup: the std is the unbiased one (torch.std's default), accumulated in
// double; fitness and its division stay fp32 as in the reference.
__global__ __launch_bounds__(1024) void update_weights_kernel(const float *__restrict__ losses, int64_t F,
                                                              int64_t pairs, float *__restrict__ weight) {
    __shared__ double red[1024];
    const int tid = threadIdx.x;
    auto block_sum = [&](double v) {
        red[tid] = v;
        __syncthreads();
        for (int s = 512; s > 0; s >>= 1) {
            if (tid < s) red[tid] += red[tid + s];
            __syncthreads();
        }
        const double r = red[0];
        __syncthreads();
        return r;
    };
    double s = 0.0;
    for (int64_t i = tid; i < F; i += 1024) s += (double)(losses[2 * i + 1] - losses[2 * i]);
    const double mean = block_sum(s) / (double)F;
    double q = 0.0;
    for (int64_t i = tid; i < F; i += 1024) {
        const double e = (double)(losses[2 * i + 1] - losses[2 * i]) - mean;
        q += e * e;
    }
    const float denom = (float)sqrt(block_sum(q) / (double)(F - 1)) + 1e-8f;
    for (int64_t d = tid; d < pairs; d += 1024) {
        float w = 0.0f;
        for (int64_t i = d; i < F; i += pairs) w += (losses[2 * i + 1] - losses[2 * i]) / denom;
        weight[d] = w;
    }
}

// position of direction k's hi half in a table row ([hi x 32 | lo x 32] per 32 directions; lo 32 after it)
__device__ __forceinline__ int64_t tab_pos(int64_t k) { return (k >> 5) * 64 + (k & 31); }

// One table row per workgroup, 256 directions per thread block column: row r of parameter p holds, for
// direction d0 + k, the element off_d + r of the draw (a for r < rows, scaled by weight * scale; b after).
// Directions k >= n (padding up to np) are zero.
__global__ __launch_bounds__(256) void update_tables_kernel(UpdateSet s, int64_t d0, int64_t n, int64_t np,
                                                            const float *__restrict__ weight, float scale,
                                                            DrawLayout dl, int64_t numel) {
    const int r = blockIdx.x;
    int p = 0;
    while (p + 1 < s.n && s.row_start[p + 1] <= r) ++p;
    const int rl = r - s.row_start[p];
    const bool is_a = rl < s.rows[p];
    __bf16 *row = s.table[p] + (int64_t)rl * 2 * np;
    const int64_t k = (int64_t)blockIdx.y * 256 + threadIdx.x;
    float v = 0.0f;
    if (k < n) {
        const int64_t d = d0 + k;
        v = noise_at(dl, s.offsets[p][d] + rl, numel);
        if (is_a) v *= weight[d] * scale;
    }
    {
        // v rounded to fp32 first, then lo = v - hi exactly (no fused multiply-subtract)
#pragma clang fp contract(off)
        const __bf16 hi = (__bf16)v;
        row[tab_pos(k)] = hi;
        row[tab_pos(k) + 32] = (__bf16)(v - (float)hi);
    }
}

// As update_tables_kernel, reading the draw from a materialised buffer (fp32 [numel]) instead of the Philox
// counter: a workgroup reads 32 directions x 256 consecutive elements (1 KiB per direction, coalesced) into
// LDS, all 32 loads of a thread in flight together, then writes the 256 table rows' block of 32 directions
// (4 lanes x 2 x 16 B per row: one whole 128 B line). The 33 KB tile lets four workgroups share a CU, which
// keeps enough bytes in flight for the HBM's latency. grid = (rows_total / 256, np / 32).
constexpr int kTabK = 32, kTabPad = 257;
__global__ __launch_bounds__(256) void update_tables_from_buffer_kernel(UpdateSet s, int64_t d0, int64_t n,
                                                                        int64_t np, const float *__restrict__ weight,
                                                                        float scale, const float *__restrict__ buf,
                                                                        int64_t numel) {
    __shared__ float sm[kTabK * kTabPad];
    const int r0 = blockIdx.x * 256, tid = threadIdx.x;
    int p = 0;
    while (p + 1 < s.n && s.row_start[p + 1] <= r0) ++p;
    const int rl0 = r0 - s.row_start[p];  // the 256 rows lie in one parameter (its row count is a multiple of 256)
    const int64_t k0 = (int64_t)blockIdx.y * kTabK;
    const int kv = n - k0 < kTabK ? (int)(n - k0) : kTabK;  // valid directions of this block (>= 1)
    const int64_t *off = s.offsets[p] + d0 + k0;
    // the tile's loads in flight together: addresses clamped into the buffer, out-of-range elements set after
    for (int kb = 0; kb < kTabK; kb += 32) {
        float v[32];
        bool ok[32];
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const int64_t L = (kb + e < kv ? off[kb + e] : 0) + rl0 + tid;
            ok[e] = L >= 0 && L < numel;
            v[e] = buf[L < 0 ? 0 : (L < numel ? L : numel - 1)];
        }
#pragma unroll
        for (int e = 0; e < 32; ++e)
            sm[(kb + e) * kTabPad + tid] = kb + e < kv ? (ok[e] ? v[e] : __builtin_nanf("")) : 0.0f;
    }
    __syncthreads();
    const int c = tid & 3;  // directions 8c .. 8c + 7 of the block's 32
    float wk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) wk[e] = k0 + 8 * c + e < n ? weight[d0 + k0 + 8 * c + e] * scale : 0.0f;
    for (int pass = 0; pass < 4; ++pass) {
        const int rr = pass * 64 + (tid >> 2), rl = rl0 + rr;
        const bool is_a = rl < s.rows[p];
        bf16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // v rounded to fp32 first, then lo = v - hi exactly (no fused multiply-subtract)
#pragma clang fp contract(off)
            float v = sm[(8 * c + e) * kTabPad + rr];
            if (is_a) v *= wk[e];
            hi[e] = (__bf16)v;
            lo[e] = (__bf16)(v - (float)hi[e]);
        }
        __bf16 *row = s.table[p] + (int64_t)rl * 2 * np + tab_pos(k0 + 8 * c);
        *reinterpret_cast<bf16x8 *>(row) = hi;
        *reinterpret_cast<bf16x8 *>(row + 32) = lo;
    }
}

// G[o][i] (+)= sum_d A[o][d] B[i][d] over the chunk's np directions, A = hi_a + lo_a and B = hi_b + lo_b, as
// hi_a hi_b + hi_a lo_b + lo_a hi_b: one 256 x 256 tile of one parameter per workgroup. 8 waves of 128 (A rows)
// x 64 (B rows), four 32 x 32 accumulator blocks by two. Workgroups past the first `full` take part q of `split`
// equal ranges of the chunk's directions for tile full + (wg - full) / split and write that partial tile to part
// (summed in order by update_reduce_kernel): the last, partial round of workgroups then runs `split` times
// shorter. Per stage, 32 directions of the tile's 512 rows (64 KiB), two stages in flight; per 16 directions a
// wave reads its hi and lo fragments once for 24 products.
//
// Tables (RAW false): a stage is one 128 B line of each row ([hi | lo] of 32 directions) copied global -> LDS,
// chunks XOR-swizzled by row pair, read as 16 B fragments.
//
// Buffer (RAW true): no tables. A stage is the 32 directions' fp32 slices themselves, [direction][A rows | B
// rows] at a stride of 2176 B (2 KiB + 128), copied straight from the buffer (16 B per lane; slices start at any
// element). Each wave copies 4 directions and, once its copies have landed, splits them in place: the 32 B
// holding rows 8 c .. 8 c + 7 of a direction become [hi x 8 | lo x 8] (lo first where bit 1 of the direction is
// set), so nothing crosses lanes or waves before the stage's barrier. Fragments are then read with gfx950's
// transposing LDS read (ds_read_b64_tr_b16: in each 16 lanes, lane i takes element i % 4 of the 8 B that lane
// i / 4 + 4 e addresses), which gathers a row's 4 consecutive directions from 4 direction rows. The odd stride
// (128 B apart mod 256) and the hi / lo swap put a read's 4 directions on 4 disjoint sets of banks. The values,
// hence the products and G, are those of the tables.
struct UpdateRaw {
    int64_t d0, n;             // the chunk's first direction and its valid directions (the rest up to np is zero)
    const float *weight;
    float scale;
    const float *buf;          // fp32 [numel], numel <= 2^30 (lane offsets are 32-bit byte offsets)
    int64_t numel;
};
constexpr int kUgStage = 512 * 128;  // tables: bytes per stage, 256 A rows, then 256 B rows
constexpr int kUgDir = 2176;         // buffer: bytes per direction of a stage (2 KiB of rows, 128 B apart)
constexpr int kUgRawStage = 32 * kUgDir;
template <bool RAW>
__global__ __launch_bounds__(512) void update_gemm_kernel(UpdateSet s, int np, int accumulate, int full, int split,
                                                          float *__restrict__ part, UpdateRaw raw) {
    constexpr int kSt = RAW ? kUgRawStage : kUgStage;
    __shared__ __attribute__((aligned(16))) char lds[2 * kSt];
    // workgroups are dispatched round-robin over the 8 XCDs: each XCD takes a contiguous range of the full
    // tiles (and of the partial items), so the tiles that share a table panel run under one L2
    int wg = blockIdx.x;
    if (wg < full) {
        if ((full & 7) == 0) wg = (wg & 7) * (full >> 3) + (wg >> 3);
    } else {
        const int items = (int)gridDim.x - full, i = wg - full;
        if ((items & 7) == 0) wg = full + (i & 7) * (items >> 3) + (i >> 3);
    }
    const bool partial = wg >= full;
    const int item = wg - full;  // partial workgroups: item = split * (tile - full) + q
    const int tile = partial ? full + item / split : wg;
    int p = 0;
    while (p + 1 < s.n && s.tile_start[p + 1] <= tile) ++p;
    const int t = tile - s.tile_start[p];
    const int rows = s.rows[p], cols = s.cols[p];
    const int ot = t / (cols / kTile), ct = t % (cols / kTile);
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn0 = 128 * (wave & 1), wm0 = 64 * (wave >> 1);
    const int64_t ld = 2 * (int64_t)np;  // table row length (elements)
    const __bf16 *A = s.table[p] + (int64_t)ot * kTile * ld, *B = s.table[p] + (int64_t)(rows + ct * kTile) * ld;
    const unsigned lbase = lds_addr(lds);
    // stages k0 .. k0 + nk - 1 of the chunk's np / 32 (np is a multiple of 256: np / 32 divides by split)
    const int nk = partial ? np / 32 / split : np / 32;
    const int k0 = partial ? (item % split) * nk : 0;

    // tables: copy i (0 .. 7) of a stage: tile rows 64 i + 8 wave .. + 8 (A for i < 4, B after); lane: row
    // lane / 8 of the copy, LDS slot lane % 8 holds the line's chunk (lane % 8) ^ ((row >> 1) & 7)
    const int rl = 8 * wave + (lane >> 3);
    const int cl = (lane & 7) ^ ((rl >> 1) & 7);
    const unsigned off = (unsigned)(rl * ld * 2 + cl * 16);
    auto issue = [&](int ks) {  // stage k0 + ks into buffer ks % 2
        const unsigned st = lbase + (ks & 1) * kUgStage + wave * 1024;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const __bf16 *src = (i < 4 ? A + (int64_t)(64 * i) * ld : B + (int64_t)(64 * (i - 4)) * ld) + 64 * (k0 + ks);
            lds_dma16_at(src, off, st + i * 8192);
        }
    };

    // buffer: wave w copies and splits directions 4 w + i (i = 0 .. 3) of each stage. The offsets and weights
    // are read through the scalar cache (address space 4: this kernel writes neither).
    typedef const __attribute__((address_space(4))) int64_t *c_i64p;
    typedef const __attribute__((address_space(4))) float *c_f32p;
    const c_i64p offs = (c_i64p)s.offsets[p];
    const c_f32p wts = (c_f32p)raw.weight;
    const int64_t side0 = (int64_t)ot * kTile, side1 = (int64_t)rows + ct * kTile;  // first slice element per side
    // a side of a direction (256 rows, 1 KiB) in one copy of 16 B per lane (lane l: rows 4 l .. + 4; a slice may
    // start at any element, so a lane's 16 B are 4 B aligned, which multi-dword global loads accept). The split
    // of a stage follows its copies' issue with no other issue between (issue 0, split 0, issue 1, ...; split
    // ks + 1 then issue ks + 2), so each direction's offset, scaled weight and kind pass from one to the other
    // in wave-uniform registers. kind: 0 padding, 1 inside the buffer, 2 leaving it (elements outside: NaN)
    int64_t d_off[4];
    float d_w[4];
    int d_kind[4];
    auto issue_raw = [&](int ks) {
        const unsigned st = lbase + (ks & 1) * kUgRawStage;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int dl = 4 * wave + i;
            const int64_t k = (int64_t)(k0 + ks) * 32 + dl;
            int64_t o = 0;
            int kind = 0;
            float w = 0.0f;
            if (k < raw.n) {
                o = offs[raw.d0 + k];
                w = wts[raw.d0 + k] * raw.scale;
                kind = o + side0 >= 0 && o + side1 + kTile <= raw.numel ? 1 : 2;
            }
            d_off[i] = o;
            d_w[i] = w;
            d_kind[i] = kind;
            if (kind == 1) {
                lds_dma16_at(raw.buf + o + side0, (unsigned)(16 * lane), st + dl * kUgDir);
                lds_dma16_at(raw.buf + o + side1, (unsigned)(16 * lane), st + dl * kUgDir + 1024);
            } else {
                // 4 B copies with every lane's element clamped into the buffer (a padding direction reads row 0)
#pragma unroll
                for (int side = 0; side < 2; ++side)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        int64_t L = kind ? o + (side ? side1 : side0) + 64 * q + lane : 0;
                        L = L < 0 ? 0 : (L < raw.numel ? L : raw.numel - 1);
                        lds_dma4_at(raw.buf, (unsigned)(4 * L), st + dl * kUgDir + side * 1024 + 256 * q);
                    }
            }
        }
    };
    // split stage ks (buffer ks % 2) in place: lane l takes side l / 32, rows 64 q + 8 c .. + 8 (q = (l / 8) % 4,
    // c = l % 8) of each of the wave's 4 directions
    auto split_raw = [&](int ks) {
        char *st = lds + (ks & 1) * kUgRawStage;
        const int side = lane >> 5, q = (lane >> 3) & 3, cp = lane & 7;
        // the two 16 B halves (rows + 0 .. 3, + 4 .. 7) in the order h, 1 - h with h = bit 3 of the lane: each
        // 16-lane pass then covers every bank once
        const int h0 = (lane >> 3) & 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int dl = 4 * wave + i, sb = (i >> 1) & 1;
            char *c = st + dl * kUgDir + side * 1024 + 256 * q + 32 * cp;
            const float4 v4[2] = {*reinterpret_cast<const float4 *>(c + 16 * h0),
                                  *reinterpret_cast<const float4 *>(c + 16 * (1 - h0))};
            // a rows: weight * scale; b rows: 1. Each case converts on its own, so that the common one (kind 1)
            // keeps its loaded registers (a merge after the rare cases' rewrites would copy them)
            const float w = side ? 1.0f : d_w[i];
            auto convert = [&](const float4 (&x)[2], float wx) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    // v rounded to fp32 first, then lo = v - hi exactly (no fused multiply-subtract), as the tables
#pragma clang fp contract(off)
                    const int hh = t ? 1 - h0 : h0;
                    const float v[4] = {x[t].x * wx, x[t].y * wx, x[t].z * wx, x[t].w * wx};
                    bf16x4 hi, lo;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        hi[e] = (__bf16)v[e];
                        lo[e] = (__bf16)(v[e] - (float)hi[e]);
                    }
                    *reinterpret_cast<bf16x4 *>(c + 16 * sb + 8 * hh) = hi;
                    *reinterpret_cast<bf16x4 *>(c + 16 * (1 - sb) + 8 * hh) = lo;
                }
            };
            if (d_kind[i] == 1) {
                convert(v4, w);
            } else if (d_kind[i] == 0) {
                // a padding direction: zeros
                const float4 z[2] = {float4{0.f, 0.f, 0.f, 0.f}, float4{0.f, 0.f, 0.f, 0.f}};
                convert(z, 1.0f);
            } else {
                // the slice leaves the buffer: its elements outside read as NaN
                const int64_t L = d_off[i] + (side ? side1 : side0) + 64 * q + 8 * cp;  // the first of the 8 rows
                float4 y[2] = {v4[0], v4[1]};
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int64_t Lh = L + 4 * (t ? 1 - h0 : h0);
                    float *f = reinterpret_cast<float *>(&y[t]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) f[e] = (Lh + e >= 0 && Lh + e < raw.numel) ? f[e] : __builtin_nanf("");
                }
                convert(y, w);
            }
        }
    };

    // tables: fragment rows wn0 + 32 fb + j (A) and 256 + wm0 + 32 tb + j (B) share the swizzle of row j; chunk
    // 2 s + hf is the hi half of directions 16 s + 8 hf .. + 8, chunk 4 + 2 s + hf its lo half
    int fo[2][2];
#pragma unroll
    for (int sk = 0; sk < 2; ++sk)
#pragma unroll
        for (int h = 0; h < 2; ++h) fo[sk][h] = j * 128 + (((4 * h + 2 * sk + hf) ^ ((j >> 1) & 7)) << 4);
    // buffer: lane 16 G + i addresses direction 8 (G / 2) + i / 4 (+ 16 sk + 4 e) and rows 16 (G % 2) + 4 (i % 4)
    // .. + 4 of a 32-row block; bit 1 of that direction (bit 3 of i) swaps hi and lo. tro[lo]
    int tro[2];
    {
        const int G = lane >> 4, i = lane & 15;
        const int grp = 2 * (G & 1) + ((i & 3) >> 1);  // row group within the block (0 .. 3)
#pragma unroll
        for (int lo = 0; lo < 2; ++lo)
            tro[lo] = (8 * (G >> 1) + (i >> 2)) * kUgDir + 32 * grp + 16 * (((i >> 3) & 1) ^ lo) + 8 * (i & 1);
    }
    // 32 rows from row R (a multiple of 32 within the side), directions 16 sk + 8 hf + 0 .. 7
    auto tr_frag = [&](const char *st, int side, int R, int sk, int lo) {
        const char *b = st + tro[lo] + side * 1024 + 4 * R + 16 * sk * kUgDir;
        const bf16x4 x = lds_read_tr16(b), y = lds_read_tr16(b + 4 * kUgDir);
        return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int fb = 0; fb < 4; ++fb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) acc[fb][tb] = f32x16{};
    // fragments of 16 directions, double buffered: those of the next step are read while this step's run
    bf16x8 ah[2][4], al[2][4], bh[2][2], bl[2][2];
    auto fetch = [&](int buf, const char *st, int sk) {
        if constexpr (RAW) {
#pragma unroll
            for (int fb = 0; fb < 4; ++fb) {
                ah[buf][fb] = tr_frag(st, 0, wn0 + 32 * fb, sk, 0);
                al[buf][fb] = tr_frag(st, 0, wn0 + 32 * fb, sk, 1);
            }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                bh[buf][tb] = tr_frag(st, 1, wm0 + 32 * tb, sk, 0);
                bl[buf][tb] = tr_frag(st, 1, wm0 + 32 * tb, sk, 1);
            }
        } else {
#pragma unroll
            for (int fb = 0; fb < 4; ++fb) {
                ah[buf][fb] = *reinterpret_cast<const bf16x8 *>(st + (wn0 + 32 * fb) * 128 + fo[sk][0]);
                al[buf][fb] = *reinterpret_cast<const bf16x8 *>(st + (wn0 + 32 * fb) * 128 + fo[sk][1]);
            }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                bh[buf][tb] = *reinterpret_cast<const bf16x8 *>(st + (256 + wm0 + 32 * tb) * 128 + fo[sk][0]);
                bl[buf][tb] = *reinterpret_cast<const bf16x8 *>(st + (256 + wm0 + 32 * tb) * 128 + fo[sk][1]);
            }
        }
    };
    // the three products as three passes over the 8 accumulators: dependent products 8 apart
    auto products = [&](int buf) {
#pragma unroll
        for (int pr = 0; pr < 3; ++pr)
#pragma unroll
            for (int fb = 0; fb < 4; ++fb)
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
                    acc[fb][tb] = mfma32x32x16(pr == 2 ? al[buf][fb] : ah[buf][fb], pr == 1 ? bl[buf][tb] : bh[buf][tb],
                                               acc[fb][tb]);
    };
    if constexpr (RAW) {
        // (a direction's copies number 2 or 8, so stage 0 lands and is split before stage 1 is issued: every
        // later wait is for all copies in flight)
        issue_raw(0);
        vm_wait<0>();
        asm volatile("" ::: "memory");
        split_raw(0);
        __syncthreads();
        if (nk > 1) issue_raw(1);
    } else {
        issue(0);
        if (nk > 1) issue(1);
        vm_wait_groups<8, 1>(nk > 1 ? 1 : 0);
        __syncthreads();
    }
    fetch(0, lds, 0);
#pragma unroll 1
    for (int ks = 0; ks < nk; ++ks) {
        const char *st = lds + (ks & 1) * kSt;
        fetch(1, st, 1);
        products(0);
        if constexpr (RAW) {
            // buffer: this wave splits its part of stage ks + 1 once its copies landed (nothing was issued after
            // them), under the tail of this stage's products and with no fragments held
            products(1);
            if (ks + 1 < nk) {
                vm_wait<0>();
                asm volatile("" ::: "memory");
                split_raw(ks + 1);
                __syncthreads();  // stage ks + 1 split; every wave has read its fragments of stage ks
                if (ks + 2 < nk) issue_raw(ks + 2);
                fetch(0, lds + ((ks + 1) & 1) * kSt, 0);
            }
        } else {
            if (ks + 1 < nk) {
                // stage ks + 1 landed (nothing was issued after it); every wave has read its fragments of stage
                // ks, whose buffer takes stage ks + 2
                vm_wait<0>();
                __syncthreads();
                if (ks + 2 < nk) issue(ks + 2);
                fetch(0, lds + ((ks + 1) & 1) * kUgStage, 0);
            }
            products(1);
        }
    }
    // lane (j, hf), register 4 g + e of block (fb, tb): row o = wn0 + 32 fb + 8 g + 4 hf + e, column
    // i = wm0 + 32 tb + j; the 32 lanes of a half-wave write 128 contiguous bytes of one row (a partial tile:
    // [256][256] of its own)
    float *g = partial ? part + (int64_t)item * kTile * kTile : s.grad[p] + (int64_t)ot * kTile * cols + ct * kTile;
    const int64_t ldg = partial ? kTile : cols;
    const bool add = accumulate && !partial;
#pragma unroll
    for (int fb = 0; fb < 4; ++fb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int o = wn0 + 32 * fb + 8 * (q >> 2) + 4 * hf + (q & 3);
                float *dst = g + (int64_t)o * ldg + wm0 + 32 * tb + j;
                const float v = acc[fb][tb][q];
                *dst = add ? *dst + v : v;
            }
}

// The partial tiles of update_gemm_kernel summed in order (part 0 first) into G (+=): 1024 entries per
// workgroup, 64 workgroups per tile. grid = (tiles - full) * 64.
__global__ __launch_bounds__(256) void update_reduce_kernel(UpdateSet s, int full, int split,
                                                            const float *__restrict__ part, int accumulate) {
    const int tile = full + blockIdx.x / 64, e = (blockIdx.x % 64) * 1024 + 4 * threadIdx.x;
    int p = 0;
    while (p + 1 < s.n && s.tile_start[p + 1] <= tile) ++p;
    const int t = tile - s.tile_start[p], cols = s.cols[p];
    const int ot = t / (cols / kTile), ct = t % (cols / kTile);
    const float *src = part + (int64_t)(tile - full) * split * kTile * kTile + e;
    float4 v = ld4(src);
    for (int q = 1; q < split; ++q) {
        const float4 w = ld4(src + (int64_t)q * kTile * kTile);
        v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
    }
    float *dst = s.grad[p] + (int64_t)(ot * kTile + e / kTile) * cols + ct * kTile + e % kTile;
    if (accumulate) {
        const float4 g = ld4(dst);
        v.x += g.x; v.y += g.y; v.z += g.z; v.w += g.w;
    }
    st4(dst, v);
}

// One gradient entry per workgroup: scale * sum_d weight[d] a_d[o] (b_d[i] or 1), 256 threads striding
// over the directions, then a fixed-order tree.
__global__ __launch_bounds__(256) void update_small_kernel(UpdateSmall s, int64_t pairs,
                                                           const float *__restrict__ weight, float scale,
                                                           DrawLayout dl, int64_t numel) {
    __shared__ float red[256];
    const int e = blockIdx.x, tid = threadIdx.x;
    int p = 0;
    while (p + 1 < s.n && s.start[p + 1] <= e) ++p;
    const int el = e - s.start[p], rows = s.rows[p], cols = s.cols[p];
    const int o = cols ? el / cols : el, i = cols ? el % cols : 0;
    const int64_t *off = s.offsets[p];
    float acc = 0.0f;
    for (int64_t d = tid; d < pairs; d += 256) {
        const float a = noise_at(dl, off[d] + o, numel);
        const float b = cols ? noise_at(dl, off[d] + rows + i, numel) : 1.0f;
        acc += weight[d] * a * b;
    }
    red[tid] = acc;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red[tid] += red[tid + st];
        __syncthreads();
    }
    if (tid == 0) s.grad[p][el] = scale * red[0];
}

bool is_big(const noise_update_param_t &q) {
    return q.cols > 0 && q.rows % kTile == 0 && q.cols % kTile == 0;
}

int64_t padded_chunk(int64_t chunk, int64_t pairs) {
    const int64_t c = chunk < pairs ? chunk : pairs;
    return (c + 255) / 256 * 256;
}

// The GEMM's last, partial round of workgroups (one per CU) over `cus` compute units: tiles full .. tiles - 1
// run as `split` shorter partial workgroups each, so that round fills the device; split 1: no partials.
void gemm_split(int64_t tiles, int64_t cus, int64_t &full, int &split) {
    const int64_t r = cus > 0 ? tiles % cus : 0;
    const int64_t sp = r ? cus / r : 1;
    split = sp >= 4 ? 4 : sp >= 2 ? 2 : 1;
    full = split > 1 ? tiles - r : tiles;
}

int64_t partial_bytes(int64_t tiles, int64_t full, int split) {
    return split > 1 ? (tiles - full) * split * kTile * kTile * (int64_t)sizeof(float) : 0;
}

// compute units of the current device (gfx950 parts have 256), cached per device (any host thread may ask)
int64_t device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cached[dev].load(std::memory_order_relaxed);
    if (!c) {
        int n = 0;
        c = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
        cached[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_update_weights(const float *losses, int64_t members, int64_t pairs, float *weight,
                                    noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(members >= 4 && members % 2 == 0,
                    "noise_update_weights: members must be even and >= 4 (two fitness values for a std), got %lld",
                    (long long)members);
    NOISE_CHECK_ARG(pairs >= 1, "noise_update_weights: pairs must be >= 1");
    NOISE_CHECK_ARG(losses != nullptr && weight != nullptr, "noise_update_weights: losses and weight must be non-NULL");
    hipLaunchKernelGGL(update_weights_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, losses, members / 2,
                       pairs, weight);
    return launch_status("noise_update_weights");
}

extern "C" int64_t noise_update_workspace_bytes(const noise_update_param_t *params, int nparams, int64_t pairs,
                                                int64_t chunk) {
    if (params == nullptr || nparams < 0 || pairs < 1 || chunk < 1) return -1;
    const int64_t np = padded_chunk(chunk, pairs);
    int64_t bytes = 0, tiles = 0;
    for (int i = 0; i < nparams; ++i)
        if (is_big(params[i])) {
            bytes += (params[i].rows + params[i].cols) * 2 * np * 2;
            tiles += (params[i].rows / kTile) * (params[i].cols / kTile);
        }
    // the tables, then the GEMM's partial tiles for a device of 256 compute units
    int64_t full;
    int split;
    gemm_split(tiles, 256, full, split);
    return bytes + partial_bytes(tiles, full, split);
}

extern "C" int noise_update_gradients(const noise_update_param_t *params, int nparams, int64_t pairs,
                                      const float *weight, float scale, int64_t chunk, int64_t numel, uint64_t seed,
                                      uint64_t offset, int64_t threads, const float *buffer, void *workspace,
                                      int64_t workspace_bytes, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(params != nullptr && nparams >= 0 && nparams <= kMaxParams,
                    "noise_update_gradients: 0 .. %d parameters per call, got %d", kMaxParams, nparams);
    NOISE_CHECK_ARG(pairs >= 1 && chunk >= 1, "noise_update_gradients: pairs and chunk must be >= 1");
    NOISE_CHECK_ARG(weight != nullptr, "noise_update_gradients: weight must be non-NULL");
    NOISE_CHECK_ARG(threads > 0 && threads % 256 == 0,
                    "noise_update_gradients: threads must be a positive multiple of 256");
    NOISE_CHECK_ARG(offset % 4 == 0, "noise_update_gradients: generator offset must be a multiple of 4");
    NOISE_CHECK_ARG(numel > 0, "noise_update_gradients: numel must be positive");
    NOISE_CHECK_ARG(buffer == nullptr || aligned(buffer, 4), "noise_update_gradients: buffer must be 4-byte aligned");
    const int64_t np = padded_chunk(chunk, pairs);
    // (the GEMM's 32-bit copy offsets span 64 table rows of 2 np elements)
    NOISE_CHECK_ARG(np <= (1 << 22), "noise_update_gradients: chunk too large (at most 4194304 directions)");
    UpdateSet big{};
    UpdateSmall small{};
    int64_t rows_total = 0, tiles_total = 0, entries_total = 0, need = 0;
    char *ws = static_cast<char *>(workspace);
    for (int i = 0; i < nparams; ++i) {
        const noise_update_param_t &q = params[i];
        NOISE_CHECK_ARG(q.offsets != nullptr && q.grad != nullptr && aligned(q.offsets, 8) && aligned(q.grad, 4),
                        "noise_update_gradients: parameter %d: offsets and grad must be non-NULL and aligned", i);
        NOISE_CHECK_ARG(q.rows >= 1 && q.cols >= 0, "noise_update_gradients: parameter %d: bad shape", i);
        if (is_big(q)) {
            NOISE_CHECK_ARG(q.rows + q.cols <= 65536 && q.rows / kTile * (q.cols / kTile) <= 65536,
                            "noise_update_gradients: parameter %d: %lld x %lld is too large", i, (long long)q.rows,
                            (long long)q.cols);
            const int b = big.n++;
            big.offsets[b] = q.offsets;
            big.grad[b] = q.grad;
            big.rows[b] = (int)q.rows;
            big.cols[b] = (int)q.cols;
            big.row_start[b] = (int)rows_total;
            big.tile_start[b] = (int)tiles_total;
            big.table[b] = reinterpret_cast<__bf16 *>(ws + need);
            rows_total += q.rows + q.cols;
            tiles_total += (q.rows / kTile) * (q.cols / kTile);
            need += (q.rows + q.cols) * 2 * np * 2;
        } else {
            const int64_t entries = q.rows * (q.cols ? q.cols : 1);
            NOISE_CHECK_ARG(entries <= 65536,
                            "noise_update_gradients: parameter %d: %lld x %lld is neither a multiple of 256 on both "
                            "sides nor small (<= 65536 entries)", i, (long long)q.rows, (long long)q.cols);
            const int sm = small.n++;
            small.offsets[sm] = q.offsets;
            small.grad[sm] = q.grad;
            small.rows[sm] = (int)q.rows;
            small.cols[sm] = (int)q.cols;
            small.start[sm] = (int)entries_total;
            entries_total += entries;
        }
    }
    big.row_start[big.n] = (int)rows_total;
    big.tile_start[big.n] = (int)tiles_total;
    small.start[small.n] = (int)entries_total;
    NOISE_CHECK_ARG(rows_total < (1ll << 31) && tiles_total < (1ll << 31) && entries_total < (1ll << 31),
                    "noise_update_gradients: too many rows");
    NOISE_CHECK_ARG(need == 0 || (workspace != nullptr && aligned(workspace, 16) && workspace_bytes >= need),
                    "noise_update_gradients: workspace must be 16-byte aligned and hold %lld bytes (got %lld); "
                    "see noise_update_workspace_bytes", (long long)need, (long long)workspace_bytes);
    DrawLayout dl{seed, offset, (uint64_t)threads};
    hipStream_t s = (hipStream_t)stream;
    // the GEMM's partial tiles after the tables, when the workspace holds them (else whole tiles only)
    int64_t full;
    int split;
    gemm_split(tiles_total, device_cus(), full, split);
    while (split > 1 && (workspace == nullptr || workspace_bytes - need < partial_bytes(tiles_total, full, split))) {
        split /= 2;
        if (split == 1) full = tiles_total;
    }
    float *part = split > 1 ? reinterpret_cast<float *>(ws + need) : nullptr;
    if (small.n) {
        hipLaunchKernelGGL(update_small_kernel, dim3((unsigned)entries_total), dim3(256), 0, s, small, pairs, weight,
                           scale, dl, numel);
        int st = launch_status("noise_update_gradients (small parameters)");
        if (st) return st;
    }
    if (big.n) {
        // with a buffer of at most 2^30 elements the GEMM reads the slices itself; otherwise tables first
        const bool direct = buffer != nullptr && numel <= (1ll << 30);
        for (int64_t d0 = 0; d0 < pairs; d0 += np) {
            const int64_t n = pairs - d0 < np ? pairs - d0 : np;
            const int64_t wgs = full + (tiles_total - full) * split;
            int st;
            if (direct) {
                const UpdateRaw raw{d0, n, weight, scale, buffer, numel};
                hipLaunchKernelGGL(update_gemm_kernel<true>, dim3((unsigned)wgs), dim3(512), 0, s, big, (int)np,
                                   d0 > 0 ? 1 : 0, (int)full, split, part, raw);
            } else {
                if (buffer)
                    hipLaunchKernelGGL(update_tables_from_buffer_kernel, dim3((unsigned)(rows_total / 256),
                                       (unsigned)(np / kTabK)), dim3(256), 0, s, big, d0, n, np, weight, scale, buffer,
                                       numel);
                else
                    hipLaunchKernelGGL(update_tables_kernel, dim3((unsigned)rows_total, (unsigned)(np / 256)),
                                       dim3(256), 0, s, big, d0, n, np, weight, scale, dl, numel);
                st = launch_status("noise_update_gradients (tables)");
                if (st) return st;
                hipLaunchKernelGGL(update_gemm_kernel<false>, dim3((unsigned)wgs), dim3(512), 0, s, big, (int)np,
                                   d0 > 0 ? 1 : 0, (int)full, split, part, UpdateRaw{});
            }
            st = launch_status("noise_update_gradients (gemm)");
            if (st) return st;
            if (split > 1) {
                hipLaunchKernelGGL(update_reduce_kernel, dim3((unsigned)((tiles_total - full) * 64)), dim3(256), 0, s,
                                   big, (int)full, split, part, d0 > 0 ? 1 : 0);
                st = launch_status("noise_update_gradients (partial tiles)");
                if (st) return st;
            }
        }
    }
    return NOISE_OK;
}
