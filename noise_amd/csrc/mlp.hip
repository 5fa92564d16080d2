// The whole MLP of a block with its residual writer in one kernel (eggroll.py:93 and the mixing, norm and
// next-matrix dots that follow it, eggroll.py:77-82 / 94):
//
//   hid = relu(h W_fc^T + sign (h . b_fc) a_fc)^2                 mlp.c_fc, ReLU^2   (never stored)
//   y   = x + hid W_proj^T + sign (hid . b_proj) a_proj             mlp.c_proj + residual
//   [y = rl y + ml x0]  ->  xout = y, hout = bf16(norm(y)), next_dots = norm(y) . b_next
//
// The [tokens, 2048] hidden layer stays on chip. A workgroup owns 128 tokens of one member with 4 waves,
// one per SIMD (512 registers each); wave w owns tokens 32w .. 32w+31 and ALL 512 outputs of them:
//   - its h rows (32 tokens x 512, the B operand of the first product) live in 128 registers for the whole
//     kernel;
//   - the hidden units are swept in 64 steps of 32: step j's c_fc rows [32 x 512] and mlp.c_proj columns
//     [512 x 32] (64 KiB) are copied global -> LDS by direct copies, double buffered, and shared by the 4 waves;
//   - the first product's 32 x 32 accumulator (hidden x tokens) gets its rank-1 term and ReLU^2 in
//     registers and is packed to bf16 as the B operand of the second product without leaving the lane: the
//     D layout of v_mfma_f32_32x32x16_bf16 (lane l, register r = 4b + i holds row 8b + 4(l/32) + i) is the
//     B layout of two 16-deep k-steps once the contraction index is permuted within each 16, so mlp.c_proj's
//     columns are stored in that permuted order (noise_mlp_proj_layout);
//   - the second product accumulates the wave's [512 outputs x 32 tokens] (16 MFMA blocks, 256 accumulators);
//   - step j's first product runs interleaved with step j-1's second product, so consecutive products on the
//     same accumulator are never adjacent and the matrix core has independent work while the ReLU^2 of the
//     previous step is formed.
// The residual epilogue then has every output of a token in one lane pair: RMSNorm and the next-matrix dots
// need one exchange with lane ^ 32 and no workgroup reduction.
//
// With the attention projection in front (noise_pop_attn_mlp, eggroll.py:92 then 93), the same workgroup first
// forms x_mid = x + y W_o^T + sign (y . b_o) a_o for its tokens: the attention output rows y take the register
// slots of the h rows, W_o streams through the mlp.c_proj buffers in 16 steps of [512 rows x 32 k], and the
// product accumulates in the output accumulators. After the residual add, h = bf16(norm(x_mid)) is packed
// straight from the accumulators into the B operand of the first MLP product: the D layout's groups of four
// (r % 4 within a lane, lane / 32 alternating) are that operand once the contraction index is permuted within
// each 16, so c_fc's columns come in the same permuted order as mlp.c_proj's (noise_mlp_proj_layout). x_mid
// stays in the accumulators, the MLP adds to it, and neither x_mid nor h ever reaches HBM.
#include "common.hpp"
#include "mfma.hpp"
#include "tile.hpp"

namespace noise {
namespace {

constexpr float kNormEps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps
constexpr int kMlpThreads = 256;   // 4 waves, one per SIMD
constexpr int kTileTok = 128;      // tokens per workgroup (32 per wave)
constexpr int kHid = 2048, kEmb = 512;
constexpr int kStep = 32;          // hidden units per step
constexpr int kNumSteps = kHid / kStep;
constexpr int kFcBytes = kStep * kEmb * 2;   // c_fc rows of a step: [8 k-tiles][32 rows][128 B]
constexpr int kPjBytes = kEmb * kStep * 2;   // mlp.c_proj columns of a step: [512 rows][64 B]
constexpr int kFcOff = 0, kPjOff = 2 * kFcBytes;
constexpr int kVecOff = 2 * kFcBytes + 2 * kPjBytes;  // 128 KiB of operand buffers, then fp32 vectors:
constexpr int kAfc = kVecOff;                  // c_fc's a            [2048]
constexpr int kBpj = kAfc + kHid * 4;          // mlp.c_proj's b      [2048]
constexpr int kApj = kBpj + kHid * 4;          // mlp.c_proj's a      [512]
constexpr int kNb = kApj + kEmb * 4;           // next matrices' b    [3][512]
constexpr int kAo = kNb + 3 * kEmb * 4;        // attn.c_proj's a     [512] (with the projection in front)
constexpr int kBfc = kAo + kEmb * 4;           // c_fc's b            [512] (with the projection in front)
constexpr int kMlpLds = kBfc + kEmb * 4;       // 156 KiB
static_assert(kMlpLds <= 160 * 1024, "LDS of one CU");

struct MlpPop {
    int members, tokens;
    const float *sign;
    int dir_div;
};

struct MlpArgs {
    MlpPop pop;
    const __bf16 *x;               // h = norm of the block's mid residual, bf16 [m][T][512] (strided)
    int64_t xs_m, xs_t;
    const __bf16 *wfc;             // mlp.c_fc [2048][512]
    const __bf16 *wpj;             // mlp.c_proj [512][2048], hidden index permuted within each 16
    const float *afc;              // c_fc rank-1 a [dirs][2048] or NULL
    int64_t afc_stride;
    const float *dots_fc;          // h . b_fc per row, or NULL with afc NULL
    const float *apj, *bpj;        // mlp.c_proj rank-1 a [dirs][512], b [dirs][2048] or NULL
    int64_t apj_stride, bpj_stride;
    const float *xres;             // residual in, fp32 (may equal xout)
    int64_t xr_m, xr_t;
    float *xout;                   // residual out [m][T][512] fp32, or NULL
    const float *lam_r, *lam_x;    // next block's mixing scalars (device)
    const float *eps_r, *eps_x;
    int64_t eps_stride;
    const float *x0;
    int64_t x0_m, x0_t;
    __bf16 *hout;                  // [m][T][512], or [m][T][1536] = [hi | lo | hi] with split3
    const float *nb[3];
    int64_t nb_stride[3];
    float *ndots;                  // [rows][NNEXT]
    // the attention projection in front (FRONT): x (above) is the attention output y, xres the block's
    // residual input; c_fc's columns then come permuted like mlp.c_proj's and its x . b is formed here
    const __bf16 *wo;              // attn.c_proj [512][512]
    const float *ao;               // its rank-1 a [dirs][512] or NULL
    int64_t ao_stride;
    const float *odots;            // y . b_o partial sums [rows][odots_n] (per head)
    int odots_n;
    const float *bfc;              // c_fc's rank-1 b [dirs][512] (with afc)
    int64_t bfc_stride;
};

// LDS offset of (k-tile kt, row r, 16 B chunk c) in a c_fc step buffer: 128 B rows, chunks XOR-swizzled by
// row pair so a fragment's 32 rows spread over all banks
__device__ __forceinline__ int fc_off(int kt, int r, int c) { return kt * 4096 + r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }
// ... and of (row r, chunk c) in an mlp.c_proj step buffer: 64 B rows, chunks swizzled by row quad
__device__ __forceinline__ int pj_off(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

template <bool MIX, int NNEXT, bool SPLIT3, bool FRONT>
__global__ __launch_bounds__(kMlpThreads, 1) void mlp_kernel(MlpArgs p) {
    __shared__ __attribute__((aligned(16))) char lds[kMlpLds];
    const int T = p.pop.tokens, tiles_t = T / kTileTok;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * kTileTok;
    const int tid = threadIdx.x, lane = tid & 63, jl = lane & 31, hf = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dir = m / p.pop.dir_div;
    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;
    const int tok = t0 + 32 * wave + jl;
    const int64_t row = (int64_t)m * T + tok;
    const unsigned lbase = lds_addr(lds);

    // the tile's h rows [128 tokens x 512] into the (still free) operand buffers by whole-row direct copies, in
    // the c_fc buffers' layout ([8 k-tiles][128 rows][128 B], chunks swizzled by row pair): 128 copies of 1 KiB,
    // 32 per wave (copy i: k-tile i / 16, rows 8 (i % 16) ..)
    {
        const __bf16 *xt = p.x + m * p.xs_m + (int64_t)t0 * p.xs_t;
#pragma unroll
        for (int ci = 0; ci < 32; ++ci) {
            const int i = wave * 32 + ci, kt = i >> 4, q = i & 15;
            const int r = q * 8 + (lane >> 3);
            const int c = (lane & 7) ^ ((r >> 1) & 7);
            lds_dma16_at(xt + (int64_t)(q * 8) * p.xs_t + kt * 64, (unsigned)((lane >> 3) * p.xs_t * 2 + c * 16),
                         lbase + kt * 16384 + q * 1024);
        }
    }
    // per-member vectors into LDS (zeros when a matrix is unperturbed, so the step needs no branches)
    {
        auto vcopy = [&](const float *src, int off, int n) {
            float *dst = reinterpret_cast<float *>(lds + off);
            for (int i = tid; i < n / 4; i += kMlpThreads) st4(dst + 4 * i, src ? ld4(src + 4 * i) : float4{0.f, 0.f, 0.f, 0.f});
        };
        vcopy(p.afc ? p.afc + dir * p.afc_stride : nullptr, kAfc, kHid);
        vcopy(p.apj ? p.bpj + dir * p.bpj_stride : nullptr, kBpj, kHid);
        vcopy(p.apj ? p.apj + dir * p.apj_stride : nullptr, kApj, kEmb);
#pragma unroll
        for (int k = 0; k < NNEXT; ++k) vcopy(p.nb[k] + dir * p.nb_stride[k], kNb + k * kEmb * 4, kEmb);
        if constexpr (FRONT) {
            vcopy(p.ao ? p.ao + dir * p.ao_stride : nullptr, kAo, kEmb);
            vcopy(p.afc ? p.bfc + dir * p.bfc_stride : nullptr, kBfc, kEmb);
        }
    }
    float corr_fc = 0.f;
    if constexpr (!FRONT) corr_fc = p.afc ? sgn * p.dots_fc[row] : 0.f;
    vm_wait<0>();
    __syncthreads();
    // this lane's h row: the B operand of all 32 k-steps of the first product (k-tile s / 4, chunk 2s + hf)
    bf16x8 xf[32];
    {
        const int r = 32 * wave + jl;
#pragma unroll
        for (int s = 0; s < 32; ++s)
            xf[s] = *reinterpret_cast<const bf16x8 *>(lds + (s >> 2) * 16384 + r * 128 +
                                                      ((((2 * s + hf) & 7) ^ ((r >> 1) & 7)) << 4));
    }
    __syncthreads();  // every wave holds its h rows: the buffers take the weight copies

    // step copies: c_fc step j is 32 wave-copies of 1 KiB (copy i: k-tile i / 4, rows 8 (i % 4) ..), mlp.c_proj
    // step j is 32 (copy i: rows 16 i .. 16 i + 15); wave w issues copies 8w .. 8w + 7 of each
    auto issue_fc = [&](int js) {
        const unsigned dst = lbase + kFcOff + (js & 1) * kFcBytes;
#pragma unroll
        for (int ci = 0; ci < 8; ++ci) {
            const int i = wave * 8 + ci, kt = i >> 2, q = i & 3;
            const int r = q * 8 + (lane >> 3);
            const int c = (lane & 7) ^ ((r >> 1) & 7);
            lds_dma16_at(p.wfc + (int64_t)(kStep * js + q * 8) * kEmb + kt * 64,
                         (unsigned)((lane >> 3) * kEmb * 2 + c * 16), dst + kt * 4096 + q * 1024);
        }
    };
    auto issue_pj = [&](int js) {
        const unsigned dst = lbase + kPjOff + (js & 1) * kPjBytes;
        const int c = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
        for (int ci = 0; ci < 8; ++ci) {
            const int i = wave * 8 + ci;
            lds_dma16_at(p.wpj + (int64_t)(16 * i) * kHid + kStep * js, (unsigned)((lane >> 2) * kHid * 2 + c * 16),
                         dst + i * 1024);
        }
    };

    f32x16 out[16];
#pragma unroll
    for (int rb = 0; rb < 16; ++rb) out[rb] = f32x16{};
    f32x16 hacc;
    bf16x8 hb[2];
    float pd = 0.f;  // this lane's share of hid . b_proj

    // whole-line copies of a quarter of the features (32 tokens x 512 B) of fp32 rows into LDS at dst: copy i
    // covers rows 2i, 2i + 1; the 16 B chunk c of row r sits at position c ^ (r % 16), so the MFMA layout's reads
    // (32 rows, one chunk) spread over the banks
    auto issue_rows = [&](const float *src, int64_t ld, int q, unsigned dst) {
        const int r = lane >> 5;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int cc = (lane & 31) ^ ((2 * i + r) & 15);
            lds_dma16_at(src + (int64_t)(2 * i) * ld + 128 * q, (unsigned)(r * ld * 4 + cc * 16), dst + i * 1024);
        }
    };
    if constexpr (FRONT) {
        // x_mid = x + (y W_o^T + sign (y . b_o) a_o): W_o [512][512] through the mlp.c_proj buffers, step i holding
        // columns 32 i .. 32 i + 31 of every row (the layout of an mlp.c_proj step); xf holds the y rows
        auto issue_o = [&](int i) {
            const unsigned dst = lbase + kPjOff + (i & 1) * kPjBytes;
            const int c = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
            for (int ci = 0; ci < 8; ++ci) {
                const int q = wave * 8 + ci;
                lds_dma16_at(p.wo + (int64_t)(16 * q) * kEmb + kStep * i, (unsigned)((lane >> 2) * kEmb * 2 + c * 16),
                             dst + q * 1024);
            }
        };
        issue_o(0);
        vm_wait<0>();
        __syncthreads();
        // (unrolled: the y rows are indexed by the step, and register arrays need static indices)
#pragma unroll
        for (int i = 0; i < kEmb / kStep; ++i) {
            if (i + 1 < kEmb / kStep) issue_o(i + 1);  // its buffer was last read in step i - 1 (barrier below)
            const char *bo = lds + kPjOff + (i & 1) * kPjBytes;
            auto fo = [&](int s) {
                return *reinterpret_cast<const bf16x8 *>(bo + pj_off(32 * (s >> 1) + jl, 2 * (s & 1) + hf));
            };
            bf16x8 pa[2];
            pa[0] = fo(0);
            pa[1] = fo(1);
#pragma unroll
            for (int s = 0; s < 32; ++s) {
                const bf16x8 a = pa[s & 1];
                if (s + 2 < 32) pa[s & 1] = fo(s + 2);
                out[s >> 1] = mfma32x32x16(a, xf[2 * i + (s & 1)], out[s >> 1]);
            }
            vm_wait<0>();
            __syncthreads();  // step i + 1 landed; every wave is done with buffer i & 1
        }
        // rank-1 term and the residual rows (x, by whole-line copies a quarter at a time, double buffered in the
        // wave's own 32 KiB of the fc buffers and the first pj buffer)
        float osum = 0.f;
        if (p.ao) {
            for (int k = 0; k < p.odots_n; ++k) osum += p.odots[row * p.odots_n + k];
        }
        const float corr_o = sgn * osum;  // 0 without perturbation (and the a_o vector is zeros then)
        const float *xtile = p.xres + m * p.xr_m + (int64_t)(t0 + 32 * wave) * p.xr_t;
        const float *ao = reinterpret_cast<const float *>(lds + kAo) + 4 * hf;
        const unsigned wbase = lbase + wave * 32768;
        issue_rows(xtile, p.xr_t, 0, wbase);
        issue_rows(xtile, p.xr_t, 1, wbase + 16384);
        float ssq = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (q < 3) vm_wait<16>(); else vm_wait<0>();
            wave_lds_sync();
            const char *xb = lds + wave * 32768 + (q & 1) * 16384 + jl * 512;
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int rb = 4 * q + r4;
                    const int c = 8 * r4 + 2 * b + hf;
                    const float4 xv = *reinterpret_cast<const float4 *>(xb + ((c ^ (jl & 15)) << 4));
                    const float4 a4 = ld4(ao + 32 * rb + 8 * b);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float y = f4get(xv, e) + (out[rb][4 * b + e] + corr_o * f4get(a4, e));
                        out[rb][4 * b + e] = y;
                        ssq += y * y;
                    }
                }
            wave_lds_sync();  // this quarter's reads are done before the next copies overwrite the buffer
            if (q + 2 < 4) issue_rows(xtile, p.xr_t, q + 2, wbase + (q & 1) * 16384);
        }
        ssq += swap_halves(ssq);
        const float rstd = rsqrtf(ssq * (1.0f / kEmb) + kNormEps);
        // c_fc's x . b from the fp32 normalised row (as the residual writer forms it), and h = bf16(norm(x_mid))
        // packed as the first product's B operand: k-step s holds features 16 s + 4 hf + (0..3) and
        // 16 s + 8 + 4 hf + (0..3), registers 8 (s % 2) .. 8 (s % 2) + 7 of output block s / 2
        if (p.afc) {
            const float *bf = reinterpret_cast<const float *>(lds + kBfc) + 4 * hf;
            float d = 0.f;
#pragma unroll
            for (int rb = 0; rb < 16; ++rb)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const float4 b4 = ld4(bf + 32 * rb + 8 * b);
#pragma unroll
                    for (int e = 0; e < 4; ++e) d += out[rb][4 * b + e] * f4get(b4, e);
                }
            d += swap_halves(d);
            corr_fc = sgn * (rstd * d);
        }
#pragma unroll
        for (int s = 0; s < 32; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[s][e] = (__bf16)(out[s >> 1][8 * (s & 1) + e] * rstd);
        __syncthreads();  // every wave is done with the residual rows: the buffers take the weight copies
    }

    // first product of step js (32 k-steps), optionally interleaved with the second product of step js - 1
    // (32 MFMAs over the 16 output blocks), so consecutive products on the first product's accumulator always
    // have an independent one between them. Fragments are read from LDS two products ahead.
    auto products = [&](int js, bool first, bool second) {
        const char *bfc = lds + kFcOff + (js & 1) * kFcBytes;
        const char *bpj = lds + kPjOff + ((js - 1) & 1) * kPjBytes;
        auto fa = [&](int s) { return *reinterpret_cast<const bf16x8 *>(bfc + fc_off(s >> 2, jl, (2 * s + hf) & 7)); };
        auto fb = [&](int s) {
            return *reinterpret_cast<const bf16x8 *>(bpj + pj_off(32 * (s >> 1) + jl, 2 * (s & 1) + hf));
        };
        if (first) hacc = f32x16{};
        bf16x8 pa[2], pb[2];
        if (first) { pa[0] = fa(0); pa[1] = fa(1); }
        if (second) { pb[0] = fb(0); pb[1] = fb(1); }
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            if (first) {
                const bf16x8 a = pa[s & 1];
                if (s + 2 < 32) pa[s & 1] = fa(s + 2);
                hacc = mfma32x32x16(a, xf[s], hacc);
            }
            if (second) {
                const bf16x8 a = pb[s & 1];
                if (s + 2 < 32) pb[s & 1] = fb(s + 2);
                out[s >> 1] = mfma32x32x16(a, hb[s & 1], out[s >> 1]);
            }
        }
    };
    // ReLU^2 of step js's first product: rank-1 term, ReLU, square, bf16; the hid . b_proj share; the bf16
    // values packed as the second product's B operand (register r holds hidden 32 js + 8 (r / 4) + 4 hf + r % 4)
    auto relu2 = [&](int js) {
        const float *afc = reinterpret_cast<const float *>(lds + kAfc) + kStep * js + 4 * hf;
        const float *bpj = reinterpret_cast<const float *>(lds + kBpj) + kStep * js + 4 * hf;
        __bf16 o[16];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float4 a4 = ld4(afc + 8 * b), b4 = ld4(bpj + 8 * b);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y = hacc[4 * b + e] + corr_fc * f4get(a4, e);
                y = fmaxf(y, 0.f);
                o[4 * b + e] = (__bf16)(y * y);
            }
            // hid . b with both in bf16, as the reference's autocast x @ b (eggroll.py:58) multiplies them
            pd = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{o[4 * b], o[4 * b + 1]}, bf16x2{(__bf16)b4.x, (__bf16)b4.y}, pd,
                                                 false);
            pd = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{o[4 * b + 2], o[4 * b + 3]}, bf16x2{(__bf16)b4.z, (__bf16)b4.w},
                                                 pd, false);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            hb[0][e] = o[e];
            hb[1][e] = o[8 + e];
        }
    };

    issue_fc(0);
    // step 0: its first product only
    vm_wait<0>();
    __syncthreads();
    issue_fc(1);
    issue_pj(0);
    products(0, true, false);
#pragma unroll 1
    for (int js = 1; js < kNumSteps; ++js) {
        // this wave's copies of c_fc step js and mlp.c_proj step js - 1 landed; after the barrier every wave's
        // have, and every wave is done with the buffers the next copies overwrite (read in step js - 1)
        vm_wait<0>();
        __syncthreads();
        if (js + 1 < kNumSteps) issue_fc(js + 1);
        issue_pj(js);
        relu2(js - 1);
        products(js, true, true);
    }
    vm_wait<0>();
    __syncthreads();
    relu2(kNumSteps - 1);
    products(kNumSteps, false, true);

    // residual epilogue: y = x + product + sign (hid . b_proj) a_proj [, mixing], then norm and next dots
    const float corr = p.apj ? sgn * (pd + swap_halves(pd)) : 0.f;
    float rl = 0.f, ml = 0.f;
    if constexpr (MIX) {
        rl = *p.lam_r;
        ml = *p.lam_x;
        if (p.eps_r) rl += sgn * p.eps_r[dir * p.eps_stride];
        if (p.eps_x) ml += sgn * p.eps_x[dir * p.eps_stride];
    }
    const float *apj = reinterpret_cast<const float *>(lds + kApj) + 4 * hf;
    float *xo = p.xout ? p.xout + row * kEmb + 4 * hf : nullptr;
    float ssq = 0.f;
    // the residual rows (and, when mixing, the x0 rows) arrive by whole-line direct copies into the wave's own
    // 32 KiB of the (now free) operand buffers, a quarter of the features (32 tokens x 512 B each) at a time:
    // double buffered without mixing, x and x0 side by side with it. Copy i of a quarter covers rows 2i, 2i + 1;
    // the 16 B chunk c of row r sits at position c ^ (r % 16), so the MFMA layout's reads (32 rows, one chunk)
    // spread over the banks. Every load of the epilogue is such a copy, so the explicit waits count them all.
    __syncthreads();  // every wave is done with the operand buffers
    char *wst = lds + wave * 32768;
    // the rows this epilogue loads: the residual x (unless it is already in the accumulators, FRONT) and x0
    // (mixing); one kind double buffered, two kinds side by side
    constexpr bool LOADX = !FRONT;
    constexpr int NLOAD = (LOADX ? 1 : 0) + (MIX ? 1 : 0);
    const float *xtile = p.xres + m * p.xr_m + (int64_t)(t0 + 32 * wave) * p.xr_t;
    const float *ztile = MIX ? p.x0 + m * p.x0_m + (int64_t)(t0 + 32 * wave) * p.x0_t : nullptr;
    auto issue_q = [&](int q) {
        const unsigned dst = lbase + wave * 32768 + (NLOAD == 2 ? 0 : (q & 1) * 16384);
        if constexpr (LOADX) issue_rows(xtile, p.xr_t, q, dst);
        if constexpr (MIX) issue_rows(ztile, p.x0_t, q, dst + (LOADX ? 16384 : 0));
    };
    if constexpr (NLOAD > 0) issue_q(0);
    if constexpr (NLOAD == 1) issue_q(1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if constexpr (NLOAD > 0) {
            if (NLOAD == 1 && q < 3) vm_wait<16>(); else vm_wait<0>();
            wave_lds_sync();
        }
        const char *xb = wst + (NLOAD == 2 ? 0 : (q & 1) * 16384) + jl * 512;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int rb = 4 * q + r4;
                const int c = 8 * r4 + 2 * b + hf;  // chunk of the quarter's row holding features 32 r4 + 8 b + 4 hf
                const int pos = (c ^ (jl & 15)) << 4;
                float4 xv{0.f, 0.f, 0.f, 0.f}, zv{0.f, 0.f, 0.f, 0.f};
                if constexpr (LOADX) xv = *reinterpret_cast<const float4 *>(xb + pos);
                if constexpr (MIX) zv = *reinterpret_cast<const float4 *>(xb + (LOADX ? 16384 : 0) + pos);
                const float4 a4 = ld4(apj + 32 * rb + 8 * b);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // FRONT: the accumulators already hold x_mid + the MLP product
                    float y = LOADX ? f4get(xv, e) + (out[rb][4 * b + e] + corr * f4get(a4, e))
                                    : out[rb][4 * b + e] + corr * f4get(a4, e);
                    if constexpr (MIX) y = rl * y + ml * f4get(zv, e);
                    out[rb][4 * b + e] = y;
                    ssq += y * y;
                }
            }
        if constexpr (NLOAD > 0) {
            wave_lds_sync();  // this quarter's reads are done before the next copies overwrite the buffer
            if (NLOAD == 2 ? q + 1 < 4 : q + 2 < 4) issue_q(NLOAD == 2 ? q + 1 : q + 2);
        }
    }
    ssq += swap_halves(ssq);
    const float rstd = rsqrtf(ssq * (1.0f / kEmb) + kNormEps);
#pragma unroll
    for (int k = 0; k < NNEXT; ++k) {
        const float *nb = reinterpret_cast<const float *>(lds + kNb + k * kEmb * 4) + 4 * hf;
        float d = 0.f;
#pragma unroll
        for (int rb = 0; rb < 16; ++rb)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float4 b4 = ld4(nb + 32 * rb + 8 * b);
#pragma unroll
                for (int e = 0; e < 4; ++e) d += out[rb][4 * b + e] * f4get(b4, e);
            }
        d += swap_halves(d);
        if (hf == 0) p.ndots[row * NNEXT + k] = rstd * d;
    }
    if constexpr (SPLIT3) {
        // the fp32 head's [hi | lo | hi] input, stored from the MFMA layout (the last block only)
        __bf16 *ho = p.hout + row * (3 * kEmb) + 4 * hf;
        if (xo) {
#pragma unroll
            for (int rb = 0; rb < 16; ++rb)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    st4(xo + 32 * rb + 8 * b, float4{out[rb][4 * b], out[rb][4 * b + 1], out[rb][4 * b + 2],
                                                     out[rb][4 * b + 3]});
        }
#pragma unroll
        for (int rb = 0; rb < 16; ++rb)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                bf16x4 hi, lo;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = out[rb][4 * b + e] * rstd;
                    hi[e] = (__bf16)v;
                    lo[e] = (__bf16)(v - (float)hi[e]);
                }
                const int f = 32 * rb + 8 * b;
                store_bf16x4(ho + f, hi);
                store_bf16x4(ho + kEmb + f, lo);
                store_bf16x4(ho + 2 * kEmb + f, hi);
            }
        return;
    }
    // xout and hout by whole-line stores: each quarter of the features (4 output blocks) is staged in the
    // wave's own part of the operand buffers, [32 tokens][128 + 4] fp32 and [32][128 + 8] bf16 (the pads put
    // consecutive rows 16 B apart in the banks), and stored back row by row
    float *sy = reinterpret_cast<float *>(lds + wave * 32768);
    __bf16 *sh = reinterpret_cast<__bf16 *>(lds + wave * 32768 + 32 * 132 * 4);
    float *xrow = xo ? xo - 4 * hf - jl * (int64_t)kEmb : nullptr;  // row of token t0 + 32 wave
    __bf16 *hrow = p.hout + (row - jl) * kEmb;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int rb = 4 * q + r4, f = 32 * r4 + 8 * b + 4 * hf;
                const float4 y4{out[rb][4 * b], out[rb][4 * b + 1], out[rb][4 * b + 2], out[rb][4 * b + 3]};
                if (xo) st4(sy + jl * 132 + f, y4);
                bf16x4 hv;
                hv[0] = (__bf16)(y4.x * rstd);
                hv[1] = (__bf16)(y4.y * rstd);
                hv[2] = (__bf16)(y4.z * rstd);
                hv[3] = (__bf16)(y4.w * rstd);
                store_bf16x4(sh + jl * 136 + f, hv);
            }
        wave_lds_sync();
        if (xo) {
#pragma unroll
            for (int it = 0; it < 16; ++it) {
                const int c = it * 64 + lane, r = c >> 5, ch = c & 31;
                st4(xrow + (int64_t)r * kEmb + 128 * q + 4 * ch, ld4(sy + r * 132 + 4 * ch));
            }
        }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int c = it * 64 + lane, r = c >> 4, ch = c & 15;
            store_bf16x8(hrow + (int64_t)r * kEmb + 128 * q + 8 * ch, load_bf16x8(sh + r * 136 + 8 * ch));
        }
        wave_lds_sync();  // the staging rows are rewritten by the next quarter
    }
}

// mlp.c_proj [rows][2048] -> the kernel's column order: within each 16 hidden units, the 4-wide groups
// (0, 1, 2, 3) are stored as (0, 2, 1, 3). One thread per 4-wide group.
__global__ __launch_bounds__(256) void mlp_proj_layout_kernel(const __bf16 *w, __bf16 *out, int64_t groups) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= groups) return;
    const int64_t q = i >> 2;   // 16-wide block
    const int g = (int)(i & 3);
    const int src = g == 1 ? 2 : g == 2 ? 1 : g;
    store_bf16x4(out + 4 * i, load_bf16x4(w + 16 * q + 4 * src));
}

template <bool MIX, int NNEXT, bool FRONT>
void launch_mlp_n(const MlpArgs &a, bool split3, dim3 grid, hipStream_t s) {
    if (split3)
        hipLaunchKernelGGL((mlp_kernel<MIX, NNEXT, true, FRONT>), grid, dim3(kMlpThreads), 0, s, a);
    else
        hipLaunchKernelGGL((mlp_kernel<MIX, NNEXT, false, FRONT>), grid, dim3(kMlpThreads), 0, s, a);
}

template <bool MIX, bool FRONT>
void launch_mlp(const MlpArgs &a, int nnext, bool split3, dim3 grid, hipStream_t s) {
    switch (nnext) {
        case 0: launch_mlp_n<MIX, 0, FRONT>(a, split3, grid, s); break;
        case 1: launch_mlp_n<MIX, 1, FRONT>(a, split3, grid, s); break;
        case 2: launch_mlp_n<MIX, 2, FRONT>(a, split3, grid, s); break;
        default: launch_mlp_n<MIX, 3, FRONT>(a, split3, grid, s); break;
    }
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_mlp_proj_layout(const void *w, void *out, int64_t rows, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(w && out && w != out && rows > 0 && aligned(w, 8) && aligned(out, 8),
                    "noise_mlp_proj_layout: bad arguments (distinct 8 B aligned buffers, rows > 0)");
    const int64_t groups = rows * kHid / 4;
    hipLaunchKernelGGL(mlp_proj_layout_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const __bf16 *)w, (__bf16 *)out, groups);
    return launch_status("noise_mlp_proj_layout");
}

namespace {

// Checks shared by both entry points and the MlpArgs they fill (dots_fc only without the projection in front).
int mlp_setup(const char *fn, const noise_population_t *pop, noise_view_t x, const void *w_fc, const noise_rank1_t *r_fc,
              const float *dots_fc, bool front, const void *w_proj, const noise_rank1_t *r_proj, noise_view_t xres,
              float *xout, int mix, const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x,
              int64_t eps_stride, noise_view_t x0, void *hout, const noise_rank1_t *next, int64_t nnext,
              float *next_dots, MlpArgs &a) {
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(pop->tokens % kTileTok == 0, "%s: tokens (%lld) must be a multiple of %d", fn,
                    (long long)pop->tokens, kTileTok);
    NOISE_CHECK_ARG(pop->members * pop->tokens < (1ll << 31), "%s: members * tokens must stay below 2^31", fn);
    NOISE_CHECK_ARG(pop->rounding == NOISE_ROUNDING_FUSED, "%s: fused rounding only (eager: noise_pop_fc + "
                    "noise_pop_residual)", fn);
    NOISE_CHECK_ARG(x.ptr && aligned(x.ptr, 16) && x.sm % 8 == 0 && x.st % 8 == 0, "%s: x misaligned", fn);
    NOISE_CHECK_ARG(w_fc && w_proj && aligned(w_fc, 16) && aligned(w_proj, 16), "%s: weights NULL or misaligned", fn);
    NOISE_CHECK_ARG(xres.ptr && aligned(xres.ptr, 16) && xres.sm % 4 == 0 && xres.st % 4 == 0, "%s: bad xres", fn);
    NOISE_CHECK_ARG(!xout || aligned(xout, 16), "%s: xout misaligned", fn);
    NOISE_CHECK_ARG(!mix || (x0.ptr && aligned(x0.ptr, 16) && x0.sm % 4 == 0 && x0.st % 4 == 0 && lam_r && lam_x),
                    "%s: mixing needs x0 and the mixing scalars", fn);
    NOISE_CHECK_ARG(!(eps_r || eps_x) || (mix && pop->sign), "%s: mixing-scalar noise needs mix and sign", fn);
    NOISE_CHECK_ARG(hout && aligned(hout, 8), "%s: hout NULL or misaligned", fn);
    NOISE_CHECK_ARG(nnext >= 0 && nnext <= 3 && (nnext == 0 || (next && next_dots)), "%s: bad next-dot request", fn);
    const bool pfc = r_fc && r_fc->a, ppj = r_proj && r_proj->a;
    if (front)
        NOISE_CHECK_ARG(!pfc || (pop->sign && r_fc->b && aligned(r_fc->a, 16) && aligned(r_fc->b, 16) &&
                                 r_fc->a_stride % 4 == 0 && r_fc->b_stride % 4 == 0),
                        "%s: c_fc noise needs sign and 16 B aligned a, b rows", fn);
    else
        NOISE_CHECK_ARG(!pfc || (dots_fc && pop->sign && aligned(r_fc->a, 16) && r_fc->a_stride % 4 == 0),
                        "%s: c_fc noise needs dots, sign and 16 B aligned a rows", fn);
    NOISE_CHECK_ARG(!ppj || (pop->sign && r_proj->b && aligned(r_proj->a, 16) && aligned(r_proj->b, 16) &&
                             r_proj->a_stride % 4 == 0 && r_proj->b_stride % 4 == 0),
                    "%s: mlp.c_proj noise needs sign and 16 B aligned a, b rows", fn);
    a = MlpArgs{};
    a.pop = MlpPop{(int)pop->members, (int)pop->tokens, pop->sign, (int)pop->dir_div};
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    a.wfc = (const __bf16 *)w_fc; a.wpj = (const __bf16 *)w_proj;
    a.afc = pfc ? r_fc->a : nullptr; a.afc_stride = pfc ? r_fc->a_stride : 0; a.dots_fc = front ? nullptr : dots_fc;
    a.bfc = front && pfc ? r_fc->b : nullptr; a.bfc_stride = front && pfc ? r_fc->b_stride : 0;
    a.apj = ppj ? r_proj->a : nullptr; a.bpj = ppj ? r_proj->b : nullptr;
    a.apj_stride = ppj ? r_proj->a_stride : 0; a.bpj_stride = ppj ? r_proj->b_stride : 0;
    a.xres = (const float *)xres.ptr; a.xr_m = xres.sm; a.xr_t = xres.st;
    a.xout = xout;
    a.lam_r = lam_r; a.lam_x = lam_x; a.eps_r = eps_r; a.eps_x = eps_x; a.eps_stride = eps_stride;
    a.x0 = (const float *)x0.ptr; a.x0_m = x0.sm; a.x0_t = x0.st;
    a.hout = (__bf16 *)hout;
    for (int k = 0; k < 3; ++k) {
        a.nb[k] = k < nnext ? next[k].b : nullptr;
        a.nb_stride[k] = k < nnext ? next[k].b_stride : 0;
        if (k < nnext)
            NOISE_CHECK_ARG(next[k].b && aligned(next[k].b, 16) && next[k].b_stride % 4 == 0,
                            "%s: next b %d NULL or misaligned", fn, k);
    }
    a.ndots = next_dots;
    return NOISE_OK;
}

}  // namespace

extern "C" int noise_pop_mlp(const noise_population_t *pop, noise_view_t x, const void *w_fc, const noise_rank1_t *r_fc,
                             const float *dots_fc, const void *w_proj, const noise_rank1_t *r_proj, noise_view_t xres,
                             float *xout, int mix, const float *lam_r, const float *lam_x, const float *eps_r,
                             const float *eps_x, int64_t eps_stride, noise_view_t x0, void *hout, int split3,
                             const noise_rank1_t *next, int64_t nnext, float *next_dots, noise_stream_t stream) {
    clear_error();
    MlpArgs a;
    const int st = mlp_setup("noise_pop_mlp", pop, x, w_fc, r_fc, dots_fc, false, w_proj, r_proj, xres, xout, mix, lam_r,
                             lam_x, eps_r, eps_x, eps_stride, x0, hout, next, nnext, next_dots, a);
    if (st != NOISE_OK) return st;
    const dim3 grid((unsigned)(pop->members * (pop->tokens / kTileTok)));
    if (mix)
        launch_mlp<true, false>(a, (int)nnext, split3 != 0, grid, (hipStream_t)stream);
    else
        launch_mlp<false, false>(a, (int)nnext, split3 != 0, grid, (hipStream_t)stream);
    return launch_status("noise_pop_mlp");
}

extern "C" int noise_pop_attn_mlp(const noise_population_t *pop, noise_view_t y, const void *w_o, const noise_rank1_t *r_o,
                                  const float *o_dots, int64_t o_dots_n, noise_view_t xres, const void *w_fc,
                                  const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj, float *xout,
                                  int mix, const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x,
                                  int64_t eps_stride, noise_view_t x0, void *hout, int split3, const noise_rank1_t *next,
                                  int64_t nnext, float *next_dots, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_attn_mlp";
    MlpArgs a;
    const int st = mlp_setup(fn, pop, y, w_fc, r_fc, nullptr, true, w_proj, r_proj, xres, xout, mix, lam_r, lam_x, eps_r,
                             eps_x, eps_stride, x0, hout, next, nnext, next_dots, a);
    if (st != NOISE_OK) return st;
    NOISE_CHECK_ARG(w_o && aligned(w_o, 16), "%s: w_o NULL or misaligned", fn);
    const bool po = r_o && r_o->a;
    NOISE_CHECK_ARG(!po || (pop->sign && o_dots && o_dots_n >= 1 && aligned(r_o->a, 16) && r_o->a_stride % 4 == 0),
                    "%s: attn.c_proj noise needs sign, dots and 16 B aligned a rows", fn);
    a.wo = (const __bf16 *)w_o;
    a.ao = po ? r_o->a : nullptr; a.ao_stride = po ? r_o->a_stride : 0;
    a.odots = po ? o_dots : nullptr; a.odots_n = po ? (int)o_dots_n : 0;
    const dim3 grid((unsigned)(pop->members * (pop->tokens / kTileTok)));
    if (mix)
        launch_mlp<true, true>(a, (int)nnext, split3 != 0, grid, (hipStream_t)stream);
    else
        launch_mlp<false, true>(a, (int)nnext, split3 != 0, grid, (hipStream_t)stream);
    return launch_status(fn);
}
