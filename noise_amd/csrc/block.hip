// The tail of a population block in one kernel, two waves per SIMD (eggroll.py:92-93, then the next block's
// mixing, norm and dots, eggroll.py:77-82 / 94):
//
//   x_mid = x + y W_o^T + sign (y . b_o) a_o                      attn.c_proj + residual      (never stored)
//   h     = bf16(norm(x_mid))                                                                  (never stored)
//   hid   = relu(h W_fc^T + sign (h . b_fc) a_fc)^2               mlp.c_fc, ReLU^2            (never stored)
//   y     = x_mid + hid W_proj^T + sign (hid . b_proj) a_proj     mlp.c_proj + residual
//   [y = rl y + ml x0]  ->  xout = y, hout = bf16(norm(y)), next_dots = norm(y) . b_next
//
// A workgroup owns 128 tokens of one member in 8 waves of 16 tokens, two waves per SIMD (about 250 registers
// each), on v_mfma_f32_16x16x32_bf16 with the weights as the A operand and the wave's tokens as the B operand:
//   - a wave's 16 token rows (y, then h) sit in registers as the B operand of every product (64 registers);
//   - its [512 outputs x 16 tokens] accumulate in 32 blocks of 16 x 16 (128 registers): x_mid, then x_mid plus
//     the MLP product;
//   - weights stream through LDS by direct global -> LDS copies of whole rows segments, double buffered:
//     W_o in 8 steps of 64 columns ([512 rows][128 B]), then 64 hidden steps of 32 units, each holding those
//     units' c_fc rows ([8 k tiles][32 rows][128 B]) and mlp.c_proj columns ([512 rows][64 B]); the 16 B chunks
//     of a row are XOR-swizzled by row so that a fragment read (16 rows, 4 consecutive chunks) is free of bank
//     conflicts: gfx950 serves a wave's ds_read_b128 in four passes of 16 lanes (lanes with equal bit 5 and
//     equal parity of bits 2..4, found with the LDS bank-conflict counter), each pass covering the 64 banks;
//   - the 16 x 16 D layout (lane l: token l % 16, rows 4 (l / 16) .. + 4) of two consecutive row blocks is the
//     B operand of one 32-deep k block once the k index is permuted within each 32 (lane group g holds rows
//     4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3): h goes from the x_mid accumulators into the first product's
//     operand, and the ReLU^2 of the first product's two blocks into the second product's, without leaving the
//     lane. c_fc and mlp.c_proj therefore come with their columns in that permuted order
//     (noise_block_weight_layout);
//   - a token's 512 features are spread over the four lanes l % 16 + 16 g: RMSNorm and the dots need two
//     exchanges (lane ^ 16, lane ^ 32).
// The second wave on each SIMD issues while the other waits on its fragment reads, its ReLU^2 or the barrier.
//
// noise_pop_block_qkv runs the next block's value-embedding gates and q/k/v (qkv_phase.hpp) after the tail in
// the same workgroup: h = bf16(norm(y)) goes from the accumulators into the phase's B operand in the permuted
// k order (c_q, c_k, c_v come permuted like c_fc), the next dots stay in registers as the phase's rank-1
// scales, and neither h nor the dots reach HBM; the phase's stage buffers reuse the step buffers once every
// wave has stored its residual rows.
#include "common.hpp"
#include "mfma.hpp"
#include "qkv_phase.hpp"
#include "tile.hpp"

namespace noise {
namespace {

constexpr float kBlkEps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps
constexpr int kBlkThreads = 512;   // 8 waves, two per SIMD
constexpr int kBlkTok = 128;       // tokens per workgroup (16 per wave)
constexpr int kHidden = 2048, kModel = 512;
constexpr int kUnits = 32;         // hidden units per step
constexpr int kSteps = kHidden / kUnits;
// fragment reads in flight ahead of the product that uses them; each product ends a scheduling region so that
// the compiler keeps them that far ahead (left to itself it moves each read next to its product)
#ifndef BLOCK_AHEAD
#define BLOCK_AHEAD 4
#endif
constexpr int kAhead = BLOCK_AHEAD;
#ifndef BLOCK_PIN
#define BLOCK_PIN() __builtin_amdgcn_sched_barrier(0)
#endif
constexpr int kBuf = 65536;        // a W_o step ([512 rows][128 B]); two per LDS
constexpr int kStage = 32768;      // an MLP stage (a step's c_fc rows or its mlp.c_proj columns); four per LDS
constexpr int kVec = 2 * kBuf;     // fp32 vectors after the two step buffers:
constexpr int kVAfc = kVec;                      // c_fc's a       [2048]
constexpr int kVBpj = kVAfc + kHidden * 4;       // mlp.c_proj's b [2048]
constexpr int kVApj = kVBpj + kHidden * 4;       // mlp.c_proj's a [512]
constexpr int kVNb = kVApj + kModel * 4;         // next b         [3][512]
constexpr int kVAo = kVNb + 3 * kModel * 4;      // attn.c_proj's a [512]
constexpr int kVBfc = kVAo + kModel * 4;         // c_fc's b       [512]
constexpr int kBlkLds = kVBfc + kModel * 4;      // 156 KiB
static_assert(kBlkLds <= 160 * 1024, "LDS of one CU");
// JIT (an unperturbed block with DUST's per-token jitter): the rank-1 vectors are not used, and the c_fc jitter of
// three steps ([128 tokens][32 units] bf16, 8 KiB each) rides in their place, copied with the c_fc stages
constexpr int kJitRing = kVAfc;
constexpr int kJitSlot = kBlkTok * kUnits * 2;
static_assert(kJitRing + 3 * kJitSlot <= kVAo, "the jitter ring overlaps the vectors the x_mid epilogue reads");
constexpr int kBlkQkvLds = kBlkLds > kQLds ? kBlkLds : kQLds;  // with the next block's q/k/v phase

struct BlockArgs {
    int members, tokens, dir_div;
    const float *sign;
    const __bf16 *y;                       // attention output, bf16 [m][T][512] (strided)
    int64_t ys_m, ys_t;
    const __bf16 *wo;                      // attn.c_proj [512][512]
    const float *ao;                       // its rank-1 a [dirs][512] or NULL
    int64_t ao_stride;
    const float *odots;                    // y . b_o partial sums [rows][odots_n]
    int odots_n;
    const float *xres;                     // block residual input fp32 (member stride may be 0)
    int64_t xr_m, xr_t;
    const __bf16 *wfc;                     // mlp.c_fc [2048][512], columns permuted
    const float *afc, *bfc;                // c_fc rank-1 a [dirs][2048], b [dirs][512] or NULL
    int64_t afc_stride, bfc_stride;
    const __bf16 *wpj;                     // mlp.c_proj [512][2048], columns permuted
    const float *apj, *bpj;                // mlp.c_proj rank-1 a [dirs][512], b [dirs][2048] or NULL
    int64_t apj_stride, bpj_stride;
    float *xout;                           // residual out [m][T][512] fp32, or NULL
    const float *lam_r, *lam_x;            // next block's mixing scalars (device)
    const float *eps_r, *eps_x;
    int64_t eps_stride;
    const float *x0;
    int64_t x0_m, x0_t;
    __bf16 *hout;                          // [m][T][512], or [m][T][1536] = [hi | lo | hi] with split3
    const float *nb[3];
    int64_t nb_stride[3];
    float *ndots;                          // [rows][NNEXT]
    QkvRowsArgs q;                         // the next block's q/k/v (QKV): its x is h, its dots come from the epilogue
    const __bf16 *jfc;                     // JIT: mlp.c_fc jitter bf16 [m * T][2048] (added before ReLU^2) or NULL
    const __bf16 *jmlp;                    // JIT: mlp.c_proj jitter bf16, row r at r * jmlp_st (added to its product)
    int64_t jmlp_st;                       //   512, or 0 with one zero row when the block has no mlp.c_proj jitter
};

// sum over the four lanes holding one token's features (l % 16 + 16 g)
__device__ __forceinline__ float token_sum(float v) { return sum_lanes_16_32(v); }

// QKV: 0, or the next block's q/k/v after the tail (1; 2 with its value embeddings) in place of the hout and
// next_dots stores
// JIT: the block unperturbed (no rank-1 terms) with DUST's jitter: 1 at mlp.c_fc (p.jfc, staged with the c_fc
// stages) and optionally mlp.c_proj (p.jmlp); 2 at mlp.c_proj only
template <bool MIX, int NNEXT, bool SPLIT3, int QKV, int JIT = 0>
__global__ __launch_bounds__(kBlkThreads, 1) void block_kernel(BlockArgs p) {
    static_assert(JIT == 0 || NNEXT == 0, "a jittered block is unperturbed: no next-matrix dots");
    constexpr bool kJit = JIT != 0, kJitFc = JIT == 1;
    __shared__ __attribute__((aligned(16))) char lds[QKV ? kBlkQkvLds : kBlkLds];
    const int T = p.tokens, tiles_t = T / kBlkTok;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * kBlkTok;
    const int tid = threadIdx.x, lane = tid & 63, tl = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dir = m / p.dir_div;
    const float sgn = p.sign ? p.sign[m] : 0.f;
    const int tok = t0 + 16 * wave + tl;
    const int64_t row = (int64_t)m * T + tok;
    const unsigned lbase = lds_addr(lds);
    // the next block's mixing scalars, read at entry so that the epilogue does not wait for them (wave-uniform)
    float rl = 0.f, ml = 0.f;
    if constexpr (MIX) {
        rl = *p.lam_r;
        ml = *p.lam_x;
        if (p.eps_r) rl += sgn * p.eps_r[dir * p.eps_stride];
        if (p.eps_x) ml += sgn * p.eps_x[dir * p.eps_stride];
        rl = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, rl)));
        ml = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, ml)));
    }

    // per-member vectors into LDS (zeros when a matrix is unperturbed, so no branches later), by direct copies of
    // 1 KiB per wave-wide copy that land with the rows below (a load, a wait and an LDS store per vector would be
    // one global round trip each)
    if constexpr (!kJit) {
        auto vcopy = [&](const float *src, int off, int n) {  // n a multiple of 256
            if (src) {
                for (int c = wave; c < n / 256; c += kBlkThreads / 64)
                    lds_dma16_at(src + 256 * c, (unsigned)(16 * lane), lbase + off + 1024 * c);
            } else {
                float *dst = reinterpret_cast<float *>(lds + off);
                for (int i = tid; i < n / 4; i += kBlkThreads) st4(dst + 4 * i, float4{0.f, 0.f, 0.f, 0.f});
            }
        };
        vcopy(p.afc ? p.afc + dir * p.afc_stride : nullptr, kVAfc, kHidden);
        vcopy(p.apj ? p.bpj + dir * p.bpj_stride : nullptr, kVBpj, kHidden);
        vcopy(p.apj ? p.apj + dir * p.apj_stride : nullptr, kVApj, kModel);
#pragma unroll
        for (int k = 0; k < NNEXT; ++k)
            vcopy(p.nb[k] ? p.nb[k] + dir * p.nb_stride[k] : nullptr, kVNb + k * kModel * 4, kModel);
        vcopy(p.ao ? p.ao + dir * p.ao_stride : nullptr, kVAo, kModel);
        vcopy(p.afc ? p.bfc + dir * p.bfc_stride : nullptr, kVBfc, kModel);
    }

    // LDS byte offset of 16 B chunk c of row r: in 128 B rows and in 64 B rows, chunks swizzled by row pair;
    // either way each 16-lane pass of a fragment read (rows r with 4 consecutive chunks) covers all banks once
    auto off128 = [](int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); };
    auto off64 = [](int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 3)) << 4); };
    // copies of whole 128 B row segments (8 rows per wave-wide copy) and of 64 B ones (16 rows)
    const int r8 = lane >> 3, p8 = lane & 7, r16 = lane >> 2, p16 = lane & 3;
    auto copy128 = [&](const __bf16 *rows, int64_t ld, int r0, unsigned dst) {  // rows r0 .. r0 + 7
        const int c = p8 ^ (((r0 + r8) >> 1) & 7);
        lds_dma16_at(rows + (int64_t)r0 * ld, (unsigned)(r8 * ld * 2 + c * 16), dst + r0 * 128);
    };
    auto copy64 = [&](const __bf16 *rows, int64_t ld, int r0, unsigned dst) {  // rows r0 .. r0 + 15
        const int c = p16 ^ (((r0 + r16) >> 1) & 3);
        lds_dma16_at(rows + (int64_t)r0 * ld, (unsigned)(r16 * ld * 2 + c * 16), dst + r0 * 64);
    };
    auto issue_o = [&](int s) {  // W_o columns 64 s .. + 64: [512 rows][128 B], 64 copies, 8 per wave
        const unsigned dst = lbase + (s & 1) * kBuf;
#pragma unroll
        for (int i = 0; i < 8; ++i) copy128(p.wo + 64 * s, kModel, 8 * (8 * wave + i), dst);
    };
    // the MLP's weights in 128 stages of 32 KiB through four stage buffers: stage 2 js holds the c_fc rows of
    // hidden units 32 js .. + 32 as [8 k tiles][32 rows][128 B] (wave w copies k tile w), stage 2 js + 1 their
    // mlp.c_proj columns as [512 rows][64 B] (wave w copies rows 64 w .. + 64); 4 copies per wave per stage
    auto issue_stage = [&](int k) {
        const unsigned dst = lbase + (k & 3) * kStage;
        const int js = k >> 1;
        if ((k & 1) == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                copy128(p.wfc + (int64_t)(kUnits * js) * kModel + 64 * wave, kModel, 8 * i, dst + wave * 4096);
            if constexpr (kJitFc) {
                // the step's c_fc jitter of this wave's 16 tokens: token row (lane / 4), 16 B chunk (lane % 4) of
                // its 32 units, into slot js % 3 of the ring as [16 tokens][64 B] (a fifth copy of this stage)
                const __bf16 *src = p.jfc + ((int64_t)m * T + t0 + 16 * wave) * kHidden + kUnits * js;
                lds_dma16_at(src, (unsigned)((lane >> 2) * kHidden * 2 + (lane & 3) * 16),
                             lbase + kJitRing + (js % 3) * kJitSlot + wave * 1024);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) copy64(p.wpj + kUnits * js, kHidden, 64 * wave + 16 * i, dst);
        }
    };
    const int fr = lane & 15, fc = lane >> 4;  // the row and chunk a lane reads in a fragment
    // A fragments: W_o rows 16 ob .. + 16, k block h of the step; c_fc rows 16 hb .. + 16 of k block kb;
    // mlp.c_proj rows 16 ob .. + 16
    auto frag_o = [&](const char *buf, int ob, int h) {
        return *reinterpret_cast<const bf16x8 *>(buf + off128(16 * ob + fr, 4 * h + fc));
    };
    auto frag_fc = [&](const char *buf, int hb, int kb) {
        return *reinterpret_cast<const bf16x8 *>(buf + (kb >> 1) * 4096 + off128(16 * hb + fr, 4 * (kb & 1) + fc));
    };
    auto frag_pj = [&](const char *buf, int ob) {
        return *reinterpret_cast<const bf16x8 *>(buf + off64(16 * ob + fr, fc));
    };

    issue_o(0);
    // this lane's y row: xf[kb] = y[tok][32 kb + 8 g .. + 8], the B operand of k block kb
    bf16x8 xf[16];
    {
        const __bf16 *yr = p.y + m * p.ys_m + (int64_t)tok * p.ys_t + 8 * g;
#pragma unroll
        for (int kb = 0; kb < 16; ++kb) xf[kb] = load_bf16x8(yr + 32 * kb);
    }
    // the products accumulate onto the residual rows (x_mid = x + y W_o^T + rank-1): their loads fly together
    // with the y rows and the first W_o step (block ob, register r holds feature 16 ob + 4 g + r)
    f32x4 out[32];
    {
        const float *xr = p.xres + m * p.xr_m + (int64_t)tok * p.xr_t + 4 * g;
#pragma unroll
        for (int ob = 0; ob < 32; ++ob) {
            const float4 v = ld4(xr + 16 * ob);
            out[ob] = f32x4{v.x, v.y, v.z, v.w};
        }
    }
    // y . b_o from the attention kernel's per-head partial sums, read with the rows (read after the MLP's first
    // copies, they would wait for those too)
    float osum = 0.f;
    if (p.ao)
        for (int k = 0; k < p.odots_n; ++k) osum += p.odots[row * p.odots_n + k];
    vm_wait<0>();
    __syncthreads();

    // ---- attn.c_proj: out[ob] = W_o[16 ob ..] . y^T in 8 steps of two k blocks (unrolled: xf is indexed by
    // the step)
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s + 1 < 8) issue_o(s + 1);  // its buffer was last read in step s - 1, before the barrier below
        const char *buf = lds + (s & 1) * kBuf;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            bf16x8 a[kAhead + 1];
#pragma unroll
            for (int i = 0; i < kAhead; ++i) a[i] = frag_o(buf, i, h);
#pragma unroll
            for (int ob = 0; ob < 32; ++ob) {
                if (ob + kAhead < 32) a[(ob + kAhead) % (kAhead + 1)] = frag_o(buf, ob + kAhead, h);
                out[ob] = mfma16x16x32(a[ob % (kAhead + 1)], xf[2 * s + h], out[ob]);
                BLOCK_PIN();
            }
        }
        vm_wait<0>();
        __syncthreads();
    }
    // all stage buffers are free: the first three MLP stages arrive during the epilogue below
    issue_stage(0);
    issue_stage(1);
    issue_stage(2);

    // ---- x_mid = (x + product) + sign (y . b_o) a_o; h = bf16(norm(x_mid)) into xf; c_fc's h . b from fp32
    float corr_fc = 0.f;
    {
        const float corr_o = sgn * osum;
        const float *ao = reinterpret_cast<const float *>(lds + kVAo) + 4 * g;
        float ssq = 0.f;
#pragma unroll
        for (int ob = 0; ob < 32; ++ob) {
            if constexpr (kJit) {
#pragma unroll
                for (int r = 0; r < 4; ++r) ssq += out[ob][r] * out[ob][r];
                continue;
            }
            const float4 a4 = ld4(ao + 16 * ob);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float v = out[ob][r] + corr_o * f4get(a4, r);
                out[ob][r] = v;
                ssq += v * v;
            }
        }
        const float rstd = rsqrtf(token_sum(ssq) * (1.0f / kModel) + kBlkEps);
        if (p.afc) {
            const float *bf = reinterpret_cast<const float *>(lds + kVBfc) + 4 * g;
            float d = 0.f;
#pragma unroll
            for (int ob = 0; ob < 32; ++ob) {
                const float4 b4 = ld4(bf + 16 * ob);
#pragma unroll
                for (int r = 0; r < 4; ++r) d += out[ob][r] * f4get(b4, r);
            }
            corr_fc = sgn * (rstd * token_sum(d));
        }
        // k block kb of the first product: features 32 kb + 4 g + (0..3) from block 2 kb, 32 kb + 16 + 4 g + (0..3)
        // from block 2 kb + 1 (c_fc's columns come in that order)
#pragma unroll
        for (int kb = 0; kb < 16; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                xf[kb][r] = (__bf16)(out[2 * kb][r] * rstd);
                xf[kb][4 + r] = (__bf16)(out[2 * kb + 1][r] * rstd);
            }
    }

    // ---- the MLP over 64 steps of 32 hidden units, accumulating onto x_mid
    float pd = 0.f;  // this lane's share of hid . b_proj
    const float *afc_l = reinterpret_cast<const float *>(lds + kVAfc) + 4 * g;
    const float *bpj_l = reinterpret_cast<const float *>(lds + kVBpj) + 4 * g;
    // stage 0 landed (stages 1 and 2 may still be in flight: 4 copies per wave each, 5 for a c_fc stage with JIT)
    vm_wait<kJitFc ? 9 : 8>();
    __syncthreads();
    constexpr int kStages = 2 * kSteps;
    // after stage k: stage k + 1 must have landed; the stages issued after it (up to k + 3) may still fly
    auto stage_end = [&](int k) {
        if constexpr (kJitFc) {
            // two stages in flight are one c_fc stage (5 copies) and one mlp.c_proj stage (4); one is the last,
            // an mlp.c_proj stage
            const int r = kStages - 2 - k;
            if (r >= 2)
                vm_wait<9>();
            else if (r == 1)
                vm_wait<4>();
            else
                vm_wait<0>();
        } else {
            vm_wait_groups<4, 2>(kStages - 2 - k < 2 ? kStages - 2 - k : 2);
        }
        __syncthreads();  // every wave's copies of stage k + 1 landed; every wave is done with buffer k & 3
    };
#pragma unroll 1
    for (int js = 0; js < kSteps; ++js) {
        // stage 2 js (c_fc rows): its buffer was last read in stage 2 js - 1 ... the copies of stage 2 js + 3 go
        // into the buffer of stage 2 js - 1, which every wave finished before the barrier that ended it
        if (2 * js + 3 < kStages) issue_stage(2 * js + 3);
        const char *buf;
        buf = lds + ((2 * js) & 3) * kStage;
        // first product: hacc[hb] = c_fc rows 32 js + 16 hb .. + 16 against the 16 k blocks of h
        f32x4 hacc[2] = {f32x4{}, f32x4{}};
        {
            bf16x8 a[kAhead + 1];
#pragma unroll
            for (int i = 0; i < kAhead; ++i) a[i] = frag_fc(buf, i & 1, i >> 1);
#pragma unroll
            for (int f = 0; f < 32; ++f) {
                if (f + kAhead < 32) a[(f + kAhead) % (kAhead + 1)] = frag_fc(buf, (f + kAhead) & 1, (f + kAhead) >> 1);
                hacc[f & 1] = mfma16x16x32(a[f % (kAhead + 1)], xf[f >> 1], hacc[f & 1]);
                BLOCK_PIN();
            }
        }
        stage_end(2 * js);
        // stage 2 js + 1 (mlp.c_proj columns)
        if (2 * js + 4 < kStages) issue_stage(2 * js + 4);
        buf = lds + ((2 * js + 1) & 3) * kStage;
        // ReLU^2 with the rank-1 term, bf16, packed as the second product's B operand (k = 8 g + j holds hidden unit
        // 4 g + j of block 0 for j < 4, of block 1 for j >= 4); this lane's share of hid . b_proj
        bf16x8 hb;
        if constexpr (kJit) {
            // the c_fc jitter of this lane's token (units 4 g .. + 3 of each 16-unit block), then ReLU^2
            bf16x4 j0, j1;
            if constexpr (kJitFc) {
                const char *jr = lds + kJitRing + (js % 3) * kJitSlot + (16 * wave + tl) * 64 + 8 * g;
                j0 = *reinterpret_cast<const bf16x4 *>(jr);
                j1 = *reinterpret_cast<const bf16x4 *>(jr + 32);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) j0[r] = j1[r] = (__bf16)0.0f;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v0 = fmaxf(hacc[0][r] + (float)j0[r], 0.f);
                float v1 = fmaxf(hacc[1][r] + (float)j1[r], 0.f);
                hb[r] = (__bf16)(v0 * v0);
                hb[4 + r] = (__bf16)(v1 * v1);
            }
        } else {
            const float4 a0 = ld4(afc_l + kUnits * js), a1 = ld4(afc_l + kUnits * js + 16);
            const float4 b0 = ld4(bpj_l + kUnits * js), b1 = ld4(bpj_l + kUnits * js + 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v0 = fmaxf(hacc[0][r] + corr_fc * f4get(a0, r), 0.f);
                float v1 = fmaxf(hacc[1][r] + corr_fc * f4get(a1, r), 0.f);
                hb[r] = (__bf16)(v0 * v0);
                hb[4 + r] = (__bf16)(v1 * v1);
            }
            // hid . b with both in bf16, as the reference's autocast x @ b (eggroll.py:58) multiplies them
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
                pd = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{hb[r], hb[r + 1]},
                                                     bf16x2{(__bf16)f4get(b0, r), (__bf16)f4get(b0, r + 1)}, pd, false);
                pd = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{hb[4 + r], hb[5 + r]},
                                                     bf16x2{(__bf16)f4get(b1, r), (__bf16)f4get(b1, r + 1)}, pd, false);
            }
        }
        // second product: out[ob] += mlp.c_proj rows 16 ob .. + 16, columns of this step
        {
            bf16x8 a[kAhead + 1];
#pragma unroll
            for (int i = 0; i < kAhead; ++i) a[i] = frag_pj(buf, i);
#pragma unroll
            for (int ob = 0; ob < 32; ++ob) {
                if (ob + kAhead < 32) a[(ob + kAhead) % (kAhead + 1)] = frag_pj(buf, ob + kAhead);
                out[ob] = mfma16x16x32(a[ob % (kAhead + 1)], hb, out[ob]);
                BLOCK_PIN();
            }
        }
        stage_end(2 * js + 1);
    }

    // ---- epilogue: y = out + sign (hid . b_proj) a_proj [, mixing], RMSNorm, next dots, stores
    // QKV: the next block's per-token scalars (rotary rows, value-table row) in flight under the epilogue
    QkvLane L;
    if constexpr (QKV != 0) {
        L.m = m; L.t0 = t0; L.tok = tok; L.wave = wave; L.lane = lane; L.tid = tid; L.dir = dir; L.row = row;
        L.sgn = sgn;
        qkv_token_scalars<QKV == 2>(p.q, L);
    }
    const float corr = p.apj ? sgn * token_sum(pd) : 0.f;
    float ssq = 0.f;
    {
        const float *apj = reinterpret_cast<const float *>(lds + kVApj) + 4 * g;
        const float *zr = MIX ? p.x0 + m * p.x0_m + (int64_t)tok * p.x0_t + 4 * g : nullptr;
        const __bf16 *jr = kJit ? p.jmlp + row * p.jmlp_st + 4 * g : nullptr;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float4 zv[8];
            if constexpr (MIX) {
#pragma unroll
                for (int i = 0; i < 8; ++i) zv[i] = ld4(zr + 16 * (8 * q + i));
            }
            bf16x4 jv[8];
            if constexpr (kJit) {
#pragma unroll
                for (int i = 0; i < 8; ++i) jv[i] = load_bf16x4(jr + 16 * (8 * q + i));
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int ob = 8 * q + i;
                const float4 a4 = kJit ? float4{0.f, 0.f, 0.f, 0.f} : ld4(apj + 16 * ob);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // with JIT: the block's mlp.c_proj product plus its jitter (the rank-1 terms are off)
                    float v = kJit ? out[ob][r] + (float)jv[i][r] : out[ob][r] + corr * f4get(a4, r);
                    if constexpr (MIX) v = rl * v + ml * f4get(zv[i], r);
                    out[ob][r] = v;
                    ssq += v * v;
                }
            }
            // with JIT, one chunk's x0 and jitter rows at a time: hoisting all four chunks' loads spills
            if constexpr (kJit) __builtin_amdgcn_sched_barrier(0);
        }
    }
    const float rstd = rsqrtf(token_sum(ssq) * (1.0f / kModel) + kBlkEps);
    float dq[3] = {0.f, 0.f, 0.f};  // QKV: sign * (h . b) of the next c_q, c_k, c_v from the fp32 norm
#pragma unroll
    for (int k = 0; k < NNEXT; ++k) {
        const float *nb = reinterpret_cast<const float *>(lds + kVNb + k * kModel * 4) + 4 * g;
        float d = 0.f;
#pragma unroll
        for (int ob = 0; ob < 32; ++ob) {
            const float4 b4 = ld4(nb + 16 * ob);
#pragma unroll
            for (int r = 0; r < 4; ++r) d += out[ob][r] * f4get(b4, r);
        }
        d = token_sum(d);
        if constexpr (QKV != 0)
            dq[k] = p.q.a[k] ? sgn * (rstd * d) : 0.f;
        else if (g == 0)
            p.ndots[row * NNEXT + k] = rstd * d;
    }
    // whole-line stores through the wave's 16 KiB of the (free) step buffers: rows of 1 KiB, 16 B chunk c of
    // row t at position c ^ t
    char *stg = lds + wave * 16384;
    const int64_t row0 = (int64_t)m * T + t0 + 16 * wave;  // the wave's first token row
    if (p.xout) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ob = 16 * half + i, c = 4 * i + g;
                st4(reinterpret_cast<float *>(stg + tl * 1024 + ((c ^ tl) << 4)),
                    float4{out[ob][0], out[ob][1], out[ob][2], out[ob][3]});
            }
            wave_lds_sync();
#pragma unroll
            for (int it = 0; it < 16; ++it)
                st4_nt(p.xout + (row0 + it) * kModel + 256 * half + 4 * lane,
                    *reinterpret_cast<const float4 *>(stg + it * 1024 + ((lane ^ it) << 4)));
            wave_lds_sync();  // the staging rows are rewritten next
        }
    }
    if constexpr (QKV != 0) {
        // the next block's q/k/v from h = bf16(norm(y)), packed as the B operand in the permuted k order (c_q, c_k
        // and c_v come with their columns permuted as c_fc's)
#pragma unroll
        for (int kb = 0; kb < 16; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                xf[kb][r] = (__bf16)(out[2 * kb][r] * rstd);
                xf[kb][4 + r] = (__bf16)(out[2 * kb + 1][r] * rstd);
            }
        __syncthreads();  // every wave has read back its staged rows: the stage buffers are free
#pragma unroll
        for (int k = 0; k < 3; ++k) qkv_issue(p.q, lbase, wave, lane, k);
        L.dq0 = dq[0]; L.dq1 = dq[1]; L.dq2 = dq[2];
        vm_wait<0>();  // the three stages and the scalars landed
        __syncthreads();
        qkv_phase<QKV == 2, true>(p.q, lds, xf, L);
        return;
    }
    // bf16 rows (hi, and lo for the split3 head input): 1 KiB rows, 16 B chunk c of row t at c ^ t
    const int width = SPLIT3 ? 3 * kModel : kModel;
#pragma unroll
    for (int part = 0; part < (SPLIT3 ? 2 : 1); ++part) {
#pragma unroll
        for (int ob = 0; ob < 32; ++ob) {
            bf16x4 v;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float h = out[ob][r] * rstd;
                const __bf16 hi = (__bf16)h;
                v[r] = part == 0 ? hi : (__bf16)(h - (float)hi);
            }
            const int c16 = 2 * ob + (g >> 1);
            store_bf16x4(reinterpret_cast<__bf16 *>(stg + tl * 1024 + ((c16 ^ tl) << 4) + 8 * (g & 1)), v);
        }
        wave_lds_sync();
#pragma unroll
        for (int it = 0; it < 16; ++it) {
            const bf16x8 v = *reinterpret_cast<const bf16x8 *>(stg + it * 1024 + ((lane ^ it) << 4));
            __bf16 *dst = p.hout + (row0 + it) * width + 8 * lane;
            if (part == 0) {
                store_bf16x8(dst, v);
                if constexpr (SPLIT3) store_bf16x8(dst + 2 * kModel, v);
            } else {
                store_bf16x8(dst + kModel, v);
            }
        }
        wave_lds_sync();
    }
}

// w [rows][cols] bf16 -> the column order block_kernel reads: within every 32 columns, position 8 g + j holds
// column 4 g + j (j < 4) or 16 + 4 g + (j - 4) (j >= 4). One thread per 4-wide group.
__global__ __launch_bounds__(256) void block_layout_kernel(const __bf16 *w, __bf16 *out, int64_t groups) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= groups) return;
    const int64_t q = i >> 3;        // 32-wide block
    const int pos = (int)(i & 7);    // 4-wide group at positions 4 pos .. 4 pos + 3
    const int gq = pos >> 1, hi = pos & 1;
    const int src = hi ? 4 + gq : gq;  // source 4-wide group within the 32
    store_bf16x4(out + 4 * i, load_bf16x4(w + 32 * q + 4 * src));
}

template <bool MIX, int NNEXT>
void launch_block_n(const BlockArgs &a, bool split3, dim3 grid, hipStream_t s) {
    if (split3)
        hipLaunchKernelGGL((block_kernel<MIX, NNEXT, true, 0>), grid, dim3(kBlkThreads), 0, s, a);
    else
        hipLaunchKernelGGL((block_kernel<MIX, NNEXT, false, 0>), grid, dim3(kBlkThreads), 0, s, a);
}

template <bool MIX>
void launch_block(const BlockArgs &a, int nnext, bool split3, dim3 grid, hipStream_t s) {
    switch (nnext) {
        case 0: launch_block_n<MIX, 0>(a, split3, grid, s); break;
        case 1: launch_block_n<MIX, 1>(a, split3, grid, s); break;
        case 2: launch_block_n<MIX, 2>(a, split3, grid, s); break;
        default: launch_block_n<MIX, 3>(a, split3, grid, s); break;
    }
}

// with the next block's q/k/v: its dots for all three matrices or none
template <bool MIX, int NNEXT>
void launch_block_qkv_n(const BlockArgs &a, bool ve, dim3 grid, hipStream_t s) {
    if (ve)
        hipLaunchKernelGGL((block_kernel<MIX, NNEXT, false, 2>), grid, dim3(kBlkThreads), 0, s, a);
    else
        hipLaunchKernelGGL((block_kernel<MIX, NNEXT, false, 1>), grid, dim3(kBlkThreads), 0, s, a);
}

template <bool MIX>
void launch_block_qkv(const BlockArgs &a, int nnext, bool ve, dim3 grid, hipStream_t s) {
    if (nnext)
        launch_block_qkv_n<MIX, 3>(a, ve, grid, s);
    else
        launch_block_qkv_n<MIX, 0>(a, ve, grid, s);
}

// the jittered (unperturbed) block: the last block before the fp32 head (no mixing, split3 head input), or a
// block followed by the next block's q/k/v with or without its value embeddings (with the next mixing)
template <int JIT>
bool launch_block_jit_n(const BlockArgs &a, bool mix, bool split3, int qkv, dim3 grid, hipStream_t s) {
    if (qkv == 0 && !mix && split3)
        hipLaunchKernelGGL((block_kernel<false, 0, true, 0, JIT>), grid, dim3(kBlkThreads), 0, s, a);
    else if (qkv == 1 && mix)
        hipLaunchKernelGGL((block_kernel<true, 0, false, 1, JIT>), grid, dim3(kBlkThreads), 0, s, a);
    else if (qkv == 2 && mix)
        hipLaunchKernelGGL((block_kernel<true, 0, false, 2, JIT>), grid, dim3(kBlkThreads), 0, s, a);
    else
        return false;
    return true;
}

int launch_block_jit(const char *fn, const BlockArgs &a, bool mix, bool split3, int qkv, dim3 grid, hipStream_t s) {
    const bool ok = a.jfc ? launch_block_jit_n<1>(a, mix, split3, qkv, grid, s)
                          : launch_block_jit_n<2>(a, mix, split3, qkv, grid, s);
    if (!ok)
        NOISE_CHECK_ARG(false, "%s: jitter is served for the last block with the split3 head input and no mixing, "
                               "or for a block followed by the next block's q/k/v with its mixing", fn);
    return launch_status(fn);
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_block_weight_layout(const void *w, void *out, int64_t rows, int64_t cols, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(w && out && w != out && rows > 0 && cols > 0 && cols % 32 == 0 && aligned(w, 8) && aligned(out, 8),
                    "noise_block_weight_layout: distinct 8 B aligned buffers, rows > 0, cols a multiple of 32");
    const int64_t groups = rows * cols / 4;
    hipLaunchKernelGGL(block_layout_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const __bf16 *)w, (__bf16 *)out, groups);
    return launch_status("noise_block_weight_layout");
}

namespace noise {
namespace {

// checks and arguments of the block's tail, shared by the two block entry points
int block_args(const char *fn, BlockArgs &a, const noise_population_t *pop, noise_view_t y, const void *w_o,
               const noise_rank1_t *r_o, const float *o_dots, int64_t o_dots_n, noise_view_t xres, const void *w_fc,
               const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj, float *xout, int mix,
               const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x, int64_t eps_stride,
               noise_view_t x0, const noise_rank1_t *next, int64_t nnext) {
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(pop->tokens % kBlkTok == 0, "%s: tokens (%lld) must be a multiple of %d", fn,
                    (long long)pop->tokens, kBlkTok);
    NOISE_CHECK_ARG(pop->members * pop->tokens < (1ll << 31), "%s: members * tokens must stay below 2^31", fn);
    NOISE_CHECK_ARG(pop->rounding == NOISE_ROUNDING_FUSED, "%s: fused rounding only", fn);
    NOISE_CHECK_ARG(y.ptr && aligned(y.ptr, 16) && y.sm % 8 == 0 && y.st % 8 == 0, "%s: y misaligned", fn);
    NOISE_CHECK_ARG(w_o && w_fc && w_proj && aligned(w_o, 16) && aligned(w_fc, 16) && aligned(w_proj, 16),
                    "%s: weights NULL or misaligned", fn);
    NOISE_CHECK_ARG(xres.ptr && aligned(xres.ptr, 16) && xres.sm % 4 == 0 && xres.st % 4 == 0, "%s: bad xres", fn);
    NOISE_CHECK_ARG(!xout || aligned(xout, 16), "%s: xout misaligned", fn);
    NOISE_CHECK_ARG(!mix || (x0.ptr && aligned(x0.ptr, 16) && x0.sm % 4 == 0 && x0.st % 4 == 0 && lam_r && lam_x),
                    "%s: mixing needs x0 and the mixing scalars", fn);
    NOISE_CHECK_ARG(!(eps_r || eps_x) || (mix && pop->sign), "%s: mixing-scalar noise needs mix and sign", fn);
    NOISE_CHECK_ARG(nnext >= 0 && nnext <= 3 && (nnext == 0 || next), "%s: bad next-dot request", fn);
    const bool po = r_o && r_o->a, pfc = r_fc && r_fc->a, ppj = r_proj && r_proj->a;
    NOISE_CHECK_ARG(!po || (pop->sign && o_dots && o_dots_n >= 1 && aligned(r_o->a, 16) && r_o->a_stride % 4 == 0),
                    "%s: attn.c_proj noise needs sign, dots and 16 B aligned a rows", fn);
    NOISE_CHECK_ARG(!pfc || (pop->sign && r_fc->b && aligned(r_fc->a, 16) && aligned(r_fc->b, 16) &&
                             r_fc->a_stride % 4 == 0 && r_fc->b_stride % 4 == 0),
                    "%s: c_fc noise needs sign and 16 B aligned a, b rows", fn);
    NOISE_CHECK_ARG(!ppj || (pop->sign && r_proj->b && aligned(r_proj->a, 16) && aligned(r_proj->b, 16) &&
                             r_proj->a_stride % 4 == 0 && r_proj->b_stride % 4 == 0),
                    "%s: mlp.c_proj noise needs sign and 16 B aligned a, b rows", fn);
    a = BlockArgs{};
    a.members = (int)pop->members; a.tokens = (int)pop->tokens; a.dir_div = (int)pop->dir_div; a.sign = pop->sign;
    a.y = (const __bf16 *)y.ptr; a.ys_m = y.sm; a.ys_t = y.st;
    a.wo = (const __bf16 *)w_o;
    a.ao = po ? r_o->a : nullptr; a.ao_stride = po ? r_o->a_stride : 0;
    a.odots = po ? o_dots : nullptr; a.odots_n = po ? (int)o_dots_n : 0;
    a.xres = (const float *)xres.ptr; a.xr_m = xres.sm; a.xr_t = xres.st;
    a.wfc = (const __bf16 *)w_fc;
    a.afc = pfc ? r_fc->a : nullptr; a.bfc = pfc ? r_fc->b : nullptr;
    a.afc_stride = pfc ? r_fc->a_stride : 0; a.bfc_stride = pfc ? r_fc->b_stride : 0;
    a.wpj = (const __bf16 *)w_proj;
    a.apj = ppj ? r_proj->a : nullptr; a.bpj = ppj ? r_proj->b : nullptr;
    a.apj_stride = ppj ? r_proj->a_stride : 0; a.bpj_stride = ppj ? r_proj->b_stride : 0;
    a.xout = xout;
    a.lam_r = lam_r; a.lam_x = lam_x; a.eps_r = eps_r; a.eps_x = eps_x; a.eps_stride = eps_stride;
    a.x0 = (const float *)x0.ptr; a.x0_m = x0.sm; a.x0_t = x0.st;
    for (int k = 0; k < 3; ++k) {
        a.nb[k] = k < nnext ? next[k].b : nullptr;
        a.nb_stride[k] = k < nnext ? next[k].b_stride : 0;
        if (k < nnext)
            NOISE_CHECK_ARG(next[k].b && aligned(next[k].b, 16) && next[k].b_stride % 4 == 0,
                            "%s: next b %d NULL or misaligned", fn, k);
    }
    return NOISE_OK;
}

}  // namespace
}  // namespace noise

namespace noise {
namespace {

// the jitter of a jittered block: the block must be unperturbed (DUST's block_forward, run.py:102-117); the
// rows are [members * tokens][2048] (mlp.c_fc) and [members * tokens][512] (mlp.c_proj), bf16, 16 B aligned
int block_jitter(const char *fn, BlockArgs &a, const noise_block_jitter_t *jit) {
    NOISE_CHECK_ARG(jit && (jit->fc || jit->mlp), "%s: jitter NULL or empty", fn);
    NOISE_CHECK_ARG(!a.ao && !a.afc && !a.apj && !a.eps_r && !a.eps_x && !a.nb[0] && !a.nb[1] && !a.nb[2],
                    "%s: a jittered block takes no rank-1 or mixing-scalar noise", fn);
    NOISE_CHECK_ARG((!jit->fc || aligned(jit->fc, 16)) && (!jit->mlp || aligned(jit->mlp, 16)),
                    "%s: jitter rows must be 16 B aligned", fn);
    // no mlp.c_proj jitter: every row reads one zero row (the kernel's epilogue loads unconditionally)
    a.jmlp = (const __bf16 *)jit->mlp;
    a.jmlp_st = kModel;
    if (!a.jmlp) {
        NOISE_CHECK_ARG(jit->zero_row && aligned(jit->zero_row, 16), "%s: without mlp jitter a 512-element zero row "
                        "(bf16, 16 B aligned) must be given", fn);
        a.jmlp = (const __bf16 *)jit->zero_row;
        a.jmlp_st = 0;
    }
    a.jfc = (const __bf16 *)jit->fc;   // each workgroup copies only its own token rows of it
    return NOISE_OK;
}

int pop_block_impl(const char *fn, const noise_population_t *pop, noise_view_t y, const void *w_o,
                   const noise_rank1_t *r_o, const float *o_dots, int64_t o_dots_n, noise_view_t xres,
                   const void *w_fc, const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj,
                   float *xout, int mix, const float *lam_r, const float *lam_x, const float *eps_r,
                   const float *eps_x, int64_t eps_stride, noise_view_t x0, void *hout, int split3,
                   const noise_rank1_t *next, int64_t nnext, float *next_dots, const noise_block_jitter_t *jit,
                   noise_stream_t stream) {
    BlockArgs a;
    const int st = block_args(fn, a, pop, y, w_o, r_o, o_dots, o_dots_n, xres, w_fc, r_fc, w_proj, r_proj, xout, mix,
                              lam_r, lam_x, eps_r, eps_x, eps_stride, x0, next, nnext);
    if (st != NOISE_OK) return st;
    NOISE_CHECK_ARG(hout && aligned(hout, 16), "%s: hout NULL or misaligned", fn);
    NOISE_CHECK_ARG(nnext == 0 || next_dots, "%s: next dots need an output", fn);
    a.hout = (__bf16 *)hout;
    a.ndots = next_dots;
    const dim3 grid((unsigned)(pop->members * (pop->tokens / kBlkTok)));
    if (jit) {
        const int js = block_jitter(fn, a, jit);
        if (js != NOISE_OK) return js;
        return launch_block_jit(fn, a, mix != 0, split3 != 0, 0, grid, (hipStream_t)stream);
    }
    if (mix)
        launch_block<true>(a, (int)nnext, split3 != 0, grid, (hipStream_t)stream);
    else
        launch_block<false>(a, (int)nnext, split3 != 0, grid, (hipStream_t)stream);
    return launch_status(fn);
}

int pop_block_qkv_impl(const char *fn, const noise_population_t *pop, noise_view_t y, const void *w_o,
                       const noise_rank1_t *r_o, const float *o_dots, int64_t o_dots_n, noise_view_t xres,
                       const void *w_fc, const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj,
                       float *xout, int mix, const float *lam_r, const float *lam_x, const float *eps_r,
                       const float *eps_x, int64_t eps_stride, noise_view_t x0, const void *const w_qkv[3],
                       const noise_rank1_t r_qkv[3], const void *rope_cos, const void *rope_sin, const float *ve,
                       int64_t vocab, const int64_t *idx, int64_t idx_sm, const float *gate_w,
                       const noise_rank1_t *gate_noise, const noise_rank1_t *ve_noise, void *const out[3],
                       const noise_block_jitter_t *jit, noise_stream_t stream) {
    const bool pq = r_qkv && (r_qkv[0].a || r_qkv[1].a || r_qkv[2].a);
    BlockArgs a;
    const int st = block_args(fn, a, pop, y, w_o, r_o, o_dots, o_dots_n, xres, w_fc, r_fc, w_proj, r_proj, xout, mix,
                              lam_r, lam_x, eps_r, eps_x, eps_stride, x0, nullptr, 0);
    if (st != NOISE_OK) return st;
    NOISE_CHECK_ARG(xout, "%s: xout (the next block's residual) must not be NULL", fn);
    // the dots of the perturbed matrices (an unperturbed one's b reads as zeros)
    for (int k = 0; k < 3 && pq; ++k) {
        if (!r_qkv[k].a) continue;
        NOISE_CHECK_ARG(r_qkv[k].b && aligned(r_qkv[k].b, 16) && r_qkv[k].b_stride % 4 == 0,
                        "%s: q/k/v noise b %d NULL or misaligned", fn, k);
        a.nb[k] = r_qkv[k].b;
        a.nb_stride[k] = r_qkv[k].b_stride;
    }
    NOISE_CHECK_ARG(w_qkv && out && rope_cos && rope_sin && aligned(rope_cos, 16) && aligned(rope_sin, 16),
                    "%s: NULL q/k/v weight or output array, or rotary tables not 16 B aligned", fn);
    for (int i = 0; i < 3; ++i) {
        NOISE_CHECK_ARG(w_qkv[i] && out[i] && aligned(w_qkv[i], 16) && aligned(out[i], 16),
                        "%s: q/k/v weight or output %d NULL or not 16 B aligned", fn, i);
        NOISE_CHECK_ARG(!pq || !r_qkv[i].a || (pop->sign && aligned(r_qkv[i].a, 16) && r_qkv[i].a_stride % 4 == 0),
                        "%s: perturbed matrix %d needs sign and 16 B aligned a rows", fn, i);
    }
    NOISE_CHECK_ARG(!ve || (idx && gate_w && vocab > 0), "%s: value embeddings need idx, gate weights and vocab", fn);
    NOISE_CHECK_ARG(idx_sm == 0 || idx_sm >= pop->tokens, "%s: idx_sm must be 0 or >= tokens", fn);
    const bool gn = ve && gate_noise && gate_noise->a;
    NOISE_CHECK_ARG(!gn || (pop->sign && gate_noise->b), "%s: gate noise needs sign and b", fn);
    const bool vn = ve && ve_noise && ve_noise->a;
    NOISE_CHECK_ARG(!vn || (pop->sign && ve_noise->b && aligned(ve_noise->b, 16) && ve_noise->b_stride % 4 == 0),
                    "%s: value-embedding noise needs sign and 16 B aligned b rows", fn);
    a.q = qkv_rows_args(pop, noise_view_t{nullptr, 0, 0}, w_qkv, r_qkv, nullptr, rope_cos, rope_sin, ve, vocab, idx,
                        idx_sm, nullptr, ve_noise, out);
    a.q.gate_w = gate_w;
    a.q.gate_a = gn ? gate_noise->a : nullptr; a.q.gate_b = gn ? gate_noise->b : nullptr;
    a.q.gate_a_stride = gn ? gate_noise->a_stride : 0; a.q.gate_b_stride = gn ? gate_noise->b_stride : 0;
    const dim3 grid((unsigned)(pop->members * (pop->tokens / kBlkTok)));
    if (jit) {
        NOISE_CHECK_ARG(!pq && !gn && !vn, "%s: a jittered block's next q/k/v take no noise", fn);
        const int js = block_jitter(fn, a, jit);
        if (js != NOISE_OK) return js;
        return launch_block_jit(fn, a, mix != 0, false, ve ? 2 : 1, grid, (hipStream_t)stream);
    }
    if (mix)
        launch_block_qkv<true>(a, pq ? 3 : 0, ve != nullptr, grid, (hipStream_t)stream);
    else
        launch_block_qkv<false>(a, pq ? 3 : 0, ve != nullptr, grid, (hipStream_t)stream);
    return launch_status(fn);
}

}  // namespace
}  // namespace noise

extern "C" int noise_pop_block(const noise_population_t *pop, noise_view_t y, const void *w_o, const noise_rank1_t *r_o,
                               const float *o_dots, int64_t o_dots_n, noise_view_t xres, const void *w_fc,
                               const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj, float *xout,
                               int mix, const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x,
                               int64_t eps_stride, noise_view_t x0, void *hout, int split3, const noise_rank1_t *next,
                               int64_t nnext, float *next_dots, noise_stream_t stream) {
    clear_error();
    return pop_block_impl("noise_pop_block", pop, y, w_o, r_o, o_dots, o_dots_n, xres, w_fc, r_fc, w_proj, r_proj,
                          xout, mix, lam_r, lam_x, eps_r, eps_x, eps_stride, x0, hout, split3, next, nnext, next_dots,
                          nullptr, stream);
}

extern "C" int noise_pop_block_jit(const noise_population_t *pop, noise_view_t y, const void *w_o, noise_view_t xres,
                                   const void *w_fc, const void *w_proj, int mix, const float *lam_r,
                                   const float *lam_x, noise_view_t x0, void *hout, int split3,
                                   const noise_block_jitter_t *jit, noise_stream_t stream) {
    clear_error();
    return pop_block_impl("noise_pop_block_jit", pop, y, w_o, nullptr, nullptr, 0, xres, w_fc, nullptr, w_proj,
                          nullptr, nullptr, mix, lam_r, lam_x, nullptr, nullptr, 0, x0, hout, split3, nullptr, 0,
                          nullptr, jit, stream);
}

extern "C" int noise_pop_block_qkv(const noise_population_t *pop, noise_view_t y, const void *w_o,
                                   const noise_rank1_t *r_o, const float *o_dots, int64_t o_dots_n, noise_view_t xres,
                                   const void *w_fc, const noise_rank1_t *r_fc, const void *w_proj,
                                   const noise_rank1_t *r_proj, float *xout, int mix, const float *lam_r,
                                   const float *lam_x, const float *eps_r, const float *eps_x, int64_t eps_stride,
                                   noise_view_t x0, const void *const w_qkv[3], const noise_rank1_t r_qkv[3],
                                   const void *rope_cos, const void *rope_sin, const float *ve, int64_t vocab,
                                   const int64_t *idx, int64_t idx_sm, const float *gate_w,
                                   const noise_rank1_t *gate_noise, const noise_rank1_t *ve_noise, void *const out[3],
                                   noise_stream_t stream) {
    clear_error();
    return pop_block_qkv_impl("noise_pop_block_qkv", pop, y, w_o, r_o, o_dots, o_dots_n, xres, w_fc, r_fc, w_proj,
                              r_proj, xout, mix, lam_r, lam_x, eps_r, eps_x, eps_stride, x0, w_qkv, r_qkv, rope_cos,
                              rope_sin, ve, vocab, idx, idx_sm, gate_w, gate_noise, ve_noise, out, nullptr, stream);
}

extern "C" int noise_pop_block_qkv_jit(const noise_population_t *pop, noise_view_t y, const void *w_o,
                                       noise_view_t xres, const void *w_fc, const void *w_proj, float *xout,
                                       const float *lam_r, const float *lam_x, noise_view_t x0,
                                       const void *const w_qkv[3], const void *rope_cos, const void *rope_sin,
                                       const float *ve, int64_t vocab, const int64_t *idx, int64_t idx_sm,
                                       const float *gate_w, void *const out[3], const noise_block_jitter_t *jit,
                                       noise_stream_t stream) {
    clear_error();
    return pop_block_qkv_impl("noise_pop_block_qkv_jit", pop, y, w_o, nullptr, nullptr, 0, xres, w_fc, nullptr,
                              w_proj, nullptr, xout, 1, lam_r, lam_x, nullptr, nullptr, 0, x0, w_qkv, nullptr,
                              rope_cos, rope_sin, ve, vocab, idx, idx_sm, gate_w, nullptr, nullptr, out, jit, stream);
}
