// Perturbed linears of the population forward and the fused head + soft-capped cross-entropy.
//
// Replaces eggroll.py:56-58 `lowrank` (x W^T + sign (x b) a^T, the rank-1 term never materialised) at
// every call site of population_loss (eggroll.py:80-93, 99), together with the elementwise work the
// reference runs between them (rotary + per-head norm, eggroll.py:90 / model.py:55-58, 46-47; value
// embedding gate, eggroll.py:85-89; residual adds and mixing scalars, eggroll.py:77-79, 92-93; ReLU^2,
// eggroll.py:93; RMSNorm, model.py:46-47) and the head's softcap + cross-entropy + per-member mean
// (eggroll.py:94-103; run.py:89-94 for the fp32 head).
//
// Shape of every product: out[(m,t), n] = sum_k W[n, k] x[(m,t), k], computed transposed (W rows are the
// MFMA A operand, token rows the B operand) so that each lane of a v_mfma_f32_32x32x16_bf16 result holds
// 16 output features of ONE token: per-token / per-head epilogue reductions stay in the lane plus one
// exchange with lane ^ 32. A workgroup of 8 waves (two per SIMD, so one wave's LDS waits and barriers
// overlap the other's MFMAs) computes a BN x BM (features x tokens) tile; each wave owns 128 x 64
// (4 x 2 MFMA blocks, 128 fp32 accumulators). K is streamed through LDS stages filled by direct
// global -> LDS copies (Mma in tile.hpp).
#include "common.hpp"
#include "mfma.hpp"
#include "tile.hpp"

namespace noise {
namespace {

constexpr float kEps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps, F.rms_norm's default
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kThreads = 512;                     // 8 waves

// Copy the two feature blocks of head HD (blocks 2HD, 2HD+1) of token block TB into plain registers
// (static indices keep the accumulators in registers).
template <int TB, int HD>
__device__ __forceinline__ void copy_head(const f32x16 (&acc)[4][2], float (&v)[2][16]) {
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[half][r] = acc[2 * HD + half][TB][r];
}

// Epilogue staging: each wave writes its finished tile into a private LDS region (rows padded to kStg)
// and re-reads it as 16 B row chunks, so global stores are whole, contiguous lines. A wave's LDS
// instructions execute in order, so its own write -> read needs no barrier.
constexpr int kStg = 136;
constexpr int kStgV = 72;  // transposed V tile: [128 features][64 tokens]

struct Pop {
    int members, tokens;
    const float *sign;
    int dir_div;
};

struct Rank1 {
    const float *a, *b;
    int64_t a_stride, b_stride;
};

// ------------------------------------------------------------------------------------------------
// Q, K, V: rank-1 correction, value-embedding gate (V), rotary + per-head RMSNorm (Q, K); Q, K written
// bf16 [m][H][T][64], V transposed [m][H][64][T].
// ------------------------------------------------------------------------------------------------
struct QkvArgs {
    Pop pop;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const __bf16 *w[3];
    Rank1 r1[3];
    const float *dots;        // [rows][3]: x . b_q, x . b_k, x . b_v
    const __bf16 *cos_t, *sin_t;  // [T][32] bf16 (model.py:177-183's tables)
    const float *ve;          // [V][512] fp32 or NULL; member m reads rows ve + m * ve_m
    int64_t ve_m;             // 0 (one table for all members) or the member stride of per-member rows
    const int64_t *idx;       // token ids: member m, token t at idx[m * idx_m + t]
    int64_t idx_m;            // 0 (one sequence for all members) or the member stride of per-member tokens
    int64_t vocab;            // rows of the value table: other ids read row 0 and give NaN values
    const float *gates;       // [rows][8] value-embedding gates (noise_pop_gate)
    Rank1 ve_r1;              // value-embedding noise (a [dirs][V], b [dirs][512]) or a == NULL
    __bf16 *out[3];           // q, k: [m][8][T][64]; v transposed: [m][8][64][T]
};

// rotary rows of a 256-token tile in LDS: [token][32] bf16, 64 B rows whose four 16 B chunks are
// XOR-swizzled by (token / 4) mod 4, so the 8 B reads of 16 consecutive tokens hit distinct banks
__device__ __forceinline__ int rope_off(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4); }

// EAGER: the eager autocast forward's roundings (every elementwise op's result rounded to bf16; unperturbed
// calls only): q, k, v rounded as linear outputs, v + bf16(gate * ve), rotary products and sums rounded.
template <bool EAGER = false>
__global__ __launch_bounds__(kThreads) void qkv_kernel(QkvArgs p) {
    using M = Mma<8, 256, 256, 64, 2>;
    // LDS: the K loop's two stages of 64 KiB. During the last stage (slot 1) slot 0 takes the tile's rotary
    // rows (cos then sin, 32 KiB) and the a and value-embedding b vectors (2 KiB); after the loop, per-wave,
    // per-head staging ([64][72] bf16: Q, K as tokens x dims, V^T as dims x tokens) follows them.
    constexpr int kStgH = 72;
    constexpr int kWaveStg = 64 * kStgH;
    constexpr int kRope = 2 * 256 * 64;
    constexpr int kVec = 2 * 256 * 4;
    constexpr int kStgOff = kRope + kVec;
    static_assert(kStgOff <= M::STAGE, "rotary rows and vectors within free slot 0");
    static_assert(kStgOff + 8 * kWaveStg * 2 <= M::LDS_BYTES, "staging within the stages");
    constexpr int kLds = M::LDS_BYTES;
    __shared__ __attribute__((aligned(16))) __bf16 lds[kLds / 2];
    const int T = p.pop.tokens;
    const int tiles_t = T / 256;
    int nt, tt;
    tile_order(blockIdx.x, 6, p.pop.members * tiles_t, tt, nt);
    const int m = tt / tiles_t, t0 = (tt % tiles_t) * 256;
    const int n0 = nt * 256, mat = n0 / 512, nl0 = n0 % 512;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wn0 = M::wn0(wave), wm0 = M::wm0(wave);
    const int dir = m / p.pop.dir_div;
    const Rank1 r1 = p.r1[mat];
    const int head0 = (nl0 + wn0) / 64;
    const bool ve_on = mat == 2 && p.ve;

    // epilogue inputs: rotary rows and per-feature vectors by direct copy into LDS during the last K stage
    // (the K loop waits for them before its final barrier), per-token scalars into registers ahead of it
    char *rope = reinterpret_cast<char *>(lds);
    float *vec = reinterpret_cast<float *>(rope + kRope);
    const float *a0 = r1.a ? r1.a + dir * r1.a_stride + nl0 : nullptr;
    const float *vb0 = ve_on && p.ve_r1.a ? p.ve_r1.b + dir * p.ve_r1.b_stride + nl0 : nullptr;
    auto copy_inputs = [&]() {
        if (mat < 2) {
            // 32 copies of 16 rows (1 KiB): copy i covers rows 16 (i % 16) .. of table i / 16; lane l fetches
            // row 16 (i % 16) + l / 4, chunk (l % 4) ^ (l / 16) (the row's swizzle, rows 16 apart share it)
            const int chunk = (lane & 3) ^ (lane >> 4);
            const unsigned off = (unsigned)((lane >> 2) * 64 + chunk * 16);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = 8 * k + wave;
                const __bf16 *tab = i < 16 ? p.cos_t : p.sin_t;
                lds_dma16(tab + (int64_t)(t0 + 16 * (i & 15)) * 32, off, rope + i * 1024);
            }
        }
        // (an absent vector reads as zeros, so the epilogue needs no branches)
        if (wave < 2) {
            const float *src = wave == 0 ? a0 : vb0;
            if (src)
                lds_dma16(src, lane * 16, vec + 256 * wave);
            else
                st4(vec + 256 * wave + 4 * lane, float4{0.f, 0.f, 0.f, 0.f});
        }
    };
    float dt[2] = {0.f, 0.f}, gt[2][2] = {{0.f, 0.f}, {0.f, 0.f}}, vesc[2] = {0.f, 0.f};
    int64_t tokv[2] = {0, 0};
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int t = t0 + wm0 + 32 * tb + j;
        const int64_t row = (int64_t)m * T + t;
        if (a0) dt[tb] = p.dots[row * 3 + mat];
        if (ve_on) {
            const int64_t tok = p.idx[m * p.idx_m + t];
            const bool bad = tok < 0 || tok >= p.vocab;  // an id outside the table: no read leaves it, V is NaN
            tokv[tb] = bad ? 0 : tok;
            gt[tb][0] = bad ? __builtin_nanf("") : p.gates[row * 8 + head0];
            gt[tb][1] = bad ? __builtin_nanf("") : p.gates[row * 8 + head0 + 1];
            if (p.ve_r1.a) vesc[tb] = p.ve_r1.a[dir * p.ve_r1.a_stride + tokv[tb]];
        }
    }

    f32x16 acc[4][2];
    M::run(p.w[mat] + (int64_t)nl0 * 512, 512, p.x + m * p.xs_m + (int64_t)t0 * p.xs_t, p.xs_t, 512, lds, acc, tid,
           wn0, wm0, copy_inputs);

    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;  // unperturbed calls may pass no signs
    const float *arow = vec + wn0;  // zeros when unperturbed
    __bf16 *outm = p.out[mat];
    __bf16 *stg = lds + kStgOff / 2 + wave * kWaveStg;

    // one head at a time: its two token blocks (32 accumulators each, copied out with static indices so
    // the body is compiled once and only one block's values are live), staged, then stored
#pragma unroll
    for (int hd = 0; hd < 2; ++hd) {
#pragma unroll 1
        for (int tb = 0; tb < 2; ++tb) {
            float v[2][16];
            if (hd == 0) {
                if (tb == 0) copy_head<0, 0>(acc, v); else copy_head<1, 0>(acc, v);
            } else {
                if (tb == 0) copy_head<0, 1>(acc, v); else copy_head<1, 1>(acc, v);
            }
            const int tl = wm0 + 32 * tb + j;  // token within the tile
            {
                const float corr = sgn * (tb ? dt[1] : dt[0]);  // dt = 0 without perturbation
#pragma unroll
                for (int half = 0; half < 2; ++half)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const float4 a4 = ld4(arow + 64 * hd + 32 * half + 8 * g + 4 * hf);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[half][4 * g + e] += corr * f4get(a4, e);
                    }
            }
            if constexpr (EAGER) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    v[0][r] = bfr(v[0][r]);
                    v[1][r] = bfr(v[1][r]);
                }
            }
            if (ve_on) {
                // v += gate[row, head] * (ve[idx[t], head*64 + d] (+ lowrank_embed term))   (eggroll.py:85-89);
                // the gates 2 sigmoid(x[:32] . Wg[head] (+ rank-1)) come precomputed (noise_pop_gate)
                const int64_t tok = tb ? tokv[1] : tokv[0];
                const float gate = tb ? (hd ? gt[1][1] : gt[1][0]) : (hd ? gt[0][1] : gt[0][0]);
                const float *ver = p.ve + m * p.ve_m + tok * 512 + (head0 + hd) * 64;
                // lowrank_embed of the value table (eggroll.py:61-63): + sign * a_ve[tok] * b_ve[:]
                const float ves = sgn * (tb ? vesc[1] : vesc[0]);     // 0 without value-table noise
                const float *veb = vec + 256 + wn0 + hd * 64;           // zeros without value-table noise
                float4 e4[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) e4[q] = ld4(ver + 32 * (q >> 2) + 8 * (q & 3) + 4 * hf);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int half = q >> 2, g = q & 3;
                    const float4 b4 = ld4(veb + 32 * half + 8 * g + 4 * hf);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (EAGER)
                            v[half][4 * g + e] = bfr(v[half][4 * g + e] + bfr(gate * f4get(e4[q], e)));
                        else
                            v[half][4 * g + e] += gate * (f4get(e4[q], e) + ves * f4get(b4, e));
                    }
                }
            }
            if (mat < 2) {
                // rotary (model.py:55-58) then RMSNorm over the head (model.py:46-47)
                float ss = 0.f;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int o = rope_off(tl, g) + 8 * hf;
                    const bf16x4 c4 = *reinterpret_cast<const bf16x4 *>(rope + o);
                    const bf16x4 s4 = *reinterpret_cast<const bf16x4 *>(rope + 256 * 64 + o);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = 4 * g + e;
                        const float c = (float)c4[e], sn = (float)s4[e];
                        const float x1 = v[0][r], x2 = v[1][r];
                        const float o1 = EAGER ? bfr(bfr(x1 * c) + bfr(x2 * sn)) : x1 * c + x2 * sn;
                        const float o2 = EAGER ? bfr(bfr(x1 * -sn) + bfr(x2 * c)) : x1 * -sn + x2 * c;
                        v[0][r] = o1;
                        v[1][r] = o2;
                        ss += o1 * o1 + o2 * o2;
                    }
                }
                ss += swap_halves(ss);
                const float rstd = rsqrtf(ss * (1.0f / 64.0f) + kEps);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    v[0][r] *= rstd;
                    v[1][r] *= rstd;
                }
            }
            // stage the head: Q, K as [token][dim]; V transposed as [dim][token]
            const int tw = 32 * tb + j;  // token within the wave
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * half + 8 * g + 4 * hf;
                    if (mat < 2) {
                        bf16x4 o;
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[e] = (__bf16)v[half][4 * g + e];
                        store_bf16x4(stg + tw * kStgH + d, o);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) stg[(d + e) * kStgH + tw] = (__bf16)v[half][4 * g + e];
                    }
                }
        }
        // whole-line stores of the head: Q, K rows [m][h][t][0:64] (128 B); V^T rows [m][h][d][t0+wm0 .. +64)
        // (a wave's own LDS writes and reads stay in order: no barrier)
        const int64_t hbase = ((int64_t)m * 8 + head0 + hd);
#pragma unroll 4
        for (int it = 0; it < 8; ++it) {
            const int c = it * 64 + lane, r = c >> 3, ch = c & 7;
            const bf16x8 v = load_bf16x8(stg + r * kStgH + ch * 8);
            if (mat < 2)
                store_bf16x8(outm + (hbase * T + t0 + wm0 + r) * 64 + ch * 8, v);
            else
                store_bf16x8(outm + (hbase * 64 + r) * T + t0 + wm0 + ch * 8, v);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Q, K, V of a block whose input every member shares (block 0 of the population when the embedding and
// mixing scalars are unperturbed): the product base = x [c_q; c_k; c_v]^T is the same for all members
// (fp32 [T][1536], computed once), so each member's Q, K, V are base + sign * dot * a (eggroll.py:58) then
// rotary and per-head RMSNorm on Q and K (eggroll.py:90, model.py:55-58, 46-47), as qkv_kernel's epilogue
// computes them (no value embedding). An HBM-write stream instead of a per-member GEMM.
// Workgroup = (64-token tile, head, member), members fastest so a tile's base rows stay in L2; 256
// threads: token tl = tid / 4, part = tid % 4 holds dims 8 part .. +8 of both rotary halves.
// ------------------------------------------------------------------------------------------------
struct QkvSharedArgs {
    Pop pop;
    const float *base;                // [T][1536]
    Rank1 r1[3];
    const float *dots;                // [rows][3]
    const __bf16 *cos_t, *sin_t;      // [T][32]
    __bf16 *out[3];                   // q, k: [m][8][T][64]; v transposed: [m][8][64][T]
};

__global__ __launch_bounds__(256) void qkv_shared_kernel(QkvSharedArgs p) {
    __shared__ __attribute__((aligned(16))) __bf16 vt[64][72];  // V^T tile [dim][token]
    const int M = p.pop.members, T = p.pop.tokens;
    const int m = blockIdx.x % M, th = blockIdx.x / M, h = th % 8, t0 = (th / 8) * 64;
    const int tid = threadIdx.x, tl = tid >> 2, part = tid & 3, t = t0 + tl;
    const int64_t row = (int64_t)m * T + t;
    const int dir = m / p.pop.dir_div;
    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;
    const float *brow = p.base + (int64_t)t * 1536 + h * 64;
    const int64_t hrow = ((int64_t)m * 8 + h) * T + t;  // row of Q, K [m][h][t]
#pragma unroll
    for (int mat = 0; mat < 3; ++mat) {
        // dims d = 8 part + i (first half) and 32 + 8 part + i (second half), i < 8
        float x1[8], x2[8];
        const float *b = brow + mat * 512 + 8 * part;
        const float4 u0 = ld4(b), u1 = ld4(b + 4), w0 = ld4(b + 32), w1 = ld4(b + 36);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x1[e] = f4get(u0, e); x1[4 + e] = f4get(u1, e);
            x2[e] = f4get(w0, e); x2[4 + e] = f4get(w1, e);
        }
        const Rank1 r = p.r1[mat];
        if (r.a) {
            const float corr = sgn * p.dots[row * 3 + mat];
            const float *a = r.a + dir * r.a_stride + h * 64 + 8 * part;
            const float4 a0 = ld4(a), a1 = ld4(a + 4), c0 = ld4(a + 32), c1 = ld4(a + 36);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x1[e] += corr * f4get(a0, e); x1[4 + e] += corr * f4get(a1, e);
                x2[e] += corr * f4get(c0, e); x2[4 + e] += corr * f4get(c1, e);
            }
        }
        if (mat < 2) {
            const bf16x8 c8 = load_bf16x8(p.cos_t + (int64_t)t * 32 + 8 * part);
            const bf16x8 s8 = load_bf16x8(p.sin_t + (int64_t)t * 32 + 8 * part);
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float c = (float)c8[i], sn = (float)s8[i];
                const float o1 = x1[i] * c + x2[i] * sn;
                const float o2 = x1[i] * -sn + x2[i] * c;
                x1[i] = o1;
                x2[i] = o2;
                ss += o1 * o1 + o2 * o2;
            }
            ss += __shfl_xor(ss, 1, 64);
            ss += __shfl_xor(ss, 2, 64);
            const float rstd = rsqrtf(ss * (1.0f / 64.0f) + kEps);
            bf16x8 lo, hi;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = (__bf16)(x1[i] * rstd);
                hi[i] = (__bf16)(x2[i] * rstd);
            }
            __bf16 *o = p.out[mat] + hrow * 64;
            store_bf16x8_nt(o + 8 * part, lo);
            store_bf16x8_nt(o + 32 + 8 * part, hi);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                vt[8 * part + i][tl] = (__bf16)x1[i];
                vt[32 + 8 * part + i][tl] = (__bf16)x2[i];
            }
        }
    }
    __syncthreads();
    // V^T rows [m][h][d][t0 .. t0 + 64): 64 rows of 128 B, 8 chunks of 16 B each
    __bf16 *ov = p.out[2] + ((int64_t)m * 8 + h) * 64 * T + t0;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int c = it * 256 + tid, d = c >> 3, ch = c & 7;
        store_bf16x8_nt(ov + (int64_t)d * T + ch * 8, load_bf16x8(&vt[d][ch * 8]));
    }
}

// ------------------------------------------------------------------------------------------------
// Residual writers (attn.c_proj, mlp.c_proj; N = 512, whole rows per workgroup):
//   y = xres + (x W^T + sign * dot * a)        [+ mix: y = rl * y + ml * x0 for the next block]
//   write y (fp32) if xout; h = RMSNorm(y) as bf16 (or its [hi | lo | hi] bf16 split for the fp32 head);
//   next_dots[row][k] = h . b_k for the next perturbed linear(s).
// ------------------------------------------------------------------------------------------------
struct ResidArgs {
    Pop pop;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const __bf16 *w;
    int K;
    Rank1 r1;
    const float *dots;
    int64_t dots_stride;
    int dots_count;
    const float *xres;
    int64_t xr_m, xr_t;
    float *xout;              // [m][T][512] or NULL
    int mix;
    const float *lam_r, *lam_x;  // the next block's mixing scalars (device, read when mixing)
    const float *eps_r, *eps_x;  // per-direction lambda noise (eps[dir * eps_stride]) or NULL
    int64_t eps_stride;
    const float *x0;
    int64_t x0_m, x0_t;
    __bf16 *hout;             // [m][T][512] or [m][T][1536] (split3)
    int split3;
    const float *nb[3];
    int64_t nb_stride[3];
    int nnext;
    float *ndots;             // [rows][nnext]
    const __bf16 *jit;        // DUST jitter added to the product (run.py:115-117), [m][T][512] bf16, or NULL
    int64_t jit_m, jit_t;
};

// MIX: apply the next block's mixing (x0 read); NNEXT: number of next-matrix dots (0..3); JIT: add a
// per-token jitter to the product. All fixed at compile time so the epilogue's loads carry no per-group
// branches and can be issued in batches.
// EAGER: the eager forward's roundings (unperturbed, no next dots): y = bf16(xres + bf16(x W^T)) and the
// mix bf16(bf16(rl * y) + bf16(ml * x0)), so the residual stream stays bf16-valued.
template <int KD, bool MIX, int NNEXT, bool JIT = false, bool EAGER = false>
__global__ __launch_bounds__(kThreads) void resid_kernel(ResidArgs p) {
    using M = Mma<8, 512, 128, 64, 2>;
    static_assert(KD % 128 == 0, "an even number of K stages: the last one runs in slot 1");
    // LDS: the K loop's two stages of 80 KiB fill all 160 KiB. During the last stage (slot 1) slot 0 is free
    // and takes the a vector and up to three next b vectors (512 floats each, at 72 KiB). After the loop:
    // per-wave staging of 17 KiB (fp32 [32 tokens][136], or bf16 [64][136] for the hi/lo rows of the split3
    // output) for waves 0-3 below the vectors and waves 4-7 above them, then the per-token statistics
    // [128 tokens][4 feature waves][4].
    constexpr int kStgF = 136;
    constexpr int kStgBytes = 32 * kStgF * 4;
    constexpr int kVecOff = 72 * 1024, kVecBytes = 4 * 512 * 4;
    constexpr int kRedOff = kVecOff + kVecBytes + 4 * kStgBytes;
    constexpr int kLds = M::LDS_BYTES;
    static_assert(4 * kStgBytes <= kVecOff && kVecOff + kVecBytes <= M::STAGE, "vectors within free slot 0");
    static_assert(kRedOff + 128 * 4 * 4 * 4 <= kLds, "epilogue layout fits");
    static_assert(32 * kStgF * 4 >= 64 * kStg * 2, "bf16 split3 staging must fit the wave's region");
    __shared__ __attribute__((aligned(16))) __bf16 lds[kLds / 2];
    const int T = p.pop.tokens;
    const int tiles_t = T / 128;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * 128;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wn0 = M::wn0(wave), wm0 = M::wm0(wave), wq = wave % 4;
    const int dir = m / p.pop.dir_div;

    // epilogue inputs: the per-feature vectors by direct copy into LDS during the last K stage (wave
    // 2v + h copies half h of vector v; the K loop waits for them before its final barrier), the per-token
    // rank-1 dot sums and the mixing scalars into registers ahead of the K loop
    char *ldsb = reinterpret_cast<char *>(lds);
    float *vec = reinterpret_cast<float *>(ldsb + kVecOff);
    auto copy_vectors = [&]() {
        const int v = wave >> 1, h = wave & 1;
        const float *src = v == 0 ? (p.r1.a ? p.r1.a + dir * p.r1.a_stride : nullptr)
                                  : (v - 1 < NNEXT ? p.nb[v - 1] + dir * p.nb_stride[v - 1] : nullptr);
        if (src)
            lds_dma16(src + 256 * h, lane * 16, vec + 512 * v + 256 * h);
        else if (v == 0)
            st4(vec + 256 * h + 4 * lane, float4{0.f, 0.f, 0.f, 0.f});  // no perturbation: a = 0
    };
    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;  // unperturbed calls may pass no signs
    float dsum[2] = {0.f, 0.f};
    if (p.r1.a) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int64_t row = (int64_t)m * T + t0 + wm0 + 32 * tb + j;
            for (int i = 0; i < p.dots_count; ++i) dsum[tb] += p.dots[row * p.dots_stride + i];
        }
    }
    float rl = 0.f, ml = 0.f;
    if (MIX) {
        rl = *p.lam_r;
        ml = *p.lam_x;
        if (p.eps_r) rl += sgn * p.eps_r[dir * p.eps_stride];
        if (p.eps_x) ml += sgn * p.eps_x[dir * p.eps_stride];
    }
    if constexpr (EAGER) {
        // eager autocast multiplies a bf16 tensor by the 0-dim fp32 lambdas in bf16: they enter rounded
        rl = bfr(rl);
        ml = bfr(ml);
    }

    f32x16 acc[4][2];
    M::run(p.w, KD, p.x + m * p.xs_m + (int64_t)t0 * p.xs_t, p.xs_t, KD, lds, acc, tid, wn0, wm0, copy_vectors);

    float *stgf = reinterpret_cast<float *>(ldsb + (wave < 4 ? wave * kStgBytes : kVecOff + kVecBytes + (wave - 4) * kStgBytes));
    __bf16 *stgb = reinterpret_cast<__bf16 *>(stgf);
    float *red = reinterpret_cast<float *>(ldsb + kRedOff);

#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int tl = wm0 + 32 * tb + j;
        const int t = t0 + tl;
        const float corr = sgn * (tb ? dsum[1] : dsum[0]);  // dsum = 0 without perturbation
        const float *xr = p.xres + m * p.xr_m + (int64_t)t * p.xr_t + wn0;
        const float *x0r = MIX ? p.x0 + m * p.x0_m + (int64_t)t * p.x0_t + wn0 : nullptr;
        const __bf16 *jr = JIT ? p.jit + m * p.jit_m + (int64_t)t * p.jit_t + wn0 : nullptr;
        float ssq = 0.f;
        // one feature block (4 groups of 4) at a time: its residual (and x0) loads are issued, then used
#pragma unroll
        for (int fb = 0; fb < 4; ++fb) {
            float4 xv[4], zv[4];
            bf16x4 jv[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int f0 = 32 * fb + 8 * g + 4 * hf;
                xv[g] = ld4(xr + f0);
                if constexpr (MIX) zv[g] = ld4(x0r + f0);
                if constexpr (JIT) jv[g] = *reinterpret_cast<const bf16x4 *>(jr + f0);
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int f0 = 32 * fb + 8 * g + 4 * hf;
                const float4 a4 = ld4(vec + wn0 + f0);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float prod = acc[fb][tb][4 * g + e] + corr * f4get(a4, e);
                    if constexpr (JIT) prod += (float)jv[g][e];
                    float y;
                    if constexpr (EAGER) {
                        y = bfr(f4get(xv[g], e) + bfr(prod));
                        if constexpr (MIX) y = bfr(bfr(rl * y) + bfr(ml * f4get(zv[g], e)));
                    } else {
                        y = f4get(xv[g], e) + prod;
                        if constexpr (MIX) y = rl * y + ml * f4get(zv[g], e);
                    }
                    acc[fb][tb][4 * g + e] = y;
                    ssq += y * y;
                }
                if (p.xout)
                    st4(stgf + j * kStgF + f0, float4{acc[fb][tb][4 * g], acc[fb][tb][4 * g + 1],
                                                      acc[fb][tb][4 * g + 2], acc[fb][tb][4 * g + 3]});
            }
        }
        if (p.xout) {
            // whole-line stores: 32 rows x 512 B of this wave's 128 features
            float *xo = p.xout + ((int64_t)m * T + t0 + wm0 + 32 * tb) * 512 + wn0;
#pragma unroll 4
            for (int it = 0; it < 16; ++it) {
                const int c = it * 64 + lane, r = c >> 5, ch = c & 31;
                st4(xo + (int64_t)r * 512 + ch * 4, ld4(stgf + r * kStgF + ch * 4));
            }
        }
        // per-token partials over this wave's 128 features: sum of squares, then y . b_k of each next matrix
        ssq += swap_halves(ssq);
        if (hf == 0) red[(tl * 4 + wq) * 4] = ssq;
#pragma unroll 1
        for (int k = 0; k < NNEXT; ++k) {
            float d = 0.f;
#pragma unroll
            for (int fb = 0; fb < 4; ++fb)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 b4 = ld4(vec + 512 * (k + 1) + wn0 + 32 * fb + 8 * g + 4 * hf);
#pragma unroll
                    for (int e = 0; e < 4; ++e) d += acc[fb][tb][4 * g + e] * f4get(b4, e);
                }
            d += swap_halves(d);
            if (hf == 0) red[(tl * 4 + wq) * 4 + 1 + k] = d;
        }
    }
    __syncthreads();
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int tl = wm0 + 32 * tb + j;
        const int t = t0 + tl;
        const int64_t row = (int64_t)m * T + t;
        float tot[1 + NNEXT];
#pragma unroll
        for (int k = 0; k <= NNEXT; ++k) tot[k] = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int k = 0; k <= NNEXT; ++k) tot[k] += red[(tl * 4 + w) * 4 + k];
        const float rstd = rsqrtf(tot[0] * (1.0f / 512.0f) + kEps);
        // stage bf16 rows: [32][kStg] for hi (and lo after it when split3)
#pragma unroll
        for (int fb = 0; fb < 4; ++fb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                bf16x4 hi, lo;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float h = acc[fb][tb][4 * g + e] * rstd;
                    hi[e] = (__bf16)h;
                    lo[e] = (__bf16)(h - (float)hi[e]);
                }
                const int f0 = 32 * fb + 8 * g + 4 * hf;
                store_bf16x4(stgb + j * kStg + f0, hi);
                if (p.split3) store_bf16x4(stgb + (32 + j) * kStg + f0, lo);
            }
        const int width = p.split3 ? 1536 : 512;
        __bf16 *hb = p.hout + ((int64_t)m * T + t0 + wm0 + 32 * tb) * width + wn0;
#pragma unroll 4
        for (int it = 0; it < 8; ++it) {
            const int c = it * 64 + lane, r = c >> 4, ch = c & 15;
            bf16x8 hv = load_bf16x8(stgb + r * kStg + ch * 8);
            store_bf16x8(hb + (int64_t)r * width + ch * 8, hv);
            if (p.split3) {
                store_bf16x8(hb + (int64_t)r * width + 512 + ch * 8, load_bf16x8(stgb + (32 + r) * kStg + ch * 8));
                store_bf16x8(hb + (int64_t)r * width + 1024 + ch * 8, hv);
            }
        }
        if (wq == 0 && hf == 0) {
#pragma unroll
            for (int k = 0; k < NNEXT; ++k) p.ndots[row * NNEXT + k] = rstd * tot[1 + k];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// MLP hidden (mlp.c_fc, N = 2048): act = relu(x W^T + sign * dot * a)^2 as bf16, and the partial dots
// act . b of the following mlp.c_proj over each wave's 128 features: pdots[row][n / 128].
// ------------------------------------------------------------------------------------------------
struct FcArgs {
    Pop pop;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const __bf16 *w;
    Rank1 r1;
    const float *dots;        // [rows]
    __bf16 *act;              // [m][T][2048]
    const float *nb;          // next b rows [dirs][2048] or NULL
    int64_t nb_stride;
    float *pdots;             // [rows][16]
    const __bf16 *jit;        // DUST jitter on the hidden pre-activation (run.py:116), [rows][2048] bf16, or NULL
};

// EAGER: relu(bf16(x W^T)) squared and rounded (the eager forward; unperturbed calls only)
template <bool JIT = false, bool EAGER = false>
__global__ __launch_bounds__(kThreads) void fc_kernel(FcArgs p) {
    using M = Mma<8, 256, 256, 64, 2>;
    constexpr int kMain = cmax(M::LDS_BYTES, 8 * 64 * kStg * 2);  // K loop, then per-wave act staging
    constexpr int kLds = kMain + 2 * 256 * 4;                      // + the tile's a and next-b vectors
    __shared__ __attribute__((aligned(16))) __bf16 lds[kLds / 2];
    const int T = p.pop.tokens;
    const int tiles_t = T / 256;
    int nt, tt;
    tile_order(blockIdx.x, 8, p.pop.members * tiles_t, tt, nt);
    const int m = tt / tiles_t, t0 = (tt % tiles_t) * 256;
    const int n0 = nt * 256;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wn0 = M::wn0(wave), wm0 = M::wm0(wave);
    const int dir = m / p.pop.dir_div;

    // the epilogue's per-feature vectors go to LDS by direct copy ahead of the K loop (whose waits and
    // barriers then cover them), so the epilogue reads them without a global round trip per use
    float *vec = reinterpret_cast<float *>(reinterpret_cast<char *>(lds) + kMain);
    const float *a0 = p.r1.a ? p.r1.a + dir * p.r1.a_stride + n0 : nullptr;
    const float *b0 = p.nb ? p.nb + dir * p.nb_stride + n0 : nullptr;
    // (an absent vector reads as zeros, so the epilogue needs no branches)
    if (wave < 2) {
        const float *src = wave == 0 ? a0 : b0;
        if (src)
            lds_dma16(src, lane * 16, vec + 256 * wave);
        else
            st4(vec + 256 * wave + 4 * lane, float4{0.f, 0.f, 0.f, 0.f});
    }
    // this lane's two tokens' x . b dots, loaded now and used after the K loop
    float dt[2] = {0.f, 0.f};
    if (a0) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) dt[tb] = p.dots[(int64_t)m * T + t0 + wm0 + 32 * tb + j];
    }

    f32x16 acc[4][2];
    M::run(p.w + (int64_t)n0 * 512, 512, p.x + m * p.xs_m + (int64_t)t0 * p.xs_t, p.xs_t, 512, lds, acc, tid, wn0,
           wm0);

    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;  // unperturbed calls may pass no signs
    const int nf0 = n0 + wn0;
    const float *arow = vec + wn0, *brow = vec + 256 + wn0;  // zeros when absent
    __bf16 *stg = lds + wave * 64 * kStg;
    if constexpr (JIT) {
        // the wave's jitter rows [64 tokens][128 features] staged by whole-line loads (read in the MFMA
        // layout, one 8 B load would touch 32 rows); each lane then reads its values from the staging rows and
        // writes its outputs over them
        const __bf16 *jbase = p.jit + ((int64_t)m * T + t0 + wm0) * 2048 + nf0;
#pragma unroll 4
        for (int it = 0; it < 16; ++it) {
            const int c = it * 64 + lane, r = c >> 4, ch = c & 15;
            store_bf16x8(stg + r * kStg + ch * 8, load_bf16x8(jbase + (int64_t)r * 2048 + ch * 8));
        }
        wave_lds_sync();
    }
    // feature-major: each a / b vector chunk is read from LDS once and used for both tokens
    int64_t row[2];
    float corr[2], pd[2] = {0.f, 0.f};
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        row[tb] = (int64_t)m * T + t0 + wm0 + 32 * tb + j;
        corr[tb] = sgn * dt[tb];  // dt = 0 without perturbation
    }
#pragma unroll
    for (int fb = 0; fb < 4; ++fb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int f = 32 * fb + 8 * g + 4 * hf;
            const float4 a4 = ld4(arow + f), b4 = ld4(brow + f);
            const bf16x2 b01{(__bf16)b4.x, (__bf16)b4.y}, b23{(__bf16)b4.z, (__bf16)b4.w};
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                bf16x4 jv;
                if constexpr (JIT) jv = *reinterpret_cast<const bf16x4 *>(stg + (32 * tb + j) * kStg + f);
                bf16x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float y = acc[fb][tb][4 * g + e] + corr[tb] * f4get(a4, e);
                    if constexpr (JIT) y += (float)jv[e];
                    if constexpr (EAGER) y = bfr(y);
                    y = fmaxf(y, 0.f);
                    o[e] = (__bf16)(y * y);
                }
                // act . b with both in bf16, as the reference's autocast x @ b (eggroll.py:58) multiplies them
                pd[tb] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{o[0], o[1]}, b01, pd[tb], false);
                pd[tb] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{o[2], o[3]}, b23, pd[tb], false);
                store_bf16x4(stg + (32 * tb + j) * kStg + f, o);
            }
        }
    if (p.pdots) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const float t = pd[tb] + swap_halves(pd[tb]);
            if (hf == 0) p.pdots[row[tb] * 16 + nf0 / 128] = t;
        }
    }
    // whole-line stores of act rows [m][t][nf0 .. nf0 + 128) (256 B each)
    __bf16 *abase = p.act + ((int64_t)m * T + t0 + wm0) * 2048 + nf0;
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
        const int c = it * 64 + lane, r = c >> 4, ch = c & 15;
        store_bf16x8(abase + (int64_t)r * 2048 + ch * 8, load_bf16x8(stg + r * kStg + ch * 8));
    }
}

// ------------------------------------------------------------------------------------------------
// Generic perturbed linear (eggroll.py:56-58): y = x W^T + sign * dot * a, bf16 or fp32 out.
// grid: (N / 256) * (T / 256) * members; N, T multiples of 256, K multiple of 64.
// ------------------------------------------------------------------------------------------------
struct LowrankArgs {
    Pop pop;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const __bf16 *w;
    int K, N;
    Rank1 r1;
    const float *dots;        // [rows] (x . b per row) or NULL when unperturbed
    void *y;
    int y_fp32;               // 0 bf16 out, 1 fp32, 2 fp32 of the bf16-rounded product and dot (autocast)
    int64_t ys_m, ys_t;
};

__global__ __launch_bounds__(kThreads) void lowrank_kernel(LowrankArgs p) {
    using M = Mma<8, 256, 256, 64, 2>;
    __shared__ __attribute__((aligned(16))) __bf16 lds[M::LDS_BYTES / 2];
    const int T = p.pop.tokens, ntiles = p.N / 256, tiles_t = T / 256;
    int nt, tt;
    tile_order(blockIdx.x, ntiles, p.pop.members * tiles_t, tt, nt);
    const int m = tt / tiles_t, t0 = (tt % tiles_t) * 256;
    const int n0 = nt * 256;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wn0 = M::wn0(wave), wm0 = M::wm0(wave);

    f32x16 acc[4][2];
    M::run(p.w + (int64_t)n0 * p.K, p.K, p.x + m * p.xs_m + (int64_t)t0 * p.xs_t, p.xs_t, p.K, lds, acc, tid, wn0,
           wm0);
    const int dir = m / p.pop.dir_div;
    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;
    const int nf0 = n0 + wn0;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int t = t0 + wm0 + 32 * tb + j;
        const int64_t row = (int64_t)m * T + t;
        // autocast form (y_fp32 == 2): the product and the x . b dot enter rounded to bf16, as autocast's
        // matmuls return them (eggroll.py:58 under eggroll.py:144)
        const bool ac = p.y_fp32 == 2;
        const float corr = p.r1.a ? sgn * (ac ? bfr(p.dots[row]) : p.dots[row]) : 0.f;
#pragma unroll
        for (int fb = 0; fb < 4; ++fb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int f = nf0 + 32 * fb + 8 * g + 4 * hf;
                float4 a4 = p.r1.a ? ld4(p.r1.a + dir * p.r1.a_stride + f) : float4{0, 0, 0, 0};
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float prod = acc[fb][tb][4 * g + e];
                    o[e] = (ac ? bfr(prod) : prod) + corr * f4get(a4, e);
                }
                if (p.y_fp32) {
                    st4((float *)p.y + m * p.ys_m + (int64_t)t * p.ys_t + f, float4{o[0], o[1], o[2], o[3]});
                } else {
                    bf16x4 ob;
#pragma unroll
                    for (int e = 0; e < 4; ++e) ob[e] = (__bf16)o[e];
                    store_bf16x4((__bf16 *)p.y + m * p.ys_m + (int64_t)t * p.ys_t + f, ob);
                }
            }
    }
}

// ------------------------------------------------------------------------------------------------
// Head + softcap 15 + cross-entropy per token (eggroll.py:94-103, model.py:202-209, run.py:89-94).
// A workgroup owns 256 tokens of one member and sweeps the vocabulary in 256-wide chunks. With
// z = 15 tanh(l / 15) <= 15 the log-sum-exp needs no running max: lse = 15 + log sum exp(z - 15), and
// exp(z - 15) = exp(-30 / (e^(2l/15) + 1)). K = 1536 with [hi|hi|lo] weights and [hi|lo|hi] inputs gives
// the split-bf16x3 fp32 head.
// ------------------------------------------------------------------------------------------------
struct HeadArgs {
    Pop pop;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const __bf16 *w;
    int K, vocab;
    Rank1 r1;
    const float *dots;
    const int64_t *targets;   // [T] shared by all members, or [m][T] when targets_sm != 0
    int64_t targets_sm;
    float *loss;              // [m][T] per-token CE (0 where target == -1, NaN for targets outside [0, vocab))
};

// EAGER: logits rounded to bf16 before the soft cap (the autocast head's bf16 output; unperturbed calls only)
template <bool EAGER = false>
__global__ __launch_bounds__(kThreads) void head_ce_kernel(HeadArgs p) {
    using M = Mma<8, 256, 256, 64, 2>;
    __shared__ __attribute__((aligned(16))) __bf16 lds[M::LDS_BYTES / 2];
    const int T = p.pop.tokens, tiles_t = T / 256;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * 256;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wn0 = M::wn0(wave), wm0 = M::wm0(wave), wq = wave % 2;
    const int dir = m / p.pop.dir_div;
    const float sgn = p.pop.sign ? p.pop.sign[m] : 0.f;

    float corr[2];
    int64_t tgt[2];
    float sum[2] = {0.f, 0.f}, zt[2] = {0.f, 0.f};
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        const int t = t0 + wm0 + 32 * tb + j;
        const int64_t row = (int64_t)m * T + t;
        corr[tb] = p.r1.a ? sgn * p.dots[row] : 0.f;
        tgt[tb] = p.targets[m * p.targets_sm + t];
    }
    const float k1 = (2.0f / 15.0f) * kLog2e, k2 = -30.0f * kLog2e;
    f32x16 acc[4][2];
    for (int v0 = 0; v0 < p.vocab; v0 += 256) {
        M::run(p.w + (int64_t)v0 * p.K, p.K, p.x + m * p.xs_m + (int64_t)t0 * p.xs_t, p.xs_t, p.K, lds, acc, tid, wn0,
               wm0);
        const int nf0 = v0 + wn0;
#pragma unroll
        for (int fb = 0; fb < 4; ++fb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int f = nf0 + 32 * fb + 8 * g + 4 * hf;
                float4 a4 = p.r1.a ? ld4(p.r1.a + dir * p.r1.a_stride + f) : float4{0, 0, 0, 0};
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float l = EAGER ? bfr(acc[fb][tb][4 * g + e])
                                              : acc[fb][tb][4 * g + e] + corr[tb] * f4get(a4, e);
                        const float u = exp2_fast(l * k1) + 1.0f;
                        const float ru = __builtin_amdgcn_rcpf(u);
                        sum[tb] += exp2_fast(k2 * ru);
                        if (f + e == tgt[tb]) zt[tb] = 15.0f - 30.0f * ru;
                    }
            }
    }
    // combine the two lane halves and the two feature waves
    float *red = reinterpret_cast<float *>(lds);  // [256 tokens][2 feature waves][2]
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        sum[tb] += swap_halves(sum[tb]);
        zt[tb] += swap_halves(zt[tb]);
        if (hf == 0) {
            const int tl = wm0 + 32 * tb + j;
            red[(tl * 2 + wq) * 2 + 0] = sum[tb];
            red[(tl * 2 + wq) * 2 + 1] = zt[tb];
        }
    }
    __syncthreads();
    if (wq == 0 && hf == 0) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            const int tl = wm0 + 32 * tb + j;
            const float s = red[(tl * 2) * 2] + red[(tl * 2 + 1) * 2];
            const float z = red[(tl * 2) * 2 + 1] + red[(tl * 2 + 1) * 2 + 1];
            const float ce = 15.0f + __logf(s) - z;
            // ignore_index -1 contributes 0; any other id outside [0, vocab) is an error, reported as NaN
            const int64_t tg = tgt[tb];
            p.loss[(int64_t)m * T + t0 + tl] = tg == -1 ? 0.f : (tg < 0 || tg >= p.vocab ? __builtin_nanf("") : ce);
        }
    }
}

// The bf16 head (K = 512) with each token row read once: a workgroup owns 256 tokens of one member in 8 waves
// (two per SIMD); wave w keeps its 32 token rows [32 x 512] in registers as the B operand of every product and
// the head weights stream through LDS in 64 steps of 64 vocabulary rows (64 KiB, double buffered, copied
// global -> LDS by direct copies, wave w copying k-tile w). Per step a wave forms its 64 x 32 logits (64
// MFMAs) and folds them into the running sum of exp(z - 15) (softcap identity above: 6 VALU operations per
// logit, 3 of them transcendental); the target logit is picked in the steps whose 64 rows hold some lane's
// target. Every row of the vocabulary is in one wave, so the per-token loss needs no workgroup reduction.
constexpr int kHxThreads = 512, kHxTok = 256, kHxRows = 64;
constexpr int kHxStepBytes = kHxRows * 512 * 2;  // [8 k-tiles][64 rows][128 B]

template <bool EAGER, bool PERT>
__global__ __launch_bounds__(kHxThreads, 1) void head_x_kernel(HeadArgs p) {
    __shared__ __attribute__((aligned(16))) char lds[2 * kHxStepBytes];
    const int T = p.pop.tokens, tiles_t = T / kHxTok;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * kHxTok;
    const int tid = threadIdx.x, lane = tid & 63, jl = lane & 31, hf = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tok = t0 + 32 * wave + jl;
    const int64_t row = (int64_t)m * T + tok;
    const int dir = m / p.pop.dir_div;
    const unsigned lbase = lds_addr(lds);
    // copies of step js: wave w copies k-tile w of the step's 64 rows, 8 copies of 8 rows (chunk c of row r
    // lands at position c ^ ((r >> 1) & 7) of the row's 128 B)
    auto issue = [&](int js) {
        const unsigned dst = lbase + (js & 1) * kHxStepBytes + wave * 8192;
#pragma unroll
        for (int ci = 0; ci < 8; ++ci) {
            const int r = 8 * ci + (lane >> 3);
            const int c = (lane & 7) ^ ((r >> 1) & 7);
            lds_dma16_at(p.w + (int64_t)(kHxRows * js + 8 * ci) * 512 + wave * 64, (unsigned)((lane >> 3) * 1024 + c * 16),
                         dst + ci * 1024);
        }
    };
    issue(0);
    // this lane's token row: xf[s] = x[tok][16 s + 8 hf .. + 8], the B operand of k-step s
    bf16x8 xf[32];
    {
        const __bf16 *xr = p.x + m * p.xs_m + (int64_t)tok * p.xs_t + 8 * hf;
#pragma unroll
        for (int s = 0; s < 32; ++s) xf[s] = load_bf16x8(xr + 16 * s);
    }
    const int64_t tgt = p.targets[m * p.targets_sm + tok];
    const float corr = PERT ? p.pop.sign[m] * p.dots[row] : 0.f;
    const float *arow = PERT ? p.r1.a + dir * p.r1.a_stride + 4 * hf : nullptr;
    const float k1 = (2.0f / 15.0f) * kLog2e;     // u = 2^(k1 l) = e^(2 l / 15)
    const float c2 = 1.0f / (-30.0f * kLog2e);    // rcp(c2 (1 + u)) = -30 log2(e) / (1 + u) = log2 e^(z - 15)
    float sum = 0.f, zl = 0.f;                    // sum of e^(z - 15) over this lane's rows; the target's logit
    vm_wait<0>();
    __syncthreads();
    const int nsteps = p.vocab / kHxRows;
    f32x16 acc[2];
#pragma unroll 1
    for (int js = 0; js < nsteps; ++js) {
        if (js + 1 < nsteps) issue(js + 1);  // its buffer was last read in step js - 1, before the barrier below
        const char *buf = lds + (js & 1) * kHxStepBytes;
        auto frag = [&](int vb, int s) {
            return *reinterpret_cast<const bf16x8 *>(buf + (s >> 2) * 8192 + (32 * vb + jl) * 128 +
                                                     ((((2 * s + hf) & 7) ^ ((jl >> 1) & 7)) << 4));
        };
        acc[0] = f32x16{};
        acc[1] = f32x16{};
        bf16x8 fa[2][2];
        fa[0][0] = frag(0, 0);
        fa[0][1] = frag(1, 0);
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            if (s + 1 < 32) {
                fa[(s + 1) & 1][0] = frag(0, s + 1);
                fa[(s + 1) & 1][1] = frag(1, s + 1);
            }
            acc[0] = mfma32x32x16(fa[s & 1][0], xf[s], acc[0]);
            acc[1] = mfma32x32x16(fa[s & 1][1], xf[s], acc[1]);
        }
        // register r of block vb holds vocabulary row v0 + 32 vb + 8 (r / 4) + 4 hf + r % 4
        const int v0 = kHxRows * js;
        // the logit of register r of block vb: rounded (eager) or with the rank-1 term (perturbed head)
        auto logit = [&](int vb, int r, const float4 &a4) {
            float x = acc[vb][r];
            if constexpr (EAGER) x = bfr(x);
            if constexpr (PERT) x = __builtin_fmaf(corr, f4get(a4, r & 3), x);
            return x;
        };
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                float4 a4{0.f, 0.f, 0.f, 0.f};
                if constexpr (PERT) a4 = ld4(arow + v0 + 32 * vb + 8 * b);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float u = exp2_fast(logit(vb, 4 * b + e, a4) * k1);
                    sum += exp2_fast(__builtin_amdgcn_rcpf(__builtin_fmaf(u, c2, c2)));
                }
            }
        // the target's logit, in the steps whose rows hold some lane's target (-1 and out-of-range ids never do)
        const bool here = (uint64_t)(tgt - v0) < (uint64_t)kHxRows;
        if (__builtin_amdgcn_ballot_w64(here)) {
            const int d = here ? (int)(tgt - v0) - 4 * hf : -1;
#pragma unroll
            for (int vb = 0; vb < 2; ++vb)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    float4 a4{0.f, 0.f, 0.f, 0.f};
                    if constexpr (PERT) a4 = ld4(arow + v0 + 32 * vb + 8 * b);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d == 32 * vb + 8 * b + e) zl = logit(vb, 4 * b + e, a4);
                }
        }
        vm_wait<0>();
        __syncthreads();  // step js + 1 landed for every wave; every wave is done with buffer js & 1
    }
    sum += swap_halves(sum);
    zl += swap_halves(zl);  // exactly one lane of the pair holds the target's row
    if (hf == 0) {
        const float z = 15.0f - 30.0f / (exp2_fast(zl * k1) + 1.0f);
        const float ce = 15.0f + __logf(sum) - z;
        p.loss[row] = tgt == -1 ? 0.f : (tgt < 0 || tgt >= p.vocab ? __builtin_nanf("") : ce);
    }
}

// The fp32 head as split-bf16x3 (K = 1536: x rows [hi | lo | hi], w rows [hi | hi | lo]), logits = x_hi w_hi +
// x_lo w_hi + x_hi w_lo, with each token row read once: a workgroup owns 128 tokens of one member in 8 waves
// (two per SIMD) of 16; wave w keeps its tokens' hi and lo rows (x's first two segments; the third repeats hi
// and is not read) in registers as the B operands of v_mfma_f32_16x16x32_bf16 (128 registers) and the weights'
// hi and lo segments stream through LDS in steps of 32 vocabulary rows (2 x 32 KiB, double buffered; wave w
// copies k-tile w of both). Per step and k block a wave reads the two weight fragments once for its three
// products. The soft-capped log-sum-exp and the target pick are those of head_x_kernel; a token's rows sit in
// the four lanes l % 16 + 16 g, which are summed at the end.
constexpr int kH3Threads = 512, kH3Tok = 128, kH3Rows = 32;
constexpr int kH3Part = kH3Rows * 512 * 2;    // one segment's rows of a step: [8 k-tiles][32 rows][128 B]
constexpr int kH3Step = 2 * kH3Part;          // hi then lo
#ifndef HEAD3_AHEAD
#define HEAD3_AHEAD 4
#endif

template <bool PERT>
__global__ __launch_bounds__(kH3Threads, 1) void head3_kernel(HeadArgs p) {
    __shared__ __attribute__((aligned(16))) char lds[2 * kH3Step];
    const int T = p.pop.tokens, tiles_t = T / kH3Tok;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * kH3Tok;
    const int tid = threadIdx.x, lane = tid & 63, tl = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tok = t0 + 16 * wave + tl;
    const int64_t row = (int64_t)m * T + tok;
    const int dir = m / p.pop.dir_div;
    const unsigned lbase = lds_addr(lds);
    // copies of step js: wave w copies k-tile w (columns 64 w .. + 64) of the step's 32 rows of both segments,
    // 4 copies of 8 rows each; chunk c of row r lands at position c ^ ((r >> 1) & 7) of the row's 128 B
    const int r8 = lane >> 3, p8 = lane & 7;
    auto issue = [&](int js) {
        const unsigned dst = lbase + (js & 1) * kH3Step + wave * 4096;
#pragma unroll
        for (int part = 0; part < 2; ++part)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r0 = 8 * i;
                const int c = p8 ^ (((r0 + r8) >> 1) & 7);
                lds_dma16_at(p.w + (int64_t)(kH3Rows * js + r0) * 1536 + 1024 * part + 64 * wave,
                             (unsigned)(r8 * 1536 * 2 + c * 16), dst + part * kH3Part + r0 * 128);
            }
    };
    issue(0);
    // this lane's rows: xh[kb] = x_hi[tok][32 kb + 8 g .. + 8], xl[kb] the same of x_lo
    bf16x8 xh[16], xl[16];
    {
        const __bf16 *xr = p.x + m * p.xs_m + (int64_t)tok * p.xs_t + 8 * g;
#pragma unroll
        for (int kb = 0; kb < 16; ++kb) {
            xh[kb] = load_bf16x8(xr + 32 * kb);
            xl[kb] = load_bf16x8(xr + 512 + 32 * kb);
        }
    }
    const int64_t tgt = p.targets[m * p.targets_sm + tok];
    const float corr = PERT ? p.pop.sign[m] * p.dots[row] : 0.f;
    const float *arow = PERT ? p.r1.a + dir * p.r1.a_stride + 4 * g : nullptr;
    const float k1 = (2.0f / 15.0f) * kLog2e;     // u = 2^(k1 l) = e^(2 l / 15)
    const float c2 = 1.0f / (-30.0f * kLog2e);    // rcp(c2 (1 + u)) = -30 log2(e) / (1 + u) = log2 e^(z - 15)
    float sum = 0.f, zl = 0.f;                    // sum of e^(z - 15) over this lane's rows; the target's logit
    vm_wait<0>();
    __syncthreads();
    const int nsteps = p.vocab / kH3Rows;
    const int fr = lane & 15, fc = lane >> 4;
    constexpr int kA = HEAD3_AHEAD;
#pragma unroll 1
    for (int js = 0; js < nsteps; ++js) {
        if (js + 1 < nsteps) issue(js + 1);  // its buffer was last read in step js - 1, before the barrier below
        const char *buf = lds + (js & 1) * kH3Step;
        // fragment f = 4 kb + 2 vb + part: rows 16 vb .. + 16 of segment part, k block kb
        auto frag = [&](int f) {
            const int kb = f >> 2, vb = (f >> 1) & 1, part = f & 1;
            const int r = 16 * vb + fr, c = 4 * (kb & 1) + fc;
            return *reinterpret_cast<const bf16x8 *>(buf + part * kH3Part + (kb >> 1) * 4096 + r * 128 +
                                                     ((c ^ ((r >> 1) & 7)) << 4));
        };
        f32x4 acc[2] = {f32x4{}, f32x4{}};
        bf16x8 a[kA + 2];
#pragma unroll
        for (int i = 0; i < kA; ++i) a[i] = frag(i);
#pragma unroll
        for (int f = 0; f < 64; f += 2) {
            // the two fragments of (kb, vb) are f and f + 1; the reads run kA fragments ahead
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (f + kA + i < 64) a[(f + kA + i) % (kA + 2)] = frag(f + kA + i);
            const int kb = f >> 2, vb = (f >> 1) & 1;
            const bf16x8 ah = a[f % (kA + 2)], al = a[(f + 1) % (kA + 2)];
            acc[vb] = mfma16x16x32(ah, xh[kb], acc[vb]);
            acc[vb] = mfma16x16x32(ah, xl[kb], acc[vb]);
            acc[vb] = mfma16x16x32(al, xh[kb], acc[vb]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // register r of block vb holds vocabulary row v0 + 16 vb + 4 g + r
        const int v0 = kH3Rows * js;
        float4 a4[2] = {float4{0.f, 0.f, 0.f, 0.f}, float4{0.f, 0.f, 0.f, 0.f}};
        if constexpr (PERT) {
            a4[0] = ld4(arow + v0);
            a4[1] = ld4(arow + v0 + 16);
        }
        auto logit = [&](int vb, int r) {
            float x = acc[vb][r];
            if constexpr (PERT) x = __builtin_fmaf(corr, f4get(a4[vb], r), x);
            return x;
        };
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float u = exp2_fast(logit(vb, r) * k1);
                sum += exp2_fast(__builtin_amdgcn_rcpf(__builtin_fmaf(u, c2, c2)));
            }
        // the target's logit, in the steps whose rows hold some lane's target (-1 and out-of-range ids never do)
        const bool here = (uint64_t)(tgt - v0) < (uint64_t)kH3Rows;
        if (__builtin_amdgcn_ballot_w64(here)) {
            const int d = here ? (int)(tgt - v0) - 4 * g : -1;
#pragma unroll
            for (int vb = 0; vb < 2; ++vb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (d == 16 * vb + r) zl = logit(vb, r);
        }
        vm_wait<0>();
        __syncthreads();  // step js + 1 landed for every wave; every wave is done with buffer js & 1
    }
    // the four lanes of a token: sums add; exactly one of them holds the target's row (the others hold 0)
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    zl += __shfl_xor(zl, 16, 64);
    zl += __shfl_xor(zl, 32, 64);
    if (g == 0) {
        const float z = 15.0f - 30.0f / (exp2_fast(zl * k1) + 1.0f);
        const float ce = 15.0f + __logf(sum) - z;
        p.loss[row] = tgt == -1 ? 0.f : (tgt < 0 || tgt >= p.vocab ? __builtin_nanf("") : ce);
    }
}

Pop make_pop(const noise_population_t *pp) {
    Pop p;
    p.members = (int)pp->members;
    p.tokens = (int)pp->tokens;
    p.sign = pp->sign;
    p.dir_div = (int)pp->dir_div;
    return p;
}

Rank1 make_r1(const noise_rank1_t *r) {
    Rank1 o{nullptr, nullptr, 0, 0};
    if (r && r->a) {
        o.a = r->a;
        o.b = r->b;
        o.a_stride = r->a_stride;
        o.b_stride = r->b_stride;
    }
    return o;
}

int check_pop(const noise_population_t *pp, int tile, const char *fn) {
    NOISE_CHECK_ARG(pp != nullptr, "%s: population is NULL", fn);
    NOISE_CHECK_ARG(pp->members > 0 && pp->tokens > 0, "%s: members and tokens must be positive", fn);
    NOISE_CHECK_ARG(pp->tokens % tile == 0, "%s: tokens (%lld) must be a multiple of %d", fn, (long long)pp->tokens, tile);
    NOISE_CHECK_ARG(pp->dir_div >= 1, "%s: dir_div must be >= 1", fn);
    NOISE_CHECK_ARG(pp->members * pp->tokens < (1ll << 31), "%s: members * tokens must stay below 2^31", fn);
    NOISE_CHECK_ARG(pp->rounding == NOISE_ROUNDING_FUSED || pp->rounding == NOISE_ROUNDING_EAGER,
                    "%s: unknown rounding mode %lld", fn, (long long)pp->rounding);
    return NOISE_OK;
}

bool eager(const noise_population_t *pp) { return pp->rounding == NOISE_ROUNDING_EAGER; }

int check_view(const noise_view_t &v, const char *fn, const char *name) {
    NOISE_CHECK_ARG(v.ptr != nullptr, "%s: %s is NULL", fn, name);
    NOISE_CHECK_ARG(aligned(v.ptr, 16) && v.sm % 8 == 0 && v.st % 8 == 0,
                    "%s: %s must be 16 B aligned with strides multiple of 8 elements", fn, name);
    return NOISE_OK;
}

template <int KD, bool MIX>
void launch_resid_mix(const ResidArgs &a, dim3 grid, hipStream_t s) {
    switch (a.nnext) {
        case 0: hipLaunchKernelGGL((resid_kernel<KD, MIX, 0>), grid, dim3(kThreads), 0, s, a); break;
        case 1: hipLaunchKernelGGL((resid_kernel<KD, MIX, 1>), grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((resid_kernel<KD, MIX, 2>), grid, dim3(kThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((resid_kernel<KD, MIX, 3>), grid, dim3(kThreads), 0, s, a); break;
    }
}

template <int KD>
void launch_resid(const ResidArgs &a, dim3 grid, hipStream_t s, bool eager) {
    if (eager) {
        if (a.mix)
            hipLaunchKernelGGL((resid_kernel<KD, true, 0, false, true>), grid, dim3(kThreads), 0, s, a);
        else
            hipLaunchKernelGGL((resid_kernel<KD, false, 0, false, true>), grid, dim3(kThreads), 0, s, a);
    } else if (a.mix)
        launch_resid_mix<KD, true>(a, grid, s);
    else
        launch_resid_mix<KD, false>(a, grid, s);
}

#define NOISE_TRY(x)                 \
    do {                             \
        int _s = (x);                \
        if (_s != NOISE_OK) return _s; \
    } while (0)

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_pop_qkv(const noise_population_t *pop, noise_view_t x, const void *const w[3],
                             const noise_rank1_t r1[3], const float *dots, const void *rope_cos, const void *rope_sin,
                             const float *ve, int64_t vocab, const int64_t *idx, int64_t idx_sm, const float *gates,
                             const noise_rank1_t *ve_noise, void *const out[3], noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_qkv";
    NOISE_TRY(check_pop(pop, 256, fn));
    NOISE_TRY(check_view(x, fn, "x"));
    NOISE_CHECK_ARG(w && out && rope_cos && rope_sin, "%s: NULL weight/output/rotary pointer", fn);
    NOISE_CHECK_ARG(aligned(rope_cos, 16) && aligned(rope_sin, 16), "%s: rotary tables must be 16 B aligned", fn);
    for (int i = 0; i < 3; ++i) {
        NOISE_CHECK_ARG(w[i] && out[i] && aligned(w[i], 16) && aligned(out[i], 8), "%s: weight/output %d NULL or misaligned", fn, i);
        NOISE_CHECK_ARG(!r1 || !r1[i].a || (dots && pop->sign && aligned(r1[i].a, 16) && r1[i].a_stride % 4 == 0),
                        "%s: perturbed matrix %d needs dots, sign and 16 B aligned a rows", fn, i);
    }
    NOISE_CHECK_ARG(!ve || (idx && gates && vocab > 0), "%s: value embeddings need idx, gates and vocab", fn);
    NOISE_CHECK_ARG(idx_sm == 0 || idx_sm >= pop->tokens, "%s: idx_sm must be 0 or >= tokens", fn);
    NOISE_CHECK_ARG(!eager(pop) || ((!r1 || (!r1[0].a && !r1[1].a && !r1[2].a)) && (!ve_noise || !ve_noise->a)),
                    "%s: eager rounding is for unperturbed calls", fn);
    QkvArgs a;
    a.pop = make_pop(pop);
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    for (int i = 0; i < 3; ++i) {
        a.w[i] = (const __bf16 *)w[i];
        a.r1[i] = make_r1(r1 ? &r1[i] : nullptr);
        a.out[i] = (__bf16 *)out[i];
    }
    a.dots = dots; a.cos_t = (const __bf16 *)rope_cos; a.sin_t = (const __bf16 *)rope_sin; a.ve = ve; a.ve_m = 0; a.idx = idx;
    a.idx_m = idx_sm;
    a.vocab = vocab;
    a.gates = gates;
    a.ve_r1 = make_r1(ve ? ve_noise : nullptr);
    NOISE_CHECK_ARG(!a.ve_r1.a || (pop->sign && aligned(a.ve_r1.b, 16) && a.ve_r1.b_stride % 4 == 0),
                    "%s: value-embedding noise b rows must be 16 B aligned", fn);
    if (!eager(pop) && aligned(out[0], 16) && aligned(out[1], 16) && aligned(out[2], 16))
        return qkv_rows_launch(pop, x, w, r1, dots, rope_cos, rope_sin, ve, vocab, idx, idx_sm, gates, ve_noise, out,
                               stream);
    dim3 grid((unsigned)(6 * pop->members * (pop->tokens / 256)));
    if (eager(pop))
        hipLaunchKernelGGL(qkv_kernel<true>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(qkv_kernel<false>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    return launch_status(fn);
}

extern "C" int noise_pop_qkv_shared(const noise_population_t *pop, const float *base, const noise_rank1_t r1[3],
                                    const float *dots, const void *rope_cos, const void *rope_sin, void *const out[3],
                                    noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_qkv_shared";
    NOISE_TRY(check_pop(pop, 64, fn));
    NOISE_CHECK_ARG(!eager(pop), "%s: eager rounding has per-member inputs; use noise_pop_qkv", fn);
    NOISE_CHECK_ARG(base && aligned(base, 16), "%s: base must be a 16 B aligned [tokens][1536] fp32 array", fn);
    NOISE_CHECK_ARG(out && rope_cos && rope_sin && aligned(rope_cos, 16) && aligned(rope_sin, 16),
                    "%s: NULL output, or rotary tables not 16 B aligned", fn);
    NOISE_CHECK_ARG(pop->members * 8 * (pop->tokens / 64) < (1ll << 31), "%s: too many workgroups", fn);
    QkvSharedArgs a;
    a.pop = make_pop(pop);
    a.base = base;
    for (int i = 0; i < 3; ++i) {
        NOISE_CHECK_ARG(out[i] && aligned(out[i], 16), "%s: output %d NULL or not 16 B aligned", fn, i);
        NOISE_CHECK_ARG(!r1 || !r1[i].a || (dots && pop->sign && aligned(r1[i].a, 16) && r1[i].a_stride % 4 == 0),
                        "%s: perturbed matrix %d needs dots, sign and 16 B aligned a rows", fn, i);
        a.r1[i] = make_r1(r1 ? &r1[i] : nullptr);
        a.out[i] = (__bf16 *)out[i];
    }
    a.dots = dots;
    a.cos_t = (const __bf16 *)rope_cos;
    a.sin_t = (const __bf16 *)rope_sin;
    hipLaunchKernelGGL(qkv_shared_kernel, dim3((unsigned)(pop->members * 8 * (pop->tokens / 64))), dim3(256), 0,
                       (hipStream_t)stream, a);
    return launch_status(fn);
}

extern "C" int noise_pop_residual(const noise_population_t *pop, noise_view_t x, const void *w, int64_t K,
                                  const noise_rank1_t *r1, const float *dots, int64_t dots_stride, int64_t dots_count,
                                  noise_view_t xres, float *xout, int mix, const float *lam_r, const float *lam_x,
                                  const float *eps_r, const float *eps_x, int64_t eps_stride, noise_view_t x0,
                                  void *hout, int split3, const noise_rank1_t *next, int64_t nnext, float *next_dots,
                                  noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_residual";
    NOISE_TRY(check_pop(pop, 128, fn));
    NOISE_TRY(check_view(x, fn, "x"));
    NOISE_CHECK_ARG(w && aligned(w, 16) && (K == 512 || K == 2048), "%s: w must be 16 B aligned and K 512 or 2048", fn);
    NOISE_CHECK_ARG(xres.ptr && aligned(xres.ptr, 16) && xres.sm % 4 == 0 && xres.st % 4 == 0, "%s: bad xres", fn);
    NOISE_CHECK_ARG(!xout || aligned(xout, 16), "%s: xout must be 16 B aligned", fn);
    NOISE_CHECK_ARG(!mix || (x0.ptr && aligned(x0.ptr, 16) && x0.sm % 4 == 0 && x0.st % 4 == 0), "%s: mix needs x0", fn);
    NOISE_CHECK_ARG(!mix || (lam_r && lam_x), "%s: mix needs the mixing scalars lam_r, lam_x", fn);
    NOISE_CHECK_ARG(hout && aligned(hout, 8), "%s: hout NULL or misaligned", fn);
    NOISE_CHECK_ARG(nnext >= 0 && nnext <= 3 && (nnext == 0 || (next && next_dots)), "%s: bad next-dot request", fn);
    NOISE_CHECK_ARG(!r1 || !r1->a || (dots && pop->sign && dots_count >= 1 && aligned(r1->a, 16) && r1->a_stride % 4 == 0),
                    "%s: perturbation needs dots, sign and 16 B aligned a rows", fn);
    NOISE_CHECK_ARG(!(eps_r || eps_x) || pop->sign, "%s: mixing-scalar noise needs sign", fn);
    NOISE_CHECK_ARG(!eager(pop) || ((!r1 || !r1->a) && !eps_r && !eps_x && nnext == 0 && !split3),
                    "%s: eager rounding is for unperturbed calls with a bf16 head input", fn);
    ResidArgs a;
    a.pop = make_pop(pop);
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    a.w = (const __bf16 *)w; a.K = (int)K;
    a.r1 = make_r1(r1);
    a.dots = dots; a.dots_stride = dots_stride; a.dots_count = (int)dots_count;
    a.xres = (const float *)xres.ptr; a.xr_m = xres.sm; a.xr_t = xres.st;
    a.xout = xout;
    a.mix = mix; a.lam_r = lam_r; a.lam_x = lam_x; a.eps_r = eps_r; a.eps_x = eps_x; a.eps_stride = eps_stride;
    a.x0 = (const float *)x0.ptr; a.x0_m = x0.sm; a.x0_t = x0.st;
    a.hout = (__bf16 *)hout; a.split3 = split3;
    a.nnext = (int)nnext; a.ndots = next_dots;
    a.jit = nullptr; a.jit_m = 0; a.jit_t = 0;
    for (int k = 0; k < 3; ++k) {
        a.nb[k] = (k < nnext) ? next[k].b : nullptr;
        a.nb_stride[k] = (k < nnext) ? next[k].b_stride : 0;
        if (k < nnext)
            NOISE_CHECK_ARG(next[k].b && aligned(next[k].b, 16) && next[k].b_stride % 4 == 0,
                            "%s: next b %d NULL or misaligned", fn, k);
    }
    dim3 grid((unsigned)(pop->members * (pop->tokens / 128)));
    if (K == 512)
        launch_resid<512>(a, grid, (hipStream_t)stream, eager(pop));
    else
        launch_resid<2048>(a, grid, (hipStream_t)stream, eager(pop));
    return launch_status(fn);
}

extern "C" int noise_pop_fc(const noise_population_t *pop, noise_view_t x, const void *w, const noise_rank1_t *r1,
                            const float *dots, void *act, const noise_rank1_t *next, float *partial_dots,
                            noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_fc";
    NOISE_TRY(check_pop(pop, 256, fn));
    NOISE_TRY(check_view(x, fn, "x"));
    NOISE_CHECK_ARG(w && aligned(w, 16) && act && aligned(act, 8), "%s: w/act NULL or misaligned", fn);
    NOISE_CHECK_ARG(!r1 || !r1->a || (dots && pop->sign), "%s: perturbation needs dots and sign", fn);
    NOISE_CHECK_ARG(!next || !next->b || partial_dots, "%s: next b needs partial_dots", fn);
    NOISE_CHECK_ARG(!r1 || !r1->a || (aligned(r1->a, 16) && r1->a_stride % 4 == 0),
                    "%s: a rows must be 16 B aligned (stride a multiple of 4)", fn);
    NOISE_CHECK_ARG(!next || !next->b || (aligned(next->b, 16) && next->b_stride % 4 == 0),
                    "%s: next b rows must be 16 B aligned (stride a multiple of 4)", fn);
    FcArgs a;
    a.pop = make_pop(pop);
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    a.w = (const __bf16 *)w;
    a.r1 = make_r1(r1);
    a.dots = dots;
    a.act = (__bf16 *)act;
    a.nb = (next && next->b) ? next->b : nullptr;
    a.nb_stride = (next && next->b) ? next->b_stride : 0;
    a.pdots = a.nb ? partial_dots : nullptr;
    a.jit = nullptr;
    dim3 grid((unsigned)(8 * pop->members * (pop->tokens / 256)));
    if (eager(pop)) {
        NOISE_CHECK_ARG((!r1 || !r1->a) && !a.nb, "%s: eager rounding is for unperturbed calls", fn);
        hipLaunchKernelGGL((fc_kernel<false, true>), grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    } else {
        hipLaunchKernelGGL(fc_kernel<false>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    }
    return launch_status(fn);
}

extern "C" int noise_pop_linear(const noise_population_t *pop, noise_view_t x, const void *w, int64_t K, int64_t N,
                                const noise_rank1_t *r1, const float *dots, void *y, int y_fp32, int64_t ys_m,
                                int64_t ys_t, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_linear";
    NOISE_TRY(check_pop(pop, 256, fn));
    NOISE_TRY(check_view(x, fn, "x"));
    NOISE_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0 && N % 256 == 0, "%s: K must be a multiple of 64 and N of 256", fn);
    NOISE_CHECK_ARG(w && aligned(w, 16) && y && aligned(y, 16) && ys_m % 4 == 0 && ys_t % 4 == 0,
                    "%s: w/y NULL or misaligned", fn);
    NOISE_CHECK_ARG(!r1 || !r1->a || (dots && pop->sign), "%s: perturbation needs dots and sign", fn);
    LowrankArgs a;
    a.pop = make_pop(pop);
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    a.w = (const __bf16 *)w; a.K = (int)K; a.N = (int)N;
    a.r1 = make_r1(r1);
    a.dots = dots; a.y = y; a.y_fp32 = y_fp32; a.ys_m = ys_m; a.ys_t = ys_t;
    int64_t grid = (N / 256) * pop->members * (pop->tokens / 256);
    NOISE_CHECK_ARG(grid < (1ll << 31), "%s: too many tiles", fn);
    hipLaunchKernelGGL(lowrank_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream, a);
    return launch_status(fn);
}

extern "C" int noise_pop_head_ce(const noise_population_t *pop, noise_view_t x, const void *w, int64_t K,
                                 int64_t vocab, const noise_rank1_t *r1, const float *dots, const int64_t *targets,
                                 int64_t targets_sm, float *token_loss, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_head_ce";
    NOISE_TRY(check_pop(pop, 256, fn));
    NOISE_TRY(check_view(x, fn, "x"));
    NOISE_CHECK_ARG(K > 0 && K % 64 == 0 && vocab > 0 && vocab % 256 == 0, "%s: K multiple of 64, vocab of 256", fn);
    NOISE_CHECK_ARG(w && aligned(w, 16) && targets && token_loss, "%s: NULL w/targets/loss", fn);
    NOISE_CHECK_ARG(!r1 || !r1->a || (dots && pop->sign), "%s: perturbation needs dots and sign", fn);
    NOISE_CHECK_ARG(!eager(pop) || ((!r1 || !r1->a) && K == 512), "%s: eager rounding is for the unperturbed bf16 head", fn);
    HeadArgs a;
    a.pop = make_pop(pop);
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    a.w = (const __bf16 *)w; a.K = (int)K; a.vocab = (int)vocab;
    a.r1 = make_r1(r1);
    a.dots = dots; a.targets = targets; a.targets_sm = targets_sm; a.loss = token_loss;
    dim3 grid((unsigned)(pop->members * (pop->tokens / 256)));
    if (K == 512 && vocab % kHxRows == 0 && x.st % 8 == 0 && x.sm % 8 == 0) {
        // the bf16 head: token rows resident in registers, weights streamed once per 256 tokens
        if (eager(pop))
            hipLaunchKernelGGL((head_x_kernel<true, false>), grid, dim3(kHxThreads), 0, (hipStream_t)stream, a);
        else if (a.r1.a)
            hipLaunchKernelGGL((head_x_kernel<false, true>), grid, dim3(kHxThreads), 0, (hipStream_t)stream, a);
        else
            hipLaunchKernelGGL((head_x_kernel<false, false>), grid, dim3(kHxThreads), 0, (hipStream_t)stream, a);
    } else if (K == 1536 && !eager(pop) && vocab % kH3Rows == 0 && x.st % 8 == 0 && x.sm % 8 == 0) {
        // the split-bf16x3 fp32 head: hi and lo token rows resident in registers, weights streamed once per 128 tokens
        const dim3 g3((unsigned)(pop->members * (pop->tokens / kH3Tok)));
        if (a.r1.a)
            hipLaunchKernelGGL(head3_kernel<true>, g3, dim3(kH3Threads), 0, (hipStream_t)stream, a);
        else
            hipLaunchKernelGGL(head3_kernel<false>, g3, dim3(kH3Threads), 0, (hipStream_t)stream, a);
    } else if (eager(pop)) {
        hipLaunchKernelGGL(head_ce_kernel<true>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    } else {
        hipLaunchKernelGGL(head_ce_kernel<false>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    }
    return launch_status(fn);
}

// ------------------------------------------------------------------------------------------------
// DUST's block_forward (run.py:102-117): one unperturbed block over N sequences with optional per-token
// jitter at the attention output (o), the two residual writers' products (attn, mlp) and the MLP hidden
// pre-activation (fc). The same kernels as the population forward, with the rank-1 terms off:
//   h = norm(x) -> q, k, v (+ gated value embedding, rotary, q/k norm) -> attention (+ o) ->
//   x_mid = x + (y Wproj^T + attn), h2 = norm(x_mid) -> act = relu(h2 Wfc^T + fc)^2 ->
//   x_out = x_mid + (act Wout^T + mlp)
// ------------------------------------------------------------------------------------------------
namespace noise {
namespace {

__global__ __launch_bounds__(256) void rmsnorm_bf16_kernel(const float *__restrict__ x, int64_t rows,
                                                           __bf16 *__restrict__ h) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * 512 + 8 * lane;
    const float4 a = ld4(xr), b = ld4(xr + 4);
    float ss = a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z + b.w * b.w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float r = rsqrtf(ss * (1.0f / 512.0f) + kEps);
    bf16x8 v;
    v[0] = (__bf16)(a.x * r); v[1] = (__bf16)(a.y * r); v[2] = (__bf16)(a.z * r); v[3] = (__bf16)(a.w * r);
    v[4] = (__bf16)(b.x * r); v[5] = (__bf16)(b.y * r); v[6] = (__bf16)(b.z * r); v[7] = (__bf16)(b.w * r);
    *reinterpret_cast<bf16x8 *>(h + row * 512 + 8 * lane) = v;
}

// y = bf16(y + o), 8 elements per thread
__global__ __launch_bounds__(256) void add_bf16_kernel(__bf16 *__restrict__ y, const __bf16 *__restrict__ o,
                                                       int64_t n8) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    bf16x8 a = reinterpret_cast<const bf16x8 *>(y)[i];
    const bf16x8 b = reinterpret_cast<const bf16x8 *>(o)[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = (__bf16)((float)a[e] + (float)b[e]);
    reinterpret_cast<bf16x8 *>(y)[i] = a;
}

// value-embedding rows bf16 -> fp32 (the qkv epilogue's table format), and the identity token map
__global__ __launch_bounds__(256) void ve_rows_kernel(const __bf16 *__restrict__ ve, int64_t n8, float *__restrict__ out,
                                                      int64_t *__restrict__ iota, int64_t T) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < T) iota[i] = i;
    if (i >= n8) return;
    const bf16x8 a = reinterpret_cast<const bf16x8 *>(ve)[i];
    float4 lo, hi;
    lo.x = (float)a[0]; lo.y = (float)a[1]; lo.z = (float)a[2]; lo.w = (float)a[3];
    hi.x = (float)a[4]; hi.y = (float)a[5]; hi.z = (float)a[6]; hi.w = (float)a[7];
    st4(out + 8 * i, lo);
    st4(out + 8 * i + 4, hi);
}

struct DustLayout {
    int64_t h, vef, gates, q, k, v, y, xmid, h2, act, hs, iota, total;
};

DustLayout dust_layout(int64_t rows, int64_t T, bool ve) {
    DustLayout L;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
        const int64_t o = off;
        off += (bytes + 255) / 256 * 256;
        return o;
    };
    L.h = take(rows * 512 * 2);
    L.vef = ve ? take(rows * 512 * 4) : -1;
    L.gates = ve ? take(rows * 8 * 4) : -1;
    L.q = take(rows * 512 * 2);
    L.k = take(rows * 512 * 2);
    L.v = take(rows * 512 * 2);
    L.y = take(rows * 512 * 2);
    L.xmid = take(rows * 512 * 4);
    L.h2 = take(rows * 512 * 2);
    L.act = take(rows * 2048 * 2);
    L.hs = take(rows * 512 * 2);
    L.iota = ve ? take(T * 8) : -1;
    L.total = off;
    return L;
}

}  // namespace
}  // namespace noise

extern "C" int64_t noise_dust_block_workspace_bytes(int64_t sequences, int64_t tokens, int with_ve) {
    if (sequences < 1 || tokens < 1) return -1;
    return dust_layout(sequences * tokens, tokens, with_ve != 0).total;
}

extern "C" int noise_dust_block(const float *x, float *x_out, int64_t sequences, int64_t tokens,
                                const void *const w[7], const void *ve, const void *rope_cos, const void *rope_sin,
                                int64_t window, const void *jit_o, const void *jit_attn, const void *jit_fc,
                                const void *jit_mlp, void *workspace, int64_t workspace_bytes,
                                noise_stream_t stream) {
    clear_error();
    return noise::dust_block_run(x, x_out, sequences, tokens, w, ve, rope_cos, rope_sin, window, jit_o, jit_attn,
                                 jit_fc, jit_mlp, workspace, workspace_bytes, stream, "noise_dust_block");
}

// The DUST block chain over a caller-provided workspace (both dust-block entry points run it).
int noise::dust_block_run(const float *x, float *x_out, int64_t sequences, int64_t tokens, const void *const w[7],
                          const void *ve, const void *rope_cos, const void *rope_sin, int64_t window,
                          const void *jit_o, const void *jit_attn, const void *jit_fc, const void *jit_mlp,
                          void *workspace, int64_t workspace_bytes, noise_stream_t stream, const char *fn) {
    NOISE_CHECK_ARG(sequences >= 1 && tokens >= 256 && tokens % 256 == 0 && sequences * tokens < (1ll << 31),
                    "%s: tokens must be a positive multiple of 256 and sequences * tokens < 2^31", fn);
    NOISE_CHECK_ARG(x && x_out && aligned(x, 16) && aligned(x_out, 16), "%s: x / x_out NULL or misaligned", fn);
    NOISE_CHECK_ARG(w != nullptr, "%s: weights NULL", fn);
    for (int i = 0; i < 7; ++i)
        NOISE_CHECK_ARG(i == 3 ? (!ve || w[3] != nullptr) : (w[i] && aligned(w[i], 16)),
                        "%s: weight %d NULL or misaligned (the gate may be NULL only without value embeddings)", fn, i);
    NOISE_CHECK_ARG(!ve || aligned(ve, 16), "%s: value embeddings misaligned", fn);
    NOISE_CHECK_ARG(rope_cos && rope_sin && aligned(rope_cos, 16) && aligned(rope_sin, 16), "%s: rotary tables", fn);
    const void *jit[4] = {jit_o, jit_attn, jit_fc, jit_mlp};
    for (int i = 0; i < 4; ++i)
        NOISE_CHECK_ARG(!jit[i] || aligned(jit[i], 16), "%s: jitter %d misaligned", fn, i);
    const int64_t rows = sequences * tokens;
    const DustLayout L = dust_layout(rows, tokens, ve != nullptr);
    NOISE_CHECK_ARG(workspace && aligned(workspace, 256) && workspace_bytes >= L.total,
                    "%s: workspace must be 256 B aligned and hold %lld bytes (noise_dust_block_workspace_bytes)", fn,
                    (long long)L.total);
    char *ws = static_cast<char *>(workspace);
    hipStream_t s = (hipStream_t)stream;
    __bf16 *h = (__bf16 *)(ws + L.h), *q = (__bf16 *)(ws + L.q), *k = (__bf16 *)(ws + L.k), *v = (__bf16 *)(ws + L.v);
    __bf16 *y = (__bf16 *)(ws + L.y), *h2 = (__bf16 *)(ws + L.h2), *act = (__bf16 *)(ws + L.act);
    __bf16 *hs = (__bf16 *)(ws + L.hs);
    float *xmid = (float *)(ws + L.xmid);
    noise_population_t pop{sequences, tokens, nullptr, 1};

    hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, rows, h);
    NOISE_TRY(launch_status(fn));
    float *vef = nullptr, *gates = nullptr;
    int64_t *iota = nullptr;
    if (ve) {
        vef = (float *)(ws + L.vef);
        gates = (float *)(ws + L.gates);
        iota = (int64_t *)(ws + L.iota);
        const int64_t n8 = rows * 512 / 8, work = n8 > tokens ? n8 : tokens;
        hipLaunchKernelGGL(ve_rows_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, s,
                           (const __bf16 *)ve, n8, vef, iota, tokens);
        NOISE_TRY(launch_status(fn));
        NOISE_TRY(noise_pop_gate(&pop, noise_view_t{h, tokens * 512, 512}, (const float *)w[3], nullptr, gates, stream));
    }
    {
        QkvArgs a{};
        a.pop = make_pop(&pop);
        a.x = h; a.xs_m = tokens * 512; a.xs_t = 512;
        for (int i = 0; i < 3; ++i) a.w[i] = (const __bf16 *)w[i];
        a.out[0] = q; a.out[1] = k; a.out[2] = v;
        a.cos_t = (const __bf16 *)rope_cos; a.sin_t = (const __bf16 *)rope_sin;
        a.ve = vef; a.ve_m = tokens * 512; a.idx = iota; a.idx_m = 0; a.vocab = tokens; a.gates = gates;
        hipLaunchKernelGGL(qkv_kernel<false>, dim3((unsigned)(6 * sequences * (tokens / 256))), dim3(kThreads), 0, s,
                           a);
        NOISE_TRY(launch_status(fn));
    }
    // q, k: [N][8][T][64]; v transposed [N][8][64][T]; y token-major [N][T][512]
    NOISE_TRY(noise_attention_fwd(q, k, v, y, sequences, 8, tokens, 64, 8 * tokens * 64, tokens * 64, 64,
                                  8 * tokens * 64, tokens * 64, 64, 8 * 64 * tokens, 64 * tokens, tokens,
                                  NOISE_ATTN_V_TRANSPOSED | NOISE_ATTN_QK_NORMED, tokens * 512, 64, 512, window,
                                  0.125f, nullptr, 0, 1, nullptr, stream));
    if (jit_o) {
        const int64_t n8 = rows * 512 / 8;
        hipLaunchKernelGGL(add_bf16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, y,
                           (const __bf16 *)jit_o, n8);
        NOISE_TRY(launch_status(fn));
    }
    auto resid = [&](const __bf16 *xin, int K, const void *wt, const float *xres, float *xo, __bf16 *hout,
                     const void *jt) {
        ResidArgs a{};
        a.pop = make_pop(&pop);
        a.x = xin; a.xs_m = tokens * K; a.xs_t = K;
        a.w = (const __bf16 *)wt; a.K = K;
        a.xres = xres; a.xr_m = tokens * 512; a.xr_t = 512;
        a.xout = xo; a.hout = hout;
        a.jit = (const __bf16 *)jt; a.jit_m = tokens * 512; a.jit_t = 512;
        const dim3 grid((unsigned)(sequences * (tokens / 128)));
        if (K == 512) {
            if (jt) hipLaunchKernelGGL((resid_kernel<512, false, 0, true>), grid, dim3(kThreads), 0, s, a);
            else hipLaunchKernelGGL((resid_kernel<512, false, 0>), grid, dim3(kThreads), 0, s, a);
        } else {
            if (jt) hipLaunchKernelGGL((resid_kernel<2048, false, 0, true>), grid, dim3(kThreads), 0, s, a);
            else hipLaunchKernelGGL((resid_kernel<2048, false, 0>), grid, dim3(kThreads), 0, s, a);
        }
        return launch_status(fn);
    };
    NOISE_TRY(resid(y, 512, w[4], x, xmid, h2, jit_attn));
    {
        FcArgs a{};
        a.pop = make_pop(&pop);
        a.x = h2; a.xs_m = tokens * 512; a.xs_t = 512;
        a.w = (const __bf16 *)w[5];
        a.act = act;
        a.jit = (const __bf16 *)jit_fc;
        const dim3 grid((unsigned)(8 * sequences * (tokens / 256)));
        if (jit_fc) hipLaunchKernelGGL(fc_kernel<true>, grid, dim3(kThreads), 0, s, a);
        else hipLaunchKernelGGL(fc_kernel<false>, grid, dim3(kThreads), 0, s, a);
        NOISE_TRY(launch_status(fn));
    }
    NOISE_TRY(resid(act, 2048, w[6], xmid, x_out, hs, jit_mlp));
    return NOISE_OK;
}
