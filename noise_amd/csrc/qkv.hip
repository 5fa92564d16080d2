// Q, K, V of a population block with two waves per SIMD (eggroll.py:81-90): the block's normalised input
// times c_q, c_k, c_v, the rank-1 terms (eggroll.py:58), the gated value embedding on V (eggroll.py:85-89),
// rotary and the per-head RMSNorm on Q and K (eggroll.py:90, utils/model.py:55-58, 46-47).
//
// A workgroup owns 128 tokens of one member in 8 waves of 16 tokens (v_mfma_f32_16x16x32_bf16, weights as
// the A operand): each wave keeps its 16 input rows in registers (64) and the three matrices stream through
// LDS one head (64 rows) per pair of 32 KiB stages (stage 2s: rows 64 hd .. + 32, stage 2s + 1: the next 32;
// heads 0-7 of Q, then K, then V), through four stage buffers by whole-line copies into XOR-swizzled rows.
// A head's 64 x 16 block sits in four 16 x 16 accumulators (lane l: token l % 16, features 16 b + 4 (l / 16)
// + 0..3): the rotary pairs (d, d + 32) are the same register of blocks b and b + 2, and the head's RMSNorm
// needs two exchanges (lane ^ 16, lane ^ 32). The head's epilogue inputs (rank-1 a, value-table rows) are
// loaded at the start of its second stage so that they arrive under the products. Q and K heads are staged
// per wave and stored as whole 128 B rows; V^T is staged for the whole workgroup ([64 dims][128 tokens]) and
// stored as 256 B row segments, at the start of the next stage.
#include "common.hpp"
#include "mfma.hpp"
#include "tile.hpp"

namespace noise {
namespace {

constexpr float kQkvEps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps
constexpr int kQThreads = 512, kQTok = 128, kQModel = 512;
constexpr int kQStage = 32768;
constexpr int kQStages = 48;            // 24 heads x 2
constexpr int kQVt = 4 * kQStage;       // V^T staging [64 dims][128 tokens] bf16 (16 KiB)
constexpr int kQQk = kQVt + 16384;      // Q / K staging per wave [16 tokens][128 B] (2 KiB)
constexpr int kQLds = kQQk + 8 * 2048;  // 160 KiB
static_assert(kQLds <= 160 * 1024, "LDS of one CU");
// fragment reads in flight ahead of the product that uses them; each product ends a scheduling region so that
// the compiler keeps them that far ahead
#ifndef QKV_AHEAD
#define QKV_AHEAD 4
#endif
constexpr int kQAhead = QKV_AHEAD;
#ifndef QKV_PIN
#define QKV_PIN() __builtin_amdgcn_sched_barrier(0)
#endif

struct QkvRowsArgs {
    int members, tokens, dir_div;
    const float *sign;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const __bf16 *w[3];
    const float *a[3];                 // rank-1 a rows per matrix or NULL
    int64_t a_stride[3];
    const float *dots;                 // [rows][3]
    const __bf16 *cos_t, *sin_t;       // [T][32] bf16
    const float *ve;                   // [V][512] fp32 or NULL
    const int64_t *idx;
    int64_t idx_m, vocab;
    const float *gates;                // [rows][8]
    const float *ve_a, *ve_b;          // value-table noise a [dirs][V], b [dirs][512] or NULL
    int64_t ve_a_stride, ve_b_stride;
    __bf16 *out[3];                    // q, k [m][8][T][64]; v transposed [m][8][64][T]
};

__device__ __forceinline__ float token_sum4(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

template <bool VE>
__global__ __launch_bounds__(kQThreads, 1) void qkv16_kernel(QkvRowsArgs p) {
    __shared__ __attribute__((aligned(16))) char lds[kQLds];
    const int T = p.tokens, tiles_t = T / kQTok;
    const int m = blockIdx.x / tiles_t, t0 = (blockIdx.x % tiles_t) * kQTok;
    const int tid = threadIdx.x, lane = tid & 63, tl = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int dir = m / p.dir_div;
    const float sgn = p.sign ? p.sign[m] : 0.f;  // unperturbed calls may pass no signs
    const int tok = t0 + 16 * wave + tl;
    const int64_t row = (int64_t)m * T + tok;
    const unsigned lbase = lds_addr(lds);

    // stage k: rows 64 (s % 8) + 32 (k % 2) .. + 32 of matrix s / 8 (s = k / 2) as [8 k tiles][32 rows][128 B]
    // (wave w copies k tile w: 4 copies of 8 rows); chunk c of row r at position c ^ ((r >> 1) & 7)
    const int r8 = lane >> 3, p8 = lane & 7;
    auto issue = [&](int k) {
        const int s = k >> 1;
        const __bf16 *w = p.w[s >> 3] + (int64_t)(64 * (s & 7) + 32 * (k & 1)) * kQModel + 64 * wave;
        const unsigned dst = lbase + (k & 3) * kQStage + wave * 4096;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r0 = 8 * i;
            const int c = p8 ^ (((r0 + r8) >> 1) & 7);
            lds_dma16_at(w + (int64_t)r0 * kQModel, (unsigned)(r8 * kQModel * 2 + c * 16), dst + r0 * 128);
        }
    };
    const int fr = lane & 15, fc = lane >> 4;
    auto frag = [&](const char *buf, int rb, int kb) {
        const int r = 16 * rb + fr, c = 4 * (kb & 1) + fc;
        return *reinterpret_cast<const bf16x8 *>(buf + (kb >> 1) * 4096 + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
    };
    issue(0);
    issue(1);
    issue(2);
    // this lane's input row: xf[kb] = x[tok][32 kb + 8 g .. + 8]
    bf16x8 xf[16];
    {
        const __bf16 *xr = p.x + m * p.xs_m + (int64_t)tok * p.xs_t + 8 * g;
#pragma unroll
        for (int kb = 0; kb < 16; ++kb) xf[kb] = load_bf16x8(xr + 32 * kb);
    }
    // per-token scalars: rank-1 scales, the rotary rows (dims 4 g .. + 4 and 16 + 4 g .. + 4), value row and gate id
    float dq[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) dq[i] = p.a[i] ? sgn * p.dots[row * 3 + i] : 0.f;
    bf16x4 cs[2], sn[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        cs[b] = load_bf16x4(p.cos_t + (int64_t)tok * 32 + 16 * b + 4 * g);
        sn[b] = load_bf16x4(p.sin_t + (int64_t)tok * 32 + 16 * b + 4 * g);
    }
    int64_t tv = 0;
    bool bad = false;
    float vesc = 0.f;
    if constexpr (VE) {
        const int64_t id = p.idx[m * p.idx_m + tok];
        bad = id < 0 || id >= p.vocab;  // an id outside the table: no read leaves it, V is NaN
        tv = bad ? 0 : id;
        if (p.ve_a) vesc = sgn * p.ve_a[dir * p.ve_a_stride + tv];
    }
    vm_wait<8>();  // stage 0 landed (stages 1 and 2 may still be in flight); the rows and scalars above too
    __syncthreads();

    char *qk_stg = lds + kQQk + wave * 2048;
    char *vt_stg = lds + kQVt;
    int qk_pending = -1;  // head whose Q / K rows sit in this wave's staging
    int vt_pending = -1;  // head whose V^T sits in the workgroup's staging
    // whole-line stores of a staged head (called at the start of a stage: after the barrier that ended the
    // stage in which every wave staged it)
    auto flush_qk = [&](int s) {
        const int mat = s >> 3, hd = s & 7;
        __bf16 *dst = p.out[mat] + (((int64_t)m * 8 + hd) * T + t0 + 16 * wave) * 64;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int c = it * 64 + lane, r = c >> 3, ch = c & 7;
            store_bf16x8(dst + r * 64 + ch * 8,
                         *reinterpret_cast<const bf16x8 *>(qk_stg + r * 128 + ((ch ^ (r & 7)) << 4)));
        }
    };
    auto flush_vt = [&](int s) {
        const int hd = s & 7;
        __bf16 *dst = p.out[2] + ((int64_t)(m * 8 + hd) * 64) * T + t0;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int c = it * 512 + tid, d = c >> 4, ch = c & 15;
            store_bf16x8(dst + (int64_t)d * T + 8 * ch,
                         *reinterpret_cast<const bf16x8 *>(vt_stg + d * 256 + ((ch ^ ((d >> 2) & 15)) << 4)));
        }
    };

    f32x4 acc[4];
    float4 av[4], ev[4], bv[4];  // the head's epilogue inputs (rank-1 a; value rows and value-table b)
    float gate = 0.f;
#pragma unroll 1
    for (int s = 0; s < 24; ++s) {
        const int mat = s >> 3, hd = s & 7;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 2 * s + h;
            if (k + 3 < kQStages) issue(k + 3);  // into the buffer of stage k - 1 (every wave passed its barrier)
            if (qk_pending >= 0) {
                flush_qk(qk_pending);
                qk_pending = -1;
            }
            if (vt_pending >= 0) {
                flush_vt(vt_pending);
                vt_pending = -1;
            }
            if (h == 1) {
                // the epilogue's inputs, under this stage's products
                if (p.a[mat]) {
                    const float *ar = p.a[mat] + dir * p.a_stride[mat] + 64 * hd + 4 * g;
#pragma unroll
                    for (int b = 0; b < 4; ++b) av[b] = ld4(ar + 16 * b);
                }
                if constexpr (VE) {
                    if (mat == 2) {
                        gate = bad ? __builtin_nanf("") : p.gates[row * 8 + hd];
                        const float *er = p.ve + tv * 512 + 64 * hd + 4 * g;  // one value table for every member
#pragma unroll
                        for (int b = 0; b < 4; ++b) ev[b] = ld4(er + 16 * b);
                        if (p.ve_a) {
                            const float *br = p.ve_b + dir * p.ve_b_stride + 64 * hd + 4 * g;
#pragma unroll
                            for (int b = 0; b < 4; ++b) bv[b] = ld4(br + 16 * b);
                        }
                    }
                }
            }
            const char *buf = lds + (k & 3) * kQStage;
            if (h == 0) {
                acc[0] = f32x4{}; acc[1] = f32x4{}; acc[2] = f32x4{}; acc[3] = f32x4{};
            }
            {
                bf16x8 a[kQAhead + 1];
#pragma unroll
                for (int i = 0; i < kQAhead; ++i) a[i] = frag(buf, i & 1, i >> 1);
#pragma unroll
                for (int f = 0; f < 32; ++f) {
                    if (f + kQAhead < 32) a[(f + kQAhead) % (kQAhead + 1)] = frag(buf, (f + kQAhead) & 1, (f + kQAhead) >> 1);
                    acc[2 * h + (f & 1)] = mfma16x16x32(a[f % (kQAhead + 1)], xf[f >> 1], acc[2 * h + (f & 1)]);
                    QKV_PIN();
                }
            }
            if (h == 1) {
                // epilogue of head s: register r of block b holds feature 16 b + 4 g + r of the head
                if (p.a[mat]) {
                    const float corr = mat == 0 ? dq[0] : mat == 1 ? dq[1] : dq[2];
#pragma unroll
                    for (int b = 0; b < 4; ++b)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[b][r] += corr * f4get(av[b], r);
                }
                if (mat == 2) {
                    if constexpr (VE) {
                        // v += gate * (ve[idx[t], head*64 + d] (+ sign a_ve[idx[t]] b_ve[d]))   (eggroll.py:85-89)
#pragma unroll
                        for (int b = 0; b < 4; ++b)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float e = f4get(ev[b], r) + (p.ve_a ? vesc * f4get(bv[b], r) : 0.f);
                                acc[b][r] += gate * e;
                            }
                    }
                    // V^T staged as [64 dims][128 tokens]: 256 B rows, chunk c (8 tokens) of row d at c ^ ((d >> 2) & 15)
                    const int tw = 16 * wave + tl;
#pragma unroll
                    for (int b = 0; b < 4; ++b)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int d = 16 * b + 4 * g + r;
                            *reinterpret_cast<__bf16 *>(vt_stg + d * 256 + ((((tw >> 3) ^ ((d >> 2) & 15))) << 4) +
                                                        (tw & 7) * 2) = (__bf16)acc[b][r];
                        }
                    vt_pending = s;
                } else {
                    // rotary (model.py:55-58) on the pairs (d, d + 32), then RMSNorm over the head (model.py:46-47)
                    float ss = 0.f;
#pragma unroll
                    for (int b = 0; b < 2; ++b)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float c = (float)cs[b][r], sv = (float)sn[b][r];
                            const float x1 = acc[b][r], x2 = acc[b + 2][r];
                            const float o1 = x1 * c + x2 * sv, o2 = x1 * -sv + x2 * c;
                            acc[b][r] = o1;
                            acc[b + 2][r] = o2;
                            ss += o1 * o1 + o2 * o2;
                        }
                    const float rstd = rsqrtf(token_sum4(ss) * (1.0f / 64.0f) + kQkvEps);
                    // [16 tokens][64 dims] staged as 128 B rows: 16 B chunk c of row t at c ^ (t & 7)
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        bf16x4 o;
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] = (__bf16)(acc[b][r] * rstd);
                        const int c16 = 2 * b + (g >> 1);
                        store_bf16x4(reinterpret_cast<__bf16 *>(qk_stg + tl * 128 + ((c16 ^ (tl & 7)) << 4) + 8 * (g & 1)), o);
                    }
                    wave_lds_sync();  // the staged rows are read back by other lanes of the wave
                    qk_pending = s;
                }
            }
            // stage k + 1 landed for every wave (the stages issued after it may still fly); every wave is done
            // with buffer k & 3 and with the staging it filled in this stage
            vm_wait_groups<4, 2>(kQStages - 2 - k < 2 ? kQStages - 2 - k : 2);
            __syncthreads();
        }
    }
    if (qk_pending >= 0) flush_qk(qk_pending);
    if (vt_pending >= 0) flush_vt(vt_pending);
}

}  // namespace

int qkv_rows_launch(const noise_population_t *pop, noise_view_t x, const void *const w[3], const noise_rank1_t r1[3],
                    const float *dots, const void *rope_cos, const void *rope_sin, const float *ve, int64_t vocab,
                    const int64_t *idx, int64_t idx_sm, const float *gates, const noise_rank1_t *ve_noise,
                    void *const out[3], noise_stream_t stream) {
    QkvRowsArgs a{};
    a.members = (int)pop->members; a.tokens = (int)pop->tokens; a.dir_div = (int)pop->dir_div; a.sign = pop->sign;
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    for (int i = 0; i < 3; ++i) {
        a.w[i] = (const __bf16 *)w[i];
        a.a[i] = r1 && r1[i].a ? r1[i].a : nullptr;
        a.a_stride[i] = r1 && r1[i].a ? r1[i].a_stride : 0;
        a.out[i] = (__bf16 *)out[i];
    }
    a.dots = dots;
    a.cos_t = (const __bf16 *)rope_cos; a.sin_t = (const __bf16 *)rope_sin;
    a.ve = ve; a.idx = idx; a.idx_m = idx_sm; a.vocab = vocab; a.gates = gates;
    const bool vn = ve && ve_noise && ve_noise->a;
    a.ve_a = vn ? ve_noise->a : nullptr; a.ve_b = vn ? ve_noise->b : nullptr;
    a.ve_a_stride = vn ? ve_noise->a_stride : 0; a.ve_b_stride = vn ? ve_noise->b_stride : 0;
    const dim3 grid((unsigned)(pop->members * (pop->tokens / kQTok)));
    if (ve)
        hipLaunchKernelGGL(qkv16_kernel<true>, grid, dim3(kQThreads), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(qkv16_kernel<false>, grid, dim3(kQThreads), 0, (hipStream_t)stream, a);
    return launch_status("noise_pop_qkv");
}

}  // namespace noise
