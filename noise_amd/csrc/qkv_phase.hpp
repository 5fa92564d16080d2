// The q/k/v phase shared by the q/k/v kernel and the block kernel that runs the next block's q/k/v after its
// own tail: the block's normalised input rows h (16 tokens per wave, in registers as the B operand of
// v_mfma_f32_16x16x32_bf16) times c_q, c_k, c_v streamed through LDS one head (64 rows) per pair of 32 KiB
// stages, with the rank-1 terms (eggroll.py:58), the gated value embedding on V (eggroll.py:85-89), rotary and
// the per-head RMSNorm on Q and K (eggroll.py:90, utils/model.py:55-58, 46-47). The k order of h and of the
// weights' columns only has to agree: the block kernel passes h in its permuted order with the weights
// permuted the same way.
#pragma once
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
    // the gates computed in the kernel (qkv_phase<.., true>) instead of read from `gates`
    const float *gate_w;               // [8][32] fp32
    const float *gate_a, *gate_b;      // [dirs][8], [dirs][32] or NULL
    int64_t gate_a_stride, gate_b_stride;
};

// what a lane of the q/k/v phase knows about its token
struct QkvLane {
    int m, t0, tok, wave, lane, tid, dir;
    int64_t row;
    float sgn;
    float dq0, dq1, dq2;               // sign * (h . b) of c_q, c_k, c_v (0 where unperturbed)
    bf16x4 cs[2], sn[2];               // rotary rows: dims 4 g .. + 4 and 16 + 4 g .. + 4
    int64_t tv;                        // value-table row
    bool bad;                          // token id outside the table (V is NaN)
    float vesc;                        // sign * a_ve[dir][id]
};

// the phase's arguments from noise_pop_qkv's (the gates read from `gates`)
inline QkvRowsArgs qkv_rows_args(const noise_population_t *pop, noise_view_t x, const void *const w[3],
                                 const noise_rank1_t r1[3], const float *dots, const void *rope_cos,
                                 const void *rope_sin, const float *ve, int64_t vocab, const int64_t *idx,
                                 int64_t idx_sm, const float *gates, const noise_rank1_t *ve_noise, void *const out[3]) {
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
    return a;
}

__device__ __forceinline__ float token_sum4(float v) { return sum_lanes_16_32(v); }

// the per-token scalars of the phase's epilogues: rotary rows, value-table row and its noise scale
template <bool VE>
__device__ __forceinline__ void qkv_token_scalars(const QkvRowsArgs &p, QkvLane &L) {
    const int g = L.lane >> 4;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        L.cs[b] = load_bf16x4(p.cos_t + (int64_t)L.tok * 32 + 16 * b + 4 * g);
        L.sn[b] = load_bf16x4(p.sin_t + (int64_t)L.tok * 32 + 16 * b + 4 * g);
    }
    L.tv = 0;
    L.bad = false;
    L.vesc = 0.f;
    if constexpr (VE) {
        const int64_t id = p.idx[L.m * p.idx_m + L.tok];
        L.bad = id < 0 || id >= p.vocab;  // an id outside the table: no read leaves it, V is NaN
        L.tv = L.bad ? 0 : id;
        if (p.ve_a) L.vesc = L.sgn * p.ve_a[L.dir * p.ve_a_stride + L.tv];
    }
}

// h[:32] of this lane's token from the four lanes l % 16 + 16 g that hold it; x0 is k block 0 of the B operand in
// the permuted order (lane group g: features 4 g .. + 4, then 16 + 4 g .. + 4)
__device__ __forceinline__ void gather_h32(const bf16x8 &x0, int tl, float (&xg)[32]) {
    unsigned w[4];
    __builtin_memcpy(w, &x0, 16);
#pragma unroll
    for (int gq = 0; gq < 4; ++gq)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned v = (unsigned)__shfl((int)w[i], tl + 16 * gq, 64);
            const int j = 2 * i, f = j < 4 ? 4 * gq + j : 12 + 4 * gq + j;
            xg[f] = __uint_as_float(v << 16);
            xg[f + 1] = __uint_as_float(v & 0xffff0000u);
        }
}

// the gates of the 8 value heads: 2 sigmoid(h[:32] . gate_w[hd] + sign (h[:32] . gate_b[dir]) gate_a[dir][hd]), each
// summed over features 0 .. 31 in order, as noise_pop_gate sums them (eggroll.py:88, utils/model.py:89)
__device__ __forceinline__ void local_gates(const QkvRowsArgs &p, const float (&xg)[32], float sgn, int dir,
                                            float (&gates)[8]) {
    float dg = 0.f;
    if (p.gate_a) {
#pragma unroll
        for (int c = 0; c < 32; ++c) dg += xg[c] * p.gate_b[dir * p.gate_b_stride + c];
        dg *= sgn;
    }
#pragma unroll
    for (int hd = 0; hd < 8; ++hd) {
        float z = 0.f;
#pragma unroll
        for (int c = 0; c < 32; ++c) z += xg[c] * p.gate_w[hd * 32 + c];
        if (p.gate_a) z += dg * p.gate_a[dir * p.gate_a_stride + hd];
        gates[hd] = 2.0f / (1.0f + __expf(-z));
    }
}

// stage k of the phase: rows 64 (s % 8) + 32 (k % 2) .. + 32 of matrix s / 8 (s = k / 2) as [8 k tiles][32
// rows][128 B] into stage buffer k % 4 (wave w copies k tile w: 4 copies of 8 rows); chunk c of row r at
// position c ^ ((r >> 1) & 7)
__device__ __forceinline__ void qkv_issue(const QkvRowsArgs &p, unsigned lbase, int wave, int lane, int k) {
    const int r8 = lane >> 3, p8 = lane & 7;
    const int s = k >> 1;
    const __bf16 *w = p.w[s >> 3] + (int64_t)(64 * (s & 7) + 32 * (k & 1)) * kQModel + 64 * wave;
    const unsigned dst = lbase + (k & 3) * kQStage + wave * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r0 = 8 * i;
        const int c = p8 ^ (((r0 + r8) >> 1) & 7);
        lds_dma16_at(w + (int64_t)r0 * kQModel, (unsigned)(r8 * kQModel * 2 + c * 16), dst + r0 * 128);
    }
}

// The phase itself; stages 0 .. 2 are issued and stage 0 has landed for every wave (a barrier) when it starts.
// GATE_LOCAL: the V heads' gates computed from h[:32] (xf in the permuted k order) instead of read from p.gates.
template <bool VE, bool GATE_LOCAL>
__device__ __forceinline__ void qkv_phase(const QkvRowsArgs &p, char *lds, const bf16x8 (&xf)[16], const QkvLane &L) {
    const int T = p.tokens, m = L.m, t0 = L.t0, wave = L.wave, lane = L.lane, tid = L.tid, dir = L.dir;
    const int tl = lane & 15, g = lane >> 4;
    const int64_t row = L.row;
    const unsigned lbase = lds_addr(lds);
    const float dq[3] = {L.dq0, L.dq1, L.dq2};
    const bf16x4 cs[2] = {L.cs[0], L.cs[1]}, sn[2] = {L.sn[0], L.sn[1]};
    const int64_t tv = L.tv;
    const bool bad = L.bad;
    const float vesc = L.vesc;
    const int fr = lane & 15, fc = lane >> 4;
    auto issue = [&](int k) { qkv_issue(p, lbase, wave, lane, k); };
    auto frag = [&](const char *buf, int rb, int kb) {
        const int r = 16 * rb + fr, c = 4 * (kb & 1) + fc;
        return *reinterpret_cast<const bf16x8 *>(buf + (kb >> 1) * 4096 + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
    };
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
            store_bf16x8_nt(dst + r * 64 + ch * 8,
                         *reinterpret_cast<const bf16x8 *>(qk_stg + r * 128 + ((ch ^ (r & 7)) << 4)));
        }
    };
    auto flush_vt = [&](int s) {
        const int hd = s & 7;
        __bf16 *dst = p.out[2] + ((int64_t)(m * 8 + hd) * 64) * T + t0;
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int c = it * 512 + tid, d = c >> 4, ch = c & 15;
            store_bf16x8_nt(dst + (int64_t)d * T + 8 * ch,
                         *reinterpret_cast<const bf16x8 *>(vt_stg + d * 256 + ((ch ^ ((d >> 2) & 15)) << 4)));
        }
    };

    // GATE_LOCAL: the token's 8 value-head gates, once for the phase (NaN for a token id outside the table)
    float gates[8];
    if constexpr (VE && GATE_LOCAL) {
        float xg[32];
        gather_h32(xf[0], tl, xg);
        local_gates(p, xg, L.sgn, dir, gates);
#pragma unroll
        for (int hd = 0; hd < 8; ++hd) gates[hd] = bad ? __builtin_nanf("") : gates[hd];
    }
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
            if (h == 0) {
                // the head's epilogue inputs, issued a stage before the epilogue: waiting for them then also waits
                // only for copies that had a stage to land (the vector memory counter retires in issue order)
                if (p.a[mat]) {
                    const float *ar = p.a[mat] + dir * p.a_stride[mat] + 64 * hd + 4 * g;
#pragma unroll
                    for (int b = 0; b < 4; ++b) av[b] = ld4(ar + 16 * b);
                }
                if constexpr (VE) {
                    if (mat == 2) {
                        if constexpr (GATE_LOCAL) {
                            gate = gates[0];
#pragma unroll
                            for (int i = 1; i < 8; ++i) gate = hd == i ? gates[i] : gate;
                        } else {
                            gate = bad ? __builtin_nanf("") : p.gates[row * 8 + hd];
                        }
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
}  // namespace noise
