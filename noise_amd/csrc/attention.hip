// Causal attention with a left window, forward only, bf16 in / fp32 accumulate / bf16 out.
//
// Replaces utils/model.py:24-31 `attention(q, k, v, window)` (flex_attention over the block mask of
// model.py:17-21, q >= k and q - k <= window, scale 1/sqrt(D) = torch's flex default,
// torch: nn/attention/flex_attention.py:1543-1544). Tensors are [batch, token, head, dim] in the
// reference; here any strides with a contiguous head dim (and, for V, optionally the transposed
// [.., dim, token] layout the population path writes).
//
// Work decomposition: one 256-thread workgroup per (batch*head, 256-query tile); each of its 4 waves owns
// 64 queries. Per 64-key tile a wave computes S^T = K Q^T (2x2 blocks of v_mfma_f32_32x32x16_bf16,
// 4 k-steps over D = 64), so a lane holds 32 scores of one query and the row max / sum need only one
// exchange with lane ^ 32. P = exp2(S*scale*log2e - m) is fed, in registers, as the B operand of
// O^T = V^T P^T, with the key index permuted identically in V^T (read from LDS) so no LDS round trip
// is needed. K and V^T tiles are double buffered in LDS (rows padded to 144 B: conflict-free 16 B reads).
// Key tiles outside every query's band are skipped; masking is applied only on band-edge tiles.
// All query tiles of one head run on one XCD (workgroups are dispatched round-robin over the 8 XCDs),
// heaviest tile first, so that head's K/V stay in that XCD's L2.
#include "common.hpp"
#include "mfma.hpp"

namespace noise {
namespace {

constexpr int kD = 64;
constexpr int kBKV = 64;
constexpr int kWaves = 4;
constexpr int kQW = 64;                 // queries per wave
constexpr int kBQ = kWaves * kQW;       // queries per workgroup
constexpr int kLds = 72;                // padded LDS row (bf16)
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const __bf16 *q, *k, *v;
    __bf16 *o;
    int64_t qs_b, qs_h, qs_t;
    int64_t ks_b, ks_h, ks_t;
    int64_t vs_b, vs_h, vs_x;           // vs_x: token stride (natural) or dim stride (transposed)
    int64_t os_b, os_h, os_t;
    int heads, seq, qtiles, bh_total;
    int window;
    int xcd_grouped;                    // 1: bh_total % 8 == 0, map heads onto XCDs
    float scale_log2;                   // softmax scale * log2(e)
    // optional fused output: dot[b, t, h] = sum_d O[b,t,h,d] * dvec[(b / ddiv) * ds_b + h*D + d]
    const float *dvec;
    float *dot;
    int64_t ds_b;
    int ddiv;
};

template <bool VT>
__device__ __forceinline__ void load_tile_regs(const AttnArgs &a, const __bf16 *Kb, const __bf16 *Vb, int k0,
                                               int tid, bf16x8 (&kr)[2], bf16x8 (&vr)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int c = tid + 256 * i;
        int row = c >> 3, ch = c & 7;
        int kv = k0 + row;
        kr[i] = kv < a.seq ? load_bf16x8(Kb + (int64_t)kv * a.ks_t + ch * 8) : zero_bf16x8();
        if (VT) {
            // V^T: row = dim, chunk = 8 consecutive keys
            int kk = k0 + ch * 8;
            const __bf16 *src = Vb + (int64_t)row * a.vs_x + kk;
            if (kk + 8 <= a.seq) {
                vr[i] = load_bf16x8(src);
            } else {
                bf16x8 t = zero_bf16x8();
                for (int e = 0; e < 8; ++e)
                    if (kk + e < a.seq) t[e] = src[e];
                vr[i] = t;
            }
        } else {
            // natural V: row = key, chunk = 8 consecutive dims
            vr[i] = kv < a.seq ? load_bf16x8(Vb + (int64_t)kv * a.vs_x + ch * 8) : zero_bf16x8();
        }
    }
}

template <bool VT>
__device__ __forceinline__ void store_tile_lds(__bf16 (*sK)[kLds], __bf16 (*sV)[kLds], int tid,
                                               const bf16x8 (&kr)[2], const bf16x8 (&vr)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int c = tid + 256 * i;
        int row = c >> 3, ch = c & 7;
        store_bf16x8(&sK[row][ch * 8], kr[i]);
        if (VT) {
            store_bf16x8(&sV[row][ch * 8], vr[i]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) sV[ch * 8 + e][row] = vr[i][e];
        }
    }
}

template <bool VT>
__global__ __launch_bounds__(256, 2) void attention_fwd_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) __bf16 sK[2][kBKV][kLds];
    __shared__ __attribute__((aligned(16))) __bf16 sV[2][kD][kLds];

    // workgroup -> (batch*head, query tile)
    int wg = blockIdx.x;
    int bh, qt;
    if (a.xcd_grouped) {
        int xcd = wg & 7, slot = wg >> 3;
        bh = (slot / a.qtiles) * 8 + xcd;
        qt = a.qtiles - 1 - (slot % a.qtiles);
    } else {
        bh = wg / a.qtiles;
        qt = a.qtiles - 1 - (wg % a.qtiles);
    }
    const int b = bh / a.heads, h = bh - b * a.heads;
    const __bf16 *Qb = a.q + b * a.qs_b + h * a.qs_h;
    const __bf16 *Kb = a.k + b * a.ks_b + h * a.ks_h;
    const __bf16 *Vb = a.v + b * a.vs_b + h * a.vs_h;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, hf = lane >> 5;
    const int T = a.seq, W = a.window;
    const int q0w = qt * kBQ + wave * kQW;

    // this wave's queries as MFMA B operands: qf[qb][s] = Q[q0w + 32qb + j][16s + 8hf .. +7]
    bf16x8 qf[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        int qrow = q0w + 32 * qb + j;
#pragma unroll
        for (int s = 0; s < 4; ++s)
            qf[qb][s] = qrow < T ? load_bf16x8(Qb + (int64_t)qrow * a.qs_t + 16 * s + 8 * hf) : zero_bf16x8();
    }

    float m[2] = {-1e30f, -1e30f}, l[2] = {0.f, 0.f};
    f32x16 o[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x16{};

    const int wg_q_lo = qt * kBQ;
    const int wg_q_hi = min(T, wg_q_lo + kBQ) - 1;
    const int kv_first = max(0, wg_q_lo - W) / kBKV;
    const int kv_last = wg_q_hi / kBKV;
    const int wq_lo = q0w, wq_hi = min(q0w + kQW, T) - 1;

    bf16x8 kr[2], vr[2];
    load_tile_regs<VT>(a, Kb, Vb, kv_first * kBKV, tid, kr, vr);
    store_tile_lds<VT>(sK[0], sV[0], tid, kr, vr);
    __syncthreads();

    for (int t = kv_first; t <= kv_last; ++t) {
        const int buf = (t - kv_first) & 1;
        const int k0 = t * kBKV;
        if (t < kv_last) load_tile_regs<VT>(a, Kb, Vb, k0 + kBKV, tid, kr, vr);

        const bool active = wq_lo <= wq_hi && k0 <= wq_hi && k0 + kBKV - 1 >= wq_lo - W;
        if (active) {
            const bool edge = (k0 + kBKV - 1 > wq_lo) || (k0 < wq_hi - W) || (k0 + kBKV > T);
            f32x16 st[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) st[kb][qb] = f32x16{};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    bf16x8 ka = load_bf16x8(&sK[buf][32 * kb + j][16 * s + 8 * hf]);
#pragma unroll
                    for (int qb = 0; qb < 2; ++qb) st[kb][qb] = mfma32x32x16(ka, qf[qb][s], st[kb][qb]);
                }
            }

            bf16x8 pf[2][4];  // [qb][s] B operands of O^T = V^T P^T
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                const int q = q0w + 32 * qb + j;
                if (edge) {
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            int kv = k0 + 32 * kb + 8 * (r >> 2) + 4 * hf + (r & 3);
                            bool vis = kv <= q && q - kv <= W && kv < T;
                            st[kb][qb][r] = vis ? st[kb][qb][r] : -__builtin_inff();
                        }
                }
                float mx = -__builtin_inff();
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[kb][qb][r]);
                mx = fmaxf(mx, swap_halves(mx));
                const float m_new = fmaxf(m[qb], mx * a.scale_log2);
                const float alpha = exp2_fast(m[qb] - m_new);
                m[qb] = m_new;
                float rs = 0.f;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float p = exp2_fast(__builtin_fmaf(st[kb][qb][r], a.scale_log2, -m_new));
                        st[kb][qb][r] = p;
                        rs += p;
                    }
                l[qb] = l[qb] * alpha + rs;
#pragma unroll
                for (int db = 0; db < 2; ++db) o[db][qb] *= alpha;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    bf16x8 v;
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = (__bf16)st[s >> 1][qb][8 * (s & 1) + e];
                    pf[qb][s] = v;
                }
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const __bf16 *row = &sV[buf][32 * db + j][0];
                    bf16x8 va = cat(load_bf16x4(row + 16 * s + 4 * hf), load_bf16x4(row + 16 * s + 8 + 4 * hf));
#pragma unroll
                    for (int qb = 0; qb < 2; ++qb) o[db][qb] = mfma32x32x16(va, pf[qb][s], o[db][qb]);
                }
            }
        }
        if (t < kv_last) store_tile_lds<VT>(sK[buf ^ 1], sV[buf ^ 1], tid, kr, vr);
        __syncthreads();
    }

    // normalise and store O[q][d], d = 32db + 8(r/4) + 4hf + (r%4): 4 consecutive dims per 8 B store
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int q = q0w + 32 * qb + j;
        float lt = l[qb] + swap_halves(l[qb]);
        float inv = lt > 0.f ? 1.0f / lt : 0.f;
        float dsum = 0.f;
        const float *dv = nullptr;
        if (a.dot) dv = a.dvec + (int64_t)(b / a.ddiv) * a.ds_b + h * kD;
        if (q < T) {
            __bf16 *orow = a.o + b * a.os_b + h * a.os_h + (int64_t)q * a.os_t;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    bf16x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = (__bf16)(o[db][qb][4 * g + e] * inv);
                    const int d = 32 * db + 8 * g + 4 * hf;
                    store_bf16x4(orow + d, v);
                    if (dv) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) dsum += (float)v[e] * dv[d + e];
                    }
                }
        }
        if (a.dot) {
            dsum += swap_halves(dsum);
            if (q < T && hf == 0) a.dot[((int64_t)b * T + q) * a.heads + h] = dsum;
        }
    }
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_attention_fwd(const void *q, const void *k, const void *v, void *o, int64_t batch,
                                   int64_t heads, int64_t seq, int64_t head_dim, int64_t qs_b, int64_t qs_h,
                                   int64_t qs_t, int64_t ks_b, int64_t ks_h, int64_t ks_t, int64_t vs_b,
                                   int64_t vs_h, int64_t vs_x, int v_transposed, int64_t os_b, int64_t os_h,
                                   int64_t os_t, int64_t window, float scale, const float *dot_vec,
                                   int64_t dot_vec_stride, int64_t dot_div, float *dot_out,
                                   noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(head_dim == kD, "noise_attention_fwd: head_dim must be 64, got %lld", (long long)head_dim);
    NOISE_CHECK_ARG(batch >= 0 && heads > 0 && seq >= 0, "noise_attention_fwd: bad batch/heads/seq");
    NOISE_CHECK_ARG(seq <= (1 << 30) && window >= 0, "noise_attention_fwd: seq too large or window < 0");
    if (batch == 0 || seq == 0) return NOISE_OK;
    NOISE_CHECK_ARG(q && k && v && o, "noise_attention_fwd: NULL tensor pointer");
    NOISE_CHECK_ARG(aligned(q, 16) && aligned(k, 16) && aligned(o, 8) && aligned(v, v_transposed ? 2 : 16),
                    "noise_attention_fwd: q, k (16 B), o (8 B) and v must be aligned");
    NOISE_CHECK_ARG(qs_t % 8 == 0 && ks_t % 8 == 0 && qs_b % 8 == 0 && qs_h % 8 == 0 && ks_b % 8 == 0 &&
                        ks_h % 8 == 0 && os_t % 4 == 0 && os_b % 4 == 0 && os_h % 4 == 0,
                    "noise_attention_fwd: q/k strides must be multiples of 8 elements, o strides of 4");
    if (v_transposed) {
        NOISE_CHECK_ARG(vs_x % 8 == 0 && vs_b % 8 == 0 && vs_h % 8 == 0 && aligned(v, 16),
                        "noise_attention_fwd: transposed v needs 16 B alignment and strides multiple of 8");
    } else {
        NOISE_CHECK_ARG(vs_x % 8 == 0 && vs_b % 8 == 0 && vs_h % 8 == 0,
                        "noise_attention_fwd: v strides must be multiples of 8 elements");
    }
    NOISE_CHECK_ARG(dot_out == nullptr || (dot_vec != nullptr && dot_div >= 1),
                    "noise_attention_fwd: dot_out needs dot_vec and dot_div >= 1");
    int64_t bh = batch * heads;
    int64_t qtiles = (seq + kBQ - 1) / kBQ;
    NOISE_CHECK_ARG(bh * qtiles < (1ll << 31), "noise_attention_fwd: too many workgroups");
    AttnArgs a;
    a.q = (const __bf16 *)q; a.k = (const __bf16 *)k; a.v = (const __bf16 *)v; a.o = (__bf16 *)o;
    a.qs_b = qs_b; a.qs_h = qs_h; a.qs_t = qs_t;
    a.ks_b = ks_b; a.ks_h = ks_h; a.ks_t = ks_t;
    a.vs_b = vs_b; a.vs_h = vs_h; a.vs_x = vs_x;
    a.os_b = os_b; a.os_h = os_h; a.os_t = os_t;
    a.heads = (int)heads; a.seq = (int)seq; a.qtiles = (int)qtiles; a.bh_total = (int)bh;
    a.window = (int)(window > seq ? seq : window);
    a.xcd_grouped = (bh % 8 == 0) ? 1 : 0;
    a.scale_log2 = scale * kLog2e;
    a.dvec = dot_vec; a.dot = dot_out; a.ds_b = dot_vec_stride; a.ddiv = (int)dot_div;
    dim3 grid((unsigned)(bh * qtiles));
    if (v_transposed)
        hipLaunchKernelGGL(attention_fwd_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(attention_fwd_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, a);
    return launch_status("noise_attention_fwd");
}
