// Causal attention with a left window, forward only, bf16 in / fp32 accumulate / bf16 out.
//
// Replaces utils/model.py:24-31 `attention(q, k, v, window)` (flex_attention over the block mask of
// model.py:17-21, q >= k and q - k <= window, scale 1/sqrt(D) = torch's flex default,
// torch: nn/attention/flex_attention.py:1543-1544). Tensors are [batch, token, head, dim] in the
// reference; here any strides with a contiguous head dim (and, for V, optionally the transposed
// [.., dim, token] layout the population path writes).
//
// Two kernels share one decomposition: a workgroup per (batch*head, 256-query tile), S^T = K Q^T per
// 64-key tile with v_mfma_f32_32x32x16_bf16 (4 k-steps over D = 64), so a lane holds the scores of one
// query and row reductions need one exchange with lane ^ 32; P is fed from registers as the B operand of
// O^T = V^T P^T with the key index permuted identically on both sides, so P never touches LDS.
//  - attention_fwd_kernel (any layout and length): 4 waves of 64 queries, K / V tiles register-staged
//    into double-buffered LDS (rows padded to 144 B), running-max softmax (rescaled only when the maximum
//    grows by more than 2^8).
//  - attention_vt_kernel (length a multiple of 256; V transposed, the population path, or natural, the
//    drop-in's): 8 waves of 32 queries (four waves per SIMD) in two groups half a tile apart, K and V (or V^T)
//    copied global -> LDS into a four-stage swizzled ring, and an optional fixed-shift softmax for RMS-normed
//    q, k (described at the kernel).
// Key tiles outside a wave's band are skipped; masking runs only on band-edge tiles. All query tiles of
// one head run on one XCD (workgroups are dispatched round-robin over the 8 XCDs), heaviest tile first,
// so that head's K/V stay in that XCD's L2.
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
    int tile_major;                     // 1 (transposed-V kernel, small grids): all heads' heaviest query
                                        //   tiles first, so the causal imbalance does not set the tail
    int o_lines;                        // 1: o 16 B aligned with strides multiple of 8 (staged row stores)
    float scale_log2;                   // softmax scale * log2(e)
    float shift;                        // fixed log2-domain shift of the bounded-score kernel
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
                // lazy rescale, as in the ring kernel: m moves only when a row's maximum passes it by more than
                // 8 (log2 units); the weights then stay below 2^8 and o and l share the stale m
                const float mc = mx * a.scale_log2;
                if (__builtin_amdgcn_ballot_w64(mc > m[qb] + 8.0f)) {
                    const float m_new = fmaxf(m[qb], mc);
                    const float alpha = exp2_fast(m[qb] - m_new);
                    m[qb] = m_new;
                    l[qb] *= alpha;
#pragma unroll
                    for (int db = 0; db < 2; ++db) o[db][qb] *= alpha;
                }
                const float mb = m[qb];
                float rs = 0.f;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float p = exp2_fast(__builtin_fmaf(st[kb][qb][r], a.scale_log2, -mb));
                        st[kb][qb][r] = p;
                        rs += p;
                    }
                l[qb] += rs;
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


// ------------------------------------------------------------------------------------------------
// Ring kernel (seq a multiple of 256; shown for V^T, the population layout). K and V^T tiles are copied
// global -> LDS directly (global_load_lds_dwordx4) into a ring of four stages, rows of 128 B with the
// 16 B chunks XOR-swizzled by row pair (conflict-free fragment reads). The K rows of each 32-key block
// are read in the order sigma (bits 2 and 3 of the key index swapped), which makes register r of a
// lane's S^T block hold key 16 (r / 8) + 8 hf + (r % 8): the 8 scores P^T needs as one B fragment of
// O^T = V^T P^T are consecutive keys, so V^T is read as plain 16 B fragments and P is packed with four
// v_cvt_pk_bf16_f32. BOUNDED: the caller guarantees q and k rows of RMS <= 1 (RMSNorm outputs, as
// utils/model.py:94 applies to both), so |score * scale * log2 e| <= D * scale * log2 e (+ bf16 rounding)
// = shift, and exp2(score * scale * log2 e - shift) <= 1 needs no running maximum (softmax is
// shift-invariant; fp32 and bf16 keep full relative precision down to 2^-126). There q is pre-scaled by
// scale * log2 e and the products accumulate onto -shift, so each score leaves the MFMA as its exponent, and
// the row sum is taken from the bf16 weights that P V uses (v_dot2_f32_bf16): one exp, half a pack and a
// quarter dot per score.
// ------------------------------------------------------------------------------------------------
constexpr int kStage = 2 * 64 * 128;  // K [64 keys][64 d] then V^T [64 d][64 keys], 128 B rows
constexpr int kVtQT = 256;  // queries per workgroup of the transposed-V kernel

__device__ __forceinline__ int key_sigma(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// 256 queries per workgroup in 8 waves of 32 (~120 VGPRs: four waves per SIMD with two workgroups per CU).
// Ping-pong: waves 0-3 (A) and 4-7 (B, one of each per SIMD) run the same tile sequence half a phase apart, so one wave's softmax (VALU) overlaps the other's products (MFMA) instead
// of every wave of the workgroup switching between them together after each barrier. Per barrier interval
// A does S = K Q^T, softmax, O += V^T P^T of tile t; B does the softmax and O of tile t - 1, then S of tile t.
// Both groups pass the same barriers (one per tile), placed at different points of their loops. A alone
// copies the K / V^T tiles (4 copies per wave per tile) into a 4-slot ring; after barrier t + 1 it refills
// the slot of tile t - 1, which B finished reading before that barrier.
// VNAT: V in its natural layout [.., token, dim] (the drop-in's), copied as K is, with the 16 B chunks of row R
// swizzled by 2 (R % 4) instead, and each V^T fragment put together from two transposing LDS reads.
template <bool BOUNDED, bool VNAT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void attention_vt_kernel(AttnArgs a) {
    constexpr int QT = kVtQT, NS = 4;
    constexpr int QB = 1, NW = QT / 32, QW = 32, CPW = 4;  // waves, queries per wave, copies per A wave
    __shared__ __attribute__((aligned(16))) char lds[NS * kStage];

    int wg = blockIdx.x;
    int bh, qt;
    if (a.tile_major) {
        // query tile descending, then head: with bh_total % 8 == 0 head bh still runs on XCD bh % 8
        bh = wg % a.bh_total;
        qt = a.qtiles - 1 - wg / a.bh_total;
    } else if (a.xcd_grouped) {
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

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, hf = lane >> 5;
    const int T = a.seq, W = a.window;
    const int q0w = qt * QT + wave * QW;

    bf16x8 qf[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int s = 0; s < 4; ++s) qf[qb][s] = load_bf16x8(Qb + (int64_t)(q0w + 32 * qb + j) * a.qs_t + 16 * s + 8 * hf);
    // the query fragments land before any tile copy is issued: the compiler's own wait for them inside the
    // tile loop would otherwise be a vmcnt that also drains the copies in flight
    vm_wait<0>();
    if constexpr (BOUNDED) {
        // q pre-scaled by scale * log2 e (one more bf16 rounding of q, within the shift's margin): with the
        // products accumulated onto -shift, a score leaves the MFMA as its softmax exponent
        const float c = a.scale_log2;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int e = 0; e < 8; ++e) qf[qb][s][e] = (__bf16)((float)qf[qb][s][e] * c);
    }

    // copies: per stage 16 of 1 KB (8 rows); A wave w issues copies c = 4 i + w, rows 8 (c % 8) .. of K (c < 8)
    // or V^T. Row R's slot P holds chunk P ^ ((R >> 1) & 7); for this lane R = 8 c' + lane / 8, so the chunk
    // it fetches is (lane % 8) ^ (4 (c' & 1) + lane / 16), the same for all of a wave's copies (c' & 1 = w & 1).
    const int chunk = (lane & 7) ^ (4 * (wave & 1) + (lane >> 4));
    // VNAT: row R = 8 c' + lane / 8 of a V tile keeps chunk C at slot C ^ 2 (R % 4), R % 4 = (lane / 8) % 4. The
    // four rows that one transposing read takes from each group of 16 lanes then lie in four different 32 B
    // of a 128 B row (the row-pair swizzle of K would put all four on the same banks)
    const int vchunk = VNAT ? (lane & 7) ^ (2 * ((lane >> 3) & 3)) : chunk;
    const bool group_a = wave < 4;
    const unsigned koff = (unsigned)((lane >> 3) * a.ks_t * 2 + chunk * 16);
    const unsigned voff = (unsigned)((lane >> 3) * a.vs_x * 2 + vchunk * 16);
    const unsigned lb = lds_addr(lds);
    auto issue = [&](int k0, unsigned st) {  // st: LDS byte address of the stage
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const int c = 4 * i + wave;  // A waves only: copy c's row parity is the wave's
            if (c < 8)
                lds_dma16_at(Kb + (int64_t)(k0 + 8 * c) * a.ks_t, koff, st + c * 1024);
            else if constexpr (VNAT)
                lds_dma16_at(Vb + (int64_t)(k0 + 8 * (c - 8)) * a.vs_x, voff, st + c * 1024);
            else
                lds_dma16_at(Vb + (int64_t)(8 * (c - 8)) * a.vs_x + k0, voff, st + c * 1024);
        }
    };
    // fragment byte offsets within a stage for k-step s: K row sigma(j) (+32 kb), V^T row j (+32 db)
    const int sj = key_sigma(j);
    int kfo[4], vfo[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        kfo[s] = sj * 128 + (((2 * s + hf) ^ ((sj >> 1) & 7)) << 4);
        vfo[s] = 64 * 128 + j * 128 + (((2 * s + hf) ^ ((j >> 1) & 7)) << 4);
    }
    // VNAT: the fragment of lane j + 32 hf (dims j (+ 32 db), keys 16 s + 8 hf .. + 8) from two transposing reads
    // (keys + 0 .. 3, + 4 .. 7): as a source, lane 16 g + i addresses key 8 (g / 2) + i / 4 (+ 16 s, + 4), dims
    // 16 (g % 2) + 4 (i % 4) .. + 4 (+ 32 db, which flips bit 2 of the chunk: byte offset ^ 64)
    const int vnr = 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int vnb = 64 * 128 + vnr * 128 +
                    (((2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) ^ (2 * (vnr & 3))) << 4) + 8 * (lane & 1);

    float m[QB], l[QB];
    f32x16 o[2][QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        m[qb] = -1e30f;
        l[qb] = 0.f;
#pragma unroll
        for (int db = 0; db < 2; ++db) o[db][qb] = f32x16{};
    }

    const int wg_q_lo = qt * QT;
    const int wg_q_hi = wg_q_lo + QT - 1;
    const int kv_first = max(0, wg_q_lo - W) / kBKV;
    const int kv_last = wg_q_hi / kBKV;
    const int nt = kv_last - kv_first + 1;
    const int wq_lo = q0w, wq_hi = q0w + QW - 1;
    const float c2 = a.scale_log2, shift = a.shift;

    f32x16 sc[2][QB];
    bf16x8 pf[QB][4];
    auto tile_k0 = [&](int t) { return (kv_first + t) * kBKV; };
    auto active = [&](int t) { return tile_k0(t) <= wq_hi && tile_k0(t) + kBKV - 1 >= wq_lo - W; };
    // S = K Q^T of tile t (slot t % NS); BOUNDED: K (c2 Q)^T - shift, the exponents
    auto qk = [&](int t) {
        const char *st = lds + (t & (NS - 1)) * kStage;
        f32x16 init = f32x16{};
        if constexpr (BOUNDED) {
#pragma unroll
            for (int r = 0; r < 16; ++r) init[r] = -shift;
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) sc[kb][qb] = init;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x8 ka = *reinterpret_cast<const bf16x8 *>(st + kfo[s] + kb * 32 * 128);
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) sc[kb][qb] = mfma32x32x16(ka, qf[qb][s], sc[kb][qb]);
            }
        }
    };
    // masked softmax weights of tile t into pf (and l, m, o for the running maximum)
    auto softmax = [&](int t) {
        const int k0 = tile_k0(t);
        const bool edge = (k0 + kBKV - 1 > wq_lo) || (k0 < wq_hi - W);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
            const int q = q0w + 32 * qb + j;
            if (edge) {
                // key of register r in block kb: k0 + 8 hf + c with c = 32 kb + 16 (r / 8) + r % 8 (0 .. 63,
                // an inline constant); visible iff c <= d0 (causal) and c >= d0 - W (window), d0 = q - k0 - 8 hf.
                // Each bound is applied only in tiles that reach it (wave-uniform): one compare per score.
                int d0 = q - k0 - 8 * hf, dw = d0 - W;
                // (pinned here: compares hoisted above the products would each hold a 64-bit lane mask)
                asm volatile("" : "+v"(d0), "+v"(dw));
                const bool causal_edge = k0 + kBKV - 1 > wq_lo, window_edge = k0 < wq_hi - W;
                auto mask = [&](auto visible) {
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int c = 32 * kb + 16 * (r >> 3) + (r & 7);
                            sc[kb][qb][r] = visible(c) ? sc[kb][qb][r] : -__builtin_inff();
                        }
                };
                if (causal_edge) mask([&](int c) { return c <= d0; });
                if (window_edge) mask([&](int c) { return c >= dw; });
            }
            float mb;
            if constexpr (BOUNDED) {
                mb = shift;
            } else {
                float mx = -__builtin_inff();
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[kb][qb][r]);
                mx = fmaxf(mx, swap_halves(mx));
                // the reference maximum m moves only in tiles where some row's maximum passes it by more than 8
                // (log2 units): the weights exp2(s c2 - m) then stay below 2^8, and the output and the row sum
                // share the stale m, so the softmax is unchanged. The rescale of o and l (a wave-uniform branch)
                // runs in the few tiles that raise m instead of in every tile
                const float mc = mx * c2;
                if (__builtin_amdgcn_ballot_w64(mc > m[qb] + 8.0f)) {
                    const float m_new = fmaxf(m[qb], mc);
                    const float alpha = exp2_fast(m[qb] - m_new);
                    m[qb] = m_new;
                    l[qb] *= alpha;
#pragma unroll
                    for (int db = 0; db < 2; ++db) o[db][qb] *= alpha;
                }
                mb = m[qb];
            }
            float rs = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float p = BOUNDED ? exp2_fast(sc[kb][qb][r]) : exp2_fast(__builtin_fmaf(sc[kb][qb][r], c2, -mb));
                    sc[kb][qb][r] = p;
                    if constexpr (!BOUNDED) rs += p;
                }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bf16x8 v;
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (__bf16)sc[s >> 1][qb][8 * (s & 1) + e];
                pf[qb][s] = v;
                if constexpr (BOUNDED) {
                    // the row sum of the bf16 weights P^T carries into O^T, two per dot
#pragma unroll
                    for (int e = 0; e < 8; e += 2)
                        rs = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[e], v[e + 1]}, bf16x2{(__bf16)1.0f, (__bf16)1.0f},
                                                             rs, false);
                }
            }
            l[qb] += rs;
        }
    };
    // O += V^T P^T of tile t
    auto pv = [&](int t) {
        const char *st = lds + (t & (NS - 1)) * kStage;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int db = 0; db < 2; ++db) {
                bf16x8 va;
                if constexpr (VNAT) {
                    const char *p = st + (vnb ^ (64 * db)) + 2048 * s;
                    const bf16x4 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 512);
                    va = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                } else {
                    va = *reinterpret_cast<const bf16x8 *>(st + vfo[s] + db * 32 * 128);
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) o[db][qb] = mfma32x32x16(va, pf[qb][s], o[db][qb]);
            }
        }
    };

    if (group_a) {
        // tiles 0 .. 2 in flight; tile 0 landed when min(2, nt - 1) later tiles may still be
#pragma unroll
        for (int t = 0; t < 3; ++t)
            if (t < nt) issue(tile_k0(t), lb + t * kStage);
        vm_wait_groups<CPW, 2>(nt - 1 < 2 ? nt - 1 : 2);
    }
    __syncthreads();  // barrier 0: tile 0 landed
    // the tile loops step by the ring's depth (NS = 4), so that each unrolled tile's slot t & 3 is a constant
    // (the compiler does not unroll loops with barriers at run-time trip counts); the guards are uniform
    if (group_a) {
#pragma unroll 1
        for (int t0 = 0; t0 < nt; t0 += NS) {
#pragma unroll
            for (int u = 0; u < NS; ++u) {
                const int t = t0 + u;
                if (t < nt) {
                    if (active(t)) {
                        qk(t);
                        softmax(t);
                        pv(t);
                    }
                    if (t + 1 < nt) {
                        // tile t + 1 landed: tiles after it issued so far: min(t + 2, nt - 1) - (t + 1)
                        vm_wait_groups<CPW, 1>(nt - 2 - t < 1 ? nt - 2 - t : 1);
                        __syncthreads();  // barrier t + 1
                        if (t + 3 < nt) issue(tile_k0(t + 3), lb + ((t + 3) & (NS - 1)) * kStage);
                    }
                }
            }
        }
    } else {
        if (active(0)) qk(0);
#pragma unroll 1
        for (int t0 = 0; t0 < nt; t0 += NS) {
#pragma unroll
            for (int u = 0; u < NS; ++u) {
                const int t = t0 + u;
                if (t >= 1 && t < nt) {
                    __syncthreads();  // barrier t: tile t landed
                    if (active(t - 1)) {
                        softmax(t - 1);
                        pv(t - 1);
                    }
                    if (active(t)) qk(t);
                }
            }
        }
        if (active(nt - 1)) {
            softmax(nt - 1);
            pv(nt - 1);
        }
    }

#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int q = q0w + 32 * qb + j;
        const float lt = l[qb] + swap_halves(l[qb]);
        const float inv = 1.0f / lt;  // the diagonal key is always visible: lt > 0
        float dsum = 0.f;
        const float *dv = a.dot ? a.dvec + (int64_t)(b / a.ddiv) * a.ds_b + h * kD : nullptr;
        __bf16 *orow = a.o + b * a.os_b + h * a.os_h + (int64_t)q * a.os_t;
        // with 16 B aligned output rows the wave's 32 x 64 block is staged in LDS (the K / V ring, free once
        // both groups are past their last tile) and stored as whole 128 B row segments: in the MFMA layout
        // one 8 B store would touch 32 rows
        constexpr int kOP = 72;  // staging row pitch (bf16)
        static_assert(QB == 1, "one staging block per wave");
        __bf16 *stg = reinterpret_cast<__bf16 *>(lds) + wave * 32 * kOP;
        if (a.o_lines) __syncthreads();
        __bf16 *dst = a.o_lines ? stg + j * kOP : orow;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                bf16x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = (__bf16)(o[db][qb][4 * g + e] * inv);
                const int d = 32 * db + 8 * g + 4 * hf;
                store_bf16x4(dst + d, v);
                if (dv) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) dsum += (float)v[e] * dv[d + e];
                }
            }
        if (a.o_lines) {
            wave_lds_sync();
            __bf16 *ob = a.o + b * a.os_b + h * a.os_h + (int64_t)(q0w + 32 * qb) * a.os_t;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int c = it * 64 + lane, r = c >> 3, ch = c & 7;
                store_bf16x8(ob + (int64_t)r * a.os_t + ch * 8, load_bf16x8(stg + r * kOP + ch * 8));
            }
        }
        if (a.dot) {
            dsum += swap_halves(dsum);
            if (hf == 0) a.dot[((int64_t)b * T + q) * a.heads + h] = dsum;
        }
    }
}



// V [b, t, h, d] (d contiguous) -> V^T [b][h][d][t]: one workgroup per (b*h, 64-token tile); each thread
// reads two 16 B pieces of token rows and writes two 16 B pieces of dim rows through a padded LDS tile.
__global__ __launch_bounds__(256) void v_transpose_kernel(const __bf16 *v, int64_t vs_b, int64_t vs_h, int64_t vs_t,
                                                          int heads, int seq, __bf16 *vt) {
    constexpr int kP = 72;  // LDS row pitch (bf16): 144 B rows keep the column reads 4 B apart in the banks
    __shared__ __attribute__((aligned(16))) __bf16 tile[64 * kP];
    const int tiles = seq / 64;
    const int bh = blockIdx.x / tiles, t0 = (blockIdx.x % tiles) * 64;
    const int b = bh / heads, h = bh - b * heads;
    const __bf16 *src = v + b * vs_b + h * vs_h + (int64_t)t0 * vs_t;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + 256 * i, t = c >> 3, d8 = (c & 7) * 8;
        const bf16x8 x = load_bf16x8(src + (int64_t)t * vs_t + d8);
#pragma unroll
        for (int e = 0; e < 8; ++e) tile[(d8 + e) * kP + t] = x[e];
    }
    __syncthreads();
    __bf16 *dst = vt + (int64_t)bh * kD * seq + t0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + 256 * i, d = c >> 3, t8 = (c & 7) * 8;
        store_bf16x8(dst + (int64_t)d * seq + t8, *reinterpret_cast<const bf16x8 *>(tile + d * kP + t8));
    }
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_v_transpose(const void *v, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                                 int64_t vs_b, int64_t vs_h, int64_t vs_t, void *vt, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(head_dim == kD, "noise_v_transpose: head_dim must be 64, got %lld", (long long)head_dim);
    NOISE_CHECK_ARG(batch > 0 && heads > 0 && seq > 0 && seq % 64 == 0 && seq <= (1 << 30),
                    "noise_v_transpose: batch, heads > 0 and seq a positive multiple of 64 required");
    NOISE_CHECK_ARG(v && vt && v != vt && aligned(v, 16) && aligned(vt, 16),
                    "noise_v_transpose: distinct 16 B aligned buffers required");
    NOISE_CHECK_ARG(vs_b % 8 == 0 && vs_h % 8 == 0 && vs_t % 8 == 0, "noise_v_transpose: strides must be multiples of 8");
    const int64_t blocks = batch * heads * (seq / 64);
    NOISE_CHECK_ARG(blocks < (1ll << 31), "noise_v_transpose: too many tiles");
    hipLaunchKernelGGL(v_transpose_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const __bf16 *)v, vs_b, vs_h, vs_t, (int)heads, (int)seq, (__bf16 *)vt);
    return launch_status("noise_v_transpose");
}

extern "C" int noise_attention_fwd(const void *q, const void *k, const void *v, void *o, int64_t batch,
                                   int64_t heads, int64_t seq, int64_t head_dim, int64_t qs_b, int64_t qs_h,
                                   int64_t qs_t, int64_t ks_b, int64_t ks_h, int64_t ks_t, int64_t vs_b,
                                   int64_t vs_h, int64_t vs_x, int flags, int64_t os_b, int64_t os_h,
                                   int64_t os_t, int64_t window, float scale, const float *dot_vec,
                                   int64_t dot_vec_stride, int64_t dot_div, float *dot_out,
                                   noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG((flags & ~(NOISE_ATTN_V_TRANSPOSED | NOISE_ATTN_QK_NORMED)) == 0,
                    "noise_attention_fwd: unknown flags 0x%x", flags);
    const bool v_transposed = flags & NOISE_ATTN_V_TRANSPOSED;
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
    // lengths in whole 256-query tiles run the ring kernel, with V in either layout
    const bool vt_path = seq % kVtQT == 0;
    const int64_t qtile = vt_path ? kVtQT : kBQ;
    int64_t qtiles = (seq + qtile - 1) / qtile;
    NOISE_CHECK_ARG(bh * qtiles < (1ll << 31), "noise_attention_fwd: too many workgroups");
    AttnArgs a;
    a.q = (const __bf16 *)q; a.k = (const __bf16 *)k; a.v = (const __bf16 *)v; a.o = (__bf16 *)o;
    a.qs_b = qs_b; a.qs_h = qs_h; a.qs_t = qs_t;
    a.ks_b = ks_b; a.ks_h = ks_h; a.ks_t = ks_t;
    a.vs_b = vs_b; a.vs_h = vs_h; a.vs_x = vs_x;
    a.os_b = os_b; a.os_h = os_h; a.os_t = os_t;
    a.o_lines = (aligned(o, 16) && os_b % 8 == 0 && os_h % 8 == 0 && os_t % 8 == 0) ? 1 : 0;
    a.heads = (int)heads; a.seq = (int)seq; a.qtiles = (int)qtiles; a.bh_total = (int)bh;
    a.window = (int)(window > seq ? seq : window);
    a.xcd_grouped = (bh % 8 == 0) ? 1 : 0;
    // a grid of a few rounds of the 512 resident workgroups (256 CUs x 2) is set by its heaviest tiles:
    // start them all first. Larger grids keep a head's tiles together for its K / V in L2.
    a.tile_major = (vt_path && bh * qtiles <= 8 * 512) ? 1 : 0;
    a.scale_log2 = scale * kLog2e;
    a.dvec = dot_vec; a.dot = dot_out; a.ds_b = dot_vec_stride; a.ddiv = (int)dot_div;
    // rows of RMS <= 1 (rounded to bf16): |q . k| <= D (1 + 2^-8)^2 < 1.0079 D
    a.shift = kD * fabsf(scale) * kLog2e * 1.0079f;
    dim3 grid((unsigned)(bh * qtiles));
    if (vt_path) {
        const bool bounded = flags & NOISE_ATTN_QK_NORMED;
        auto kernel = v_transposed ? (bounded ? attention_vt_kernel<true, false> : attention_vt_kernel<false, false>)
                                   : (bounded ? attention_vt_kernel<true, true> : attention_vt_kernel<false, true>);
        hipLaunchKernelGGL(kernel, grid, dim3(512), 0, (hipStream_t)stream, a);
    } else if (v_transposed)
        hipLaunchKernelGGL(attention_fwd_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(attention_fwd_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, a);
    return launch_status("noise_attention_fwd");
}
