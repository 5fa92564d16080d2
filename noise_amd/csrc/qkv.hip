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
#include "qkv_phase.hpp"

namespace noise {
namespace {

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

#pragma unroll
    for (int k = 0; k < 3; ++k) qkv_issue(p, lbase, wave, lane, k);
    // this lane's input row: xf[kb] = x[tok][32 kb + 8 g .. + 8]
    bf16x8 xf[16];
    {
        const __bf16 *xr = p.x + m * p.xs_m + (int64_t)tok * p.xs_t + 8 * g;
#pragma unroll
        for (int kb = 0; kb < 16; ++kb) xf[kb] = load_bf16x8(xr + 32 * kb);
    }
    QkvLane L;
    L.m = m; L.t0 = t0; L.tok = tok; L.wave = wave; L.lane = lane; L.tid = tid; L.dir = dir; L.row = row; L.sgn = sgn;
    // per-token scalars: rank-1 scales, the rotary rows, value row
    L.dq0 = p.a[0] ? sgn * p.dots[row * 3] : 0.f;
    L.dq1 = p.a[1] ? sgn * p.dots[row * 3 + 1] : 0.f;
    L.dq2 = p.a[2] ? sgn * p.dots[row * 3 + 2] : 0.f;
    qkv_token_scalars<VE>(p, L);
    vm_wait<8>();  // stage 0 landed (stages 1 and 2 may still be in flight); the rows and scalars above too
    __syncthreads();
    qkv_phase<VE, false>(p, lds, xf, L);
}

}  // namespace

int qkv_rows_launch(const noise_population_t *pop, noise_view_t x, const void *const w[3], const noise_rank1_t r1[3],
                    const float *dots, const void *rope_cos, const void *rope_sin, const float *ve, int64_t vocab,
                    const int64_t *idx, int64_t idx_sm, const float *gates, const noise_rank1_t *ve_noise,
                    void *const out[3], noise_stream_t stream) {
    const QkvRowsArgs a = qkv_rows_args(pop, x, w, r1, dots, rope_cos, rope_sin, ve, vocab, idx, idx_sm, gates,
                                        ve_noise, out);
    const dim3 grid((unsigned)(pop->members * (pop->tokens / kQTok)));
    if (ve)
        hipLaunchKernelGGL(qkv16_kernel<true>, grid, dim3(kQThreads), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(qkv16_kernel<false>, grid, dim3(kQThreads), 0, (hipStream_t)stream, a);
    return launch_status("noise_pop_qkv");
}

}  // namespace noise
