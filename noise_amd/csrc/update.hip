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
// halves of every value (v = hi + lo to 2^-16), laid out so that one bf16 product over K = 3 np sums
// hi_a hi_b + hi_a lo_b + lo_a hi_b (split-bf16x3, fp32 accumulation): per row of a (weights folded in)
// [hi | hi | lo], per row of b [hi | lo | hi]. The GEMM is the shared Mma K loop; chunks accumulate into G
// in order (deterministic). Parameters whose sides are not multiples of 256 (ve_gate [8, 32], the 1-D
// mixing scalars) are small: one workgroup per gradient entry sums over all directions.
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
    __bf16 *table[kMaxParams];        // [rows + cols][3 np]: a rows, then b rows
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
    __bf16 *row = s.table[p] + (int64_t)rl * 3 * np;
    const int64_t k = (int64_t)blockIdx.y * 256 + threadIdx.x;
    float v = 0.0f;
    if (k < n) {
        const int64_t d = d0 + k;
        v = noise_at(dl, s.offsets[p][d] + rl, numel);
        if (is_a) v *= weight[d] * scale;
    }
    const __bf16 hi = (__bf16)v;
    const __bf16 lo = (__bf16)(v - (float)hi);
    row[k] = hi;
    row[np + k] = is_a ? hi : lo;
    row[2 * np + k] = is_a ? lo : hi;
}

// As update_tables_kernel, reading the draw from a materialised buffer (fp32 [numel]) instead of the Philox
// counter: a workgroup reads 64 directions x 256 consecutive elements (1 KiB per direction, coalesced) into
// LDS, then writes the 256 table rows' 64 columns of each third (8 lanes x 16 B per row: whole 128 B lines).
// grid = (rows_total / 256, np / 64).
constexpr int kTabK = 64, kTabPad = 257;
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
    // 16 loads in flight per thread: addresses clamped into the buffer, out-of-range elements set after
    for (int kb = 0; kb < kTabK; kb += 16) {
        float v[16];
        bool ok[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t L = (kb + e < kv ? off[kb + e] : 0) + rl0 + tid;
            ok[e] = L >= 0 && L < numel;
            v[e] = buf[L < 0 ? 0 : (L < numel ? L : numel - 1)];
        }
#pragma unroll
        for (int e = 0; e < 16; ++e)
            sm[(kb + e) * kTabPad + tid] = kb + e < kv ? (ok[e] ? v[e] : __builtin_nanf("")) : 0.0f;
    }
    __syncthreads();
    const int c = tid & 7;  // columns 8c .. 8c + 7 of the block's 64
    float wk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) wk[e] = k0 + 8 * c + e < n ? weight[d0 + k0 + 8 * c + e] * scale : 0.0f;
    for (int pass = 0; pass < 8; ++pass) {
        const int rr = pass * 32 + (tid >> 3), rl = rl0 + rr;
        const bool is_a = rl < s.rows[p];
        bf16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = sm[(8 * c + e) * kTabPad + rr];
            if (is_a) v *= wk[e];
            hi[e] = (__bf16)v;
            lo[e] = (__bf16)(v - (float)hi[e]);
        }
        __bf16 *row = s.table[p] + (int64_t)rl * 3 * np + k0 + 8 * c;
        *reinterpret_cast<bf16x8 *>(row) = hi;
        *reinterpret_cast<bf16x8 *>(row + np) = is_a ? hi : lo;
        *reinterpret_cast<bf16x8 *>(row + 2 * np) = is_a ? lo : hi;
    }
}

// G[o][i] (+)= sum_k table_a[o][k] table_b[i][k]: one 256 x 256 tile of one parameter per workgroup.
__global__ __launch_bounds__(512) void update_gemm_kernel(UpdateSet s, int K, int accumulate) {
    using M = Mma<8, kTile, kTile, 64, 2>;
    __shared__ __attribute__((aligned(16))) __bf16 lds[M::LDS_BYTES / 2];
    const int wg = blockIdx.x;
    int p = 0;
    while (p + 1 < s.n && s.tile_start[p + 1] <= wg) ++p;
    const int t = wg - s.tile_start[p];
    const int rows = s.rows[p], cols = s.cols[p];
    const int ot = t / (cols / kTile), ct = t % (cols / kTile);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, hf = lane >> 5;
    const int wn0 = M::wn0(wave), wm0 = M::wm0(wave);
    const __bf16 *tab = s.table[p];
    f32x16 acc[4][2];
    M::run(tab + (int64_t)ot * kTile * K, K, tab + (int64_t)(rows + ct * kTile) * K, K, K, lds, acc, tid, wn0, wm0);
    // lane (j, hf), register 4 g + e of block (fb, tb): row o = wn0 + 32 fb + 8 g + 4 hf + e, column
    // i = wm0 + 32 tb + j; the 32 lanes of a half-wave write 128 contiguous bytes of one row
    float *g = s.grad[p] + (int64_t)ot * kTile * cols + ct * kTile;
#pragma unroll
    for (int fb = 0; fb < 4; ++fb)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int o = wn0 + 32 * fb + 8 * (q >> 2) + 4 * hf + (q & 3);
                float *dst = g + (int64_t)o * cols + wm0 + 32 * tb + j;
                const float v = acc[fb][tb][q];
                *dst = accumulate ? *dst + v : v;
            }
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
    int64_t bytes = 0;
    for (int i = 0; i < nparams; ++i)
        if (is_big(params[i])) bytes += (params[i].rows + params[i].cols) * 3 * np * 2;
    return bytes;
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
    NOISE_CHECK_ARG(3 * np < (1ll << 31) && np / 256 <= 65535, "noise_update_gradients: chunk too large");
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
            need += (q.rows + q.cols) * 3 * np * 2;
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
    if (small.n) {
        hipLaunchKernelGGL(update_small_kernel, dim3((unsigned)entries_total), dim3(256), 0, s, small, pairs, weight,
                           scale, dl, numel);
        int st = launch_status("noise_update_gradients (small parameters)");
        if (st) return st;
    }
    if (big.n) {
        for (int64_t d0 = 0; d0 < pairs; d0 += np) {
            const int64_t n = pairs - d0 < np ? pairs - d0 : np;
            if (buffer)
                hipLaunchKernelGGL(update_tables_from_buffer_kernel, dim3((unsigned)(rows_total / 256),
                                   (unsigned)(np / kTabK)), dim3(256), 0, s, big, d0, n, np, weight, scale, buffer,
                                   numel);
            else
                hipLaunchKernelGGL(update_tables_kernel, dim3((unsigned)rows_total, (unsigned)(np / 256)), dim3(256),
                                   0, s, big, d0, n, np, weight, scale, dl, numel);
            int st = launch_status("noise_update_gradients (tables)");
            if (st) return st;
            hipLaunchKernelGGL(update_gemm_kernel, dim3((unsigned)tiles_total), dim3(512), 0, s, big, (int)(3 * np),
                               d0 > 0 ? 1 : 0);
            st = launch_status("noise_update_gradients (gemm)");
            if (st) return st;
        }
    }
    return NOISE_OK;
}
