// Noise kernels: slices of torch-ROCm's seeded device draws, regenerated from the Philox counter.
//
// Replaces, bit for bit, the reference's noise producers:
//   Eggroll.__init__  buffer = torch.randn(2**28, generator=cuda seed)           eggroll.py:114
//   Eggroll.offsets   torch.randint(0, NOISE - sum(p.shape), (P,), generator=g)  eggroll.py:117-120
//   Eggroll.noise     buffer[offsets[name][directions, None] + arange(width)]    eggroll.py:122-128
//   DUST.noise / signs / orthogonal_noise (Hadamard rows, patterns, signs)      run.py:143-152, 215-238
// The draw layout is torch's grid-stride distribution kernel (torch: ATen/native/hip/
// DistributionTemplates.h:52-89) and rocRAND's Philox4x32-10 + Box-Muller (rocrand_philox4x32_10.h,
// rocrand_normal.h:53-68); philox.hpp states the closed form.
#include "common.hpp"
#include "philox.hpp"

namespace noise {
namespace {

constexpr int kBlock = 256;

// Element-wise: out[i] = element first+i. One Philox block per element.
__global__ __launch_bounds__(kBlock) void normal_elementwise_kernel(float *__restrict__ out, int64_t n,
                                                                    int64_t first, DrawLayout d, float mean,
                                                                    float stdv) {
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        out[i] = draw_normal(d, (uint64_t)(first + i), mean, stdv);
    }
}

// Block-wise, for ranges covering whole Philox planes: work item (k, t) computes block k of thread t
// once and writes its four lanes L = 4Sk + qS + t that fall in [first, first + n). Writes are
// coalesced along t. Covers k in [k0, k1].
__global__ __launch_bounds__(kBlock) void normal_blockwise_kernel(float *__restrict__ out, int64_t n,
                                                                  int64_t first, DrawLayout d, float mean,
                                                                  float stdv, int64_t k0, int64_t items) {
    const int64_t S = (int64_t)d.threads;
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t w = (int64_t)blockIdx.x * kBlock + threadIdx.x; w < items; w += stride) {
        int64_t k = k0 + w / S;
        int64_t t = w - (w / S) * S;
        uint64_t c = d.offset / 4 + (uint64_t)k;
        Philox4 b = philox4x32_10((uint32_t)c, (uint32_t)(c >> 32), (uint32_t)t, (uint32_t)((uint64_t)t >> 32),
                                  (uint32_t)d.seed, (uint32_t)(d.seed >> 32));
        int64_t base = 4 * S * k + t;
        float v0 = box_muller_one(b.x, b.y, false) * stdv + mean;
        float v1 = box_muller_one(b.x, b.y, true) * stdv + mean;
        float v2 = box_muller_one(b.z, b.w, false) * stdv + mean;
        float v3 = box_muller_one(b.z, b.w, true) * stdv + mean;
        int64_t L0 = base - first;
        if (L0 >= 0 && L0 < n) out[L0] = v0;
        if (L0 + S >= 0 && L0 + S < n) out[L0 + S] = v1;
        if (L0 + 2 * S >= 0 && L0 + 2 * S < n) out[L0 + 2 * S] = v2;
        if (L0 + 3 * S >= 0 && L0 + 3 * S < n) out[L0 + 3 * S] = v3;
    }
}

__global__ __launch_bounds__(kBlock) void randint_kernel(int64_t *__restrict__ out, int64_t n, DrawLayout d,
                                                         uint64_t range, int64_t base) {
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        uint32_t u = draw_u32(d, (uint64_t)i);
        out[i] = (int64_t)(u % range) + base;
    }
}

// grid = (ceil(width / 256), nrows)
__global__ __launch_bounds__(kBlock) void gather_slices_kernel(float *__restrict__ out, int64_t width,
                                                               const int64_t *__restrict__ offsets,
                                                               const int64_t *__restrict__ rows, int64_t numel,
                                                               DrawLayout d) {
    int64_t r = blockIdx.y;
    int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (j >= width) return;
    int64_t src = rows ? rows[r] : r;
    int64_t L = offsets[src] + j;
    float v = (L >= 0 && L < numel) ? draw_normal(d, (uint64_t)L, 0.0f, 1.0f) : __builtin_nanf("");
    out[r * width + j] = v;
}

// The slices of several parameters in one launch: group k's elements (offsets_k[rows[r]] + j) for j < width_k
// go to out[r * ld + col_k + j]. grid = (widest group / kBlock, rows, groups): blockIdx.z is the group, so its
// descriptor entries are one uniform load each; the blocks past a narrower group's width exit at once.
__global__ __launch_bounds__(kBlock) void gather_groups_kernel(float *__restrict__ out, int64_t ld,
                                                               noise_slice_groups_t g,
                                                               const int64_t *__restrict__ rows, int64_t numel,
                                                               DrawLayout d) {
    const int k = blockIdx.z;
    const int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (j >= g.width[k]) return;
    const int64_t r = blockIdx.y;
    const int64_t src = rows ? rows[r] : r;
    const int64_t L = g.offsets[k][src] + j;
    const float v = (L >= 0 && L < numel) ? draw_normal(d, (uint64_t)L, 0.0f, 1.0f) : __builtin_nanf("");
    out[r * ld + g.col[k] + j] = v;
}

// Orthogonal draws (run.py:223-238): out[(i * bt + f) * d + j] = H[row][j] * pattern * sign with
// H[r][j] = (-1)^popcount(r & j), the Sylvester Hadamard matrix of run.py:143-152 (its recursion
// [[H, H], [H, -H]] flips the sign exactly where both indices have the new top bit set).
__global__ __launch_bounds__(kBlock) void orthogonal_kernel(void *__restrict__ out, int out_bf16, int64_t n,
                                                            int64_t bt, int64_t d, int64_t index0,
                                                            const int64_t *__restrict__ offset,
                                                            const int64_t *__restrict__ pattern,
                                                            const int64_t *__restrict__ sign) {
    const int64_t total = n * bt * d;
    for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += (int64_t)gridDim.x * kBlock) {
        const int64_t j = e % d, f = (e / d) % bt, i = e / (d * bt);
        const int64_t index = index0 + i;
        const int64_t row = (offset[f] + index) & (d - 1);  // d a power of two
        int neg = __builtin_popcountll((uint64_t)(row & j)) & 1;
        neg ^= (int)((pattern[(index / d) * d + j] & 1) ^ 1);  // randint(0, 2) * 2 - 1
        neg ^= (int)((sign[i * bt + f] & 1) ^ 1);
        const float v = neg ? -1.0f : 1.0f;
        if (out_bf16)
            static_cast<__bf16 *>(out)[e] = (__bf16)v;
        else
            static_cast<float *>(out)[e] = v;
    }
}

// The same draws, 8 coordinates per thread for 8 <= d <= 2048: a workgroup takes one draw i and a run of frame
// positions f, threads tile each row in 8-wide chunks (d / 8 threads per row, 2048 / d rows side by side). For
// a chunk at j0 (a multiple of 8), popcount(row & (j0 + e)) has the parity of popcount(row & j0) xor that of
// popcount(row & e), the latter a byte of kLowParity indexed by row mod 8; the pattern bits of the chunk are
// read once per workgroup; a row costs two index loads, a byte of logic and one 16 B (bf16) or 32 B store.
constexpr uint64_t kLowParity = 0x963C5AF066CCAA00ull;  // byte r: bit e = popcount(r & e) mod 2, r, e < 8

template <bool BF16>
__global__ __launch_bounds__(kBlock) void orthogonal8_kernel(void *__restrict__ out, int64_t bt, int64_t d,
                                                             int64_t index0, const int64_t *__restrict__ offset,
                                                             const int64_t *__restrict__ pattern,
                                                             const int64_t *__restrict__ sign, int64_t rows_per_block) {
    const int tpr = (int)(d >> 3);                  // threads per row (d <= 2048: at most kBlock)
    const int rpi = kBlock / tpr;                   // rows side by side
    const int tr = threadIdx.x / tpr, tc = threadIdx.x - tr * tpr;
    const int64_t i = blockIdx.y, index = index0 + i;
    const int64_t j0 = 8 * (int64_t)tc;
    const int64_t *pat = pattern + (index / d) * d + j0;
    unsigned pbits = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) pbits |= (unsigned)(pat[e] & 1) << e;
    const int64_t f0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t f1 = f0 + rows_per_block < bt ? f0 + rows_per_block : bt;
    for (int64_t f = f0 + tr; f < f1; f += rpi) {
        const int64_t row = (offset[f] + index) & (d - 1);
        unsigned neg = (unsigned)(kLowParity >> (8 * (row & 7))) & 0xFFu;
        neg ^= (__builtin_popcountll((uint64_t)(row & j0)) & 1) ? 0xFFu : 0u;
        neg ^= pbits ^ ((sign[i * bt + f] & 1) ? 0xFFu : 0u);
        const int64_t at = (i * bt + f) * d + j0;
        if constexpr (BF16) {
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w[k] = (0x3F80u | (((neg >> (2 * k)) & 1u) << 15)) |
                       ((0x3F80u | (((neg >> (2 * k + 1)) & 1u) << 15)) << 16);
            *reinterpret_cast<uint4 *>(static_cast<__bf16 *>(out) + at) = uint4{w[0], w[1], w[2], w[3]};
        } else {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = ((neg >> e) & 1u) ? -1.0f : 1.0f;
            float *o = static_cast<float *>(out) + at;
            *reinterpret_cast<float4 *>(o) = float4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<float4 *>(o + 4) = float4{v[4], v[5], v[6], v[7]};
        }
    }
}

int grid_for(int64_t work) {
    int64_t g = (work + kBlock - 1) / kBlock;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return (int)g;
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_draw_layout(int device, int64_t numel, int64_t *threads_out, int64_t *offset_increment_out) {
    clear_error();
    NOISE_CHECK_ARG(numel > 0, "noise_draw_layout: numel must be positive, got %lld", (long long)numel);
    NOISE_CHECK_ARG(threads_out != nullptr, "noise_draw_layout: threads_out is NULL");
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        set_error("noise_draw_layout: hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
        return (int)e;
    }
    int64_t blocks = (numel + 255) / 256;
    int64_t cap = (int64_t)prop.multiProcessorCount * (prop.maxThreadsPerMultiProcessor / 256);
    if (blocks > cap) blocks = cap;
    int64_t S = blocks * 256;
    *threads_out = S;
    if (offset_increment_out) *offset_increment_out = ((numel - 1) / (S * 4) + 1) * 4;
    return NOISE_OK;
}

extern "C" int noise_normal_fill(float *out, int64_t n, int64_t first, uint64_t seed, uint64_t offset,
                                 int64_t threads, float mean, float stdv, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(n >= 0 && first >= 0, "noise_normal_fill: n and first must be >= 0");
    NOISE_CHECK_ARG(threads > 0 && threads % 256 == 0, "noise_normal_fill: threads must be a positive multiple of 256, got %lld",
                    (long long)threads);
    NOISE_CHECK_ARG(offset % 4 == 0, "noise_normal_fill: generator offset must be a multiple of 4");
    if (n == 0) return NOISE_OK;
    NOISE_CHECK_ARG(out != nullptr, "noise_normal_fill: out is NULL");
    NOISE_CHECK_ARG(aligned(out, 4), "noise_normal_fill: out must be 4-byte aligned");
    DrawLayout d{seed, offset, (uint64_t)threads};
    hipStream_t s = (hipStream_t)stream;
    if (n >= 4 * threads) {
        int64_t k0 = first / (4 * threads);
        int64_t k1 = (first + n - 1) / (4 * threads);
        int64_t items = (k1 - k0 + 1) * threads;
        hipLaunchKernelGGL(normal_blockwise_kernel, dim3(grid_for(items)), dim3(kBlock), 0, s, out, n, first, d,
                           mean, stdv, k0, items);
    } else {
        hipLaunchKernelGGL(normal_elementwise_kernel, dim3(grid_for(n)), dim3(kBlock), 0, s, out, n, first, d,
                           mean, stdv);
    }
    return launch_status("noise_normal_fill");
}

extern "C" int noise_randint(int64_t *out, int64_t n, uint64_t seed, uint64_t offset, int64_t threads,
                             uint64_t range, int64_t base, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(n >= 0, "noise_randint: n must be >= 0");
    NOISE_CHECK_ARG(threads > 0 && threads % 256 == 0, "noise_randint: threads must be a positive multiple of 256");
    NOISE_CHECK_ARG(offset % 4 == 0, "noise_randint: generator offset must be a multiple of 4");
    NOISE_CHECK_ARG(range >= 1 && range < (1ull << 28),
                    "noise_randint: range must be in [1, 2^28) (torch's 32-bit path), got %llu",
                    (unsigned long long)range);
    if (n == 0) return NOISE_OK;
    NOISE_CHECK_ARG(out != nullptr && aligned(out, 8), "noise_randint: out must be a non-NULL 8-byte aligned pointer");
    DrawLayout d{seed, offset, (uint64_t)threads};
    hipLaunchKernelGGL(randint_kernel, dim3(grid_for(n)), dim3(kBlock), 0, (hipStream_t)stream, out, n, d, range, base);
    return launch_status("noise_randint");
}

extern "C" int noise_gather_slices(float *out, int64_t nrows, int64_t width, const int64_t *offsets,
                                   const int64_t *rows, int64_t numel, uint64_t seed, uint64_t offset,
                                   int64_t threads, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(nrows >= 0 && width >= 0, "noise_gather_slices: nrows and width must be >= 0");
    NOISE_CHECK_ARG(nrows <= 65535, "noise_gather_slices: at most 65535 rows per call, got %lld", (long long)nrows);
    NOISE_CHECK_ARG(threads > 0 && threads % 256 == 0, "noise_gather_slices: threads must be a positive multiple of 256");
    NOISE_CHECK_ARG(offset % 4 == 0, "noise_gather_slices: generator offset must be a multiple of 4");
    NOISE_CHECK_ARG(numel > 0, "noise_gather_slices: numel must be positive");
    if (nrows == 0 || width == 0) return NOISE_OK;
    NOISE_CHECK_ARG(out != nullptr && offsets != nullptr, "noise_gather_slices: out and offsets must be non-NULL");
    DrawLayout d{seed, offset, (uint64_t)threads};
    dim3 grid((unsigned)((width + kBlock - 1) / kBlock), (unsigned)nrows);
    hipLaunchKernelGGL(gather_slices_kernel, grid, dim3(kBlock), 0, (hipStream_t)stream, out, width, offsets, rows,
                       numel, d);
    return launch_status("noise_gather_slices");
}

extern "C" int noise_gather_slice_groups(float *out, int64_t nrows, int64_t ld, const noise_slice_groups_t *groups,
                                         const int64_t *rows, int64_t numel, uint64_t seed, uint64_t offset,
                                         int64_t threads, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_gather_slice_groups";
    NOISE_CHECK_ARG(groups != nullptr, "%s: groups NULL", fn);
    const noise_slice_groups_t g = *groups;
    NOISE_CHECK_ARG(g.count >= 1 && g.count <= NOISE_SLICE_GROUPS_MAX, "%s: 1 .. %d groups, got %d", fn,
                    NOISE_SLICE_GROUPS_MAX, g.count);
    NOISE_CHECK_ARG(nrows >= 0 && nrows <= 65535, "%s: 0 .. 65535 rows per call, got %lld", fn, (long long)nrows);
    NOISE_CHECK_ARG(threads > 0 && threads % 256 == 0, "%s: threads must be a positive multiple of 256", fn);
    NOISE_CHECK_ARG(offset % 4 == 0, "%s: generator offset must be a multiple of 4", fn);
    NOISE_CHECK_ARG(numel > 0, "%s: numel must be positive", fn);
    int64_t end = 0, widest = 0;
    for (int k = 0; k < g.count; ++k) {
        NOISE_CHECK_ARG(g.offsets[k] != nullptr && g.width[k] > 0 && g.width[k] % kBlock == 0 && g.col[k] == end,
                        "%s: group %d needs offsets, a width that is a positive multiple of %d, and to start at "
                        "column %lld (groups are packed in order)", fn, k, kBlock, (long long)end);
        end += g.width[k];
        widest = g.width[k] > widest ? g.width[k] : widest;
    }
    NOISE_CHECK_ARG(ld >= end, "%s: row stride %lld below the groups' total width %lld", fn, (long long)ld,
                    (long long)end);
    if (nrows == 0) return NOISE_OK;
    NOISE_CHECK_ARG(out != nullptr, "%s: out NULL", fn);
    DrawLayout d{seed, offset, (uint64_t)threads};
    NOISE_CHECK_ARG(widest / kBlock <= 65535, "%s: a group wider than %d columns", fn, 65535 * kBlock);
    dim3 grid((unsigned)(widest / kBlock), (unsigned)nrows, (unsigned)g.count);
    hipLaunchKernelGGL(gather_groups_kernel, grid, dim3(kBlock), 0, (hipStream_t)stream, out, ld, g, rows, numel, d);
    return launch_status(fn);
}

extern "C" int noise_orthogonal_draws(void *out, int out_bf16, int64_t n, int64_t bt, int64_t d, int64_t index0,
                                      const int64_t *offset, const int64_t *pattern, int64_t cycles,
                                      const int64_t *sign, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(n >= 0 && bt >= 0 && index0 >= 0, "noise_orthogonal_draws: n, bt and index0 must be >= 0");
    NOISE_CHECK_ARG(d >= 1 && (d & (d - 1)) == 0,
                    "noise_orthogonal_draws: orthogonal draws need a power-of-two width, not %lld", (long long)d);
    NOISE_CHECK_ARG(cycles >= 1 && index0 + n <= cycles * d,
                    "noise_orthogonal_draws: draws %lld..%lld need %lld cycles of patterns, got %lld",
                    (long long)index0, (long long)(index0 + n), (long long)((index0 + n + d - 1) / d),
                    (long long)cycles);
    NOISE_CHECK_ARG(n * bt * d < (1ll << 40), "noise_orthogonal_draws: output too large");
    if (n == 0 || bt == 0) return NOISE_OK;
    NOISE_CHECK_ARG(out && offset && pattern && sign, "noise_orthogonal_draws: NULL pointer");
    NOISE_CHECK_ARG(aligned(out, out_bf16 ? 2 : 4) && aligned(offset, 8) && aligned(pattern, 8) && aligned(sign, 8),
                    "noise_orthogonal_draws: misaligned pointer");
    if (d >= 8 && d <= 8 * kBlock && n <= 65535 && aligned(out, 16)) {
        // rows per workgroup: about 16 row-iterations, at most 65535 workgroups along the frame
        const int64_t rpi = kBlock / (d / 8);
        int64_t rows = rpi * 16;
        if ((bt + rows - 1) / rows > 65535) rows = (bt + 65534) / 65535;
        const dim3 grid((unsigned)((bt + rows - 1) / rows), (unsigned)n);
        if (out_bf16)
            hipLaunchKernelGGL(orthogonal8_kernel<true>, grid, dim3(kBlock), 0, (hipStream_t)stream, out, bt, d, index0,
                               offset, pattern, sign, rows);
        else
            hipLaunchKernelGGL(orthogonal8_kernel<false>, grid, dim3(kBlock), 0, (hipStream_t)stream, out, bt, d,
                               index0, offset, pattern, sign, rows);
        return launch_status("noise_orthogonal_draws");
    }
    hipLaunchKernelGGL(orthogonal_kernel, dim3(grid_for(n * bt * d)), dim3(kBlock), 0, (hipStream_t)stream, out,
                       out_bf16, n, bt, d, index0, offset, pattern, sign);
    return launch_status("noise_orthogonal_draws");
}
