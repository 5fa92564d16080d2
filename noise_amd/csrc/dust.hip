// DUST's head error (run.py:380-389 head_error over run.py:121-137 coordinate_differences): for every token
// and every logit j, the central difference of the token's soft-capped cross-entropy along its own raw logit,
//   (loss(raw_j + sigma) - loss(raw_j - sigma)) / (2 sigma),
// in the reference's closed form: moving one logit changes the partition function by one term, so with
// z = cap(raw), cap(v) = 15 tanh(v / 15), w = softmax(z) and z' the capped moved logit,
//   loss(z_j -> z') - loss(z) = log1p(w_j expm1(z' - z_j)) - [j = target] (z' - z_j).
// Zero for ignored tokens (target < 0) and for the padding columns vocab .. out_width.
//
// One wave per token row: pass 1 sums exp(z - 15) over the row (z <= 15, so no running maximum is needed and
// nothing overflows), pass 2 re-reads the row (<= 16 KiB, from the cache) and writes the differences. fp32 throughout with the device library's tanhf /
// expm1f / log1pf, as the reference's fp32 torch ops.
#include "common.hpp"
#include "mfma.hpp"

namespace noise {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each

__device__ inline float load_logit(const void *raw, int bf16, int64_t i) {
    return bf16 ? (float)static_cast<const __bf16 *>(raw)[i] : static_cast<const float *>(raw)[i];
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The moved logits through tanh's addition theorem: with t = tanh(raw / 15) and c = tanh(sigma / 15),
// cap(raw +- sigma) - cap(raw) = +-15 c (1 - t)(1 + t) / (1 +- c t), free of the cancellation of subtracting
// two capped values (and one tanh per logit instead of three).
__global__ __launch_bounds__(64 * kRowsPerBlock) void coordinate_differences_kernel(
    const void *__restrict__ raw, int raw_bf16, int64_t rows, int64_t vocab, int64_t raw_stride,
    const int64_t *__restrict__ targets, float sigma, float *__restrict__ out, int64_t out_width,
    int64_t out_stride) {
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    float *orow = out + row * out_stride;
    const int64_t y = targets[row];
    if (y < 0) {
        for (int64_t j = lane; j < out_width; j += 64) orow[j] = 0.0f;
        return;
    }
    const int64_t base = row * raw_stride;
    const float c = tanhf(sigma * (1.0f / 15.0f)), inv_2s = 1.0f / (2.0f * sigma);
    float s = 0.0f;
    for (int64_t j = lane; j < vocab; j += 64)
        s += __expf(15.0f * tanhf(load_logit(raw, raw_bf16, base + j) * (1.0f / 15.0f)) - 15.0f);
    const float inv_z = 1.0f / wave_sum(s);
    for (int64_t j = lane; j < out_width; j += 64) {
        float d = 0.0f;
        if (j < vocab) {
            const float t = tanhf(load_logit(raw, raw_bf16, base + j) * (1.0f / 15.0f));
            const float w = __expf(15.0f * t - 15.0f) * inv_z, omt2 = (1.0f - t) * (1.0f + t);
            // (quotients as products by reciprocals: v_rcp_f32 is within 1 ulp, against the IEEE division's
            // ten instructions)
            const float du = 15.0f * c * omt2 * __builtin_amdgcn_rcpf(1.0f + c * t);
            const float dd = -15.0f * c * omt2 * __builtin_amdgcn_rcpf(1.0f - c * t);
            // log1p(a) - log1p(b) = log1p((a - b) / (1 + b)); a - b = w (expm1(du) - expm1(dd)) adds two
            // terms of opposite sign (du > 0 > dd), so nothing cancels
            const float eu = expm1f(du), ed = expm1f(dd);
            d = log1pf(w * (eu - ed) * __builtin_amdgcn_rcpf(1.0f + w * ed));
            if (j == y) d -= du - dd;
            d *= inv_2s;
        }
        orow[j] = d;
    }
}

// DUST.direct_errors' estimate update (run.py:351-355): errors[r][j] += scale * e[r][j] with
//   e = einsum('nbt,nbtd->btd', reward.to(bf16), a)   (bf16 operands, fp32 sums, a bf16 result)
// over the n draws of a chunk, rows r = (b, t). One thread per 8 consecutive coordinates of a row.
__global__ __launch_bounds__(256) void draw_errors_kernel(const float *__restrict__ reward, const __bf16 *__restrict__ a,
                                                          int64_t n, int64_t rows, int64_t d, float scale,
                                                          float *__restrict__ errors) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over rows * d / 8
    const int64_t per_row = d / 8;
    if (i >= rows * per_row) return;
    const int64_t r = i / per_row, j = (i - r * per_row) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t q = 0; q < n; ++q) {
        const float w = (float)(__bf16)reward[q * rows + r];
        const bf16x8 v = *reinterpret_cast<const bf16x8 *>(a + (q * rows + r) * d + j);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += w * (float)v[e];
    }
    float *out = errors + r * d + j;
    float4 o0 = *reinterpret_cast<const float4 *>(out), o1 = *reinterpret_cast<const float4 *>(out + 4);
    o0.x += scale * (float)(__bf16)acc[0]; o0.y += scale * (float)(__bf16)acc[1];
    o0.z += scale * (float)(__bf16)acc[2]; o0.w += scale * (float)(__bf16)acc[3];
    o1.x += scale * (float)(__bf16)acc[4]; o1.y += scale * (float)(__bf16)acc[5];
    o1.z += scale * (float)(__bf16)acc[6]; o1.w += scale * (float)(__bf16)acc[7];
    *reinterpret_cast<float4 *>(out) = o0;
    *reinterpret_cast<float4 *>(out + 4) = o1;
}

// direct_errors' per-chunk draw preparation (run.py:344-349): a[i][r] *= mask[r] for the n draws (mask bf16 0/1
// over one draw's rows * d coordinates, or none) and scaled[i][r] = bf16(scale * a[i][r]), the jitter the rerun
// adds. One thread per 8 coordinates.
__global__ __launch_bounds__(256) void mask_scale_kernel(__bf16 *__restrict__ a, const __bf16 *__restrict__ mask,
                                                         int64_t n8, int64_t per_draw8, float scale,
                                                         __bf16 *__restrict__ scaled) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    bf16x8 v = *reinterpret_cast<const bf16x8 *>(a + 8 * i);
    if (mask) {
        const bf16x8 m = *reinterpret_cast<const bf16x8 *>(mask + 8 * (i % per_draw8));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (__bf16)((float)v[e] * (float)m[e]);
        *reinterpret_cast<bf16x8 *>(a + 8 * i) = v;
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (__bf16)(scale * (float)v[e]);
    *reinterpret_cast<bf16x8 *>(scaled + 8 * i) = o;
}

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_mask_scale(void *a, const void *mask, int64_t n, int64_t per_draw, float scale, void *scaled,
                                noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_mask_scale";
    NOISE_CHECK_ARG(n >= 1 && per_draw >= 8 && per_draw % 8 == 0, "%s: n >= 1 and per_draw a positive multiple of 8", fn);
    NOISE_CHECK_ARG(a && scaled && aligned(a, 16) && aligned(scaled, 16) && (!mask || aligned(mask, 16)),
                    "%s: a, scaled (and mask) must be non-NULL and 16 B aligned", fn);
    const int64_t n8 = n * per_draw / 8;
    NOISE_CHECK_ARG((n8 + 255) / 256 < (1ll << 31), "%s: too many elements", fn);
    hipLaunchKernelGGL(mask_scale_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (__bf16 *)a, (const __bf16 *)mask, n8, per_draw / 8, scale, (__bf16 *)scaled);
    return launch_status(fn);
}

extern "C" int noise_draw_errors(const float *reward, const void *a, int64_t n, int64_t rows, int64_t d, float scale,
                                 float *errors, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(n >= 1 && rows >= 0 && d >= 8 && d % 8 == 0,
                    "noise_draw_errors: need n >= 1, rows >= 0 and d a positive multiple of 8");
    if (rows == 0) return NOISE_OK;
    NOISE_CHECK_ARG(reward && a && errors && aligned(reward, 4) && aligned(a, 16) && aligned(errors, 16),
                    "noise_draw_errors: reward, a and errors must be non-NULL and aligned (a and errors 16 B)");
    const int64_t work = rows * (d / 8);
    NOISE_CHECK_ARG((work + 255) / 256 < (1ll << 31), "noise_draw_errors: too many rows");
    hipLaunchKernelGGL(draw_errors_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       reward, (const __bf16 *)a, n, rows, d, scale, errors);
    return launch_status("noise_draw_errors");
}

extern "C" int noise_coordinate_differences(const void *raw, int raw_bf16, int64_t rows, int64_t vocab,
                                            int64_t raw_stride, const int64_t *targets, float sigma, float *out,
                                            int64_t out_width, int64_t out_stride, noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(rows >= 0 && vocab >= 1 && out_width >= vocab && raw_stride >= vocab && out_stride >= out_width,
                    "noise_coordinate_differences: need rows >= 0, 1 <= vocab <= out_width <= out_stride, "
                    "raw_stride >= vocab");
    NOISE_CHECK_ARG(sigma > 0.0f, "noise_coordinate_differences: sigma must be positive");
    if (rows == 0) return NOISE_OK;
    NOISE_CHECK_ARG(raw != nullptr && targets != nullptr && out != nullptr,
                    "noise_coordinate_differences: raw, targets and out must be non-NULL");
    NOISE_CHECK_ARG(aligned(raw, raw_bf16 ? 2 : 4) && aligned(targets, 8) && aligned(out, 4),
                    "noise_coordinate_differences: misaligned pointer");
    const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    NOISE_CHECK_ARG(blocks < (1ll << 31), "noise_coordinate_differences: too many rows");
    hipLaunchKernelGGL(coordinate_differences_kernel, dim3((unsigned)blocks), dim3(64 * kRowsPerBlock), 0,
                       (hipStream_t)stream, raw, raw_bf16, rows, vocab, raw_stride, targets, sigma, out, out_width,
                       out_stride);
    return launch_status("noise_coordinate_differences");
}
