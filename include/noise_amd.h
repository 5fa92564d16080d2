/*
 * libnoise_amd -- C ABI of the MI355X (gfx950) population-forward hot path of pculaf/noise.
 *
 * Plain pointers, sizes and scalars only; no torch types. Every buffer is owned by the caller (device
 * memory unless stated); nothing is allocated, freed or retained by these calls. Launches are
 * asynchronous on the caller's HIP stream (`stream`, a hipStream_t; NULL = the null stream) and never
 * synchronise the host. Calls are stateless and reentrant.
 *
 * Return value: NOISE_OK (0) on success; NOISE_EINVAL (<0) when an argument is invalid (shape, stride,
 * alignment, null pointer, unsupported size), with a message in noise_last_error(); a positive
 * hipError_t when a launch fails.
 *
 * Reference citations are to files of pculaf/noise (train/val/eggroll.py, train/val/run.py,
 * utils/model.py) and, where the reference's arithmetic lives in torch-ROCm or rocRAND, to their headers.
 */
#ifndef NOISE_AMD_H
#define NOISE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NOISE_OK 0
#define NOISE_EINVAL (-1)

typedef void *noise_stream_t; /* hipStream_t */

/* ABI version of this header (bumped on any signature change). */
int noise_abi_version(void);

/* Message of the last failing call on the calling host thread ("" if none). */
const char *noise_last_error(void);

/* ------------------------------------------------------------------------------------------------
 * Noise: torch-ROCm device-generator draws, regenerated in-kernel (no materialised buffer).
 * A draw is identified by (seed, offset, threads): the generator's seed and philox offset at the call,
 * and threads = 256 * grid blocks of torch's grid-stride launch for that draw's numel on that device
 * (noise_draw_threads). Element L of the draw is a closed form of (seed, offset, threads, L).
 * ---------------------------------------------------------------------------------------------- */

/* threads (S) and generator-offset increment of a draw of `numel` values on `device`
 * (torch: ATen/native/hip/DistributionTemplates.h:52-65, calc_execution_policy with unroll 4).
 * Replaces nothing in the reference directly: it is the layout parameter every draw below needs. */
int noise_draw_layout(int device, int64_t numel, int64_t *threads_out, int64_t *offset_increment_out);

/* out[i] = mean + std * element (first + i) of torch.randn(numel) on a device generator at (seed,
 * offset), for i < n. Replaces torch.randn(2**28, generator=...) (eggroll.py:114) and DUST.noise's
 * torch.randn (run.py:216): any slice of the draw, without materialising the rest. */
int noise_normal_fill(float *out, int64_t n, int64_t first, uint64_t seed, uint64_t offset, int64_t threads,
                      float mean, float std, noise_stream_t stream);

/* out[i] = base + (u32 element i of the draw) % range, i < n; range in [1, 2^28). Replaces
 * torch.randint(0, NOISE - sum(p.shape), (P,), generator=g) (eggroll.py:119) and the 32-bit path of
 * torch's random_from_to (torch: DistributionTemplates.h:338-346). */
int noise_randint(int64_t *out, int64_t n, uint64_t seed, uint64_t offset, int64_t threads, uint64_t range,
                  int64_t base, noise_stream_t stream);

/* out[r * width + j] = element (offsets[rows[r]] + j) of the normal draw (seed, offset, threads), for
 * r < nrows, j < width (rows == NULL: rows[r] = r). Replaces Eggroll.noise's gather
 * buffer[offsets[name][directions, None] + arange(sum(p.shape))] (eggroll.py:126) over the 1 GiB
 * buffer; offsets[] + width must stay within the draw's numel (checked on the device: out-of-range
 * elements are written as NaN). */
int noise_gather_slices(float *out, int64_t nrows, int64_t width, const int64_t *offsets, const int64_t *rows,
                        int64_t numel, uint64_t seed, uint64_t offset, int64_t threads, noise_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Attention
 * ---------------------------------------------------------------------------------------------- */

/* Causal attention with a left window: query s attends to keys s - window .. s (window >= seq - 1 is
 * plain causal), softmax(q k^T * scale) v, bf16 in and out, fp32 accumulation. Replaces utils/model.py:24-31
 * `attention(q, k, v, window)` (flex_attention with the block mask q >= k & q - k <= window,
 * model.py:17-21; scale 1/sqrt(head_dim), torch: nn/attention/flex_attention.py:1543-1544).
 * q, k, o: element (b, t, h, d) at b*s_b + h*s_h + t*s_t + d (the reference's [B, T, H, D] and its
 * transposes are all expressible). v: the same with vs_x = token stride when v_transposed == 0, or
 * element (b, t, h, d) at b*vs_b + h*vs_h + d*vs_x + t when v_transposed == 1. head_dim must be 64.
 * Optional fused output (dot_out != NULL): dot_out[(b*seq + t)*heads + h] = sum_d o[b,t,h,d] *
 * dot_vec[(b / dot_div)*dot_vec_stride + h*64 + d], with o the bf16 output values; this is the
 * per-head part of the next perturbed linear's x.b (eggroll.py:58), NULL to skip. */
int noise_attention_fwd(const void *q, const void *k, const void *v, void *o, int64_t batch, int64_t heads,
                        int64_t seq, int64_t head_dim, int64_t qs_b, int64_t qs_h, int64_t qs_t, int64_t ks_b,
                        int64_t ks_h, int64_t ks_t, int64_t vs_b, int64_t vs_h, int64_t vs_x, int v_transposed,
                        int64_t os_b, int64_t os_h, int64_t os_t, int64_t window, float scale,
                        const float *dot_vec, int64_t dot_vec_stride, int64_t dot_div, float *dot_out,
                        noise_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NOISE_AMD_H */
