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

#ifdef __cplusplus
}
#endif

#endif /* NOISE_AMD_H */
