// Shared host/device helpers of libnoise_amd: status codes, the per-thread error message, bf16
// conversions and launch checks. Every extern "C" entry point validates its arguments on the host and
// returns a status (0 ok, <0 invalid argument, >0 hipError_t of a failed launch) instead of crashing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/noise_amd.h"

namespace noise {

// The message of the last failing call on this host thread (read back through noise_last_error()).
void set_error(const char *fmt, ...);
void clear_error();

#define NOISE_CHECK_ARG(cond, ...)                 \
    do {                                           \
        if (!(cond)) {                             \
            ::noise::set_error(__VA_ARGS__);       \
            return NOISE_EINVAL;                   \
        }                                          \
    } while (0)

// Status of the launch just issued (hipGetLastError also clears the sticky launch error).
inline int launch_status(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return (int)e;
    }
    return NOISE_OK;
}

inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// bf16 <-> fp32 with round-to-nearest-even (the rounding torch's .bfloat16() uses). NaN stays NaN.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    uint32_t rounding = 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)((u + rounding) >> 16);
}

__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

__host__ __device__ inline float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// DUST's block_forward chain (noise_dust_block) over a caller-provided workspace of workspace_bytes
// (noise_dust_block_workspace_bytes); fn names the entry point in error messages.
int dust_block_run(const float *x, float *x_out, int64_t sequences, int64_t tokens, const void *const w[7],
                   const void *ve, const void *rope_cos, const void *rope_sin, int64_t window, const void *jit_o,
                   const void *jit_attn, const void *jit_fc, const void *jit_mlp, void *workspace,
                   int64_t workspace_bytes, noise_stream_t stream, const char *fn);

// noise_pop_qkv's fused-rounding path with two waves per SIMD (qkv.hip): arguments validated by the caller,
// tokens a multiple of 128, outputs 16 B aligned, one value table for every member.
int qkv_rows_launch(const noise_population_t *pop, noise_view_t x, const void *const w[3], const noise_rank1_t r1[3],
                    const float *dots, const void *rope_cos, const void *rope_sin, const float *ve, int64_t vocab,
                    const int64_t *idx, int64_t idx_sm, const float *gates, const noise_rank1_t *ve_noise,
                    void *const out[3], noise_stream_t stream);

}  // namespace noise
