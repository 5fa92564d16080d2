// DUST's block_forward without an allocation: noise_dust_block over a library-owned, statically sized
// device array instead of a caller workspace, for callers that cannot allocate (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Each GPU holds its own copy of `scratch` (64 MiB, for as long as the process runs). Host code never
// passes the array's name to a kernel -- on the host it is only a stand-in symbol -- but the device
// address hipGetSymbolAddress returns for it, looked up once per device on that device's first call.
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU (different streams, or
// different host threads) race and must be ordered by the caller. The chain writes every byte it reads
// from the array before reading it, so nothing needs clearing between calls.
#include <mutex>

#include "common.hpp"

namespace noise {

constexpr int64_t kScratchBytes = 64ll << 20;

static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once looked up

// The current device's address of `scratch` (0 ok, else a status with the message set).
int scratch_address(void **out, const char *fn) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("%s: hipGetDevice: %s", fn, hipGetErrorString(e));
        return (int)e;
    }
    NOISE_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "%s: device %d outside the %d this library serves", fn, dev,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev, hipGetErrorString(e));
            return e != hipSuccess ? (int)e : NOISE_EINVAL;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return NOISE_OK;
}

}  // namespace
}  // namespace noise

extern "C" int64_t noise_dust_block_static_max_bytes(void) { return noise::kScratchBytes; }

extern "C" int noise_dust_block_static(const float *x, float *x_out, int64_t sequences, int64_t tokens,
                                       const void *const w[7], const void *ve, const void *rope_cos,
                                       const void *rope_sin, int64_t window, const void *jit_o, const void *jit_attn,
                                       const void *jit_fc, const void *jit_mlp, noise_stream_t stream) {
    using namespace noise;
    clear_error();
    const char *fn = "noise_dust_block_static";
    NOISE_CHECK_ARG(sequences >= 1 && tokens >= 1, "%s: sequences and tokens must be positive", fn);
    const int64_t need = noise_dust_block_workspace_bytes(sequences, tokens, ve != nullptr);
    NOISE_CHECK_ARG(need > 0 && need <= kScratchBytes,
                    "%s: %lld sequences x %lld tokens need %lld bytes of scratch; the static array holds %lld "
                    "(call noise_dust_block with a workspace for larger inputs)", fn, (long long)sequences,
                    (long long)tokens, (long long)need, (long long)kScratchBytes);
    void *ptr = nullptr;
    const int st = scratch_address(&ptr, fn);
    if (st != NOISE_OK) return st;
    return dust_block_run(x, x_out, sequences, tokens, w, ve, rope_cos, rope_sin, window, jit_o, jit_attn, jit_fc,
                          jit_mlp, ptr, kScratchBytes, stream, fn);
}
