// Counter-based noise, regenerated on the device instead of read from a materialised buffer.
//
// The reference slices every perturbation from one buffer drawn once by
//   torch.randn(2**28, generator=torch.Generator('cuda').manual_seed(SEED))      (eggroll.py:35, 114)
// and draws its per-step slice offsets with torch.randint on a seeded device generator
// (eggroll.py:117-120). On torch-ROCm both are torch's grid-stride distribution kernel over rocRAND's
// Philox4x32-10 (torch: ATen/native/hip/DistributionTemplates.h:52-89, 318-348, 446-457;
// rocrand: rocrand_philox4x32_10.h:124-300, rocrand_normal.h:53-68). Element L of a draw of `numel`
// values by S = 256*G threads is lane (L mod 4S)/S of the k = L/4S'th Philox block of thread L mod S,
// whose counter is (offset/4 + k, 0, thread) under key = seed. A block's four words give two Box-Muller
// pairs (words 0,1 -> lanes 0,1; words 2,3 -> lanes 2,3). Any element is therefore a closed form of
// (seed, offset, S, L), and a kernel can regenerate exactly the elements it needs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace noise {

struct Philox4 {
    uint32_t x, y, z, w;
};

// Philox4x32-10 (Salmon et al., SC'11): ten rounds of two 32x32->64 multiplies, key bumped by the
// golden-ratio Weyl constants between rounds.
__host__ __device__ inline Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                 uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return Philox4{c0, c1, c2, c3};
}

// Where element L of a draw lives: the Philox block (counter words) and the lane inside it.
struct DrawLayout {
    uint64_t seed;
    uint64_t offset;        // generator offset at the draw, a multiple of 4
    uint64_t threads;       // S = 256 * grid blocks of torch's launch
};

__host__ __device__ inline Philox4 draw_block(const DrawLayout &d, uint64_t L, int *lane) {
    uint64_t k, t;
    if ((d.threads & (d.threads - 1)) == 0) {
        // S a power of two (torch's grid on MI355X is 2048 blocks: S = 2^19): shifts and masks instead of two
        // 64-bit divisions, the larger part of a regenerated element's integer work besides Philox itself
        const int s = __builtin_ctzll(d.threads);
        k = L >> (s + 2);
        *lane = (int)((L >> s) & 3);
        t = L & (d.threads - 1);
    } else {
        const uint64_t four_s = 4 * d.threads;
        k = L / four_s;
        const uint64_t r = L - k * four_s;
        const uint64_t q = r / d.threads;
        t = r - q * d.threads;
        *lane = (int)q;
    }
    uint64_t c = d.offset / 4 + k;
    return philox4x32_10((uint32_t)c, (uint32_t)(c >> 32), (uint32_t)t, (uint32_t)(t >> 32),
                         (uint32_t)d.seed, (uint32_t)(d.seed >> 32));
}

// u32 of element L of an integer draw.
__host__ __device__ inline uint32_t draw_u32(const DrawLayout &d, uint64_t L) {
    int lane;
    Philox4 b = draw_block(d, L, &lane);
    return lane == 0 ? b.x : lane == 1 ? b.y : lane == 2 ? b.z : b.w;
}

// ln(u) for u in [2^-32, 1] exactly as torch-ROCm's device build evaluates rocRAND's logf: log2 from
// v_log_f32, then times ln 2 held as a head/tail float pair (0x1.62e42ep-1 + 0x1.efa39ep-25) with an
// FMA-compensated product, each step rounded to fp32. (Measured on MI355X against torch.randn: this and
// only this reproduces every element; hipcc 7.2's own logf differs in ~15% of draws by 1-2 ulp.)
__device__ inline float ln_compensated(float u) {
#pragma clang fp contract(off)
    const float head = 0x1.62e42ep-1f;
    const float tail = 0x1.efa39ep-25f;
    float y = __builtin_amdgcn_logf(u);
    float r = y * head;
    float e = __builtin_fmaf(y, head, -r);
    float f = __builtin_fmaf(y, tail, e);
    return r + f;
}

// One Box-Muller value with rocRAND's device arithmetic (rocrand_normal.h:53-68): u = 2^-32 + x*2^-32 in
// (0,1], v = 2^-32*2pi + y*2^-32*2pi, s = sqrt(-2 ln u) (correctly rounded sqrt), result sin(v)*s or
// cos(v)*s with the hardware sin/cos of __sincosf. The two affine maps are fused multiply-adds, as the
// reference's build contracts them.
__device__ inline float box_muller_one(uint32_t x, uint32_t y, bool take_cos) {
    const float inv = 2.3283064e-10f;
    const float inv_2pi = 1.46291807e-09f;
    float u = __builtin_fmaf((float)x, inv, inv);
    float v = __builtin_fmaf((float)y, inv_2pi, inv_2pi);
    float s = sqrtf(-2.0f * ln_compensated(u));
    float sn, cs;
    __sincosf(v, &sn, &cs);
    return (take_cos ? cs : sn) * s;
}

// torch.randn's element L (mean 0, std 1; torch applies val * std + mean with runtime scalars,
// TransformationHelper.h:97-99, which the caller passes in).
__device__ inline float draw_normal(const DrawLayout &d, uint64_t L, float mean, float stdv) {
    int lane;
    Philox4 b = draw_block(d, L, &lane);
    uint32_t x = lane < 2 ? b.x : b.z;
    uint32_t y = lane < 2 ? b.y : b.w;
    float v = box_muller_one(x, y, (lane & 1) != 0);
    return v * stdv + mean;
}

}  // namespace noise
