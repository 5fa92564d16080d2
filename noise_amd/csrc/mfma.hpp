// CDNA4 (gfx950) MFMA operand types and small device helpers shared by the kernels.
//
// v_mfma_f32_32x32x16_bf16 lane layout (64 lanes, l = lane, h = l / 32):
//   A (32 x 16): lane l holds A[l % 32][8h .. 8h+7]
//   B (16 x 32): lane l holds B[8h .. 8h+7][l % 32]
//   D (32 x 32): lane l, register r holds D[8(r/4) + 4h + (r%4)][l % 32]
// Any permutation of the contraction index applied to A and B alike leaves D unchanged, which the
// attention kernel uses to feed softmax registers straight into the second product.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace noise {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// x rounded to the nearest bf16 (ties to even), as a float
__device__ __forceinline__ float bfr(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ bf16x8 load_bf16x8(const __bf16 *p) { return *reinterpret_cast<const bf16x8 *>(p); }

__device__ __forceinline__ bf16x4 load_bf16x4(const __bf16 *p) { return *reinterpret_cast<const bf16x4 *>(p); }

__device__ __forceinline__ void store_bf16x8(__bf16 *p, bf16x8 v) { *reinterpret_cast<bf16x8 *>(p) = v; }

// a streaming store (nt): output that no later work in the kernel reads, kept from displacing cached weights
__device__ __forceinline__ void store_bf16x8_nt(__bf16 *p, bf16x8 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<bf16x8 *>(p));
}

__device__ __forceinline__ void store_bf16x4(__bf16 *p, bf16x4 v) { *reinterpret_cast<bf16x4 *>(p) = v; }

__device__ __forceinline__ bf16x8 cat(bf16x4 lo, bf16x4 hi) {
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Direct global -> LDS copy (global_load_lds_dwordx4): lane i fetches 16 B from base + off_i (base wave-uniform,
// off_i a 32-bit byte offset); the wave's 64 results land contiguously at LDS address l + 16 * i (l
// wave-uniform). Issued through inline asm so that the compiler's wait-count pass, which would otherwise
// wait for every outstanding copy before each LDS read, leaves the pipeline to the explicit vm_wait below.
// Such loads only add to vmcnt, so the compiler's own waits for its loads stay correct (they can only
// become stricter). M0 is saved and restored.
// LDS byte address of a pointer into a __shared__ array
__device__ __forceinline__ unsigned lds_addr(const void *l) {
    return (unsigned)(size_t)((__attribute__((address_space(3))) const void *)l);
}

// As lds_dma16 below, with the destination given as an LDS byte address (wave-uniform).
__device__ __forceinline__ void lds_dma16_at(const void *base, unsigned off, unsigned la) {
    // base and la are wave-uniform by contract; readfirstlane lets the compiler hold them in SGPRs. The
    // builtin returns a signed int: both halves are zero-extended before the 64-bit address is formed.
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint64_t ub = ((uint64_t)hi << 32) | (uint64_t)lo;
    const unsigned l = (unsigned)__builtin_amdgcn_readfirstlane((int)la);
    unsigned save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "v"(off), "s"(ub), "s"(l)
                 : "memory");
}

__device__ __forceinline__ void lds_dma16(const void *base, unsigned off, const void *l) {
    lds_dma16_at(base, off, lds_addr(l));
}

// As lds_dma16_at with 4 B per lane: lane l's dword lands at LDS byte la + 4 l (256 B per wave-wide copy); the
// global address needs only 4 B alignment.
__device__ __forceinline__ void lds_dma4_at(const void *base, unsigned off, unsigned la) {
    const uint64_t b = (uint64_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint64_t ub = ((uint64_t)hi << 32) | (uint64_t)lo;
    const unsigned l = (unsigned)__builtin_amdgcn_readfirstlane((int)la);
    unsigned save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "v"(off), "s"(ub), "s"(l)
                 : "memory");
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left alone)
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// wait until at most r groups of G loads remain in flight (0 <= r <= RMAX, r known at run time only)
template <int G, int RMAX>
__device__ __forceinline__ void vm_wait_groups(int r) {
    static_assert(RMAX <= 5 && G * RMAX < 64, "vmcnt is 6 bits");
    if constexpr (RMAX >= 5) {
        if (r >= 5) { vm_wait<5 * G>(); return; }
    }
    if constexpr (RMAX >= 4) {
        if (r == 4) { vm_wait<4 * G>(); return; }
    }
    if constexpr (RMAX >= 3) {
        if (r == 3) { vm_wait<3 * G>(); return; }
    }
    if constexpr (RMAX >= 2) {
        if (r == 2) { vm_wait<2 * G>(); return; }
    }
    if constexpr (RMAX >= 1) {
        if (r == 1) { vm_wait<G>(); return; }
    }
    vm_wait<0>();
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Value of lane (l ^ 32): the other half of a 32x32 MFMA column.
__device__ __forceinline__ float swap_halves(float x) { return __shfl_xor(x, 32, 64); }

// The sum over the four lanes l % 16 + 16 g, in the order two xor shuffles give it:
// (v[l] + v[l ^ 16]) + (v[l ^ 32] + v[l ^ 48]). It uses gfx950's lane swaps (VALU) instead of two LDS permutes.
// A swap exchanges half of one register with half of another. Given two copies of a value, every lane ends up
// with its own value in one register and its partner's in the other. fp32 addition commutes, so each lane's sum
// is bitwise the shuffles' sum. The swaps are inline asm because the compiler's builtin loses its second result.
// A VALU write read by a lane swap needs two wait states: hence the s_nop.
__device__ __forceinline__ float sum_lanes_16_32(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    v = a + b;
    a = v;
    b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return a + b;
}

// gfx950's transposing LDS read (ds_read_b64_tr_b16). Every lane gives the address of 8 B (four 16-bit
// elements). Within each group of 16 lanes, lane i receives as its element e (e = 0 .. 3) element i % 4 of
// the 8 B that lane i / 4 + 4 e of its group addressed. So if lane s of a group points at row r0 + s / 4,
// columns c0 + 4 (s % 4) .. + 4 of a row-major matrix, lane i receives column c0 + i of rows r0 .. r0 + 3.
__device__ __forceinline__ bf16x4 lds_read_tr16(const void *p) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)p);
    bf16x4 r;
    __builtin_memcpy(&r, &v, 8);
    return r;
}

// orders this wave's LDS writes before its lanes read what other lanes of the wave wrote (the compiler
// otherwise reasons per lane and may move such a read ahead of the writes)
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8 zero_bf16x8() {
    bf16x8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (__bf16)0.0f;
    return z;
}

}  // namespace noise
