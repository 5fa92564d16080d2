// Shared GEMM machinery of the bf16 MFMA kernels: the K loop (Mma) and the XCD-aware tile order.
#pragma once
#include "common.hpp"
#include "mfma.hpp"

namespace noise {
namespace {

constexpr int cmax(int a, int b) { return a > b ? a : b; }

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
// a streaming store (nt) of output that no later work in the kernel reads
__device__ __forceinline__ void st4_nt(float *p, float4 v) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(v4f{v.x, v.y, v.z, v.w}, reinterpret_cast<v4f *>(p));
}
__device__ __forceinline__ float f4get(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// ------------------------------------------------------------------------------------------------
// K loop: acc[fb][tb] += W[wn0 + 32fb + .., :] . X[wm0 + 32tb + .., :]
// NW waves laid out WN (features) x WM (tokens); wave w owns features wn0 = 128 (w % WN) .. +128 and tokens
// wm0 = 64 (w / WN) .. +64. The (BN + BM) x BK operand tiles stream through NS LDS stages by direct
// global -> LDS copies (no register staging); rows are 2 BK bytes with the 16 B chunks XOR-swizzled by
// row pair, so the 32 rows of a fragment read hit distinct banks. The fragments of the next 16-wide
// k-step are read while the current step's MFMAs run; the wait for stage ks + 1 and the workgroup
// barrier sit just before the read that crosses into it, and the stage just finished is refilled with
// stage ks + NS right after that barrier. Ends with a barrier: the LDS may be reused at once.
// Optional tail (callers with K >= 2 BK): called once by every wave right after the barrier that precedes
// the last stage, when every slot but the last stage's ((K / BK - 1) % NS) is free for good; it may issue
// copies into those slots (the loop then waits for all of a wave's copies before its final barrier).
// ------------------------------------------------------------------------------------------------
struct NoTail {
    __device__ void operator()() const {}
};

template <int NW, int BN, int BM, int BK, int NS>
struct Mma {
    static constexpr int WN = BN / 128;
    static constexpr int WM = BM / 64;
    static_assert(WN * WM == NW, "NW waves of 128 x 64");
    static constexpr int RB = BK * 2;          // bytes per LDS row
    static constexpr int CPR = BK / 8;         // 16 B chunks per row
    static constexpr int RPI = 1024 / RB;      // rows per wave-wide copy (64 lanes x 16 B)
    static constexpr int RPB = 256 / RB;       // rows per 256 B of banks
    static constexpr int STAGE = (BN + BM) * RB;
    static constexpr int NBLK = (BN + BM) / RPI;
    static_assert(NBLK % NW == 0, "whole copies per wave");
    static constexpr int NI = NBLK / NW;       // copies per wave per stage
    static constexpr int SPK = BK / 16;
    static_assert(SPK % 2 == 0, "fragment double buffer alternates within and across stages");
    static_assert(NS >= 2 && NS <= 4 && NI * (NS - 1) < 64, "pipeline depth");
    static constexpr int LDS_BYTES = NS * STAGE;

    __device__ static int wn0(int wave) { return 128 * (wave % WN); }
    __device__ static int wm0(int wave) { return 64 * (wave / WN); }
    __device__ static int swz(int r, int c) { return c ^ ((r / RPB) % CPR); }

    // W: BN rows of stride ldw; X: BM rows of stride ldx (elements, multiples of 8; 16 B aligned bases);
    // K a multiple of BK
    template <class Tail = NoTail>
    __device__ static void run(const __bf16 *W, int64_t ldw, const __bf16 *X, int64_t ldx, int K, void *lds_v,
                               f32x16 (&acc)[4][2], int tid, int wn, int wm, Tail tail = Tail{}) {
        constexpr bool kTail = !__is_same(Tail, NoTail);
        char *lds = static_cast<char *>(lds_v);
        const int lane = tid & 63, j = lane & 31, hf = lane >> 5;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: copy targets stay scalar
        const unsigned lbase = lds_addr(lds);
#pragma unroll
        for (int fb = 0; fb < 4; ++fb)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) acc[fb][tb] = f32x16{};
        // copy i of a stage covers rows (i NW + wave) RPI .. +RPI: W for i < IW, X after. Row steps between
        // copies are multiples of RPB * CPR, so a lane's swizzled chunk and byte offset are the same for all
        // of its copies into one matrix; only the uniform base moves.
        constexpr int STEP = NW * RPI;
        static_assert(BN % STEP == 0 && BM % STEP == 0 && STEP % (RPB * CPR) == 0, "uniform copy steps");
        constexpr int IW = BN / STEP;
        const int rl = wave * RPI + lane / CPR;
        const int cl = swz(rl, lane % CPR);
        const unsigned offw = (unsigned)(rl * ldw * 2 + cl * 16), offx = (unsigned)(rl * ldx * 2 + cl * 16);
        // fragment rows wn + 32 fb + j and BN + wm + 32 tb + j share the swizzle of row j
        static_assert(32 % (RPB * CPR) == 0 && BN % (RPB * CPR) == 0, "fragment swizzle depends on j only");
        int lo[SPK];
#pragma unroll
        for (int s = 0; s < SPK; ++s) lo[s] = j * RB + swz(j, 2 * s + hf) * 16;
        const int nk = K / BK;
        auto issue = [&](int p) {
            const unsigned st = lbase + (p % NS) * STAGE + wave * 1024;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                if (i < IW)
                    lds_dma16_at(W + (int64_t)(i * STEP) * ldw + p * BK, offw, st + i * NW * 1024);
                else
                    lds_dma16_at(X + (int64_t)((i - IW) * STEP) * ldx + p * BK, offx, st + i * NW * 1024);
            }
        };
        bf16x8 fa[2][4], fx[2][2];
        auto fetch = [&](int buf, const char *st, int s) {
            const char *pa = st + wn * RB + lo[s], *px = st + (BN + wm) * RB + lo[s];
#pragma unroll
            for (int fb = 0; fb < 4; ++fb) fa[buf][fb] = *reinterpret_cast<const bf16x8 *>(pa + fb * 32 * RB);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) fx[buf][tb] = *reinterpret_cast<const bf16x8 *>(px + tb * 32 * RB);
        };
        // every stage buffer is free: stages 0 .. NS-1 in flight; stage 0 landed when min(NS-1, nk-1) remain
#pragma unroll
        for (int p = 0; p < NS; ++p)
            if (p < nk) issue(p);
        vm_wait_groups<NI, NS - 1>(nk - 1 < NS - 1 ? nk - 1 : NS - 1);
        __syncthreads();
        fetch(0, lds, 0);
#pragma unroll 1
        for (int ks = 0; ks < nk; ++ks) {
            const char *st = lds + (ks % NS) * STAGE;
#pragma unroll
            for (int s = 0; s < SPK; ++s) {
                const int cur = s & 1;
                if (s + 1 < SPK) {
                    fetch(cur ^ 1, st, s + 1);
                } else if (ks + 1 < nk) {
                    // stage ks+1 landed for every wave: stages up to min(ks + NS - 1, nk - 1) were issued
                    vm_wait_groups<NI, NS - 2>(nk - 2 - ks < NS - 2 ? nk - 2 - ks : NS - 2);
                    __syncthreads();
                    // every wave has read its last fragments of stage ks: its buffer takes stage ks + NS
                    if (ks + NS < nk) issue(ks + NS);
                    if constexpr (kTail) {
                        if (ks + 2 == nk) tail();
                    }
                    fetch(cur ^ 1, lds + ((ks + 1) % NS) * STAGE, 0);
                }
#pragma unroll
                for (int fb = 0; fb < 4; ++fb)
#pragma unroll
                    for (int tb = 0; tb < 2; ++tb) acc[fb][tb] = mfma32x32x16(fa[cur][fb], fx[cur][tb], acc[fb][tb]);
            }
        }
        if constexpr (kTail) vm_wait<0>();  // the tail's copies
        __syncthreads();
    }
};

// Workgroup -> (token tile, feature tile). Workgroups are dispatched round-robin over the 8 XCDs, so the
// feature tiles of one token tile are given consecutive slots of one XCD: its x rows are fetched into that
// XCD's L2 once and re-read from there. Falls back to row-major order when token tiles are not a
// multiple of 8.
__device__ __forceinline__ void tile_order(int wg, int ntiles_n, int ntiles_t, int &tt, int &nt) {
    if ((ntiles_t & 7) == 0) {
        const int slot = wg >> 3;
        nt = slot % ntiles_n;
        tt = (slot / ntiles_n) * 8 + (wg & 7);
    } else {
        nt = wg % ntiles_n;
        tt = wg / ntiles_n;
    }
}

}  // namespace
}  // namespace noise
