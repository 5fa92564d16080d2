// Row-wise kernels of the population forward: embedding entry, member dot products, loss reduction and
// the split-bf16x3 operands of the fp32 head. One 64-lane wave per 512-wide row, 8 elements per lane.
#include "common.hpp"
#include "mfma.hpp"
#include "tile.hpp"

namespace noise {
namespace {

constexpr float kEps = 1.1920928955078125e-07f;  // torch.finfo(torch.float32).eps

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ void ld8(const float *p, float (&v)[8]) {
    float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void st8(float *p, const float (&v)[8]) {
    *reinterpret_cast<float4 *>(p) = float4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<float4 *>(p + 4) = float4{v[4], v[5], v[6], v[7]};
}

// Embedding entry of population_loss (eggroll.py:74-79 for block 0, model.py:196-199):
//   e = W[idx[t]] (+ sign * a[dir, idx[t]] * b[dir, :])      lowrank_embed, eggroll.py:61-63
//   x0 = norm(e); x = rl * x0 + ml * x0 (block 0's mix); h = bf16(norm(x))
// eager: x0, the two products and their sum each rounded to bf16 (the eager autocast forward's bf16 stream).
// rows = (member or shared, token); grid = rows / 4 workgroups of 4 waves.
struct EmbedArgs {
    int rows, tokens, per_member, dir_div, eager;
    const float *wte;
    const int64_t *idx;
    const float *sign;
    const float *ea, *eb;     // embedding noise rows or NULL
    int64_t ea_stride, eb_stride;
    const float *lam_r, *lam_x;   // block 0's mixing scalars (device)
    const float *eps_r, *eps_x;
    int64_t eps_stride;
    int64_t vocab;                // rows of wte; other ids give NaN rows
    float *x0, *xin;
    __bf16 *h;
};

__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs p) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const int m = p.per_member ? row / p.tokens : 0;
    const int t = row - (p.per_member ? m * p.tokens : 0);
    const int dir = m / p.dir_div;
    const float sgn = p.per_member && p.sign ? p.sign[m] : 0.f;
    const int64_t id = p.idx[t];
    const bool bad = id < 0 || id >= p.vocab;  // an id outside the table: no read leaves it, the row is NaN
    const int64_t tok = bad ? 0 : id;
    float e[8];
    ld8(p.wte + tok * 512 + lane * 8, e);
    if (bad) {
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = __builtin_nanf("");
    }
    if (p.ea) {
        const float s = sgn * p.ea[dir * p.ea_stride + tok];
        float b[8];
        ld8(p.eb + dir * p.eb_stride + lane * 8, b);
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] += s * b[i];
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += e[i] * e[i];
    float r = rsqrtf(wave_sum(ss) * (1.0f / 512.0f) + kEps);
    float rl = *p.lam_r, ml = *p.lam_x;
    if (p.eps_r) rl += sgn * p.eps_r[dir * p.eps_stride];
    if (p.eps_x) ml += sgn * p.eps_x[dir * p.eps_stride];
    if (p.eager) {
        // eager autocast multiplies a bf16 tensor by the 0-dim fp32 lambdas in bf16: they enter rounded
        rl = bfr(rl);
        ml = bfr(ml);
    }
    float x0[8], x[8];
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x0[i] = e[i] * r;
        if (p.eager) {
            x0[i] = bfr(x0[i]);
            x[i] = bfr(bfr(rl * x0[i]) + bfr(ml * x0[i]));
        } else {
            x[i] = rl * x0[i] + ml * x0[i];
        }
        ss += x[i] * x[i];
    }
    r = rsqrtf(wave_sum(ss) * (1.0f / 512.0f) + kEps);
    const int64_t o = (int64_t)row * 512 + lane * 8;
    st8(p.x0 + o, x0);
    st8(p.xin + o, x);
    bf16x8 hv;
#pragma unroll
    for (int i = 0; i < 8; ++i) hv[i] = (__bf16)(x[i] * r);
    store_bf16x8(p.h + o, hv);
}

// out[(m*T + t)*nk + k] = sum_n x[m, t, n] * b_k[m / dir_div, n], x bf16 with strides, n < width.
struct DotsArgs {
    int members, tokens, width, nk, dir_div;
    const __bf16 *x;
    int64_t xs_m, xs_t;
    const float *b[3];
    int64_t b_stride[3];
    float *out;
};

// The same dots when every member reads the same rows (x member stride 0): each (token, direction) pair once,
// 32 tokens x 64 directions per workgroup (4 x 4 per thread, fp32 FMAs over k in order), x and the b rows
// staged through LDS in k chunks of 32; each result goes to the dir_div members of its direction.
constexpr int kSdT = 32, kSdD = 64, kSdK = 32, kSdThreads = 128;
__global__ __launch_bounds__(kSdThreads) void shared_dots_kernel(DotsArgs p, int dirs) {
    __shared__ float xs[kSdK][kSdT + 4];
    __shared__ float bs[3][kSdK][kSdD + 4];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int t0 = blockIdx.x * kSdT, d0 = blockIdx.y * kSdD;
    float acc[3][4][4];
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[k][i][j] = 0.f;
    for (int n0 = 0; n0 < p.width; n0 += kSdK) {
        {
            // x: token tid / 4, k 8 (tid % 4) .. + 8 (zeros past the last token)
            const int t = tid >> 2, k8 = (tid & 3) * 8;
            bf16x8 v = bf16x8{};
            if (t0 + t < p.tokens) v = load_bf16x8(p.x + (int64_t)(t0 + t) * p.xs_t + n0 + k8);
#pragma unroll
            for (int e = 0; e < 8; ++e) xs[k8 + e][t] = (float)v[e];
        }
#pragma unroll
        for (int kk = 0; kk < 3; ++kk) {
            if (kk < p.nk) {
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const int c = it * kSdThreads + tid, d = c >> 3, k4 = (c & 7) * 4;
                    float4 v = float4{0.f, 0.f, 0.f, 0.f};
                    if (d0 + d < dirs) v = ld4(p.b[kk] + (int64_t)(d0 + d) * p.b_stride[kk] + n0 + k4);
                    bs[kk][k4][d] = v.x; bs[kk][k4 + 1][d] = v.y; bs[kk][k4 + 2][d] = v.z; bs[kk][k4 + 3][d] = v.w;
                }
            }
        }
        __syncthreads();
#pragma unroll 4
        for (int k = 0; k < kSdK; ++k) {
            const float4 xv = *reinterpret_cast<const float4 *>(&xs[k][4 * ty]);
#pragma unroll
            for (int kk = 0; kk < 3; ++kk) {
                if (kk < p.nk) {
                    const float4 bv = *reinterpret_cast<const float4 *>(&bs[kk][k][4 * tx]);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[kk][i][j] += f4get(xv, i) * f4get(bv, j);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = t0 + 4 * ty + i;
        if (t >= p.tokens) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = d0 + 4 * tx + j;
            if (d >= dirs) continue;
            for (int r = 0; r < p.dir_div; ++r) {
                const int m = d * p.dir_div + r;
                if (m >= p.members) break;
                float *o = p.out + ((int64_t)m * p.tokens + t) * p.nk;
#pragma unroll
                for (int kk = 0; kk < 3; ++kk)
                    if (kk < p.nk) o[kk] = acc[kk][i][j];
            }
        }
    }
}

__global__ __launch_bounds__(256) void dots_kernel(DotsArgs p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (int64_t)p.members * p.tokens) return;
    const int m = (int)(row / p.tokens), t = (int)(row - (int64_t)m * p.tokens);
    const int dir = m / p.dir_div;
    const __bf16 *xr = p.x + m * p.xs_m + (int64_t)t * p.xs_t;
    float acc[3] = {0.f, 0.f, 0.f};
    for (int n0 = lane * 8; n0 < p.width; n0 += 512) {
        bf16x8 xv = load_bf16x8(xr + n0);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if (k < p.nk) {
                float b[8];
                ld8(p.b[k] + dir * p.b_stride[k] + n0, b);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[k] += (float)xv[i] * b[i];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (k < p.nk) {
            float v = wave_sum(acc[k]);
            if (lane == 0) p.out[row * p.nk + k] = v;
        }
    }
}

// out[m] = mean_t loss[m, t] (eggroll.py:102 `.mean(-1)`), fixed-order tree: deterministic.
__global__ __launch_bounds__(256) void member_mean_kernel(const float *loss, int tokens, float *out) {
    __shared__ float part[256];
    const int m = blockIdx.x;
    const float *l = loss + (int64_t)m * tokens;
    float s = 0.f;
    for (int t = threadIdx.x; t < tokens; t += 256) s += l[t];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[m] = part[0] / (float)tokens;
}

// fp32 head operands split into bf16 pairs (hi = bf16(v), lo = bf16(v - hi)):
//   rows:   out[r] = [hi | lo | hi] of norm(x[r]) (norm optional)   -- the activations
//   weight: out[r] = [hi | hi | lo] of w[r]                           -- the head matrix
__global__ __launch_bounds__(256) void split3_kernel(const float *x, int64_t rows, int do_norm, int weight_order,
                                                     __bf16 *out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[8];
    ld8(x + row * 512 + lane * 8, v);
    if (do_norm) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
        const float r = rsqrtf(wave_sum(ss) * (1.0f / 512.0f) + kEps);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= r;
    }
    bf16x8 hi, lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = (__bf16)v[i];
        lo[i] = (__bf16)(v[i] - (float)hi[i]);
    }
    __bf16 *o = out + row * 1536 + lane * 8;
    store_bf16x8(o, hi);
    store_bf16x8(o + 512, weight_order ? hi : lo);
    store_bf16x8(o + 1024, weight_order ? lo : hi);
}

unsigned rows_grid(int64_t rows) { return (unsigned)((rows + 3) / 4); }

}  // namespace
}  // namespace noise

using namespace noise;

extern "C" int noise_pop_embed(const noise_population_t *pop, int per_member, const float *wte, int64_t vocab,
                               const int64_t *idx, const noise_rank1_t *emb_noise, const float *lam_r,
                               const float *lam_x, const float *eps_r,
                               const float *eps_x, int64_t eps_stride, float *x0, float *xin, void *h,
                               noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_embed";
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(wte && idx && x0 && xin && h && lam_r && lam_x, "%s: NULL pointer", fn);
    NOISE_CHECK_ARG(vocab > 0, "%s: vocab must be positive", fn);
    NOISE_CHECK_ARG(aligned(wte, 16) && aligned(x0, 16) && aligned(xin, 16) && aligned(h, 16), "%s: 16 B alignment", fn);
    const bool noisy = (emb_noise && emb_noise->a) || eps_r || eps_x;
    NOISE_CHECK_ARG(!noisy || (per_member && pop->sign), "%s: per-member noise needs per_member = 1 and sign", fn);
    NOISE_CHECK_ARG(pop->rounding == NOISE_ROUNDING_FUSED || pop->rounding == NOISE_ROUNDING_EAGER,
                    "%s: unknown rounding mode", fn);
    NOISE_CHECK_ARG(pop->rounding == NOISE_ROUNDING_FUSED || !noisy, "%s: eager rounding is for unperturbed calls", fn);
    EmbedArgs a;
    a.tokens = (int)pop->tokens;
    a.per_member = per_member;
    a.rows = (int)(per_member ? pop->members * pop->tokens : pop->tokens);
    a.dir_div = (int)pop->dir_div;
    a.wte = wte; a.idx = idx; a.sign = pop->sign;
    a.ea = emb_noise && emb_noise->a ? emb_noise->a : nullptr;
    a.eb = a.ea ? emb_noise->b : nullptr;
    a.ea_stride = a.ea ? emb_noise->a_stride : 0;
    a.eb_stride = a.ea ? emb_noise->b_stride : 0;
    a.lam_r = lam_r; a.lam_x = lam_x; a.eps_r = eps_r; a.eps_x = eps_x; a.eps_stride = eps_stride;
    a.vocab = vocab;
    a.x0 = x0; a.xin = xin; a.h = (__bf16 *)h;
    a.eager = pop->rounding == NOISE_ROUNDING_EAGER;
    hipLaunchKernelGGL(embed_kernel, dim3(rows_grid(a.rows)), dim3(256), 0, (hipStream_t)stream, a);
    return launch_status(fn);
}

extern "C" int noise_member_dots(const noise_population_t *pop, noise_view_t x, int64_t width,
                                 const noise_rank1_t *vecs, int64_t nk, float *out, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_member_dots";
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(nk >= 1 && nk <= 3 && vecs && out, "%s: need 1..3 vectors and an output", fn);
    NOISE_CHECK_ARG(width > 0 && width % 512 == 0, "%s: width must be a multiple of 512", fn);
    NOISE_CHECK_ARG(x.ptr && aligned(x.ptr, 16) && x.sm % 8 == 0 && x.st % 8 == 0, "%s: x misaligned", fn);
    DotsArgs a;
    a.members = (int)pop->members; a.tokens = (int)pop->tokens; a.width = (int)width; a.nk = (int)nk;
    a.dir_div = (int)pop->dir_div;
    a.x = (const __bf16 *)x.ptr; a.xs_m = x.sm; a.xs_t = x.st;
    for (int k = 0; k < 3; ++k) {
        a.b[k] = k < nk ? vecs[k].b : nullptr;
        a.b_stride[k] = k < nk ? vecs[k].b_stride : 0;
        if (k < nk) NOISE_CHECK_ARG(vecs[k].b && aligned(vecs[k].b, 16), "%s: b %d NULL or misaligned", fn, k);
    }
    a.out = out;
    if (x.sm == 0 && pop->members > 1) {
        // rows shared by every member: one dot per (token, direction)
        for (int k = 0; k < nk; ++k)
            NOISE_CHECK_ARG(vecs[k].b_stride % 4 == 0, "%s: b %d rows must be 16 B aligned", fn, k);
        const int64_t dirs = (pop->members + pop->dir_div - 1) / pop->dir_div;
        const dim3 grid((unsigned)((pop->tokens + kSdT - 1) / kSdT), (unsigned)((dirs + kSdD - 1) / kSdD));
        hipLaunchKernelGGL(shared_dots_kernel, grid, dim3(kSdThreads), 0, (hipStream_t)stream, a, (int)dirs);
    } else {
        hipLaunchKernelGGL(dots_kernel, dim3(rows_grid(pop->members * pop->tokens)), dim3(256), 0, (hipStream_t)stream,
                           a);
    }
    return launch_status(fn);
}

extern "C" int noise_member_mean(const float *token_loss, int64_t members, int64_t tokens, float *out,
                                 noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(token_loss && out && members > 0 && tokens > 0, "noise_member_mean: bad arguments");
    hipLaunchKernelGGL(member_mean_kernel, dim3((unsigned)members), dim3(256), 0, (hipStream_t)stream, token_loss,
                       (int)tokens, out);
    return launch_status("noise_member_mean");
}

extern "C" int noise_split3(const float *x, int64_t rows, int64_t width, int normalize, int weight_order, void *out,
                            noise_stream_t stream) {
    clear_error();
    NOISE_CHECK_ARG(x && out && rows > 0 && width == 512, "noise_split3: x/out NULL or width != 512");
    NOISE_CHECK_ARG(aligned(x, 16) && aligned(out, 16), "noise_split3: 16 B alignment");
    hipLaunchKernelGGL(split3_kernel, dim3(rows_grid(rows)), dim3(256), 0, (hipStream_t)stream, x, rows, normalize,
                       weight_order, (__bf16 *)out);
    return launch_status("noise_split3");
}

namespace noise {
namespace {

// lowrank_embed (eggroll.py:61-63): out[m, t, :] = W[idx[t], :] + sign[m] * a[dir, idx[t]] * b[dir, :]
__global__ __launch_bounds__(256) void lowrank_embed_kernel(float *out, const float *w, const int64_t *idx, int tokens,
                                                            int width, const float *a, const float *b,
                                                            int64_t a_stride, int64_t b_stride, const float *sign,
                                                            int dir_div, int64_t vocab, int64_t total) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= total) return;
    const int64_t row = i / width;
    const int n = (int)(i - row * width);
    const int m = (int)(row / tokens), t = (int)(row - (int64_t)m * tokens);
    const int dir = m / dir_div;
    const int64_t id = idx[t];
    if (id < 0 || id >= vocab) {  // an id outside the table: no read leaves it, the row is NaN
        const float nan = __builtin_nanf("");
        *reinterpret_cast<float4 *>(out + i) = float4{nan, nan, nan, nan};
        return;
    }
    const int64_t tok = id;
    float4 v = *reinterpret_cast<const float4 *>(w + tok * width + n);
    if (a) {
        const float s = sign[m] * a[dir * a_stride + tok];
        float4 bv = *reinterpret_cast<const float4 *>(b + dir * b_stride + n);
        v.x += s * bv.x; v.y += s * bv.y; v.z += s * bv.z; v.w += s * bv.w;
    }
    *reinterpret_cast<float4 *>(out + i) = v;
}

// Rank-1 expansion of a shared product (lowrank with x broadcast over members, eggroll.py:58):
// y[m, t, n] = base[t, n] + sign[m] * dots[t * dots_stride + m / dir_div] * a[m / dir_div, n], bf16 (y_fp32 = 0)
// or fp32 (1; 2 = the dot rounded to bf16 first, as autocast's x . b product). The x . b dots of a shared x
// depend on the direction only.
// A workgroup owns kExpRows token rows x 1024 columns: their base values stay in registers while it walks the
// members, reading each direction's a row (L2-resident) once for all of that direction's members, one
// direction ahead. Each store instruction covers 1 KiB (fp32) of one output row, lane after lane: stores
// whose lanes leave gaps (32 B per lane as two 16 B halves) measured 20% slower on this HBM-write stream.
constexpr int kExpRows = 4, kExpCols = 1024;
// DD: members per direction as a constant (2: antithetic pairs), or 0 to take dir_div at run time; FULL: every
// tile has all its rows and every direction all its members (no guards between the stores)
template <int DD, bool F32, bool FULL>
__global__ __launch_bounds__(256) void rank1_expand_kernel(void *__restrict__ y, int round_dot,
                                                           const float *__restrict__ base,
                                                           const float *__restrict__ dots, int64_t dots_stride,
                                                           const float *__restrict__ a, int64_t a_stride,
                                                           const float *__restrict__ sign, int members, int dir_div,
                                                           int tokens, int width) {
    const int dd = DD ? DD : dir_div;
    const int col_tiles = (width + kExpCols - 1) / kExpCols;
    const int t0 = (blockIdx.x / col_tiles) * kExpRows;
    const int n = (blockIdx.x % col_tiles) * kExpCols + 4 * threadIdx.x;
    if (n >= width) return;  // width is a multiple of 4: a lane's 4 columns are all in range or all out
    const int rows = FULL ? kExpRows : min(kExpRows, tokens - t0);
    float4 bv[kExpRows];
#pragma unroll
    for (int r = 0; r < kExpRows; ++r)
        bv[r] = r < rows ? ld4(base + (int64_t)(t0 + r) * width + n) : float4{0.f, 0.f, 0.f, 0.f};
    const int dirs = (members + dd - 1) / dd;
    const int64_t mstride = (int64_t)tokens * width;
    float4 av[2];
    float dv[2][kExpRows];
    auto fetch = [&](int d, int slot) {
        av[slot] = ld4(a + (int64_t)d * a_stride + n);
#pragma unroll
        for (int r = 0; r < kExpRows; ++r) dv[slot][r] = r < rows ? dots[(int64_t)(t0 + r) * dots_stride + d] : 0.f;
    };
    auto emit = [&](int m, int u, const float4 &ad) {
        const float sg = sign[m];
        char *ym = (char *)y + (m * mstride + (int64_t)t0 * width + n) * (F32 ? 4 : 2);
#pragma unroll
        for (int r = 0; r < kExpRows; ++r) {
            if (!FULL && r >= rows) break;
            const float c = sg * (round_dot ? bfr(dv[u][r]) : dv[u][r]);
            const float4 o{bv[r].x + c * ad.x, bv[r].y + c * ad.y, bv[r].z + c * ad.z, bv[r].w + c * ad.w};
            if constexpr (F32) {
                st4(reinterpret_cast<float *>(ym) + (int64_t)r * width, o);
            } else {
                store_bf16x4(reinterpret_cast<__bf16 *>(ym) + (int64_t)r * width,
                             bf16x4{(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w});
            }
        }
    };
    fetch(0, 0);
    for (int d0 = 0; d0 < dirs; d0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int d = d0 + u;
            if (d >= dirs) break;
            if (d + 1 < dirs) fetch(d + 1, u ^ 1);
            const float4 ad = av[u];
            if constexpr (DD != 0) {
#pragma unroll
                for (int e = 0; e < DD; ++e)
                    if (FULL || d * DD + e < members) emit(d * DD + e, u, ad);
            } else {
                for (int m = d * dd; m < (d + 1) * dd && m < members; ++m) emit(m, u, ad);
            }
        }
    }
}

// lowrank (eggroll.py:56-58) for shapes the MFMA tiles do not take, such as the value-embedding gate's
// [8, 32] weight applied to h[..., :32] (eggroll.py:88):
//   y[m, t, o] = bf16(x[m, t] . W[o]) + sign[m] * bf16(x[m, t] . bf16(b[dir])) * a[dir, o]
// with fp32 accumulation and the two products rounded to bf16 as autocast's matmuls return them (b enters
// the matmul rounded, a multiplies in fp32); y fp32 [m][T][out]. One thread per output element.
__global__ __launch_bounds__(256) void lowrank_rows_kernel(int tokens, int n_in, int n_out, int dir_div,
                                                           const __bf16 *x, int64_t xs_m, int64_t xs_t,
                                                           const __bf16 *w, const float *a, const float *b,
                                                           int64_t a_stride, int64_t b_stride, const float *sign,
                                                           float *y, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int64_t row = i / n_out;
    const int o = (int)(i - row * n_out);
    const int m = (int)(row / tokens), t = (int)(row - (int64_t)m * tokens);
    const int dir = m / dir_div;
    const __bf16 *xr = x + m * xs_m + (int64_t)t * xs_t;
    const __bf16 *wr = w + (int64_t)o * n_in;
    const float *br = a ? b + dir * b_stride : nullptr;
    float prod = 0.f, dot = 0.f;
    for (int k = 0; k < n_in; ++k) {
        const float xv = (float)xr[k];
        prod += xv * (float)wr[k];
        if (br) dot += xv * bfr(br[k]);
    }
    float v = bfr(prod);
    if (a) v += sign[m] * bfr(dot) * a[dir * a_stride + o];
    y[i] = v;
}

}  // namespace
}  // namespace noise

extern "C" int noise_lowrank_embed(float *out, const float *w, int64_t vocab, int64_t width, const int64_t *idx,
                                   const noise_population_t *pop, const noise_rank1_t *r1, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_lowrank_embed";
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(out && w && idx && vocab > 0 && width > 0 && width % 4 == 0, "%s: bad arguments", fn);
    NOISE_CHECK_ARG(aligned(out, 16) && aligned(w, 16), "%s: 16 B alignment", fn);
    const bool noisy = r1 && r1->a;
    NOISE_CHECK_ARG(!noisy || (pop->sign && r1->b && aligned(r1->b, 16) && r1->b_stride % 4 == 0),
                    "%s: noise needs sign and 16 B aligned b rows", fn);
    const int64_t total = pop->members * pop->tokens * width;
    hipLaunchKernelGGL(lowrank_embed_kernel, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, out, w, idx, (int)pop->tokens, (int)width, noisy ? r1->a : nullptr,
                       noisy ? r1->b : nullptr, noisy ? r1->a_stride : 0, noisy ? r1->b_stride : 0, pop->sign,
                       (int)pop->dir_div, vocab, total);
    return launch_status(fn);
}

extern "C" int noise_rank1_expand(const noise_population_t *pop, const float *base, int64_t width, const float *dots,
                                  int64_t dots_stride, const noise_rank1_t *r1, void *y, int y_fp32,
                                  noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_rank1_expand";
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1 && pop->sign, "%s: bad population", fn);
    NOISE_CHECK_ARG(base && dots && r1 && r1->a && y && width > 0 && width % 4 == 0 && width <= INT32_MAX, "%s: bad arguments", fn);
    const int64_t dirs = (pop->members + pop->dir_div - 1) / pop->dir_div;
    NOISE_CHECK_ARG(dots_stride >= dirs, "%s: dots rows hold %lld directions, %lld needed", fn, (long long)dots_stride,
                    (long long)dirs);
    NOISE_CHECK_ARG(aligned(base, 16) && aligned(r1->a, 16) && r1->a_stride % 4 == 0 && aligned(y, y_fp32 ? 16 : 8),
                    "%s: alignment", fn);
    const int64_t tiles = (pop->tokens + kExpRows - 1) / kExpRows * ((width + kExpCols - 1) / kExpCols);
    NOISE_CHECK_ARG(tiles <= INT32_MAX, "%s: too many tiles", fn);
    const dim3 grid((unsigned)tiles), block(256);
    const int rd = y_fp32 == 2;
    const int m = (int)pop->members, dd = (int)pop->dir_div, T = (int)pop->tokens, W = (int)width;
    hipStream_t st = (hipStream_t)stream;
    const bool full = T % kExpRows == 0 && m % dd == 0;
#define NOISE_EXPAND(DD, F, FULL)                                                                                    \
    hipLaunchKernelGGL((rank1_expand_kernel<DD, F, FULL>), grid, block, 0, st, y, rd, base, dots, dots_stride, r1->a, \
                       r1->a_stride, pop->sign, m, dd, T, W)
    if (dd == 2 && y_fp32 && full) NOISE_EXPAND(2, true, true);
    else if (dd == 2 && y_fp32) NOISE_EXPAND(2, true, false);
    else if (dd == 2 && full) NOISE_EXPAND(2, false, true);
    else if (dd == 2) NOISE_EXPAND(2, false, false);
    else if (y_fp32) NOISE_EXPAND(0, true, false);
    else NOISE_EXPAND(0, false, false);
#undef NOISE_EXPAND
    return launch_status(fn);
}

namespace noise {
namespace {

// Value-embedding gates (eggroll.py:88, model.py:89): gates[row, h] = 2 sigmoid(x[row, :32] . Wg[h] (+ sign *
// (x[:32] . b_g) * a_g[h] for lowrank ve_gate)), one thread per row.
__global__ __launch_bounds__(256) void gate_kernel(int members, int tokens, int dir_div, const __bf16 *x, int64_t xs_m,
                                                   int64_t xs_t, const float *wg, const float *sign, const float *ga,
                                                   const float *gb, int64_t ga_stride, int64_t gb_stride, float *out,
                                                   int eager) {
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= (int64_t)members * tokens) return;
    const int m = (int)(row / tokens), t = (int)(row - (int64_t)m * tokens);
    const __bf16 *xr = x + m * xs_m + (int64_t)t * xs_t;
    float xf[32];
#pragma unroll
    for (int c8 = 0; c8 < 4; ++c8) {
        bf16x8 v = load_bf16x8(xr + 8 * c8);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[8 * c8 + e] = (float)v[e];
    }
    float dg = 0.f;
    const int dir = m / dir_div;
    if (ga) {
#pragma unroll
        for (int c = 0; c < 32; ++c) dg += xf[c] * gb[dir * gb_stride + c];
        dg *= sign[m];
    }
#pragma unroll
    for (int h = 0; h < 8; ++h) {
        float z = 0.f;
#pragma unroll
        for (int c = 0; c < 32; ++c) z += xf[c] * wg[h * 32 + c];
        if (ga) z += dg * ga[dir * ga_stride + h];
        // eager: bf16 linear output, bf16 sigmoid, times 2 (exact)
        out[row * 8 + h] = eager ? 2.0f * bfr(1.0f / (1.0f + __expf(-bfr(z)))) : 2.0f / (1.0f + __expf(-z));
    }
}

}  // namespace
}  // namespace noise

extern "C" int noise_pop_gate(const noise_population_t *pop, noise_view_t x, const float *gate_w,
                              const noise_rank1_t *gate_noise, float *gates, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_pop_gate";
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(x.ptr && aligned(x.ptr, 16) && x.sm % 8 == 0 && x.st % 8 == 0, "%s: x misaligned", fn);
    NOISE_CHECK_ARG(gate_w && gates, "%s: NULL gate weights or output", fn);
    const bool noisy = gate_noise && gate_noise->a;
    NOISE_CHECK_ARG(!noisy || (pop->sign && gate_noise->b), "%s: gate noise needs sign and b", fn);
    NOISE_CHECK_ARG(pop->rounding == NOISE_ROUNDING_FUSED || (pop->rounding == NOISE_ROUNDING_EAGER && !noisy),
                    "%s: unknown rounding mode, or eager rounding with gate noise", fn);
    const int64_t rows = pop->members * pop->tokens;
    hipLaunchKernelGGL(gate_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (int)pop->members, (int)pop->tokens, (int)pop->dir_div, (const __bf16 *)x.ptr, x.sm, x.st, gate_w,
                       pop->sign, noisy ? gate_noise->a : nullptr, noisy ? gate_noise->b : nullptr,
                       noisy ? gate_noise->a_stride : 0, noisy ? gate_noise->b_stride : 0, gates,
                       (int)(pop->rounding == NOISE_ROUNDING_EAGER));
    return launch_status(fn);
}

extern "C" int noise_lowrank_rows(const noise_population_t *pop, noise_view_t x, int64_t n_in, const void *w,
                                  int64_t n_out, const noise_rank1_t *r1, float *y, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_lowrank_rows";
    NOISE_CHECK_ARG(pop && pop->members > 0 && pop->tokens > 0 && pop->dir_div >= 1, "%s: bad population", fn);
    NOISE_CHECK_ARG(x.ptr && w && y && n_in > 0 && n_out > 0, "%s: NULL pointer or empty shape", fn);
    NOISE_CHECK_ARG(pop->members * pop->tokens * n_out < (1ll << 38), "%s: output too large", fn);
    const bool noisy = r1 && r1->a;
    NOISE_CHECK_ARG(!noisy || (pop->sign && r1->b), "%s: noise needs sign and b rows", fn);
    const int64_t total = pop->members * pop->tokens * n_out;
    hipLaunchKernelGGL(lowrank_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (int)pop->tokens, (int)n_in, (int)n_out, (int)pop->dir_div, (const __bf16 *)x.ptr, x.sm, x.st,
                       (const __bf16 *)w, noisy ? r1->a : nullptr, noisy ? r1->b : nullptr,
                       noisy ? r1->a_stride : 0, noisy ? r1->b_stride : 0, pop->sign, y, total);
    return launch_status(fn);
}

namespace noise {
namespace {

// DUST.rerun's glue between blocks (run.py:262-268), over rows of 512 (one wave per row):
//   entry (x0 == NULL): out[r] = norm(e[r % e_rows] (+ add[r]))      the jittered embedding entry
//   mix   (x0 != NULL): out[r] = rl * x[r] + ml * x0[r % x0_rows]     the next block's mixing scalars
// e / x fp32, add bf16 or NULL, x0 fp32; rl, ml read on the device. With h, the mixed row's norm is also
// stored as bf16 (the normalised input of the block the row enters, utils/model.py:117).
__global__ __launch_bounds__(256) void rerun_rows_kernel(const float *x, int64_t x_rows, const __bf16 *add,
                                                         const float *x0, int64_t x0_rows, const float *lam_r,
                                                         const float *lam_x, int64_t rows, float *out,
                                                         __bf16 *h) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[8];
    ld8(x + (row % x_rows) * 512 + lane * 8, v);
    if (x0) {
        const float rl = *lam_r, ml = *lam_x;
        float z[8];
        ld8(x0 + (row % x0_rows) * 512 + lane * 8, z);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = rl * v[i] + ml * z[i];
    } else {
        if (add) {
            const bf16x8 a = load_bf16x8(add + row * 512 + lane * 8);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] += (float)a[i];
        }
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
        const float r = rsqrtf(wave_sum(ss) * (1.0f / 512.0f) + kEps);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= r;
    }
    st8(out + row * 512 + lane * 8, v);
    if (h) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
        const float r = rsqrtf(wave_sum(ss) * (1.0f / 512.0f) + kEps);
        bf16x8 hb;
#pragma unroll
        for (int i = 0; i < 8; ++i) hb[i] = (__bf16)(v[i] * r);
        store_bf16x8(h + row * 512 + lane * 8, hb);
    }
}

}  // namespace
}  // namespace noise

extern "C" int noise_rerun_rows(const float *x, int64_t x_rows, const void *add, const float *x0, int64_t x0_rows,
                                const float *lam_r, const float *lam_x, int64_t rows, float *out,
                                noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_rerun_rows";
    NOISE_CHECK_ARG(x && out && rows > 0 && x_rows > 0 && aligned(x, 16) && aligned(out, 16), "%s: bad x / out", fn);
    NOISE_CHECK_ARG(!add || aligned(add, 16), "%s: add must be 16 B aligned", fn);
    NOISE_CHECK_ARG(!x0 || (x0_rows > 0 && aligned(x0, 16) && lam_r && lam_x && !add),
                    "%s: mixing needs x0 rows, both lambdas and no add", fn);
    hipLaunchKernelGGL(rerun_rows_kernel, dim3(rows_grid(rows)), dim3(256), 0, (hipStream_t)stream, x, x_rows,
                       (const __bf16 *)add, x0, x0_rows, lam_r, lam_x, rows, out, nullptr);
    return launch_status(fn);
}

namespace noise {
namespace {

// A jittered block's entry (run.py:265, 102-110): out[r] = x[r % x_rows] + add[r] (the attn.c_proj jitter folded
// into the residual the block adds its product to), h[r] = bf16(norm(x[r % x_rows])) (the block's own input).
__global__ __launch_bounds__(256) void block_entry_kernel(const float *x, int64_t x_rows, const __bf16 *add,
                                                          int64_t rows, float *out, __bf16 *h) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float v[8];
    ld8(x + (row % x_rows) * 512 + lane * 8, v);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
    const float r = rsqrtf(wave_sum(ss) * (1.0f / 512.0f) + kEps);
    bf16x8 hb;
#pragma unroll
    for (int i = 0; i < 8; ++i) hb[i] = (__bf16)(v[i] * r);
    store_bf16x8(h + row * 512 + lane * 8, hb);
    if (add) {
        const bf16x8 a = load_bf16x8(add + row * 512 + lane * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += (float)a[i];
    }
    st8(out + row * 512 + lane * 8, v);
}

// y = bf16(y + add), 8 elements per thread
__global__ __launch_bounds__(256) void add_bf16_rows_kernel(__bf16 *__restrict__ y, const __bf16 *__restrict__ add,
                                                            int64_t n8) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    bf16x8 a = load_bf16x8(y + 8 * i);
    const bf16x8 b = load_bf16x8(add + 8 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = (__bf16)((float)a[e] + (float)b[e]);
    store_bf16x8(y + 8 * i, a);
}

}  // namespace
}  // namespace noise

extern "C" int noise_block_entry(const float *x, int64_t x_rows, const void *add, int64_t rows, float *out, void *h,
                                 noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_block_entry";
    NOISE_CHECK_ARG(x && out && h && rows > 0 && x_rows > 0 && aligned(x, 16) && aligned(out, 16) && aligned(h, 16),
                    "%s: bad x / out / h", fn);
    NOISE_CHECK_ARG(!add || aligned(add, 16), "%s: add must be 16 B aligned", fn);
    hipLaunchKernelGGL(block_entry_kernel, dim3(rows_grid(rows)), dim3(256), 0, (hipStream_t)stream, x, x_rows,
                       (const __bf16 *)add, rows, out, (__bf16 *)h);
    return launch_status(fn);
}

extern "C" int noise_add_bf16(void *y, const void *add, int64_t n, noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_add_bf16";
    NOISE_CHECK_ARG(y && add && n > 0 && n % 8 == 0 && aligned(y, 16) && aligned(add, 16),
                    "%s: 16 B aligned y and add and n a positive multiple of 8 required", fn);
    const int64_t n8 = n / 8;
    NOISE_CHECK_ARG((n8 + 255) / 256 < (1ll << 31), "%s: n too large", fn);
    hipLaunchKernelGGL(add_bf16_rows_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (__bf16 *)y, (const __bf16 *)add, n8);
    return launch_status(fn);
}

extern "C" int noise_rerun_mix_norm(const float *x, int64_t x_rows, const float *x0, int64_t x0_rows,
                                    const float *lam_r, const float *lam_x, int64_t rows, float *out, void *h,
                                    noise_stream_t stream) {
    clear_error();
    const char *fn = "noise_rerun_mix_norm";
    NOISE_CHECK_ARG(x && out && h && rows > 0 && x_rows > 0 && aligned(x, 16) && aligned(out, 16) && aligned(h, 16),
                    "%s: bad x / out / h", fn);
    NOISE_CHECK_ARG(x0 && x0_rows > 0 && aligned(x0, 16) && lam_r && lam_x, "%s: mixing needs x0 rows and both lambdas",
                    fn);
    hipLaunchKernelGGL(rerun_rows_kernel, dim3(rows_grid(rows)), dim3(256), 0, (hipStream_t)stream, x, x_rows,
                       (const __bf16 *)nullptr, x0, x0_rows, lam_r, lam_x, rows, out, (__bf16 *)h);
    return launch_status(fn);
}
