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

/* Several parameters' slices in one launch (Eggroll.noise's gathers for every perturbed parameter of a step,
 * eggroll.py:126-127, at the same directions): group k writes element (offsets[k][rows[r]] + j) of the draw to
 * out[r * ld + col[k] + j] for j < width[k]. Groups are packed in order (col[0] = 0, col[k+1] = col[k] +
 * width[k]), widths are multiples of 256, ld >= the total width; out-of-range elements are NaN as in
 * noise_gather_slices. The descriptor is passed by value to the kernel (no device copy). */
#define NOISE_SLICE_GROUPS_MAX 64
typedef struct {
    int32_t count;
    const int64_t *offsets[NOISE_SLICE_GROUPS_MAX];
    int64_t width[NOISE_SLICE_GROUPS_MAX];
    int64_t col[NOISE_SLICE_GROUPS_MAX];
} noise_slice_groups_t;
int noise_gather_slice_groups(float *out, int64_t nrows, int64_t ld, const noise_slice_groups_t *groups,
                              const int64_t *rows, int64_t numel, uint64_t seed, uint64_t offset, int64_t threads,
                              noise_stream_t stream);

/* Orthogonal draws of DUST.orthogonal_noise (run.py:223-238; hadamard run.py:143-152): out[i][f][j] for
 * draws i < n, frame positions f < bt (the reference's b*t tokens) and coordinates j < d (a power of two):
 *   index = index0 + i (the reference's rank*draws + chunk*n + i), row = (offset[f] + index) mod d,
 *   out = H_d[row][j] * (2*pattern[index / d][j] - 1) * (2*sign[i*bt + f] - 1)
 * with H_d the Sylvester Hadamard matrix (entry (-1)^popcount(row & j)), pattern [cycles][d] and offset
 * [bt] the raw torch.randint(0, 2) / randint(0, d) outputs of the shared generator, sign [n][bt] the raw
 * randint(0, 2) of the rank generator (int64 as torch returns them; noise_randint produces them bit for
 * bit). out is fp32, or bf16 when out_bf16 (+-1 is exact in both). index0 + n must be <= cycles*d. */
int noise_orthogonal_draws(void *out, int out_bf16, int64_t n, int64_t bt, int64_t d, int64_t index0,
                           const int64_t *offset, const int64_t *pattern, int64_t cycles, const int64_t *sign,
                           noise_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Attention
 * ---------------------------------------------------------------------------------------------- */

/* Causal attention with a left window: query s attends to keys s - window .. s (window >= seq - 1 is
 * plain causal), softmax(q k^T * scale) v, bf16 in and out, fp32 accumulation. Replaces utils/model.py:24-31
 * `attention(q, k, v, window)` (flex_attention with the block mask q >= k & q - k <= window,
 * model.py:17-21; scale 1/sqrt(head_dim), torch: nn/attention/flex_attention.py:1543-1544).
 * q, k, o: element (b, t, h, d) at b*s_b + h*s_h + t*s_t + d (the reference's [B, T, H, D] and its
 * transposes are all expressible). v: the same with vs_x = token stride, or, with flag
 * NOISE_ATTN_V_TRANSPOSED, element (b, t, h, d) at b*vs_b + h*vs_h + d*vs_x + t. head_dim must be 64.
 * A seq in whole 256-query tiles runs the ring kernel with either V layout, other lengths the general one.
 * NOISE_ATTN_QK_NORMED: the caller guarantees every q and k row has RMS <= 1, as RMSNorm outputs do (the
 * reference normalises both, utils/model.py:94); scores are then bounded and the softmax runs with a
 * fixed shift instead of a running maximum (same result; rows that break the promise by less than a
 * factor of about 3 in RMS still stay finite). Optional fused output (dot_out != NULL):
 * dot_out[(b*seq + t)*heads + h] = sum_d o[b,t,h,d] * dot_vec[(b / dot_div)*dot_vec_stride + h*64 + d],
 * with o the bf16 output values; this is the per-head part of the next perturbed linear's x.b
 * (eggroll.py:58), NULL to skip. */
#define NOISE_ATTN_V_TRANSPOSED 1
#define NOISE_ATTN_QK_NORMED 2

/* V element (b, t, h, d) at b*vs_b + h*vs_h + t*vs_t + d -> vt [batch][heads][64][seq] contiguous, the
 * NOISE_ATTN_V_TRANSPOSED layout that the population path writes (no counterpart in the reference; a layout
 * utility: noise_attention_fwd takes V in either layout, so the attention(q, k, v, window) drop-in,
 * utils/model.py:24-31, passes V as it is). seq a multiple of 64, head_dim 64. */
int noise_v_transpose(const void *v, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim, int64_t vs_b,
                      int64_t vs_h, int64_t vs_t, void *vt, noise_stream_t stream);
int noise_attention_fwd(const void *q, const void *k, const void *v, void *o, int64_t batch, int64_t heads,
                        int64_t seq, int64_t head_dim, int64_t qs_b, int64_t qs_h, int64_t qs_t, int64_t ks_b,
                        int64_t ks_h, int64_t ks_t, int64_t vs_b, int64_t vs_h, int64_t vs_x, int flags,
                        int64_t os_b, int64_t os_h, int64_t os_t, int64_t window, float scale,
                        const float *dot_vec, int64_t dot_vec_stride, int64_t dot_div, float *dot_out,
                        noise_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Perturbed linears of the population forward (eggroll.py:56-58 `lowrank`, fused with what the
 * reference runs around each one in population_loss, eggroll.py:66-103).
 *
 * Rows are (member, token) pairs. A member m uses noise row m / dir_div of each [directions, width]
 * noise table (dir_div = 2 for antithetic pairs, eggroll.py:141) and scale sign[m] (+-sigma,
 * eggroll.py:138). The rank-1 term sign[m] * (x . b) * a^T is split: the x . b dots of a layer's input
 * are produced by the kernel that writes that input (its epilogue), and the consumer adds
 * sign[m] * dot * a[n]. Matrices are bf16 [out, in] row-major (torch Linear layout). Activations are
 * bf16 unless stated; the residual stream is fp32. tokens must be a multiple of the tile (256).
 * ---------------------------------------------------------------------------------------------- */

/* Strided 3-D view: element (m, t, j) at ptr + m*sm + t*st + j. sm = 0 broadcasts one row-set to all
 * members. Strides are in elements. */
typedef struct {
    const void *ptr;
    int64_t sm, st;
} noise_view_t;

/* Per-member rank-1 noise of one matrix: a [dirs, out], b [dirs, in] fp32 rows (a_stride, b_stride
 * elements apart); NULL a means the matrix is unperturbed. */
typedef struct {
    const float *a;
    const float *b;
    int64_t a_stride, b_stride;
} noise_rank1_t;

/* Rounding of the forward between its stored tensors (noise_population_t.rounding):
 * FUSED  the training scripts' compiled population forward (eggroll.py:66-103 under torch.compile): elementwise
 *        chains in fp32, the residual stream fp32, bf16 only where a tensor is materialised in bf16;
 * EAGER  the scorer's eager autocast forward (utils/eval.py:43-46 over utils/model.py:193-209 with the bf16
 *        embeddings of model.py:170-174): every elementwise op's result rounded to bf16, so the residual
 *        stream is bf16-valued. Unperturbed calls only (no rank-1 terms, lambda noise or next-matrix dots). */
#define NOISE_ROUNDING_FUSED 0
#define NOISE_ROUNDING_EAGER 1

/* Shared member bookkeeping of one population call. */
typedef struct {
    int64_t members, tokens;
    const float *sign;   /* [members] +-sigma (or any per-member scale) */
    int64_t dir_div;     /* member m uses noise row m / dir_div */
    int64_t rounding;    /* NOISE_ROUNDING_FUSED (0) or NOISE_ROUNDING_EAGER */
} noise_population_t;

/* Block entry (eggroll.py:74-79 for block 0; model.py:196-199): e = wte[idx[t]] (+ sign * a[idx[t]] * b,
 * lowrank_embed eggroll.py:61-63), x0 = norm(e), x = rl*x0 + ml*x0 (rl = *lam_r, ml = *lam_x: block 0's
 * resid / x0 lambda, read on the device, + sign * eps when eps_* != NULL, eggroll.py:77-78),
 * h = bf16(norm(x)). per_member = 0 writes one shared [tokens][512] set (no embedding or lambda noise);
 * per_member = 1 writes [members][tokens][512]. wte is fp32 [vocab][512] (eggroll.py:50). x0, xin fp32,
 * h bf16. A token id outside [0, vocab) reads no memory outside the table and yields NaN rows (the
 * reference raises an IndexError there). */
int noise_pop_embed(const noise_population_t *pop, int per_member, const float *wte, int64_t vocab,
                    const int64_t *idx, const noise_rank1_t *emb_noise, const float *lam_r, const float *lam_x,
                    const float *eps_r, const float *eps_x, int64_t eps_stride, float *x0, float *xin, void *h,
                    noise_stream_t stream);

/* out[(m*tokens + t)*nk + k] = sum_n x[m, t, n] * vecs[k].b[(m / dir_div)*b_stride + n], n < width:
 * the x . b factor of eggroll.py:58's rank-1 term for up to 3 matrices sharing input x. */
int noise_member_dots(const noise_population_t *pop, noise_view_t x, int64_t width, const noise_rank1_t *vecs,
                      int64_t nk, float *out, noise_stream_t stream);

/* Value-embedding gates of one block (eggroll.py:88 / model.py:89): gates[row*8 + h] =
 * 2 sigmoid(x[row, :32] . gate_w[h] + sign * (x[:32] . b) * a[h]) with x the block's normalised input
 * (bf16), gate_w fp32 [8][32] = attn.ve_gate.weight, gate_noise its rank-1 noise (a [dirs][8], b [dirs][32])
 * or NULL. */
int noise_pop_gate(const noise_population_t *pop, noise_view_t x, const float *gate_w, const noise_rank1_t *gate_noise,
                   float *gates, noise_stream_t stream);

/* Q, K, V of one block for every member (eggroll.py:81-90): x (= norm of the block input, bf16) times
 * c_q, c_k, c_v (w[0..2], bf16 [512][512]) + sign * dots[row*3 + i] * a_i; on V, + gates[row*8 + h] *
 * (ve[idx[m * idx_sm + t], :] + lowrank_embed noise of the value table, ve_noise a [dirs][V], b [dirs][512],
 * or NULL) when ve (fp32 [V][512]) is not NULL; idx_sm = 0 when every member reads the same sequence (the
 * population), else the member stride of per-member token ids (>= tokens: scoring distinct sequences); rotary (rope_cos/rope_sin: model.py:177-183's bf16 tables,
 * [tokens][32] bf16, 16 B aligned) then per-head RMSNorm on Q and K. Outputs bf16: Q, K
 * [members][8][tokens][64]; V transposed [members][8][64][tokens]. ve has `vocab` rows: a token id outside
 * [0, vocab) reads no memory outside it and makes that token's V NaN. */
int noise_pop_qkv(const noise_population_t *pop, noise_view_t x, const void *const w[3], const noise_rank1_t r1[3],
                  const float *dots, const void *rope_cos, const void *rope_sin, const float *ve, int64_t vocab,
                  const int64_t *idx, int64_t idx_sm, const float *gates, const noise_rank1_t *ve_noise,
                  void *const out[3], noise_stream_t stream);

/* noise_pop_qkv for an input every member shares (block 0 of the population when the embedding and the
 * mixing scalars are unperturbed; no value embeddings): base = x [c_q; c_k; c_v]^T, fp32 [tokens][1536],
 * computed once by the caller (noise_pop_linear with one member), then per member base + sign * dots[row*3 +
 * i] * a_i, rotary and per-head RMSNorm on Q and K. Same outputs as noise_pop_qkv (16 B aligned); tokens a
 * multiple of 64; fused rounding only. No counterpart in the reference beyond eggroll.py:81-90 itself: the
 * shared product is this library's restructuring of the same arithmetic. */
int noise_pop_qkv_shared(const noise_population_t *pop, const float *base, const noise_rank1_t r1[3],
                         const float *dots, const void *rope_cos, const void *rope_sin, void *const out[3],
                         noise_stream_t stream);

/* Residual writer (eggroll.py:92 attn.c_proj and :93 mlp.c_proj): y = xres + x w^T + sign * (sum of
 * dots_count dots at dots[row*dots_stride]) * a; if mix: y = rl*y + ml*x0 (the next block's mixing,
 * eggroll.py:79, rl = *lam_r and ml = *lam_x read on the device, + sign * eps); xout = y (fp32, may be NULL); hout = bf16(norm(y)) [m][T][512]
 * or, with split3, its [hi | lo | hi] bf16 split [m][T][1536] for the fp32 head; next_dots[row*nnext+k]
 * = norm(y) . next[k].b (0 <= nnext <= 3). w bf16 [512][K], K = 512 (attn.c_proj) or 2048 (mlp.c_proj). */
int noise_pop_residual(const noise_population_t *pop, noise_view_t x, const void *w, int64_t K,
                       const noise_rank1_t *r1, const float *dots, int64_t dots_stride, int64_t dots_count,
                       noise_view_t xres, float *xout, int mix, const float *lam_r, const float *lam_x, const float *eps_r,
                       const float *eps_x, int64_t eps_stride, noise_view_t x0, void *hout, int split3,
                       const noise_rank1_t *next, int64_t nnext, float *next_dots, noise_stream_t stream);

/* MLP hidden (eggroll.py:93): act = relu(x w^T + sign * dots[row] * a)^2 as bf16 [m][T][2048];
 * partial_dots[row*16 + n/128] = sum over that 128-feature slice of act * next->b (for mlp.c_proj's
 * rank-1 term; NULL next skips). w bf16 [2048][512]. */
int noise_pop_fc(const noise_population_t *pop, noise_view_t x, const void *w, const noise_rank1_t *r1,
                 const float *dots, void *act, const noise_rank1_t *next, float *partial_dots,
                 noise_stream_t stream);

/* Perturbed linear (eggroll.py:56-58 `lowrank`): y[m, t, :] = x[m, t, :] w^T + sign[m] * dots[m*T+t] *
 * a[m / dir_div] (dots = x . b from noise_member_dots; r1 NULL or r1->a NULL: plain linear). bf16 x and
 * w [N][K]; y with strides ys_m, ys_t: bf16 (y_fp32 = 0), fp32 (1), or fp32 in autocast's form (2: the
 * product and the dot rounded to bf16 before the fp32 sum, as eggroll.py:58 runs under autocast).
 * N multiple of 256, K of 64. */
int noise_pop_linear(const noise_population_t *pop, noise_view_t x, const void *w, int64_t K, int64_t N,
                     const noise_rank1_t *r1, const float *dots, void *y, int y_fp32, int64_t ys_m, int64_t ys_t,
                     noise_stream_t stream);

/* Head, soft cap 15 and per-token cross-entropy (eggroll.py:94-101, model.py:202-209, run.py:89-94):
 * logits = x w^T (+ sign * dots * a), z = 15 tanh(logits / 15), token_loss[m*T + t] = logsumexp(z) -
 * z[target]: 0 where target == -1 (ignore_index), NaN for any other target outside [0, vocab) (where
 * F.cross_entropy raises). w bf16 [vocab][K]; K = 512, or 1536 for the split-bf16x3 fp32 head
 * (x = [hi|lo|hi], w = [hi|hi|lo], noise_split3). targets int64 [T] shared (targets_sm = 0) or per member. */
int noise_pop_head_ce(const noise_population_t *pop, noise_view_t x, const void *w, int64_t K, int64_t vocab,
                      const noise_rank1_t *r1, const float *dots, const int64_t *targets, int64_t targets_sm,
                      float *token_loss, noise_stream_t stream);

/* The block's whole MLP with its residual writer (eggroll.py:93, then the next block's mixing, eggroll.py:77-79,
 * and what noise_pop_residual derives from the new residual): with x = h (bf16, the norm of the block's mid
 * residual) and per member m,
 *   hid = relu(x w_fc^T + sign * dots_fc * a_fc)^2 (bf16),  y = xres + hid w_proj^T + sign * (hid . b_proj) * a_proj,
 *   if mix: y = rl*y + ml*x0 (rl = *lam_r, ml = *lam_x, + sign * eps); xout = y (fp32, may equal xres, may be
 *   NULL); hout = bf16(norm(y)) [m][T][512] or its [hi | lo | hi] split [m][T][1536] (split3);
 *   next_dots[row*nnext + k] = norm(y) . next[k].b.
 * The [m][T][2048] hidden layer never reaches memory. w_fc: mlp.c_fc bf16 [2048][512]; w_proj: mlp.c_proj bf16
 * [512][2048] in the layout noise_mlp_proj_layout writes. r_fc: c_fc's rank-1 noise (a [dirs][2048]) with
 * dots_fc = x . b_fc per row (noise_pop_residual's next dots); r_proj: mlp.c_proj's (a [dirs][512],
 * b [dirs][2048]); NULL or a == NULL: unperturbed. tokens a multiple of 128; fused rounding only. Same results
 * as noise_pop_fc followed by noise_pop_residual with K = 2048, up to fp32 summation order. */
int noise_pop_mlp(const noise_population_t *pop, noise_view_t x, const void *w_fc, const noise_rank1_t *r_fc,
                  const float *dots_fc, const void *w_proj, const noise_rank1_t *r_proj, noise_view_t xres, float *xout,
                  int mix, const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x,
                  int64_t eps_stride, noise_view_t x0, void *hout, int split3, const noise_rank1_t *next, int64_t nnext,
                  float *next_dots, noise_stream_t stream);

/* Attention projection, residual, RMSNorm and the whole MLP of a block in one kernel (eggroll.py:92-93 and
 * the mixing, norm and next-matrix dots that follow, eggroll.py:77-82 / 94; replaces noise_pop_residual with
 * K = 512 followed by noise_pop_mlp): x_mid = xres + y w_o^T + sign (sum of the o_dots_n partial dots
 * o_dots[row][.]) a_o, h = norm(x_mid) (in registers), then noise_pop_mlp's arithmetic on h with x_mid as its
 * residual. y: the attention output, bf16 [members][tokens][512]; w_o bf16 [512][512]; r_o: attn.c_proj's
 * rank-1 noise (a [dirs][512]) or NULL; w_fc AND w_proj both in the column order noise_mlp_proj_layout
 * writes (w_fc [2048][512] permuted as 512 rows of 2048); r_fc needs a and b (c_fc's x . b is formed here from
 * the fp32 normalised row). Other arguments as noise_pop_mlp. Fused rounding only. */
int noise_pop_attn_mlp(const noise_population_t *pop, noise_view_t y, const void *w_o, const noise_rank1_t *r_o,
                       const float *o_dots, int64_t o_dots_n, noise_view_t xres, const void *w_fc,
                       const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj, float *xout, int mix,
                       const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x,
                       int64_t eps_stride, noise_view_t x0, void *hout, int split3, const noise_rank1_t *next,
                       int64_t nnext, float *next_dots, noise_stream_t stream);

/* noise_pop_attn_mlp's arithmetic with two waves per SIMD (8 waves of 16 tokens per 128-token tile on
 * v_mfma_f32_16x16x32_bf16): same arguments and results (up to fp32 summation order), with w_fc and w_proj
 * in the column order noise_block_weight_layout writes instead. hout 16 B aligned. No counterpart in the
 * reference beyond the call sites noise_pop_attn_mlp replaces (eggroll.py:92-93). */
int noise_pop_block(const noise_population_t *pop, noise_view_t y, const void *w_o, const noise_rank1_t *r_o,
                    const float *o_dots, int64_t o_dots_n, noise_view_t xres, const void *w_fc, const noise_rank1_t *r_fc,
                    const void *w_proj, const noise_rank1_t *r_proj, float *xout, int mix, const float *lam_r,
                    const float *lam_x, const float *eps_r, const float *eps_x, int64_t eps_stride, noise_view_t x0,
                    void *hout, int split3, const noise_rank1_t *next, int64_t nnext, float *next_dots,
                    noise_stream_t stream);

/* noise_pop_block followed, in the same kernel, by the next block's noise_pop_gate and noise_pop_qkv on
 * h = bf16(norm(xout)) (eggroll.py:92-94, then 81-90 of the next block): h and the next dots never reach HBM.
 * The first 19 arguments as noise_pop_block (xout required; no hout); then noise_pop_qkv's w, r1 (their b rows
 * replace noise_pop_block's next vectors: the dots of every perturbed matrix are formed from the fp32 norm),
 * rotary tables, ve, vocab, idx, idx_sm and ve_noise, with the value-embedding gate's weights gate_w
 * ([8][32] fp32) and noise (noise_pop_gate's gate_noise) in place of precomputed gates. w_qkv in the column
 * order noise_block_weight_layout writes; outputs 16 B aligned. q, k, v as noise_pop_qkv writes them (up to the
 * products' summation order); the gates bit for bit as noise_pop_gate's. No counterpart in the reference beyond
 * the call sites it replaces. */
int noise_pop_block_qkv(const noise_population_t *pop, noise_view_t y, const void *w_o, const noise_rank1_t *r_o,
                        const float *o_dots, int64_t o_dots_n, noise_view_t xres, const void *w_fc,
                        const noise_rank1_t *r_fc, const void *w_proj, const noise_rank1_t *r_proj, float *xout,
                        int mix, const float *lam_r, const float *lam_x, const float *eps_r, const float *eps_x,
                        int64_t eps_stride, noise_view_t x0, const void *const w_qkv[3], const noise_rank1_t r_qkv[3],
                        const void *rope_cos, const void *rope_sin, const float *ve, int64_t vocab,
                        const int64_t *idx, int64_t idx_sm, const float *gate_w, const noise_rank1_t *gate_noise,
                        const noise_rank1_t *ve_noise, void *const out[3], noise_stream_t stream);

/* DUST's jitter on a population block (block_forward, run.py:102-117, for the block a rerun enters at): bf16 rows
 * [members * tokens][2048] added to mlp.c_fc's product before ReLU^2 (fc) and [members * tokens][512] added to
 * mlp.c_proj's product (mlp), either may be NULL (not both); without mlp rows, zero_row is 512 zero bf16 values
 * (16 B aligned) the kernel reads instead. The attention-output and attn.c_proj jitter go in before the call
 * (noise_add_bf16 on y, noise_block_entry's residual). */
typedef struct {
    const void *fc;
    const void *mlp;
    const void *zero_row;
} noise_block_jitter_t;

/* noise_pop_block / noise_pop_block_qkv for an unperturbed block with jitter (no rank-1 or mixing-scalar noise,
 * no next-matrix dots; no counterpart in the reference beyond block_forward's jitter arguments): the last block
 * (mix 0, split3 1: the fp32 head input), or a block followed by the next block's q/k/v (mixing on). */
int noise_pop_block_jit(const noise_population_t *pop, noise_view_t y, const void *w_o, noise_view_t xres,
                        const void *w_fc, const void *w_proj, int mix, const float *lam_r, const float *lam_x,
                        noise_view_t x0, void *hout, int split3, const noise_block_jitter_t *jit,
                        noise_stream_t stream);
int noise_pop_block_qkv_jit(const noise_population_t *pop, noise_view_t y, const void *w_o, noise_view_t xres,
                            const void *w_fc, const void *w_proj, float *xout, const float *lam_r, const float *lam_x,
                            noise_view_t x0, const void *const w_qkv[3], const void *rope_cos, const void *rope_sin,
                            const float *ve, int64_t vocab, const int64_t *idx, int64_t idx_sm, const float *gate_w,
                            void *const out[3], const noise_block_jitter_t *jit, noise_stream_t stream);

/* w [rows][cols] bf16 -> the column order noise_pop_block reads: within every 32 columns, position 8g + j
 * (g < 4) holds column 4g + j for j < 4 and 16 + 4g + (j - 4) for j >= 4. cols a multiple of 32. */
int noise_block_weight_layout(const void *w, void *out, int64_t rows, int64_t cols, noise_stream_t stream);

/* mlp.c_proj [rows][2048] bf16 -> the column order noise_pop_mlp reads: within every 16 columns, the groups of
 * 4 are stored in the order 0, 2, 1, 3 (so each 16-deep slice of the hidden layer pairs with the registers the
 * c_fc product leaves it in). out and w distinct; one pass per weight update. */
int noise_mlp_proj_layout(const void *w, void *out, int64_t rows, noise_stream_t stream);

/* out[m] = mean over tokens of token_loss[m][:] (eggroll.py:102), deterministic order. */
int noise_member_mean(const float *token_loss, int64_t members, int64_t tokens, float *out, noise_stream_t stream);

/* bf16x3 split of fp32 rows of width 512: out[r] = [hi | lo | hi] of (normalize ? norm(x[r]) : x[r]), or
 * [hi | hi | lo] when weight_order (hi = bf16(v), lo = bf16(v - hi)). Feeds the fp32 head of run.py:273-278
 * (TF32 on the reference's H100; split-bf16x3 on gfx950, which has no xf32 MFMA). */
int noise_split3(const float *x, int64_t rows, int64_t width, int normalize, int weight_order, void *out,
                 noise_stream_t stream);

/* lowrank_embed (eggroll.py:61-63): out[m, t, :] = w[idx[t], :] + sign[m] * a[m/dir_div, idx[t]] *
 * b[m/dir_div, :] (r1 NULL or r1->a NULL: plain gather), fp32 [members][tokens][width]. An id outside
 * [0, vocab) reads nothing and gives a NaN row. */
int noise_lowrank_embed(float *out, const float *w, int64_t vocab, int64_t width, const int64_t *idx,
                        const noise_population_t *pop, const noise_rank1_t *r1, noise_stream_t stream);

/* Rank-1 expansion of a product shared by all members (eggroll.py:58 with x broadcast over members):
 * y[m, t, n] = base[t, n] + sign[m] * dots[t * dots_stride + m/dir_div] * a[m/dir_div, n], y bf16
 * (y_fp32 = 0) or fp32 (1; 2: the dot rounded to bf16 first, autocast's form) [m][T][width], base fp32
 * [T][width], width a multiple of 4. With x shared the dot x[t] . b depends on the direction only: dots
 * [T][dots_stride >= directions]. An HBM-write stream: the shared x W^T and x B^T are computed once
 * (noise_pop_linear). */
int noise_rank1_expand(const noise_population_t *pop, const float *base, int64_t width, const float *dots,
                       int64_t dots_stride, const noise_rank1_t *r1, void *y, int y_fp32, noise_stream_t stream);

/* lowrank (eggroll.py:56-58) for any shape, in autocast's form: y[m, t, o] = bf16(x[m, t, :] . w[o, :]) +
 * sign[m] * bf16(x[m, t, :] . bf16(b[m/dir_div, :])) * a[m/dir_div, o], fp32 accumulation, y fp32
 * [members][tokens][n_out]. x bf16 through the strided view (element (m, t, k) at x + m*sm + t*st + k),
 * w bf16 [n_out][n_in]. Serves the call sites whose shapes the MFMA tiles of noise_pop_linear do not take,
 * e.g. the value-embedding gate linear('attn.ve_gate.weight', h[..., :32]) (eggroll.py:88 via :80): w [8, 32]
 * on a 32-wide slice of a 512-wide row. One thread per output element. */
int noise_lowrank_rows(const noise_population_t *pop, noise_view_t x, int64_t n_in, const void *w, int64_t n_out,
                       const noise_rank1_t *r1, float *y, noise_stream_t stream);

/* ---- DUST --------------------------------------------------------------------------------------------- */

/* DUST.head_error (run.py:380-389) over coordinate_differences (run.py:121-137): for each row (token) r and
 * logit j < vocab, out[r][j] = (loss(raw_j + sigma) - loss(raw_j - sigma)) / (2 sigma) with loss the
 * token's soft-capped (15 tanh(v / 15)) cross-entropy against targets[r], in the reference's closed form
 * log1p(softmax(z)_j expm1(z' - z_j)) - [j = target] (z' - z_j); rows with targets[r] < 0 and columns
 * vocab .. out_width are 0. raw: bf16 (raw_bf16) or fp32 [rows][raw_stride]; out fp32 [rows][out_stride]. */
int noise_coordinate_differences(const void *raw, int raw_bf16, int64_t rows, int64_t vocab, int64_t raw_stride,
                                 const int64_t *targets, float sigma, float *out, int64_t out_width,
                                 int64_t out_stride, noise_stream_t stream);

/* direct_errors' draws of one site for a chunk (run.py:344-349), in place and in one pass: a[i][r] *= mask[r] for
 * i < n draws and r < per_draw (mask bf16 0/1 [per_draw], the live units of an mlp.c_fc site, or NULL), and
 * scaled[i][r] = bf16(scale * a[i][r]) (the rerun's jitter sigma * a). bf16, 16 B aligned, per_draw a multiple
 * of 8. */
int noise_mask_scale(void *a, const void *mask, int64_t n, int64_t per_draw, float scale, void *scaled,
                     noise_stream_t stream);

/* DUST.direct_errors' estimate update (run.py:351-355) for one site and chunk of n draws:
 * errors[r][j] += scale * e[r][j], e = einsum('nbt,nbtd->btd', reward.to(bf16), a) with rows r = (b, t):
 * reward fp32 [n][rows], a bf16 [n][rows][d] (the site's draws), fp32 sums rounded to bf16 as the
 * reference's bf16 einsum; errors fp32 [rows][d]; the reference's scale is -1 / sigma. d a multiple of 8. */
int noise_draw_errors(const float *reward, const void *a, int64_t n, int64_t rows, int64_t d, float scale,
                      float *errors, noise_stream_t stream);

/* DUST.rerun's glue between blocks (run.py:262-268) over rows of width 512, fp32:
 *   x0 == NULL: out[r] = norm(x[r mod x_rows] + add[r]) (add bf16 [rows][512] or NULL): the jittered embedding
 *               entry x = x0 = norm(embedding.repeat(n) + jitter) (run.py:262-263);
 *   x0 != NULL: out[r] = rl * x[r mod x_rows] + ml * x0[r mod x0_rows], rl = *lam_r, ml = *lam_x read on the
 *               device: the mixing of the blocks after the entry (run.py:267-268), x0 repeated by indexing. */
int noise_rerun_rows(const float *x, int64_t x_rows, const void *add, const float *x0, int64_t x0_rows,
                     const float *lam_r, const float *lam_x, int64_t rows, float *out, noise_stream_t stream);

/* A jittered block's entry on the population kernels (DUST.rerun, run.py:265 with block_forward's attn jitter,
 * run.py:114): out[r] = x[r mod x_rows] + add[r] (fp32; add bf16 [rows][512] or NULL: the attn.c_proj jitter
 * folded into the residual the block adds its product to) and h[r] = bf16(norm(x[r mod x_rows])), the block's
 * normalised input. */
int noise_block_entry(const float *x, int64_t x_rows, const void *add, int64_t rows, float *out, void *h,
                      noise_stream_t stream);

/* y = bf16(y + add) over n bf16 elements (n a multiple of 8, 16 B aligned): block_forward's attention-output
 * jitter (run.py:114). */
int noise_add_bf16(void *y, const void *add, int64_t n, noise_stream_t stream);

/* DUST.rerun's mixing into a block that runs on the population kernels (run.py:266-268, then the block's
 * norm(x), utils/model.py:117): out[r] = rl * x[r mod x_rows] + ml * x0[r mod x0_rows] (fp32, rl = *lam_r,
 * ml = *lam_x on the device) and h[r] = bf16(norm(out[r])) (bf16 [rows][512]), the block's normalised input. */
int noise_rerun_mix_norm(const float *x, int64_t x_rows, const float *x0, int64_t x0_rows, const float *lam_r,
                         const float *lam_x, int64_t rows, float *out, void *h, noise_stream_t stream);

/* DUST's block_forward (run.py:102-117) over `sequences` rows of `tokens` (a multiple of 256) tokens: the fixed
 * model's block (utils/model.py:103-110) on x fp32 [sequences][tokens][512] -> x_out fp32 (same layout), with
 * the weights unperturbed and optional jitter, bf16 [sequences][tokens][width] or NULL, added where the
 * reference adds it: jit_o to the attention output, jit_attn to attn.c_proj's product, jit_fc to mlp.c_fc's
 * product (before ReLU^2, width 2048), jit_mlp to mlp.c_proj's product. w = {c_q, c_k, c_v (bf16 [512][512]),
 * ve_gate (fp32 [8][32], NULL without value embeddings), c_proj (bf16 [512][512]), c_fc (bf16 [2048][512]),
 * mlp.c_proj (bf16 [512][2048])}; ve: the value embedding rows bf16 [sequences][tokens][512] or NULL;
 * rope_cos / rope_sin: bf16 [tokens][32]; window: the block's attention window. The workspace (256 B
 * aligned) holds the intermediates; its size comes from noise_dust_block_workspace_bytes. */
int64_t noise_dust_block_workspace_bytes(int64_t sequences, int64_t tokens, int with_ve);
int noise_dust_block(const float *x, float *x_out, int64_t sequences, int64_t tokens, const void *const w[7],
                     const void *ve, const void *rope_cos, const void *rope_sin, int64_t window, const void *jit_o,
                     const void *jit_attn, const void *jit_fc, const void *jit_mlp, void *workspace,
                     int64_t workspace_bytes, noise_stream_t stream);

/* noise_dust_block without a workspace argument and without any allocation: the intermediates live in a
 * static device array of the library (64 MiB per GPU, held until the process ends; its size is
 * noise_dust_block_static_max_bytes()). No counterpart in the reference: it is for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. Inputs whose
 * noise_dust_block_workspace_bytes exceed the array are rejected with NOISE_EINVAL (about 4,000 sequence
 * tokens with value embeddings, e.g. 2 sequences of 2048). All calls on one GPU share that GPU's array:
 * calls that overlap on one GPU (other streams, other host threads) race and must be ordered by the caller.
 * Same arguments and results as noise_dust_block otherwise. */
int64_t noise_dust_block_static_max_bytes(void);
int noise_dust_block_static(const float *x, float *x_out, int64_t sequences, int64_t tokens, const void *const w[7],
                            const void *ve, const void *rope_cos, const void *rope_sin, int64_t window,
                            const void *jit_o, const void *jit_attn, const void *jit_fc, const void *jit_mlp,
                            noise_stream_t stream);

/* ---- EGGROLL update reassembly (eggroll.py:151-163) ---------------------------------------------------- */

/* Fitness weights (eggroll.py:151-154): f_i = losses[2i+1] - losses[2i] (i < members/2),
 * z = f / (std(f) + 1e-8) with the unbiased std, weight[d] = sum of z_i over i = d (mod pairs), d < pairs.
 * members even and >= 4. */
int noise_update_weights(const float *losses, int64_t members, int64_t pairs, float *weight, noise_stream_t stream);

/* One parameter of an update: its [pairs] noise offsets (Eggroll.offsets, eggroll.py:117-120) and its
 * gradient, fp32 [rows][cols], or [rows] for a 1-D parameter (cols = 0). */
typedef struct {
    const int64_t *offsets;
    float *grad;
    int64_t rows, cols;
} noise_update_param_t;

/* Bytes of workspace noise_update_gradients needs for these parameters at this chunk of directions: the split-bf16
 * tables, then room for the GEMM's partial tiles on a 256-CU device (a workspace that holds only the tables is
 * accepted: the GEMM then runs whole tiles only, with the same results up to summation order). */
int64_t noise_update_workspace_bytes(const noise_update_param_t *params, int nparams, int64_t pairs,
                                     int64_t chunk);

/* Gradients of eggroll.py:155-163 for up to 64 parameters: grad = scale * sum_{d < pairs} weight[d] a_d b_d^T
 * with a_d = elements [off_d, off_d + rows) and b_d = [off_d + rows, off_d + rows + cols) of the normal draw
 * (seed, offset, threads, numel) — the reference's buffer slices (eggroll.py:126) — and
 * grad = scale * sum_d weight[d] a_d for 1-D parameters. The reference's p.grad is scale = -1/len(fitness).
 * Parameters with both sides multiples of 256 run as split-bf16x3 MFMA GEMMs over chunks of `chunk`
 * directions (rounded up to 256), accumulated in order; others (<= 65536 entries) are summed directly.
 * The matrices' slices are regenerated from the Philox counter in-kernel (through the split tables), or, when
 * `buffer` is non-NULL, read from that materialised draw (fp32 [numel], noise_normal_fill of the same draw):
 * cheaper once pairs * sum(rows + cols) exceeds numel, since every buffer element then serves several
 * directions. With a buffer of at most 2^30 elements the GEMM copies the slices straight from it and splits
 * them itself (the workspace's table area is then unused; the results are the same bits). An element of a
 * slice outside [0, numel) reads as NaN. */
int noise_update_gradients(const noise_update_param_t *params, int nparams, int64_t pairs, const float *weight,
                           float scale, int64_t chunk, int64_t numel, uint64_t seed, uint64_t offset,
                           int64_t threads, const float *buffer, void *workspace, int64_t workspace_bytes,
                           noise_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NOISE_AMD_H */
