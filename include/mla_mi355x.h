/*
 * mla_mi355x.h -- C ABI of the MI355X (gfx950) Multi-Head Latent Attention kernels.
 *
 * Plain C: device pointers, element strides and sizes; no torch or HIP types.
 * Every entry point enqueues work on the HIP stream passed as `stream`
 * (a hipStream_t, or NULL for the null stream), never synchronises the host,
 * never allocates device memory, and returns MLA_OK (0) or a negative
 * MLA_ERR_* code; mla_last_error() then describes the failure (thread-local).
 *
 * Layout conventions (all strides are in ELEMENTS, the innermost dim is contiguous):
 *   q_nope [B, Tq, H, d_nope], q_rope [B, Tq, H, 64]
 *   k_nope [B, Tk, H, d_nope], k_rope [B, Tk, Hr, 64]   (Hr = 1 => head stride 0)
 *   v      [B, Tk, H, d_v],    o      [B, Tq, H, d_v]
 *   lse    [B, H, Tq] fp32 contiguous, natural log
 * Supported: d_nope in {64, 128}, d_rope = 64, d_v = 128; bf16 tensors.
 * A softmax `scale` must be finite and positive (else MLA_ERR_INVALID_ARG): the kernels
 * take a row's reference max before scaling.
 *
 * Each entry point replaces one step of the reference's MLA.forward
 * (manningwu07/transformer, transformer.py) as cited on its declaration.
 */
#ifndef MLA_MI355X_H
#define MLA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLA_OK 0
#define MLA_ERR_INVALID_ARG (-1)  /* null pointer, bad shape, stride or alignment */
#define MLA_ERR_UNSUPPORTED (-2)  /* head dims / dtype outside the built set      */
#define MLA_ERR_WORKSPACE (-3)    /* workspace missing or too small               */
#define MLA_ERR_LAUNCH (-4)       /* the HIP runtime rejected a launch            */

#define MLA_DTYPE_BF16 0
#define MLA_DTYPE_F32 1

#define MLA_ABI_VERSION 3

/* strides (elements) of a [B, T, heads, dim] tensor with unit innermost stride */
typedef struct {
  int64_t b, t, h;
} mla_strides;

/* ------------------------------------------------------------------ RoPE --
 * Decoupled RoPE on the 64-wide rope slice of `n_heads` head vectors per token,
 * in one pass over all heads (the q heads and the k heads of the qk_rope GEMM
 * output [B, T, H + Hr, 64] are rotated together):
 *   y[i]    = x[i] c - x[i+32] s,   y[i+32] = x[i] s + x[i+32] c,
 *   (c, s)  = (cos[p][i], sin[p][i]),  p = pos_offset + t.
 * `inverse` != 0 rotates by -angle (the backward: dx = R^T dy).
 * cos/sin: bf16 [table_rows, 32] contiguous (the module's bf16 tables).
 * x and y may alias exactly (in place).  dtype: MLA_DTYPE_BF16 or MLA_DTYPE_F32.
 *
 * Replaces: RotaryEmbedding.forward + apply_rope on q_pos and k_pos_new
 *           (transformer.py:46-60, applied at :228-239).
 */
typedef struct {
  const void* x;
  void* y;
  const void* cos;
  const void* sin;
  int64_t B, T, n_heads, table_rows, pos_offset;
  mla_strides x_stride, y_stride;
  int32_t dtype, inverse;
} mla_rope_args;
int mla_rope(const mla_rope_args* a, void* stream);

/* RoPE with the KV-cache append in the same pass (a decode step, or any T new tokens):
 *   q heads 0 .. H-1 of qk     -> q_out[b][t][h]           (rotated)
 *   k heads H .. H+Hr-1 of qk  -> k_cache[b][hr][p][:]     (rotated: the cache holds post-RoPE k)
 *   c_new[b][t]                -> latent[b][p][:]          (copied)
 *   seq_lens[b] = pos + T for every b (int32; skipped when NULL)
 *   *pos_next   = pos + T (int64; skipped when NULL; must not be pos_dev)
 * with p = pos + t and pos = pos_offset + (pos_dev ? *pos_dev : 0).  pos_dev is read on the
 * device, so a recorded HIP graph can replay the step while the position advances.  Rows
 * with p >= min(table_rows, capacity) (or p < 0) are not written: a device position past
 * the end is skipped, never written out of bounds.  All tensors bf16, 16-byte aligned,
 * strides multiples of 8 elements; d_latent a multiple of 8.
 *
 * Replaces: apply_rope of q_pos / k_pos_new (transformer.py:228-239) and the cache appends
 *           torch.cat([latent, kv_latent_new]) / torch.cat([k_rope, k_pos_new])
 *           (transformer.py:215-218, :241-244), writing only the new tokens.
 */
typedef struct {
  const void* qk;
  void* q_out;
  const void* c_new;
  void* latent;
  void* k_cache;
  const void* cos;
  const void* sin;
  const int64_t* pos_dev;
  int32_t* seq_lens;
  int64_t* pos_next;
  int64_t B, T, H, Hr, d_latent, capacity, table_rows, pos_offset;
  mla_strides qk_stride, q_stride;
  int64_t c_new_sb, c_new_st, latent_sb, latent_st, k_cache_sb, k_cache_sh, k_cache_st;
} mla_rope_append_args;
int mla_rope_append(const mla_rope_append_args* a, void* stream);

/* ---------------------------------------------------------- prefill fwd --
 * Causal flash attention over the decoupled-RoPE Q/K (nope ++ rope, rope last):
 *   O = softmax((q_nope k_nope^T + q_rope k_rope^T) * scale + M) V,
 *   M masks key j for query i when causal and j > i + q_offset.
 * Writes O (bf16) and the natural-log row LSE (fp32, [B, H, Tq] contiguous).
 *
 * Replaces: F.scaled_dot_product_attention(cat[q_content,q_pos], cat[k_content,k_pos],
 *           v, is_causal=True) (transformer.py:311-314), and the absorbed branch for
 *           T > 1 with its bottom-right mask triu(diagonal=pos_offset+1)
 *           (transformer.py:249-291) via q_offset = pos_offset.
 */
typedef struct {
  const void *q_nope, *q_rope, *k_nope, *k_rope, *v;
  void* o;
  float* lse;
  int64_t B, H, Tq, Tk, d_nope, d_rope, d_v;
  mla_strides q_nope_stride, q_rope_stride, k_nope_stride, k_rope_stride, v_stride, o_stride;
  float scale;
  int32_t causal;
  int64_t q_offset;
  void* workspace;        /* key-split partials; may be NULL (then the unsplit kernel runs) */
  size_t workspace_bytes;
  /* RoPE folded into the Q load (no counterpart field in the reference, which rotates before the
   * attention call, transformer.py:228-239): with rope_cos / rope_sin (bf16 [rope_rows, 32]
   * tables) set, q_rope is the unrotated slice and query row t is rotated at position
   * q_pos_offset + t as the reference's apply_rope (transformer.py:55-60) before use; the rotated
   * slice is also written to q_rope_out when that is non-NULL (what a backward needs).  NULL
   * tables: q_rope is already rotated. */
  const void *rope_cos, *rope_sin;
  int64_t rope_rows, q_pos_offset;
  void* q_rope_out;
  mla_strides q_rope_out_stride;
} mla_prefill_fwd_args;
/* Bytes of 256-byte aligned device memory for `workspace`; 0 when the shape fills the chip
 * without a key split.  When the mirrored q-tile pairs (B * H * ceil(ceil(Tq / 128) / 2)) give
 * at most 128 workgroups, each pair's key tiles are cut into up to 8 segments; a q-tile whose keys
 * span several segments leaves per-segment partials (fp32 O, log2 LSE) here and a second kernel
 * on the same stream merges them in segment order (deterministic).  With a NULL or smaller
 * workspace the call runs unsplit, with the same results up to rounding. */
size_t mla_prefill_fwd_workspace_bytes(const mla_prefill_fwd_args* a);
int mla_prefill_fwd(const mla_prefill_fwd_args* a, void* stream);

/* ---------------------------------------------------------- prefill bwd --
 * Gradients of mla_prefill_fwd given dO, the forward's O and LSE:
 *   dV = P^T dO,  dS = P o (dO V^T - rowsum(dO o O)),
 *   dQ = dS K scale,  dK = dS^T Q scale, split back into nope/rope parts.
 * For a shared k_rope head (k_rope_stride.h == 0) dk_rope is the sum over the H
 * query heads, reduced in a fixed order (deterministic).
 * Outputs are bf16 with the given strides; dk_rope [B, Tk, Hr, 64].
 * Needs `workspace` of mla_prefill_bwd_workspace_bytes(a) bytes (device memory).
 * That size includes room for the dS blocks (2 KiB per visible 32 x 32 block of every (b, h), offered
 * while at most 8 GiB): dQ is then formed from the dS the dK/dV pass stores.  A workspace of
 * only mla_prefill_bwd_workspace_min_bytes(a) bytes makes the dQ pass recompute S and dP
 * instead; both give the same gradients within bf16 rounding.
 *
 * Replaces: the autograd backward of SDPA at transformer.py:314 (run under
 *           ckpt.checkpoint recompute at :330-335, :470-471).
 */
typedef struct {
  const void *dout, *q_nope, *q_rope, *k_nope, *k_rope, *v, *o;
  const float* lse;
  void *dq_nope, *dq_rope, *dk_nope, *dk_rope, *dv;
  void* workspace;
  size_t workspace_bytes;
  int64_t B, H, Tq, Tk, d_nope, d_rope, d_v;
  mla_strides dout_stride, q_nope_stride, q_rope_stride, k_nope_stride, k_rope_stride, v_stride, o_stride;
  mla_strides dq_nope_stride, dq_rope_stride, dk_nope_stride, dk_rope_stride, dv_stride;
  float scale;
  int32_t causal;
  int64_t q_offset;
  /* The forward's RoPE fold, undone in the dQ epilogue: with rope_cos / rope_sin (bf16
   * [rope_rows, 32] tables) set, q_rope is the rotated slice the forward stored (q_rope_out) and
   * dq_rope is returned for the unrotated slice: rotated by the opposite angle at position
   * q_pos_offset + t before its one rounding (the gradient of transformer.py:55-60, which the
   * reference leaves to autograd).  NULL tables: dq_rope is for the rotated slice. */
  const void *rope_cos, *rope_sin;
  int64_t rope_rows, q_pos_offset;
} mla_prefill_bwd_args;
size_t mla_prefill_bwd_workspace_bytes(const mla_prefill_bwd_args* a);
/* The smaller workspace of the recompute path (no counterpart in the reference: it lets a
 * caller short of memory trade the stored dS for a recomputation of S and dP). */
size_t mla_prefill_bwd_workspace_min_bytes(const mla_prefill_bwd_args* a);
int mla_prefill_bwd(const mla_prefill_bwd_args* a, void* stream);

/* --------------------------------------------------------------- decode --
 * Absorbed latent-KV attention for one query token per sequence, reading the
 * compressed cache once for all heads (split-K over the context + ordered LSE merge):
 *   s_j   = (q_lat . c_kv[j] + q_rope . k_rope[j]) * scale,   j < seq_len
 *   ctx   = softmax(s) c_kv,   lse = logsumexp(s)
 *   q_lat  [B, H, d_latent]  (q_nope absorbed through W_UK)   strides (b, h)
 *   q_rope [B, H, 64]                                        strides (b, h)
 *   c_kv   [B, L, d_latent]                                  strides (b, t)
 *   k_rope [B, Hr, L, 64]  (Hr = 1: h stride 0)               strides (b, h, t)
 *   ctx    [B, H, d_latent] bf16                             strides (b, h)
 *   lse    [B, H] fp32 contiguous
 * seq_lens: optional int32 [B] device array of valid lengths (NULL: all L);
 * a length of 0 yields ctx = 0, lse = -inf.  With seq_lens, each sequence's own
 * length is divided over the splits on the device, so a cache of capacity L far above the
 * lengths costs no idle splits (the call can be captured in a graph and replayed as
 * the lengths grow).  num_splits <= 0 picks a split count
 * (one workgroup per CU); with more than one split the partials (bf16 with fp32
 * log-sum-exp, in the workspace) are merged in split order by a second kernel on the same stream, so the
 * result is deterministic and does not depend on the split count beyond rounding (more than 32
 * splits are merged 8 at a time by parallel thread groups whose sums are then added in group
 * order).
 * d_latent in {64, 128, 256, 384, 512}.  Needs mla_decode_workspace_bytes() bytes of
 * 256-byte aligned device memory (0 when a single split is chosen); its contents on
 * entry do not matter.
 *
 * Replaces: the absorbed inference branch for T == 1 (transformer.py:249-286:
 *           scores :259-269, softmax :283, P . latent :286).
 */
typedef struct {
  const void *q_lat, *q_rope, *c_kv, *k_rope;
  const int32_t* seq_lens;
  void* ctx;
  float* lse;
  void* workspace;
  size_t workspace_bytes;
  int64_t B, H, L, d_latent, d_rope, n_k_rope_heads;
  int64_t q_lat_sb, q_lat_sh, q_rope_sb, q_rope_sh;
  int64_t c_kv_sb, c_kv_st;
  int64_t k_rope_sb, k_rope_sh, k_rope_st;
  int64_t ctx_sb, ctx_sh;
  float scale;
  int32_t num_splits;
} mla_decode_args;
size_t mla_decode_workspace_bytes(const mla_decode_args* a);
int mla_decode(const mla_decode_args* a, void* stream);

/* mla_decode without a workspace: allocates nothing and ignores a->workspace and
 * a->workspace_bytes.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * The split partials live in a static device array of MLA_DECODE_STATIC_SCRATCH_BYTES on
 * each GPU, held until the process ends; a call whose mla_decode_workspace_bytes(a) exceeds
 * it returns MLA_ERR_WORKSPACE (any automatic split count at d_latent <= 512 fits).  The
 * stream must belong to the current device.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (on different streams, or from different threads) race.
 * Results are those of mla_decode with the same arguments. */
#define MLA_DECODE_STATIC_SCRATCH_BYTES ((size_t)12 << 20)
int mla_decode_static(const mla_decode_args* a, void* stream);

/* W_UK absorption of the decode queries:
 *   q_lat[b][h][c] = sum_d q_nope[b][h][d] W_UK[h][d][c],   W_UK[h] = w_uk + h * w_uk_sh, [d_nope, d_latent]
 * with rows of d_latent contiguous at row stride w_uk_sd (k_up.weight [H * d_nope, d_latent]
 * viewed per head: w_uk_sh = d_nope * d_latent, w_uk_sd = d_latent).  q_nope [B, H, d_nope]
 * (strides q_sb, q_sh: q_up's output rows read in place), q_lat bf16 [B, H, d_latent]
 * (strides out_sb, out_sh); fp32 accumulation, one rounding.  d_nope a multiple of 32 up to 256,
 * d_latent a multiple of 8 up to 512.
 *
 * Replaces: q_latent = q_nope . W_UK (transformer.py:252-254) for the decode step.
 */
typedef struct {
  const void* q_nope;
  const void* w_uk;
  void* q_lat;
  int64_t B, H, d_nope, d_latent;
  int64_t q_sb, q_sh, w_uk_sh, w_uk_sd, out_sb, out_sh;
} mla_absorb_q_args;
int mla_absorb_q(const mla_absorb_q_args* a, void* stream);

/* Absorbed decode with the W_UV product in the split merge:
 *   out[b][h][:] = bf16(ctx[b][h][:]) . W_UV[h]^T,   W_UV[h] = w_uv + h * w_uv_sh, [d_v, d_latent]
 * with rows of d_latent contiguous at row stride w_uv_sd (v_up.weight [H * d_v, d_latent]
 * viewed per head: w_uv_sh = d_v * d_latent, w_uv_sd = d_latent).  out: bf16 [B, H, d_v] with
 * strides (out_sb, out_sh) -- [B, H * d_v] contiguous is the layout o_proj reads.  ctx is
 * the same as mla_decode's (bf16-rounded); dec.ctx may be NULL (then ctx is not written, and
 * with one split or more than 32 a ctx scratch sits in the workspace, past the partials).
 * Needs mla_decode_out_workspace_bytes(a) bytes of 256-byte aligned device memory.
 * d_v = 128.
 *
 * Replaces: transformer.py:286-291 (P . latent, then the per-head W_UV product) for T == 1,
 *           fusing the up-projection of ctx into the merge of the context splits.
 */
typedef struct {
  mla_decode_args dec;
  const void* w_uv;
  void* out;
  int64_t w_uv_sh, w_uv_sd;
  int64_t out_sb, out_sh;
  int64_t d_v;
} mla_decode_out_args;
size_t mla_decode_out_workspace_bytes(const mla_decode_out_args* a);
int mla_decode_out(const mla_decode_out_args* a, void* stream);

/* ------------------------------------------------- prefill with a cache --
 * Absorbed attention of a chunk of T query tokens per sequence over a cache that already
 * holds the chunk's own keys (positions L0 .. L0 + T - 1 written before the call):
 *   s[b][t][h][j] = (q_lat[b][t][h] . c_kv[b][j] + q_rope[b][t][h] . k_rope[b][j]) * scale,
 *                   j <= L0 + t (query t of the chunk sits at position L0 + t)
 *   ctx[b][t][h]  = bf16(softmax_j(s) . c_kv[b]),   lse[b][h][t] = logsumexp_j(s)  (natural log)
 * q_lat [B, T, H, d_latent], q_rope [B, T, H, 64] (strides q_lat_stride, q_rope_stride);
 * c_kv [B, L, d_latent] (strides c_kv_sb, c_kv_st), k_rope shared by the heads [B, L, 64]
 * (k_rope_sb, k_rope_st); ctx bf16 [B, T, H, d_latent] (ctx_stride), lse fp32 [B, H, T]
 * contiguous or NULL.  L (the rows the cache holds) >= L0 + T.  d_latent in {128, 256, 384,
 * 512}, d_rope = 64; inputs 16-byte aligned with strides multiples of 8, ctx 8-byte aligned
 * with strides multiples of 4.  One workgroup per (sequence, 16 heads, block of queries, key
 * range).  With num_splits S > 1 (0: chosen automatically, so that small batches fill the
 * chip) the keys are cut into S ranges whose fp32 partials go to `workspace`
 * (mla_prefill_cached_workspace_bytes() bytes, 256-byte aligned, 0 when one range is chosen)
 * and a second kernel on the same stream merges them in range order: deterministic, and
 * independent of S beyond rounding.  A cache with per-head k_rope goes through the expanded
 * path (up-projected K and V into mla_prefill_fwd with q_offset = L0).
 *
 * Replaces: the absorbed inference branch for T > 1 over a cache (transformer.py:247-291:
 *           q_latent :254 is the caller's, scores :259-269, the causal mask with
 *           diagonal = pos_offset + 1 :273-281, softmax :283, attn . latent :286; W_UV :291
 *           is the caller's).
 */
typedef struct {
  const void *q_lat, *q_rope, *c_kv, *k_rope;
  void* ctx;
  float* lse;
  void* workspace;
  size_t workspace_bytes;
  int64_t B, T, H, L, L0, d_latent, d_rope;
  mla_strides q_lat_stride, q_rope_stride, ctx_stride;
  int64_t c_kv_sb, c_kv_st, k_rope_sb, k_rope_st;
  float scale;
  int32_t num_splits;
} mla_prefill_cached_args;
size_t mla_prefill_cached_workspace_bytes(const mla_prefill_cached_args* a);
int mla_prefill_cached(const mla_prefill_cached_args* a, void* stream);

/* ---------------------------------------------------------- decode rows --
 * Products of a few rows (one token of each sequence) with a weight matrix, in G groups:
 *   y[g][m][n] = sum_k x[g][m][k] W[g][n][k]      (fp32 accumulation, one rounding to bf16)
 * x[g][m][k] at x + g x_sg + m x_sm + k; W[g][n][k] at w + g w_sg + n w_sn + k (an nn.Linear
 * weight [N, K], or per-head slices of one); y[g][m][n] at y + g y_sg + m y_sm + n.  bf16;
 * x and w 16-byte aligned with strides multiples of 8; y 8-byte aligned with strides multiples
 * of 4; K a multiple of 128 up to 4096, N a multiple of 4.  Built for M <= 64 (larger M runs in passes of 64
 * rows); deterministic.
 *
 * Replaces, for the decode step (T == 1, 32 sequences at the benchmark dims: d_model 2048, 16 heads): q_down / qk_rope /
 *           kv_down (transformer.py:208-213, as one product over the concatenated weights),
 *           q_up (:208), the W_UK absorption q_latent = q_nope . W_UK (:252-254, G = H heads
 *           against W_UK transposed per head) and o_proj (:300).
 */
typedef struct {
  const void* x;
  const void* w;
  void* y;
  int64_t M, N, K, G;
  int64_t x_sm, x_sg, w_sn, w_sg, y_sm, y_sg;
} mla_linear_rows_args;
int mla_linear_rows(const mla_linear_rows_args* a, void* stream);

/* mla_linear_rows and mla_rope_append in one launch, with the arguments and results of each:
 * the decode step's q_up product (transformer.py:208) beside the RoPE of the new token's q and k
 * heads with the cache append (:215-218, :228-244), both reading only the down-projections'
 * output.  Each part's arithmetic is its own entry point's (bit for bit).  The product's y must
 * not overlap what the append reads or writes, nor the append's outputs the product's x or w.
 *
 * Replaces: transformer.py:208 and :215-244 for T == 1, as the pair of entry points above does;
 *           it saves the second launch of the step.
 */
int mla_linear_rows_rope_append(const mla_linear_rows_args* rows, const mla_rope_append_args* rope, void* stream);

/* -------------------------------------------------------------- RMSNorm --
 * Row RMSNorm in front of the MLA down-projections (the block's norm1):
 *   r[m]    = 1 / sqrt(sum_k x[m][k]^2 / K + eps)
 *   y[m][k] = (x[m][k] * r[m]) * w[k]           (fp32 arithmetic, one rounding to y_dtype)
 * x: [M, K], row stride x_stride (elements), dtype x_dtype (MLA_DTYPE_BF16 / _F32);
 * w: fp32 [K]; y: [M, K] of y_dtype (MLA_DTYPE_BF16 / _F32), row stride y_stride;
 * inv_rms: fp32 [M] (r), or NULL.
 * K a multiple of 8 and at most 4096; pointers 16-byte aligned; strides multiples of 8.
 * A bf16 y is what the down-projection GEMM reads under autocast (autocast casts the
 * reference's fp32 norm output to bf16 at that point); an fp32 y is the reference's own
 * result for an fp32 module outside autocast.
 *
 * Replaces: RMSNorm.forward (transformer.py:26-27) as norm1 in front of the
 *           down-projections (transformer.py:338 -> :208-213), i.e. the normalisation
 *           phases of fused_rmsnorm_down_kernel (fused_mla_triton_kernels.py:178-213).
 */
typedef struct {
  const void* x;
  const float* w;
  void* y;
  float* inv_rms;
  int64_t M, K, x_stride, y_stride;
  float eps;
  int32_t x_dtype, y_dtype;
} mla_rmsnorm_args;
int mla_rmsnorm(const mla_rmsnorm_args* a, void* stream);

/* Backward of mla_rmsnorm from dy ([M, K] of dy_dtype, row stride dy_stride) and the forward's r:
 *   g = w o dy,   dx = r g - x (r^3 / K) sum_k(g o x),   dw = sum_m dy o (x r)
 * dx: x's dtype, row stride dx_stride; dw: fp32 [K] (overwritten).  dw is summed from
 * per-workgroup partials in a fixed order (deterministic); the partials need
 * mla_rmsnorm_bwd_workspace_bytes(a) bytes of device memory.
 *
 * Replaces: the autograd backward of RMSNorm.forward (transformer.py:26-27).
 */
typedef struct {
  const void* dy;
  const void* x;
  const float* w;
  const float* inv_rms;
  void* dx;
  float* dw;
  void* workspace;
  size_t workspace_bytes;
  int64_t M, K, dy_stride, x_stride, dx_stride;
  int32_t x_dtype, dy_dtype;
} mla_rmsnorm_bwd_args;
size_t mla_rmsnorm_bwd_workspace_bytes(const mla_rmsnorm_bwd_args* a);
int mla_rmsnorm_bwd(const mla_rmsnorm_bwd_args* a, void* stream);

/* RMSNorm fused into the down-projection:
 *   r[m]     = 1 / sqrt(sum_k x[m][k]^2 / K + eps)                     (written to inv_rms)
 *   xn[m][k] = bf16((x[m][k] r[m]) w_norm[k])                           (fp32 arithmetic)
 *   y[m][n]  = bf16(sum_k xn[m][k] W[n][k])                             (fp32 accumulation)
 * W [N, K]: nn.Linear down-projection weights (q_down, qk_rope, kv_down concatenated, or the
 * reference wrapper's w_down [K, N] transposed).  x [M, K] bf16 (row stride x_stride), W bf16
 * (row stride w_stride), w_norm fp32 [K], y [M, N] bf16 (row stride y_stride), inv_rms fp32 [M].
 * A first kernel reads x once for r; the GEMM reads it again and normalises each tile in LDS
 * before its products, so the normalised rows are never stored (the reference's two phases).
 * K a multiple of 32 up to 4096, N a multiple of 4; x, W and w_norm 16-byte aligned with
 * strides multiples of 8, y 8-byte aligned with a stride multiple of 4.  Deterministic.
 *
 * Replaces: RMSNorm.forward (transformer.py:26-27) as norm1 (:338) feeding q_down / qk_rope /
 *           kv_down (:208-213), i.e. fused_rmsnorm_down_kernel (fused_mla_triton_kernels.py:
 *           105-230) and its wrapper (:233-274).
 */
typedef struct {
  const void* x;
  const void* w;
  const float* w_norm;
  void* y;
  float* inv_rms;
  int64_t M, N, K, x_stride, w_stride, y_stride;
  float eps;
} mla_norm_linear_args;
int mla_norm_linear(const mla_norm_linear_args* a, void* stream);

/* ---------------------------------------------------- chunked linear CE --
 * One vocabulary chunk of the exact softmax cross-entropy over tied output weights, given
 * that chunk's logits [N, Vc] (row stride ld) = x . W[v0 : v0 + Vc]^T of `dtype`
 * (MLA_DTYPE_BF16 under autocast, MLA_DTYPE_F32 for an fp32 caller outside it):
 *   forward  (backward == 0):
 *     lse[n]    = logaddexp(lse[n], logsumexp_j logits[n][j])    fp32, in/out (start at -inf)
 *     tlogit[n] = logits[n][y_n - v0]   if v0 <= y_n < v0 + Vc   fp32, in/out (start at 0)
 *   backward (backward != 0), with the final lse:
 *     dlogits[n][j] = g_n (exp(logits[n][j] - lse[n]) - [y_n == v0 + j])   `dtype`, row stride ld_out
 *     g_n = g_scale * (g_vec ? g_vec[n] : 1); dlogits may alias logits exactly.
 * targets: int64 [N].  Vc and the row strides multiples of 8; pointers 16-byte aligned.
 * The loss is lse - tlogit per row.
 *
 * Replaces: the per-chunk body of chunked_linear_cross_entropy (transformer.py:91-108:
 *           logits.float(), logsumexp, logaddexp, the in-chunk target gather) and, for the
 *           backward, autograd through it.
 */
typedef struct {
  const void* logits;
  void* dlogits;
  const int64_t* targets;
  float* lse;
  float* tlogit;
  const float* g_vec;
  float g_scale;
  int32_t backward;
  int64_t N, Vc, v0, ld, ld_out;
  int32_t dtype;
} mla_ce_chunk_args;
int mla_ce_chunk(const mla_ce_chunk_args* a, void* stream);

/* --------------------------------------------------------------- misc --
 * mla_last_error: description of the last non-zero return on this thread.
 * mla_abi_version: MLA_ABI_VERSION of the built library.
 * mla_args_size: sizeof() of the argument structs, for binding checks
 *   (0 rope, 1 prefill_fwd, 2 prefill_bwd, 3 decode, 4 rmsnorm, 5 rmsnorm_bwd, 6 decode_out,
 *    7 rope_append, 8 absorb_q, 9 ce_chunk, 10 linear_rows, 11 prefill_cached, 12 norm_linear).
 */
const char* mla_last_error(void);
int mla_abi_version(void);
size_t mla_args_size(int which);

#ifdef __cplusplus
}
#endif
#endif /* MLA_MI355X_H */
