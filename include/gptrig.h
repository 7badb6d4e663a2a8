/*
 * gptrig: C ABI of the MI355X (gfx950) training-step hot path of the GPT
 * speedrun rig (honglu2875/GPT-speedrun-TPU).
 *
 * Conventions (every entry point):
 *   - returns GPTRIG_OK (0) or a negative GPTRIG_E_* status; nothing throws;
 *   - validation happens on the host before any launch (bad shape, null
 *     pointer, unsupported head_dim ...), mirroring the reference's
 *     ValueError/TypeError-before-compilation contract;
 *   - the caller owns every buffer (inputs, outputs, workspace); nothing here
 *     allocates, frees or synchronises the host;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = the null stream);
 *   - "bf16" buffers hold bfloat16, "f32" float32, "i32" int32.
 *
 * Each entry point maps 1:1 onto an XLA-FFI custom-call handler (buffers,
 * stream, scalar attributes) or a ctypes call from a torch front end.
 */
#ifndef GPTRIG_H_
#define GPTRIG_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPTRIG_OK 0
#define GPTRIG_E_NULL (-1)        /* a required pointer is NULL */
#define GPTRIG_E_SHAPE (-2)       /* sizes/strides violate the contract */
#define GPTRIG_E_DTYPE (-3)       /* unsupported element type */
#define GPTRIG_E_UNSUPPORTED (-4) /* legal but not implemented (e.g. head_dim) */
#define GPTRIG_E_LAUNCH (-5)      /* the HIP launch failed */
#define GPTRIG_E_WORKSPACE (-6)   /* workspace smaller than the query says */

/* Library identity and status text. */
const char* gptrig_version(void);
const char* gptrig_status_string(int status);

/* ------------------------------------------------------------------------
 * Causal flash attention.
 * Replaces the Pallas kernels of rig/kernels/tpu_flash_attention.py:
 *   forward  _tpu_flash_forward            (:351-476, kernel :236-348)
 *   backward _tpu_flash_backward           (:704-904, kernels :479-701)
 * Tensors are logical BHSD [batch, heads, seq, head_dim] bf16 with head_dim
 * contiguous.  `strides` (nullable) gives element strides (batch, head, seq)
 * per tensor, 3 int64 each, in the order the tensors appear in the argument
 * list; NULL means contiguous BHSD for all.  head_dim in {64, 128}; any
 * seq >= 1 (keys at or past `seq` never exist, so right-padding is implicit).
 * segment_ids (nullable) is i32 [batch, seq]: positions attend only within
 * their own id (document masking, :312-318).  lse is f32 [batch, heads, seq],
 * natural log: log(sum_j exp(scale*q.k_j)).
 * ---------------------------------------------------------------------- */
int gptrig_attn_fwd(const void* q, const void* k, const void* v, const int32_t* segment_ids, void* o, float* lse,
                    int batch, int heads, int seq, int head_dim, const int64_t* strides /* q,k,v,o */,
                    float softmax_scale, void* stream);

/* Workspace of gptrig_attn_bwd: Delta (f32 [B,H,S]) and the f32 dQ accumulator. */
size_t gptrig_attn_bwd_workspace_bytes(int batch, int heads, int seq, int head_dim);

/* dQ, dK, dV (bf16) from q, k, v, o, dO (bf16) and the forward's lse. */
int gptrig_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                    const int32_t* segment_ids, void* dq, void* dk, void* dv, void* workspace,
                    size_t workspace_bytes, int batch, int heads, int seq, int head_dim,
                    const int64_t* strides /* q,k,v,o,dout,dq,dk,dv */, float softmax_scale, void* stream);

/* The same backward followed by the VJP of the RoPE the block applies to q and
 * k before attention (recipes/reference/train.py:1141-1142, apply_rotary =
 * rig/nn.py:36-52): q and k are the rotated tensors the forward saw; dq and dk
 * come back as the cotangents of the unrotated ones, each first rounded to
 * bf16 and then rotated by -angle, as gptrig_rope_bwd would do in a second
 * pass.  rope_cos / rope_sin: the bf16 [seq, head_dim/2] tables of
 * gptrig_rope_table, 8-byte aligned. */
int gptrig_attn_bwd_rope(const void* q, const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, const int32_t* segment_ids, void* dq, void* dk, void* dv, void* workspace,
                         size_t workspace_bytes, int batch, int heads, int seq, int head_dim,
                         const int64_t* strides /* q,k,v,o,dout,dq,dk,dv */, float softmax_scale,
                         const void* rope_cos, const void* rope_sin, void* stream);

/* ------------------------------------------------------------------------
 * Fused linear cross-entropy (LM head + online log-sum-exp + loss + dh/dW).
 * Replaces rig/kernels/linear_cross_entropy.py:
 *   forward  _losses_and_residual   (:115-179)
 *   backward _tiled_losses_bwd      (:220-302)
 * hidden bf16 [n, d] (d % 64 == 0), weight bf16 [vocab, d] (the compute-dtype
 * copy of the embedding), targets i32 [n].  Rows at or past `semantic_vocab`
 * get no probability mass and exactly zero weight gradient; a target outside
 * [0, semantic_vocab) gives loss +inf and contributes no gradient.
 * ---------------------------------------------------------------------- */
size_t gptrig_flce_fwd_workspace_bytes(int n, int d, int vocab);
int gptrig_flce_fwd(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                    void* workspace, size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab,
                    void* stream);

/* The forward with no workspace argument and no allocation.  It has no
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Its scratch is a fixed file-scope device array of
 * GPTRIG_FLCE_FWD_NOALLOC_SCRATCH_BYTES (32 MiB) per GPU, held until the
 * process ends: sizes whose gptrig_flce_fwd_workspace_bytes exceed it return
 * GPTRIG_E_WORKSPACE (e.g. up to 16384 tokens at vocab 50304).  The first call
 * on a device looks up that device's copy (with the device current).  Every
 * call on one GPU shares the array: calls that overlap on one GPU (different
 * streams, or host threads) race; calls in one stream are ordered.  Results
 * equal gptrig_flce_fwd's on the same inputs. */
#define GPTRIG_FLCE_FWD_NOALLOC_SCRATCH_BYTES (32u << 20)
int gptrig_flce_fwd_noalloc(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                            int n, int d, int vocab, int semantic_vocab, void* stream);

/* Backward.  cotangent: f32 [n] per-token loss cotangents, or NULL to use the
 * scalar `cotangent_scale` for every token (1/n for the mean loss).
 * dhidden: bf16 [n, d].  dweight: f32 [vocab, d]; accumulate_dweight != 0 adds
 * into it (micro-batch accumulation), otherwise it is overwritten.
 * vocab_chunk (a multiple of 256; 0 = 2048, the reference's default
 * vocab_tile_size) is the vocabulary chunk whose logits are recomputed at a
 * time: the workspace holds one bf16 [n, vocab_chunk] logit gradient, the f32
 * [n, d] dh accumulator of the reference's loop (:247) and, with more than one
 * chunk, a few KB of work-queue counters.  Several chunks run as pipelined
 * launches (each recomputes one half of the buffer while the dW / dh products
 * read the other); a chunk covering the whole vocabulary (vocab_chunk >=
 * vocab) runs as three launches with no accumulator passes. */
size_t gptrig_flce_bwd_workspace_bytes(int n, int d, int vocab, int vocab_chunk);
int gptrig_flce_bwd(const void* hidden, const void* weight, const int32_t* targets, const float* lse,
                    const float* cotangent, float cotangent_scale, void* dhidden, float* dweight,
                    int accumulate_dweight, void* workspace, size_t workspace_bytes, int n, int d, int vocab,
                    int semantic_vocab, int vocab_chunk, void* stream);

/* The same forward and backward with float32 compute, the reference's
 * compute_dtype=float32 (rig/kernels/linear_cross_entropy.py:38-41,
 * _tile_logits :92-112): hidden f32 [n, d], weight f32 [vocab, d], every
 * product and sum in float32 (lse and losses as gptrig_flce_fwd); the
 * backward recomputes the logits per chunk of vocab_chunk rows (0: 2048,
 * rounded up to 64) with a float32 [n, chunk] logit-gradient workspace, the
 * reference's [n, vocab_tile_size] bound, and writes dhidden f32 [n, d] and
 * dweight f32 [vocab, d] (+= with accumulate_dweight).  Any n, d. */
size_t gptrig_flce32_fwd_workspace_bytes(int n, int d, int vocab);
int gptrig_flce32_fwd(const float* hidden, const float* weight, const int32_t* targets, float* losses, float* lse,
                      void* workspace, size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab,
                      void* stream);
size_t gptrig_flce32_bwd_workspace_bytes(int n, int d, int vocab, int vocab_chunk);
int gptrig_flce32_bwd(const float* hidden, const float* weight, const int32_t* targets, const float* lse,
                      const float* cotangent, float cotangent_scale, float* dhidden, float* dweight,
                      int accumulate_dweight, void* workspace, size_t workspace_bytes, int n, int d, int vocab,
                      int semantic_vocab, int vocab_chunk, void* stream);

/* Kept-softmax forward and backward: the one-chunk backward without the
 * logits recompute.  The reference's backward recomputes the logits tile by
 * tile from the saved (hidden, weight) (rig/kernels/linear_cross_entropy.py:
 * 220-302); this pair instead keeps the forward's probabilities for the
 * backward, as fp16 exp(logit - m) with m the max over 128 vocabulary rows,
 * plus m: a [vocab, n] 16-bit array, so a caller that can hold it trades
 * the recompute GEMM for two bandwidth passes.  The trainer calls the pair
 * on token chunks sized so the array stays within the reference's fp32
 * [tokens, vocab_tile_size] logits (or on all tokens at once, 6.6 GB at
 * 65536, when asked for the whole vocabulary), accumulating dweight.  Same
 * losses and lse as gptrig_flce_fwd; gradient values as gptrig_flce_bwd's up
 * to one fp16 rounding of each probability before its bf16 rounding.  d a
 * multiple of 128 and n of 8 (else GPTRIG_E_UNSUPPORTED).  keep: gptrig_flce_keep_bytes(n, vocab) bytes, 16-byte
 * aligned, written by the forward and consumed (overwritten) by the backward,
 * which must see the forward's lse.  The backward's workspace is the f32
 * [n, d] dh accumulator. */
size_t gptrig_flce_keep_bytes(int n, int vocab);
int gptrig_flce_fwd_keep(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                         void* keep, size_t keep_bytes, void* workspace, size_t workspace_bytes, int n, int d,
                         int vocab, int semantic_vocab, void* stream);
size_t gptrig_flce_bwd_keep_workspace_bytes(int n, int d);
int gptrig_flce_bwd_keep(const void* hidden, const void* weight, const int32_t* targets, const float* lse,
                         const float* cotangent, float cotangent_scale, void* dhidden, float* dweight,
                         int accumulate_dweight, void* keep, size_t keep_bytes, void* workspace,
                         size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab, void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm, rig/nn.py:26-33 (rms_norm): y = bf16(bf16(x*rsqrt(mean(x^2)+1e-5)) * scale).
 * x, y bf16 [rows, d]; scale bf16 [d]; rstd f32 [rows] (saved for backward).
 * ---------------------------------------------------------------------- */
int gptrig_rmsnorm_fwd(const void* x, const void* scale, void* y, float* rstd, int rows, int d, void* stream);
/* The block's residual add fused with the norm that follows it
 * (recipes/reference/train.py:1164-1169 and :1172-1176: x = residual +
 * s * linear(...), then rms_norm(x)): sum bf16 [rows, d] =
 * bf16(x + bf16(branch * branch_scale)), then y, rstd = gptrig_rmsnorm_fwd(sum).
 * sum may be x (in place); y must not alias x, branch or sum. */
int gptrig_add_rmsnorm_fwd(const void* x, const void* branch, float branch_scale, const void* scale, void* sum,
                           void* y, float* rstd, int rows, int d, void* stream);
/* The same with the bias add of the linear that produced branch done here:
 * rig/nn.py:55-56 rounds the GEMM output to bf16 and then adds
 * b.astype(bf16) with a second rounding, so branch (the bf16 GEMM output
 * without bias) becomes bf16(branch + branch_bias[column]) before the
 * residual add.  branch_bias bf16 [d] (8-byte aligned), or NULL for none. */
int gptrig_add_bias_rmsnorm_fwd(const void* x, const void* branch, const void* branch_bias, float branch_scale,
                                const void* scale, void* sum, void* y, float* rstd, int rows, int d, void* stream);
size_t gptrig_rmsnorm_bwd_workspace_bytes(int rows, int d);
/* dx bf16 = d rms_norm/dx (+ dresidual if non-NULL); dscale f32 [d] (+= if accumulate). */
int gptrig_rmsnorm_bwd(const void* dy, const void* x, const void* scale, const float* rstd, const void* dresidual,
                       void* dx, float* dscale, int accumulate_dscale, void* workspace, size_t workspace_bytes,
                       int rows, int d, void* stream);

/* Weight and bias gradients of rig/nn.py:55-56 (linear, y = x W + b):
 * dw f32 [rows_in, cols_out] += x^T dy for x bf16 [n, rows_in], dy bf16
 * [n, cols_out] (rows_in, cols_out multiples of 8), and, when db is not NULL,
 * db f32 [cols_out] += column sums of dy in the same pass.  Accumulates with
 * fp32 atomics. */
int gptrig_weight_grad(const void* x, const void* dy, float* dw, float* db, int n, int rows_in, int cols_out,
                       void* stream);

/* Bias gradient of rig/nn.py:55-56 (linear): db f32 [cols] += sum over rows of
 * dy bf16 [rows, cols] (cols % 8 == 0). */
int gptrig_bias_grad(const void* dy, int rows, int cols, float* db, void* stream);

/* Dense linear layer, rig/nn.py:55-56 (linear(x, w, b) = bf16(x w) + b):
 * y bf16 [n, f] (row stride ldy) = bf16(bf16(x w) + bias) for x bf16 [n, k]
 * (row stride ldx) and bias bf16 [f] (NULL: no bias, y = bf16(x w)).  The
 * weight is w [k, f] (w_kmajor = 0, the reference's layout, row stride ldw)
 * or its transpose [f, k] (w_kmajor = 1), which the kernel reads faster; an
 * input gradient dx = dy w^T is gptrig_linear(dy, w as [f = d_in, k = d_out],
 * w_kmajor = 1, bias NULL).  k, f, ldx, ldw, ldy multiples of 8; x, w and y
 * 16-byte aligned. */
int gptrig_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias, void* y,
                  int64_t ldy, int n, int k, int f, void* stream);
/* The MLP up-projection and its GELU (recipes/reference/train.py:1170-1171):
 * h = linear(x, w, b) as gptrig_linear, g = bf16(gelu_tanh(h)), both [n, f]
 * with row stride ldy (h is kept for the backward). */
int gptrig_linear_gelu(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias,
                       void* h, void* g, int64_t ldy, int n, int k, int f, void* stream);
/* The QKV projection and the RoPE of q and k (recipes/reference/train.py:
 * 1136-1142, rig/nn.py:36-52): y = linear(x, w, b) as gptrig_linear, then
 * columns [0, rope_cols) rotated as gptrig_rope_fwd does (head_dim-wide
 * groups, position = row % seq, tables from gptrig_rope_table; head_dim % 8
 * == 0, rope_cols a multiple of head_dim). */
int gptrig_linear_rope(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias,
                       void* y, int64_t ldy, int n, int k, int f, const void* cos_table, const void* sin_table,
                       int seq, int rope_cols, int head_dim, void* stream);
/* Input gradient of the down-projection times the GELU VJP (the backward of
 * recipes/reference/train.py:1171-1173): dx bf16 [n, f] = bf16(bf16(dy w^T) *
 * gelu_tanh'(h)), dy bf16 [n, k], w as in gptrig_linear ([f, k] with
 * w_kmajor = 1 is the reference's [d_in, d_out] weight), h bf16 [n, f] the
 * saved pre-activation (row stride ldh, a multiple of 8, h 16-byte aligned);
 * equal to gptrig_linear then gptrig_gelu_bwd on the same GEMM output. */
int gptrig_linear_dgelu(const void* dy, int64_t lddy, const void* w, int64_t ldw, int w_kmajor, const void* h,
                        int64_t ldh, void* dx, int64_t lddx, int n, int k, int f, void* stream);

/* GELU, tanh approximation: jax.nn.gelu(approximate=True) at
 * recipes/reference/train.py:1171.  bf16 [n]. */
int gptrig_gelu_fwd(const void* x, void* y, int64_t n, void* stream);
int gptrig_gelu_bwd(const void* dy, const void* x, void* dx, int64_t n, void* stream);
/* The same after the up-projection's bias add (rig/nn.py:55-56, the GEMM
 * output rounded to bf16, then + b.astype(bf16) rounded again,
 * recipes/reference/train.py:1170-1171): x bf16 [rows, cols] is the GEMM
 * output without bias, bias bf16 [cols]; y = bf16(gelu(bf16(x + bias))) and
 * dx = bf16(dy * gelu'(bf16(x + bias))).  cols a multiple of 8, every
 * pointer 16-byte aligned. */
int gptrig_bias_gelu_fwd(const void* x, const void* bias, void* y, int rows, int cols, void* stream);
int gptrig_bias_gelu_bwd(const void* dy, const void* x, const void* bias, void* dx, int rows, int cols,
                         void* stream);

/* Interleaved RoPE, base 10000: rig/nn.py:36-52 (apply_rotary).
 * rope_table fills bf16 cos/sin [seq, head_dim/2].  rope_fwd/bwd rotate, in
 * place, the first `heads` head_dim-wide column groups of each row of a bf16
 * [rows, row_stride] buffer; the position of a row is row % seq. */
int gptrig_rope_table(void* cos_table, void* sin_table, int seq, int head_dim, void* stream);
int gptrig_rope_fwd(void* x, int64_t row_stride, int rows, int seq, int heads, int head_dim, const void* cos_table,
                    const void* sin_table, void* stream);
int gptrig_rope_bwd(void* dx, int64_t row_stride, int rows, int seq, int heads, int head_dim,
                    const void* cos_table, const void* sin_table, void* stream);
/* The fused projection's bias add and the RoPE of its q / k columns in one
 * in-place pass (rig/nn.py:55-56 then :36-52, recipes/reference/train.py:
 * 1136-1142): columns [0, cols) of each row become bf16(x + bias[column]),
 * the rounding of the linear's bias add after its bf16 GEMM output, and the
 * first heads * head_dim of them are then rotated as gptrig_rope_fwd does.
 * cols, head_dim and row_stride multiples of 8, heads * head_dim <= cols <=
 * row_stride; x and bias 16-byte aligned. */
int gptrig_bias_rope_fwd(void* x, int64_t row_stride, int rows, int cols, const void* bias, int seq, int heads,
                         int head_dim, const void* cos_table, const void* sin_table, void* stream);

/* Token-embedding gather (recipes/reference/train.py:1107) and its transpose:
 * out bf16 [n, d] = table[tokens]; dtable f32 [vocab, d] += scatter(dout). */
int gptrig_embedding_fwd(const int32_t* tokens, const void* table, void* out, int n, int d, int vocab,
                         void* stream);
int gptrig_embedding_bwd(const int32_t* tokens, const void* dout, float* dtable, int n, int d, int vocab,
                         void* stream);

/* ------------------------------------------------------------------------
 * AdamW over one flat f32 arena: recipes/reference/train.py:1386-1445
 * (_apply_training_update), with the per-tensor multipliers of
 * optimizer_hyperparameter_trees (:1274-1333) and the decay mask of
 * weight_decay_mask (:1252-1271) folded into tensor_hparams[t] =
 * {lr_mult, epsilon, decay}.  Every tensor starts on a `chunk` boundary
 * (chunk % 1024 == 0) and chunk_tensor[c] names chunk c's tensor.
 * param_bf16 (nullable) receives bf16(updated param).  clip_scale (nullable
 * device scalar) multiplies the gradient.  sq_partials (nullable, f32
 * [n_chunks]) receives each chunk's sum of squared raw gradients.
 * ---------------------------------------------------------------------- */
int gptrig_adamw(float* param, const float* grad, float* m, float* v, void* param_bf16, const int32_t* chunk_tensor,
                 const float* tensor_hparams, int64_t n_chunks, int chunk, float lr, float beta1, float beta2,
                 int step, const float* clip_scale, float* sq_partials, void* stream);
/* Per-chunk sums of squares of an f32 arena (for clipping before the update). */
int gptrig_sq_norm_partials(const float* x, int64_t n_chunks, int chunk, float* partials, void* stream);
/* norm = sqrt(sum partials); clip = min(1, grad_clip/(norm+1e-6)) (1 if grad_clip <= 0);
 * history_row (nullable) = {*loss, lr, norm} (train.py:1446-1447). */
int gptrig_finalize_norm(const float* partials, int parts, float grad_clip, float* norm_out, float* clip_out,
                         const float* loss, float lr, float* history_row, void* stream);

/* bf16 transpose dst [cols, rows] = src [rows, cols]^T (cols a multiple of 8):
 * the K-major copy of a linear weight (rig/nn.py:55-56), which the forward
 * GEMM reads faster than the [d_in, d_out] layout. */
int gptrig_transpose_bf16(const void* src, void* dst, int rows, int cols, void* stream);

/* Small helpers of the step: f32 -> bf16 cast, out += weight * sum(x), fill. */
int gptrig_cast_f32_bf16(const float* x, void* y, int64_t n, void* stream);
int gptrig_weighted_sum(const float* x, int64_t n, float weight, float* out, void* stream);
/* Masked loss sum of eval_step (recipes/reference/train.py:1493-1525):
 * out[0] += sum(x * mask), out[1] += sum(mask), x and mask f32 [n]. */
int gptrig_masked_sum(const float* x, const float* mask, int64_t n, float* out, void* stream);
int gptrig_fill_f32(float* x, int64_t n, float value, void* stream);

/* ------------------------------------------------------------------------
 * MoE routing: recipes/reference_moe/train.py:1259-1273 (routed_mlp_local).
 * logits f32 [tokens, experts] (experts <= 64, top_k <= experts):
 *   probs f32 [tokens, experts] = softmax(logits)          (nullable)
 *   chosen i32 [tokens, top_k] = jax.lax.top_k indices (descending value,
 *     lower index first on ties), gate f32 [tokens, top_k] = softmax of the
 *     chosen logits;
 *   counts i32 [experts] = assignments per expert;
 *   order i32 [tokens*top_k] = stable argsort of chosen.reshape(-1);
 *   rows i32 [tokens*top_k] = order / top_k (the source token of each slot);
 *   position i32 [tokens*top_k] (nullable) = inverse of order: the bucket
 *     row of assignment t*top_k + j.
 * workspace: gptrig_moe_route_workspace_bytes(tokens, experts, top_k).
 * ---------------------------------------------------------------------- */
size_t gptrig_moe_route_workspace_bytes(int tokens, int experts, int top_k);
int gptrig_moe_route(const float* logits, float* probs, int32_t* chosen, float* gate, int32_t* counts,
                     int32_t* order, int32_t* rows, int32_t* position, void* workspace, size_t workspace_bytes,
                     int tokens, int experts, int top_k, void* stream);

/* Router logits of routed_mlp_local (reference_moe/train.py:1259-1264):
 * logits f32 [tokens, experts] = f32(x) @ router_w, x bf16 [tokens, width],
 * router_w f32 [width, experts]; experts <= 16, width * experts <= 8192. */
int gptrig_moe_router_logits(const void* x, const float* router_w, float* logits, int tokens, int width, int experts,
                             void* stream);

/* Bucket-order copy of the token rows, grouped = flat[rows]
 * (reference_moe/train.py:1278): grouped bf16 [n_rows, width] with
 * grouped[p] = x[rows[p]]; width a multiple of 8. */
int gptrig_moe_gather_rows(const void* x, const int32_t* rows, void* grouped, int n_rows, int width, void* stream);

/* Grouped expert GEMM, the megablox.gmm calls of routed_mlp_local
 * (reference_moe/train.py:1279-1285) with their bias / GELU epilogues:
 * for each expert e and each of its counts[e] bucket rows r (buckets are
 * consecutive in expert order, rows = sum(counts)):
 *   acc[r][j] = sum_i lhs[r][i] * W_e(i, j)   (lhs bf16, leading dim lda),
 *   W_e = rhs + e*k*n as bf16 [k][n], or as [n][k] (its transpose) when
 *   rhs_transposed (the input-gradient GEMM of the backward);
 *   mode 0: out = bf16(acc) (+ bias[e][j] when bias is not NULL)
 *   mode 1: pre = bf16(bf16(acc) + bias[e][j]), out = bf16(gelu_tanh(pre))
 *   mode 2: out = bf16(bf16(acc) * gelu_tanh'(pre))   (pre is an input)
 * out / pre bf16 [rows, n] with leading dim ldo; k, n multiples of 8. */
int gptrig_moe_gmm(const void* lhs, int64_t lda, const void* rhs, int rhs_transposed, const int32_t* counts,
                   const void* bias, int mode, void* out, void* pre, int64_t ldo, int rows, int k, int n, int experts,
                   void* stream);

/* Expert weight and bias gradients (the transposed gmm of the backward):
 * dw f32 [experts, k, n] += sum over bucket rows r of expert e of
 * lhs[r][i] * dy[r][j]; db f32 [experts, n] (nullable) += column sums of
 * dy over each bucket.  fp32 atomics. */
int gptrig_moe_gmm_dw(const void* lhs, int64_t lda, const void* dy, int64_t ldy, const int32_t* counts, float* dw,
                      float* db, int rows, int k, int n, int experts, void* stream);

/* Gated combine (reference_moe/train.py:1287-1288): combined bf16 [tokens,
 * width] = sum over the token's top_k bucket rows, in bucket order, of
 * bf16(out[p] * bf16(gate)), accumulated in bf16 like zeros.at[rows].add.
 * position from gptrig_moe_route; top_k <= 8. */
int gptrig_moe_combine(const void* out, const int32_t* position, const float* gate, void* combined, int tokens,
                       int width, int top_k, void* stream);
/* Its VJP: dout bf16 [rows, width] = dcombined[t] * bf16(gate[a]) at the
 * slot's bucket row, dgate f32 [tokens*top_k] = <dcombined[t], out[p]>. */
int gptrig_moe_combine_bwd(const void* dcombined, const void* out, const int32_t* position, const float* gate,
                           void* dout, float* dgate, int tokens, int width, int top_k, void* stream);
/* VJP of grouped = flat[rows]: dx bf16 [tokens, width] = bf16 sum over the
 * token's bucket rows (bucket order) of dgrouped. */
int gptrig_moe_gather_bwd(const void* dgrouped, const int32_t* position, void* dx, int tokens, int width, int top_k,
                          void* stream);

/* Router statistics of routed_mlp_local (reference_moe/train.py:1290-1306):
 * mean_probability f32 [experts], load f32 [experts] = counts / (tokens *
 * top_k), summary f32 [3] = (mean entropy, mean top-1 gate, logit RMS). */
int gptrig_moe_stats(const float* logits, const float* probs, const float* gate, const int32_t* counts, int tokens,
                     int experts, int top_k, float* mean_probability, float* load, float* summary, void* stream);

/* Router backward: gate-softmax and probability-softmax VJPs (dgate from
 * gptrig_moe_combine_bwd; dmean_probability f32 [experts] nullable, the
 * gradient of the balance loss w.r.t. mean_probability, load_balance_loss
 * :1347-1371), then dx bf16 [tokens, width] += bf16(dlogits @ router_w^T)
 * in place and dw_router f32 [width, experts] += f32(x)^T dlogits. */
int gptrig_moe_router_bwd(const void* x, const float* router_w, const float* probs, const int32_t* chosen,
                          const float* gate, const float* dgate, const float* dmean_probability, void* dx,
                          float* dw_router, int tokens, int width, int experts, int top_k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GPTRIG_H_ */
