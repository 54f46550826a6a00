/*
 * llamazero_hip.h — C ABI of libllamazero_hip.so, the gfx950 (MI355X) kernels
 * behind the single-GPU LLaMA training step of the llama-zero harness.
 *
 * Conventions shared by every entry point:
 *   - pointers are device pointers; sizes and leading dimensions are element
 *     counts (int64_t); `stream` is a hipStream_t passed as void*;
 *   - work is enqueued asynchronously on `stream`; nothing here synchronizes
 *     the host;
 *   - return 0 on success, a negative status on invalid arguments (-1) or a
 *     launch failure (-2); lz_last_error() returns the calling thread's last
 *     message;
 *   - nothing allocates device memory: every buffer, including workspaces, is
 *     passed in by the caller;
 *   - dtype codes: LZ_F32 = 0, LZ_BF16 = 1, LZ_F16 = 2 (16-bit formats stored
 *     as uint16 bits).  Entry points that do not list LZ_F16 refuse it.
 *
 * The reference (dannyadkins/cs244c-llama-zero) is pure PyTorch and has no
 * FFI; each declaration names the reference code whose computation it
 * replaces.  The Python binding is cs244c-llama-zero_amd/lzhip/_lib.py.
 */
#ifndef LLAMAZERO_HIP_H
#define LLAMAZERO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LZ_F32 0
#define LZ_BF16 1
#define LZ_F16 2

/* ---- library ------------------------------------------------------------ */
const char* lz_last_error(void);
int lz_version(void);
int lz_device_cus(void); /* compute units of the current device */

/* ---- optimizer path ----------------------------------------------------- */

/* Fused AdamW over a flat fp32 master partition, one pass:
 *   g' = g * (*grad_scale)   (grad_scale may be NULL)
 *   m = b1*m + (1-b1)*g';  v = b2*v + (1-b2)*g'^2;  p *= 1 - lr*wd;
 *   p -= lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps)
 * and optionally writes p in p_out_dtype to p_out (the model's parameters).
 * Replaces the unfused update of zero/stage0_ddp.py:73-88 (identical in
 * zero/stage1_optimizer.py:73-88, zero/stage2_optimizer.py:145-160,
 * zero/stage3_optimizer.py:454-470) and the .to(param_dtype) +
 * assign_flat_params write-back of zero/common.py:202-216. */
int lz_adamw(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype, int64_t n,
             double lr, double beta1, double beta2, double eps, double weight_decay, int64_t step,
             const float* grad_scale, void* stream);

/* Device-resident step count for callers that capture the optimizer in a HIP
 * graph, where launch arguments are frozen (no reference counterpart; the
 * reference's torch.optim.AdamW keeps the step on the host).
 * lz_adamw_step advances *step (device int64) and writes hyper[3] =
 * {-lr / (1 - beta1^t), sqrt(1 - beta2^t), 1 - lr * weight_decay} for the new
 * t; lz_adamw_dev is lz_adamw with those three factors read from hyper. */
int lz_adamw_step(int64_t* step, double lr, double beta1, double beta2, double weight_decay, float* hyper,
                  void* stream);
int lz_adamw_dev(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype, int64_t n,
                 double beta1, double beta2, double eps, double weight_decay, const float* hyper,
                 const float* grad_scale, void* stream);

/* *acc += sum(x^2) (acc is a device double).  Replaces flat_grads.norm(2)
 * (zero/stage0_ddp.py:66) and sum(g*g) (zero/stage2_optimizer.py:162-166,
 * zero/stage3_optimizer.py:438-444). */
int lz_sumsq(const void* x, int dtype, int64_t n, double* acc, void* stream);

/* lz_adamw that also adds sum(g^2) (g as stored, before grad_scale) to *acc,
 * for a step whose norm is reported but does not clip: the reference's
 * default max_grad_norm = 0.0 (zero/stage0_ddp.py:62-71, stage1/2/3 alike)
 * computes the norm and never uses it in the update, so the update's own read
 * of g serves both instead of a second pass (lz_sumsq + lz_adamw).  With
 * p, m, v, g (and p_out) 16-byte aligned the sum is taken in a fixed order
 * (workgroup partials into `workspace`, then two reduction launches), so it
 * is the same from run to run; otherwise the update takes the scalar kernel
 * and the sum a separate lz_sumsq-style pass.  lz_adamw_norm_workspace(n)
 * gives the float64 words `workspace` must hold. */
int64_t lz_adamw_norm_workspace(int64_t n);
int lz_adamw_norm(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype, int64_t n,
                  double lr, double beta1, double beta2, double eps, double weight_decay, int64_t step,
                  const float* grad_scale, double* acc, double* workspace, int64_t workspace_words, void* stream);
/* Multi-tensor forms of lz_adamw and lz_sumsq for per-parameter optimizers
 * (reference train.py:206-211,259-271: torch.optim.AdamW over the model's
 * parameter list and clip_grad_norm_ over their gradients): one launch per 24
 * tensors instead of one per tensor.  table is a HOST array of nseg rows:
 * lz_adamw_multi rows are {p, m, v, g, p_out (0 = none), numel} (int64; every
 * row shares g_dtype and p_out_dtype; hyper as in lz_adamw_dev, or NULL to use
 * lr and step); lz_sumsq_multi rows are {x, numel}.  Element math is that of
 * lz_adamw / lz_sumsq. */
int lz_adamw_multi(const int64_t* table, int nseg, int g_dtype, int p_out_dtype, double lr, double beta1, double beta2,
                   double eps, double weight_decay, int64_t step, const float* hyper, const float* grad_scale,
                   void* stream);
int lz_sumsq_multi(const int64_t* table, int nseg, int dtype, double* acc, void* stream);

/* norm = sqrt(*acc) * inv_grad_scale; scale = inv_grad_scale * (max/(norm+1e-6)
 * if 0 < max < norm else 1).  Replaces the clip decision of
 * zero/stage0_ddp.py:66-71 (and stage1/2/3) and, with inv_grad_scale = 1 /
 * the loss scale, GradScaler.unscale_ before clip_grad_norm_
 * (train.py:254-262): the gradients stay scaled and AdamW applies `scale`. */
int lz_clip_finalize(const double* acc, float max_norm, float inv_grad_scale, float* norm_out, float* scale_out,
                     void* stream);

/* Multi-tensor gather: dst[i-begin] = src_seg[i-off] for flat i in [begin,end).
 * table: device int64 records {ptr, numel, flat_offset} sorted by offset; a
 * NULL ptr reads as zeros; accumulate=1 adds into an fp32 dst.  Replaces the
 * torch.cat flattens of zero/common.py:132-200 and
 * zero/stage3_optimizer.py:32-40 (and builds the 25M-element gradient buckets). */
int lz_mt_gather(const int64_t* table, int nseg, int src_dtype, void* dst, int dst_dtype, int64_t begin, int64_t end,
                 int accumulate, void* stream);

/* Multi-tensor scatter: dst_seg[i-off] = src[i-begin] with a cast.  Replaces
 * assign_flat_params (zero/common.py:202-216) and the ZeRO-3 materialise
 * (zero/stage3_optimizer.py:65-74). */
int lz_mt_scatter(const void* src, int src_dtype, const int64_t* table, int nseg, int dst_dtype, int64_t begin,
                  int64_t end, void* stream);

/* The same two operations with the records in HOST memory: they are passed to
 * the kernels by value (up to 48 per launch, split automatically), so no
 * table upload or host synchronisation is needed.  This is what the engines
 * call every step. */
int lz_mt_gather_host(const int64_t* host_table, int nseg, int src_dtype, void* dst, int dst_dtype, int64_t begin,
                      int64_t end, int accumulate, void* stream);
int lz_mt_scatter_host(const void* src, int src_dtype, const int64_t* host_table, int nseg, int dst_dtype,
                       int64_t begin, int64_t end, void* stream);

/* dst(fp32) += alpha * src.  Replaces grad_shard.add_(local_grads.to(fp32))
 * (zero/stage3_optimizer.py:98-103, zero/stage2_optimizer.py:134-139). */
int lz_axpy_f32(float* dst, const void* src, int src_dtype, int64_t n, float alpha, void* stream);

/* dst = dst + src in the storage dtype.  Replaces the post-accumulate hook add
 * flat_grad_buffer[start:end].add_(grad) (zero/stage2_optimizer.py:109-114). */
int lz_add_inplace(void* dst, const void* src, int dtype, int64_t n, void* stream);

/* x *= alpha in the storage dtype (grad averaging / clipping in place). */
int lz_scale_inplace(void* x, int dtype, int64_t n, float alpha, void* stream);
/* x *= *scale with `scale` a device float: applies an upstream gradient that
 * is only known on the device (the fused LM-head + cross-entropy gradients,
 * computed in the forward for a unit loss gradient). */
int lz_scale_dev(void* x, int dtype, int64_t n, const float* scale, void* stream);

/* Fill / cast.  Replace torch.zeros(...) for gradient buffers
 * (zero/stage2_optimizer.py:88-89) and dtype casts (.to()).  lz_fill also
 * takes dtype 3 (float64) for the norm accumulators. */
int lz_fill(void* x, int dtype, int64_t n, double value, void* stream);
int lz_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream);

/* ---- model ops ----------------------------------------------------------- */

/* RMSNorm (model/llama.py:14-22): y = x * rsqrt(mean(x^2)+eps) * w, rstd[row]
 * saved (fp32).  x, w, y in `dtype`. */
int lz_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int dtype, int64_t rows, int64_t cols,
                   int64_t ldx, int64_t ldy, float eps, void* stream);
/* Backward: dx = rstd*w*dy - rstd^3/n * (sum dy*w*x) * x (+ dres); dw (=/+=)
 * sum over rows of dy*x*rstd (fp32 partial rows in the workspace, then a
 * fixed-order column sum).  workspace (16-byte aligned) >=
 * lz_rmsnorm_bwd_workspace(rows, cols) bytes; calls sharing a workspace must
 * not overlap. */
int64_t lz_rmsnorm_bwd_workspace(int64_t rows, int64_t cols);
int lz_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, const void* dres, void* dx, void* dw,
                   int dw_accumulate, void* workspace, int64_t workspace_bytes, int dtype, int64_t rows, int64_t cols,
                   int64_t ldx, int64_t lddy, int64_t lddx, void* stream);

/* lz_rmsnorm_bwd without a workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).  The
 * dw partial rows live in the library's own 8 MiB device array,
 * one per device, held until the process ends; shapes that need more are
 * refused (bf16 or fp16 rows of up to 4096 columns fit at any row count).  Same
 * results as lz_rmsnorm_bwd bit for bit.  Every call on a device shares that
 * array: calls that overlap in time on one device race. */
int lz_rmsnorm_bwd_noalloc(const void* x, const void* w, const float* rstd, const void* dy, const void* dres, void* dx,
                           void* dw, int dw_accumulate, int dtype, int64_t rows, int64_t cols, int64_t ldx,
                           int64_t lddy, int64_t lddx, void* stream);

/* RoPE table (model/llama.py:42-69 RotaryEmbedding._build_cache): cos/sin
 * [seq, hd] in dtype from the module's inv_freq buffer (hd/2 values of
 * freq_dtype); position, angle and cos/sin are rounded to freq_dtype, as the
 * reference's cache is after Module.to(dtype) casts that buffer. */
int lz_rope_table(void* cos_t, void* sin_t, int dtype, int64_t seq, int64_t hd, const void* inv_freq, int freq_dtype,
                  void* stream);
/* In-place rotary embedding of `nheads` heads per row (model/llama.py:25-39
 * rotate_half/apply_rotary_pos_emb); backward=1 applies the transpose. */
int lz_rope(void* x, int dtype, int64_t ld, int64_t rows, int64_t seq, int64_t nheads, int64_t hd, const void* cos_t,
            const void* sin_t, int64_t pos_offset, int backward, void* stream);

/* SwiGLU pointwise part (model/llama.py:145): h = silu(g) * u, and its
 * backward. */
int lz_swiglu_fwd(const void* g, int64_t ldg, const void* u, int64_t ldu, void* h, int64_t ldh, int64_t rows,
                  int64_t cols, int dtype, void* stream);
int lz_swiglu_bwd(const void* g, int64_t ldg, const void* u, int64_t ldu, const void* dh, int64_t lddh, void* dg,
                  int64_t lddg, void* du, int64_t lddu, int64_t rows, int64_t cols, int dtype, void* stream);

/* Embedding gather (model/llama.py:174,212) and gradient (fp32 atomics into a
 * vocab*dim fp32 workspace, then written/added in dtype).  bad_flag (nullable)
 * is set to 1 when an id is out of range. */
int lz_embedding_fwd(const int64_t* ids, int64_t ntok, const void* table, int64_t vocab, int64_t dim, void* out,
                     int64_t ldo, int dtype, int* bad_flag, void* stream);
int lz_embedding_bwd(const int64_t* ids, int64_t ntok, const void* dout, int64_t ldo, int64_t vocab, int64_t dim,
                     void* grad, int accumulate, float* workspace, int dtype, void* stream);

/* Shifted cross entropy (model/llama.py:273-302, ignore_index -100):
 * lse/row_loss per row, lz_ce_reduce forms the mean (clamp_count=1 gives the
 * chunked variant's division by max(count,1)), lz_ce_bwd writes
 * (softmax - onehot) * grad/count (may run in place over the logits). */
int lz_ce_fwd(const void* logits, int64_t ld, int64_t rows, int64_t vocab, int dtype, const int64_t* labels,
              int64_t seq, int64_t ignore_index, float* lse, float* row_loss, void* stream);
int lz_ce_reduce(const float* row_loss, const int64_t* labels, int64_t rows, int64_t seq, int64_t vocab,
                 int64_t ignore_index, float* loss_out, float* count_out, int clamp_count, void* stream);
int lz_ce_bwd(const void* logits, int64_t ld, int64_t rows, int64_t vocab, int dtype, const int64_t* labels,
              int64_t seq, int64_t ignore_index, const float* lse, const float* grad_loss, const float* count,
              void* dlogits, int64_t ldd, int ddtype, void* stream);

/* Batched transpose dst[b1][b2][c][r] = src[b1][b2][r][c] (operand layout
 * for the backward GEMMs and attention; replaces the .transpose(1, 2) views
 * of model/llama.py:97-99,132). */
int lz_transpose(const void* src, void* dst, int dtype, int64_t nb1, int64_t nb2, int64_t rows, int64_t cols,
                 int64_t lds, int64_t sb1s, int64_t sb2s, int64_t ldd, int64_t sb1d, int64_t sb2d, void* stream);

/* dst[r][c] = src[r][c] over a rows x cols window (re-strides an operand whose
 * leading dimension the GEMM cannot take, and concatenates weights; replaces
 * torch.cat / .contiguous() copies). */
int lz_copy2d(const void* src, int64_t lds, void* dst, int64_t ldd, int64_t rows, int64_t cols, int dtype,
              void* stream);

/* bf16 / fp16 MFMA GEMM C[M,N] = alpha * sum_k A(m,k) B(n,k) (+beta*C) (+R):
 * the nn.Linear products of model/llama.py:81-84,133,139-141,178 and their
 * gradients (bf16 models, and fp16 ones: train.py --dtype float16).  A and B
 * in ab_dtype (LZ_BF16 or LZ_F16), fp32 accumulation, C in ab_dtype or fp32,
 * R an optional residual in ab_dtype.
 *   a_kmajor = 1: A(m,k) = A[m*lda + k]   a_kmajor = 0: A(m,k) = A[k*lda + m]
 *   b_kmajor = 1: B(n,k) = B[n*ldb + k]   b_kmajor = 0: B(n,k) = B[k*ldb + n]
 * so y = x.W^T is (1,1), dx = dy.W is (1,0) and dW = dy^T.x is (0,0).
 * A and B 16-byte aligned, lda and ldb multiples of 8, K % 8 == 0 when an
 * operand is K-major, M % 8 == 0 (N % 8 == 0) for an M-major A (N-major B).
 * When few output tiles meet a long K the product is split along K into
 * fp32 partial slabs in `ws` (lz_gemm_workspace bytes) and summed in a fixed
 * order; with a smaller workspace it runs unsplit. */
int64_t lz_gemm_workspace(int64_t M, int64_t N, int64_t K, int a_kmajor, int b_kmajor);
/* The kernel lz_gemm picks for a shape and layout, as 64 * cfg + splits
 * (cfg 5: direct-to-LDS 256x256 tile, 8 waves; 0 / 1: register-staged
 * 256x256, 8 / 4 waves; 2: 128x128, 4 waves; splits: K slices, 1 = unsplit).
 * Diagnostic only (used to attribute timings to kernels); no reference
 * counterpart. */
int lz_gemm_plan(int64_t M, int64_t N, int64_t K, int a_kmajor, int b_kmajor);
int lz_gemm(const void* A, int64_t lda, int a_kmajor, const void* B, int64_t ldb, int b_kmajor, int ab_dtype, void* C,
            int64_t ldc, int c_dtype, const void* R, int64_t ldr, int64_t M, int64_t N, int64_t K, float alpha,
            float beta, void* ws, int64_t ws_bytes, void* stream);
/* lz_gemm with both operands K-major and no workspace. */
int lz_gemm_nt(const void* A, int64_t lda, const void* B, int64_t ldb, int ab_dtype, void* C, int64_t ldc, int c_dtype,
               const void* R, int64_t ldr, int64_t M, int64_t N, int64_t K, float alpha, float beta, void* stream);
/* fp32 MFMA GEMM with lz_gemm's operand layouts and epilogue: the nn.Linear
 * products when the model is kept in float32 (train.py:148-160 and
 * train_zero.py:74,150-164 with --dtype float32).  fp32 operands, fp32
 * accumulation, C fp32 or bf16, R an optional fp32 residual.  Any M, N, K
 * and leading dimensions.  Products with few output tiles and a long K are
 * split along K into `ws` (at least lz_gemm_f32_workspace() bytes, 16-byte
 * aligned; with less, or NULL, the product runs unsplit). */
int64_t lz_gemm_f32_workspace(int64_t M, int64_t N, int64_t K);
int lz_gemm_f32_plan(int64_t M, int64_t N, int64_t K);
int lz_gemm_f32(const float* A, int64_t lda, int a_kmajor, const float* B, int64_t ldb, int b_kmajor, void* C,
                int64_t ldc, int c_dtype, const float* R, int64_t ldr, int64_t M, int64_t N, int64_t K, float alpha,
                float beta, void* ws, int64_t ws_bytes, void* stream);
/* Fused gate/up projections + SwiGLU (model/llama.py:139-145: gate_proj(x),
 * up_proj(x), silu(gate) * up): w = [gate rows; up rows] ([2F, K]);
 * h = silu(x.Wg^T) * (x.Wu^T) as bf16 [M, F], and x.w^T itself to gu
 * ([M, 2F], may be NULL).  Bit-identical to lz_gemm (bf16 out) followed by
 * lz_swiglu_fwd.  Needs M % 256 == 0, F % 128 == 0, K % 64 == 0 and
 * 16-byte aligned rows. */
int lz_gemm_swiglu(const void* x, int64_t ldx, const void* w, int64_t ldw, void* gu, int64_t ldgu, void* h,
                   int64_t ldh, int64_t M, int64_t F, int64_t K, void* stream);
/* Fused QKV projection + RoPE (model/llama.py:95-103: q/k/v_proj and
 * apply_rotary_pos_emb on q and k): out = x.w^T ([M, N] bf16) with columns
 * [0, nrope) rotated as heads of 128, output row m taking position m % S of
 * the bf16 cos/sin tables ([>= S, 128]).  Bit-identical to lz_gemm (bf16 out)
 * followed by lz_rope on those columns.  Needs M, N and nrope multiples of
 * 256, K % 64 == 0 and 16-byte aligned rows. */
int lz_gemm_rope(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out, int64_t ldo, const void* cos_t,
                 const void* sin_t, int64_t S, int64_t nrope, int64_t M, int64_t N, int64_t K, void* stream);
/* lz_gemm_rope for heads of hd = 128 or 64 (the same call sites,
 * model/llama.py:95-103, at the 125M model's head dim 64): tables
 * [>= S, hd]; lz_gemm_rope is this with hd = 128.  Bit-identical to lz_gemm
 * (bf16 out) followed by lz_rope on columns [0, nrope). */
int lz_gemm_rope_hd(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out, int64_t ldo,
                    const void* cos_t, const void* sin_t, int64_t S, int64_t nrope, int64_t hd, int64_t M, int64_t N,
                    int64_t K, void* stream);
/* Down projection input gradient fused with SwiGLU's backward
 * (model/llama.py:136-146: autograd of down_proj(silu(gate_proj x) *
 * up_proj x)): dm = dy.W_down (dy [M, K], W_down [K, F] row-major) meets
 * gu = [gate | up] ([M, 2F]) and dgate, dup go to columns [0, F) and [F, 2F)
 * of dgu; dm is never stored.  Bit-identical to lz_gemm (bf16 out, W_down
 * read N-major) followed by lz_swiglu_bwd.  Needs M % 256 == 0,
 * F % 256 == 0, K % 64 == 0 and 16-byte aligned rows; dgu != gu. */
int lz_gemm_swiglu_bwd(const void* dy, int64_t lddy, const void* w, int64_t ldw, const void* gu, int64_t ldgu,
                       void* dgu, int64_t lddgu, int64_t M, int64_t F, int64_t K, void* stream);

/* Causal GQA flash attention (model/llama.py:88-117: repeat_kv +
 * F.scaled_dot_product_attention(is_causal=True)).  lz_attn_path reports the
 * path lz_attn_fwd/bwd take: 2 = MFMA on LDS tiles (bf16 or fp16, hd 64 or 128, S a
 * multiple of 64; the transposed-operand arguments may be NULL), 1 = MFMA
 * with the transposed operand buffers (vt for the forward; qt, kt, dot for the
 * backward, each [B, heads, hd, S]), 0 = generic. */
int lz_attn_path(int dtype, int64_t S, int64_t hd, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo);
int lz_attn_fwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, const void* vt,
                void* o, int64_t ldo, float* lse, int64_t B, int64_t S, int64_t H, int64_t KV, int64_t hd, float scale,
                int dtype, void* stream);
int lz_attn_delta(const void* o, int64_t ldo, const void* dout, int64_t lddo, float* delta, int64_t B, int64_t S,
                  int64_t H, int64_t hd, int dtype, void* stream);
/* Backward.  rope_cos/rope_sin (both or NULL; lz_rope's tables): dq and dk
 * are returned as the gradients of q and k before RoPE (model/llama.py:35-39
 * backward), folded into the bf16 MFMA kernels' stores or, on the other
 * paths, applied by lz_rope afterwards. */
/* Attention on the one-wave-per-row kernels with the options the MFMA tile
 * paths do not take (model/llama.py:105-117, F.scaled_dot_product_attention):
 *  - an explicit mask in place of the causal one (attn_mask with
 *    is_causal=False): mask_kind 1 = bool bytes (nonzero: the key takes
 *    part), 2 = fp32, 3 = bf16, 4 = fp16 (added to the scaled scores); mstride = 4
 *    element strides over [B, H, S(query), S(key)], 0 where the mask
 *    broadcasts; mask_kind 0 = causal (mask, mstride ignored).  A query row
 *    whose keys are all masked gives NaN, as the reference's softmax does;
 *  - attention dropout (dropout_p, model/llama.py:107,115): probability
 *    (b, h, s, kv) is kept, scaled by 1/(1-p), when element
 *    ((b*H + h)*S + s)*S + kv of seed's keep stream (lz_dropout_mask) is 1.
 * Any head dim up to 256, bf16 or fp32.  The backward takes the forward's
 * mask, dropout_p and seed; delta from lz_attn_delta. */
int lz_attn_fwd_general(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                        const void* mask, int mask_kind, const int64_t* mstride, float dropout_p, uint64_t seed,
                        void* o, int64_t ldo, float* lse, int64_t B, int64_t S, int64_t H, int64_t KV, int64_t hd,
                        float scale, int dtype, void* stream);
int lz_attn_bwd_general(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                        const void* dout, int64_t lddo, const float* lse, const float* delta, const void* mask,
                        int mask_kind, const int64_t* mstride, float dropout_p, uint64_t seed, void* dq, int64_t lddq,
                        void* dk, int64_t lddk, void* dv, int64_t lddv, int64_t B, int64_t S, int64_t H, int64_t KV,
                        int64_t hd, float scale, int dtype, void* stream);
int lz_attn_bwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, const void* dout,
                int64_t lddo, const float* lse, const float* delta, const void* qt, const void* kt, const void* dot,
                void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv, int64_t B, int64_t S,
                int64_t H, int64_t KV, int64_t hd, float scale, const void* rope_cos, const void* rope_sin, int dtype,
                void* stream);
/* lz_attn_delta + lz_attn_bwd in one call, for the shapes lz_attn_path
 * reports as 2 (LDS-tile kernels; others are refused): the same backward of
 * model/llama.py:88-117, with delta = rowsum(dO * O) computed by the dQ
 * kernel from the dO rows it loads anyway (O: [B*S, ldo] rows like dout, 16-byte
 * aligned) and written to `delta` ([B, H, S] fp32, an output), which the
 * dK/dV kernel then reads; saves the separate pass over O and dO. */
int lz_attn_bwd_with_o(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                       const void* o, int64_t ldo, const void* dout, int64_t lddo, const float* lse, float* delta,
                       void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv, int64_t B, int64_t S,
                       int64_t H, int64_t KV, int64_t hd, float scale, const void* rope_cos, const void* rope_sin,
                       int dtype, void* stream);

/* ---- dropout (model/llama.py:142,146 on the MLP's gated activations and
 * :175,213 on the token embeddings: nn.Dropout in training mode) ----
 * y = x * keep / (1 - p) over n contiguous elements (x == y allowed).  The
 * keep mask is not stored: element i is kept when the top 24 bits of
 * SplitMix64(seed, i) are >= ceil(p * 2^24), so the backward is the same
 * call on the gradient with the same seed, and a recompute that replays the
 * seed replays the mask.  p in [0, 1]; p == 1 zeroes y.  dtype LZ_BF16 or
 * LZ_F32.  lz_dropout_mask writes that keep mask (1 byte per element). */
int lz_dropout(const void* x, void* y, int64_t n, float p, uint64_t seed, int dtype, void* stream);
int lz_dropout_mask(uint8_t* keep, int64_t n, float p, uint64_t seed, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLAMAZERO_HIP_H */
