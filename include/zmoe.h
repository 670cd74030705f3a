/*
 * zmoe.h — C ABI of the MI355X (gfx950) MoE-layer hot path.
 *
 * One shared library, libzmoe_hip.so, behind the reference's ScatterMoE op
 * layer and its aux-loss-free gate. Every entry point:
 *   - takes caller-owned device pointers, element counts/strides (in elements),
 *     and a hipStream_t passed as void* (NULL = the legacy default stream);
 *   - never allocates device memory (scratch comes in through `workspace`);
 *   - enqueues work on `stream` and returns without synchronising;
 *   - returns ZMOE_OK or a ZMOE_ERR_* code; zmoe_last_error() gives a message
 *     (thread-local) for the most recent failure on the calling thread.
 * Index arrays are int64 like the reference's torch.long tensors.
 *
 * Reference paths (file:line) are relative to the reference repository root.
 */
#ifndef ZMOE_H_
#define ZMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZMOE_ABI_VERSION 3

/* element types */
enum { ZMOE_DTYPE_F32 = 0, ZMOE_DTYPE_BF16 = 1 };

/* status codes */
enum {
  ZMOE_OK = 0,
  ZMOE_ERR_NULL = 1,      /* a required pointer is NULL                        */
  ZMOE_ERR_SHAPE = 2,     /* sizes inconsistent, out of range or unsupported    */
  ZMOE_ERR_DTYPE = 3,     /* element type not supported by this entry point     */
  ZMOE_ERR_ALIGN = 4,     /* pointer/stride not aligned for 16-byte accesses    */
  ZMOE_ERR_WORKSPACE = 5, /* workspace missing or smaller than required         */
  ZMOE_ERR_HIP = 6        /* HIP runtime or launch error                        */
};

int zmoe_abi_version(void);
const char* zmoe_status_string(int status);
const char* zmoe_last_error(void);

/* ---------------------------------------------------------------------------
 * Routing — replaces the post-projection part of MoEGate.forward,
 * modeling/moe_gate.py:27-34 (sigmoid, +expert_biases, topk, gather,
 * F.normalize(p=1)).
 *   logits [T, E] (row stride E), dtype F32 or BF16; expert_biases [E] f32.
 *   p = sigmoid(logit) correctly rounded to fp32, 0 for logits at or below
 *   -88.72283935546875 (where torch's fp32 exp(-z) overflows and its sigmoid
 *   returns 0); if round_probs_bf16, p = bf16(p) (the reference under bf16
 *   autocast). s = p + bias. Slots ordered by
 *   (s desc, expert asc); NaN ranks above all numbers.
 *   Outputs: topk_idx [T, k] int64, topk_weight [T, k] f32 =
 *   p_sel / max(sum p_sel, 1e-12), topk_prob [T, k] f32 = p_sel (may be NULL).
 *   1 <= k <= E <= 1024.
 * ------------------------------------------------------------------------- */
int zmoe_route_topk(const void* logits, int logits_dtype, int64_t T, int E, int k,
                    const float* expert_biases, int round_probs_bf16,
                    int64_t* topk_idx, float* topk_weight, float* topk_prob,
                    void* stream);

/* Autograd of modeling/moe_gate.py:27,33-34: d_weight [T, k] f32 ->
 * d_logits [T, E] (dense, zeros off the selected experts), dtype F32/BF16,
 * rows ld_d_logits >= E elements apart (E for a packed [T, E]). */
int zmoe_route_topk_backward(const float* d_weight, const float* topk_prob,
                             const int64_t* topk_idx, int64_t T, int E, int k,
                             void* d_logits, int64_t ld_d_logits, int d_logits_dtype,
                             void* stream);

/* ---------------------------------------------------------------------------
 * Counting and sorting — scattermoe/parallel_experts.py:6-28.
 * ------------------------------------------------------------------------- */
/* compileable_bincount (parallel_experts.py:6-15): counts [E] int64. Indices
 * outside [0, E) are not counted; the workspace-free call cannot report them. */
int zmoe_bincount(const int64_t* expert_idxs, int64_t R, int E, int64_t* counts,
                  void* stream);

/* Bytes of device workspace zmoe_flatten_sort_count needs for (R, E); 0 for sizes
 * it rejects (E outside [1, 1024], R >= 2^31 - 1). */
size_t zmoe_sort_workspace_bytes(int64_t R, int E);

/* flatten_sort_count (parallel_experts.py:21-28), a stable counting sort:
 *   sorted_expert_idxs [R], sorted_scattered_idxs [R] (flat slot ids, equal
 *   experts in slot order), expert_offsets [E] (inclusive cumsum of counts),
 *   all int64; inverse [R] int32 (inverse[slot] = sorted position, may be NULL).
 * Indices outside [0, E) are placed after every valid slot with their original
 * value (the outputs stay a permutation; expert_offsets counts only valid ones)
 * and set the int32 flag at workspace offset 0 to 1; read it with
 * zmoe_sort_error_flag.                                                       */
int zmoe_flatten_sort_count(const int64_t* expert_idxs, int64_t R, int E,
                            int64_t* sorted_expert_idxs,
                            int64_t* sorted_scattered_idxs,
                            int64_t* expert_offsets, int32_t* inverse,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Device address of the out-of-range flag inside a sort workspace. */
const int32_t* zmoe_sort_error_flag(const void* workspace);

/* ---------------------------------------------------------------------------
 * flatten_sort_count without a workspace argument: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * kernels and results as zmoe_flatten_sort_count; the tile table lives in a
 * file-scope device array of ZMOE_SORT_NOALLOC_MAX_BYTES per GPU (held until the
 * process ends), so the call allocates nothing. Sizes whose workspace
 * (zmoe_sort_workspace_bytes(R, E)) exceeds that maximum return
 * ZMOE_ERR_WORKSPACE: R up to ~8.3 M slots at E = 128, ~1.05 M at E = 1024.
 * error_flag (nullable, caller-owned device int32) receives 1 when an id was
 * outside [0, E), else 0. Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (different streams, threads) race; the array needs no
 * clearing (each call writes what it reads).
 * ------------------------------------------------------------------------- */
#define ZMOE_SORT_NOALLOC_MAX_BYTES ((size_t)4 << 20)
int zmoe_flatten_sort_count_noalloc(const int64_t* expert_idxs, int64_t R, int E,
                                    int64_t* sorted_expert_idxs, int64_t* sorted_scattered_idxs,
                                    int64_t* expert_offsets, int32_t* inverse, int32_t* error_flag,
                                    void* stream);

/* expert_offsets [E] (inclusive) from an already sorted expert list; used by
 * scatter2scatter callers that do not carry offsets (ops.py:192 signature). */
int zmoe_offsets_from_sorted(const int64_t* sorted_expert_idxs, int64_t R, int E,
                             int64_t* expert_offsets, void* stream);

/* ---------------------------------------------------------------------------
 * group — scattermoe/kernels/ops.py:449-529:
 *   Y[n, :] = A[idx[n] / fan_out, :] * coeff[idx[n]]   (coeff may be NULL)
 * A [*, K] row stride lda; Y [N, K] row stride ldy; dtype F32/BF16 for A and Y;
 * coeff f32 or bf16 (coeff_dtype).
 * ------------------------------------------------------------------------- */
int zmoe_group(const void* A, int64_t lda, int64_t K, int dtype,
               const int64_t* sorted_idxs, int64_t N, int fan_out,
               const void* coeff, int coeff_dtype, void* Y, int64_t ldy,
               void* stream);

/* ---------------------------------------------------------------------------
 * scatter2scatter — scattermoe/kernels/ops.py:192-255 (grouped GEMM):
 *   sorted row i, expert e = sorted_expert_idxs[i]:
 *   in  = X[i] if x_grouped else X[sorted_scattered_idxs[i] / k]
 *   out = Y[i] if y_grouped else Y[sorted_scattered_idxs[i]]
 *   out[:] = in[:] @ W[e] (+ b[e])   with W the logical [E, K, N] operand.
 * W strides (w_stride_k, w_stride_n): one must be 1 (the reference passes the
 * parameter [E, N, K] as a permuted view, or its transpose in backward).
 * expert_offsets is required (see zmoe_offsets_from_sorted).
 * R = rows of the sorted list = (x_grouped ? M : M * k).
 * ------------------------------------------------------------------------- */
int zmoe_scatter2scatter(const void* X, int64_t x_stride_m, const void* W,
                         int64_t w_stride_e, int64_t w_stride_k, int64_t w_stride_n,
                         const void* b, int64_t b_stride_e,
                         const int64_t* sorted_expert_idxs,
                         const int64_t* sorted_scattered_idxs,
                         const int64_t* expert_offsets, int64_t M, int64_t K,
                         int64_t N, int E, int k, int x_grouped, int y_grouped,
                         int dtype, void* Y, int64_t y_stride_m, void* stream);

/* ---------------------------------------------------------------------------
 * group_bwd_W — scattermoe/kernels/ops.py:263-438 (grouped weight gradient):
 *   DWt[e, n, c] = sum_{i in expert e} DY[i, n] * Xrow(i)[c]
 *   Xrow(i) = X[i] if x_gather_idxs == NULL else X[x_gather_idxs[i] / x_gather_div]
 *   (the gather replaces the reference's group() copy, parallel_experts.py:102).
 * DWt [E, N, K] contiguous = the reference's DWt (its DW is DWt.permute(0,2,1));
 * experts with no rows get exact zeros. Db [E, N] (may be NULL) = row sums.
 * out_dtype: DWt's element type, `dtype` (the reference's, ops.py:264-265) or
 * F32 for BF16 operands: the fp32 accumulators written unrounded, the grads of
 * fp32 master weights under bf16 autocast (Db then NULL).
 * ------------------------------------------------------------------------- */
int zmoe_group_bwd_w(const void* DY, int64_t dy_stride_m, const void* X,
                     int64_t x_stride_m, const int64_t* x_gather_idxs,
                     int x_gather_div, const int64_t* expert_offsets, int64_t M,
                     int64_t N, int64_t K, int E, int dtype, int out_dtype, void* DWt,
                     void* Db, void* stream);

/* The same with the gather on DY's rows instead (parallel_experts.py:102 applied to
 * the output grad; bf16 only): DYrow(i) = DY[dy_gather_idxs[i] / dy_gather_div],
 * X rows in sorted order. With X the gate-scaled activations this is the W2 grad
 * straight from the output grad's rows (no grouped copy of them). */
int zmoe_group_bwd_w_gather_dy(const void* DY, int64_t dy_stride_m,
                               const int64_t* dy_gather_idxs, int dy_gather_div,
                               const void* X, int64_t x_stride_m,
                               const int64_t* expert_offsets, int64_t M, int64_t N,
                               int64_t K, int E, int dtype, int out_dtype, void* DWt,
                               void* stream);

/* ---------------------------------------------------------------------------
 * Dense weight gradient DW[N, K] = DY^T X over M rows (DY [M, N], X [M, K]), for
 * the nn.Linear weights around the routed experts: the shared expert's
 * gate/up/down projections (modeling/expert_layer.py:23-24) and the gate
 * projection (modeling/moe_gate.py:26), whose backward in the reference is
 * torch autograd of F.linear. Their outputs are small next to M, so the rows are
 * split into `splits` ranges computed by the grouped wgrad kernel into fp32
 * partials, then summed in a fixed order and rounded once (deterministic).
 * workspace: zmoe_dense_wgrad_workspace_bytes(N, K, splits) bytes, 16-byte
 * aligned (0 for sizes dense_wgrad rejects: N or K >= 2^30, splits > 64). fp32 runs unsplit. out_dtype: `dtype`, or F32 for BF16 operands
 * (the fp32 sum written unrounded: fp32 master weights under bf16 autocast).
 * ------------------------------------------------------------------------- */
size_t zmoe_dense_wgrad_workspace_bytes(int64_t N, int64_t K, int splits);
int zmoe_dense_wgrad(const void* DY, int64_t dy_stride_m, const void* X,
                     int64_t x_stride_m, int64_t M, int64_t N, int64_t K,
                     int dtype, int out_dtype, int splits, void* DW, void* workspace,
                     size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * rowwise_sum_product — scattermoe/kernels/ops.py:9-80:
 *   out[t, j] = sum_h A[t, j, h] * B[t, h] (fp32 accumulation)
 * A [T, F, H], B [T, H] contiguous; each F32 or BF16; out F32 or BF16.
 * ------------------------------------------------------------------------- */
int zmoe_rowwise_sum_product(const void* A, int a_dtype, const void* B, int b_dtype,
                             int64_t T, int F, int64_t H, void* out, int out_dtype,
                             void* stream);

/* ---------------------------------------------------------------------------
 * Fused GLU-expert pieces. Each replaces a sequence of reference calls.
 * ------------------------------------------------------------------------- */

/* scattermoe/mlp.py:80-86 — W1 scatter2scatter (grouped_out=True) fused with
 * chunk(2) and silu(gates) * h:
 *   H[i, :] = X[sorted_scattered_idxs[i] / k] @ W1[e]^T   ([R, 2f], sorted rows)
 *   A[i, j] = silu(H[i, f + j]) * H[i, j]                 ([R, f])
 * W1 [E, 2f, d] contiguous (ParallelExperts.weight). */
int zmoe_glu_w1_forward(const void* X, int64_t x_stride_m, const void* W1,
                        const int64_t* sorted_expert_idxs,
                        const int64_t* sorted_scattered_idxs,
                        const int64_t* expert_offsets, int64_t T, int64_t d,
                        int64_t f, int E, int k, int dtype, void* H, void* A,
                        void* stream);

/* The same with each activation row scaled by its routing weight (bf16 only):
 *   A[i, j] = row_scale[i] * silu(H[i, f + j]) * H[i, j]   (one rounding)
 * row_scale [R] f32 in sorted order (gates[sorted_scattered_idxs[i]]). The W2
 * product of these rows is then already gate-weighted, so the combine sums the k
 * rows of a token with unit weights (parallel_experts.py:50-52 reassociated). */
int zmoe_glu_w1_forward_scaled(const void* X, int64_t x_stride_m, const void* W1,
                               const int64_t* sorted_expert_idxs,
                               const int64_t* sorted_scattered_idxs,
                               const int64_t* expert_offsets, int64_t T, int64_t d,
                               int64_t f, int E, int k, int dtype, const float* row_scale,
                               void* H, void* A, void* stream);

/* scattermoe/parallel_experts.py:112-120 (W2 input grad, x_grouped and
 * y_grouped) fused with the backward of silu(gates) * h (mlp.py:86):
 *   dA[i, :] = dYg[i, :] @ W2[e]                 (W2 [E, d, f] contiguous)
 *   dH[i, j]     = dA[i, j] * silu(g)             (g = H[i, f + j], h = H[i, j])
 *   dH[i, f + j] = dA[i, j] * h * s * (1 + g (1 - s)),  s = sigmoid(g)        */
int zmoe_glu_w2_backward_dh(const void* dYg, const void* W2, const void* H,
                            const int64_t* sorted_expert_idxs,
                            const int64_t* expert_offsets, int64_t R, int64_t d,
                            int64_t f, int E, int dtype, void* dH, void* stream);

/* The same with the weighted combine's backward folded in (parallel_experts.py:
 * 80-97: the gate-scaled grouping of the output grad, and the gate grads of :82
 * via ops.py:9-80, rowwise_sum_product), bf16 only. The A rows are the output grad's rows, read in place:
 *   dYg[i] = gates[s_i] * dout[s_i / k]   (s_i = sorted_scattered_idxs[i]), so
 *   dA[i]  = gates[s_i] * (dout[s_i / k] @ W2[e])   -> dH as above, and
 *   d_gates[s_i] = <dout[s_i / k], Y[s_i]> = <dout[s_i / k] @ W2[e], A_i>,
 * with A_i = silu(g) * h from H (as the forward stored it). dout [T, d], gates and
 * d_gates [T * k] f32 in slot order; d_gates is written (not accumulated), in a
 * fixed summation order. Workspace: zmoe_glu_w2_backward_dh_gates_workspace_bytes. */
size_t zmoe_glu_w2_backward_dh_gates_workspace_bytes(int64_t R, int64_t f);
int zmoe_glu_w2_backward_dh_gates(const void* dout, int64_t T, int k, const void* W2,
                                  const void* H, const int64_t* sorted_expert_idxs,
                                  const int64_t* sorted_scattered_idxs,
                                  const int64_t* expert_offsets, const float* gates,
                                  int64_t d, int64_t f, int E, int dtype, void* dH,
                                  float* d_gates, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* scattermoe/parallel_experts.py:50-52 (gates @ output_expanded) plus the
 * residual sum of modeling/moe_layer.py:53:
 *   out[t, :] = addend[t, :] + sum_j gates[t, j] * Y[t * k + j, :]
 * Y [T*k, d] in slot order; addend may be NULL; gates may be NULL (all 1: rows
 * already scaled, e.g. by the W1 forward's row_gates); fp32 accumulation in j order. */
int zmoe_combine(const void* Y, const float* gates, const void* addend, int64_t T,
                 int k, int64_t d, int dtype, void* out, void* stream);

/* scattermoe/parallel_experts.py:80-97 (rowwise_sum_product + group with
 * coeff=gates) in one pass over grad_out:
 *   d_gates[t, j] = sum_h Y[t*k+j, h] * grad_out[t, h]
 *   grouped_grad_out[inverse[t*k+j], :] = gates[t, j] * grad_out[t, :]
 * Y and d_gates may both be NULL: then only grouped_grad_out is written (the
 * gates' grad formed elsewhere, e.g. by zmoe_glu_w2_backward_dh_gates).       */
int zmoe_combine_backward(const void* Y, const void* grad_out, const float* gates,
                          const int32_t* inverse, int64_t T, int k, int64_t d,
                          int dtype, float* d_gates, void* grouped_grad_out,
                          void* stream);

/* The two calls above with the unpad/re-pad of moe_layer.py:39-42 and :55-56 folded in:
 * token t's output row is out_rows[t] of out [out_total, d] (rows not listed are left
 * untouched, so the caller zero-fills the padded output), and token t's gradient is read
 * from row grad_rows[t] of the padded grad_out [grad_total, d]. Row numbers outside
 * [0, total) are not written / read as zero.                                      */
int zmoe_combine_rows(const void* Y, const float* gates, const void* addend, int64_t T,
                      int k, int64_t d, int dtype, const int64_t* out_rows, int64_t out_total,
                      void* out, void* stream);
int zmoe_combine_backward_rows(const void* Y, const void* grad_out, const int64_t* grad_rows,
                               int64_t grad_total, const float* gates, const int32_t* inverse,
                               int64_t T, int k, int64_t d, int dtype, float* d_gates,
                               void* grouped_grad_out, void* stream);

/* scattermoe/parallel_experts.py:125 (d_expanded_input.view(T,k,d).sum(-2))
 * plus up to two addends (gate and shared-expert input grads):
 *   out[t, :] = sum_j Xe[t*k + j, :] + add0[t, :] + add1[t, :]
 * summed in fp32; out_dtype `dtype`, or F32 for BF16 rows (the sum unrounded: the
 * input grad of an fp32 residual stream under bf16 autocast).                 */
int zmoe_sum_k(const void* Xe, int64_t T, int k, int64_t d, int dtype,
               const void* add0, const void* add1, int out_dtype, void* out, void* stream);

/* The bf16 compute copy of fp32 master weights (the cast torch autocast applies to
 * fp32 parameters, main.py:595, :746): dst[i] = bf16(src[i]), round to nearest
 * even, NaN kept. src and dst 16-byte aligned. */
int zmoe_cast_f32_bf16(const float* src, int64_t n, void* dst, void* stream);

/* scattermoe/mlp.py:86 stand-alone (shapes the fused kernels reject):
 * A = silu(H[:, f:]) * H[:, :f]; and its backward dH from (dA, H), rows of dH
 * ld_dh >= 2f elements apart (2f for a packed [R, 2f]). */
int zmoe_swiglu(const void* H, int64_t R, int64_t f, int dtype, void* A, void* stream);
int zmoe_swiglu_backward(const void* dA, const void* H, int64_t R, int64_t f,
                         int dtype, void* dH, int64_t ld_dh, void* stream);

/* The SwiGLU backward of gate-scaled rows with the gates' grad (the combine backward
 * of parallel_experts.py:80-97 reassociated, as in zmoe_glu_w2_backward_dh_gates,
 * after a plain dA GEMM on the output grad's rows), per sorted row r:
 *   dH[r] = swiglu_backward(row_scale[r] * dA[r], H[r])
 *   d_gates[slot_of_row[r]] = sum_j dA[r, j] * silu(H[r, f + j]) * H[r, j]
 * dA [R, f], H and dH [R, 2f] packed; d_gates [R] f32 written in slot order. */
int zmoe_swiglu_backward_gates(const void* dA, const void* H, int64_t R, int64_t f,
                               const float* row_scale, const int64_t* slot_of_row,
                               int dtype, void* dH, float* d_gates, void* stream);

/* main.py:161-175 (aux-loss-free bias update) from the sort's offsets:
 *   counts = diff(expert_offsets); b += rate * sign(mean(counts) - counts)    */
int zmoe_bias_update(const int64_t* expert_offsets, int E, float update_rate,
                     float* expert_biases, void* stream);

/* ---------------------------------------------------------------------------
 * ZeroCenteredRMSNorm (modeling/zRMSNorm.py:10-17) fused with the unpad gather
 * that follows it (modeling/transformer_block.py:41-42 normalises, then
 * modeling/moe_layer.py:39-42 gathers the valid tokens with index_first_axis):
 *   Y[i] = X[rows[i]] * rsqrt(mean_j X[rows[i], j]^2 + eps) * (1 + w)
 * in fp32, stored in X's dtype. X [x_rows, x_stride]; rows [n] int64 (NULL:
 * rows[i] = i; a row outside [0, x_rows) gives a zero output row); Y [n, d]
 * contiguous; rstd [n] fp32 (nullable) receives each row's rsqrt, which the
 * backward needs. weight [d] in w_dtype (F32 or BF16). d <= 16384 (bf16) /
 * 8192 (f32), a multiple of 8 (bf16) or 4 (f32) elements.
 * ------------------------------------------------------------------------- */
int zmoe_rmsnorm_rows(const void* X, int64_t x_stride, int64_t x_rows, const int64_t* rows, int64_t n,
                      int64_t d, const void* weight, int w_dtype, float eps, int dtype, void* Y,
                      float* rstd, void* stream);

/* Backward of zmoe_rmsnorm_rows (the autograd of zRMSNorm.py:10-17 and of the
 * gather): dX[rows[i]] = r (1 + w) dY[i] - X[rows[i]] r^3 / d * sum_j dY[i,j] (1 + w_j) X[rows[i],j]
 * with r = rstd[i]; the caller zero-fills dX [x_rows, dx_stride] (rows outside
 * the gather keep their zeros; rows must be distinct, as unpad indices are).
 * dweight[j] = sum_i dY[i,j] X[rows[i],j] r_i in w_dtype, from fp32 partials
 * summed in a fixed order (deterministic). Workspace:
 * zmoe_rmsnorm_rows_backward_workspace_bytes(n, d, dtype), 16-byte aligned. */
size_t zmoe_rmsnorm_rows_backward_workspace_bytes(int64_t n, int64_t d, int dtype);
int zmoe_rmsnorm_rows_backward(const void* dY, const void* X, int64_t x_stride, int64_t x_rows,
                               const int64_t* rows, int64_t n, int64_t d, const float* rstd,
                               const void* weight, int w_dtype, int dtype, void* dX, int64_t dx_stride,
                               void* dweight, void* workspace, size_t workspace_bytes, void* stream);

/* optimizer/muon.py:6-32 (zeropower_via_newtonschulz5) on a stack of E matrices,
 * the orthogonalisation inside the MuonMD step on 3-D expert weights
 * (muon.py:399-508, called at :449). X [E, m, n] bf16, contiguous, m <= n (the
 * caller transposes a tall stack first, as muon.py:18-19 does), updated in place:
 *   X = X / (||X||_F + 1e-7);  repeat steps: A = X X^T; B = b A + (c A) A; X = a X + B X
 * with bf16 rounding after every product and sum, as in bf16 tensor arithmetic.
 * Any E: the stack runs in passes of at most min(1024, (2 GiB - 64 KiB) / (2 m n))
 * matrices over one pass-sized workspace (one matrix must span less than that).
 * Workspace: zmoe_newton_schulz5_workspace_bytes(E, m, n), 256-byte aligned (0 when
 * one matrix spans 2 GiB - 64 KiB or more, or a size is below 1).                  */
size_t zmoe_newton_schulz5_workspace_bytes(int64_t E, int64_t m, int64_t n);
int zmoe_newton_schulz5(void* X, int64_t E, int64_t m, int64_t n, int steps, float a, float b, float c,
                        void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ZMOE_H_ */
