/*
 * mt_flce.h -- C ABI of the MI355X (gfx950) fused LM-head linear + per-token
 * cross-entropy library (libmt_flce.so).
 *
 * The library replaces the arithmetic that mini_trainer reaches through
 *   none_reduction_losses.py:5-25  liger_fixed_fused_linear_cross_entropy_none_reduction
 *     -> liger_kernel.transformers.functional.liger_fused_linear_cross_entropy(
 *            reduction='none', ignore_index, softcap)        (none_reduction_losses.py:16-23)
 * i.e. loss[t] = logsumexp_v(x_t . w_v) - x_t . w_{y_t}, and +0.0 where
 * y_t == ignore_index, without materialising the [T, V] logits, plus the
 * gradients w.r.t. hidden states and lm_head weight for an arbitrary
 * per-token upstream gradient (train.py:97-104 supplies a uniform one).
 *
 * Conventions
 *   - Every tensor is owned by the caller (PyTorch).  Pointers are device
 *     pointers; sizes are element counts.  The library never allocates and
 *     never frees device memory: scratch space is a caller-provided
 *     workspace whose size is returned by the *_workspace_bytes queries.
 *   - Every entry point is asynchronous on the caller's stream and never
 *     synchronises.  Errors found on the host come back as a non-zero status;
 *     errors that can only be found on the device (labels out of range,
 *     malformed cu_seqlens) are written to a caller-provided device word that
 *     the caller reads when it next synchronises.
 *   - Return value 0 == MT_OK.  mt_flce_last_error() returns a thread-local,
 *     human-readable description of the last non-zero status.
 *   - Layouts: X [T, H] with leading dimension ldx (elements), W [V, H] with
 *     leading dimension ldw, both row-major with unit stride along H.
 *     Row pitches (ldx, ldw times the element size) must be multiples of 16
 *     bytes and the base pointers 16-byte aligned; H must be a multiple of 8
 *     (bf16) or 4 (fp32), i.e. whole 16-byte chunks -- a partial last K
 *     stage is masked inside the kernels.  dtype selects bf16 (MFMA path) or fp32
 *     inputs; loss / lse / dW are always fp32, dX has the dtype of X.
 *   - mt_flce_fused and the bf16 mt_flce_backward run dW beside dX in one
 *     launch on the caller's stream (dX's workgroups dispatched first, dW's
 *     on the CUs dX leaves free and then the rest).  Measurement hook:
 *     MT_FLCE_SPLIT_PHASE=1 launches them as two kernels instead, dW on a
 *     second stream of the library's own (one per device, created on first
 *     use, default priority) forked from and joined back to the caller's
 *     stream with events inside the call, so that each has its own timing
 *     events and counters; either way the call stays ordered on the
 *     caller's stream.
 *   - Test hook: the environment variable MT_FLCE_GRID_CAP=n (> 0) caps the
 *     persistent bf16 GEMM grids (logits, recompute) and the dW grids at n
 *     workgroups, and the general backward takes n as the CU count when it
 *     decides whether dW runs beside dX, so small problems exercise the
 *     multi-tile schedules; dX always runs one workgroup per output tile.
 *     Unset in production.
 */
#ifndef MT_FLCE_H
#define MT_FLCE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MT_FLCE_ABI_VERSION 7

typedef struct ihipStream_t* mt_stream_t; /* == hipStream_t */

enum mt_dtype { MT_DTYPE_F32 = 0, MT_DTYPE_BF16 = 1 };

enum mt_status {
  MT_OK = 0,
  MT_ERR_INVALID_ARGUMENT = 1,
  MT_ERR_WORKSPACE_TOO_SMALL = 2,
  MT_ERR_UNSUPPORTED = 3,
  MT_ERR_HIP = 4
};

/* Library version of this header; mt_flce_abi_version() must equal it. */
int mt_flce_abi_version(void);

/* Thread-local text for the last non-zero status on this thread. */
const char* mt_flce_last_error(void);

/*
 * Valid-row compaction and label check.
 * Replaces the host-side pass of the reference's fused loss that counts the
 * non-ignored targets ((target != ignore_index).sum().item() inside
 * LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_forward,
 * reached from none_reduction_losses.py:16-23), and, with shift != 0, the
 * label shift of TF/loss/loss_utils.py:61-64 (target[t] = labels[t+1],
 * target[T-1] = ignore_index).
 *   labels     int64 [T] (device)
 *   row_index  int32 [T] out: positions t of valid rows, ascending, first N used
 *   row_label  int32 [T] out: their labels
 *   counts     int32 [4] out (device): {N, #labels outside [0,V), first bad t or -1, 0}
 * One workgroup; no synchronisation.  The caller reads counts (one 16-byte
 * device->host copy, the single sync of a training step) to size the rest.
 */
int mt_flce_prepare(const int64_t* labels, int64_t T, int64_t V,
                    int64_t ignore_index, int shift, int32_t* row_index,
                    int32_t* row_label, int32_t* counts, mt_stream_t stream);

/* Workspace for mt_flce_forward (bytes). */
size_t mt_flce_forward_workspace_bytes(int64_t T, int64_t n_valid, int64_t H,
                                       int64_t V, int dtype);

/*
 * Forward: per-token loss and per-valid-row log-sum-exp.
 * Replaces LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_forward
 * (chunk loop of X_c @ W^T + liger_cross_entropy_kernel, reduction='none'),
 * called from none_reduction_losses.py:16-23, with the semantics of
 * F.linear -> .float() -> F.cross_entropy(reduction='none')
 * (none_reduction_losses.py:35, TF/loss/loss_utils.py:59).
 *   loss  fp32 [T] out: lse_t - logit_{t,y_t}; exactly +0.0 at ignored rows
 *   lse   fp32 [n_valid] out: log-sum-exp of valid row i = row_index[i]
 *   softcap > 0 applies logits = softcap * tanh(logits / softcap)
 *           (final_logit_softcapping, none_reduction_losses.py:11,22); 0 = off.
 */
int mt_flce_forward(const void* X, const void* W, int64_t T, int64_t H,
                    int64_t V, int64_t ldx, int64_t ldw, int dtype,
                    float softcap, const int32_t* row_index,
                    const int32_t* row_label, int64_t n_valid, float* loss,
                    float* lse, void* workspace, size_t workspace_bytes,
                    mt_stream_t stream);

/*
 * mt_flce_forward (bf16, softcap off) that also keeps, for the backward,
 * the exponentials exp(logit) (rounded to bf16) of vocabulary columns
 * [0, keep_cols) of every valid row: keep receives them as rows of keep_cols
 * entries (round_up(n_valid, 256) rows, keep_bytes >= that times keep_cols
 * times 2), keep_cols a multiple of 256 below V.  *guard (a device int32) is
 * reset and then raised if some row's largest logit lies outside the range
 * in which those exponentials hold their terms ([-48, 48]).  Handing keep
 * (as the G block of the backward's workspace, keep_cols = chunk_vocab) and
 * guard to mt_flce_backward_narrow spares that block's recomputation: the
 * forward already computes every logit once (the Liger forward reached from
 * none_reduction_losses.py:16-23 keeps its chunk's logits for the same
 * reason).  Same loss and lse as mt_flce_forward, bit for bit.
 */
int mt_flce_forward_keep(const void* X, const void* W, int64_t T, int64_t H,
                         int64_t V, int64_t ldx, int64_t ldw, int dtype,
                         float softcap, const int32_t* row_index,
                         const int32_t* row_label, int64_t n_valid,
                         float* loss, float* lse, void* workspace,
                         size_t workspace_bytes, void* keep, int64_t keep_cols,
                         size_t keep_bytes, int32_t* guard, mt_stream_t stream);

/*
 * Bytes one bf16 operand buffer may span (the kernels address X, the
 * weight's vocabulary blocks, G, the fused logits chunk and X^T with 32-bit
 * offsets): 4 GiB - 1, lowered by the test hook MT_FLCE_MAX_BUFFER_BYTES.
 * bf16 X beyond it is rejected (MT_ERR_UNSUPPORTED: the caller splits the
 * call over row ranges); a weight beyond it runs in vocabulary blocks on
 * mt_flce_forward / mt_flce_backward, and mt_flce_fused rejects it.
 * No counterpart in the reference.
 */
uint64_t mt_flce_max_buffer_bytes(void);

/*
 * Forward without allocation (no counterpart in the reference): the same
 * results as mt_flce_forward -- bit-identical for bf16 -- for callers that
 * cannot allocate device memory or hand the library a workspace (code under
 * HIP graph capture, tight serving and evaluation loops, harnesses that
 * forbid hipMalloc; under capture, with the library's profiling hook off
 * and after one call on the device outside the capture, which looks the
 * scratch's address up).  Its scratch (the forward's (max, sum) partials and
 * label logits) is a static device array of mt_flce_noalloc_scratch_bytes()
 * bytes (16 MiB) per GPU, held until the process ends; valid rows are
 * processed in chunks that fit it.  A V whose single row of partials does
 * not fit is rejected with MT_ERR_UNSUPPORTED.  The call allocates and frees
 * nothing.  Every call on one GPU shares that GPU's scratch, which keeps the
 * last call's contents (nothing in it needs clearing: each chunk writes what
 * it reads), so calls that overlap on one GPU -- on different streams, or
 * from different host threads -- race; serialise them.
 */
size_t mt_flce_noalloc_scratch_bytes(void);
int mt_flce_forward_noalloc(const void* X, const void* W, int64_t T, int64_t H,
                            int64_t V, int64_t ldx, int64_t ldw, int dtype,
                            float softcap, const int32_t* row_index,
                            const int32_t* row_label, int64_t n_valid,
                            float* loss, float* lse, mt_stream_t stream);

/*
 * Backward blocking plan.  The backward recomputes logit tiles block by
 * block (chunk_rows valid tokens x chunk_vocab vocabulary entries); this
 * picks the largest blocks whose workspace fits budget_bytes (0 = default:
 * 5% of T*V*sizeof(dtype)).  Writes the block shape and workspace size.
 */
int mt_flce_backward_plan(int64_t T, int64_t n_valid, int64_t H, int64_t V,
                          int dtype, size_t budget_bytes, int64_t* chunk_rows,
                          int64_t* chunk_vocab, size_t* workspace_bytes);

/*
 * The blocking plan of a bf16 backward whose weight gradient is wanted in
 * bf16 and not added into anything (autograd's lm_head gradient,
 * none_reduction_losses.py:35 through its backward).  When one row block
 * (chunk_rows >= n_valid) fits the budget and its cost model ranks it first,
 * the caller runs mt_flce_backward_narrow with it: every dW tile contracts
 * all valid rows at once and is written once, in bf16 -- no read-modify-
 * write of an fp32 dW, no narrowing pass -- and dX's fp32 accumulator and
 * X^T live in the scratch buffer of mt_flce_narrow_scratch_bytes (in the
 * room a bf16 gradient leaves of the fp32 one the budget counts), so the
 * workspace holds only the G block and counters.  Otherwise (chunk_rows < n_valid) the caller runs
 * mt_flce_backward_tiles and mt_flce_narrow_tiles with the same blocking
 * and workspace.  Same arguments and outputs as mt_flce_backward_plan.  (No
 * reference counterpart: the blocking of the backward that replaces
 * LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_backward.)
 */
int mt_flce_backward_narrow_plan(int64_t T, int64_t n_valid, int64_t H,
                                 int64_t V, int dtype, size_t budget_bytes,
                                 int64_t* chunk_rows, int64_t* chunk_vocab,
                                 size_t* workspace_bytes);

/*
 * Backward: dX = G W and dW (+)= G^T X with
 *   G[t, v] = g_t * (softmax(logits_t)[v] - [v == y_t]) (times the softcap
 *   derivative when softcap > 0), G = 0 on ignored rows.
 * Replaces LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_backward
 * (+ element_mul_kernel), which is exact only for a uniform grad_output;
 * this one takes a per-token upstream gradient.
 *   grad_loss    fp32, element t at grad_loss[t * grad_stride] (stride 0 = one
 *                scalar broadcast to every token, as train.py:102 produces)
 *   dX           [T, H] (dtype of X, leading dimension lddx) out; rows of
 *                ignored tokens are written as zeros
 *   dW           fp32 [V, H] (leading dimension lddw) out;
 *                accumulate_dW != 0 adds into it, else it is overwritten
 *   chunk_rows / chunk_vocab / workspace from mt_flce_backward_plan.
 */
int mt_flce_backward(const void* X, const void* W, int64_t T, int64_t H,
                     int64_t V, int64_t ldx, int64_t ldw, int dtype,
                     float softcap, const int32_t* row_index,
                     const int32_t* row_label, int64_t n_valid,
                     const float* lse, const float* grad_loss,
                     int64_t grad_stride, void* dX, int64_t lddx, float* dW,
                     int64_t lddw, int accumulate_dW, int64_t chunk_rows,
                     int64_t chunk_vocab, void* workspace,
                     size_t workspace_bytes, mt_stream_t stream);

/*
 * Fused forward + backward plan (bf16 only): the largest chunk of valid rows
 * (multiple of 256) whose workspace -- the chunk's bf16 exponentials [chunk,
 * round_up(V, 256)], the (max, sum) partials, the label logits, the chunk's
 * X^T, its row factors and a few counters -- fits budget_bytes (0 = default:
 * 5% of T*V*2), then evened out over
 * the chunks.  Writes the chunk size, the workspace size and *pays = 1 if
 * a cost model expects the fused path to beat the general one under the
 * same budget, else 0: small budgets force small chunks, with few long dX
 * tiles and one dW read-modify-write per chunk, which the general path's
 * two-dimensional blocking avoids.  with_accumulator != 0: the weight
 * gradient is added into an fp32 accumulator, and the general path priced
 * is mt_flce_forward + mt_flce_backward; 0: it is wanted in bf16, and the
 * general path priced is the one mt_flce_backward_narrow_plan plans (one
 * row block through mt_flce_backward_narrow after mt_flce_forward_keep, or
 * mt_flce_backward_tiles and the narrowing pass).
 */
int mt_flce_fused_plan(int64_t T, int64_t n_valid, int64_t H, int64_t V,
                       int dtype, size_t budget_bytes, int with_accumulator,
                       int64_t* chunk_rows, size_t* workspace_bytes,
                       int* pays);

/*
 * Fused forward + backward for a caller that knows the upstream gradient of
 * every token before the forward -- as train.py:97-104 does: it scales the
 * summed loss by world_size / batch_num_loss_counted_tokens, a number fixed
 * by the batch.  Produces loss and lse as mt_flce_forward, dX and dW as
 * mt_flce_backward would for that gradient, with 6*H*V*n_valid flops (each
 * logits tile is computed once and kept in bf16 for its chunk, the structure
 * of LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_forward
 * reached from none_reduction_losses.py:16-23, which computes the gradients
 * in its forward and rescales them in its backward).
 *   grad_loss / grad_stride  as in mt_flce_backward
 *   chunk_rows / workspace   from mt_flce_fused_plan
 * bf16 only (MT_ERR_UNSUPPORTED otherwise).
 */
int mt_flce_fused(const void* X, const void* W, int64_t T, int64_t H, int64_t V,
                  int64_t ldx, int64_t ldw, int dtype, float softcap,
                  const int32_t* row_index, const int32_t* row_label,
                  int64_t n_valid, const float* grad_loss, int64_t grad_stride,
                  float* loss, float* lse, void* dX, int64_t lddx, float* dW,
                  int64_t lddw, int accumulate_dW, int64_t chunk_rows,
                  void* workspace, size_t workspace_bytes, mt_stream_t stream);

/*
 * mt_flce_backward with dW formed as 256 x 256 fp32 tiles in the two buffers
 * of mt_flce_dw_tiles_layout instead of rows, bf16 only: the same
 * arithmetic, so mt_flce_narrow_tiles of the result equals mt_flce_backward
 * + mt_flce_scale_grads bit for bit.  accumulate_dW != 0 adds into the
 * tiles already there (a call split over row ranges), else they are
 * overwritten.  Replaces the same reference interface as mt_flce_backward
 * (the lm_head backward's dW = dS^T X, none_reduction_losses.py:35 through
 * autograd).
 */
int mt_flce_backward_tiles(const void* X, const void* W, int64_t T, int64_t H,
                           int64_t V, int64_t ldx, int64_t ldw, int dtype,
                           float softcap, const int32_t* row_index,
                           const int32_t* row_label, int64_t n_valid,
                           const float* lse, const float* grad_loss,
                           int64_t grad_stride, void* dX, int64_t lddx,
                           void* dW_lo, size_t dw_lo_bytes, float* dW_hi,
                           size_t dw_hi_bytes, int accumulate_dW,
                           int64_t chunk_rows, int64_t chunk_vocab,
                           void* workspace, size_t workspace_bytes,
                           mt_stream_t stream);

/*
 * mt_flce_backward for one row block (chunk_rows >= n_valid, from
 * mt_flce_backward_narrow_plan) whose weight gradient is written in bf16,
 * bf16 only, H a multiple of 8: dW_out (at least V H 2 bytes, 16-byte
 * aligned) receives the gradient as contiguous bf16 rows [V, H] -- each
 * 256 x 256 tile narrowed once from its fp32 accumulators (round to nearest
 * even).  scratch (mt_flce_narrow_scratch_bytes(V, H, chunk_rows) bytes; may
 * be NULL when that is 0) holds dX's fp32 accumulator and the block's X^T
 * for the duration of the call: the plan puts them there when they fit in
 * the V H 2 bytes that a bf16 gradient leaves of an fp32 one, so the call's
 * peak is that of an fp32 weight gradient, and the weight gradient is the
 * right size afterwards.  Bit for bit what mt_flce_backward_tiles and
 * mt_flce_narrow_tiles with a unit scale give for the same blocking.
 *   kept_guard   NULL, or (softcap off, chunk_vocab < V) the guard word of an
 *                mt_flce_forward_keep call that kept keep_cols = chunk_vocab
 *                columns in this workspace's first bytes (the G block): the
 *                first vocabulary block then takes its G from those
 *                exponentials instead of recomputing its logits, unless the
 *                guard was raised.
 * Replaces the same reference interface as mt_flce_backward (the lm_head
 * backward's dW = dS^T X, none_reduction_losses.py:35 through autograd).
 */
int mt_flce_backward_narrow(const void* X, const void* W, int64_t T, int64_t H,
                            int64_t V, int64_t ldx, int64_t ldw, int dtype,
                            float softcap, const int32_t* row_index,
                            const int32_t* row_label, int64_t n_valid,
                            const float* lse, const float* grad_loss,
                            int64_t grad_stride, void* dX, int64_t lddx,
                            void* dW_out, size_t dw_out_bytes, void* scratch,
                            size_t scratch_bytes, int64_t chunk_rows,
                            int64_t chunk_vocab, void* workspace,
                            size_t workspace_bytes, const int32_t* kept_guard,
                            mt_stream_t stream);

/*
 * Bytes of the scratch buffer mt_flce_backward_narrow needs for one row
 * block of chunk_rows (0: dX's accumulator and X^T stay in the workspace,
 * or bad sizes).  No counterpart in the reference.
 */
size_t mt_flce_narrow_scratch_bytes(int64_t V, int64_t H, int64_t chunk_rows);

/*
 * Layout of the tiled fp32 weight gradient that mt_flce_fused_tiles and
 * mt_flce_backward_tiles form: ceil(V/256) x ceil(H/256) tiles of 256 x 256
 * fp32 in the order the dW GEMM holds them, row-major over the tile grid,
 * over two caller buffers.  dW_lo is the weight gradient's own buffer of
 * *lo_bytes = V H 2 bytes (a bf16 [V, H]): after a pad of 256 *
 * round_up(H, 256) bf16 elements it holds tile rows [0, *lo_tile_rows);
 * dW_hi (*hi_bytes, 0 when every tile row fits in dW_lo) holds the rest.
 * mt_flce_narrow_tiles narrows the gradient into dW_lo in place, after
 * which dW_hi can be freed: the weight gradient then occupies exactly the
 * V H 2 bytes of a bf16 tensor, while the two buffers together hold the
 * fp32 gradient the kernels accumulate.  No counterpart in the reference.
 */
int mt_flce_dw_tiles_layout(int64_t V, int64_t H, size_t* lo_bytes,
                            int64_t* lo_tile_rows, size_t* hi_bytes);

/*
 * mt_flce_fused with dW formed as tiles in the two buffers of
 * mt_flce_dw_tiles_layout instead of rows: every load and store of the dW
 * GEMM's accumulators is one contiguous KiB, without the transpose a
 * row-major tile edge needs.  Same arithmetic, so mt_flce_narrow_tiles of
 * the result equals mt_flce_fused + mt_flce_scale_grads bit for bit.
 * accumulate_dW != 0 adds into the tiles already there (a call split over
 * row ranges), else they are overwritten.  Replaces the same reference
 * interface as mt_flce_fused (none_reduction_losses.py:16-23 -> LIGER's
 * fused_linear_cross_entropy_forward, whose grad_weight is the tensor here).
 */
int mt_flce_fused_tiles(const void* X, const void* W, int64_t T, int64_t H,
                        int64_t V, int64_t ldx, int64_t ldw, int dtype,
                        float softcap, const int32_t* row_index,
                        const int32_t* row_label, int64_t n_valid,
                        const float* grad_loss, int64_t grad_stride, float* loss,
                        float* lse, void* dX, int64_t lddx, void* dW_lo,
                        size_t dw_lo_bytes, float* dW_hi, size_t dw_hi_bytes,
                        int accumulate_dW, int64_t chunk_rows, void* workspace,
                        size_t workspace_bytes, mt_stream_t stream);

/*
 * scale * tiled dW (the two buffers of mt_flce_dw_tiles_layout) -> the
 * weight gradient in bf16, rows [V, H] of pitch H in place in dW_lo; the
 * tiled counterpart of mt_flce_scale_grads's dW part (LIGER's
 * fused_linear_cross_entropy_backward: grad_weight times grad_output[0]).
 * The tile rows are narrowed in launches {0}, {1}, [2, 4), [4, 8), ... so
 * that none is overwritten before it is read; dW_hi is only read, and can
 * be freed once the stream has passed this call.  bf16 output, H % 8 == 0;
 * rounds to nearest even.  scale fp32 [1] on the device.
 */
int mt_flce_narrow_tiles(const float* scale, void* dW_lo, size_t dw_lo_bytes,
                         const float* dW_hi, size_t dw_hi_bytes, int64_t V,
                         int64_t H, mt_stream_t stream);

/*
 * Per-sample sums over a packed batch (no counterpart in the reference, which
 * only sums the whole minibatch at train.py:98; sample boundaries follow the
 * packed layout of sampler.py:182-188 and the cu_seqlens derivation of
 * TF/modeling_flash_attention_utils.py:458-481).
 *   cu_seqlens int32 [S+1], non-decreasing, cu[0] = 0, cu[S] = T
 *   shift      0: position t's target is target[t]; != 0: it is target[t + 1]
 *              (ignore_index at t = T - 1), the causal shift of
 *              TF/loss/loss_utils.py:61-64 applied to unshifted labels
 *   seg_loss   fp32 [S] out: sum of loss over [cu[s], cu[s+1])
 *   seg_count  int32 [S] out: number of t in that range whose target != ignore_index
 *   status     int32 [1] out (device): 0, or 1 if cu_seqlens is malformed
 *              (then seg_loss / seg_count are zero)
 */
int mt_segment_sum(const float* loss, const int64_t* target, int64_t T,
                   int64_t ignore_index, int shift, const int32_t* cu_seqlens,
                   int64_t S, float* seg_loss, int32_t* seg_count,
                   int32_t* status, mt_stream_t stream);

/*
 * Rescale gradients formed for a unit upstream gradient once the real
 * (uniform) one is known: dX *= scale in place, dW_out = scale * dW.
 * Replaces the backward of the reference's fused loss,
 * LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_backward
 * (element_mul_kernel: grad_input and grad_weight times grad_output[0]),
 * reached from none_reduction_losses.py:16-23 -- the gradients were formed
 * in the forward (mt_flce_fused with grad_loss = 1, grad_stride = 0).
 *   scale      fp32 [1] (device): read by the kernels, no host sync
 *   dX         [T, H] of dtype_x, leading dimension lddx, scaled in place
 *   dW         fp32 [V, H], leading dimension lddw
 *   dW_out     [V, H] of dtype_out, leading dimension ldo: a separate buffer
 *              (it may not partially overlap dW), or dW itself (ldo == lddw):
 *              fp32 is then scaled in place, and bf16 is narrowed in place --
 *              bf16 row r goes to element offset r * ldo (bf16 units) from
 *              dW's base, i.e. the first half of dW's bytes when lddw == H,
 *              so the weight gradient in the weight's dtype needs no second
 *              allocation (H <= 16384; rows are processed in launches of
 *              doubling length so that no fp32 row is overwritten before it
 *              is read).  bf16 output rounds to nearest even.
 * Base pointers 16-byte aligned; row pitches multiples of 16 bytes (of 8
 * bytes for a bf16 dW_out).  T = 0 or V = 0 skips that tensor.
 */
int mt_flce_scale_grads(const float* scale, void* dX, int64_t T, int64_t H,
                        int64_t lddx, int dtype_x, const float* dW, int64_t V,
                        int64_t lddw, void* dW_out, int64_t ldo, int dtype_out,
                        mt_stream_t stream);

/*
 * Measurement hook (no counterpart in the reference; for benchmarks and
 * profilers).  While enabled, every kernel launch of mt_flce_forward,
 * mt_flce_backward, mt_flce_fused and mt_flce_scale_grads made on the device
 * that was current at enable time is bracketed by two timing events on the
 * stream it runs on, tagged with the kernel's name and algorithmic work
 * (flops of the unpadded GEMM, or bytes of an HBM pass); the dX and dW
 * GEMMs that run side by side are also recorded as one "dx_dw_phase" from
 * the fork to the join.  mt_flce_profile_report synchronises on the recorded
 * events, writes a JSON object {name: {launches, ms_total, ms_min, ms_max,
 * flops, bytes}} into buf (needed = its size including the terminating
 * zero; MT_ERR_INVALID_ARGUMENT if len is smaller, keeping the records for
 * a retry with a larger buffer) and releases the records.
 * Call the report only when no call of this library is in flight.
 */
int mt_flce_profile_enable(int enable);
int mt_flce_profile_report(char* buf, size_t len, size_t* needed);

/*
 * Measurement hook (no counterpart in the reference): the ceiling the GEMM
 * kernels are measured against -- a register-only stream of bf16 MFMAs on
 * `workgroups` workgroups of 256 threads, one per CU (each reserves the
 * whole LDS), every wave iters x (shape 0: 64 v_mfma_f32_16x16x32_bf16, the
 * GEMM kernels' instruction; 1: 16 v_mfma_f32_32x32x16_bf16) on independent
 * accumulators (2^20 and 2^19 flops per wave and iteration).  operands:
 * workgroups x 256 x 16 x 16 bytes of bf16 operand values (device, 16-byte
 * aligned, loaded once); out: workgroups x 256 fp32 (the accumulator sums).
 * No memory traffic inside the loop.  Asynchronous on stream.
 */
int mt_flce_probe_mfma(int shape, int64_t workgroups, int32_t iters,
                       const void* operands, float* out, mt_stream_t stream);

/*
 * Cross-entropy over materialised logits, reduction 'none' -- the HF slot of
 * the reference, hf_fixed_cross_entropy_none_reduction
 * (none_reduction_losses.py:27-36 -> F.cross_entropy(source, target,
 * ignore_index, reduction='none') at :35), with source = logits.float()
 * (TF/loss/loss_utils.py:59).
 *   logits  [T, V] (dtype: fp32 or bf16, computed in fp32), leading dimension ld
 *   loss    fp32 [T] out (+0.0 at ignored rows);  lse fp32 [T] out (0 at ignored)
 *   status  int32 [1] out (device): 1 if some target lies outside [0, V) and is
 *           not ignore_index (that row then gets loss 0)
 */
int mt_ce_forward(const void* logits, int64_t T, int64_t V, int64_t ld, int dtype,
                  const int64_t* target, int64_t ignore_index, float* loss, float* lse,
                  int32_t* status, mt_stream_t stream);

/* dlogits[t, v] = g_t * (softmax(logits_t)[v] - [v == y_t]), 0 on ignored rows;
 * written in the logits dtype with leading dimension ldd. */
int mt_ce_backward(const void* logits, int64_t T, int64_t V, int64_t ld, int dtype,
                   const int64_t* target, int64_t ignore_index, const float* lse,
                   const float* grad_loss, int64_t grad_stride, void* dlogits, int64_t ldd,
                   mt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MT_FLCE_H */
