/*
 * mirl.h — C ABI of libmirl.so, the MI355X (gfx950) token-logprob and
 * clipped-policy-gradient hot path.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are raw device pointers plus element strides.  The
 *     vocabulary (last) dimension of a logits tensor must be unit-stride; the
 *     Python layer calls .contiguous() when it is not.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Every call only
 *     enqueues work on that stream: no device synchronisation, no host copies,
 *     and no device memory allocation.  Scratch memory, when a kernel needs it,
 *     is passed in by the caller.
 *   - Every function returns MIRL_OK (0) or a non-zero status.  The message of
 *     the last failure on the calling thread is available from
 *     mirl_last_error().  No entry point aborts or exits.
 *   - Row r of a [B, R, V] logits tensor is the logits of sequence position r.
 *     Row (b, r) is paired with target (b, r); callers that want next-token
 *     logprobs pass a target view shifted by one position (ids[:, 1:]).
 *
 * The reference implementation this replaces is pure PyTorch; each function
 * below names the reference code (path:line inside the NeMo-RL tree) whose
 * semantics it reproduces.
 */
#ifndef MIRL_H
#define MIRL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MIRL_OK 0
#define MIRL_ERR_INVALID_ARGUMENT 1
#define MIRL_ERR_HIP 2
#define MIRL_ERR_UNSUPPORTED 3

/* element types of logits / gradient tensors */
#define MIRL_DTYPE_F32 0
#define MIRL_DTYPE_BF16 1
#define MIRL_DTYPE_F16 2
/* element type of the per-token loss tensors (ClippedPG) */
#define MIRL_DTYPE_F64 3

/* Last error message on the calling thread ("" when none). */
const char* mirl_last_error(void);

/* Library version string, e.g. "mirl 0.1.0 gfx950". */
const char* mirl_version(void);

/*
 * Selected-token log-probabilities, one row per (b, r):
 *   m        = max_v x[v]
 *   logsum   = log(sum_v exp(x[v] - m))
 *   out[b,r] = (x[t'] - m) - logsum      where t' = target - vocab_start,
 *   out[b,r] = 0                          when target < vocab_start or >= vocab_end.
 * Arithmetic is fp32 for every input dtype; one read of the logits row.
 * If `row_stats` is non-NULL it receives {m, logsum} per row (2 floats, row
 * major [B, R, 2]) for mirl_logprob_bwd.
 *
 * Replaces: nemo_rl/distributed/model_utils.py:87-135
 * (_compute_distributed_selected_logprobs), the per-chunk forward of
 * ChunkedDistributedLogprob (model_utils.py:240-290) and the forward of
 * DistributedLogprob (model_utils.py:145-182) with a vocab group of size 1.
 */
int mirl_logprob_fwd(const void* logits, int dtype, int64_t B, int64_t R,
                     int64_t V, int64_t stride_b, int64_t stride_r,
                     const int64_t* target, int64_t t_stride_b,
                     int64_t t_stride_r, int64_t vocab_start,
                     int64_t vocab_end, float* out, float* row_stats,
                     void* stream);

/*
 * Gradient of the selected-token log-probabilities with respect to the logits:
 *   grad[b,r,v] = (onehot(t')[v] - exp((x[v] - m) - logsum)) * g[b,r]
 * written in the logits dtype (round to nearest even).  Rows with r >= R
 * (positions the forward did not compute, up to R_total) and rows whose
 * upstream gradient is exactly zero are written as zeros without reading the
 * logits.  `grad_in` may alias `logits` (in-place, each element is read before
 * it is overwritten by the same thread).
 *
 * Replaces: ChunkedDistributedLogprob.backward (model_utils.py:293-349) and
 * DistributedLogprob.backward (model_utils.py:185-225).
 */
int mirl_logprob_bwd(const void* logits, int dtype, int64_t B, int64_t R,
                     int64_t R_total, int64_t V, int64_t stride_b,
                     int64_t stride_r, const int64_t* target,
                     int64_t t_stride_b, int64_t t_stride_r,
                     int64_t vocab_start, int64_t vocab_end,
                     const float* row_stats, const float* grad_out,
                     int64_t g_stride_b, int64_t g_stride_r, void* grad_in,
                     int64_t gi_stride_b, int64_t gi_stride_r, void* stream);

/*
 * Early-backward check for mirl_logprob_bwd.  A caller that launched
 * mirl_logprob_bwd for an upstream gradient `grad_used` (contiguous fp32
 * [B, R]) before the real upstream gradient `grad_out` was known passes both
 * here: one kernel compares them bit for bit and writes `flag` (device ints,
 * one per checking workgroup, at most MIRL_RECHECK_FLAGS; nonzero = they
 * differ); a second recomputes grad_in from grad_out when any flag is set and
 * returns at once otherwise.  The recomputation leaves the rows whose
 * grad_out equals grad_used (and the rows past R) as the earlier call wrote
 * them, so grad_in must still hold that call's output there.  Arguments as
 * for mirl_logprob_bwd.  row_list (or NULL): B * R int32 of scratch; with it
 * the check also lists the rows that differ (each flag is then its
 * workgroup's count) and the recomputation visits those rows only.
 *
 * Replaces: nothing in the reference (an ordering device: it lets the
 * backward start before the host has synchronised on the loss's metrics).
 */
#define MIRL_RECHECK_FLAGS 64
int mirl_logprob_bwd_recheck(const void* logits, int dtype, int64_t B, int64_t R,
                             int64_t R_total, int64_t V, int64_t stride_b,
                             int64_t stride_r, const int64_t* target,
                             int64_t t_stride_b, int64_t t_stride_r,
                             int64_t vocab_start, int64_t vocab_end,
                             const float* row_stats, const float* grad_out,
                             int64_t g_stride_b, int64_t g_stride_r,
                             const float* grad_used, void* grad_in,
                             int64_t gi_stride_b, int64_t gi_stride_r, int* flag,
                             int32_t* row_list, void* stream);

/*
 * Log-probabilities at K given vocabulary ids per row:
 *   out[b,r,k] = (x[id - vocab_start] - m) - logsum   for vocab_start <= id < vocab_end,
 *   out[b,r,k] = 0                                     otherwise,
 * with m and logsum as in mirl_logprob_fwd (one read of the row; the K
 * re-reads hit the row just streamed).  `indices` is an int64 [B, R, K] view;
 * `out` is a contiguous fp32 [B, R, K] array; `row_stats` (optional) receives
 * {m, logsum} per row for mirl_gather_logprob_bwd.
 *
 * Replaces: ChunkedDistributedGatherLogprob.forward
 * (nemo_rl/distributed/model_utils.py:691-748) with a vocab group of size 1,
 * and the single-device log_softmax + gather of
 * get_policy_logprobs_at_sampler_topk (model_utils.py:1723-1865).
 */
int mirl_gather_logprob_fwd(const void* logits, int dtype, int64_t B, int64_t R,
                            int64_t V, int64_t stride_b, int64_t stride_r,
                            const int64_t* indices, int64_t K,
                            int64_t i_stride_b, int64_t i_stride_r,
                            int64_t i_stride_k, int64_t vocab_start,
                            int64_t vocab_end, float* out, float* row_stats,
                            void* stream);

/* fp32 scratch elements mirl_gather_logprob_bwd needs (one per row). */
int64_t mirl_gather_logprob_workspace_elems(int64_t B, int64_t R);

/*
 * Gradient of mirl_gather_logprob_fwd with respect to the logits:
 *   grad[b,r,v] = -p[v] * sum_k g[b,r,k] + sum_{k : id_k = v, in range} g[b,r,k],
 * p = exp((x - m) - logsum), formed in fp32 (the id terms added in k order
 * after the dense term) and rounded once to the logits dtype.  K must be >= 1.
 * `workspace` holds mirl_gather_logprob_workspace_elems(B, R) floats.
 *
 * Replaces: ChunkedDistributedGatherLogprob.backward (model_utils.py:750-805),
 * whose fp32 gradient autograd rounds to the logits dtype.
 */
int mirl_gather_logprob_bwd(const void* logits, int dtype, int64_t B, int64_t R,
                            int64_t V, int64_t stride_b, int64_t stride_r,
                            const int64_t* indices, int64_t K,
                            int64_t i_stride_b, int64_t i_stride_r,
                            int64_t i_stride_k, int64_t vocab_start,
                            int64_t vocab_end, const float* row_stats,
                            const float* grad_out, int64_t g_stride_b,
                            int64_t g_stride_r, int64_t g_stride_k,
                            float* workspace, void* grad_in,
                            int64_t gi_stride_b, int64_t gi_stride_r,
                            void* stream);

/*
 * mirl_gather_logprob_bwd for a gradient launched early: `grad_used` is the
 * contiguous [B, R, K] upstream gradient an earlier mirl_gather_logprob_bwd
 * already wrote `grad_in` for.  This compares `grad_out` with it bit for bit
 * (`flags`: MIRL_RECHECK_FLAGS ints of scratch, written before they are read)
 * and recomputes grad_in from grad_out only if they differ, without a host
 * synchronisation.  Same arguments otherwise.
 * Replaces: nothing in the reference (it is the device side of an early start
 * of ChunkedDistributedGatherLogprob.backward, model_utils.py:750-805, for a
 * loss that knows its gradient in closed form).
 */
int mirl_gather_logprob_bwd_recheck(const void* logits, int dtype, int64_t B, int64_t R,
                                    int64_t V, int64_t stride_b, int64_t stride_r,
                                    const int64_t* indices, int64_t K,
                                    int64_t i_stride_b, int64_t i_stride_r,
                                    int64_t i_stride_k, int64_t vocab_start,
                                    int64_t vocab_end, const float* row_stats,
                                    const float* grad_out, int64_t g_stride_b,
                                    int64_t g_stride_r, int64_t g_stride_k,
                                    const float* grad_used, int* flags,
                                    float* workspace, void* grad_in,
                                    int64_t gi_stride_b, int64_t gi_stride_r,
                                    void* stream);

/* Bytes of scratch mirl_vocab_topk needs for `rows` rows. */
int64_t mirl_vocab_topk_workspace_bytes(int64_t rows);

/*
 * The k largest logits of each row and their global ids (1 <= k <= V):
 *   values[b,r,i]  = the (i+1)-th largest x[b,r,:] (as fp32, exact),
 *   indices[b,r,i] = vocab_start + its position; equal values are ordered by
 *                    ascending position (the lower id first);
 * both contiguous [B, R, k].  NaN sorts above every number, -0.0 ties +0.0.
 * For k <= 1024 one streaming pass per row; rows with more than 1024
 * candidates at or above the k-th largest lane maximum (many equal values) are
 * redone by an exact radix selection.  Larger k take the exact radix selection
 * of the cut, then a sort of the k entries inside the kernel (in LDS up to
 * 16384 entries, else in the `indices` row itself).  `workspace` holds
 * mirl_vocab_topk_workspace_bytes(B*R).
 *
 * Replaces: distributed_vocab_topk (nemo_rl/distributed/model_utils.py:1867-1935)
 * with a vocab group of size 1 (torch.topk of the fp32 logits + the vocab offset).
 */
int mirl_vocab_topk(const void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                    int64_t stride_b, int64_t stride_r, int k, int64_t vocab_start,
                    float* values, int64_t* indices, void* workspace, void* stream);

/* ---------------------------------------------------------------------- */
/* student / teacher divergences over the full vocabulary                  */
/* ---------------------------------------------------------------------- */

/* kinds of mirl_divergence_fwd / _bwd (p = softmax(student), q = softmax(teacher)) */
#define MIRL_DIV_ENTROPY 0       /* L = sum_v p log p (teacher unused)      */
#define MIRL_DIV_CROSS_ENTROPY 1 /* L = -sum_v p log q                      */
#define MIRL_DIV_REVERSE_KL 2    /* L = sum_v p (log p - log q)             */

/*
 * Per-row divergence L[b,r] (fp32) in one read of the student row (and of the
 * teacher row for the cross entropy and reverse KL).  `row_stats` (optional)
 * receives {m_s, logZ_s, m_t, logZ_t} per row ([B, R, 4] floats) for
 * mirl_divergence_bwd; both tensors share the dtype.
 *
 * Replaces: the forwards of ChunkedDistributedEntropy,
 * ChunkedDistributedCrossEntropyToFixedLogits and
 * ChunkedDistributedReverseKLToFixedLogits
 * (nemo_rl/distributed/model_utils.py:2199-2351, reduction :2377-2434) with a
 * vocab group of size 1.
 */
int mirl_divergence_fwd(int kind, const void* student, const void* teacher,
                        int dtype, int64_t B, int64_t R, int64_t V,
                        int64_t s_stride_b, int64_t s_stride_r,
                        int64_t t_stride_b, int64_t t_stride_r, float* out,
                        float* row_stats, void* stream);

/*
 * Gradient of mirl_divergence_fwd with respect to the student logits:
 *   grad[b,r,v] = (p_v * (w_v - L[b,r])) * g[b,r],
 *   w = log p (entropy), -log q (cross entropy), log p - log q (reverse KL),
 * in fp32, rounded once to the logits dtype.  Rows with g == 0 are written as
 * zeros without reading the logits.
 *
 * Replaces: _chunked_distributed_student_teacher_backward
 * (nemo_rl/distributed/model_utils.py:2437-2499).
 */
int mirl_divergence_bwd(int kind, const void* student, const void* teacher,
                        int dtype, int64_t B, int64_t R, int64_t V,
                        int64_t s_stride_b, int64_t s_stride_r,
                        int64_t t_stride_b, int64_t t_stride_r,
                        const float* out, const float* row_stats,
                        const float* grad_out, int64_t g_stride_b,
                        int64_t g_stride_r, void* grad_in,
                        int64_t gi_stride_b, int64_t gi_stride_r,
                        void* stream);

/* ---------------------------------------------------------------------- */
/* top-k / top-p / temperature-filtered logprobs                            */
/* ---------------------------------------------------------------------- */

/* Kept entries saved per row by the filtered forward for the backward. */
#define MIRL_FILTER_KEEP_CAP 1024
/* Ties listed per 8 KB piece of a row by the filtered backward (its workspace). */
#define MIRL_FILTER_PIECE_TIE_CAP 14

/* Per-row result of the filtered forward.  The kept set is
 * { j : y_j > v_cut || (y_j == v_cut && j >= i_cut) }, y = the (temperature
 * scaled) fp32 value; m is its maximum and logsum = log(sum_kept exp(y - m)).
 * flags: bit 2 set when the row has no kept list (the backward re-reads the
 * row); bit 3 set when a top-p cut decided in the 16-bit dtype was found by
 * the exact one-element-at-a-time sum because the error bounds of the
 * parallel sum did not settle it (informational); other bits internal. */
typedef struct mirl_filter_row_info {
  float m;
  float logsum;
  float v_cut;
  int32_t i_cut;
  int32_t n_kept;
  int32_t flags;
} mirl_filter_row_info;

/*
 * Filtered selected-token logprobs, one row per (b, r):
 *   y = dtype(fl32(float(x) * r)), r = fl32(1.0 / temperature) formed in
 *     double (skipped when temperature == 1): torch's GPU x.div_(temperature)
 *   top-k (top_k > 0): keep y >= k-th largest y, every tie kept;
 *   top-p (top_p < 1): over the kept values in ascending order, ties by
 *     vocabulary index, p = softmax, keep where cumsum(p) > 1 - top_p,
 *     always keeping the maximum.  p_dtype selects the arithmetic:
 *     MIRL_DTYPE_F32: p in fp32 (exp(y - m) * (1 / Z)), the cumulative sum
 *       accumulated in double and rounded to fp32, compared with
 *       fp32(1 - top_p) -- the reference on an fp32 (upcast) tensor;
 *     the logits dtype (BF16/F16): p = dtype(exp(y - m) / Z), the cumulative
 *       sum accumulated one element at a time in fp32 with each partial sum
 *       rounded to the dtype, compared with dtype(fp32(1 - top_p)) -- the
 *       reference on the 16-bit tensor itself;
 *   out[b,r] = (y_t - m) - logsum when target t is kept, else -inf.
 * Writes row_info[B*R] (mirl_filter_row_info) and, for rows with at most
 * MIRL_FILTER_KEEP_CAP kept entries, their vocabulary indices and
 * probabilities into kept_idx / kept_p ([B*R, MIRL_FILTER_KEEP_CAP]).
 * `out` may be NULL (then `target` may be NULL too).
 *
 * Replaces: apply_top_k_top_p / _apply_top_k_top_p_fn / _apply_top_k_only_fn
 * (nemo_rl/algorithms/logits_sampling_utils.py:69-287) followed by the fp32
 * log_softmax and gather of DistributedLogprobWithSampling.forward
 * (nemo_rl/distributed/model_utils.py:382-432) and of the no-group path of
 * get_next_token_logprobs_from_logits (model_utils.py:1702-1718); the optional
 * temperature is the in-place logits.div_ of
 * nemo_rl/models/automodel/train.py:248-262.  The 16-bit p_dtype is limited
 * to vocabularies below 589824 when top_p < 1.
 */
int mirl_filtered_logprob_fwd(const void* logits, int dtype, int64_t B, int64_t R,
                              int64_t V, int64_t stride_b, int64_t stride_r,
                              const int64_t* target, int64_t t_stride_b,
                              int64_t t_stride_r, double temperature, int top_k,
                              double top_p, int p_dtype, float* out, void* row_info,
                              int32_t* kept_idx, float* kept_p, void* stream);

/*
 * Gradient of the filtered logprobs with respect to the raw logits:
 *   g32 = (onehot(t) - p) * g on the kept set, 0 elsewhere,
 *   grad = dtype(fl32(dtype(g32) * fl32(1.0 / temperature)))   (dtype(g32) when
 *   temperature == 1), then, when grad_temperature != 1,
 *   grad = dtype(fl32(grad * fl32(1.0 / grad_temperature))): the backward of an
 *   in-place division of the logits by grad_temperature made before the forward
 *   (mirl_temperature_scale), folded into this write.
 * Rows r >= R (up to R_total) and rows with g == 0 are written as zeros.
 * Rows whose kept list was saved are written without reading the logits.
 * top_k is the forward's: it selects the schedule only (with 1 <= top_k <=
 * 1024 the rows carry kept lists, so the gradient is zeroed in one flat pass
 * and the kept entries stored; otherwise the rows are rewritten whole, each
 * row written once); any value gives the same gradient.
 * workspace (or NULL): mirl_filtered_logprob_bwd_workspace_bytes(dtype, B, R, V)
 * bytes.  With it, rows without kept lists whose logits and gradient rows all
 * start at the same offset from a 16-byte boundary are written in 8 KB pieces
 * in address order; the ties of a cut in rank form are counted and listed
 * there per piece and settled by a per-row pass.  Without it (or for other
 * layouts) a workgroup walks each row.  Either way the gradient is the same.
 * Calls that share a workspace must not overlap.
 *
 * Replaces: DistributedLogprobWithSampling.backward and
 * ChunkedDistributedLogprobWithSampling.backward
 * (nemo_rl/distributed/model_utils.py:434-479, :624-688) with the autograd
 * backward of the fp32 upcast and of logits.div_(temperature).
 */
int mirl_filtered_logprob_bwd(const void* logits, int dtype, int64_t B, int64_t R,
                              int64_t R_total, int64_t V, int64_t stride_b,
                              int64_t stride_r, const int64_t* target,
                              int64_t t_stride_b, int64_t t_stride_r,
                              double temperature, double grad_temperature, int top_k,
                              const void* row_info, const int32_t* kept_idx,
                              const float* kept_p, const float* grad_out,
                              int64_t g_stride_b, int64_t g_stride_r, void* grad_in,
                              int64_t gi_stride_b, int64_t gi_stride_r, void* workspace,
                              void* stream);

/* Bytes of mirl_filtered_logprob_bwd's workspace for B x R rows of V elements
 * (32 per 8 KB piece of a row), or -1 with the error set. */
int64_t mirl_filtered_logprob_bwd_workspace_bytes(int dtype, int64_t B, int64_t R, int64_t V);

/*
 * apply_top_k_top_p on N rows of V logits: filtered[i, j] = x[i, j] where kept,
 * -inf elsewhere (in the logits dtype), keep_mask[i, j] = kept (uint8).
 * row_info / kept_idx / kept_p are scratch of the sizes above for N rows;
 * p_dtype as for mirl_filtered_logprob_fwd.
 *
 * Replaces: apply_top_k_top_p (nemo_rl/algorithms/logits_sampling_utils.py:256-287).
 */
int mirl_top_k_top_p_mask(const void* logits, int dtype, int64_t N, int64_t V,
                          int64_t row_stride, int top_k, double top_p, int p_dtype,
                          void* row_info, int32_t* kept_idx, float* kept_p,
                          void* filtered, int64_t filtered_row_stride,
                          uint8_t* keep_mask, int64_t keep_row_stride, void* stream);

/*
 * In-place temperature scaling of [B, R, V] logits (unit stride on V):
 *   x = dtype(fl32(float(x) * fl32(1.0 / temperature))), each rounding to
 *   nearest even, the reciprocal formed in double: torch's GPU division of a
 *   tensor by a Python scalar, which is where the reference runs it.
 *
 * Replaces: apply_temperature_scaling's logits.div_(temperature)
 * (nemo_rl/models/automodel/train.py:248-262,
 * nemo_rl/models/megatron/train.py:280-294).
 */
int mirl_temperature_scale(void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                           int64_t stride_b, int64_t stride_r, double temperature,
                           void* stream);

/*
 * Backward of mirl_temperature_scale: out = dtype(fl32(float(g) * r)), r =
 * fl32(1.0 / T); with `grad2` non-NULL,
 * out = dtype(fl32(float(dtype(float(g) + float(grad2))) * r))
 * (two consumers' gradients accumulated in the dtype first).  All three are
 * [B, R, V] views with unit stride on V; `out` may alias `grad`.
 *
 * Replaces: the autograd backward of logits.div_(temperature) (DivBackward)
 * and the accumulation of two gradients into it.
 */
int mirl_temperature_scale_grad(const void* grad, int dtype, int64_t B, int64_t R,
                                int64_t V, int64_t g_stride_b, int64_t g_stride_r,
                                const void* grad2, int64_t g2_stride_b,
                                int64_t g2_stride_r, double temperature, void* out,
                                int64_t o_stride_b, int64_t o_stride_r, void* stream);

/* ---------------------------------------------------------------------- */
/* logprobs from hidden states (LM-head GEMM fused with the log-sum-exp)     */
/* ---------------------------------------------------------------------- */

/* fp32 scratch elements mirl_linear_ce_fwd needs for T rows and V columns. */
int64_t mirl_linear_ce_workspace_elems(int64_t T, int64_t V);

/*
 * Selected-token logprobs from hidden states [T, H] (row r is sequence
 * position s = r / B of batch row b = r % B, i.e. a [S, B, H] tensor viewed as
 * rows) and an output weight [V, H], both of `dtype` (MIRL_DTYPE_BF16 or
 * MIRL_DTYPE_F16):
 *   x[r, v]  = dtype(sum_k hidden[r, k] * weight[v, k])   (fp32 accumulation)
 *   out[b,s] = (x[r, t'] - m) - log(sum_v exp(x[r, v] - m)),  t' = target[b, s] - vocab_start,
 *   out[b,s] = 0 when target < vocab_start or >= vocab_end.
 * The [T, V] logits are never written.  H must be a multiple of 128, row
 * strides multiples of 8 elements, both bases 16-byte aligned (the Python
 * layer copies other operands into zero-padded buffers first).  `row_stats`
 * (optional) receives {m, log sum} per row for mirl_linear_ce_grad;
 * `workspace` holds mirl_linear_ce_workspace_elems(T, V) floats.
 *
 * Replaces: the forward of ChunkedDistributedHiddenStatesToLogprobs
 * (nemo_rl/distributed/model_utils.py:2576-2644) as called by
 * from_parallel_hidden_states_to_logprobs (model_utils.py:2541-2569), with a
 * vocab group of size 1.
 */
int mirl_linear_ce_fwd(const void* hidden, int dtype, int64_t T, int64_t H, int64_t ldh,
                       const void* weight, int64_t V, int64_t ldw, int64_t B,
                       const int64_t* target, int64_t t_stride_b, int64_t t_stride_s,
                       int64_t vocab_start, int64_t vocab_end, float* out,
                       int64_t o_stride_b, int64_t o_stride_s, float* row_stats,
                       float* workspace, void* stream);

/*
 * Gradient of those logprobs with respect to the logits, for rows
 * [row0, row0 + nrows), recomputing the logits tile by tile (x in `dtype` as
 * above; the gradient is bf16 for either dtype, whose exponent range keeps the
 * small softmax terms that fp16 would flush):
 *   grad_logits[r - row0, v] = bf16((onehot(t')[v] - exp((x[r, v] - m) - logsum)) * g[b, s])
 * (row stride ldg >= V).  Tiles whose rows all have g == 0 are written as zeros
 * without the GEMM.  The hidden-state and weight gradients are the products
 * grad_logits . weight and grad_logits^T . hidden.  When grad_logits_t is not
 * NULL it also receives the transpose, grad_logits_t[v, r - row0], for the
 * 256-row tiles covering the range (rows past row0 + nrows as zeros; row
 * stride ldgt >= nrows rounded up to 256, a multiple of 8, 16-byte aligned).
 * `row_count` (a device int64, or NULL): rows r >= *row_count are absent, as
 * if nrows ended there; nothing is written for them in grad_logits, and
 * grad_logits_t holds zeros for them only inside the 256-row tile that holds
 * row *row_count - 1 (the caller's compacted active rows, counted on the
 * device so that the host need not wait for the count).
 *
 * Replaces: the per-chunk logits recompute, softmax and one-hot gradient of
 * ChunkedDistributedHiddenStatesToLogprobs.backward
 * (nemo_rl/distributed/model_utils.py:2647-2745).
 */
int mirl_linear_ce_grad(const void* hidden, int dtype, int64_t T, int64_t H, int64_t ldh,
                        const void* weight, int64_t V, int64_t ldw, int64_t B,
                        const int64_t* target, int64_t t_stride_b, int64_t t_stride_s,
                        int64_t vocab_start, int64_t vocab_end, const float* row_stats,
                        const float* grad_out, int64_t g_stride_b, int64_t g_stride_s,
                        int64_t row0, int64_t nrows, void* grad_logits, int64_t ldg,
                        void* grad_logits_t, int64_t ldgt, const int64_t* row_count,
                        void* stream);

/*
 * C = A . B^T for bf16 A [M, K] and B [N, K] (row strides lda, ldb, multiples
 * of 8 elements; K a multiple of 128; 16-byte aligned), with fp32
 * accumulation on the MFMA units (the tile loop of mirl_linear_ce_fwd):
 *   Cb != NULL: Cb[m, n] = cb_dtype(C[m, n])      (row stride ldcb; cb_dtype
 *               MIRL_DTYPE_BF16 or MIRL_DTYPE_F16);
 *   else:       C[s, m, n] = the product over the s-th of k_splits ranges of
 *               K ([k_splits][M][ldc] fp32), or C[m, n] += C when accumulate
 *               (k_splits = 1).
 * `count` (a device int64, or NULL) with c = *count - count_off:
 *   count_axis MIRL_COUNT_ROWS: rows m >= c of A are absent (not read; their
 *               output rows are not written);
 *   count_axis MIRL_COUNT_K: the reduction stops at round_up(c, 128) (columns
 *               of A and B past c up to there must hold finite values, zeros
 *               for an exact product); with accumulate set and c <= 0 nothing
 *               is written.  With both C and Cb given (k_splits = 1): the
 *               output goes to Cb = bf16(A . B^T (+ C when accumulate)) when
 *               *count <= final_at, to C otherwise: blocks of reduction rows
 *               accumulate in fp32 and the last non-empty one rounds once.
 * The backward of the hidden-state logprobs forms dH = G . W and
 * dW = G^T . H with it, from G, its transpose and transposed copies of W and H.
 *
 * Replaces: the dH and dW matmuls of ChunkedDistributedHiddenStatesToLogprobs.backward
 * (nemo_rl/distributed/model_utils.py:2701-2716).
 */
#define MIRL_COUNT_ROWS 0
#define MIRL_COUNT_K 1
int mirl_gemm_bf16_abt(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M,
                       int64_t N, int64_t K, int64_t k_splits, float* C, int64_t ldc,
                       int accumulate, void* Cb, int64_t ldcb, int cb_dtype,
                       const int64_t* count, int64_t count_off, int count_axis,
                       int64_t final_at, void* stream);

/* C = A[:, :K] . B[:, :K]^T in fp32 (A [M, >=K], B [N, >=K] fp32, row strides lda,
 * ldb multiples of 4 elements, 16-byte aligned; K a multiple of 64) on the same
 * MFMA tile loop, each 16-byte operand fragment feeding four
 * v_mfma_f32_32x32x2_f32.  C: fp32 [M, ldc] (C = or, with accumulate, C +=),
 * or [k_splits][M][ldc] partial products over k_splits ranges of K (ranges of
 * round_up(ceil(K / k_splits), 64), each non-empty).  `count` as for
 * mirl_gemm_bf16_abt (MIRL_COUNT_ROWS: rows of A at or past *count - count_off
 * are neither read nor written; MIRL_COUNT_K: the reduction stops at
 * round_up(*count - count_off, 64), and with accumulate set an empty reduction
 * writes nothing).
 * Replaces: the fp32 matmuls of ChunkedDistributedHiddenStatesToLogprobs
 * (nemo_rl/distributed/model_utils.py:2611-2616 logits, 2701-2716 dH and dW). */
int mirl_gemm_f32_abt(const float* A, int64_t lda, const float* B, int64_t ldb, int64_t M,
                      int64_t N, int64_t K, int64_t k_splits, float* C, int64_t ldc,
                      int accumulate, const int64_t* count, int64_t count_off, int count_axis,
                      void* stream);

/* out[r(m), n] = out_dtype(sum_s part[s, m, n]) summed in s order (part [k_splits][M][ld]
 * fp32, out row stride ldo, out_dtype MIRL_DTYPE_BF16, MIRL_DTYPE_F16 or
 * MIRL_DTYPE_F32): the splits of mirl_gemm_bf16_abt / mirl_gemm_f32_abt.  r(m) = out_rows[m]
 * (a device int64 row map; rows mapped outside [0, out_nrows) are skipped) or m
 * when out_rows is NULL.  With `count` (a device int64, or NULL), rows
 * m >= *count - count_off are written as zeros without reading part.
 * Replaces: part of the dH matmul above (model_utils.py:2701-2703) and the
 * scatter of the active rows' dH back to their positions. */
int mirl_sum_splits_bf16(const float* part, int64_t k_splits, int64_t M, int64_t N,
                         int64_t ld, void* out, int64_t ldo, int out_dtype,
                         const int64_t* out_rows, int64_t out_nrows, const int64_t* count,
                         int64_t count_off, void* stream);

/* dst[c, r] = bf16(src[r, c]) (src of src_dtype, MIRL_DTYPE_BF16 or
 * MIRL_DTYPE_F16; dst bf16) for r < R, c < C, and 0 for R <= r < R_pad
 * (src row stride lds, dst row stride ldd >= R_pad), R = min(R, *count) when
 * `count` (a device int64) is given: the transposed operands of the
 * hidden-state backward.
 * Replaces: the transposes inside the dH / dW matmuls (model_utils.py:2701-2716). */
int mirl_transpose_bf16(const void* src, int src_dtype, int64_t R, int64_t C, int64_t lds,
                        void* dst, int64_t ldd, int64_t R_pad, const int64_t* count,
                        void* stream);

/* dst[c, r] = src[r, c] in fp32 for r < R, c < C, and 0 for R <= r < R_pad (src row
 * stride lds, dst row stride ldd >= R_pad), R = min(R, *count - count_off) when
 * `count` (a device int64) is given: the transposed operands of the fp32
 * hidden-state backward (W, the active hidden rows, the logits gradient).
 * Replaces: the transposes inside the fp32 dH / dW matmuls (model_utils.py:2701-2716). */
int mirl_transpose_f32(const float* src, int64_t R, int64_t C, int64_t lds, float* dst,
                       int64_t ldd, int64_t R_pad, const int64_t* count, int64_t count_off,
                       void* stream);

/* ---------------------------------------------------------------------- */
/* ClippedPG loss epilogue                                                  */
/* ---------------------------------------------------------------------- */

/* KL estimator types (nemo_rl/algorithms/utils.py:56-115) */
#define MIRL_KL_K1 1
#define MIRL_KL_K2 2
#define MIRL_KL_K3 3

/* truncated importance sampling types (loss_functions.py:897-1013) */
#define MIRL_TIS_NONE 0
#define MIRL_TIS_TIS 1
#define MIRL_TIS_ICEPOP 2
#define MIRL_TIS_ADAPTIVE 3
#define MIRL_TIS_SEQ_MASK 4

/* Scalar configuration of one ClippedPGLossFn call.  Field meanings follow
 * ClippedPGLossConfig (nemo_rl/algorithms/loss/loss_functions.py:173-260). */
typedef struct mirl_pg_config {
  double ratio_clip_min;
  double ratio_clip_max;
  double ratio_clip_c;          /* <= 0 disables dual clipping */
  double kl_penalty;            /* beta; 0 disables the KL term */
  double kl_input_clamp;        /* used when has_kl_input_clamp */
  double kl_output_clamp;       /* used when has_kl_output_clamp */
  double tis_ratio;             /* truncated IS upper bound */
  double tis_ratio_min;         /* truncated IS lower bound (tis: 0 default) */
  double adaptive_hi;           /* adaptive-ppo-clip upper bound incl. k */
  double adaptive_outer;        /* adaptive-ppo-clip outer bound */
  double nll_weight;            /* VAPO positive-example NLL weight */
  int32_t kl_type;              /* MIRL_KL_K1/K2/K3 */
  int32_t tis_type;             /* MIRL_TIS_* */
  int32_t has_kl_input_clamp;
  int32_t has_kl_output_clamp;
  int32_t disable_ppo_ratio;
  int32_t token_level_loss;
  int32_t sequence_level_is;
  int32_t use_is_correction;
  int32_t use_on_policy_kl;
  int32_t force_on_policy;
  int32_t use_cispo;
  int32_t full_metrics;
  int32_t need_is;              /* full_metrics || use_is_correction */
  int32_t has_rewards;          /* rewards tensor present (VAPO) */
  int32_t has_support_mask;     /* policy_support_mask present */
  int32_t has_unfiltered;       /* curr_logprobs_unfiltered is a separate tensor */
} mirl_pg_config;

/* A [B, L] strided view: element (b, l) is ptr[b*sb + l*sl]. */
typedef struct mirl_view2d {
  const void* ptr;
  int64_t sb;
  int64_t sl;
} mirl_view2d;

/* Index of each metric in the metrics output array. */
#define MIRL_M_LOSS 0
#define MIRL_M_TOKEN_MULT_PROB_ERROR 1
#define MIRL_M_PROBS_RATIO 2
#define MIRL_M_PROBS_RATIO_CLAMPED 3
#define MIRL_M_PROBS_RATIO_MIN 4
#define MIRL_M_PROBS_RATIO_MAX 5
#define MIRL_M_PROBS_RATIO_CLAMPED_MIN 6
#define MIRL_M_PROBS_RATIO_CLAMPED_MAX 7
#define MIRL_M_GEN_KL_ERROR 8
#define MIRL_M_POLICY_KL_ERROR 9
#define MIRL_M_JS_DIVERGENCE_ERROR 10
#define MIRL_M_APPROX_ENTROPY 11
#define MIRL_M_SAMPLING_IMPORTANCE_RATIO 12
#define MIRL_M_KL_PENALTY 13
#define MIRL_M_NUM_VALID_SAMPLES 14
#define MIRL_M_POSITIVE_NLL_LOSS 15
#define MIRL_M_IS_OOB_RATIO 16
#define MIRL_M_POLICY_SUPPORT_EXCLUDED_TOKENS 17
#define MIRL_M_SCORE_CENTERING_HEAD_MASS 18
#define MIRL_NUM_METRICS 19

/* importance-sampling modes of score centering (score_centering.py:22-129) */
#define MIRL_SC_OFF 0
#define MIRL_SC_IS 1
#define MIRL_SC_TIS 2
#define MIRL_SC_ICEPOP 3
#define MIRL_SC_ADAPTIVE 4

/*
 * Score-centering inputs: the trainer's log-probs at the sampler's top-k ids
 * (`plog`, [B, L, K]) and the sampler's own log-probs at those ids (`qlog`,
 * [B, L, K]), both strided views of the loss dtype; element (b, l, k) is
 * ptr[b*sb + l*sl + k*sk].  `lo`/`hi` are the TIS / ICEPOP bounds or
 * adaptive-ppo-clip's lower and (offset) upper bound, `outer` its outer bound.
 * `grad` receives a contiguous [B, L, K] array of the loss dtype: the
 * gradient of the loss w.r.t. plog (mirl_clipped_pg) or the coefficients
 * d term / d plog (mirl_score_centering_term).
 */
typedef struct mirl_score_centering_args {
  int32_t mode;  /* MIRL_SC_* */
  int32_t pad_;
  int64_t K;
  double lo, hi, outer;
  const void* plog;
  int64_t p_sb, p_sl, p_sk;
  const void* qlog;
  int64_t q_sb, q_sl, q_sk;
  void* grad;
} mirl_score_centering_args;

/* Number of scratch elements (of the loss dtype) mirl_clipped_pg needs for
 * [B, L] tokens, with or without score centering. */
int64_t mirl_clipped_pg_workspace_elems(int64_t B, int64_t L, int score_centering);

/*
 * Fused ClippedPG loss forward + closed-form backward over [B, L] tokens
 * (L = S - 1; the caller passes the [:, 1:] views of the [B, S] data).
 * Writes: metrics[MIRL_NUM_METRICS] (metrics[MIRL_M_LOSS] is the loss), the
 * loss again into `loss` (one element; optional, NULL skips it: a caller that
 * needs the loss apart from the metrics saves a copy kernel),
 * grad_curr[B, L] = dloss/dnext_token_logprobs, and, when
 * cfg->has_unfiltered, grad_unfiltered[B, L] = dloss/dcurr_logprobs_unfiltered.
 * `dtype` is MIRL_DTYPE_F32 or MIRL_DTYPE_F64 for every float tensor;
 * support_mask is uint8 (bool); sample_mask and rewards are [B] vectors;
 * global_valid_seqs / global_valid_toks are device scalars of `dtype`.
 * `workspace` holds mirl_clipped_pg_workspace_elems(B, L, score_centering != NULL)
 * elements of `dtype`.
 * `score_centering` is NULL or adds the score-centering correction: the
 * per-token term of mirl_score_centering_term at the final loss mask, times
 * the masked advantage, reduced like the actor loss and added to it; the
 * advantages are zeroed outside the mask; metrics[MIRL_M_SCORE_CENTERING_HEAD_MASS]
 * is the masked mean head mass; score_centering->grad receives dloss/dplog.
 *
 * Replaces: ClippedPGLossFn.__call__ (loss_functions.py:698-1183) with
 * clipped_pg_actor_objective / clipped_pg_diagnostic_metrics
 * (clipped_pg.py:53-194), calculate_kl and masked_mean
 * (algorithms/utils.py:56-115, 294-306), and the autograd backward of all of
 * them.
 */
int mirl_clipped_pg(const mirl_pg_config* cfg, int dtype, int64_t B, int64_t L,
                    mirl_view2d curr, mirl_view2d unfiltered,
                    mirl_view2d token_mask, mirl_view2d advantages,
                    mirl_view2d prev, mirl_view2d generation,
                    mirl_view2d reference, mirl_view2d support_mask,
                    const void* sample_mask, const void* rewards,
                    const void* global_valid_seqs,
                    const void* global_valid_toks, void* metrics, void* loss,
                    void* grad_curr, void* grad_unfiltered,
                    const mirl_score_centering_args* score_centering,
                    void* workspace, void* stream);

/* Bytes of scratch held by mirl_clipped_pg_noalloc on each GPU (4 MiB). */
int64_t mirl_clipped_pg_noalloc_max_scratch_bytes(void);

/*
 * mirl_clipped_pg without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Arguments and results are those of mirl_clipped_pg; the scratch is a fixed
 * array of mirl_clipped_pg_noalloc_max_scratch_bytes() bytes in the
 * library's device data, one copy per GPU, held until the process ends.
 * Inputs whose workspace (mirl_clipped_pg_workspace_elems(B, L, sc) elements
 * of `dtype`) exceeds it are rejected with MIRL_ERR_INVALID_ARGUMENT.  The
 * call allocates nothing: no hipMalloc / hipFree or allocating library call.
 * The first call on a device looks up that device's scratch address; later
 * calls reuse it.  Every call on one GPU shares that GPU's scratch, so calls
 * that overlap on one GPU (two streams, two threads) race and must be
 * serialised by the caller.
 */
int mirl_clipped_pg_noalloc(const mirl_pg_config* cfg, int dtype, int64_t B, int64_t L,
                            mirl_view2d curr, mirl_view2d unfiltered,
                            mirl_view2d token_mask, mirl_view2d advantages,
                            mirl_view2d prev, mirl_view2d generation,
                            mirl_view2d reference, mirl_view2d support_mask,
                            const void* sample_mask, const void* rewards,
                            const void* global_valid_seqs,
                            const void* global_valid_toks, void* metrics, void* loss,
                            void* grad_curr, void* grad_unfiltered,
                            const mirl_score_centering_args* score_centering,
                            void* stream);

/*
 * Per-token score-centering term over [B, L] tokens:
 *   p = exp(plog), q = exp(qlog), head = sum_k q, rho = max(1 - head, 0) / max(1 - sum_k p, 1e-6)
 *   mode off: mass = q, alpha = rho;  is: mass = p, alpha = 1
 *   tis: mass = min(max(p, lo q), hi q), alpha = min(max(1, lo rho), hi rho)
 *   icepop: mass = p where lo <= p/q <= hi else 0, alpha = [lo <= 1/rho <= hi]
 *   adaptive-ppo-clip: as icepop with the advantage-signed bounds and `outer`
 *   coef = mass - alpha p,   term = sum_k coef_k plog_k,   head_mass = head,
 * all 0 where token_mask is 0.  Writes term[B, L], head_mass[B, L]
 * (contiguous, the loss dtype) and coef into args->grad.  `advantages` (a
 * [B, L] view, read by adaptive-ppo-clip only) may have a NULL pointer
 * otherwise.
 *
 * Replaces: compute_score_centering_term
 * (nemo_rl/algorithms/loss/score_centering.py:22-129); its autograd backward
 * is coef * d(term).
 */
int mirl_score_centering_term(int dtype, int64_t B, int64_t L,
                              const mirl_score_centering_args* args,
                              mirl_view2d token_mask, mirl_view2d advantages,
                              void* term, void* head_mass, void* stream);

/* ---------------------------------------------------------------------- */
/* GRPO group-normalised advantages                                         */
/* ---------------------------------------------------------------------- */

/*
 * Per sample i of B (fp32 rewards, int64 prompt keys [B, K] with row stride
 * `prompt_stride`, fp32 valid mask or NULL for all-valid, fp32 std_rewards or
 * NULL to use the rewards themselves for the spread statistics):
 *   group(i) = { j : prompts[j, :] == prompts[i, :] }
 *   n = sum_{j in group} valid[j]
 *   n <= 1 : baseline = r_i, std = 0
 *   else   : baseline = sum_{j in group, j != i if loo} r_j v_j / (n - loo)
 *            std = sqrt((sum q_j^2 v_j / (n - loo) - qbar^2)
 *                       * (n - loo) / (n - loo - 1)), NaN -> 0, inf -> FLT_MAX
 *            with q = std_rewards (or r) and qbar its group mean like baseline
 *   adv_i = r_i - baseline; when normalize and std > 0 and the comparison set
 *   (of q) is not all-equal: adv_i /= (std + 1e-6).
 * Writes adv[B] (fp32) and, when non-NULL, baseline[B], std[B] (fp32) and
 * trivial[B] (uint8: 1 when the group has <= 1 valid sample or its comparison
 * set is all-equal).
 *
 * Replaces: GRPOAdvantageEstimator.compute_advantage
 * (nemo_rl/algorithms/advantage_estimator.py:106-145) with
 * calculate_baseline_and_std_per_prompt (nemo_rl/algorithms/utils.py:118-234).
 */
int mirl_grpo_advantage(const int64_t* prompts, int64_t B, int64_t K,
                        int64_t prompt_stride, const float* rewards,
                        const float* std_rewards, const float* valid_mask,
                        int leave_one_out,
                        int normalize, float* adv, float* baseline, float* std,
                        uint8_t* trivial, void* stream);

/* ---------------------------------------------------------------------- */
/* Packed-sequence glue                                                    */
/* ---------------------------------------------------------------------- */
/* Sequence boundaries are int64 DEVICE arrays of n_seq + 1 nondecreasing
 * entries (cu_seqlens / cu_seqlens_padded uploaded by the caller).  Each
 * thread finds its sequence by a binary search of them; reads are guarded, so
 * boundaries that break the ordering give zeros, never an access outside the
 * buffers.
 *
 * mirl_pack_sequences: out[p, e] (p < total = cu_seqlens_padded[B],
 * e < row_elems, elements of elem_bytes = 1, 2, 4 or 8 bytes) =
 *   x[seq * S + off, e]  for p in [cu_pad[seq], cu_pad[seq + 1]),
 *                        off = (p - cu_pad[seq] - roll_shift) mod the
 *                        segment length (no roll when roll_shift == 0),
 *                        when off < min(cu_seqlens[seq+1] - cu_seqlens[seq], S);
 *   0                    otherwise (and for p < cu_pad[0]).
 * x is [B, S, row_elems] contiguous; out [total, row_elems] contiguous.
 * Replaces: _pack_input_ids (nemo_rl/algorithms/loss/utils.py:355-408), CP = 1.
 */
int mirl_pack_sequences(const void* x, int64_t B, int64_t S, int64_t row_elems,
                        int32_t elem_bytes, const int64_t* cu_seqlens,
                        const int64_t* cu_seqlens_padded, int64_t roll_shift,
                        void* out, int64_t total, void* stream);

/* mirl_packed_roll_targets: out[p] = target[p + 1] inside a segment
 * [b[i], b[i+1]), target[b[i]] at the segment's last position, 0 for p
 * outside [b[0], b[n_seq]).  target and out are [n] int64.
 * Replaces: the per-sequence target roll of
 * from_parallel_logits_to_logprobs_packed_sequences
 * (nemo_rl/distributed/model_utils.py:1116-1139).
 */
int mirl_packed_roll_targets(const int64_t* target, int64_t n, const int64_t* bounds,
                             int64_t n_seq, int64_t* out, void* stream);

/* mirl_unpack_rows_fwd: out[i, j] = packed[b[i] + j] for
 * j < clip(b[i+1] - b[i] - 1, 0, cols), else 0; out is [n_seq, cols] fp32,
 * packed [n_rows] fp32.
 * mirl_unpack_rows_bwd: its backward, grad_packed[p] = grad_out[i, p - b[i]]
 * for the packed rows the forward copied, 0 elsewhere ([n_rows] fp32;
 * grad_out [n_seq, cols] contiguous).
 * Replaces: the unpacking loop of from_parallel_logits_to_logprobs_packed_sequences
 * (nemo_rl/distributed/model_utils.py:1211-1229) and its autograd backward.
 */
int mirl_unpack_rows_fwd(const float* packed, int64_t n_rows, const int64_t* bounds,
                         int64_t n_seq, int64_t cols, float* out, void* stream);
int mirl_unpack_rows_bwd(const float* grad_out, int64_t n_seq, int64_t cols,
                         const int64_t* bounds, int64_t n_rows, float* grad_packed,
                         void* stream);

/* ---------------------------------------------------------------------- */
/* token-level post-processing of logprobs                                  */
/* ---------------------------------------------------------------------- */

/*
 * out[b, s] = mask[b, s] != 0 ? logprobs[b, s] : 0 over [B, S] views with
 * element strides (a stride of 0 broadcasts); logprobs and out are of `dtype`
 * (F32, BF16, F16 or F64; the selected values are copied bit for bit), the mask
 * is fp32; out may alias logprobs.  The same call with the upstream gradient in
 * place of the logprobs is the selection's backward.
 *
 * Replaces: mask_filtered_logprobs_outside_tokens
 * (nemo_rl/algorithms/utils.py:309-326), applied after the filtered logprobs
 * by the Megatron logprob post-processor (nemo_rl/models/megatron/train.py:960-964).
 */
int mirl_mask_outside_tokens(const void* logprobs, int dtype, int64_t B, int64_t S,
                             int64_t lp_sb, int64_t lp_ss, const float* mask, int64_t m_sb,
                             int64_t m_ss, void* out, int64_t o_sb, int64_t o_ss, void* stream);

/*
 * Per sequence b of [B, S] fp32 views (element strides), w_s = token_mask[b, s]
 * * sample_mask[b]:
 *   errors[b] = sum_s exp(e_s * w_s) * w_s / max(sum_s w_s, 1),
 *   e_s = w_s != 0 ? |generation[b, s] - policy[b, s]| : 0,
 *   valid[b]  = sum_s w_s > 0 (uint8).
 * A non-finite logprob on a valid token makes errors[b] non-finite.
 *
 * Replaces: compute_seq_logprob_errors (nemo_rl/algorithms/utils.py:273-291).
 */
int mirl_seq_logprob_errors(const float* policy, int64_t p_sb, int64_t p_ss,
                            const float* generation, int64_t g_sb, int64_t g_ss,
                            const float* token_mask, int64_t t_sb, int64_t t_ss,
                            const float* sample_mask, int64_t s_sb, int64_t B, int64_t S,
                            float* errors, uint8_t* valid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIRL_H */
