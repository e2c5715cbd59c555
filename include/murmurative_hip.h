/*
 * murmurative_hip.h -- C ABI of libmurmurative_hip.so (MI355X / gfx950).
 *
 * Plain pointers, sizes and element strides; no framework types.  Every call
 * enqueues asynchronously on `stream` (a hipStream_t; NULL = the null
 * stream) and never allocates device memory: buffers that outlive a call or
 * that a call needs as scratch come in through `workspace` pointers whose
 * sizes the matching *_workspace_bytes function returns.
 *
 * Layout conventions
 *   token tensors   [B,H,N,D] views: element (b,h,n,d) at ptr + b*sb + h*sh
 *                   + n*sn + d.  D must be contiguous.
 *   slot tensors    [B,H,M,D] views: ptr + b*sb + h*sh + m*sm + d (sb may be
 *                   0 for slots shared over the batch).
 *   indices         int64 [B,H,N,7], weights float32 [B,H,N,7], contiguous.
 *   dtype codes     MURM_F32, MURM_F16, MURM_BF16.
 * Limits: 7 <= M <= 65535, 1 <= D <= 128, rounds <= 16, slots per token = 7,
 * N <= 2^24, B*H*N < 2^31 tokens, token row strides (sn) < 2^32 elements.
 * The entry points that select (murm_select_attend_fwd, murm_select_fwd,
 * murm_murmurate_fwd) also stage one head's slot keys in the 160 KiB LDS of
 * a CU, which bounds M by dtype and D: murm_select_max_m() returns the bound
 * (16-bit tokens: 1024 / 560 / 288 for D <= 32 / 64 / 128; float32 tokens:
 * 1136 / 592 / 304); larger M returns MURM_ERR_UNSUPPORTED before any launch.
 *
 * Return value: MURM_OK, or an error code with a message readable through
 * murm_last_error() (per thread).  Argument errors are detected on the host
 * before anything is enqueued.
 *
 * Each entry point names the reference interface it replaces
 * (beaglabs/murmurative-attention, paths relative to the repository root).
 */
#ifndef MURMURATIVE_HIP_H
#define MURMURATIVE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MURM_OK 0
#define MURM_ERR_ARG 1
#define MURM_ERR_UNSUPPORTED 2
#define MURM_ERR_HIP 3

#define MURM_F32 0
#define MURM_F16 1
#define MURM_BF16 2

/* Version string of the library. */
const char* murm_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* murm_last_error(void);

/* ---------------------------------------------------------------------------
 * Fused select + attend, one round.
 * Replaces slot_select_attend_forward (torch-ext/cuda_ops.h:7-15,
 * src/murmurative/csrc/cuda/slot_select_attend.cu:464-589) behind the op
 * schema at torch-ext/torch_binding.cpp:7-10.  Semantics follow
 * src/murmurative/reference.py:6-68: top-7 of q.sk (+bias, masked) sorted by
 * descending score, softmax over the real scores times `scale`
 * (scale <= 0 means 1/sqrt(D)).  mask (nonzero = keep) and bias are optional
 * [B,H,N,M] views with element strides (0 for broadcast dimensions).
 * effective_M <= 0 means M.  out is written through its own strides.
 * ------------------------------------------------------------------------- */
size_t murm_select_attend_workspace_bytes(int B, int H, int N, int D, int M);
int murm_select_attend_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                           const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                           const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                           const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                           const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm,
                           const float* bias, int64_t bs_sb, int64_t bs_sh, int64_t bs_sn, int64_t bs_sm,
                           int causal, double scale, int effective_M,
                           void* out, int64_t out_sb, int64_t out_sh, int64_t out_sn,
                           float* weights, int64_t* indices,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Largest M the selecting entry points accept for this token dtype and head
 * dim (0 for an invalid dtype or D).  No counterpart in the reference, whose
 * CUDA path stops at M*D*2 <= 48 KiB (slot_select_attend.cu:486-490). */
int murm_select_max_m(int dtype, int D);

/* ---------------------------------------------------------------------------
 * Selection only: int64 indices [B,H,N,7] of the top-7 masked scores, sorted
 * by descending score.  Serves slot_select (src/murmurative/ops.py:215-228,
 * which the reference always runs through reference.py:6-39 with ATen).
 * Uses the select_attend workspace size.
 * ------------------------------------------------------------------------- */
int murm_select_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                    const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                    const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm,
                    const float* bias, int64_t bs_sb, int64_t bs_sh, int64_t bs_sn, int64_t bs_sm,
                    int causal, int effective_M, int64_t* indices,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Attend for given indices: weights = softmax(scale * q.sk[idx]) and
 * out = sum_j w_j sv[idx_j].  Serves slot_attend (src/murmurative/ops.py:
 * 231-244; semantics reference.py:42-68, indices clamped to [0, M-1]).
 * Uses the select_attend workspace size.
 * ------------------------------------------------------------------------- */
int murm_attend_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                    const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                    const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                    const int64_t* indices, double scale,
                    void* out, int64_t out_sb, int64_t out_sh, int64_t out_sn, float* weights,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Backward of the fused select + attend (indices fixed).
 * Replaces slot_select_attend_backward (torch-ext/cuda_ops.h:17-25,
 * slot_select_attend.cu:591-671; schema torch_binding.cpp:11-14), including
 * the grad_weights term that the reference CUDA kernel ignores
 * (grad_weights may be NULL = zero).  grad_q is token-dtype [B,H,N,D]
 * contiguous; grad_sk / grad_sv are slot-dtype [B,H,M,D] contiguous.
 * ------------------------------------------------------------------------- */
size_t murm_select_attend_bwd_workspace_bytes(int B, int H, int N, int D, int M);
int murm_select_attend_bwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                           const void* grad_out, int64_t g_sb, int64_t g_sh, int64_t g_sn,
                           const float* grad_weights,
                           const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                           const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                           const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                           const int64_t* indices, const float* weights, double scale,
                           void* grad_q, void* grad_sk, void* grad_sv,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Slot EMA update, in place on sk / sv.
 * Replaces slot_update_forward (torch-ext/cuda_ops.h:28-35,
 * slot_update.cu:253-288; schema torch_binding.cpp:15-18).  Semantics
 * reference.py:71-115 (float32 sums, mean over W + 1e-8, used slots only,
 * indices clamped to [0, M-1]).  Deterministic: no float atomics.
 * ------------------------------------------------------------------------- */
size_t murm_slot_update_workspace_bytes(int B, int H, int N, int D, int M);
int murm_slot_update_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                         void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                         void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                         const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn,
                         const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                         const int64_t* indices, const float* weights, double alpha,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Backward of the slot update.
 * Replaces slot_update_backward (torch-ext/cuda_ops.h:37-45,
 * slot_update.cu:290-361; schema torch_binding.cpp:19-22).  Outputs:
 * grad_tk / grad_tv token-dtype [B,H,N,D] contiguous, grad_old_sk /
 * grad_old_sv slot-dtype [B,H,M,D] contiguous, grad_w float32 [B,H,N,7].
 * ------------------------------------------------------------------------- */
size_t murm_slot_update_bwd_workspace_bytes(int B, int H, int N, int D, int M);
int murm_slot_update_bwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                         const void* gk, int64_t gk_sb, int64_t gk_sh, int64_t gk_sm,
                         const void* gv, int64_t gv_sb, int64_t gv_sh, int64_t gv_sm,
                         const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn,
                         const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                         const int64_t* indices, const float* weights, double alpha,
                         void* grad_tk, void* grad_tv, void* grad_old_sk, void* grad_old_sv,
                         float* grad_w, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Tridiagonal diffusion, in place.  Replaces slot_diffusion_forward
 * (torch-ext/cuda_ops.h:48-51, slot_diffusion.cu:121-144; schema
 * torch_binding.cpp:23-25).  reference.py:118-135.
 * ------------------------------------------------------------------------- */
int murm_slot_diffusion_fwd(int slot_dtype, int B, int H, int M, int D,
                            void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                            void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                            double gamma, void* stream);

/* Adjoint of the diffusion (grad_* outputs contiguous [B,H,M,D]).  Replaces
 * slot_diffusion_backward (torch-ext/cuda_ops.h:53-57,
 * slot_diffusion.cu:146-177; schema torch_binding.cpp:26-28); correct for
 * every M, including M = 3. */
int murm_slot_diffusion_bwd(int slot_dtype, int B, int H, int M, int D,
                            const void* gk, int64_t gk_sb, int64_t gk_sh, int64_t gk_sm,
                            const void* gv, int64_t gv_sb, int64_t gv_sh, int64_t gv_sm,
                            double gamma, void* grad_k, void* grad_v, void* stream);

/* ---------------------------------------------------------------------------
 * Update then diffusion, in place.  Replaces slot_update_diffuse_forward
 * (torch-ext/cuda_ops.h:60-68, slot_update_diffuse.cu:120-156; schema
 * torch_binding.cpp:29-32).  Diffusion reads the post-update neighbours as
 * reference.py:188-189 does (the reference CUDA kernel reads pre-update
 * neighbours).
 * ------------------------------------------------------------------------- */
int murm_slot_update_diffuse_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                                 void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                                 void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                                 const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn,
                                 const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                                 const int64_t* indices, const float* weights, double alpha,
                                 double gamma, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * All R rounds of select -> attend -> residual -> update -> diffuse, forward.
 * Replaces the per-round Python orchestration of slot_murmurate
 * (src/murmurative/ops.py:330-422 and the autograd Functions it applies,
 * ops.py:55-208) and serves the README call form (README.md:61-69).
 *   q        selection queries (all rounds)
 *   x        residual base (NULL: q, the README form)
 *   tk, tv   update sources (NULL: q)
 *   sk, sv   initial slots (slot_dtype views, sb may be 0); slots of the
 *            token dtype (16-bit) with D % 8 == 0 and 16-byte aligned rows
 *            and strides are read by the first select kernel itself, any
 *            other slot dtype or layout takes one conversion launch more
 *   mask     optional [B,H,N,M] keep-mask view
 * Outputs: out = x + sum_r attend_r (through its strides), and for the last
 * round the int64 indices (may be NULL) and float32 weights.  `workspace`
 * (murm_murmurate_workspace_bytes) keeps what murm_murmurate_bwd needs: do
 * not reuse it until the backward ran.  The last round's update is skipped:
 * its result reaches no output.
 * ------------------------------------------------------------------------- */
size_t murm_murmurate_workspace_bytes(int B, int H, int N, int D, int M, int rounds, int shared_kv);
int murm_murmurate_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, int rounds,
                       double alpha, double gamma, int causal, int effective_M, double scale,
                       const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                       const void* x, int64_t x_sb, int64_t x_sh, int64_t x_sn,
                       const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn,
                       const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                       const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                       const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                       const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm,
                       void* out, int64_t out_sb, int64_t out_sh, int64_t out_sn,
                       int64_t* indices_last, float* weights_last,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Byte offset inside the murm_murmurate_fwd workspace of one saved per-round
 * buffer (-1 if that round has none).  field: 0 slot keys, 1 slot values
 * (float32 [B*H,M,D], state entering the round), 2 indices (uint16
 * [B*H,N,8], 8th entry 0xFFFF), 3 key sums, 4 value sums (float32
 * [B*H,M,D]), 5 weight sums (float32 [B*H,M]), 6 weights (float32
 * [B*H,N,7]; the last round's live in weights_last).  No counterpart in the
 * reference; lets callers inspect the rounds. */
int64_t murm_murmurate_workspace_offset(int B, int H, int N, int D, int M, int rounds, int shared_kv,
                                        int round, int field);

/* ---------------------------------------------------------------------------
 * Backward of murm_murmurate_fwd (same geometry, q / tk / tv and the
 * forward's workspace and weights_last).  grad_weights_last may be NULL.
 * grad_q receives the selection-query gradient, plus grad_out when x was
 * NULL (README form) and plus the update-source gradient when tk/tv were
 * NULL.  grad_tk / grad_tv (token dtype, strided) are written only when the
 * forward had separate tk / tv.  grad_sk / grad_sv are slot-dtype
 * [B,H,M,D] contiguous.  The gradient of x is grad_out itself.
 * ------------------------------------------------------------------------- */
size_t murm_murmurate_bwd_workspace_bytes(int B, int H, int N, int D, int M, int rounds, int shared_kv);
int murm_murmurate_bwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, int rounds,
                       double alpha, double gamma, double scale, int x_given,
                       const void* grad_out, int64_t g_sb, int64_t g_sh, int64_t g_sn,
                       const float* grad_weights_last,
                       const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                       const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn,
                       const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                       const float* weights_last,
                       const void* fwd_workspace, size_t fwd_workspace_bytes,
                       void* grad_q, int64_t gq_sb, int64_t gq_sh, int64_t gq_sn,
                       void* grad_tk, int64_t gtk_sb, int64_t gtk_sh, int64_t gtk_sn,
                       void* grad_tv, int64_t gtv_sb, int64_t gtv_sh, int64_t gtv_sn,
                       void* grad_sk, void* grad_sv,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Graph replay of the fused rounds (no counterpart in the reference, whose
 * slot_murmurate issues its rounds op by op from Python, ops.py:376-419).
 * With replay on, murm_murmurate_fwd / murm_murmurate_bwd capture their
 * kernel sequence for each distinct argument set (pointers, sizes, scalars,
 * stream) into a hipGraph once and replay it with one hipGraphLaunch after
 * that (at most 16 cached graphs, least recently used dropped).  Calls on
 * the null stream, calls while timing is on, and calls on a stream that is
 * already being captured launch their kernels directly.  Turning replay off
 * destroys the cached graphs.  murm_graph_cached returns their number.
 * ------------------------------------------------------------------------- */
void murm_graph_replay(int on);
int murm_graph_cached(void);

/* ---------------------------------------------------------------------------
 * Measurement hooks (no counterpart in the reference).  When enabled, every
 * kernel launch records a start and a stop HIP event from its own dispatch
 * (hipExtLaunchKernel), so each pair times the kernel's execution alone;
 * murm_timing_read waits for the recorded events and returns the summed
 * device time (ms) and launch count of one kernel class.  Classes: 0 select_attend, 1 gather_out,
 * 2 seg_update, 3 seg_attbwd, 4 du, 5 tok_bwd, 6 tok_grad, 7 conversions,
 * 8 seg_update_reduce, 9 seg_attbwd_reduce (2 and 3 are the partial-sum
 * kernels when 8 and 9 run, else the whole reduction).
 * ------------------------------------------------------------------------- */
#define MURM_TIMING_CLASSES 10
void murm_timing_enable(int on);
void murm_timing_reset(void);
int murm_timing_read(int cls, double* total_ms, int64_t* launches);
const char* murm_timing_name(int cls);

/* Self-test of the 16x16x32 bf16 MFMA lane layout the kernels assume.  Runs
 * three products whose exact result is D[i][j] = 16*i + j when the assumed
 * A, B and D layouts hold:  (A = 16i+k for k < 16, B = identity),
 * (A = identity, B = 16k+j for k < 16) and (A[i][k] = (k == i+16),
 * B[k][j] = 16(k-16)+j for k >= 16).  Writes 3 x 64 lanes x 4 floats, in
 * the D layout, to `out` (device, 768 floats).  No counterpart in the
 * reference. */
int murm_selftest_mfma(float* out, void* stream);

/* ---------------------------------------------------------------------------
 * Allocation-free select + attend.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as murm_select_attend_fwd, without the workspace:
 * the library keeps MURM_NOALLOC_SCRATCH_BYTES of device scratch per GPU for
 * the life of the process and never allocates.  Shapes whose workspace
 * (murm_select_attend_workspace_bytes) exceeds it return
 * MURM_ERR_UNSUPPORTED.  The stream must belong to the current device.
 * Calls on one GPU share the scratch: calls that overlap in time on one GPU
 * (e.g. on two streams) race.
 * ------------------------------------------------------------------------- */
#define MURM_NOALLOC_SCRATCH_BYTES (64u << 20)
int murm_select_attend_fwd_noalloc(int dtype, int slot_dtype, int B, int H, int N, int D, int M,
                                   const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sn,
                                   const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                                   const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                                   const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm,
                                   const float* bias, int64_t bs_sb, int64_t bs_sh, int64_t bs_sn, int64_t bs_sm,
                                   int causal, double scale, int effective_M,
                                   void* out, int64_t out_sb, int64_t out_sh, int64_t out_sn,
                                   float* weights, int64_t* indices, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MURMURATIVE_HIP_H */
