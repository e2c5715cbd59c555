// Kernel parameter blocks and launchers (internal to libmurmurative_hip).
#pragma once

#include <atomic>

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "murm_common.h"

namespace murm {

// Events that the calling thread's next kernel launch records from its own
// dispatch (start and end of the kernel's execution); null = a plain launch.
// The C ABI's timing wrapper sets them around exactly one launch.
struct LaunchEvents {
  hipEvent_t start;
  hipEvent_t stop;
};
LaunchEvents& launch_events();

#define MURM_LAUNCH(kernel, grid, block, lds, stream, ...)                                           \
  do {                                                                                               \
    const ::murm::LaunchEvents _ev = ::murm::launch_events();                                        \
    if (_ev.start)                                                                                   \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, _ev.start, _ev.stop, 0, __VA_ARGS__);   \
    else                                                                                             \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                             \
  } while (0)

struct SAParams {
  TokView q;
  const float* sk;        // fp32 slot keys [BH, M, D]
  int B, H, N, D, M, em;
  int causal;
  float scale;
  uint32_t hi_mask, lo_mask;  // packed-key split (low bits carry the slot)
  const uint8_t* mask;        // optional, nonzero = keep; element strides over (b,h,n,m)
  int64_t mk_sb, mk_sh, mk_sn, mk_sm;
  const float* bias;          // optional position bias added to the unscaled score
  int64_t bs_sb, bs_sh, bs_sn, bs_sm;
  uint16_t* idx16;            // [BH, N, 8] or null
  int64_t* idx64;             // [BH, N, 7] or null
  float* w;                   // [BH, N, 7]
  // 16-bit tokens: the keys already split into hi / lo halves of the token
  // dtype in the kernel's LDS layout (KeySplit below); null: split from sk
  const void* ksplit;
  int keys_hi_only;  // 1: the lo halves of ksplit are all zero (keys of the token dtype)
  // First round of a fused call whose slot tensors have the token dtype: the
  // caller's keys and values (element strides over b, h, m; 16-byte aligned
  // rows, D % 8 == 0) read by the kernel itself instead of a split table; the
  // kernel writes the float32 state rows of both ([BH, M, D], each block of a
  // head its share of the rows) for the kernels that follow.  raw_k null: unused.
  const void* raw_k;
  int64_t rk_sb, rk_sh, rk_sm;
  const void* raw_v;
  int64_t rv_sb, rv_sh, rv_sm;
  float* st_k;
  float* st_v;
};

// Slot keys split for the 16-bit select kernel: per (b,h) a hi table then a lo
// table, each [Mp][DP + 8] elements of the token dtype (Mp = M rounded up to
// 16; hi = rn(k), lo = rn(k - hi); zero at d >= D and m >= M; the last 8
// columns are row padding and never read).  This is the kernel's LDS image,
// so the kernel copies it in with no conversion.
__host__ __device__ inline int ksplit_row(int DP) { return DP + 8; }
__host__ __device__ inline int ksplit_mp(int M) { return (M + 15) & ~15; }
__host__ __device__ inline size_t ksplit_head_elems(int M, int DP) { return 2 * (size_t)ksplit_mp(M) * ksplit_row(DP); }

struct KeySplitOut {   // where a kernel writes split keys (p == null: nowhere)
  void* p;
  int dtype;           // token dtype (DT_BF16 / DT_F16)
  int DP;
};

struct OutParams {
  TokView base;     // optional residual (p == null -> 0)
  TokViewMut out;
  int B, H, N, D, M, R;
  RoundPtrs rp;     // idx[r], w[r], a[r] = value table of round r
};

enum SegMode : int { SEG_UPDATE = 0, SEG_ATTBWD = 1 };

struct SegParams {
  int B, H, N, D, M, K;
  const uint16_t* idx;   // [BH, N, 8]
  const float* wgt;      // [BH, N, K] weights
  const float* ds;       // [BH, N, K] softmax-backward (ATTBWD)
  float ds_scale;        // c = attend scale (ATTBWD)
  TokView va;            // UPDATE: token keys; ATTBWD: queries
  TokView vb;            // UPDATE: token values; ATTBWD: grad of the attend output
  int b_same_as_a;       // UPDATE: token values are the token keys
  int uniq_idx;          // 1: every token's slots are distinct (indices from the select kernel)
  // UPDATE
  const float* sk_old; const float* sv_old;  // fp32 [BH, M, D]
  float* sk_new; float* sv_new;              // fp32 [BH, M, D] (null: sums only)
  float* ksum; float* vsum; float* wsum;     // optional saved sums
  float alpha, gamma, eps;
  int diffuse;
  KeySplitOut ksplit_new;                    // new keys, split for the next select
  // ATTBWD
  const float* carry_k; const float* carry_v;  // optional pass-through grads (read, halo included)
  int final_out;                               // 1: write G'' of the owned rows to gk_out / gv_out
  float* gk_out; float* gv_out;                // fp32 [BH, M, D]
  void* gk_t; void* gv_t;                      // or (non-null) the slot-dtype [B,H,M,D] grads directly
  int64_t gt_sb, gt_sh, gt_sm;                 //   their element strides
  int gt_dtype;                                //   and dtype code
  // ATTBWD epilogue for the previous round (final_out == 0)
  const float* Kp; const float* Vp; const float* Wp;  // that round's forward sums
  int combine_dk;                              // token keys == token values: dk_out = dKk + dKv
  float* dk_out; float* dv_out; float* dW_out;
  float* carry_k_out; float* carry_v_out;      // must not alias carry_k / carry_v
};

struct PartParams {       // token-chunk partial sums (scratch)
  int nchunk;             // chunks per (b,h); 0 = none carved
  int chunk_tokens;       // tokens per chunk (multiple of the staging size)
  float* partA; float* partB; float* partW;  // [nchunk, BH, M, D] and [nchunk, BH, M]
};

struct DuParams {
  int B, H, M, D;
  const float* Gk; const float* Gv;   // grads w.r.t. the post-diffusion slots
  const float* K; const float* V; const float* W;  // forward sums of the round
  float alpha, gamma, eps;
  int transpose;     // apply the diffusion adjoint first
  int combine_dk;    // token keys == token values: write dKk + dKv to dk_out
  float* dk_out; float* dv_out; float* dW_out;
  float* carry_k; float* carry_v;
};

struct TokBwdParams {
  int B, H, N, D, M;
  TokView g, tk, tv;
  const uint16_t* idx; const float* w;
  const float* sv;              // g.sv term (null: absent)
  const float* dkk; const float* dkv;  // tk.dKk / tv.dKv terms (null: absent)
  const float* dW;              // [BH, M] (null: absent)
  const float* gw;              // [BH, N, 7] external weight grads (null: absent)
  float* ds_out;                // softmax backward (null: skip)
  float* dw_out;                // raw dw (null: skip)
};

struct TokGradParams {
  int B, H, N, D, M, R;
  float c;
  TokView g;                    // residual term added to dq (p == null: none)
  TokViewMut dq, dtk, dtv;      // outputs (p == null: skip)
  int shared_kv;                // w.dK terms go to dq (README form)
  const uint16_t* idx[MAX_ROUNDS];
  const float* w[MAX_ROUNDS];
  const float* ds[MAX_ROUNDS];
  const float* sk[MAX_ROUNDS];
  const float* dkk[MAX_ROUNDS];
  const float* dkv[MAX_ROUNDS];
};

struct AttendIdxParams {
  int B, H, N, D, M;
  TokView q;
  const float* sk;        // fp32 [BH, M, D]
  const uint16_t* idx;    // [BH, N, 8]
  float scale;
  float* w;               // [BH, N, 7]
};

// Compute units of the current device (cached per device; 256 if the query
// fails).  Launchers shrink their blocks when a grid would leave CUs idle.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) {
      (void)hipGetLastError();
      c = 256;
    }
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

// Records `msg` as the calling thread's murm_last_error() and returns `code`.
int set_error(int code, const char* msg);

size_t sa_lds_bytes(int dtype, int DP, int M);
hipError_t launch_select_attend(int dtype, int DP, const SAParams& p, hipStream_t st);
hipError_t launch_gather_out(int dtype, int DP, const OutParams& p, hipStream_t st);
int seg_chunks(int B, int H, int N, int M, int D, int mode);   // 0: shape not served (d > 128)
int seg_chunk_tokens(int N, int nchunk);
// stage 0: token-chunk partial sums; stage 1: chunk reduction + epilogue.
// seg_two_stage() is false when no chunk scratch was carved (launch_seg fails then).
bool seg_two_stage(int dtype, int DP, int mode, const SegParams& p, const PartParams* pp);
hipError_t launch_seg(int dtype, int DP, int mode, const SegParams& p, const PartParams* pp, int stage,
                      hipStream_t st);
hipError_t launch_du(const DuParams& p, hipStream_t st);
// token-side kernels, one translation unit per token dtype (murm_tokens.hip)
hipError_t launch_tok_bwd_f32(int DP, const TokBwdParams& p, hipStream_t st);
hipError_t launch_tok_bwd_f16(int DP, const TokBwdParams& p, hipStream_t st);
hipError_t launch_tok_bwd_bf16(int DP, const TokBwdParams& p, hipStream_t st);
hipError_t launch_tok_grad_f32(int DP, const TokGradParams& p, hipStream_t st);
hipError_t launch_tok_grad_f16(int DP, const TokGradParams& p, hipStream_t st);
hipError_t launch_tok_grad_bf16(int DP, const TokGradParams& p, hipStream_t st);
hipError_t launch_attend_idx_f32(int DP, const AttendIdxParams& p, hipStream_t st);
hipError_t launch_attend_idx_f16(int DP, const AttendIdxParams& p, hipStream_t st);
hipError_t launch_attend_idx_bf16(int DP, const AttendIdxParams& p, hipStream_t st);
inline hipError_t launch_tok_bwd(int dtype, int DP, const TokBwdParams& p, hipStream_t st) {
  return dtype == DT_F32 ? launch_tok_bwd_f32(DP, p, st)
       : dtype == DT_F16 ? launch_tok_bwd_f16(DP, p, st)
       : dtype == DT_BF16 ? launch_tok_bwd_bf16(DP, p, st) : hipErrorInvalidValue;
}
inline hipError_t launch_tok_grad(int dtype, int DP, const TokGradParams& p, hipStream_t st) {
  return dtype == DT_F32 ? launch_tok_grad_f32(DP, p, st)
       : dtype == DT_F16 ? launch_tok_grad_f16(DP, p, st)
       : dtype == DT_BF16 ? launch_tok_grad_bf16(DP, p, st) : hipErrorInvalidValue;
}
inline hipError_t launch_attend_idx(int dtype, int DP, const AttendIdxParams& p, hipStream_t st) {
  return dtype == DT_F32 ? launch_attend_idx_f32(DP, p, st)
       : dtype == DT_F16 ? launch_attend_idx_f16(DP, p, st)
       : dtype == DT_BF16 ? launch_attend_idx_bf16(DP, p, st) : hipErrorInvalidValue;
}
template <typename S, typename D>
struct SlotConv {   // one slot tensor [B,H,M,D] (element strides) <-> fp32 state [BH,M,D]
  S src;
  int64_t sb, sh, sm;   // strides of the slot tensor (src for to_state, dst for from_state)
  D dst;
};
// two conversions in one launch (b may be null); with `split` the first one
// (the slot keys) is also written split for the 16-bit select kernel
hipError_t launch_to_state2(int dtype, const SlotConv<const void*, float*>& a,
                            const SlotConv<const void*, float*>* b, int B, int H, int M, int D, hipStream_t st,
                            const KeySplitOut* split = nullptr);
hipError_t launch_from_state2(int dtype, const SlotConv<const float*, void*>& a,
                              const SlotConv<const float*, void*>* b, int B, int H, int M, int D, hipStream_t st);
hipError_t launch_to_state(int dtype, const void* src, int64_t sb, int64_t sh, int64_t sm, float* dst,
                           int B, int H, int M, int D, hipStream_t st);
hipError_t launch_from_state(int dtype, const float* src, void* dst, int64_t sb, int64_t sh, int64_t sm,
                             int B, int H, int M, int D, hipStream_t st);
hipError_t launch_idx_pack(const int64_t* src, uint16_t* dst, int64_t rows, int K, int M, hipStream_t st);
hipError_t launch_stencil(int dtype, void* x, int64_t sb, int64_t sh, int64_t sm, void* out, int64_t ob,
                          int64_t oh, int64_t om, int B, int H, int M, int D, float g, int adjoint,
                          hipStream_t st);

}  // namespace murm
