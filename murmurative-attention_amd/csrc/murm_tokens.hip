// Token-side backward kernels.
//
// tok_bwd (one round): for every token and each of its 7 slots
//   dw_j = g.sv[I_j] + tk.dKk[I_j] + tv.dKv[I_j] + dW[I_j] + gw_j
// (each term present when its table is given), then either the softmax
// backward ds_j = w_j (dw_j - sum_i w_i dw_i) or the raw dw_j.
// Sources: attend backward (reference.py:56-66 under autograd) and the
// update backward through the weights (reference.py:93-113 under autograd).
//
// tok_grad (all rounds at once): per token
//   dq  = [g] + sum_r c sum_j ds_rj sk_r[I_rj] + [shared] sum_r sum_j w_rj dK_r[I_rj]
//   dtk = sum_r sum_j w_rj dKk_r[I_rj],   dtv likewise with dKv
// Deferring these to one pass after the slot chain writes each token
// gradient once instead of read-modify-writing it every round.

#include "murm_common.h"
#include "murm_launch.h"

namespace murm {

namespace {

__device__ __forceinline__ void unpack_idx(const uint16_t* rowp, uint32_t (&sl)[KN]) {
  const uint4 ir = *reinterpret_cast<const uint4*>(rowp);
  sl[0] = ir.x & 0xFFFF; sl[1] = ir.x >> 16;
  sl[2] = ir.y & 0xFFFF; sl[3] = ir.y >> 16;
  sl[4] = ir.z & 0xFFFF; sl[5] = ir.z >> 16;
  sl[6] = ir.w & 0xFFFF;
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void tok_bwd_kernel(TokBwdParams p) {
  constexpr int DCH = DP / 8;
  constexpr int TPB = 256 / DCH;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int n = blockIdx.x * TPB + threadIdx.x / DCH;
  const int dc = threadIdx.x % DCH;
  const bool live = n < p.N;
  const int nn = live ? n : 0;
  const int d0 = dc * 8;
  const int64_t row = (int64_t)bh * p.N + nn;
  uint32_t sl[KN];
  unpack_idx(p.idx + row * IDX_ROW, sl);
  const int64_t tb = (int64_t)bh * p.M * p.D;

  float g[8], a[8], c[8];
  const bool has_g = p.sv != nullptr;
  const bool has_k = p.dkk != nullptr;
  const bool has_v = p.dkv != nullptr;
  if (has_g) load8<T>(tok_row<T>(p.g, b, h, nn), d0, p.D, p.g.vec, g);
  if (has_k) load8<T>(tok_row<T>(p.tk, b, h, nn), d0, p.D, p.tk.vec, a);
  if (has_v) load8<T>(tok_row<T>(p.tv, b, h, nn), d0, p.D, p.tv.vec, c);

  float dw[KN];
#pragma unroll
  for (int j = 0; j < KN; ++j) {
    float s = 0.f, v[8];
    if (has_g) {
      load8f(p.sv + tb + (int64_t)sl[j] * p.D, d0, p.D, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += g[i] * v[i];
    }
    if (has_k) {
      load8f(p.dkk + tb + (int64_t)sl[j] * p.D, d0, p.D, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += a[i] * v[i];
    }
    if (has_v) {
      load8f(p.dkv + tb + (int64_t)sl[j] * p.D, d0, p.D, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += c[i] * v[i];
    }
    dw[j] = s;
  }
#pragma unroll
  for (int x = 1; x < DCH; x <<= 1)
#pragma unroll
    for (int j = 0; j < KN; ++j) dw[j] += shfl_xor_f(dw[j], x);
  if (!live || dc != 0) return;
#pragma unroll
  for (int j = 0; j < KN; ++j) {
    if (p.dW) dw[j] += p.dW[(int64_t)bh * p.M + sl[j]];
    if (p.gw) dw[j] += p.gw[row * KN + j];
  }
  if (p.dw_out) {
#pragma unroll
    for (int j = 0; j < KN; ++j) p.dw_out[row * KN + j] = dw[j];
  }
  if (p.ds_out) {
    const float* w = p.w + row * KN;
    float wj[KN], dot = 0.f;
#pragma unroll
    for (int j = 0; j < KN; ++j) { wj[j] = w[j]; dot += wj[j] * dw[j]; }
#pragma unroll
    for (int j = 0; j < KN; ++j) p.ds_out[row * KN + j] = wj[j] * (dw[j] - dot);
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void tok_grad_kernel(TokGradParams p) {
  constexpr int DCH = DP / 8;
  constexpr int TPB = 256 / DCH;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int n = blockIdx.x * TPB + threadIdx.x / DCH;
  const int dc = threadIdx.x % DCH;
  if (n >= p.N) return;
  const int d0 = dc * 8;
  const int64_t row = (int64_t)bh * p.N + n;
  const int64_t tb = (int64_t)bh * p.M * p.D;
  float aq[8], ak[8], av[8];
  if (p.g.p) {
    load8<T>(tok_row<T>(p.g, b, h, n), d0, p.D, p.g.vec, aq);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) aq[i] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) { ak[i] = 0.f; av[i] = 0.f; }
  for (int r = 0; r < p.R; ++r) {
    uint32_t sl[KN];
    unpack_idx(p.idx[r] + row * IDX_ROW, sl);
    const float* wr = p.w[r] + row * KN;
    const float* dsr = p.ds[r] ? p.ds[r] + row * KN : nullptr;
#pragma unroll
    for (int j = 0; j < KN; ++j) {
      float v[8];
      const int64_t so = tb + (int64_t)sl[j] * p.D;
      if (dsr && p.dq.p) {
        const float cj = p.c * dsr[j];
        load8f(p.sk[r] + so, d0, p.D, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) aq[i] += cj * v[i];
      }
      const float wj = wr[j];
      if (p.dkk[r]) {
        load8f(p.dkk[r] + so, d0, p.D, v);
        if (p.shared_kv) {
#pragma unroll
          for (int i = 0; i < 8; ++i) aq[i] += wj * v[i];
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) ak[i] += wj * v[i];
        }
      }
      if (p.dkv[r]) {
        load8f(p.dkv[r] + so, d0, p.D, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) av[i] += wj * v[i];
      }
    }
  }
  if (p.dq.p) store8<T>(tok_row_mut<T>(p.dq, b, h, n), d0, p.D, p.dq.vec, aq);
  if (p.dtk.p) store8<T>(tok_row_mut<T>(p.dtk, b, h, n), d0, p.D, p.dtk.vec, ak);
  if (p.dtv.p) store8<T>(tok_row_mut<T>(p.dtv, b, h, n), d0, p.D, p.dtv.vec, av);
}

// Softmax weights for given indices: w_j = softmax_j(c * q.sk[I_j])
// (reference.py:42-68 with the indices supplied by the caller).
template <typename T, int DP>
__global__ __launch_bounds__(256) void attend_idx_kernel(AttendIdxParams p) {
  constexpr int DCH = DP / 8;
  constexpr int TPB = 256 / DCH;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int n = blockIdx.x * TPB + threadIdx.x / DCH;
  const int dc = threadIdx.x % DCH;
  const bool live = n < p.N;
  const int nn = live ? n : 0;
  const int d0 = dc * 8;
  const int64_t row = (int64_t)bh * p.N + nn;
  uint32_t sl[KN];
  unpack_idx(p.idx + row * IDX_ROW, sl);
  float q[8];
  load8<T>(tok_row<T>(p.q, b, h, nn), d0, p.D, p.q.vec, q);
  const int64_t tb = (int64_t)bh * p.M * p.D;
  float s[KN];
#pragma unroll
  for (int j = 0; j < KN; ++j) {
    float v[8];
    load8f(p.sk + tb + (int64_t)sl[j] * p.D, d0, p.D, v);
    s[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s[j] += q[i] * v[i];
  }
#pragma unroll
  for (int x = 1; x < DCH; x <<= 1)
#pragma unroll
    for (int j = 0; j < KN; ++j) s[j] += shfl_xor_f(s[j], x);
  if (!live || dc != 0) return;
  float zmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < KN; ++j) { s[j] *= p.scale; zmax = fmaxf(zmax, s[j]); }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < KN; ++j) { s[j] = __expf(s[j] - zmax); sum += s[j]; }
  const float inv = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < KN; ++j) p.w[row * KN + j] = s[j] * inv;
}

template <typename T, int DP>
hipError_t launch_attend_idx_t(const AttendIdxParams& p, hipStream_t st) {
  constexpr int TPB = 256 / (DP / 8);
  dim3 grid((p.N + TPB - 1) / TPB, p.B * p.H);
  hipLaunchKernelGGL((attend_idx_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, int DP>
hipError_t launch_tok_bwd_t(const TokBwdParams& p, hipStream_t st) {
  constexpr int TPB = 256 / (DP / 8);
  dim3 grid((p.N + TPB - 1) / TPB, p.B * p.H);
  hipLaunchKernelGGL((tok_bwd_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, int DP>
hipError_t launch_tok_grad_t(const TokGradParams& p, hipStream_t st) {
  constexpr int TPB = 256 / (DP / 8);
  dim3 grid((p.N + TPB - 1) / TPB, p.B * p.H);
  hipLaunchKernelGGL((tok_grad_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_tok_bwd(int dtype, int DP, const TokBwdParams& p, hipStream_t st) {
#define MURM_TB(T)                                            \
  switch (DP) {                                               \
    case 32: return launch_tok_bwd_t<T, 32>(p, st);           \
    case 64: return launch_tok_bwd_t<T, 64>(p, st);           \
    case 128: return launch_tok_bwd_t<T, 128>(p, st);         \
    default: return hipErrorInvalidValue;                     \
  }
  switch (dtype) {
    case DT_BF16: MURM_TB(__bf16)
    case DT_F16: MURM_TB(_Float16)
    case DT_F32: MURM_TB(float)
    default: return hipErrorInvalidValue;
  }
#undef MURM_TB
}

hipError_t launch_attend_idx(int dtype, int DP, const AttendIdxParams& p, hipStream_t st) {
#define MURM_AI(T)                                            \
  switch (DP) {                                               \
    case 32: return launch_attend_idx_t<T, 32>(p, st);        \
    case 64: return launch_attend_idx_t<T, 64>(p, st);        \
    case 128: return launch_attend_idx_t<T, 128>(p, st);      \
    default: return hipErrorInvalidValue;                     \
  }
  switch (dtype) {
    case DT_BF16: MURM_AI(__bf16)
    case DT_F16: MURM_AI(_Float16)
    case DT_F32: MURM_AI(float)
    default: return hipErrorInvalidValue;
  }
#undef MURM_AI
}

hipError_t launch_tok_grad(int dtype, int DP, const TokGradParams& p, hipStream_t st) {
#define MURM_TG(T)                                            \
  switch (DP) {                                               \
    case 32: return launch_tok_grad_t<T, 32>(p, st);          \
    case 64: return launch_tok_grad_t<T, 64>(p, st);          \
    case 128: return launch_tok_grad_t<T, 128>(p, st);        \
    default: return hipErrorInvalidValue;                     \
  }
  switch (dtype) {
    case DT_BF16: MURM_TG(__bf16)
    case DT_F16: MURM_TG(_Float16)
    case DT_F32: MURM_TG(float)
    default: return hipErrorInvalidValue;
  }
#undef MURM_TG
}

}  // namespace murm
