// Slot-side kernels: deterministic per-slot reductions and the small
// per-slot epilogues.
//
// seg_reduce: one block owns a group of GS = 16 slots of one (b,h) (plus one
// halo slot on each side when the forward diffusion follows).  It scans the
// round's (token, j) -> slot entries in chunks of 1024 tokens, builds for its
// slots a list of matching entries ordered by token (64-bit LDS bitmasks per
// 64-token group give each entry its rank; integer OR is order-free, so the
// list is the same on every run), and sums the token rows of each list in
// that order with a fixed butterfly at the end.  No float atomics: the
// result is bitwise reproducible.  Two modes:
//   UPDATE   K_m = sum w*tk, V_m = sum w*tv, W_m = sum w, then the EMA
//            (reference.py:86-115) and, with diffusion, the stencil over the
//            post-update rows (reference.py:118-135, 188-189).
//   ATTBWD   dsk_m = carry_k + c * sum ds*q,  dsv_m = carry_v + sum w*g
//            (attend backward, slot side; carry is the update backward's
//            pass-through term).
// du_kernel: diffusion adjoint + EMA backward for one round (per slot):
//   G' = D^T G'', dK = (1-a)/(W+eps) G', dW = -(1-a)(K.G'k + V.G'v)/(W+eps)^2,
//   carry = a G' on used slots, G' elsewhere.

#include "murm_common.h"
#include "murm_launch.h"

namespace murm {

namespace {

constexpr int GS = 16;             // owned slots per block
constexpr int NSMAX = GS + 2;      // with halo
constexpr int CH = 1024;           // tokens per chunk
constexpr int NGRP = CH / 64;      // 64-token groups per chunk
constexpr int SPW = (NSMAX + 3) / 4;  // slots per wave (round robin)

struct SegShared {
  unsigned long long masks[NGRP][NSMAX];
  uint16_t goff[NGRP][NSMAX];
  int cnt[NSMAX];
  int loff[NSMAX];
  uint16_t list[CH * IDX_ROW];
};

template <typename T, int DP, int MODE>
__device__ void seg_accumulate(const SegParams& p, int bh, int lo, int NS, SegShared& sh,
                               float* accA, float* accB, float* accW) {
  constexpr int DCH = DP / 8;        // 8-dim chunks
  constexpr int ES = 64 / DCH;       // entries in flight per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int es = lane / DCH, dc = lane % DCH;
  const int d0 = dc * 8;
  const int b = bh / p.H, h = bh % p.H;
  const bool sameB = (MODE == SEG_UPDATE) && p.b_same_as_a;

  float aA[SPW][8], aB[SPW][8], aW[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    aW[s] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) { aA[s][i] = 0.f; aB[s][i] = 0.f; }
  }

  const uint16_t* idxb = p.idx + (int64_t)bh * p.N * IDX_ROW;
  const float* wb = p.wgt + (int64_t)bh * p.N * p.K;
  const float* db = (MODE == SEG_ATTBWD) ? p.ds + (int64_t)bh * p.N * p.K : nullptr;

  for (int c0 = 0; c0 < p.N; c0 += CH) {
    for (int i = tid; i < NGRP * NSMAX; i += blockDim.x) (&sh.masks[0][0])[i] = 0ull;
    __syncthreads();
    uint4 rows[CH / 256];
#pragma unroll
    for (int i = 0; i < CH / 256; ++i) {
      const int n = c0 + i * 256 + tid;
      rows[i] = (n < p.N) ? *reinterpret_cast<const uint4*>(idxb + (int64_t)n * IDX_ROW)
                          : make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
      const uint32_t wv[4] = {rows[i].x, rows[i].y, rows[i].z, rows[i].w};
      const int grp = i * 4 + wave;
#pragma unroll
      for (int j = 0; j < KN + 1; ++j) {
        if (j >= p.K) break;
        const uint32_t s = (wv[j >> 1] >> (16 * (j & 1))) & 0xFFFF;
        const uint32_t rel = s - (uint32_t)lo;
        if (s != IDX_NONE && rel < (uint32_t)NS) atomicOr(&sh.masks[grp][rel], 1ull << lane);
      }
    }
    __syncthreads();
    if (tid < NS) {
      int run = 0;
      for (int g = 0; g < NGRP; ++g) {
        sh.goff[g][tid] = (uint16_t)run;
        run += __popcll(sh.masks[g][tid]);
      }
      sh.cnt[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
      int o = 0;
      for (int s = 0; s < NS; ++s) { sh.loff[s] = o; o += sh.cnt[s]; }
    }
    __syncthreads();
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int i = 0; i < CH / 256; ++i) {
      const uint32_t wv[4] = {rows[i].x, rows[i].y, rows[i].z, rows[i].w};
      const int grp = i * 4 + wave;
#pragma unroll
      for (int j = 0; j < KN + 1; ++j) {
        if (j >= p.K) break;
        const uint32_t s = (wv[j >> 1] >> (16 * (j & 1))) & 0xFFFF;
        const uint32_t rel = s - (uint32_t)lo;
        if (s != IDX_NONE && rel < (uint32_t)NS) {
          const int pos = sh.loff[rel] + sh.goff[grp][rel] + __popcll(sh.masks[grp][rel] & below);
          sh.list[pos] = (uint16_t)(((i * 256 + tid) << 3) | j);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int rel = wave + 4 * s;
      if (rel >= NS) break;
      const int beg = sh.loff[rel], end = beg + sh.cnt[rel];
      for (int e = beg + es; e < end; e += ES) {
        const uint32_t ent = sh.list[e];
        const int n = c0 + (int)(ent >> 3);
        const int j = (int)(ent & 7);
        const float w = wb[(int64_t)n * p.K + j];
        float va[8];
        load8<T>(tok_row<T>(p.va, b, h, n), d0, p.D, p.va.vec, va);
        if constexpr (MODE == SEG_UPDATE) {
#pragma unroll
          for (int i = 0; i < 8; ++i) aA[s][i] += w * va[i];
          aW[s] += w;
          if (!sameB) {
            float vb[8];
            load8<T>(tok_row<T>(p.vb, b, h, n), d0, p.D, p.vb.vec, vb);
#pragma unroll
            for (int i = 0; i < 8; ++i) aB[s][i] += w * vb[i];
          }
        } else {
          const float ca = p.ds_scale * db[(int64_t)n * p.K + j];
          float vb[8];
          load8<T>(tok_row<T>(p.vb, b, h, n), d0, p.D, p.vb.vec, vb);
#pragma unroll
          for (int i = 0; i < 8; ++i) { aA[s][i] += ca * va[i]; aB[s][i] += w * vb[i]; }
        }
      }
    }
    __syncthreads();
  }

  // fixed butterfly over the entry lanes, then lanes with es == 0 publish
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    const int rel = wave + 4 * s;
#pragma unroll
    for (int x = DCH; x < 64; x <<= 1) {
      aW[s] += shfl_xor_f(aW[s], x);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        aA[s][i] += shfl_xor_f(aA[s][i], x);
        aB[s][i] += shfl_xor_f(aB[s][i], x);
      }
    }
    if (rel < NS && es == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        accA[rel * DP + d0 + i] = aA[s][i];
        accB[rel * DP + d0 + i] = sameB ? aA[s][i] : aB[s][i];
      }
      if (dc == 0) accW[rel] = aW[s];
    }
  }
  __syncthreads();
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void seg_update_kernel(SegParams p) {
  __shared__ SegShared sh;
  __shared__ float accA[NSMAX * DP], accB[NSMAX * DP], accW[NSMAX];
  const int bh = blockIdx.y;
  const int g0 = blockIdx.x * GS;
  const int halo = p.diffuse ? 1 : 0;
  const int lo = g0 - halo;
  const int NS = GS + 2 * halo;
  seg_accumulate<T, DP, SEG_UPDATE>(p, bh, lo, NS, sh, accA, accB, accW);

  const int64_t base = (int64_t)bh * p.M * p.D;
  const float a = p.alpha, oma = 1.0f - p.alpha;
  // raw sums of the owned rows (kept for the backward)
  for (int i = threadIdx.x; i < GS * DP; i += blockDim.x) {
    const int own = i / DP, d = i % DP, m = g0 + own;
    if (m >= p.M || d >= p.D) continue;
    const int j = (own + halo) * DP + d;
    if (p.ksum) p.ksum[base + (int64_t)m * p.D + d] = accA[j];
    if (p.vsum) p.vsum[base + (int64_t)m * p.D + d] = accB[j];
    if (p.wsum && d == 0) p.wsum[(int64_t)bh * p.M + m] = accW[own + halo];
  }
  if (!p.sk_new) return;
  __syncthreads();
  // EMA on every row the block holds (owned + halo)
  for (int i = threadIdx.x; i < NS * DP; i += blockDim.x) {
    const int rel = i / DP, d = i % DP, m = lo + rel;
    if (m < 0 || m >= p.M || d >= p.D) continue;
    const float W = accW[rel];
    const float ok = p.sk_old[base + (int64_t)m * p.D + d];
    const float ov = p.sv_old[base + (int64_t)m * p.D + d];
    if (W > 0.f) {
      const float inv = 1.0f / (W + p.eps);
      accA[i] = a * ok + oma * (accA[i] * inv);
      accB[i] = a * ov + oma * (accB[i] * inv);
    } else {
      accA[i] = ok;
      accB[i] = ov;
    }
  }
  __syncthreads();
  const float gm = p.gamma;
  for (int i = threadIdx.x; i < GS * DP; i += blockDim.x) {
    const int own = i / DP, d = i % DP, m = g0 + own;
    if (m >= p.M || d >= p.D) continue;
    const int rel = own + halo;
    float yk = accA[rel * DP + d], yv = accB[rel * DP + d];
    if (p.diffuse && m >= 1 && m <= p.M - 2) {
      yk = yk + gm * (accA[(rel - 1) * DP + d] + accA[(rel + 1) * DP + d] - 2.0f * yk);
      yv = yv + gm * (accB[(rel - 1) * DP + d] + accB[(rel + 1) * DP + d] - 2.0f * yv);
    }
    p.sk_new[base + (int64_t)m * p.D + d] = yk;
    p.sv_new[base + (int64_t)m * p.D + d] = yv;
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void seg_attbwd_kernel(SegParams p) {
  __shared__ SegShared sh;
  __shared__ float accA[NSMAX * DP], accB[NSMAX * DP], accW[NSMAX];
  const int bh = blockIdx.y;
  const int g0 = blockIdx.x * GS;
  seg_accumulate<T, DP, SEG_ATTBWD>(p, bh, g0, GS, sh, accA, accB, accW);
  const int64_t base = (int64_t)bh * p.M * p.D;
  for (int i = threadIdx.x; i < GS * DP; i += blockDim.x) {
    const int own = i / DP, d = i % DP, m = g0 + own;
    if (m >= p.M || d >= p.D) continue;
    const int64_t o = base + (int64_t)m * p.D + d;
    p.gk_out[o] = (p.carry_k ? p.carry_k[o] : 0.f) + accA[i];
    p.gv_out[o] = (p.carry_v ? p.carry_v[o] : 0.f) + accB[i];
  }
}

// One block per (b,h): G' = D^T G'' (optional), then the EMA backward.
__global__ __launch_bounds__(256) void du_kernel(DuParams p) {
  const int bh = blockIdx.x;
  const int64_t base = (int64_t)bh * p.M * p.D;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float g = p.gamma, a = p.alpha, oma = 1.0f - p.alpha;
  for (int m = wave; m < p.M; m += 4) {
    float dot = 0.f;
    const float W = p.W[(int64_t)bh * p.M + m];
    const bool used = W > 0.f;
    const float inv = oma / (W + p.eps);
    for (int d = lane; d < p.D; d += 64) {
      auto gp = [&](const float* G) {
        const float c = G[base + (int64_t)m * p.D + d];
        if (!p.transpose || p.M < 3) return c;
        float r = c;
        if (m >= 1 && m <= p.M - 2) r -= 2.0f * g * c;
        if (m - 1 >= 1 && m - 1 <= p.M - 2) r += g * G[base + (int64_t)(m - 1) * p.D + d];
        if (m + 1 >= 1 && m + 1 <= p.M - 2) r += g * G[base + (int64_t)(m + 1) * p.D + d];
        return r;
      };
      const float gk = gp(p.Gk), gv = gp(p.Gv);
      const int64_t o = base + (int64_t)m * p.D + d;
      if (used) dot += p.K[o] * gk + p.V[o] * gv;
      const float dk = used ? inv * gk : 0.f, dv = used ? inv * gv : 0.f;
      if (p.combine_dk) {
        p.dk_out[o] = dk + dv;
      } else {
        p.dk_out[o] = dk;
        p.dv_out[o] = dv;
      }
      p.carry_k[o] = used ? a * gk : gk;
      p.carry_v[o] = used ? a * gv : gv;
    }
#pragma unroll
    for (int x = 1; x < 64; x <<= 1) dot += shfl_xor_f(dot, x);
    if (lane == 0) {
      const float den = W + p.eps;
      p.dW_out[(int64_t)bh * p.M + m] = used ? -oma * dot / (den * den) : 0.f;
    }
  }
}

// fp32 state [BH,M,D] from a [B,H,M,D] slot tensor of any dtype and strides
template <typename T>
__global__ void to_state_kernel(const T* __restrict__ src, int64_t sb, int64_t sh, int64_t sm,
                                float* __restrict__ dst, int B, int H, int M, int D) {
  const int64_t total = (int64_t)B * H * M * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    int64_t r = i / D;
    const int m = (int)(r % M);
    r /= M;
    const int h = (int)(r % H);
    const int b = (int)(r / H);
    dst[i] = to_f(src[b * sb + h * sh + m * sm + d]);
  }
}

template <typename T>
__global__ void from_state_kernel(const float* __restrict__ src, T* __restrict__ dst, int64_t sb,
                                  int64_t sh, int64_t sm, int B, int H, int M, int D) {
  const int64_t total = (int64_t)B * H * M * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    int64_t r = i / D;
    const int m = (int)(r % M);
    r /= M;
    const int h = (int)(r % H);
    const int b = (int)(r / H);
    dst[b * sb + h * sh + m * sm + d] = from_f<T>(src[i]);
  }
}

// int64 [BH,N,K] indices (contiguous) -> u16 rows of 8, clamped to [0, M-1]
__global__ void idx_pack_kernel(const int64_t* __restrict__ src, uint16_t* __restrict__ dst,
                                int64_t rows, int K, int M) {
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * blockDim.x) {
    uint16_t o[IDX_ROW];
#pragma unroll
    for (int j = 0; j < IDX_ROW; ++j) {
      if (j < K) {
        int64_t v = src[r * K + j];
        v = v < 0 ? 0 : (v > M - 1 ? M - 1 : v);
        o[j] = (uint16_t)v;
      } else {
        o[j] = IDX_NONE;
      }
    }
    uint4 pk;
    pk.x = o[0] | ((uint32_t)o[1] << 16);
    pk.y = o[2] | ((uint32_t)o[3] << 16);
    pk.z = o[4] | ((uint32_t)o[5] << 16);
    pk.w = o[6] | ((uint32_t)o[7] << 16);
    *reinterpret_cast<uint4*>(dst + r * IDX_ROW) = pk;
  }
}

// In-place Jacobi stencil (or its adjoint into `out`) along M; one thread
// walks one (b,h,d) column keeping the neighbours it has overwritten.
template <typename T>
__global__ void stencil_kernel(T* __restrict__ x, int64_t sb, int64_t sh, int64_t sm, T* __restrict__ out,
                               int64_t ob, int64_t oh, int64_t om, int B, int H, int M, int D,
                               float g, int adjoint) {
  const int64_t col = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (col >= (int64_t)B * H * D) return;
  const int d = (int)(col % D);
  const int h = (int)((col / D) % H);
  const int b = (int)(col / ((int64_t)D * H));
  T* xc = x + b * sb + h * sh + d;
  T* oc = out + b * ob + h * oh + d;
  auto in = [&](int m) { return to_f(xc[m * sm]); };
  auto inner = [&](int m) { return m >= 1 && m <= M - 2; };
  if (!adjoint) {
    if (M < 3) {
      for (int m = 0; m < M; ++m) oc[m * om] = xc[m * sm];
      return;
    }
    float prev = in(0), cur = in(1);
    oc[0] = from_f<T>(prev);
    for (int m = 1; m <= M - 2; ++m) {
      const float next = in(m + 1);
      oc[m * om] = from_f<T>(cur + g * (prev + next - 2.0f * cur));
      prev = cur;
      cur = next;
    }
    oc[(M - 1) * om] = from_f<T>(cur);
  } else {
    for (int m = 0; m < M; ++m) {
      float r = in(m);
      if (M >= 3) {
        if (inner(m)) r -= 2.0f * g * in(m);
        if (m - 1 >= 0 && inner(m - 1)) r += g * in(m - 1);
        if (m + 1 < M && inner(m + 1)) r += g * in(m + 1);
      }
      oc[m * om] = from_f<T>(r);
    }
  }
}

template <typename T, int DP>
hipError_t launch_seg_t(const SegParams& p, int mode, hipStream_t st) {
  dim3 grid((p.M + GS - 1) / GS, p.B * p.H);
  if (mode == SEG_UPDATE)
    hipLaunchKernelGGL((seg_update_kernel<T, DP>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((seg_attbwd_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

inline int grid1d(int64_t n, int tpb = 256) {
  int64_t g = (n + tpb - 1) / tpb;
  return (int)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

}  // namespace

hipError_t launch_seg(int dtype, int DP, int mode, const SegParams& p, hipStream_t st) {
#define MURM_SEG(T)                                           \
  switch (DP) {                                               \
    case 32: return launch_seg_t<T, 32>(p, mode, st);         \
    case 64: return launch_seg_t<T, 64>(p, mode, st);         \
    case 128: return launch_seg_t<T, 128>(p, mode, st);       \
    default: return hipErrorInvalidValue;                     \
  }
  switch (dtype) {
    case DT_BF16: MURM_SEG(__bf16)
    case DT_F16: MURM_SEG(_Float16)
    case DT_F32: MURM_SEG(float)
    default: return hipErrorInvalidValue;
  }
#undef MURM_SEG
}

hipError_t launch_du(const DuParams& p, hipStream_t st) {
  hipLaunchKernelGGL(du_kernel, dim3(p.B * p.H), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_to_state(int dtype, const void* src, int64_t sb, int64_t sh, int64_t sm, float* dst,
                           int B, int H, int M, int D, hipStream_t st) {
  const int g = grid1d((int64_t)B * H * M * D);
  switch (dtype) {
    case DT_BF16: hipLaunchKernelGGL((to_state_kernel<__bf16>), dim3(g), dim3(256), 0, st,
                                     (const __bf16*)src, sb, sh, sm, dst, B, H, M, D); break;
    case DT_F16: hipLaunchKernelGGL((to_state_kernel<_Float16>), dim3(g), dim3(256), 0, st,
                                    (const _Float16*)src, sb, sh, sm, dst, B, H, M, D); break;
    case DT_F32: hipLaunchKernelGGL((to_state_kernel<float>), dim3(g), dim3(256), 0, st,
                                    (const float*)src, sb, sh, sm, dst, B, H, M, D); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_from_state(int dtype, const float* src, void* dst, int64_t sb, int64_t sh, int64_t sm,
                             int B, int H, int M, int D, hipStream_t st) {
  const int g = grid1d((int64_t)B * H * M * D);
  switch (dtype) {
    case DT_BF16: hipLaunchKernelGGL((from_state_kernel<__bf16>), dim3(g), dim3(256), 0, st,
                                     src, (__bf16*)dst, sb, sh, sm, B, H, M, D); break;
    case DT_F16: hipLaunchKernelGGL((from_state_kernel<_Float16>), dim3(g), dim3(256), 0, st,
                                    src, (_Float16*)dst, sb, sh, sm, B, H, M, D); break;
    case DT_F32: hipLaunchKernelGGL((from_state_kernel<float>), dim3(g), dim3(256), 0, st,
                                    src, (float*)dst, sb, sh, sm, B, H, M, D); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_idx_pack(const int64_t* src, uint16_t* dst, int64_t rows, int K, int M, hipStream_t st) {
  hipLaunchKernelGGL(idx_pack_kernel, dim3(grid1d(rows)), dim3(256), 0, st, src, dst, rows, K, M);
  return hipGetLastError();
}

hipError_t launch_stencil(int dtype, void* x, int64_t sb, int64_t sh, int64_t sm, void* out, int64_t ob,
                          int64_t oh, int64_t om, int B, int H, int M, int D, float g, int adjoint,
                          hipStream_t st) {
  const int64_t cols = (int64_t)B * H * D;
  const int grid = (int)((cols + 255) / 256);
  switch (dtype) {
    case DT_BF16: hipLaunchKernelGGL((stencil_kernel<__bf16>), dim3(grid), dim3(256), 0, st, (__bf16*)x,
                                     sb, sh, sm, (__bf16*)out, ob, oh, om, B, H, M, D, g, adjoint); break;
    case DT_F16: hipLaunchKernelGGL((stencil_kernel<_Float16>), dim3(grid), dim3(256), 0, st, (_Float16*)x,
                                    sb, sh, sm, (_Float16*)out, ob, oh, om, B, H, M, D, g, adjoint); break;
    case DT_F32: hipLaunchKernelGGL((stencil_kernel<float>), dim3(grid), dim3(256), 0, st, (float*)x,
                                    sb, sh, sm, (float*)out, ob, oh, om, B, H, M, D, g, adjoint); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace murm
