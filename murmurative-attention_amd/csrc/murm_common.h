// Shared device helpers for the gfx950 slot_murmurate kernels.
//
// Layout conventions used by every kernel in this directory:
//   * Token tensors (q, x, k/v projections, grad_out, grad_q) are addressed as
//     base + b*sb + h*sh + n*sn + d (element strides, d contiguous), so the
//     [B,H,N,D] README layout and the [B,N,H,Dh] legacy views both work
//     without a copy.
//   * Slot state between rounds is float32, contiguous [B*H, M, D].
//   * Per-round indices are uint16 rows of 8 (7 used, the 8th is IDX_NONE),
//     contiguous [B*H, N, 8]; weights are float32 [B*H, N, 7].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace murm {

constexpr int KN = 7;                 // slots per token (reference.py:38, k=7)
constexpr int IDX_ROW = 8;            // padded index row (u16)
constexpr uint16_t IDX_NONE = 0xFFFF; // never matches a slot
constexpr int MAX_ROUNDS = 16;

enum DType : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- scalars ---

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

// 8 consecutive elements of a token row, converted to float; elements at
// d >= D read as zero.  `vec` says the row start is 16-byte aligned and the
// full 8 elements are in range, so one wide load can be used.
template <typename T>
__device__ __forceinline__ void load8(const T* __restrict__ row, int d0, int D, bool vec, float (&o)[8]) {
  if (vec && d0 + 8 <= D) {
    if constexpr (sizeof(T) == 2) {
      uint4 raw = *reinterpret_cast<const uint4*>(row + d0);
      const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = to_f(e[i]);
    } else {
      float4 a = *reinterpret_cast<const float4*>(row + d0);
      float4 b = *reinterpret_cast<const float4*>(row + d0 + 4);
      o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
      o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (d0 + i < D) ? to_f(row[d0 + i]) : 0.f;
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* __restrict__ row, int d0, int D, bool vec, const float (&v)[8]) {
  if (vec && d0 + 8 <= D) {
    if constexpr (sizeof(T) == 2) {
      uint4 raw;
      T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = from_f<T>(v[i]);
      *reinterpret_cast<uint4*>(row + d0) = raw;
    } else {
      *reinterpret_cast<float4*>(row + d0) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(row + d0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (d0 + i < D) row[d0 + i] = from_f<T>(v[i]);
  }
}

// 8 floats from fp32 slot state (rows are D floats; D % 4 == 0 for the vector path)
__device__ __forceinline__ void load8f(const float* __restrict__ row, int d0, int D, float (&o)[8]) {
  if (d0 + 8 <= D && (D & 3) == 0) {
    float4 a = *reinterpret_cast<const float4*>(row + d0);
    float4 b = *reinterpret_cast<const float4*>(row + d0 + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (d0 + i < D) ? row[d0 + i] : 0.f;
  }
}

// ------------------------------------------------------------ wave ops ---

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Sum over aligned groups of G lanes (G = 2, 4, 8, 16), every lane of a group
// receiving the same total, with DPP lane moves (no LDS round trip):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.  The
// adds pair lanes as a xor-1/2/4/8 butterfly, so the result is bitwise the
// same in every lane of the group.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group of 1, 2, 4, 8 or 16 lanes");
  if constexpr (G >= 2) v += dpp_mov<0xB1>(v);
  if constexpr (G >= 4) v += dpp_mov<0x4E>(v);
  if constexpr (G >= 8) v += dpp_mov<0x141>(v);
  if constexpr (G >= 16) v += dpp_mov<0x140>(v);
  return v;
}

// ---------------------------------------------------- packed top-k keys ---
// A selection key is the float score with its low `bits` mantissa bits
// replaced by the slot index.  Float max/med3 then carry the index with the
// score, so inserting one score into a sorted top-7 list is 1 max + 6 med3.
// Truncation costs 2^-(23-bits) relative precision, far below the 1e-3
// relative gap at which an index is considered decided.  Masked scores use
// -FLT_MAX (finite, so the index bits survive); padding uses -inf, which can
// never be selected while M >= 7.

__device__ __forceinline__ float make_key(float s, uint32_t hi_mask, uint32_t m) {
  return __uint_as_float((__float_as_uint(s) & hi_mask) | m);
}
__device__ __forceinline__ uint32_t key_slot(float k, uint32_t lo_mask) {
  return __float_as_uint(k) & lo_mask;
}
__device__ __forceinline__ float key_score(float k, uint32_t hi_mask) {
  return __uint_as_float(__float_as_uint(k) & hi_mask);
}
constexpr float MASKED_SCORE = -3.4028234663852886e38f;  // -FLT_MAX
__device__ __forceinline__ bool key_masked(float k) { return k <= -1.0e38f; }

// Insert x into the descending list a (keeps the K largest): one med3 per
// entry and one max for the head, as a plain v_max_f32 (fmaxf would add
// NaN-quieting maxes on both operands; keys here are finite or -inf).
__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float min_raw(float a, float b) {
  float r;
  asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
template <int K>
__device__ __forceinline__ void topk_insert(float (&a)[K], float x) {
#pragma unroll
  for (int j = K - 1; j >= 1; --j) a[j] = __builtin_amdgcn_fmed3f(a[j - 1], a[j], x);
  a[0] = max_raw(a[0], x);
}

// The 7 largest of two descending lists of 7, descending.  c_j =
// max(a_j, b_{6-j}) holds them as a V-shaped (bitonic) sequence; with +inf
// appended it stays bitonic, and the 8-wide bitonic merge network (distance
// 4, 2, 1) sorts it.  The +inf entry only moves one element per stage, so
// 7 max + 9 compare-exchanges = 25 VALU (7 insertions would take 49).
__device__ __forceinline__ void ce_raw(float& hi, float& lo) {
  const float h = max_raw(hi, lo), l = min_raw(hi, lo);
  hi = h;
  lo = l;
}
__device__ __forceinline__ void top7_merge(const float (&a)[7], const float (&b)[7], float (&out)[7]) {
  float c[8];
#pragma unroll
  for (int j = 0; j < 7; ++j) c[j] = max_raw(a[j], b[6 - j]);
  ce_raw(c[0], c[4]); ce_raw(c[1], c[5]); ce_raw(c[2], c[6]); c[7] = c[3];  // c[3] <- +inf
  ce_raw(c[0], c[2]); c[3] = c[1]; ce_raw(c[4], c[6]); ce_raw(c[5], c[7]);  // c[1] <- +inf
  ce_raw(c[2], c[3]); ce_raw(c[4], c[5]); ce_raw(c[6], c[7]);               // c[0] -> second
  out[0] = c[0]; out[1] = c[2]; out[2] = c[3]; out[3] = c[4];
  out[4] = c[5]; out[5] = c[6]; out[6] = c[7];
}

// Values of lanes l and l ^ X (X = 16 or 32) without an LDS round trip:
// v_permlane{16,32}_swap_b32 on two copies of v exchange the odd rows (X = 16)
// or the upper half (X = 32) of the first copy with the even rows / lower half
// of the second, so both lanes of a pair end up holding (value of the lower
// lane, value of the upper lane) in the same order.
template <int X>
__device__ __forceinline__ void lane_pair(float v, float& lower, float& upper) {
  const uint32_t u = __float_as_uint(v);
  if constexpr (X == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    lower = __uint_as_float(r[0]);
    upper = __uint_as_float(r[1]);
  } else {
    static_assert(X == 32, "lane_pair: X is 16 or 32");
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lower = __uint_as_float(r[0]);
    upper = __uint_as_float(r[1]);
  }
}

// ------------------------------------------------------------------ MFMA ---

__device__ __forceinline__ f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Operand element type of the 16-bit MFMA for a token dtype.
template <typename T> struct Mfma16;
template <> struct Mfma16<__bf16> { using elem = __bf16; using vec = bf16x8; };
template <> struct Mfma16<_Float16> { using elem = _Float16; using vec = f16x8; };

// -------------------------------------------------------------- strides ---

struct TokView {      // a [B,H,N,D] view of a token tensor
  const void* p;
  int64_t sb, sh, sn;  // element strides
  int vec;             // 16-byte aligned rows (wide loads allowed)
};
struct TokViewMut {
  void* p;
  int64_t sb, sh, sn;
  int vec;
};

template <typename T>
__device__ __forceinline__ const T* tok_row(const TokView& v, int b, int h, int64_t n) {
  return reinterpret_cast<const T*>(v.p) + b * v.sb + h * v.sh + n * v.sn;
}
template <typename T>
__device__ __forceinline__ T* tok_row_mut(const TokViewMut& v, int b, int h, int64_t n) {
  return reinterpret_cast<T*>(v.p) + b * v.sb + h * v.sh + n * v.sn;
}

// Per-round pointer tables for the kernels that sum over every round.
struct RoundPtrs {
  const uint16_t* idx[MAX_ROUNDS];   // [BH, N, 8]
  const float* w[MAX_ROUNDS];        // [BH, N, 7]
  const float* a[MAX_ROUNDS];        // slot rows gathered with weight w (fp32 [BH, M, D])
  const float* b[MAX_ROUNDS];        // second gathered table (optional)
  const float* c[MAX_ROUNDS];        // per-(token, j) coefficient for table b (optional)
};

// ------------------------------------------------------ LDS slot tables ---
// Token-side kernels that gather slot rows stage the float32 [M, D] table of
// the (b,h) in LDS (row stride DP + 4 floats, zero past D), eight float4
// loads in flight per thread.  Rows past M are not written.
// Row stride (floats) of a slot table staged in LDS: unpadded 256-byte rows
// at d = 64 (the split lane layout keeps its reads conflict-free there), one
// 16-byte pad otherwise.
template <int DP>
constexpr int table_stride() { return DP == 64 ? 64 : DP + 4; }
// Split-layout half order of this thread's token (see split_dim): odd tokens
// swap at d = 64.
template <int DP>
__device__ __forceinline__ int tok_swap() { return DP == 64 ? (int)((threadIdx.x >> 3) & 1) : 0; }

// Slot j of a raw index row (8 u16 in one 16-byte load).
__device__ __forceinline__ uint32_t idx_at(const uint4& r, int j) {
  const uint32_t w = j < 2 ? r.x : (j < 4 ? r.y : (j < 6 ? r.z : r.w));
  return (w >> (16 * (j & 1))) & 0xFFFF;
}

// One row of KN = 7 floats (28 bytes, 4-byte aligned) with two vector
// accesses (16 + 12 bytes); global memory takes unaligned vector accesses.
__device__ __forceinline__ void load_row7(const float* src, float (&v)[KN]) {
  float4 a;
  float3 c;
  __builtin_memcpy(&a, src, 16);
  __builtin_memcpy(&c, src + 4, 12);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = c.x; v[5] = c.y; v[6] = c.z;
}
__device__ __forceinline__ void store_row7(float* dst, const float (&v)[KN]) {
  const float4 a = make_float4(v[0], v[1], v[2], v[3]);
  const float3 c = make_float3(v[4], v[5], v[6]);
  __builtin_memcpy(dst, &a, 16);
  __builtin_memcpy(dst + 4, &c, 12);
}

// Global -> LDS copy of `bytes` contiguous bytes (a multiple of 16; both
// ends 16-byte aligned) without a trip through registers: each wave issues
// global_load_lds_dwordx4 for its 1 KiB pieces (lane l's 16 bytes land at the
// piece's LDS base + 16 l), all pieces in flight at once, then waits for
// them.  The caller's barrier publishes the copy to the other waves.
__device__ __forceinline__ void issue_copy_to_lds(void* dst, const void* src, int bytes) {
  typedef __attribute__((address_space(3))) void* lds_ptr;
  typedef __attribute__((address_space(1))) void* glb_ptr;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nw = (int)(blockDim.x >> 6);
  for (int off = wave * 1024; off < bytes; off += nw * 1024) {
    const int o = off + lane * 16;
    if (o < bytes)
      __builtin_amdgcn_global_load_lds((glb_ptr)((const char*)src + o), (lds_ptr)((char*)dst + off), 16, 0, 0);
  }
}
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
__device__ __forceinline__ void copy_to_lds(void* dst, const void* src, int bytes) {
  issue_copy_to_lds(dst, src, bytes);
  wait_vm();  // this wave's pieces are in LDS
}
// A table of M rows of D floats at `src` is copied to LDS as it lies
// (unpadded rows of the full width, 16-byte aligned source).
template <int DP>
__device__ __forceinline__ bool table_direct(const float* src, int D) {
  return table_stride<DP>() == D && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
}

template <int DP>
__device__ __forceinline__ void stage_table(float* __restrict__ dst, const float* __restrict__ src, int M, int D) {
  constexpr int RSD = table_stride<DP>();
  // unpadded rows of the full width: the LDS table is the global one
  if (table_direct<DP>(src, D)) {
    copy_to_lds(dst, src, M * D * 4);
    return;
  }
  constexpr int STB = 8;
  const int nq = M * (DP / 4);
  const bool vec4 = (D & 3) == 0;
  for (int i0 = threadIdx.x; i0 < nq; i0 += STB * blockDim.x) {
    float4 v[STB];
#pragma unroll
    for (int u = 0; u < STB; ++u) {
      const int i = i0 + u * blockDim.x;
      const int m = i / (DP / 4), d4 = (i % (DP / 4)) * 4;
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < nq && d4 < D) {
        const float* s = src + (int64_t)m * D + d4;
        if (vec4) {
          v[u] = *reinterpret_cast<const float4*>(s);
        } else {
          v[u].x = s[0];
          v[u].y = d4 + 1 < D ? s[1] : 0.f;
          v[u].z = d4 + 2 < D ? s[2] : 0.f;
          v[u].w = d4 + 3 < D ? s[3] : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < STB; ++u) {
      const int i = i0 + u * blockDim.x;
      if (i >= nq) break;
      const int m = i / (DP / 4), d4 = (i % (DP / 4)) * 4;
      *reinterpret_cast<float4*>(dst + m * RSD + d4) = v[u];
    }
  }
}

// 8 raw token elements row[d0 ..] (one or two 16-byte units), so loads for
// many tokens can be in flight before any is converted.  WIDE (rows 16-byte
// aligned and D % 8 == 0, decided per launch) takes one unconditional 16-byte
// load per unit straight into the result registers (lanes with d0 >= D
// re-read unit 0; unraw8 zeroes them).  Otherwise the elements are loaded one
// by one.  The two paths are separate kernel instances: a result that may
// come from either makes the compiler wait for the wide load at once.
template <typename T>
struct Raw8 {
  uint4 u[sizeof(T) / 2];
};
template <typename T, bool WIDE>
__device__ __forceinline__ Raw8<T> raw8(const T* __restrict__ row, int d0, int D) {
  Raw8<T> r;
  if constexpr (WIDE) {
    const int dd = d0 < D ? d0 : 0;
#pragma unroll
    for (int k = 0; k < (int)(sizeof(T) / 2); ++k)
      r.u[k] = *reinterpret_cast<const uint4*>(row + dd + k * (16 / (int)sizeof(T)));
  } else {
    T* e = reinterpret_cast<T*>(&r);
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (d0 + i < D) ? row[d0 + i] : from_f<T>(0.f);
  }
  return r;
}
template <typename T>
__device__ __forceinline__ void unraw8(const Raw8<T>& r, float (&o)[8], bool live = true) {
  const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = live ? to_f(e[i]) : 0.f;
}

// Split lane layout of the staged-table kernels: lane dc of a token owns the
// 4-dim groups at 4dc and DP/2 + 4dc, so the token's lanes read one
// contiguous half of a table row per 16-byte LDS read.  With `sw` set the
// token takes the halves in the other order; at d = 64 (unpadded 256-byte
// rows) odd tokens set it, so the two tokens of a 16-lane read cover the two
// halves of the 64 banks and never meet.  Element i < 4 of the 8 is dim
// first + i, element i >= 4 is dim second + i - 4.
template <int DP>
__device__ __forceinline__ int split_dim(int dc, int sw, int i) {
  const int lo = 4 * dc, hi = DP / 2 + 4 * dc;
  return i < 4 ? (sw ? hi : lo) + i : (sw ? lo : hi) + (i - 4);
}
template <int DP>
__device__ __forceinline__ void lds8s(const float* __restrict__ row, int dc, int sw, float (&o)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(row + split_dim<DP>(dc, sw, 0));
  const float4 b = *reinterpret_cast<const float4*>(row + split_dim<DP>(dc, sw, 4));
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
// WIDE: rows 16-byte aligned and D % 4 == 0: two unconditional loads of 4
// elements (groups past D re-read dim 0; unraw8s zeroes them).
template <typename T, bool WIDE, int DP>
__device__ __forceinline__ Raw8<T> raw8s(const T* __restrict__ row, int dc, int sw, int D) {
  Raw8<T> r;
  const int da = split_dim<DP>(dc, sw, 0), db = split_dim<DP>(dc, sw, 4);
  if constexpr (WIDE) {
    const int ea = da < D ? da : 0, eb = db < D ? db : 0;
    if constexpr (sizeof(T) == 2) {
      const uint2 x = *reinterpret_cast<const uint2*>(row + ea);
      const uint2 y = *reinterpret_cast<const uint2*>(row + eb);
      r.u[0] = make_uint4(x.x, x.y, y.x, y.y);
    } else {
      r.u[0] = *reinterpret_cast<const uint4*>(row + ea);
      r.u[1] = *reinterpret_cast<const uint4*>(row + eb);
    }
  } else {
    T* e = reinterpret_cast<T*>(&r);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = split_dim<DP>(dc, sw, i);
      e[i] = d < D ? row[d] : from_f<T>(0.f);
    }
  }
  return r;
}
template <typename T, int DP>
__device__ __forceinline__ void unraw8s(const Raw8<T>& r, float (&o)[8], int dc, int sw, int D, bool live = true) {
  const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (live && split_dim<DP>(dc, sw, i) < D) ? to_f(e[i]) : 0.f;
}
template <typename T, int DP>
__device__ __forceinline__ void store8s(T* __restrict__ row, int dc, int sw, int D, bool vec, const float (&v)[8]) {
  if (vec && (D & 3) == 0) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int d = split_dim<DP>(dc, sw, 4 * g);
      if (d >= D) continue;
      if constexpr (sizeof(T) == 2) {
        T e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = from_f<T>(v[4 * g + i]);
        *reinterpret_cast<uint2*>(row + d) = *reinterpret_cast<const uint2*>(e);
      } else {
        *reinterpret_cast<float4*>(row + d) = make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = split_dim<DP>(dc, sw, i);
      if (d < D) row[d] = from_f<T>(v[i]);
    }
  }
}

// 8 floats of a staged table row (16-byte aligned: d0 % 8 == 0)
__device__ __forceinline__ void lds8(const float* __restrict__ row, int d0, float (&o)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(row + d0);
  const float4 b = *reinterpret_cast<const float4*>(row + d0 + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// Blocks of the token-side kernels that stage tables: (b,h) x chunk on a 1-D
// grid of 8 * ceil(BH/8) * nchunk ids.  Workgroups are dispatched round-robin
// over the 8 XCDs (linear id % 8 = XCD): when B*H is a multiple of 8, every
// block of one (b,h) runs on XCD bh % 8 and the head's tables reach that
// XCD's L2 once.  Otherwise the heads would not cover the XCDs evenly, and a
// head's chunks are simply consecutive.  Ids past the last head return.
constexpr int TOK_XCDS = 8;
__device__ __forceinline__ bool tok_block(int BH, int nchunk, int& bh, int& chunk) {
  const int L = blockIdx.x;
  if (BH % TOK_XCDS != 0) {
    bh = L / nchunk;
    chunk = L % nchunk;
    return bh < BH;
  }
  const int x = L % TOK_XCDS, k = L / TOK_XCDS;
  bh = x + TOK_XCDS * (k / nchunk);
  chunk = k % nchunk;
  return bh < BH;
}

}  // namespace murm
