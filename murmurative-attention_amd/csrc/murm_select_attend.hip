// Select + attend (one round) and the per-token output gather.
//
// select_attend: for every token, scores s_m = q . sk_m over all M slots on
// MFMA (the N x M score matrix never leaves registers), top-7 by a packed
// float key (score with the slot index in its low mantissa bits), then the
// softmax over the 7 selected scores.  Writes indices (u16 rows and/or the
// int64 API tensor) and float32 weights.  Semantics: reference.py:6-68.
//
// Slot keys come from float32 state.  The 16-bit MFMA path splits each key
// into hi + lo halves of the token dtype (hi = rn(x), lo = rn(x - hi)) and
// accumulates q.lo + q.hi in float32, which reproduces the float32 score to
// ~2^-16 relative: selection is decided to far better than the 1e-3 relative
// gap used by the parity gate.  float32 tokens use the f32 MFMA and recompute
// the seven winning scores exactly before the softmax.
//
// MFMA 16x16x32 lane layout (gfx950): A row = lane&15, k = 8*(lane>>4)+i;
// B col = lane&15, same k; D holds rows 4*(lane>>4)+r of column lane&15.
// Here A = slot keys (rows = slots), B = tokens (cols), so every lane holds
// four consecutive slot scores of one token per 16-slot tile.

#include "murm_common.h"
#include "murm_launch.h"

namespace murm {

namespace {

template <int DP, int WAVES_ = 4> struct SAShape {
  static constexpr int G = (DP <= 64) ? 4 : 2;   // 16-token groups per wave
  static constexpr int WAVES = WAVES_;
  static constexpr int TOK = WAVES * G * 16;     // tokens per block
};
// 16-bit kernel: 8 waves share one staging of the head's keys (one block per CU)
constexpr int SA16_WAVES = 8;

// mask / bias / causal / effective_M slow path for one score
__device__ __forceinline__ float masked_key(const SAParams& p, int b, int h, int n, int m,
                                            float s) {
  if (m >= p.M) return -INFINITY;
  bool dead = (m >= p.em) || (p.causal && m > n) || (n >= p.N);
  if (!dead && p.mask)
    dead = p.mask[b * p.mk_sb + h * p.mk_sh + (int64_t)n * p.mk_sn + m * p.mk_sm] == 0;
  if (!dead && p.bias)
    s += p.bias[b * p.bs_sb + h * p.bs_sh + (int64_t)n * p.bs_sn + m * p.bs_sm];
  return make_key(dead ? MASKED_SCORE : s, p.hi_mask, (uint32_t)m);
}

// Merge the four per-lane lists of a token (lanes l, l^16, l^32, l^48).
template <int G>
__device__ __forceinline__ void merge_quads(float (&tk)[G][KN]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float lo[KN], up[KN];
#pragma unroll
    for (int j = 0; j < KN; ++j) lane_pair<16>(tk[g][j], lo[j], up[j]);
    top7_merge(lo, up, tk[g]);
#pragma unroll
    for (int j = 0; j < KN; ++j) lane_pair<32>(tk[g][j], lo[j], up[j]);
    top7_merge(lo, up, tk[g]);
  }
}

__device__ __forceinline__ void softmax7(const float (&sc)[KN], float scale, float (&w)[KN]) {
  float z[KN], zmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < KN; ++j) { z[j] = scale * sc[j]; zmax = fmaxf(zmax, z[j]); }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < KN; ++j) { z[j] = __expf(z[j] - zmax); sum += z[j]; }
  const float inv = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < KN; ++j) w[j] = z[j] * inv;
}

__device__ __forceinline__ void write_token(const SAParams& p, int bh, int n, const uint32_t (&slot)[KN],
                                            const float (&w)[KN]) {
  const int64_t row = (int64_t)bh * p.N + n;
  if (p.idx16) {
    uint4 r;
    r.x = slot[0] | (slot[1] << 16);
    r.y = slot[2] | (slot[3] << 16);
    r.z = slot[4] | (slot[5] << 16);
    r.w = slot[6] | ((uint32_t)IDX_NONE << 16);
    *reinterpret_cast<uint4*>(p.idx16 + row * IDX_ROW) = r;
  }
  if (p.idx64) {  // 56 bytes, 8-byte aligned: vector stores
    int64_t v[KN];
#pragma unroll
    for (int j = 0; j < KN; ++j) v[j] = (int64_t)slot[j];
    __builtin_memcpy(p.idx64 + row * KN, v, sizeof(v));
  }
  store_row7(p.w + row * KN, w);
}

// Raw 8-element load of a 16-bit token row into an MFMA operand (zero fill).
template <typename T, typename V>
__device__ __forceinline__ V load_operand8(const T* row, int d0, int D, bool vec) {
  V v;
  if (vec && d0 + 8 <= D) {
    uint4 raw = *reinterpret_cast<const uint4*>(row + d0);
    v = *reinterpret_cast<V*>(&raw);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (d0 + i < D) ? row[d0 + i] : (T)0.f;
  }
  return v;
}

// Eight 16-bit values (one 16-byte unit) widened to float32 and stored as two
// float4 (dst 16-byte aligned).
template <typename T>
__device__ __forceinline__ void store8_f32(float* dst, const uint4& u) {
  const T* e = reinterpret_cast<const T*>(&u);
  reinterpret_cast<float4*>(dst)[0] = make_float4((float)e[0], (float)e[1], (float)e[2], (float)e[3]);
  reinterpret_cast<float4*>(dst)[1] = make_float4((float)e[4], (float)e[5], (float)e[6], (float)e[7]);
}

// Blocks of the select kernels: (b,h) x token chunk as tok_block maps them
// (with B*H a multiple of 8 all blocks of a head share one XCD's L2, where
// the head's slot keys then arrive once).
__device__ __forceinline__ bool sa_block(int BH, int nchunk, int& bh, int& chunk) {
  return tok_block(BH, nchunk, bh, chunk);
}

// ---------------------------------------------------------------------------
// 16-bit tokens (bf16 / fp16): hi/lo split keys in LDS, 16x16x32 MFMA
// ---------------------------------------------------------------------------
// HI: the keys are exact in the token dtype (lo halves all zero; the first
// round of a call whose slot keys have the token dtype): only the hi halves
// are copied and multiplied, which gives the same scores bit for bit.
// RAW (with HI): the hi table is read from the caller's key tensor (p.raw_k)
// instead of a split table, and the block writes its share of the float32
// state rows of the keys and values (p.st_k, p.st_v).
template <typename T, int DP, bool WIDE, int W = SA16_WAVES, bool HI = false, bool RAW = false>
__global__ __launch_bounds__(64 * W) void sa_kernel16(SAParams p, int nchunk) {
  static_assert(!RAW || HI, "the caller's keys are the hi halves");
  using V = typename Mfma16<T>::vec;
  constexpr int G = SAShape<DP>::G;
  constexpr int KC = DP / 32;
  constexpr int ROW = DP + 8;  // LDS row stride in elements (16 B pad); = ksplit_row(DP)
  extern __shared__ __align__(16) unsigned char smem[];
  T* lhi = reinterpret_cast<T*>(smem);
  const int Mp = (p.M + 15) & ~15;
  T* llo = lhi + Mp * ROW;

  int bh, chunk;
  if (!sa_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  const float* skb = p.sk + (int64_t)bh * p.M * p.D;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = lane >> 4, col = lane & 15;
  const int tok0 = chunk * SAShape<DP, W>::TOK + wave * (G * 16);

  // WIDE (16-byte aligned rows, D % 8 == 0): the wave's token rows are
  // requested before the keys are staged, unconditionally from clamped rows
  // and units, and zeroed where out of range only after the staging
  uint4 rq[G][KC];
  if constexpr (WIDE) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const T* row = tok_row<T>(p.q, b, h, min(tok0 + 16 * g + col, p.N - 1));
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        rq[g][kc] = *reinterpret_cast<const uint4*>(row + min(32 * kc + 8 * quad, p.D - 8));
    }
  }

  // stage the keys: the pre-split table is copied in as it lies (global ->
  // LDS, no registers); otherwise batches of STB float4 loads in flight per
  // thread, then the hi/lo split written as 8-byte LDS stores
  constexpr int STB = 8;
  const int nq = (RAW || p.ksplit) ? 0 : Mp * (DP / 4);
  if constexpr (RAW) {
    // 16-byte units of the caller's key rows through registers into the
    // padded LDS rows (zeros at d >= D and m >= M), one round of loads for
    // tables of up to 2048 units (M = 256 at d = 64); the rows [r0, r1) of this block's share
    // also go to the float32 key state, and the same rows of the caller's
    // values (one unit per thread in flight with the keys) to the value state
    constexpr int UPR = DP / 8, RB = 32 / W;
    const T* kb = static_cast<const T*>(p.raw_k) + b * p.rk_sb + h * p.rk_sh;
    const T* vb = static_cast<const T*>(p.raw_v) + b * p.rv_sb + h * p.rv_sh;
    float* stk = p.st_k + (size_t)bh * p.M * p.D;
    float* stv = p.st_v + (size_t)bh * p.M * p.D;
    const int rpc = (p.M + nchunk - 1) / nchunk;
    const int r0 = chunk * rpc, r1 = min(p.M, r0 + rpc);
    const int nu = Mp * UPR, nvu = max(0, r1 - r0) * UPR;
    auto value_unit = [&](int i) {
      const int d0 = (i % UPR) * 8;
      return d0 < p.D ? *reinterpret_cast<const uint4*>(vb + (r0 + i / UPR) * p.rv_sm + d0) : make_uint4(0u, 0u, 0u, 0u);
    };
    auto store_value = [&](int i, const uint4& u) {
      const int d0 = (i % UPR) * 8;
      if (d0 < p.D) store8_f32<T>(stv + (size_t)(r0 + i / UPR) * p.D + d0, u);
    };
    const int vi = threadIdx.x;
    uint4 v0 = make_uint4(0u, 0u, 0u, 0u);
    if (vi < nvu) v0 = value_unit(vi);
    for (int i0 = threadIdx.x; i0 < nu; i0 += RB * blockDim.x) {
      uint4 kk[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int i = i0 + u * blockDim.x, m = i / UPR, d0 = (i % UPR) * 8;
        kk[u] = make_uint4(0u, 0u, 0u, 0u);
        if (i < nu && m < p.M && d0 < p.D) kk[u] = *reinterpret_cast<const uint4*>(kb + m * p.rk_sm + d0);
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int i = i0 + u * blockDim.x, m = i / UPR, d0 = (i % UPR) * 8;
        if (i < nu) {
          *reinterpret_cast<uint4*>(lhi + m * ROW + d0) = kk[u];
          if (m >= r0 && m < r1 && d0 < p.D) store8_f32<T>(stk + (size_t)m * p.D + d0, kk[u]);
        }
      }
    }
    if (vi < nvu) store_value(vi, v0);
    for (int i = vi + blockDim.x; i < nvu; i += blockDim.x) store_value(i, value_unit(i));  // few chunks per head
  } else if (p.ksplit) {
    const size_t head = 2 * (size_t)Mp * ROW;
    copy_to_lds(lhi, reinterpret_cast<const T*>(p.ksplit) + (size_t)bh * head,
                (int)((HI ? head / 2 : head) * sizeof(T)));
  }
  const bool vec4 = (p.D & 3) == 0;
  for (int i0 = threadIdx.x; i0 < nq; i0 += STB * blockDim.x) {
    float4 v[STB];
#pragma unroll
    for (int u = 0; u < STB; ++u) {
      const int i = i0 + u * blockDim.x;
      const int m = i / (DP / 4), d4 = (i % (DP / 4)) * 4;
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < nq && m < p.M && d4 < p.D) {
        const float* src = skb + (int64_t)m * p.D + d4;
        if (vec4) {
          v[u] = *reinterpret_cast<const float4*>(src);
        } else {
          v[u].x = src[0];
          v[u].y = d4 + 1 < p.D ? src[1] : 0.f;
          v[u].z = d4 + 2 < p.D ? src[2] : 0.f;
          v[u].w = d4 + 3 < p.D ? src[3] : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < STB; ++u) {
      const int i = i0 + u * blockDim.x;
      if (i >= nq) break;
      const int m = i / (DP / 4), d4 = (i % (DP / 4)) * 4;
      const float f[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      T hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = (T)f[e];
        lo[e] = (T)(f[e] - (float)hi[e]);
      }
      *reinterpret_cast<uint2*>(lhi + m * ROW + d4) = *reinterpret_cast<const uint2*>(hi);
      *reinterpret_cast<uint2*>(llo + m * ROW + d4) = *reinterpret_cast<const uint2*>(lo);
    }
  }
  __syncthreads();

  if (tok0 >= p.N) return;  // whole wave past the end (no block-wide sync below)

  V bq[G][KC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int n = tok0 + 16 * g + col;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      if constexpr (WIDE) {
        bq[g][kc] = *reinterpret_cast<const V*>(&rq[g][kc]);
        if (32 * kc + 8 * quad >= p.D) bq[g][kc] = V{};
      } else {
        bq[g][kc] = load_operand8<T, V>(tok_row<T>(p.q, b, h, n < p.N ? n : 0), 32 * kc + 8 * quad, p.D, false);
      }
      if (n >= p.N) bq[g][kc] = V{};
    }
  }

  float tk[G][KN];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < KN; ++j) tk[g][j] = -INFINITY;

  // scores of slot tile t (16 slots) against the wave's G token groups
  auto scores = [&](int t, f32x4 (&acc)[G]) {
    V ahi[KC], alo[KC];
    const int arow = 16 * t + col;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      ahi[kc] = *reinterpret_cast<const V*>(lhi + arow * ROW + 32 * kc + 8 * quad);
      if constexpr (!HI) alo[kc] = *reinterpret_cast<const V*>(llo + arow * ROW + 32 * kc + 8 * quad);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!HI)
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g] = mfma_16x16x32(alo[kc], bq[g][kc], acc[g]);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = mfma_16x16x32(ahi[kc], bq[g][kc], acc[g]);
  };

  // Tiles [0, nfast) mask no score of the wave (every token in range, slots
  // below effective_M, inside the causal prefix): a branch-free loop.  The
  // rest take the per-group test and, where needed, the masked path.
  const bool plain = !p.mask && !p.bias;
  const int nT = Mp / 16;
  int nfast = 0;
  if (plain && tok0 + 16 * G <= p.N) {
    nfast = min(nT, p.em / 16);
    if (p.causal) nfast = min(nfast, (tok0 + 1) / 16);
  }
  for (int t = 0; t < nfast; ++t) {
    f32x4 acc[G];
    scores(t, acc);
    uint32_t mr[4];  // slot ids of this lane's four rows, shared by the groups
#pragma unroll
    for (int r = 0; r < 4; ++r) mr[r] = (uint32_t)(16 * t + 4 * quad + r);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) topk_insert(tk[g], make_key(acc[g][r], p.hi_mask, mr[r]));
  }
  for (int t = nfast; t < nT; ++t) {
    f32x4 acc[G];
    scores(t, acc);
    const int m0 = 16 * t + 4 * quad;
    const bool tile_ok = plain && (16 * t + 16 <= p.em);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int gmin = tok0 + 16 * g;
      const bool fast = tile_ok && (!p.causal || 16 * t + 15 <= gmin) && (gmin + 16 <= p.N);
      if (fast) {
#pragma unroll
        for (int r = 0; r < 4; ++r) topk_insert(tk[g], make_key(acc[g][r], p.hi_mask, (uint32_t)(m0 + r)));
      } else {
        const int n = gmin + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) topk_insert(tk[g], masked_key(p, b, h, n, m0 + r, acc[g][r]));
      }
    }
  }

  merge_quads<G>(tk);

#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int n = tok0 + 16 * g + col;
    uint32_t slot[KN];
    float sc[KN];
    // The attend softmax uses the real q.sk of the selected slots
    // (reference.py:56-63): re-score when a selection score was masked
    // (causal prefix, effective_M < 7, masked token) or carried a bias.
    bool masked = p.bias != nullptr;
#pragma unroll
    for (int j = 0; j < KN; ++j) {
      slot[j] = key_slot(tk[g][j], p.lo_mask);
      sc[j] = key_score(tk[g][j], p.hi_mask);
      masked |= key_masked(tk[g][j]);
    }
    if (__any(masked)) {
      float part[KN];
#pragma unroll
      for (int j = 0; j < KN; ++j) {
        part[j] = 0.f;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          const int d0 = 32 * kc + 8 * quad;
          const V hv = *reinterpret_cast<const V*>(lhi + slot[j] * ROW + d0);
          V lv{};
          if constexpr (!HI) lv = *reinterpret_cast<const V*>(llo + slot[j] * ROW + d0);
#pragma unroll
          for (int i = 0; i < 8; ++i) part[j] += (float)bq[g][kc][i] * ((float)hv[i] + (float)lv[i]);
        }
        part[j] += shfl_xor_f(part[j], 16);
        part[j] += shfl_xor_f(part[j], 32);
      }
      if (masked)
#pragma unroll
        for (int j = 0; j < KN; ++j) sc[j] = part[j];
    }
    float w[KN];
    softmax7(sc, p.scale, w);
    if (quad == 0 && n < p.N) write_token(p, bh, n, slot, w);
  }
}

// ---------------------------------------------------------------------------
// float32 tokens: f32 keys in LDS, 16x16x4 f32 MFMA, exact softmax scores
// ---------------------------------------------------------------------------
// G: 16-token groups per wave (fewer on small grids, so more CUs share the
// float32 MFMA work)
template <int DP, int G = SAShape<DP>::G>
__global__ __launch_bounds__(256) void sa_kernel32(SAParams p, int nchunk) {
  constexpr int KK = DP / 4;
  constexpr int ROW = DP + 4;
  extern __shared__ __align__(16) unsigned char smem[];
  float* lsk = reinterpret_cast<float*>(smem);
  const int Mp = (p.M + 15) & ~15;

  int bh, chunk;
  if (!sa_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  const float* skb = p.sk + (int64_t)bh * p.M * p.D;
  constexpr int STB = 8;
  const int nq = Mp * (DP / 4);
  const bool vec4 = (p.D & 3) == 0;
  for (int i0 = threadIdx.x; i0 < nq; i0 += STB * blockDim.x) {
    float4 v[STB];
#pragma unroll
    for (int u = 0; u < STB; ++u) {
      const int i = i0 + u * blockDim.x;
      const int m = i / (DP / 4), d4 = (i % (DP / 4)) * 4;
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < nq && m < p.M && d4 < p.D) {
        const float* src = skb + (int64_t)m * p.D + d4;
        if (vec4) {
          v[u] = *reinterpret_cast<const float4*>(src);
        } else {
          v[u].x = src[0];
          v[u].y = d4 + 1 < p.D ? src[1] : 0.f;
          v[u].z = d4 + 2 < p.D ? src[2] : 0.f;
          v[u].w = d4 + 3 < p.D ? src[3] : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < STB; ++u) {
      const int i = i0 + u * blockDim.x;
      if (i >= nq) break;
      const int m = i / (DP / 4), d4 = (i % (DP / 4)) * 4;
      *reinterpret_cast<float4*>(lsk + m * ROW + d4) = v[u];
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = lane >> 4, col = lane & 15;
  const int tok0 = chunk * (SAShape<DP>::WAVES * G * 16) + wave * (G * 16);
  if (tok0 >= p.N) return;

  float bq[G][KK];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int n = tok0 + 16 * g + col;
    const float* row = tok_row<float>(p.q, b, h, n < p.N ? n : 0);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int d = 4 * kk + quad;
      bq[g][kk] = (n < p.N && d < p.D) ? row[d] : 0.f;
    }
  }
  float tk[G][KN];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < KN; ++j) tk[g][j] = -INFINITY;

  auto scores = [&](int t, f32x4 (&acc)[G]) {
    const float* arow = lsk + (16 * t + col) * ROW + quad;
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const float a = arow[4 * kk];
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = mfma_16x16x4(a, bq[g][kk], acc[g]);
    }
  };

  // tiles [0, nfast): no masked score in the wave (as in sa_kernel16)
  const bool plain = !p.mask && !p.bias;
  const int nT = Mp / 16;
  int nfast = 0;
  if (plain && tok0 + 16 * G <= p.N) {
    nfast = min(nT, p.em / 16);
    if (p.causal) nfast = min(nfast, (tok0 + 1) / 16);
  }
  for (int t = 0; t < nfast; ++t) {
    f32x4 acc[G];
    scores(t, acc);
    uint32_t mr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) mr[r] = (uint32_t)(16 * t + 4 * quad + r);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) topk_insert(tk[g], make_key(acc[g][r], p.hi_mask, mr[r]));
  }
  for (int t = nfast; t < nT; ++t) {
    f32x4 acc[G];
    scores(t, acc);
    const int m0 = 16 * t + 4 * quad;
    const bool tile_ok = plain && (16 * t + 16 <= p.em);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int gmin = tok0 + 16 * g;
      const bool fast = tile_ok && (!p.causal || 16 * t + 15 <= gmin) && (gmin + 16 <= p.N);
      if (fast) {
#pragma unroll
        for (int r = 0; r < 4; ++r) topk_insert(tk[g], make_key(acc[g][r], p.hi_mask, (uint32_t)(m0 + r)));
      } else {
        const int n = gmin + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) topk_insert(tk[g], masked_key(p, b, h, n, m0 + r, acc[g][r]));
      }
    }
  }

  merge_quads<G>(tk);

#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int n = tok0 + 16 * g + col;
    uint32_t slot[KN];
    float sc[KN];
#pragma unroll
    for (int j = 0; j < KN; ++j) {
      slot[j] = key_slot(tk[g][j], p.lo_mask);
      const float* srow = lsk + slot[j] * ROW + quad;
      float part = 0.f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) part += bq[g][kk] * srow[4 * kk];
      part += shfl_xor_f(part, 16);
      part += shfl_xor_f(part, 32);
      sc[j] = part;
    }
    float w[KN];
    softmax7(sc, p.scale, w);
    if (quad == 0 && n < p.N) write_token(p, bh, n, slot, w);
  }
}

// ---------------------------------------------------------------------------
// out[n] = base[n] + sum_r sum_j w_rj * table_r[idx_rj]   (8 dims per thread)
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) void gather_out_kernel(OutParams p) {
  constexpr int DCH = DP / 8;
  constexpr int TPB = 256 / DCH;  // tokens per block
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int n = blockIdx.x * TPB + threadIdx.x / DCH;
  const int dc = threadIdx.x % DCH;
  if (n >= p.N) return;
  const int d0 = dc * 8;
  float acc[8];
  if (p.base.p) {
    load8<T>(tok_row<T>(p.base, b, h, n), d0, p.D, p.base.vec, acc);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  }
  const int64_t row = (int64_t)bh * p.N + n;
  for (int r = 0; r < p.R; ++r) {
    const uint4 ir = *reinterpret_cast<const uint4*>(p.rp.idx[r] + row * IDX_ROW);
    const uint32_t sl[KN] = {ir.x & 0xFFFF, ir.x >> 16, ir.y & 0xFFFF, ir.y >> 16,
                             ir.z & 0xFFFF, ir.z >> 16, ir.w & 0xFFFF};
    const float* wr = p.rp.w[r] + row * KN;
    const float* tab = p.rp.a[r] + (int64_t)bh * p.M * p.D;
#pragma unroll
    for (int j = 0; j < KN; ++j) {
      const float wj = wr[j];
      float v[8];
      load8f(tab + (int64_t)sl[j] * p.D, d0, p.D, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += wj * v[i];
    }
  }
  store8<T>(tok_row_mut<T>(p.out, b, h, n), d0, p.D, p.out.vec, acc);
}

// Staged variant: one block per (b,h) and token chunk; each round's value
// table is staged in LDS (row stride table_stride) in turn and every thread keeps
// the outputs of its GO_PASSES tokens in registers across the rounds.
constexpr int GO_THREADS = 512;
constexpr int GO_PASSES_MAX = 8;

template <typename T, int DP, bool WIDE, int GO_PASSES = GO_PASSES_MAX>
__global__ __launch_bounds__(GO_THREADS) void gather_out_lds_kernel(OutParams p, int nchunk) {
  constexpr int DCH = DP / 8, TPP = GO_THREADS / DCH, RSD = table_stride<DP>();
  extern __shared__ __align__(16) unsigned char smem[];
  float* tab = reinterpret_cast<float*>(smem);
  int bh, chunk;
  if (!tok_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  const int dc = threadIdx.x % DCH, sw = tok_swap<DP>();
  const int c_beg = chunk * GO_PASSES * TPP;
  float acc[GO_PASSES][8];
  if (p.base.p) {  // every pass's residual row in flight before any is converted
    Raw8<T> rb[GO_PASSES];
#pragma unroll
    for (int q = 0; q < GO_PASSES; ++q)
      rb[q] = raw8s<T, WIDE, DP>(tok_row<T>(p.base, b, h, min(c_beg + q * TPP + (int)threadIdx.x / DCH, p.N - 1)),
                                 dc, sw, p.D);
#pragma unroll
    for (int q = 0; q < GO_PASSES; ++q)
      unraw8s<T, DP>(rb[q], acc[q], dc, sw, p.D, c_beg + q * TPP + (int)threadIdx.x / DCH < p.N);
  } else {
#pragma unroll
    for (int q = 0; q < GO_PASSES; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[q][i] = 0.f;
  }
  for (int r = 0; r < p.R; ++r) {
    // the round's index rows and weights of every pass are requested before
    // its table is staged
    uint4 ix[GO_PASSES];
    float wv[GO_PASSES][KN];
#pragma unroll
    for (int q = 0; q < GO_PASSES; ++q) {
      const int n = min(c_beg + q * TPP + (int)threadIdx.x / DCH, p.N - 1);
      const int64_t row = (int64_t)bh * p.N + n;
      ix[q] = *reinterpret_cast<const uint4*>(p.rp.idx[r] + row * IDX_ROW);
      load_row7(p.rp.w[r] + row * KN, wv[q]);
    }
    if (r > 0) __syncthreads();
    stage_table<DP>(tab, p.rp.a[r] + (int64_t)bh * p.M * p.D, p.M, p.D);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < GO_PASSES; ++q) {
      const uint4 ir = ix[q];
      const uint32_t sl[KN] = {ir.x & 0xFFFF, ir.x >> 16, ir.y & 0xFFFF, ir.y >> 16,
                               ir.z & 0xFFFF, ir.z >> 16, ir.w & 0xFFFF};
#pragma unroll
      for (int j = 0; j < KN; ++j) {
        float v[8];
        lds8s<DP>(tab + sl[j] * RSD, dc, sw, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[q][i] += wv[q][j] * v[i];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < GO_PASSES; ++q) {
    const int n = c_beg + q * TPP + threadIdx.x / DCH;
    if (n < p.N) store8s<T, DP>(tok_row_mut<T>(p.out, b, h, n), dc, sw, p.D, p.out.vec, acc[q]);
  }
}

// gather_out for large grids: blocks of GO_PASSES_BIG passes, so each
// round's table is staged once for twice the tokens of the standard block.
// The outputs of all passes stay in registers across the rounds, so a
// round's index rows and weights are requested PF passes ahead instead of
// all at once (those of the first PF passes while the table is staged).
constexpr int GO_PASSES_BIG = 16;

template <typename T, int DP, bool WIDE>
__global__ __launch_bounds__(GO_THREADS) void gather_out_big_kernel(OutParams p, int nchunk) {
  constexpr int NP = GO_PASSES_BIG, PF = 2;
  constexpr int DCH = DP / 8, TPP = GO_THREADS / DCH, RSD = table_stride<DP>();
  extern __shared__ __align__(16) unsigned char smem[];
  float* tab = reinterpret_cast<float*>(smem);
  int bh, chunk;
  if (!tok_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  const int dc = threadIdx.x % DCH, sw = tok_swap<DP>();
  const int tl = threadIdx.x / DCH;
  const int c_beg = chunk * NP * TPP;
  float acc[NP][8];
  if (p.base.p) {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {  // residual rows in two halves of NP / 2 passes in flight
      Raw8<T> rb[NP / 2];
#pragma unroll
      for (int q = 0; q < NP / 2; ++q)
        rb[q] = raw8s<T, WIDE, DP>(tok_row<T>(p.base, b, h, min(c_beg + (h2 * NP / 2 + q) * TPP + tl, p.N - 1)),
                                   dc, sw, p.D);
#pragma unroll
      for (int q = 0; q < NP / 2; ++q)
        unraw8s<T, DP>(rb[q], acc[h2 * NP / 2 + q], dc, sw, p.D, c_beg + (h2 * NP / 2 + q) * TPP + tl < p.N);
    }
  } else {
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[q][i] = 0.f;
  }
  for (int r = 0; r < p.R; ++r) {
    uint4 ix[NP];
    float wv[NP][KN];
    auto fetch = [&](int q) {
      const int n = min(c_beg + q * TPP + tl, p.N - 1);
      const int64_t row = (int64_t)bh * p.N + n;
      ix[q] = *reinterpret_cast<const uint4*>(p.rp.idx[r] + row * IDX_ROW);
      load_row7(p.rp.w[r] + row * KN, wv[q]);
    };
#pragma unroll
    for (int q = 0; q < PF; ++q) fetch(q);
    if (r > 0) __syncthreads();  // the previous round's table is no longer read
    stage_table<DP>(tab, p.rp.a[r] + (int64_t)bh * p.M * p.D, p.M, p.D);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      if (q + PF < NP) fetch(q + PF);
      const uint4 ir = ix[q];
      const uint32_t sl[KN] = {ir.x & 0xFFFF, ir.x >> 16, ir.y & 0xFFFF, ir.y >> 16,
                               ir.z & 0xFFFF, ir.z >> 16, ir.w & 0xFFFF};
#pragma unroll
      for (int j = 0; j < KN; ++j) {
        float v[8];
        lds8s<DP>(tab + sl[j] * RSD, dc, sw, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[q][i] += wv[q][j] * v[i];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int n = c_beg + q * TPP + tl;
    if (n < p.N) store8s<T, DP>(tok_row_mut<T>(p.out, b, h, n), dc, sw, p.D, p.out.vec, acc[q]);
  }
}

// 1-D grid of sa_block (tok_block ids)
inline dim3 sa_grid(int BH, int nchunk) { return dim3(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk); }

template <typename T, int DP>
hipError_t launch_sa_t(const SAParams& p, hipStream_t st) {
  const int Mp = (p.M + 15) & ~15;
  const int BH = p.B * p.H;
  if constexpr (sizeof(T) == 2) {
    const size_t lds = 2 * (size_t)Mp * (DP + 8) * sizeof(T);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const bool wide = p.q.vec && p.D % 8 == 0;
    auto go = [&](auto w_c) -> hipError_t {
      constexpr int W = decltype(w_c)::value;
      const int nchunk = (p.N + SAShape<DP, W>::TOK - 1) / SAShape<DP, W>::TOK;
      const dim3 grid = sa_grid(BH, nchunk);
      auto run = [&](auto hi_c) -> hipError_t {
        constexpr bool HI = decltype(hi_c)::value;
        const void* fn = wide ? reinterpret_cast<const void*>(&sa_kernel16<T, DP, true, W, HI>)
                              : reinterpret_cast<const void*>(&sa_kernel16<T, DP, false, W, HI>);
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (wide)
          MURM_LAUNCH((sa_kernel16<T, DP, true, W, HI>), grid, dim3(64 * W), lds, st, p, nchunk);
        else
          MURM_LAUNCH((sa_kernel16<T, DP, false, W, HI>), grid, dim3(64 * W), lds, st, p, nchunk);
        return hipSuccess;
      };
      if (p.raw_k) {  // the caller's keys and values: wide rows only (checked by the caller too)
        if (!wide || !p.raw_v || !p.st_k || !p.st_v || p.ksplit) return hipErrorInvalidValue;
        const void* fn = reinterpret_cast<const void*>(&sa_kernel16<T, DP, true, W, true, true>);
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        MURM_LAUNCH((sa_kernel16<T, DP, true, W, true, true>), grid, dim3(64 * W), lds, st, p, nchunk);
        return hipSuccess;
      }
      if (p.ksplit && p.keys_hi_only) return run(std::true_type{});
      return run(std::false_type{});
    };
    // half-size blocks (4 waves) when 8-wave blocks would leave CUs idle
    using S8 = SAShape<DP, SA16_WAVES>;
    const int blocks8 = (int)sa_grid(BH, (p.N + S8::TOK - 1) / S8::TOK).x;
    hipError_t e = blocks8 >= device_cus() ? go(std::integral_constant<int, SA16_WAVES>{})
                                           : go(std::integral_constant<int, SA16_WAVES / 2>{});
    if (e != hipSuccess) return e;
  } else {
    if (p.ksplit || p.raw_k) return hipErrorInvalidValue;  // float32 tokens use the float32 keys
    const size_t lds = (size_t)Mp * (DP + 4) * sizeof(float);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    auto go = [&](auto g_c) -> hipError_t {
      constexpr int G = decltype(g_c)::value;
      constexpr int TOK = SAShape<DP>::WAVES * G * 16;
      const int nchunk = (p.N + TOK - 1) / TOK;
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&sa_kernel32<DP, G>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      MURM_LAUNCH((sa_kernel32<DP, G>), sa_grid(BH, nchunk), dim3(256), lds, st, p, nchunk);
      return hipSuccess;
    };
    // one token group per wave when full groups would leave CUs idle
    const int full = (int)sa_grid(BH, (p.N + SAShape<DP>::TOK - 1) / SAShape<DP>::TOK).x;
    hipError_t e = full >= device_cus() ? go(std::integral_constant<int, SAShape<DP>::G>{})
                                        : go(std::integral_constant<int, 1>{});
    if (e != hipSuccess) return e;
  }
  return hipGetLastError();
}

template <typename T, int DP>
hipError_t launch_out_t(const OutParams& p, hipStream_t st) {
  const size_t lds = (size_t)p.M * table_stride<DP>() * 4;
  if (lds <= 150 * 1024) {
    constexpr int TPP = GO_THREADS / (DP / 8);
    const int BH = p.B * p.H;
    const bool wide = (!p.base.p || p.base.vec) && p.D % 4 == 0;
    auto go = [&](auto np_c) -> hipError_t {
      constexpr int NP = decltype(np_c)::value;
      const int nchunk = (p.N + NP * TPP - 1) / (NP * TPP);
      const void* fn = wide ? reinterpret_cast<const void*>(&gather_out_lds_kernel<T, DP, true, NP>)
                            : reinterpret_cast<const void*>(&gather_out_lds_kernel<T, DP, false, NP>);
      hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      dim3 grid(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk);
      if (wide)
        MURM_LAUNCH((gather_out_lds_kernel<T, DP, true, NP>), grid, dim3(GO_THREADS), lds, st, p, nchunk);
      else
        MURM_LAUNCH((gather_out_lds_kernel<T, DP, false, NP>), grid, dim3(GO_THREADS), lds, st, p, nchunk);
      return hipGetLastError();
    };
    // twice the passes where such blocks still fill the device
    const int big = TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) *
                    ((p.N + GO_PASSES_BIG * TPP - 1) / (GO_PASSES_BIG * TPP));
    if (big >= device_cus()) {
      const int nchunk = (p.N + GO_PASSES_BIG * TPP - 1) / (GO_PASSES_BIG * TPP);
      const void* fn = wide ? reinterpret_cast<const void*>(&gather_out_big_kernel<T, DP, true>)
                            : reinterpret_cast<const void*>(&gather_out_big_kernel<T, DP, false>);
      hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      dim3 grid(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk);
      if (wide)
        MURM_LAUNCH((gather_out_big_kernel<T, DP, true>), grid, dim3(GO_THREADS), lds, st, p, nchunk);
      else
        MURM_LAUNCH((gather_out_big_kernel<T, DP, false>), grid, dim3(GO_THREADS), lds, st, p, nchunk);
      return hipGetLastError();
    }
    // half the passes per block when full blocks would leave CUs idle
    const int full = TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) *
                     ((p.N + GO_PASSES_MAX * TPP - 1) / (GO_PASSES_MAX * TPP));
    if (full >= device_cus()) return go(std::integral_constant<int, GO_PASSES_MAX>{});
    return go(std::integral_constant<int, GO_PASSES_MAX / 2>{});
  }
  constexpr int TPB = 256 / (DP / 8);
  dim3 grid((p.N + TPB - 1) / TPB, p.B * p.H);
  MURM_LAUNCH((gather_out_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace

size_t sa_lds_bytes(int dtype, int DP, int M) {
  const size_t Mp = (size_t)((M + 15) & ~15);
  return dtype == DT_F32 ? Mp * (DP + 4) * 4 : 2 * Mp * (DP + 8) * 2;
}

hipError_t launch_select_attend(int dtype, int DP, const SAParams& p, hipStream_t st) {
#define MURM_SA(T)                                            \
  switch (DP) {                                               \
    case 32: return launch_sa_t<T, 32>(p, st);                \
    case 64: return launch_sa_t<T, 64>(p, st);                \
    case 128: return launch_sa_t<T, 128>(p, st);              \
    default: return hipErrorInvalidValue;                     \
  }
  switch (dtype) {
    case DT_BF16: MURM_SA(__bf16)
    case DT_F16: MURM_SA(_Float16)
    case DT_F32: MURM_SA(float)
    default: return hipErrorInvalidValue;
  }
#undef MURM_SA
}

hipError_t launch_gather_out(int dtype, int DP, const OutParams& p, hipStream_t st) {
#define MURM_OUT(T)                                           \
  switch (DP) {                                               \
    case 32: return launch_out_t<T, 32>(p, st);               \
    case 64: return launch_out_t<T, 64>(p, st);               \
    case 128: return launch_out_t<T, 128>(p, st);             \
    default: return hipErrorInvalidValue;                     \
  }
  switch (dtype) {
    case DT_BF16: MURM_OUT(__bf16)
    case DT_F16: MURM_OUT(_Float16)
    case DT_F32: MURM_OUT(float)
    default: return hipErrorInvalidValue;
  }
#undef MURM_OUT
}

}  // namespace murm
