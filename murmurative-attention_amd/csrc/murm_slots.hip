// Slot-side kernels: deterministic per-slot reductions and the small
// per-slot epilogues.
//
// Slot reductions run in two launches per call: seg_partial sums the entries
// of one token chunk per slot, seg_reduce adds the chunks in a fixed order and
// runs the per-slot epilogue.  No float atomics: results are bitwise
// reproducible.
//   UPDATE   K_m = sum w*tk, V_m = sum w*tv, W_m = sum w, then the EMA
//            (reference.py:86-115) and, with diffusion, the stencil over the
//            post-update rows of the block (reference.py:118-135, 188-189).
//   ATTBWD   G''_m = carry_m + (c * sum ds*q, sum w*g): the attend backward's
//            slot side plus the update's pass-through term, which is the
//            gradient of the slots entering the round.  The epilogue then
//            either writes G'' (first round) or runs the previous round's
//            diffusion adjoint and EMA backward on it (halo rows supply the
//            stencil neighbours):
//              G' = D^T G'', dK = (1-a)/(W+eps) G', carry = a G' (used) | G',
//              dW = -(1-a)(K.G'k + V.G'v)/(W+eps)^2.
// du_kernel: the same EMA backward for the standalone update op.

#include <type_traits>

#include "murm_common.h"
#include "murm_launch.h"

namespace murm {

namespace {

constexpr int GS = 16;                 // owned slots per block
constexpr int NSMAX = GS + 2;          // with halo
// 1-D grid, XCD-aware: workgroups are dispatched round-robin over the 8 XCDs
// (linear id % 8), so every block of one (b,h) is placed on XCD bh % 8 and
// reads what the head's other blocks wrote or staged from that XCD's L2.
// Blocks past the last head return before any barrier.
constexpr int XCDS = 8;
__device__ __forceinline__ bool seg_block(const SegParams& p, int& bh, int& g0) {
  const int G = (p.M + GS - 1) / GS;
  const int L = blockIdx.x, x = L % XCDS, k = L / XCDS;
  bh = x + XCDS * (k / G);
  g0 = (k % G) * GS;
  return bh < p.B * p.H;
}

// ---------------------------------------------------------------------------
// Epilogues of the chunk reduction.  The
// block holds, in LDS, the sums of rows lo .. lo+NS-1 (lo = g0 - halo).
// ---------------------------------------------------------------------------
// The old state of the rows a thread visits first in the update epilogue's
// EMA loop (loaded at kernel start, before the partials).
struct OldState {
  float k[2], v[2];
};

__device__ __forceinline__ void load_old(const SegParams& p, int bh, int lo, int NS, int DP, OldState& os) {
  const int64_t base = (int64_t)bh * p.M * p.D;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int i = threadIdx.x + e * blockDim.x;
    const int rel = i / DP, d = i % DP, m = lo + rel;
    const bool ok = p.sk_new && i < NS * DP && m >= 0 && m < p.M && d < p.D;
    os.k[e] = ok ? p.sk_old[base + (int64_t)m * p.D + d] : 0.f;
    os.v[e] = ok ? p.sv_old[base + (int64_t)m * p.D + d] : 0.f;
  }
}

// hi + lo halves of a float32 key in the token dtype TT, stored into the
// split-key table (KeySplit layout: hi table, then lo table, rows of DP + 8)
template <typename TT>
__device__ __forceinline__ void put_split(TT* head, int Mp, int row, int m, int d, float v) {
  const TT hi = (TT)v;
  head[(size_t)m * row + d] = hi;
  head[((size_t)Mp + m) * row + d] = (TT)(v - (float)hi);
}
__device__ __forceinline__ void put_split_dt(const KeySplitOut& ks, int bh, int M, int m, int d, float v) {
  const int Mp = ksplit_mp(M), row = ksplit_row(ks.DP);
  const size_t head = (size_t)bh * ksplit_head_elems(M, ks.DP);
  if (ks.dtype == DT_BF16)
    put_split(static_cast<__bf16*>(ks.p) + head, Mp, row, m, d, v);
  else
    put_split(static_cast<_Float16*>(ks.p) + head, Mp, row, m, d, v);
}

template <int DP>
__device__ void update_epilogue(const SegParams& p, int bh, int g0, int halo, int NS, float* accA, float* accB,
                                const float* accW, const OldState& os) {
  const int lo = g0 - halo;
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
  for (int i = threadIdx.x, e = 0; i < NS * DP; i += blockDim.x, ++e) {
    const int rel = i / DP, d = i % DP, m = lo + rel;
    if (m < 0 || m >= p.M || d >= p.D) continue;
    const float W = accW[rel];
    const float ok = e == 0 ? os.k[0] : (e == 1 ? os.k[1] : p.sk_old[base + (int64_t)m * p.D + d]);
    const float ov = e == 0 ? os.v[0] : (e == 1 ? os.v[1] : p.sv_old[base + (int64_t)m * p.D + d]);
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
  // owned rows; with a split-key output also its zero padding (d >= D, and
  // rows M..Mp-1, which fall in the last slot group)
  const int Mp = ksplit_mp(p.M);
  for (int i = threadIdx.x; i < GS * DP; i += blockDim.x) {
    const int own = i / DP, d = i % DP, m = g0 + own;
    if (m >= Mp) continue;
    float yk = 0.f;
    if (m < p.M && d < p.D) {
      const int rel = own + halo;
      yk = accA[rel * DP + d];
      float yv = accB[rel * DP + d];
      if (p.diffuse && m >= 1 && m <= p.M - 2) {
        yk = yk + gm * (accA[(rel - 1) * DP + d] + accA[(rel + 1) * DP + d] - 2.0f * yk);
        yv = yv + gm * (accB[(rel - 1) * DP + d] + accB[(rel + 1) * DP + d] - 2.0f * yv);
      }
      p.sk_new[base + (int64_t)m * p.D + d] = yk;
      p.sv_new[base + (int64_t)m * p.D + d] = yv;
    }
    if (p.ksplit_new.p) put_split_dt(p.ksplit_new, bh, p.M, m, d, yk);
  }
}

// The previous round's forward sums of the slot a thread's 32-lane group owns
// first in the epilogue (loaded at kernel start, before the partials).
template <int DP>
struct PrevSums {
  float W;
  float k[DP / 32], v[DP / 32];
};

template <int DP>
__device__ __forceinline__ void load_prev(const SegParams& p, int bh, int g0, PrevSums<DP>& ps) {
  constexpr int DPT = DP / 32;
  const int own = threadIdx.x >> 5, sub = threadIdx.x & 31, m = g0 + own;
  const bool live = own < GS && m < p.M;
  const int64_t base = (int64_t)bh * p.M * p.D;
  ps.W = live ? p.Wp[(int64_t)bh * p.M + m] : 0.f;
#pragma unroll
  for (int t = 0; t < DPT; ++t) {
    const int d = sub + 32 * t;
    const bool ok = live && d < p.D;
    ps.k[t] = ok ? p.Kp[base + (int64_t)m * p.D + d] : 0.f;
    ps.v[t] = ok ? p.Vp[base + (int64_t)m * p.D + d] : 0.f;
  }
}

// accA / accB hold G'' (chunk sums + carry) of the owned and halo rows.
template <int DP>
__device__ void attbwd_epilogue(const SegParams& p, int bh, int g0, int halo, int NS, float* accA, float* accB,
                                const PrevSums<DP>& ps) {
  const int64_t base = (int64_t)bh * p.M * p.D;
  if (p.final_out) {
    const int b = bh / p.H, h = bh % p.H;
    for (int i = threadIdx.x; i < GS * DP; i += blockDim.x) {
      const int own = i / DP, d = i % DP, m = g0 + own;
      if (m >= p.M || d >= p.D) continue;
      const float gk = accA[(own + halo) * DP + d], gv = accB[(own + halo) * DP + d];
      if (p.gk_t) {  // the caller's slot-gradient tensors, converted here
        const int64_t t = b * p.gt_sb + h * p.gt_sh + (int64_t)m * p.gt_sm + d;
        if (p.gt_dtype == DT_BF16) {
          static_cast<__bf16*>(p.gk_t)[t] = (__bf16)gk;
          static_cast<__bf16*>(p.gv_t)[t] = (__bf16)gv;
        } else if (p.gt_dtype == DT_F16) {
          static_cast<_Float16*>(p.gk_t)[t] = (_Float16)gk;
          static_cast<_Float16*>(p.gv_t)[t] = (_Float16)gv;
        } else {
          static_cast<float*>(p.gk_t)[t] = gk;
          static_cast<float*>(p.gv_t)[t] = gv;
        }
      } else {
        const int64_t o = base + (int64_t)m * p.D + d;
        p.gk_out[o] = gk;
        p.gv_out[o] = gv;
      }
    }
    return;
  }
  // previous round's diffusion adjoint + EMA backward on the owned rows:
  // 32 threads per slot, DP/32 dims each (DP >= 32); uniform per 32-lane group
  constexpr int DPT = DP / 32;
  const int sub = threadIdx.x & 31;
  const float g = p.gamma, a = p.alpha, oma = 1.0f - p.alpha;
  auto inner = [&](int x) { return p.M >= 3 && x >= 1 && x <= p.M - 2; };
  for (int own = threadIdx.x >> 5; own < GS; own += blockDim.x >> 5) {
    const int m = g0 + own, rel = own + halo;
    const bool live = m < p.M;
    const bool first = own == (int)(threadIdx.x >> 5);  // prefetched
    const float W = first ? ps.W : (live ? p.Wp[(int64_t)bh * p.M + m] : 0.f);
    const bool used = W > 0.f;
    const float inv = oma / (W + p.eps);
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < DPT; ++t) {
      const int d = sub + 32 * t;
      if (!live || d >= p.D) continue;
      auto adj = [&](const float* G) {
        const float c = G[rel * DP + d];
        float r = c;
        if (inner(m)) r -= 2.0f * g * c;
        if (inner(m - 1)) r += g * G[(rel - 1) * DP + d];
        if (inner(m + 1)) r += g * G[(rel + 1) * DP + d];
        return r;
      };
      const float gk = adj(accA), gv = adj(accB);
      const int64_t o = base + (int64_t)m * p.D + d;
      if (used) dot += (first ? ps.k[t] : p.Kp[o]) * gk + (first ? ps.v[t] : p.Vp[o]) * gv;
      const float dk = used ? inv * gk : 0.f, dv = used ? inv * gv : 0.f;
      if (p.combine_dk) {
        p.dk_out[o] = dk + dv;
      } else {
        p.dk_out[o] = dk;
        p.dv_out[o] = dv;
      }
      p.carry_k_out[o] = used ? a * gk : gk;
      p.carry_v_out[o] = used ? a * gv : gv;
    }
#pragma unroll
    for (int x = 1; x < 32; x <<= 1) dot += shfl_xor_f(dot, x);
    if (live && sub == 0) {
      const float den = W + p.eps;
      p.dW_out[(int64_t)bh * p.M + m] = used ? -oma * dot / (den * den) : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// Token-chunk path.
// seg_partial: one block owns a token range of one (b,h) and one group of
// that head's slots; thread (slot, vector, part) accumulates 32 dims of one
// slot sum in registers.  Slot groups (at most 1024 threads a block) are
// adjacent in launch order, so the blocks that stage the same token rows run
// together and share them through L2.  The range is walked in sub-chunks of SUB tokens: the
// token rows (16-byte units, coalesced), index rows and coefficient rows are
// staged in LDS while the next sub-chunk's loads are already in flight in
// registers; each token sets its slots' bits in 64-bit LDS masks (integer OR:
// order-free); every thread then walks its slot's bits in token order and
// reads index, coefficients and row of a token with independent LDS loads.
// The block writes one partial sum per slot.
// seg_reduce: adds the partials of a slot group in chunk order, then runs
// the update or attend-backward epilogue.
// Blocks of one (b,h) run on one XCD (1-D grid, linear id % 8 = XCD), so the
// partials are re-read from that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int SUB = 128;    // tokens per staged sub-chunk
constexpr int CW = 8;       // coefficient row (7 used)
constexpr int NCMAX = 32;   // chunks per (b,h)
constexpr int NCB = 16;     // chunk partials loaded together by the reduction
// reduction threads: with many chunks every (vector, row, 4 dims) item of a
// group (and, in the update, every row's weight sum) gets its own thread (up
// to 1024), so all chunk loads are in flight at once; with few chunks (many
// heads) 256-thread blocks keep more groups resident.  At 4 waves per SIMD
// (128 VGPRs) a CU holds one block sized for two vectors (9 waves at
// d = 64); on grids of more blocks than CUs the one-vector update takes
// threads for its own items (5 waves), so three blocks share a CU (with one
// block per CU the larger block's shorter epilogue loops win).
constexpr int RED_THREADS = 1024;
inline int red_threads(int nchunk, int DP, int mode, const SegParams& p, int blocks) {
  if (nchunk < 8) return 256;
  const int nv = (mode == SEG_UPDATE && p.b_same_as_a && blocks > device_cus()) ? 1 : 2;
  const int items = nv * NSMAX * (DP / 4) + (mode == SEG_UPDATE ? NSMAX : 0);
  int t = (items + 63) & ~63;
  // two-vector blocks on such grids: 512 threads, two blocks per CU (a few
  // threads take a second item)
  if (nv == 2 && blocks > device_cus() && t > 512) t = 512;
  return t > RED_THREADS ? RED_THREADS : t;
}

template <typename T>
__device__ __forceinline__ uint4 load_unit(const TokView& v, int b, int h, int n, int e0, int D) {
  constexpr int E = 16 / sizeof(T);
  const T* row = tok_row<T>(v, b, h, n);
  if (v.vec && e0 + E <= D) return *reinterpret_cast<const uint4*>(row + e0);
  uint4 r;
  T* e = reinterpret_cast<T*>(&r);
#pragma unroll
  for (int i = 0; i < E; ++i) e[i] = (e0 + i < D) ? row[e0 + i] : from_f<T>(0.f);
  return r;
}

// 1-D grid: linear id % 8 = XCD = (b,h) % 8; then slot group, then chunk
__device__ __forceinline__ void part_block(int nchunk, int nsg, int BH, int& bh, int& chunk, int& sg) {
  const int L = blockIdx.x, x = L % XCDS, k = L / XCDS;
  sg = k % nsg;
  const int k2 = k / nsg;
  bh = x + XCDS * (k2 / nchunk);
  chunk = k2 % nchunk;
  if (bh >= BH) bh = -1;
}

template <typename T, int DP, int MODE>
__global__ __launch_bounds__(1024) void seg_partial_kernel(SegParams p, PartParams pp) {
  constexpr int ROW = DP + 8;                 // staged row stride (elements; bytes % 16 == 0)
  constexpr int TPS = DP / 32;                // threads per (slot, vector)
  constexpr int DPT = DP / TPS;               // dims per thread
  constexpr int E = 16 / sizeof(T);           // elements per 16-byte unit
  // 16-byte row units prefetched per thread (more spill at DP = 128 / fp32;
  // stash() loads the remainder directly)
  constexpr int PF = 2;
  constexpr int UPR = DP / E;                 // units per staged row
  constexpr int UPT = DPT / E;                // 16-byte units per thread and token
  extern __shared__ __align__(16) unsigned char smem[];
  const bool sameB = (MODE == SEG_UPDATE) && p.b_same_as_a;
  const int nvec = sameB ? 1 : 2;
  const int MS = blockDim.x / (TPS * nvec);                               // slots per block (multiple of 64)
  const int nsg = (p.M + MS - 1) / MS;
  T* rows = reinterpret_cast<T*>(smem);                                   // [nvec][SUB][ROW]
  uint4* idxs = reinterpret_cast<uint4*>(rows + nvec * SUB * ROW);        // [SUB]
  float* cw = reinterpret_cast<float*>(idxs + SUB);                       // [SUB][CW] weights
  float* cd = cw + SUB * CW;                                              // [SUB][CW] c * ds
  unsigned long long* masks =
      reinterpret_cast<unsigned long long*>(cd + (MODE == SEG_ATTBWD ? SUB * CW : 0));  // [SUB/64][MS]
  uint8_t* jt = reinterpret_cast<uint8_t*>(masks + (SUB / 64) * MS);  // [SUB][MS]: j naming the slot

  int bh, chunk, sg;
  part_block(pp.nchunk, nsg, p.B * p.H, bh, chunk, sg);
  if (bh < 0) return;  // whole block, before any barrier
  const int b = bh / p.H, h = bh % p.H;
  const int c_beg = chunk * pp.chunk_tokens;
  const int c_end = min(p.N, c_beg + pp.chunk_tokens);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int part = tid % TPS;
  const int vec = (tid / TPS) % nvec;
  const int s0 = sg * MS;
  const int slot = s0 + tid / (TPS * nvec);
  const bool own = slot < p.M;
  const int nunits = nvec * SUB * UPR;

  uint4 pf[PF];
  uint4 pidx;
  float pw[2], pd[2];
  // global -> registers (the first PF units per thread, one index row, two coefficients)
  auto fetch = [&](int n0) {
    const int cnt = min(SUB, c_end - n0);
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int u = tid + k * nthr;
      pf[k] = make_uint4(0u, 0u, 0u, 0u);
      const int v = u / (SUB * UPR), r = (u / UPR) % SUB, c = u % UPR;
      if (u < nunits && r < cnt) pf[k] = load_unit<T>(v == 0 ? p.va : p.vb, b, h, n0 + r, c * E, p.D);
    }
    const int64_t row0 = (int64_t)bh * p.N + n0;
    pidx = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (tid < cnt) pidx = *reinterpret_cast<const uint4*>(p.idx + (row0 + tid) * IDX_ROW);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = tid + k * nthr, t = i / CW, j = i % CW;
      const bool in = i < SUB * CW && t < cnt && j < KN;
      pw[k] = in ? p.wgt[(row0 + t) * KN + j] : 0.f;
      pd[k] = (MODE == SEG_ATTBWD && in) ? p.ds[(row0 + t) * KN + j] : 0.f;  // scaled when stashed
    }
  };
  // registers -> LDS, plus whatever the registers did not cover (small blocks)
  auto stash = [&](int n0) {
    const int cnt = min(SUB, c_end - n0);
    const int64_t row0 = (int64_t)bh * p.N + n0;
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int u = tid + k * nthr;
      const int v = u / (SUB * UPR), r = (u / UPR) % SUB, c = u % UPR;
      if (u < nunits) *reinterpret_cast<uint4*>(rows + (v * SUB + r) * ROW + c * E) = pf[k];
    }
    for (int u = tid + PF * nthr; u < nunits; u += nthr) {
      const int v = u / (SUB * UPR), r = (u / UPR) % SUB, c = u % UPR;
      *reinterpret_cast<uint4*>(rows + (v * SUB + r) * ROW + c * E) =
          r < cnt ? load_unit<T>(v == 0 ? p.va : p.vb, b, h, n0 + r, c * E, p.D) : make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid < SUB) idxs[tid] = pidx;
    for (int i = tid + nthr; i < SUB; i += nthr)
      idxs[i] = i < cnt ? *reinterpret_cast<const uint4*>(p.idx + (row0 + i) * IDX_ROW)
                        : make_uint4(~0u, ~0u, ~0u, ~0u);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = tid + k * nthr;
      if (i < SUB * CW) {
        cw[i] = pw[k];
        if (MODE == SEG_ATTBWD) cd[i] = p.ds_scale * pd[k];
      }
    }
    for (int i = tid + 2 * nthr; i < SUB * CW; i += nthr) {
      const int t = i / CW, j = i % CW;
      const bool in = t < cnt && j < KN;
      cw[i] = in ? p.wgt[(row0 + t) * KN + j] : 0.f;
      if (MODE == SEG_ATTBWD) cd[i] = in ? p.ds_scale * p.ds[(row0 + t) * KN + j] : 0.f;
    }
    for (int i = tid; i < (SUB / 64) * MS; i += nthr) masks[i] = 0ull;
  };

  float acc[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) acc[i] = 0.f;
  float accw = 0.f;
  const T* vrows = rows + vec * SUB * ROW + part * DPT;
  const float* coef = (MODE == SEG_ATTBWD && vec == 0) ? cd : cw;
  const bool wacc = (MODE == SEG_UPDATE) && vec == 0 && part == 0;
  // acc += a * (this thread's dims of staged row t), one 16-byte unit at a time
  auto fma_staged = [&](int t, float a) {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const uint4 x = *reinterpret_cast<const uint4*>(vrows + t * ROW + u * E);
      const T* e = reinterpret_cast<const T*>(&x);
#pragma unroll
      for (int i = 0; i < E; ++i) acc[u * E + i] += a * to_f(e[i]);
    }
  };

  fetch(c_beg);
  for (int n0 = c_beg; n0 < c_end; n0 += SUB) {
    const int cnt = min(SUB, c_end - n0);
    stash(n0);
    __syncthreads();
    if (n0 + SUB < c_end) fetch(n0 + SUB);  // in flight during marking and the walk
    // one thread per (token, j): the first j naming a slot of this group sets
    // the token's bit and records j; later js naming the same slot (caller-
    // given indices only) add their coefficients to the first one's, in j order
    for (int i = tid; i < cnt * CW; i += nthr) {
      const int t = i / CW, j = i % CW;
      const uint4 ir = idxs[t];
      const uint32_t sj = idx_at(ir, j);
      const uint32_t s = sj - (uint32_t)s0;  // slots of this group; others wrap past MS
      if (j >= KN || s >= (uint32_t)MS || sj >= (uint32_t)p.M) continue;
      uint32_t before = 0, after = 0;
#pragma unroll
      for (int q = 0; q < KN; ++q) {
        const uint32_t hit = idx_at(ir, q) == sj ? 1u : 0u;
        before |= (q < j ? hit : 0u) << q;
        after |= (q > j ? hit : 0u) << q;
      }
      if (before) continue;
      if (after) {
        float a = cw[t * CW + j], c = MODE == SEG_ATTBWD ? cd[t * CW + j] : 0.f;
        for (uint32_t r = after; r; r &= r - 1u) {
          a += cw[t * CW + __builtin_ctz(r)];
          if (MODE == SEG_ATTBWD) c += cd[t * CW + __builtin_ctz(r)];
        }
        cw[t * CW + j] = a;
        if (MODE == SEG_ATTBWD) cd[t * CW + j] = c;
      }
      atomicOr(&masks[(t >> 6) * MS + s], 1ull << (t & 63));
      jt[t * MS + s] = (uint8_t)j;
    }
    __syncthreads();
    if (own) {
#pragma unroll
      for (int g = 0; g < SUB / 64; ++g) {
        unsigned long long mk = masks[g * MS + (slot - s0)];
        while (mk) {
          const int t = g * 64 + (int)__builtin_ctzll(mk);
          mk &= mk - 1ull;
          const float a = coef[t * CW + jt[t * MS + (slot - s0)]];
          fma_staged(t, a);
          if (wacc) accw += a;
        }
      }
    }
    __syncthreads();
  }
  if (!own) return;
  const int64_t prow = ((int64_t)chunk * p.B * p.H + bh) * p.M + slot;
  float* dst = (vec == 0 ? pp.partA : pp.partB) + prow * p.D + part * DPT;
  if ((p.D & 3) == 0 && part * DPT + DPT <= p.D) {
#pragma unroll
    for (int i = 0; i < DPT; i += 4)
      *reinterpret_cast<float4*>(dst + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < DPT; ++i)
      if (part * DPT + i < p.D) dst[i] = acc[i];
  }
  if (wacc) pp.partW[prow] = accw;
}

// ---------------------------------------------------------------------------
// Token-chunk partial sums on MFMA (bf16 / fp16 tokens).
// The slot sums of a sub-chunk are the product C^T X of the coefficient
// matrix C [tokens x slots] (at most 7 nonzeros per token: w, or c*ds) and
// the token rows X [tokens x d].  Per sub-chunk (SUBT tokens) the block stages X
// transposed (d-major, so 8 consecutive tokens of one dim form one 16-byte
// MFMA operand) and C^T as hi + lo halves of the token dtype (hi = rn(c),
// lo = rn(c - hi)); their products with the exact 16-bit X accumulate in
// fp32, ~2^-16 relative to fp32 coefficients.  The marking threads write the
// C^T entries and reset them to zero after use, so the table is cleared once
// per block.  Each vector has its own 4 waves; wave w owns 16-slot tiles
// w, w+4, ... of the block's slot group and keeps their sums for every dim
// tile in MFMA accumulators across the chunk; with UPDATE a ones column gives
// the weight sums.  With TG = 2 token groups the block holds two such sets of
// waves, each with its own LDS staging, over the two halves of the chunk; the
// upper half's sums are added to the lower half's through LDS at the end, so
// the block writes one partial for twice the tokens.  Fixed k order inside
// each MFMA, sub-chunks in token order, halves added lower + upper: bitwise
// reproducible.
// ---------------------------------------------------------------------------
constexpr int MMA_WAVES = 4;       // waves per vector

// Byte offset of 16-byte chunk `c` of LDS row `row` (rows of SUBT 16-bit
// tokens).  The XOR keeps the operand reads of 16 consecutive rows (one chunk
// each) on 16 distinct 16-byte bank groups; the row >> 4 term spreads the
// transposed staging stores (rows 8 apart).
template <int SUBT>
__device__ __forceinline__ int swz(int row, int c) {
  constexpr int ROWB = SUBT * 2, CPR = ROWB / 16;
  const int f = CPR == 8 ? ((row >> 1) ^ (row >> 4)) : ((row >> 2) ^ (row >> 4));
  return row * ROWB + ((c ^ f) & (CPR - 1)) * 16;
}

template <int DP, int MODE, int NV, int SUBT, int TG = 1>
struct MmaShape {
  static constexpr int GT = 64 * MMA_WAVES * NV;            // threads of a token group: waves per vector
  static constexpr int THREADS = GT * TG;
  static constexpr int DT = DP / 16;                        // dim tiles
  static constexpr int KINDS = MODE == SEG_ATTBWD ? 2 : 1;  // coefficient kinds (c*ds, w)
  static constexpr int WTILE = MODE == SEG_UPDATE ? 1 : 0;  // ones tile for the weight sums
  static constexpr int ROWB = SUBT * 2;
  // The attend backward (d <= 64) sizes its slot group for two blocks per CU
  // (80 KiB of LDS, 128 VGPRs each), so one block's staging and marking run
  // beside the other's products; the other forms run one block per CU (the
  // update with one vector as a ping-pong pair of token groups).
  static constexpr int BLOCKS_PER_CU = MODE == SEG_ATTBWD && DP <= 64 ? 2 : 1;
  static constexpr int BUDGET = BLOCKS_PER_CU == 2 ? 80 * 1024 : 144 * 1024;
  // C^T in what is left of the budget (per token group) after the token rows,
  // in whole groups of MMA_WAVES tiles
  static constexpr int MS_LDS =
      ((BUDGET / TG - NV * DP * ROWB) / (KINDS * 2 * ROWB)) / (MMA_WAVES * 16) * (MMA_WAVES * 16);
  // slot tiles per wave: at most 64 accumulators
  static constexpr int WT = 256 / DP < MS_LDS / (MMA_WAVES * 16) ? 256 / DP : MS_LDS / (MMA_WAVES * 16);
  static constexpr int MS_REG = MMA_WAVES * WT * 16;
  static constexpr int MS = MS_REG < MS_LDS ? MS_REG : MS_LDS;    // slots per block
  static constexpr int WAVES_PER_EU = BLOCKS_PER_CU * (64 * MMA_WAVES * NV * TG / 64) / 4;
  static constexpr size_t GLDS = (size_t)NV * DP * ROWB + (size_t)KINDS * 2 * MS * ROWB;  // per group
  static constexpr int NACC = WT * DT + WTILE * WT;         // float4 accumulators per thread
  static constexpr size_t MERGE = TG > 1 ? (size_t)NACC * GT * 16 : 0;
  static constexpr size_t LDS = TG * GLDS > MERGE ? TG * GLDS : MERGE;
};

template <typename T, int DP, int MODE, int NV, int SUBT, int TG>
__global__ __launch_bounds__(64 * MMA_WAVES * NV * TG, (MmaShape<DP, MODE, NV, SUBT, TG>::WAVES_PER_EU))
void seg_mma_kernel(SegParams p, PartParams pp) {
  using V = typename Mfma16<T>::vec;
  using Sh = MmaShape<DP, MODE, NV, SUBT, TG>;
  constexpr int DT = Sh::DT, KINDS = Sh::KINDS, WT = Sh::WT, MS = Sh::MS, ROWB = Sh::ROWB;
  constexpr int MMA_THREADS = Sh::GT;             // staging and marking run per token group
  constexpr int UPR = DP / 8;                      // 16-byte units per token row
  constexpr int GROUPS = NV * UPR * (SUBT / 4);    // staging items: (vector, unit, 4 tokens)
  constexpr int GPT = (GROUPS + MMA_THREADS - 1) / MMA_THREADS;
  constexpr int TPT = MMA_THREADS / SUBT;          // marking threads per token (one wave)
  constexpr int JPT = (8 + TPT - 1) / TPT;         // js per marking thread
  extern __shared__ __align__(16) unsigned char smem[];
  const int tg = TG > 1 ? (int)threadIdx.x / MMA_THREADS : 0;  // token group
  unsigned char* xt = smem + tg * Sh::GLDS;          // [NV*DP rows][ROWB]
  unsigned char* ct = xt + NV * DP * ROWB;           // [KINDS][hi, lo][MS rows][ROWB]

  int bh, chunk, sg;
  const int nsg = (p.M + MS - 1) / MS;
  part_block(pp.nchunk, nsg, p.B * p.H, bh, chunk, sg);
  if (bh < 0) return;  // whole block, before any barrier
  const int b = bh / p.H, h = bh % p.H;
  // this token group's whole sub-chunks of the chunk (the same count for every group)
  const int k_beg = chunk * pp.chunk_tokens;
  const int nsub = (min(p.N, k_beg + pp.chunk_tokens) - k_beg + SUBT - 1) / SUBT;
  const int per = (nsub + TG - 1) / TG;
  const int c_beg = k_beg + tg * per * SUBT;
  const int c_end = min(min(p.N, k_beg + pp.chunk_tokens), c_beg + per * SUBT);
  const int s0 = sg * MS;
  const int tid = (int)threadIdx.x % MMA_THREADS, lane = tid & 63, wave = (tid >> 6) % MMA_WAVES,
            vw = (tid >> 6) / MMA_WAVES;
  const int ms_here = min(MS, p.M - s0);
  const int ntiles = (ms_here + 15) / 16;

  for (int i = tid; i < KINDS * 2 * MS * ROWB / 16; i += MMA_THREADS)
    reinterpret_cast<uint4*>(ct)[i] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();  // cleared before any marking store

  // ---- prefetch registers: token rows, then (marking) one index row and the
  // coefficients of this thread's js
  uint4 px[GPT][4];
  uint4 pidx;
  float pc[KINDS][JPT];
  const int mt = tid / TPT, mk = tid % TPT;  // marking token, j group
  // Prefetch: loads from clamped (always valid) rows straight into the
  // registers, validity applied when staging, so no load is predicated or
  // copied (either makes the wave wait for it before the products).
  const bool wide = p.va.vec && (NV == 1 || p.vb.vec) && (p.D & 7) == 0;
  auto unit_of = [&](int item, int& v, int& u, int& g4) {
    v = item / (UPR * (SUBT / 4));
    const int rem = item % (UPR * (SUBT / 4));
    u = rem % UPR;
    g4 = rem / UPR;
  };
  // Addresses: the (b,h) bases are uniform; a token's row is one unsigned
  // 32 x 32 -> 64-bit multiply-add on top (row numbers and strides < 2^32).
  const T* va0 = tok_row<T>(p.va, b, h, 0);
  const T* vb0 = tok_row<T>(p.vb, b, h, 0);
  const uint32_t sna = (uint32_t)p.va.sn, snb = (uint32_t)p.vb.sn;
  const uint32_t rbase = (uint32_t)bh * (uint32_t)p.N;
  auto fetch = [&](int n0) {
    // marking loads first, token rows last (nothing after them touches a register)
    const uint32_t row = rbase + (uint32_t)min(n0 + mt, p.N - 1);
    pidx = *reinterpret_cast<const uint4*>(p.idx + (uint64_t)row * IDX_ROW);
    const uint64_t crow = (uint64_t)row * KN;
#pragma unroll
    for (int q = 0; q < JPT; ++q) {
      const int j = min(JPT * mk + q, KN - 1);
      if (MODE == SEG_ATTBWD) {
        pc[0][q] = p.ds[crow + j];  // scaled when marked
        pc[KINDS - 1][q] = p.wgt[crow + j];
      } else {
        pc[0][q] = p.wgt[crow + j];
      }
    }
    if (wide) {
#pragma unroll
      for (int g = 0; g < GPT; ++g) {
        const int item = tid + g * MMA_THREADS;
        if (GROUPS % MMA_THREADS != 0 && item >= GROUPS) continue;
        int v, u, g4;
        unit_of(item, v, u, g4);
        const T* base = (v == 0 ? va0 : vb0) + u * 8;
        const uint32_t sn = v == 0 ? sna : snb;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          px[g][k] = *reinterpret_cast<const uint4*>(base + (uint64_t)(uint32_t)min(n0 + 4 * g4 + k, p.N - 1) * sn);
      }
    }
  };

  // ---- staging: 4 tokens x 8 dims transposed into 8 dim rows of 4 tokens
  auto stash = [&](int n0) {
    const int cnt = min(SUBT, c_end - n0);
#pragma unroll
    for (int g = 0; g < GPT; ++g) {
      const int item = tid + g * MMA_THREADS;
      if (item >= GROUPS) continue;
      int v, u, g4;
      unit_of(item, v, u, g4);
      uint4 x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int t = 4 * g4 + k;
        const bool ok = t < cnt && u * 8 < p.D;
        if (wide) {
          x[k] = px[g][k];
        } else {  // unaligned rows or a ragged last unit: element loads now, packed as dwords
          const uint16_t* e =
              reinterpret_cast<const uint16_t*>(tok_row<T>(v == 0 ? p.va : p.vb, b, h, min(n0 + t, p.N - 1))) + u * 8;
          uint32_t w[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t lo = u * 8 + 2 * q < p.D ? e[2 * q] : 0u;
            const uint32_t hi = u * 8 + 2 * q + 1 < p.D ? e[2 * q + 1] : 0u;
            w[q] = lo | (hi << 16);
          }
          x[k] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if (!ok) x[k] = make_uint4(0u, 0u, 0u, 0u);
      }
      const uint32_t* x0 = reinterpret_cast<const uint32_t*>(&x[0]);
      const uint32_t* x1 = reinterpret_cast<const uint32_t*>(&x[1]);
      const uint32_t* x2 = reinterpret_cast<const uint32_t*>(&x[2]);
      const uint32_t* x3 = reinterpret_cast<const uint32_t*>(&x[3]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
        uint2 o;
        o.x = __builtin_amdgcn_perm(x1[i >> 1], x0[i >> 1], sel);
        o.y = __builtin_amdgcn_perm(x3[i >> 1], x2[i >> 1], sel);
        const int r = v * DP + u * 8 + i;
        *reinterpret_cast<uint2*>(xt + swz<SUBT>(r, g4 >> 1) + (g4 & 1) * 8) = o;
      }
    }
  };

  // ---- marking: entries of token mt for its js (first j of a slot; later
  // js naming the same slot add their coefficients in j order)
  int prev[JPT];
#pragma unroll
  for (int q = 0; q < JPT; ++q) prev[q] = -1;
  auto put = [&](int off, int kind, float c) {
    const T hi = (T)c;
    const T lo = (T)(c - (float)hi);
    *reinterpret_cast<T*>(ct + (kind * 2 + 0) * MS * ROWB + off) = hi;
    *reinterpret_cast<T*>(ct + (kind * 2 + 1) * MS * ROWB + off) = lo;
  };
  auto mark = [&](int n0) {
    // clear this thread's entries of the previous sub-chunk first (the
    // threads of one token are one wave, so these stores precede its new ones)
#pragma unroll
    for (int q = 0; q < JPT; ++q)
      if (prev[q] >= 0)
#pragma unroll
        for (int kind = 0; kind < KINDS; ++kind) put(prev[q], kind, 0.f);
    const bool live = n0 + mt < c_end;
    const uint4 ir = live ? pidx : make_uint4(~0u, ~0u, ~0u, ~0u);
    const int64_t row = (int64_t)bh * p.N + n0 + mt;
#pragma unroll
    for (int q = 0; q < JPT; ++q) {
      prev[q] = -1;
      const int j = JPT * mk + q;
      if (j >= KN) continue;
      const uint32_t sj = idx_at(ir, j);
      const uint32_t sl = sj - (uint32_t)s0;  // slots of this group; others wrap past MS
      if (sl >= (uint32_t)MS || sj >= (uint32_t)p.M) continue;
      uint32_t before = 0, after = 0;
      if (!p.uniq_idx) {  // caller-given indices may repeat a slot
#pragma unroll
        for (int x = 0; x < KN; ++x) {
          const uint32_t hit = idx_at(ir, x) == sj ? 1u : 0u;
          before |= (x < j ? hit : 0u) << x;
          after |= (x > j ? hit : 0u) << x;
        }
        if (before) continue;
      }
      float c[KINDS];
#pragma unroll
      for (int kind = 0; kind < KINDS; ++kind) c[kind] = pc[kind][q];
      if (MODE == SEG_ATTBWD) c[0] *= p.ds_scale;
      for (uint32_t r = after; r; r &= r - 1u) {  // caller-given duplicate indices only
        const int x = __builtin_ctz(r);
        if (MODE == SEG_ATTBWD) {
          c[0] += p.ds_scale * p.ds[row * KN + x];
          c[KINDS - 1] += p.wgt[row * KN + x];
        } else {
          c[0] += p.wgt[row * KN + x];
        }
      }
      const int off = swz<SUBT>((int)sl, mt >> 3) + (mt & 7) * 2;
#pragma unroll
      for (int kind = 0; kind < KINDS; ++kind) put(off, kind, c[kind]);
      prev[q] = off;
    }
  };

  // wave group vw owns vector vw (coefficient kind vw with ATTBWD)
  const int kind = MODE == SEG_ATTBWD ? vw : 0;
  const bool wsum = Sh::WTILE && vw == 0;
  f32x4 acc[WT][DT];
  f32x4 accw[Sh::WTILE ? WT : 1];
#pragma unroll
  for (int i = 0; i < WT; ++i) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[i][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (Sh::WTILE) accw[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  V ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (T)((lane & 15) == 0 ? 1.f : 0.f);
  auto load_a = [&](int tile, int chk, V (&a)[2]) {
    const int srow = tile * 16 + (lane & 15);
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
      a[hl] = *reinterpret_cast<const V*>(ct + (kind * 2 + hl) * MS * ROWB + swz<SUBT>(srow, chk));
  };

  auto products = [&]() {
#pragma unroll
    for (int ks = 0; ks < SUBT / 32; ++ks) {
      const int chk = ks * 4 + (lane >> 4);
      V bx[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        bx[dt] = *reinterpret_cast<const V*>(xt + swz<SUBT>(vw * DP + dt * 16 + (lane & 15), chk));
      V a[2], an[2];
      if (wave < ntiles) load_a(wave, chk, a);
#pragma unroll
      for (int i = 0; i < WT; ++i) {
        const int tile = wave + MMA_WAVES * i;
        if (tile >= ntiles) break;  // wave-uniform
        if (i + 1 < WT && tile + MMA_WAVES < ntiles) load_a(tile + MMA_WAVES, chk, an);  // next tile in flight
        // lo halves of every accumulator, then hi halves
#pragma unroll
        for (int hl = 1; hl >= 0; --hl) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[i][dt] = mfma_16x16x32(a[hl], bx[dt], acc[i][dt]);
          if (Sh::WTILE && wsum) accw[i] = mfma_16x16x32(a[hl], ones, accw[i]);
        }
        a[0] = an[0];
        a[1] = an[1];
      }
    }
  };

  fetch(c_beg);
  if constexpr (TG == 1) {
    for (int it = 0; it < per; ++it) {
      const int n0 = c_beg + it * SUBT;
      stash(n0);
      mark(n0);
      __syncthreads();
      if (it + 1 < per) fetch(n0 + SUBT);  // in flight during the products
      products();
      __syncthreads();
    }
  } else {
    // Ping-pong: in each half-step one group stages a sub-chunk while the
    // other multiplies its previous one, so staging (VALU, LDS stores) and
    // products (MFMA) overlap across the groups.  A group past its tokens
    // stages zeros, so both groups run the same barriers.
    for (int k = 0; k <= per; ++k) {
      if (tg == 0) {
        if (k < per) { stash(c_beg + k * SUBT); mark(c_beg + k * SUBT); }
      } else if (k >= 1) {
        if (k < per) fetch(c_beg + k * SUBT);
        products();
      }
      __syncthreads();
      if (k < per) {
        if (tg == 0) {
          if (k + 1 < per) fetch(c_beg + (k + 1) * SUBT);
          products();
        } else {
          stash(c_beg + k * SUBT);
          mark(c_beg + k * SUBT);
        }
      }
      __syncthreads();
    }
  }

  if constexpr (TG > 1) {  // upper token group's sums added to the lower group's
    static_assert(TG == 2, "seg_mma_kernel: one or two token groups");
    float4* mb = reinterpret_cast<float4*>(smem);  // staging is no longer read
    auto slot4 = [&](int k) -> float4& { return mb[k * MMA_THREADS + tid]; };
    if (tg == 1) {
#pragma unroll
      for (int i = 0; i < WT; ++i) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          slot4(i * DT + dt) = make_float4(acc[i][dt][0], acc[i][dt][1], acc[i][dt][2], acc[i][dt][3]);
        if (Sh::WTILE) slot4(WT * DT + i) = make_float4(accw[i][0], accw[i][1], accw[i][2], accw[i][3]);
      }
    }
    __syncthreads();
    if (tg == 1) return;
#pragma unroll
    for (int i = 0; i < WT; ++i) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const float4 o = slot4(i * DT + dt);
        acc[i][dt] += f32x4{o.x, o.y, o.z, o.w};
      }
      if (Sh::WTILE) {
        const float4 o = slot4(WT * DT + i);
        accw[i] += f32x4{o.x, o.y, o.z, o.w};
      }
    }
  }

  // ---- partial sums: lane holds rows 4*(lane>>4)+r of column lane&15 per tile
  const int64_t prow0 = ((int64_t)chunk * p.B * p.H + bh) * p.M;
  float* dst0 = (vw == 0 ? pp.partA : pp.partB);
#pragma unroll
  for (int i = 0; i < WT; ++i) {
    const int tile = wave + MMA_WAVES * i;
    if (tile >= ntiles) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int slot = s0 + tile * 16 + 4 * (lane >> 4) + r;
      if (slot >= p.M) continue;
      const int64_t prow = prow0 + slot;
      float* dst = dst0 + prow * p.D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = dt * 16 + (lane & 15);
        if (d < p.D) dst[d] = acc[i][dt][r];
      }
      if (wsum && (lane & 15) == 0) pp.partW[prow] = accw[i][r];
    }
  }
}

template <int DP, int MODE>
__global__ __launch_bounds__(RED_THREADS) void seg_reduce_kernel(SegParams p, PartParams pp) {
  __shared__ float accA[NSMAX * DP], accB[NSMAX * DP], accW[NSMAX];
  int bh, g0;
  if (!seg_block(p, bh, g0)) return;
  const int halo = (MODE == SEG_UPDATE) ? (p.diffuse ? 1 : 0) : (p.final_out ? 0 : 1);
  const int lo = g0 - halo, NS = GS + 2 * halo;
  const bool sameB = (MODE == SEG_UPDATE) && p.b_same_as_a;
  const int nv = sameB ? 1 : 2;
  const int64_t cstride = (int64_t)p.B * p.H * p.M * p.D;
  const int nc = pp.nchunk;
  constexpr int QPR = DP / 4;
  // Items: quads of 4 dims of a vector row, then (UPDATE) the weight sum of
  // each row.  Every item issues its chunk loads in batches of NCB before
  // adding them in chunk order.
  const int nquad = nv * NS * QPR;
  const int nitem = nquad + (MODE == SEG_UPDATE ? NS : 0);
  PrevSums<DP> ps{};
  OldState os{};
  if (MODE == SEG_ATTBWD && !p.final_out) load_prev<DP>(p, bh, g0, ps);  // in flight with the partials
  if (MODE == SEG_UPDATE) load_old(p, bh, lo, NS, DP, os);
  for (int i = threadIdx.x; i < nitem; i += blockDim.x) {
    if (i >= nquad) {
      const int rel = i - nquad, m = lo + rel;
      float sw = 0.f;
      if (m >= 0 && m < p.M) {
        const float* src = pp.partW + (int64_t)bh * p.M + m;
        const int64_t ws = (int64_t)p.B * p.H * p.M;
        for (int c0 = 0; c0 < nc; c0 += NCB) {
          float x[NCB];
#pragma unroll
          for (int c = 0; c < NCB; ++c) x[c] = c0 + c < nc ? src[(c0 + c) * ws] : 0.f;
#pragma unroll
          for (int c = 0; c < NCB; ++c)
            if (c0 + c < nc) sw += x[c];
        }
      }
      accW[rel] = sw;
      continue;
    }
    const int v = i / (NS * QPR), rel = (i / QPR) % NS, d = (i % QPR) * 4, m = lo + rel;
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m >= 0 && m < p.M && d < p.D) {
      const float* src = (v == 0 ? pp.partA : pp.partB) + ((int64_t)bh * p.M + m) * p.D + d;
      // ATTBWD: the carried gradient of the row is added after the chunk sums
      const float* cry = MODE == SEG_ATTBWD ? (v == 0 ? p.carry_k : p.carry_v) : nullptr;
      const int64_t co = ((int64_t)bh * p.M + m) * p.D + d;
      if ((p.D & 3) == 0) {
        const float4 cv = cry ? *reinterpret_cast<const float4*>(cry + co) : make_float4(0.f, 0.f, 0.f, 0.f);
        for (int c0 = 0; c0 < nc; c0 += NCB) {  // chunk order: batches of NCB loads in flight
          float4 x[NCB];
#pragma unroll
          for (int c = 0; c < NCB; ++c)
            x[c] = c0 + c < nc ? *reinterpret_cast<const float4*>(src + (c0 + c) * cstride)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
          for (int c = 0; c < NCB; ++c) {
            if (c0 + c < nc) {
              sum.x += x[c].x; sum.y += x[c].y; sum.z += x[c].z; sum.w += x[c].w;
            }
          }
        }
        if (cry) { sum.x += cv.x; sum.y += cv.y; sum.z += cv.z; sum.w += cv.w; }
      } else {
        float t[4] = {0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < nc; ++c)
          for (int e = 0; e < 4; ++e)
            if (d + e < p.D) t[e] += src[c * cstride + e];
        if (cry)
          for (int e = 0; e < 4; ++e)
            if (d + e < p.D) t[e] += cry[co + e];
        sum = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
    float* acc = (v == 0 ? accA : accB) + rel * DP + d;
    acc[0] = sum.x; acc[1] = sum.y; acc[2] = sum.z; acc[3] = sum.w;
    if (sameB) {
      float* accb = accB + rel * DP + d;
      accb[0] = sum.x; accb[1] = sum.y; accb[2] = sum.z; accb[3] = sum.w;
    }
  }
  __syncthreads();
  if (MODE == SEG_UPDATE)
    update_epilogue<DP>(p, bh, g0, halo, NS, accA, accB, accW, os);
  else
    attbwd_epilogue<DP>(p, bh, g0, halo, NS, accA, accB, ps);
}

// One block per (b,h): G' = D^T G'' (optional), then the EMA backward.
__global__ __launch_bounds__(256) void du_kernel(DuParams p) {
  const int bh = blockIdx.y;
  const int64_t base = (int64_t)bh * p.M * p.D;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float g = p.gamma, a = p.alpha, oma = 1.0f - p.alpha;
  {
    const int m = blockIdx.x * 4 + wave;
    if (m >= p.M) return;
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

// fp32 state [BH,M,D] from a [B,H,M,D] slot tensor of any dtype and strides,
// and back; blockIdx.y picks one of up to two tensors of one launch.
template <typename T>
__global__ void to_state_kernel(SlotConv<const T*, float*> c0, SlotConv<const T*, float*> c1, int B, int H, int M,
                                int D) {
  const SlotConv<const T*, float*>& c = blockIdx.y == 0 ? c0 : c1;
  const int64_t total = (int64_t)B * H * M * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    int64_t r = i / D;
    const int m = (int)(r % M);
    r /= M;
    const int h = (int)(r % H);
    const int b = (int)(r / H);
    c.dst[i] = to_f(c.src[b * c.sb + h * c.sh + m * c.sm + d]);
  }
}

// The same with one thread per 4 consecutive elements of a row and 32-bit
// index arithmetic (B*H*M*ceil(D/4) < 2^30; the launchers check).
template <typename T>
__global__ void to_state4_kernel(SlotConv<const T*, float*> c0, SlotConv<const T*, float*> c1, int H, int M,
                                 int D, int total4) {
  const SlotConv<const T*, float*>& c = blockIdx.y == 0 ? c0 : c1;
  const int D4 = (D + 3) >> 2;
  for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < total4; q += gridDim.x * blockDim.x) {
    const int row = q / D4, d0 = (q - row * D4) * 4;
    const int bh = row / M, m = row - bh * M, b = bh / H, h = bh - b * H;
    const T* sp = c.src + b * c.sb + h * c.sh + (int64_t)m * c.sm + d0;
    float* o = c.dst + (int64_t)row * D + d0;
    if (d0 + 4 <= D) {
      const float4 v = make_float4(to_f(sp[0]), to_f(sp[1]), to_f(sp[2]), to_f(sp[3]));
      if ((D & 3) == 0) {
        *reinterpret_cast<float4*>(o) = v;
      } else {
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
      }
    } else {
      for (int e = 0; d0 + e < D; ++e) o[e] = to_f(sp[e]);
    }
  }
}

// The same conversion with the keys (blockIdx.z == 0) also written split for
// the 16-bit select kernel (Mp rows of DP dims per head, zero past M and D)
// and the values (blockIdx.z == 1) as float32 only.  Block x covers RPB rows
// of one (b,h); a thread converts 4 dims of a row, with one vector load when
// the tensor's rows are 4-element aligned (`vec`).
template <typename T>
__device__ __forceinline__ void load4f(const T* p, float (&f)[4]) {
  if constexpr (sizeof(T) == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = to_f(e[i]);
  } else {
    const float4 v = *reinterpret_cast<const float4*>(p);
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  }
}

template <typename T, typename TT, int DP>
__global__ __launch_bounds__(256) void to_state_split_kernel(SlotConv<const T*, float*> ck,
                                                             SlotConv<const T*, float*> cv, TT* split, int H, int M,
                                                             int D, int nrb, int vec_k, int vec_v) {
  constexpr int DP4 = DP / 4, RPB = 256 / DP4;
  const int bh = blockIdx.x / nrb, rb = blockIdx.x - bh * nrb;
  const int b = bh / H, h = bh - b * H;
  const int m = rb * RPB + (int)threadIdx.x / DP4, d0 = ((int)threadIdx.x % DP4) * 4;
  const bool keys = blockIdx.z == 0;
  const SlotConv<const T*, float*>& c = keys ? ck : cv;
  const int Mp = ksplit_mp(M);
  if (m >= (keys ? Mp : M)) return;
  float f[4] = {0.f, 0.f, 0.f, 0.f};
  if (m < M && d0 < D) {
    const T* sp = c.src + b * c.sb + h * c.sh + (int64_t)m * c.sm + d0;
    float* o = c.dst + ((int64_t)bh * M + m) * D + d0;
    if (keys ? vec_k : vec_v) {  // D % 4 == 0: o is 16-byte aligned too
      load4f(sp, f);
      *reinterpret_cast<float4*>(o) = make_float4(f[0], f[1], f[2], f[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (d0 + e < D) o[e] = f[e] = to_f(sp[e]);
    }
  }
  if (!keys) return;
  TT hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (TT)f[e];
    lo[e] = (TT)(f[e] - (float)hi[e]);
  }
  TT* head = split + (size_t)bh * ksplit_head_elems(M, DP);
  constexpr int SROW = DP + 8;  // ksplit_row(DP)
  *reinterpret_cast<uint2*>(head + (size_t)m * SROW + d0) = *reinterpret_cast<const uint2*>(hi);
  *reinterpret_cast<uint2*>(head + ((size_t)Mp + m) * SROW + d0) = *reinterpret_cast<const uint2*>(lo);
}

template <typename T>
__global__ void from_state4_kernel(SlotConv<const float*, T*> c0, SlotConv<const float*, T*> c1, int H, int M,
                                   int D, int total4) {
  const SlotConv<const float*, T*>& c = blockIdx.y == 0 ? c0 : c1;
  const int D4 = (D + 3) >> 2;
  for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < total4; q += gridDim.x * blockDim.x) {
    const int row = q / D4, d0 = (q - row * D4) * 4;
    const int bh = row / M, m = row - bh * M, b = bh / H, h = bh - b * H;
    const float* sp = c.src + (int64_t)row * D + d0;
    T* o = c.dst + b * c.sb + h * c.sh + (int64_t)m * c.sm + d0;
    if (d0 + 4 <= D) {
      const float4 v = (D & 3) == 0 ? *reinterpret_cast<const float4*>(sp) : make_float4(sp[0], sp[1], sp[2], sp[3]);
      o[0] = from_f<T>(v.x); o[1] = from_f<T>(v.y); o[2] = from_f<T>(v.z); o[3] = from_f<T>(v.w);
    } else {
      for (int e = 0; d0 + e < D; ++e) o[e] = from_f<T>(sp[e]);
    }
  }
}

template <typename T>
__global__ void from_state_kernel(SlotConv<const float*, T*> c0, SlotConv<const float*, T*> c1, int B, int H,
                                  int M, int D) {
  const SlotConv<const float*, T*>& c = blockIdx.y == 0 ? c0 : c1;
  const int64_t total = (int64_t)B * H * M * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    int64_t r = i / D;
    const int m = (int)(r % M);
    r /= M;
    const int h = (int)(r % H);
    const int b = (int)(r / H);
    c.dst[b * c.sb + h * c.sh + m * c.sm + d] = from_f<T>(c.src[i]);
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
// walks one (b,h,d) column keeping the neighbours it has overwritten.  The
// forward passes the same tensor as x and out, so neither is __restrict__.
template <typename T>
__global__ void stencil_kernel(T* x, int64_t sb, int64_t sh, int64_t sm, T* out,
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

// Slots per block of the token-chunk path: 32 dims per thread, at most 1024
// threads, slot groups of equal size (multiples of 64).
int part_slots(int DP, int M, int nvec) {
  const int maxs = 1024 / (nvec * (DP / 32));
  const int Mp = (M + 63) & ~63;
  const int nsg = (Mp + maxs - 1) / maxs;
  return (((Mp + nsg - 1) / nsg) + 63) & ~63;
}

template <typename T, int DP>
size_t part_lds_bytes(int MS, int mode, int nvec) {
  return (size_t)nvec * SUB * (DP + 8) * sizeof(T) + SUB * 16 + (size_t)SUB * CW * 4 * (mode == SEG_ATTBWD ? 2 : 1) +
         (SUB / 64) * (size_t)MS * 8 + (size_t)SUB * MS;
}

template <typename T, int DP, int MODE>
hipError_t launch_part(const SegParams& p, const PartParams& pp, int nvec, int MS, size_t lds, int stage,
                       hipStream_t st) {
  const int BH = p.B * p.H;
  if (stage == 0) {
    const void* fn = reinterpret_cast<const void*>(&seg_partial_kernel<T, DP, MODE>);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const int nsg = (p.M + MS - 1) / MS;
    dim3 grid(XCDS * ((BH + XCDS - 1) / XCDS) * pp.nchunk * nsg);
    const int threads = MS * nvec * (DP / 32);
    MURM_LAUNCH((seg_partial_kernel<T, DP, MODE>), grid, dim3(threads), lds, st, p, pp);
  } else {
    const int G = (p.M + GS - 1) / GS;
    const int blocks = XCDS * ((BH + XCDS - 1) / XCDS) * G;
    MURM_LAUNCH((seg_reduce_kernel<DP, MODE>), dim3(blocks), dim3(red_threads(pp.nchunk, DP, MODE, p, blocks)), 0,
                       st, p, pp);
  }
  return hipGetLastError();
}

template <typename T, int DP>
bool part_ok(const SegParams& p, int mode, const PartParams* pp, int& nvec, int& MS, size_t& lds) {
  nvec = (mode == SEG_UPDATE && p.b_same_as_a) ? 1 : 2;
  MS = part_slots(DP, p.M, nvec);
  lds = part_lds_bytes<T, DP>(MS, mode, nvec);
  while (lds > 160 * 1024 && MS > 64) {  // fp32 rows at d = 128: smaller slot groups
    MS -= 64;
    lds = part_lds_bytes<T, DP>(MS, mode, nvec);
  }
  return pp && pp->nchunk > 0 && lds <= 160 * 1024;
}

// Tokens per sub-chunk of the MFMA kernel: 64 halves the barrier rounds of
// 32 (and the sub-chunk's staging latency per token) within the LDS budget.
constexpr int MSUBT = 64;

// stage 1 of every token-chunk path: chunk sums in chunk order + epilogue
template <int DP>
hipError_t launch_reduce(int mode, const SegParams& p, const PartParams& pp, hipStream_t st) {
  const int BH = p.B * p.H;
  const int G = (p.M + GS - 1) / GS;
  const dim3 grid(XCDS * ((BH + XCDS - 1) / XCDS) * G);
  if (mode == SEG_ATTBWD)
    MURM_LAUNCH((seg_reduce_kernel<DP, SEG_ATTBWD>), grid, dim3(red_threads(pp.nchunk, DP, SEG_ATTBWD, p, grid.x)), 0,
                st, p, pp);
  else
    MURM_LAUNCH((seg_reduce_kernel<DP, SEG_UPDATE>), grid, dim3(red_threads(pp.nchunk, DP, SEG_UPDATE, p, grid.x)), 0,
                st, p, pp);
  return hipGetLastError();
}

template <typename T, int DP, int MODE, int NV, int TG>
hipError_t launch_mma(const SegParams& p, const PartParams& pp, int stage, hipStream_t st) {
  using Sh = MmaShape<DP, MODE, NV, MSUBT, TG>;
  const int BH = p.B * p.H;
  if (stage != 0) return launch_reduce<DP>(MODE, p, pp, st);
  const void* fn = reinterpret_cast<const void*>(&seg_mma_kernel<T, DP, MODE, NV, MSUBT, TG>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)Sh::LDS);
  if (e != hipSuccess) return e;
  const int nsg = (p.M + Sh::MS - 1) / Sh::MS;
  dim3 grid(XCDS * ((BH + XCDS - 1) / XCDS) * pp.nchunk * nsg);
  MURM_LAUNCH((seg_mma_kernel<T, DP, MODE, NV, MSUBT, TG>), grid, dim3(Sh::THREADS), Sh::LDS, st, p, pp);
  return hipGetLastError();
}

// stage 0: the partial-sum kernel; stage 1: the chunk reduction with the epilogue.
template <typename T, int DP>
hipError_t launch_seg_t(const SegParams& p, int mode, const PartParams* pp, int stage, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (!pp || pp->nchunk <= 0 || pp->chunk_tokens % MSUBT != 0) return hipErrorInvalidValue;
    // the MFMA kernels address token rows with 32-bit row numbers and strides
    if ((uint64_t)p.va.sn >= (uint64_t(1) << 32) || (uint64_t)p.vb.sn >= (uint64_t(1) << 32)) return hipErrorInvalidValue;
    if (mode == SEG_ATTBWD) return launch_mma<T, DP, SEG_ATTBWD, 2, 1>(p, *pp, stage, st);
    // Update with one vector: blocks of two token groups over pairs of the
    // carved chunks (same waves per CU, half the partials to write and add).
    // Both stages see the paired chunking.
    if (p.b_same_as_a) {
      PartParams q = *pp;
      q.nchunk = (pp->nchunk + 1) / 2;
      q.chunk_tokens = pp->chunk_tokens * 2;
      return launch_mma<T, DP, SEG_UPDATE, 1, 2>(p, q, stage, st);
    }
    return launch_mma<T, DP, SEG_UPDATE, 2, 1>(p, *pp, stage, st);
  } else {
    int nvec, MS;
    size_t lds;
    if (part_ok<T, DP>(p, mode, pp, nvec, MS, lds)) {
      if (mode == SEG_UPDATE) return launch_part<T, DP, SEG_UPDATE>(p, *pp, nvec, MS, lds, stage, st);
      return launch_part<T, DP, SEG_ATTBWD>(p, *pp, nvec, MS, lds, stage, st);
    }
    return hipErrorInvalidValue;  // no chunk scratch carved
  }
}

inline int grid1d(int64_t n, int tpb = 256) {
  int64_t g = (n + tpb - 1) / tpb;
  return (int)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

}  // namespace

bool seg_two_stage(int dtype, int DP, int mode, const SegParams& p, const PartParams* pp) {
  (void)dtype; (void)DP; (void)mode; (void)p;
  return pp && pp->nchunk > 0;  // every served shape fits the token-chunk kernels
}

int seg_chunks(int B, int H, int N, int M, int D, int mode) {
  // token-chunk path, whole sub-chunks, at most NCMAX per (b,h): about 512
  // (b,h,chunk,slot group) blocks for the update (a 16-bit update block holds
  // 16384/d slots; with one vector the launcher pairs the chunks into blocks
  // of two token groups), about 256 (b,h,chunk) for the attend backward (at
  // d <= 64 two 128-slot groups per (b,h,chunk), two blocks per CU: 512)
  if (D > 128 || M < 1) return 0;
  const int BH = B * H;
  const int per = (N + SUB - 1) / SUB;
  const int DP = D <= 32 ? 32 : (D <= 64 ? 64 : 128);
  const int nsg = (M + 16384 / DP - 1) / (16384 / DP);
  const int target = mode == SEG_UPDATE ? (512 + nsg - 1) / nsg : 256;
  int c = (target + BH - 1) / BH;
  if (c > NCMAX) c = NCMAX;
  return c < 1 ? 1 : (c > per ? per : c);
}

int seg_chunk_tokens(int N, int nchunk) {
  const int sub = (N + SUB - 1) / SUB;
  return ((sub + nchunk - 1) / nchunk) * SUB;
}

hipError_t launch_seg(int dtype, int DP, int mode, const SegParams& p, const PartParams* pp, int stage,
                      hipStream_t st) {
#define MURM_SEG(T)                                                  \
  switch (DP) {                                                      \
    case 32: return launch_seg_t<T, 32>(p, mode, pp, stage, st);     \
    case 64: return launch_seg_t<T, 64>(p, mode, pp, stage, st);     \
    case 128: return launch_seg_t<T, 128>(p, mode, pp, stage, st);   \
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
  MURM_LAUNCH(du_kernel, dim3((p.M + 3) / 4, p.B * p.H), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T>
bool rows_vec4(const SlotConv<const T*, float*>& c, int D) {
  return (D & 3) == 0 && c.sb % 4 == 0 && c.sh % 4 == 0 && c.sm % 4 == 0 &&
         reinterpret_cast<uintptr_t>(c.src) % (4 * sizeof(T)) == 0;
}

template <typename T, typename TT>
hipError_t launch_split_t(const SlotConv<const T*, float*>& a, const SlotConv<const T*, float*>& b, bool has_b,
                          const KeySplitOut& ks, int B, int H, int M, int D, hipStream_t st) {
  const int64_t BH = (int64_t)B * H;
  const int rpb = 256 / (ks.DP / 4), nrb = (ksplit_mp(M) + rpb - 1) / rpb;
  if (BH * nrb >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(BH * nrb), 1, has_b ? 2 : 1);
  const int vk = rows_vec4(a, D), vv = has_b && rows_vec4(b, D);
  TT* sp = static_cast<TT*>(ks.p);
  switch (ks.DP) {
    case 32: MURM_LAUNCH((to_state_split_kernel<T, TT, 32>), grid, dim3(256), 0, st, a, b, sp, H, M, D, nrb, vk, vv); break;
    case 64: MURM_LAUNCH((to_state_split_kernel<T, TT, 64>), grid, dim3(256), 0, st, a, b, sp, H, M, D, nrb, vk, vv); break;
    case 128: MURM_LAUNCH((to_state_split_kernel<T, TT, 128>), grid, dim3(256), 0, st, a, b, sp, H, M, D, nrb, vk, vv); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_to_state2(int dtype, const SlotConv<const void*, float*>& a,
                            const SlotConv<const void*, float*>* bp, int B, int H, int M, int D, hipStream_t st,
                            const KeySplitOut* split) {
  const SlotConv<const void*, float*> bb = bp ? *bp : a;
  auto cv = [](const SlotConv<const void*, float*>& c, auto* tag) {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(tag)>>;
    return SlotConv<const T*, float*>{static_cast<const T*>(c.src), c.sb, c.sh, c.sm, c.dst};
  };
  if (split && split->p) {
    auto go = [&](auto* tag) -> hipError_t {
      using T = std::remove_const_t<std::remove_pointer_t<decltype(tag)>>;
      const auto ca = cv(a, (const T*)nullptr), cb = cv(bb, (const T*)nullptr);
      if (split->dtype == DT_BF16) return launch_split_t<T, __bf16>(ca, cb, bp != nullptr, *split, B, H, M, D, st);
      if (split->dtype == DT_F16) return launch_split_t<T, _Float16>(ca, cb, bp != nullptr, *split, B, H, M, D, st);
      return hipErrorInvalidValue;
    };
    switch (dtype) {
      case DT_BF16: return go((const __bf16*)nullptr);
      case DT_F16: return go((const _Float16*)nullptr);
      case DT_F32: return go((const float*)nullptr);
      default: return hipErrorInvalidValue;
    }
  }
  const int64_t total4 = (int64_t)B * H * M * ((D + 3) / 4);
  if (total4 < (int64_t(1) << 30)) {  // 32-bit indices, grid-stride step included
    const dim3 g4(grid1d(total4), bp ? 2 : 1);
    switch (dtype) {
      case DT_BF16: MURM_LAUNCH((to_state4_kernel<__bf16>), g4, dim3(256), 0, st,
                                       cv(a, (const __bf16*)nullptr), cv(bb, (const __bf16*)nullptr), H, M, D,
                                       (int)total4); break;
      case DT_F16: MURM_LAUNCH((to_state4_kernel<_Float16>), g4, dim3(256), 0, st,
                                      cv(a, (const _Float16*)nullptr), cv(bb, (const _Float16*)nullptr), H, M, D,
                                      (int)total4); break;
      case DT_F32: MURM_LAUNCH((to_state4_kernel<float>), g4, dim3(256), 0, st,
                                      cv(a, (const float*)nullptr), cv(bb, (const float*)nullptr), H, M, D,
                                      (int)total4); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 grid(grid1d((int64_t)B * H * M * D), bp ? 2 : 1);
  switch (dtype) {
    case DT_BF16: MURM_LAUNCH((to_state_kernel<__bf16>), grid, dim3(256), 0, st,
                                     cv(a, (const __bf16*)nullptr), cv(bb, (const __bf16*)nullptr), B, H, M, D); break;
    case DT_F16: MURM_LAUNCH((to_state_kernel<_Float16>), grid, dim3(256), 0, st,
                                    cv(a, (const _Float16*)nullptr), cv(bb, (const _Float16*)nullptr), B, H, M, D);
      break;
    case DT_F32: MURM_LAUNCH((to_state_kernel<float>), grid, dim3(256), 0, st,
                                    cv(a, (const float*)nullptr), cv(bb, (const float*)nullptr), B, H, M, D); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_from_state2(int dtype, const SlotConv<const float*, void*>& a,
                              const SlotConv<const float*, void*>* bp, int B, int H, int M, int D, hipStream_t st) {
  const SlotConv<const float*, void*> bb = bp ? *bp : a;
  auto cv = [](const SlotConv<const float*, void*>& c, auto* tag) {
    using T = std::remove_pointer_t<decltype(tag)>;
    return SlotConv<const float*, T*>{c.src, c.sb, c.sh, c.sm, static_cast<T*>(c.dst)};
  };
  const int64_t total4 = (int64_t)B * H * M * ((D + 3) / 4);
  if (total4 < (int64_t(1) << 30)) {  // 32-bit indices, grid-stride step included
    const dim3 g4(grid1d(total4), bp ? 2 : 1);
    switch (dtype) {
      case DT_BF16: MURM_LAUNCH((from_state4_kernel<__bf16>), g4, dim3(256), 0, st,
                                       cv(a, (__bf16*)nullptr), cv(bb, (__bf16*)nullptr), H, M, D, (int)total4); break;
      case DT_F16: MURM_LAUNCH((from_state4_kernel<_Float16>), g4, dim3(256), 0, st,
                                      cv(a, (_Float16*)nullptr), cv(bb, (_Float16*)nullptr), H, M, D, (int)total4);
        break;
      case DT_F32: MURM_LAUNCH((from_state4_kernel<float>), g4, dim3(256), 0, st,
                                      cv(a, (float*)nullptr), cv(bb, (float*)nullptr), H, M, D, (int)total4); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 grid(grid1d((int64_t)B * H * M * D), bp ? 2 : 1);
  switch (dtype) {
    case DT_BF16: MURM_LAUNCH((from_state_kernel<__bf16>), grid, dim3(256), 0, st,
                                     cv(a, (__bf16*)nullptr), cv(bb, (__bf16*)nullptr), B, H, M, D); break;
    case DT_F16: MURM_LAUNCH((from_state_kernel<_Float16>), grid, dim3(256), 0, st,
                                    cv(a, (_Float16*)nullptr), cv(bb, (_Float16*)nullptr), B, H, M, D); break;
    case DT_F32: MURM_LAUNCH((from_state_kernel<float>), grid, dim3(256), 0, st,
                                    cv(a, (float*)nullptr), cv(bb, (float*)nullptr), B, H, M, D); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_to_state(int dtype, const void* src, int64_t sb, int64_t sh, int64_t sm, float* dst,
                           int B, int H, int M, int D, hipStream_t st) {
  return launch_to_state2(dtype, {src, sb, sh, sm, dst}, nullptr, B, H, M, D, st);
}

hipError_t launch_from_state(int dtype, const float* src, void* dst, int64_t sb, int64_t sh, int64_t sm,
                             int B, int H, int M, int D, hipStream_t st) {
  return launch_from_state2(dtype, {src, sb, sh, sm, dst}, nullptr, B, H, M, D, st);
}

hipError_t launch_idx_pack(const int64_t* src, uint16_t* dst, int64_t rows, int K, int M, hipStream_t st) {
  MURM_LAUNCH(idx_pack_kernel, dim3(grid1d(rows)), dim3(256), 0, st, src, dst, rows, K, M);
  return hipGetLastError();
}

hipError_t launch_stencil(int dtype, void* x, int64_t sb, int64_t sh, int64_t sm, void* out, int64_t ob,
                          int64_t oh, int64_t om, int B, int H, int M, int D, float g, int adjoint,
                          hipStream_t st) {
  const int64_t cols = (int64_t)B * H * D;
  const int grid = (int)((cols + 255) / 256);
  switch (dtype) {
    case DT_BF16: MURM_LAUNCH((stencil_kernel<__bf16>), dim3(grid), dim3(256), 0, st, (__bf16*)x,
                                     sb, sh, sm, (__bf16*)out, ob, oh, om, B, H, M, D, g, adjoint); break;
    case DT_F16: MURM_LAUNCH((stencil_kernel<_Float16>), dim3(grid), dim3(256), 0, st, (_Float16*)x,
                                    sb, sh, sm, (_Float16*)out, ob, oh, om, B, H, M, D, g, adjoint); break;
    case DT_F32: MURM_LAUNCH((stencil_kernel<float>), dim3(grid), dim3(256), 0, st, (float*)x,
                                    sb, sh, sm, (float*)out, ob, oh, om, B, H, M, D, g, adjoint); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace murm
