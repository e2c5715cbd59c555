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

#include <initializer_list>
#include <type_traits>

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
  for (int j = 0; j < KN; ++j) dw[j] = group_sum<DCH>(dw[j]);
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

// ---------------------------------------------------------------------------
// Staged variants: one block per (b,h) and token chunk stages the round's
// float32 slot tables in LDS (row stride table_stride), so the per-token gathers of
// seven slot rows are LDS reads instead of L2 traffic.  Used when the tables
// fit (e.g. M = 256, d = 64: 64 KiB per table).
// ---------------------------------------------------------------------------
constexpr int TOKS_THREADS = 512;

template <int DP, int NT = TOKS_THREADS>
struct TokShape {
  static constexpr int DCH = DP / 8;                   // lanes per token
  static constexpr int TPP = NT / DCH;                 // tokens per pass (NT threads)
  static constexpr int RSD = table_stride<DP>();       // staged row stride
};

template <typename T, int DP, int NP, bool HV, bool WIDE, bool SEQ, int NT = TOKS_THREADS>
__global__ __launch_bounds__(NT) void tok_bwd_lds_kernel(TokBwdParams p, int nchunk) {
  using S = TokShape<DP, NT>;
  constexpr int DCH = S::DCH, TPP = S::TPP, RSD = S::RSD;
  extern __shared__ __align__(16) unsigned char smem[];
  int bh, chunk;
  if (!tok_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  const bool has_g = p.sv != nullptr, has_k = p.dkk != nullptr;
  const int dc = threadIdx.x % DCH, sw = tok_swap<DP>();
  const int c_beg = chunk * NP * TPP;
  // every global load of the block is issued first: index rows, token rows
  // and (lane dc < 7) weight j = dc of each of the NP passes, then the tables
  constexpr int JPL = (KN + DCH - 1) / DCH;  // weights finished per lane
  uint4 ix[NP];
  Raw8<T> rg[NP], rk[NP], rv[HV ? NP : 1];
  float wq[NP][JPL], gq[NP][JPL];
  // token rows are loaded unconditionally (an absent view reads a present
  // one and is ignored): a load under the same condition as its use would be
  // merged with the conversion and waited for at once
  const TokView& vg = p.g.p ? p.g : p.tk;
  const TokView& vk = p.tk.p ? p.tk : p.g;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int n = min(c_beg + q * TPP + (int)threadIdx.x / DCH, p.N - 1);
    const int64_t row = (int64_t)bh * p.N + n;
    ix[q] = *reinterpret_cast<const uint4*>(p.idx + row * IDX_ROW);
    rg[q] = raw8s<T, WIDE, DP>(tok_row<T>(vg, b, h, n), dc, sw, p.D);
    rk[q] = raw8s<T, WIDE, DP>(tok_row<T>(vk, b, h, n), dc, sw, p.D);
    if constexpr (HV) rv[q] = raw8s<T, WIDE, DP>(tok_row<T>(p.tv, b, h, n), dc, sw, p.D);
#pragma unroll
    for (int u = 0; u < JPL; ++u) {
      const int j = dc + u * DCH;
      wq[q][u] = j < KN ? p.w[row * KN + j] : 0.f;
      gq[q][u] = (p.gw && j < KN) ? p.gw[row * KN + j] : 0.f;
    }
  }
  float* tsv = reinterpret_cast<float*>(smem);
  float* tdk = tsv + (has_g ? p.M * RSD : 0);
  float* tdv = tdk + (has_k ? p.M * RSD : 0);
  float* tdw = SEQ ? tsv + p.M * RSD : tdv + (HV ? p.M * RSD : 0);
  const int64_t tb = (int64_t)bh * p.M * p.D;
  auto slots = [&](int q, uint32_t (&sl)[KN]) {
    const uint4 ir = ix[q];
    sl[0] = ir.x & 0xFFFF; sl[1] = ir.x >> 16; sl[2] = ir.y & 0xFFFF; sl[3] = ir.y >> 16;
    sl[4] = ir.z & 0xFFFF; sl[5] = ir.z >> 16; sl[6] = ir.w & 0xFFFF;
  };
  // dw_j of pass q from the tables flagged (sums over the token's lanes)
  auto dots = [&](int q, const uint32_t (&sl)[KN], float (&dw)[KN], const float* ts, const float* tk,
                  const float* tv, auto g_c, auto k_c, auto v_c) {
    constexpr bool HG = decltype(g_c)::value, HK = decltype(k_c)::value, HVV = decltype(v_c)::value;
    float g[8], a[8], c[8];
    if constexpr (HG) unraw8s<T, DP>(rg[q], g, dc, sw, p.D);
    if constexpr (HK) unraw8s<T, DP>(rk[q], a, dc, sw, p.D);
    if constexpr (HVV) unraw8s<T, DP>(rv[q], c, dc, sw, p.D);
    // rows of slot j + 1 are read while slot j's are used; the scheduling
    // barrier keeps the compiler from reading further ahead
    float vs[2][8], vk[2][8], vv[2][8];
    auto rows = [&](int j, int o) {
      if constexpr (HG) lds8s<DP>(ts + sl[j] * RSD, dc, sw, vs[o]);
      if constexpr (HK) lds8s<DP>(tk + sl[j] * RSD, dc, sw, vk[o]);
      if constexpr (HVV) lds8s<DP>(tv + sl[j] * RSD, dc, sw, vv[o]);
    };
    rows(0, 0);
#pragma unroll
    for (int j = 0; j < KN; ++j) {
      const int o = j & 1;
      if (j + 1 < KN) rows(j + 1, o ^ 1);
      float sacc = 0.f;
      if constexpr (HG) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sacc += g[i] * vs[o][i];
      }
      if constexpr (HK) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sacc += a[i] * vk[o][i];
      }
      if constexpr (HVV) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sacc += c[i] * vv[o][i];
      }
      dw[j] = group_sum<DCH>(sacc);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // lane dc finishes weights j = dc, dc + DCH, ... of pass q
  auto finish = [&](int q, const uint32_t (&sl)[KN], const float (&dw)[KN]) {
    const int n = c_beg + q * TPP + threadIdx.x / DCH;
    float mine[JPL];
    float part = 0.f;
#pragma unroll
    for (int u = 0; u < JPL; ++u) {
      const int jj = dc + u * DCH;
      float m = dw[0];
      uint32_t ms = sl[0];
#pragma unroll
      for (int j = 1; j < KN; ++j) {
        m = jj == j ? dw[j] : m;
        ms = jj == j ? sl[j] : ms;
      }
      if (p.dW) m += tdw[ms];
      m += gq[q][u];
      mine[u] = m;
      part += jj < KN ? wq[q][u] * m : 0.f;
    }
    const int64_t row = (int64_t)bh * p.N + n;
    const float dot = p.ds_out ? group_sum<DCH>(part) : 0.f;
#pragma unroll
    for (int u = 0; u < JPL; ++u) {
      const int jj = dc + u * DCH;
      if (jj >= KN || n >= p.N) continue;
      if (p.dw_out) p.dw_out[row * KN + jj] = mine[u];
      if (p.ds_out) p.ds_out[row * KN + jj] = wq[q][u] * (mine[u] - dot);
    }
  };
  using Y = std::true_type;
  using N_ = std::false_type;
  if constexpr (!SEQ) {
    if (has_g) stage_table<DP>(tsv, p.sv + tb, p.M, p.D);
    if (has_k) stage_table<DP>(tdk, p.dkk + tb, p.M, p.D);
    if constexpr (HV) stage_table<DP>(tdv, p.dkv + tb, p.M, p.D);
    if (p.dW)
      for (int i = threadIdx.x; i < p.M; i += blockDim.x) tdw[i] = p.dW[(int64_t)bh * p.M + i];
    __syncthreads();
    // the passes, specialised on which tables are present
    auto passes = [&](auto g_c, auto k_c) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        uint32_t sl[KN];
        slots(q, sl);
        float dw[KN];
        dots(q, sl, dw, tsv, tdk, tdv, g_c, k_c, std::integral_constant<bool, HV>{});
        finish(q, sl, dw);
      }
    };
    if (has_g) { if (has_k) passes(Y{}, Y{}); else passes(Y{}, N_{}); }
    else { if (has_k) passes(N_{}, Y{}); else passes(N_{}, N_{}); }
  } else {
    // the tables do not fit together: one at a time in one LDS table, each
    // table's dot products added to dw per pass, then the weights finished
    float* t0 = tsv;
    if (p.dW)  // after the one table
      for (int i = threadIdx.x; i < p.M; i += blockDim.x) tdw[i] = p.dW[(int64_t)bh * p.M + i];
    float dwp[NP][KN];
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
      for (int j = 0; j < KN; ++j) dwp[q][j] = 0.f;
    auto pass_all = [&](auto g_c, auto k_c, auto v_c) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        uint32_t sl[KN];
        slots(q, sl);
        float dw[KN];
        dots(q, sl, dw, t0, t0, t0, g_c, k_c, v_c);
#pragma unroll
        for (int j = 0; j < KN; ++j) dwp[q][j] += dw[j];
      }
    };
    if (has_g) {
      stage_table<DP>(t0, p.sv + tb, p.M, p.D);
      __syncthreads();
      pass_all(Y{}, N_{}, N_{});
      __syncthreads();
    }
    if (has_k) {
      stage_table<DP>(t0, p.dkk + tb, p.M, p.D);
      __syncthreads();
      pass_all(N_{}, Y{}, N_{});
      __syncthreads();
    }
    if constexpr (HV) {
      stage_table<DP>(t0, p.dkv + tb, p.M, p.D);
      __syncthreads();
      pass_all(N_{}, N_{}, Y{});
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      uint32_t sl[KN];
      slots(q, sl);
      finish(q, sl, dwp[q]);
    }
  }
}

// tok_bwd with the tables staged one at a time (they do not fit together)
// for blocks of many passes: a table phase keeps one pass's token and index
// rows in flight ahead, and every (token, j) partial dw lives in LDS beside
// the table ([NP][TPP][7] floats), so a block stages each table once for NP
// passes of tokens.  Tables g.sv then tk.dKk (the form without token-value
// rows); dw is the sum of the two tables' dot products, as in the staged
// kernel's one-table-at-a-time form.
template <typename T, int DP, int NP, bool WIDE>
__global__ __launch_bounds__(TOKS_THREADS) void tok_bwd_seq_kernel(TokBwdParams p, int nchunk) {
  using S = TokShape<DP>;
  constexpr int DCH = S::DCH, TPP = S::TPP, RSD = S::RSD;
  constexpr int JPL = (KN + DCH - 1) / DCH;  // weights finished per lane
  extern __shared__ __align__(16) unsigned char smem[];
  int bh, chunk;
  if (!tok_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  const int dc = threadIdx.x % DCH, sw = tok_swap<DP>();
  const int tl = threadIdx.x / DCH;  // token of a pass
  const int c_beg = chunk * NP * TPP;
  float* tab = reinterpret_cast<float*>(smem);
  float* tdw = tab + p.M * RSD;              // dW [M]
  float* dwb = tdw + ((p.M + 3) & ~3);       // partial dw [NP][TPP][KN]
  const int64_t tb = (int64_t)bh * p.M * p.D;
  if (p.dW)
    for (int i = threadIdx.x; i < p.M; i += blockDim.x) tdw[i] = p.dW[(int64_t)bh * p.M + i];
  const int nph = (p.sv ? 1 : 0) + (p.dkk ? 1 : 0);
  for (int ph = 0; ph < nph; ++ph) {
    const bool is_sv = p.sv && ph == 0;
    const TokView& tv = is_sv ? p.g : p.tk;
    // index and token rows PF passes ahead: the first PF in flight while the
    // table is staged, pass q + PF requested as pass q starts
    constexpr int PF = NP < 8 ? NP : 8;
    uint4 ix[NP];
    Raw8<T> rx[NP];
    auto fetch = [&](int q) {
      const int n = min(c_beg + q * TPP + tl, p.N - 1);
      ix[q] = *reinterpret_cast<const uint4*>(p.idx + ((int64_t)bh * p.N + n) * IDX_ROW);
      rx[q] = raw8s<T, WIDE, DP>(tok_row<T>(tv, b, h, n), dc, sw, p.D);
    };
#pragma unroll
    for (int q = 0; q < PF; ++q) fetch(q);
    if (ph > 0) __syncthreads();  // the previous table is no longer read
    stage_table<DP>(tab, (is_sv ? p.sv : p.dkk) + tb, p.M, p.D);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      if (q + PF < NP) fetch(q + PF);
      const uint4 ir = ix[q];
      float x[8];
      unraw8s<T, DP>(rx[q], x, dc, sw, p.D);
      // rows of slot j + 1 are read while slot j's are used
      float v[2][8];
      auto rows = [&](int j, int o) { lds8s<DP>(tab + idx_at(ir, j) * RSD, dc, sw, v[o]); };
      rows(0, 0);
      float* slot = dwb + (q * TPP + tl) * KN;
#pragma unroll
      for (int j = 0; j < KN; ++j) {
        const int o = j & 1;
        if (j + 1 < KN) rows(j + 1, o ^ 1);
        float sacc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sacc += x[i] * v[o][i];
        const float dw = group_sum<DCH>(sacc);
        if (j % DCH == dc) slot[j] = ph == 0 ? dw : slot[j] + dw;
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  __syncthreads();
  // lane dc finishes weights j = dc, dc + DCH, ... of each pass; every
  // pass's index row, weights and weight grads requested at once
  uint4 fi[NP];
  float fw[NP][JPL], fg[NP][JPL];
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int n = min(c_beg + q * TPP + tl, p.N - 1);
    const int64_t row = (int64_t)bh * p.N + n;
    fi[q] = *reinterpret_cast<const uint4*>(p.idx + row * IDX_ROW);
#pragma unroll
    for (int u = 0; u < JPL; ++u) {
      const int j = dc + u * DCH;
      fw[q][u] = j < KN ? p.w[row * KN + j] : 0.f;
      fg[q][u] = (p.gw && j < KN) ? p.gw[row * KN + j] : 0.f;
    }
  }
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const uint4 ir = fi[q];
    const float* wq = fw[q];
    const float* gq = fg[q];
    const int n = c_beg + q * TPP + tl;
    const float* slot = dwb + (q * TPP + tl) * KN;
    float mine[JPL];
    float part = 0.f;
#pragma unroll
    for (int u = 0; u < JPL; ++u) {
      const int jj = dc + u * DCH;
      float m = 0.f;
      if (jj < KN) {
        m = nph > 0 ? slot[jj] : 0.f;
        if (p.dW) m += tdw[idx_at(ir, jj)];
        m += gq[u];
      }
      mine[u] = m;
      part += jj < KN ? wq[u] * m : 0.f;
    }
    const float dot = p.ds_out ? group_sum<DCH>(part) : 0.f;
    const int64_t row = (int64_t)bh * p.N + n;
#pragma unroll
    for (int u = 0; u < JPL; ++u) {
      const int jj = dc + u * DCH;
      if (jj >= KN || n >= p.N) continue;
      if (p.dw_out) p.dw_out[row * KN + jj] = mine[u];
      if (p.ds_out) p.ds_out[row * KN + jj] = wq[u] * (mine[u] - dot);
    }
  }
}

// tok_grad with each round's tables staged in LDS in turn; a thread keeps the
// gradients of its PASSES tokens in registers across the rounds.
template <typename T, int DP, int PASSES, bool KV, bool WIDE, bool SEQ>
__global__ __launch_bounds__(TOKS_THREADS) void tok_grad_lds_kernel(TokGradParams p, int nchunk) {
  constexpr bool seq = SEQ;
  using S = TokShape<DP>;
  constexpr int DCH = S::DCH, TPP = S::TPP, RSD = S::RSD;
  extern __shared__ __align__(16) unsigned char smem[];
  int bh, chunk;
  if (!tok_block(p.B * p.H, nchunk, bh, chunk)) return;
  const int b = bh / p.H, h = bh % p.H;
  float* t0 = reinterpret_cast<float*>(smem);
  const int64_t tb = (int64_t)bh * p.M * p.D;
  const int dc = threadIdx.x % DCH, sw = tok_swap<DP>();
  const int c_beg = chunk * PASSES * TPP;
  constexpr int PK = KV ? PASSES : 1;  // token-key / token-value gradients (legacy form only)
  float aq[PASSES][8], ak[PK][8], av[PK][8];
  if (p.g.p) {  // every pass's residual row in flight before any is converted
    Raw8<T> rg[PASSES];
#pragma unroll
    for (int q = 0; q < PASSES; ++q)
      rg[q] = raw8s<T, WIDE, DP>(tok_row<T>(p.g, b, h, min(c_beg + q * TPP + (int)threadIdx.x / DCH, p.N - 1)), dc, sw, p.D);
#pragma unroll
    for (int q = 0; q < PASSES; ++q)
      unraw8s<T, DP>(rg[q], aq[q], dc, sw, p.D, c_beg + q * TPP + (int)threadIdx.x / DCH < p.N);
  } else {
#pragma unroll
    for (int q = 0; q < PASSES; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i) aq[q][i] = 0.f;
  }
#pragma unroll
  for (int q = 0; q < PK; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) { ak[q][i] = 0.f; av[q][i] = 0.f; }
  // next pass's index row (raw), weights and softmax grads, requested before
  // the current pass's gathers
  uint4 irn;
  float wn[KN], dn[KN];
  for (int r = 0; r < p.R; ++r) {
    const uint16_t* idx_r = p.idx[r];
    const float* w_r = p.w[r];
    const float* ds_r = p.ds[r];
    const float* dkk_r = p.dkk[r];
    const float* dkv_r = p.dkv[r];
    const bool use_sk = ds_r && p.dq.p;
    // seq: the round's tables one at a time in one LDS table (they do not fit together)
    float* tsk = t0;
    float* tdk = seq ? t0 : tsk + (use_sk ? p.M * RSD : 0);
    float* tdv = seq ? t0 : tdk + (dkk_r ? p.M * RSD : 0);
    if (!seq) {
      if (r > 0) __syncthreads();  // the previous round's tables are no longer read
      if (use_sk) stage_table<DP>(tsk, p.sk[r] + tb, p.M, p.D);
      if (dkk_r) stage_table<DP>(tdk, dkk_r + tb, p.M, p.D);
      if (dkv_r) stage_table<DP>(tdv, dkv_r + tb, p.M, p.D);
      __syncthreads();
    }
    // the round's passes, specialised on which tables it has
    auto passes = [&](auto sk_c, auto dk_c, auto dv_c) {
      constexpr bool SK = decltype(sk_c)::value, DK = decltype(dk_c)::value, DV = decltype(dv_c)::value;
      auto fetch = [&](int q) {
        const int n = min(c_beg + q * TPP + (int)threadIdx.x / DCH, p.N - 1);
        const int64_t row = (int64_t)bh * p.N + n;
        irn = *reinterpret_cast<const uint4*>(idx_r + row * IDX_ROW);
        load_row7(w_r + row * KN, wn);
        if (SK) load_row7(ds_r + row * KN, dn);
      };
      fetch(0);
#pragma unroll
      for (int q = 0; q < PASSES; ++q) {
        const uint4 ir = irn;
        float wr[KN], dsr[KN];
#pragma unroll
        for (int j = 0; j < KN; ++j) { wr[j] = wn[j]; dsr[j] = SK ? dn[j] : 0.f; }
        if (q + 1 < PASSES) fetch(q + 1);
        const int n = c_beg + q * TPP + threadIdx.x / DCH;
        if (n >= p.N) continue;
        // rows of slot j + 1 are read while slot j's are accumulated; the
        // scheduling barrier keeps the compiler from reading further ahead
        // (all 7 slots' rows in flight would double the registers)
        float vs[2][8], vk[2][8], vv[2][8];
        auto rows = [&](int j, int o) {
          const uint32_t sl = idx_at(ir, j);
          if constexpr (SK) lds8s<DP>(tsk + sl * RSD, dc, sw, vs[o]);
          if constexpr (DK) lds8s<DP>(tdk + sl * RSD, dc, sw, vk[o]);
          if constexpr (KV && DV) lds8s<DP>(tdv + sl * RSD, dc, sw, vv[o]);
        };
        rows(0, 0);
#pragma unroll
        for (int j = 0; j < KN; ++j) {
          const int o = j & 1;
          if (j + 1 < KN) rows(j + 1, o ^ 1);
          if constexpr (SK) {
            const float cj = p.c * dsr[j];
#pragma unroll
            for (int i = 0; i < 8; ++i) aq[q][i] += cj * vs[o][i];
          }
          const float wj = wr[j];
          if constexpr (DK) {
            if constexpr (KV) {
#pragma unroll
              for (int i = 0; i < 8; ++i) ak[q][i] += wj * vk[o][i];
            } else {
#pragma unroll
              for (int i = 0; i < 8; ++i) aq[q][i] += wj * vk[o][i];
            }
          }
          if constexpr (KV && DV) {
#pragma unroll
            for (int i = 0; i < 8; ++i) av[q][i] += wj * vv[o][i];
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    using Y = std::true_type;
    using N_ = std::false_type;
    if constexpr (SEQ) {  // each present table: stage it, then its term's passes
      if (use_sk) {
        __syncthreads();
        stage_table<DP>(t0, p.sk[r] + tb, p.M, p.D);
        __syncthreads();
        passes(Y{}, N_{}, N_{});
      }
      if (dkk_r) {
        __syncthreads();
        stage_table<DP>(t0, dkk_r + tb, p.M, p.D);
        __syncthreads();
        passes(N_{}, Y{}, N_{});
      }
      if constexpr (KV) {
        if (dkv_r) {
          __syncthreads();
          stage_table<DP>(t0, dkv_r + tb, p.M, p.D);
          __syncthreads();
          passes(N_{}, N_{}, Y{});
        }
      }
      continue;
    }
    if constexpr (KV) {
      if (dkv_r) {
        if (use_sk) { if (dkk_r) passes(Y{}, Y{}, Y{}); else passes(Y{}, N_{}, Y{}); }
        else { if (dkk_r) passes(N_{}, Y{}, Y{}); else passes(N_{}, N_{}, Y{}); }
        continue;
      }
    }
    if (use_sk) { if (dkk_r) passes(Y{}, Y{}, N_{}); else passes(Y{}, N_{}, N_{}); }
    else if (dkk_r) passes(N_{}, Y{}, N_{});
  }
#pragma unroll
  for (int q = 0; q < PASSES; ++q) {
    const int n = c_beg + q * TPP + threadIdx.x / DCH;
    if (n >= p.N) continue;
    if (p.dq.p) store8s<T, DP>(tok_row_mut<T>(p.dq, b, h, n), dc, sw, p.D, p.dq.vec, aq[q]);
    if constexpr (KV) {
      if (p.dtk.p) store8s<T, DP>(tok_row_mut<T>(p.dtk, b, h, n), dc, sw, p.D, p.dtk.vec, ak[q]);
      if (p.dtv.p) store8s<T, DP>(tok_row_mut<T>(p.dtv, b, h, n), dc, sw, p.D, p.dtv.vec, av[q]);
    }
  }
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
  for (int j = 0; j < KN; ++j) s[j] = group_sum<DCH>(s[j]);
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
  MURM_LAUNCH((attend_idx_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

// staged tables fit one block's LDS (leave room for a second block's worth of nothing)
inline bool tables_fit(int nt, int M, int DP) {
  const int rsd = DP == 64 ? 64 : DP + 4;  // table_stride<DP>()
  return (size_t)nt * M * rsd * 4 + (size_t)M * 4 <= 150 * 1024;
}

// a grid of blocks of `tokens` tokens per (b,h) fills every CU (otherwise the
// launchers take blocks of fewer passes)
inline bool tok_grid_fills(int BH, int N, int tokens) {
  return TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * ((N + tokens - 1) / tokens) >= device_cus();
}

// unconditional token loads for every row the kernel reads (see raw8s)
inline bool wide_rows(std::initializer_list<const TokView*> views, int D) {
  if (D % 4 != 0) return false;
  for (const TokView* v : views)
    if (v->p && !v->vec) return false;
  return true;
}

template <typename T, int DP, int NP, bool HV, bool WIDE, bool SEQ>
hipError_t launch_tok_bwd_lds_s(const TokBwdParams& p, int nt, hipStream_t st) {
  using S = TokShape<DP>;
  const int BH = p.B * p.H;
  const int nchunk = (p.N + NP * S::TPP - 1) / (NP * S::TPP);
  const size_t lds = (size_t)(SEQ ? 1 : nt) * p.M * S::RSD * 4 + (size_t)p.M * 4;
  const void* fn = reinterpret_cast<const void*>(&tok_bwd_lds_kernel<T, DP, NP, HV, WIDE, SEQ>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk);
  MURM_LAUNCH((tok_bwd_lds_kernel<T, DP, NP, HV, WIDE, SEQ>), grid, dim3(TOKS_THREADS), lds, st, p, nchunk);
  return hipGetLastError();
}

template <typename T, int DP, int NP, bool HV, bool WIDE>
hipError_t launch_tok_bwd_lds_w(const TokBwdParams& p, int nt, hipStream_t st) {
  // tables that do not fit together are staged one at a time
  if (tables_fit(nt, p.M, DP)) return launch_tok_bwd_lds_s<T, DP, NP, HV, WIDE, false>(p, nt, st);
  return launch_tok_bwd_lds_s<T, DP, NP, HV, WIDE, true>(p, nt, st);
}

template <typename T, int DP, int NP, bool HV>
hipError_t launch_tok_bwd_lds(const TokBwdParams& p, int nt, hipStream_t st) {
  if (wide_rows({&p.g, &p.tk, &p.tv}, p.D)) return launch_tok_bwd_lds_w<T, DP, NP, HV, true>(p, nt, st);
  return launch_tok_bwd_lds_w<T, DP, NP, HV, false>(p, nt, st);
}

// LDS of tok_bwd_seq_kernel: one table, dW, the partial dw of NP passes
template <int DP>
size_t tok_bwd_seq_lds(int M, int np) {
  return (size_t)M * TokShape<DP>::RSD * 4 + (size_t)((M + 3) & ~3) * 4 + (size_t)np * TokShape<DP>::TPP * KN * 4;
}

template <typename T, int DP, int NP, bool WIDE>
hipError_t launch_tok_bwd_seq(const TokBwdParams& p, hipStream_t st) {
  const int BH = p.B * p.H;
  const int nchunk = (p.N + NP * TokShape<DP>::TPP - 1) / (NP * TokShape<DP>::TPP);
  const size_t lds = tok_bwd_seq_lds<DP>(p.M, NP);
  const void* fn = reinterpret_cast<const void*>(&tok_bwd_seq_kernel<T, DP, NP, WIDE>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk);
  MURM_LAUNCH((tok_bwd_seq_kernel<T, DP, NP, WIDE>), grid, dim3(TOKS_THREADS), lds, st, p, nchunk);
  return hipGetLastError();
}

// Blocks of 1024 threads and NP passes: the tokens and tables of a block of
// 512 threads and 2 NP passes, with 4 waves per SIMD instead of 2 to hide the
// LDS and load latency (at most 128 VGPRs; rows 16-byte aligned).
template <typename T, int DP, bool WIDE, int NP = 4>
hipError_t launch_tok_bwd_1k(const TokBwdParams& p, int nt, hipStream_t st) {
  using S = TokShape<DP, 1024>;
  const int BH = p.B * p.H;
  const int nchunk = (p.N + NP * S::TPP - 1) / (NP * S::TPP);
  const size_t lds = (size_t)nt * p.M * S::RSD * 4 + (size_t)p.M * 4;
  const void* fn = reinterpret_cast<const void*>(&tok_bwd_lds_kernel<T, DP, NP, false, WIDE, false, 1024>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk);
  MURM_LAUNCH((tok_bwd_lds_kernel<T, DP, NP, false, WIDE, false, 1024>), grid, dim3(1024), lds, st, p, nchunk);
  return hipGetLastError();
}

template <typename T, int DP>
hipError_t launch_tok_bwd_t(const TokBwdParams& p, hipStream_t st) {
  const int nt = (p.sv ? 1 : 0) + (p.dkk ? 1 : 0) + (p.dkv ? 1 : 0);
  // tables of more than half the LDS (one block per CU in any form): blocks
  // of 16 passes keep their partial dw in LDS and stage each table once for
  // twice the tokens of 8 passes
  if (nt > 0 && !p.dkv && tables_fit(1, p.M, DP) && (size_t)p.M * TokShape<DP>::RSD * 4 > 80 * 1024 &&
      tok_bwd_seq_lds<DP>(p.M, 16) <= 160 * 1024 && tok_grid_fills(p.B * p.H, p.N, 16 * TokShape<DP>::TPP)) {
    if (wide_rows({&p.g, &p.tk}, p.D)) return launch_tok_bwd_seq<T, DP, 16, true>(p, st);
    return launch_tok_bwd_seq<T, DP, 16, false>(p, st);
  }
  if (nt > 0 && tables_fit(1, p.M, DP)) {
    // tokens per lane whose loads are all in flight at once: 8 (16-bit tokens,
    // two token rows) or 4 (float32 tokens or three token rows)
    if (p.dkv) return launch_tok_bwd_lds<T, DP, 4, true>(p, nt, st);
    if (sizeof(T) == 2 && tok_grid_fills(p.B * p.H, p.N, 8 * TokShape<DP>::TPP)) {
      if (DP <= 64 && tables_fit(nt, p.M, DP) && wide_rows({&p.g, &p.tk, &p.tv}, p.D))
        return launch_tok_bwd_1k<T, DP, true>(p, nt, st);
      return launch_tok_bwd_lds<T, DP, 8, false>(p, nt, st);
    }
    if (sizeof(T) == 2 && DP <= 64 && tables_fit(nt, p.M, DP) && wide_rows({&p.g, &p.tk, &p.tv}, p.D))
      return launch_tok_bwd_1k<T, DP, true, 2>(p, nt, st);
    return launch_tok_bwd_lds<T, DP, 4, false>(p, nt, st);
  }
  constexpr int TPB = 256 / (DP / 8);
  dim3 grid((p.N + TPB - 1) / TPB, p.B * p.H);
  MURM_LAUNCH((tok_bwd_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, int DP, int PASSES, bool KV, bool WIDE, bool SEQ>
hipError_t launch_tok_grad_lds_s(const TokGradParams& p, int nt, hipStream_t st) {
  using S = TokShape<DP>;
  const int BH = p.B * p.H;
  const int nchunk = (p.N + PASSES * S::TPP - 1) / (PASSES * S::TPP);
  const size_t lds = (size_t)(SEQ ? 1 : nt) * p.M * S::RSD * 4;
  const void* fn = reinterpret_cast<const void*>(&tok_grad_lds_kernel<T, DP, PASSES, KV, WIDE, SEQ>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid(TOK_XCDS * ((BH + TOK_XCDS - 1) / TOK_XCDS) * nchunk);
  MURM_LAUNCH((tok_grad_lds_kernel<T, DP, PASSES, KV, WIDE, SEQ>), grid, dim3(TOKS_THREADS), lds, st, p, nchunk);
  return hipGetLastError();
}

template <typename T, int DP, int PASSES, bool KV, bool WIDE>
hipError_t launch_tok_grad_lds_w(const TokGradParams& p, int nt, hipStream_t st) {
  // tables that do not fit together are staged one at a time
  if (tables_fit(nt, p.M, DP)) return launch_tok_grad_lds_s<T, DP, PASSES, KV, WIDE, false>(p, nt, st);
  return launch_tok_grad_lds_s<T, DP, PASSES, KV, WIDE, true>(p, nt, st);
}

template <typename T, int DP, int PASSES, bool KV>
hipError_t launch_tok_grad_lds(const TokGradParams& p, int nt, hipStream_t st) {
  if (wide_rows({&p.g}, p.D)) return launch_tok_grad_lds_w<T, DP, PASSES, KV, true>(p, nt, st);
  return launch_tok_grad_lds_w<T, DP, PASSES, KV, false>(p, nt, st);
}

template <typename T, int DP>
hipError_t launch_tok_grad_t(const TokGradParams& p, hipStream_t st) {
  int nt = 0;  // most tables any round stages
  for (int r = 0; r < p.R; ++r) {
    const int k = ((p.ds[r] && p.dq.p) ? 1 : 0) + (p.dkk[r] ? 1 : 0) + (p.dkv[r] ? 1 : 0);
    nt = k > nt ? k : nt;
  }
  if (nt > 0 && tables_fit(1, p.M, DP)) {
    // registers: dq only (the slot-key gradient terms go to dq) keeps 8 passes
    // of tokens, with separate token-key / token-value gradients 4
    if (p.shared_kv) {
      if (tok_grid_fills(p.B * p.H, p.N, 8 * TokShape<DP>::TPP)) {
        // Two blocks per CU when two one-table blocks fit its LDS (d <= 64:
        // about 110 VGPRs at 4 passes): the tables are staged one at a time
        // and one block's staging runs beside the other's passes.
        if (DP <= 64 && 2 * (size_t)p.M * TokShape<DP>::RSD * 4 <= 160 * 1024) {
          if (wide_rows({&p.g}, p.D)) return launch_tok_grad_lds_s<T, DP, 4, false, true, true>(p, nt, st);
          return launch_tok_grad_lds_s<T, DP, 4, false, false, true>(p, nt, st);
        }
        // one table at a time (tables that do not fit together): blocks of 16
        // passes stage each table for twice the tokens, where such blocks fill the device
        if (!tables_fit(nt, p.M, DP) && tok_grid_fills(p.B * p.H, p.N, 16 * TokShape<DP>::TPP)) {
          if (wide_rows({&p.g}, p.D)) return launch_tok_grad_lds_s<T, DP, 16, false, true, true>(p, nt, st);
          return launch_tok_grad_lds_s<T, DP, 16, false, false, true>(p, nt, st);
        }
        return launch_tok_grad_lds<T, DP, 8, false>(p, nt, st);
      }
      // smaller grids: one-table blocks of 2 passes, two per CU, where they fill the device twice
      if (DP <= 64 && 2 * (size_t)p.M * TokShape<DP>::RSD * 4 <= 160 * 1024 &&
          tok_grid_fills(p.B * p.H, p.N, 4 * TokShape<DP>::TPP)) {
        if (wide_rows({&p.g}, p.D)) return launch_tok_grad_lds_s<T, DP, 2, false, true, true>(p, nt, st);
        return launch_tok_grad_lds_s<T, DP, 2, false, false, true>(p, nt, st);
      }
      return launch_tok_grad_lds<T, DP, 4, false>(p, nt, st);
    }
    return launch_tok_grad_lds<T, DP, 4, true>(p, nt, st);
  }
  constexpr int TPB = 256 / (DP / 8);
  dim3 grid((p.N + TPB - 1) / TPB, p.B * p.H);
  MURM_LAUNCH((tok_grad_kernel<T, DP>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace

// This file is compiled once per token dtype (build.py passes
// -DMURM_TOKENS_DT=0 float32, 1 float16, 2 bfloat16), so the three sets of
// kernel instances build in parallel; murm_launch.h dispatches on the dtype.
#if !defined(MURM_TOKENS_DT)
#error "build murm_tokens.hip with -DMURM_TOKENS_DT=0 (float32), 1 (float16) or 2 (bfloat16)"
#elif MURM_TOKENS_DT == 0
using TokT = float;
#define MURM_TOK_FN(name) name##_f32
#elif MURM_TOKENS_DT == 1
using TokT = _Float16;
#define MURM_TOK_FN(name) name##_f16
#elif MURM_TOKENS_DT == 2
using TokT = __bf16;
#define MURM_TOK_FN(name) name##_bf16
#else
#error "MURM_TOKENS_DT must be 0, 1 or 2"
#endif

hipError_t MURM_TOK_FN(launch_tok_bwd)(int DP, const TokBwdParams& p, hipStream_t st) {
  switch (DP) {
    case 32: return launch_tok_bwd_t<TokT, 32>(p, st);
    case 64: return launch_tok_bwd_t<TokT, 64>(p, st);
    case 128: return launch_tok_bwd_t<TokT, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t MURM_TOK_FN(launch_attend_idx)(int DP, const AttendIdxParams& p, hipStream_t st) {
  switch (DP) {
    case 32: return launch_attend_idx_t<TokT, 32>(p, st);
    case 64: return launch_attend_idx_t<TokT, 64>(p, st);
    case 128: return launch_attend_idx_t<TokT, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t MURM_TOK_FN(launch_tok_grad)(int DP, const TokGradParams& p, hipStream_t st) {
  switch (DP) {
    case 32: return launch_tok_grad_t<TokT, 32>(p, st);
    case 64: return launch_tok_grad_t<TokT, 64>(p, st);
    case 128: return launch_tok_grad_t<TokT, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace murm
