// extern "C" entry points of libmurmurative_hip (declared in
// include/murmurative_hip.h): argument checks, workspace layout and the
// kernel sequence of every operation.  Nothing here allocates device memory.

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/murmurative_hip.h"
#include "murm_common.h"
#include "murm_launch.h"

using namespace murm;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// ------------------------------------------------------------- timing ---
const char* kClassNames[MURM_TIMING_CLASSES] = {"select_attend", "gather_out", "seg_update", "seg_attbwd",
                                                "du", "tok_bwd", "tok_grad", "conversions",
                                                "seg_update_reduce", "seg_attbwd_reduce"};
enum Cls { C_SA = 0, C_OUT, C_SEGU, C_SEGB, C_DU, C_TOKB, C_TOKG, C_CONV, C_SEGUR, C_SEGBR };

struct Timing {
  std::mutex mu;
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> rec[MURM_TIMING_CLASSES];
  std::vector<hipEvent_t> pool;
  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
Timing& timing() {
  static Timing t;
  return t;
}

thread_local LaunchEvents g_launch_events{nullptr, nullptr};

// f() enqueues exactly one kernel; with timing on, that launch records a
// start and a stop event from its own dispatch (hipExtLaunchKernel), so the
// elapsed time between them is the kernel's execution alone.
template <typename F>
int run(int cls, hipStream_t st, const char* what, F&& f) {
  (void)st;
  Timing& T = timing();
  hipEvent_t e0 = nullptr, e1 = nullptr;
  bool on;
  {
    std::lock_guard<std::mutex> lk(T.mu);
    on = T.on;
    if (on) {
      e0 = T.get();
      e1 = T.get();
    }
  }
  const bool timed = on && e0 && e1;
  if (timed) g_launch_events = {e0, e1};
  const hipError_t err = f();
  g_launch_events = {nullptr, nullptr};
  if (timed) {
    std::lock_guard<std::mutex> lk(T.mu);
    if (err == hipSuccess) {
      T.rec[cls].push_back({e0, e1});
    } else {
      T.pool.push_back(e0);
      T.pool.push_back(e1);
    }
  }
  if (err != hipSuccess) return fail(MURM_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  return MURM_OK;
}

#define RUN(cls, what, expr)                                   \
  do {                                                         \
    const int _rc = run(cls, st, what, [&]() { return (expr); }); \
    if (_rc != MURM_OK) return _rc;                            \
  } while (0)

// ------------------------------------------------------------ helpers ---
size_t esize(int dt) { return dt == MURM_F32 ? 4 : 2; }
bool dtype_ok(int dt) { return dt == MURM_F32 || dt == MURM_F16 || dt == MURM_BF16; }

int pick_dp(int D) { return D <= 32 ? 32 : (D <= 64 ? 64 : 128); }

bool aligned16(const void* p, int64_t a, int64_t b, int64_t c, size_t es) {
  return ((uintptr_t)p % 16 == 0) && ((a * (int64_t)es) % 16 == 0) && ((b * (int64_t)es) % 16 == 0) &&
         ((c * (int64_t)es) % 16 == 0);
}
TokView tv_of(const void* p, int64_t sb, int64_t sh, int64_t sn, int dt) {
  TokView v;
  v.p = p; v.sb = sb; v.sh = sh; v.sn = sn;
  v.vec = aligned16(p, sb, sh, sn, esize(dt)) ? 1 : 0;
  return v;
}
TokViewMut tvm_of(void* p, int64_t sb, int64_t sh, int64_t sn, int dt) {
  TokViewMut v;
  v.p = p; v.sb = sb; v.sh = sh; v.sn = sn;
  v.vec = aligned16(p, sb, sh, sn, esize(dt)) ? 1 : 0;
  return v;
}
TokView none_tv() { TokView v{}; return v; }
TokViewMut none_tvm() { TokViewMut v{}; return v; }

void key_masks(int M, uint32_t* hi, uint32_t* lo) {
  int bits = 1;
  while ((1 << bits) < M) ++bits;
  *lo = (1u << bits) - 1u;
  *hi = ~*lo;
}

int check_geom(int dtype, int slot_dtype, int B, int H, int N, int D, int M) {
  if (!dtype_ok(dtype) || !dtype_ok(slot_dtype)) return fail(MURM_ERR_ARG, "unknown dtype code");
  if (B < 1 || H < 1 || N < 1) return fail(MURM_ERR_ARG, "B, H, N must be >= 1 (got %d, %d, %d)", B, H, N);
  if (D < 1 || D > 128) return fail(MURM_ERR_UNSUPPORTED, "head dim D=%d outside [1, 128]", D);
  if (M < KN || M > 65535) return fail(MURM_ERR_ARG, "M=%d outside [7, 65535] (7 slots are selected)", M);
  if (N > (1 << 24)) return fail(MURM_ERR_UNSUPPORTED, "N=%d too large", N);
  if ((int64_t)B * H * N >= (int64_t(1) << 31))
    return fail(MURM_ERR_UNSUPPORTED, "B*H*N=%lld tokens too many (at most 2^31 - 1)", (long long)B * H * N);
  return MURM_OK;
}

// Workspace carving: the same code sizes (base == nullptr) and fills it.
struct Carve {
  char* base;
  size_t off = 0;
  explicit Carve(void* b) : base((char*)b) {}
  template <typename T> T* take(size_t count) {
    off = (off + 255) & ~(size_t)255;
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

// token-chunk partial sums of the slot reductions (shared by every round)
PartParams carve_parts(Carve& c, int B, int H, int N, int D, int M, int mode) {
  PartParams pp{};
  pp.nchunk = seg_chunks(B, H, N, M, D, mode);
  if (pp.nchunk <= 0) return pp;
  pp.chunk_tokens = seg_chunk_tokens(N, pp.nchunk);
  const size_t BH = (size_t)B * H, S = BH * M * D;
  pp.partA = c.take<float>(pp.nchunk * S);
  pp.partB = c.take<float>(pp.nchunk * S);
  pp.partW = c.take<float>(pp.nchunk * BH * M);
  return pp;
}

struct FwdLayout {
  float* sk[MAX_ROUNDS];
  float* sv[MAX_ROUNDS];
  void* ksp[MAX_ROUNDS];   // the round's keys split for the 16-bit select kernel
  float* ksum[MAX_ROUNDS];
  float* vsum[MAX_ROUNDS];
  float* wsum[MAX_ROUNDS];
  uint16_t* idx[MAX_ROUNDS];
  float* w[MAX_ROUNDS];
  PartParams part;
  size_t bytes;
};
FwdLayout fwd_layout(void* ws, int B, int H, int N, int D, int M, int R, int shared) {
  FwdLayout L{};
  Carve c(ws);
  const size_t BH = (size_t)B * H, S = BH * M * D;
  for (int r = 0; r < R; ++r) {
    L.sk[r] = c.take<float>(S);
    L.sv[r] = c.take<float>(S);
    L.ksp[r] = c.take<uint16_t>(BH * ksplit_head_elems(M, pick_dp(D)));
    L.idx[r] = c.take<uint16_t>(BH * N * IDX_ROW);
    if (r < R - 1) {
      L.ksum[r] = c.take<float>(S);
      L.vsum[r] = shared ? L.ksum[r] : c.take<float>(S);
      L.wsum[r] = c.take<float>(BH * M);
      L.w[r] = c.take<float>(BH * N * KN);
    }
  }
  if (R > 1) L.part = carve_parts(c, B, H, N, D, M, SEG_UPDATE);
  L.bytes = c.off;
  return L;
}

struct BwdLayout {
  float* ds[MAX_ROUNDS];
  float* dk[MAX_ROUNDS];
  float* dv[MAX_ROUNDS];
  float* dW[MAX_ROUNDS];
  float* Gk; float* Gv; float* ck[2]; float* cv[2];
  PartParams part;
  size_t bytes;
};
BwdLayout bwd_layout(void* ws, int B, int H, int N, int D, int M, int R, int shared) {
  BwdLayout L{};
  Carve c(ws);
  const size_t BH = (size_t)B * H, S = BH * M * D;
  for (int r = 0; r < R; ++r) {
    L.ds[r] = c.take<float>(BH * N * KN);
    if (r < R - 1) {
      L.dk[r] = c.take<float>(S);
      L.dv[r] = shared ? nullptr : c.take<float>(S);
      L.dW[r] = c.take<float>(BH * M);
    }
  }
  L.Gk = c.take<float>(S);
  L.Gv = c.take<float>(S);
  for (int i = 0; i < 2; ++i) {
    L.ck[i] = c.take<float>(S);
    L.cv[i] = c.take<float>(S);
  }
  L.part = carve_parts(c, B, H, N, D, M, SEG_ATTBWD);
  L.bytes = c.off;
  return L;
}

struct OpLayout {   // scratch of the single-round ops
  float* sk; float* sv; float* nk; float* nv;
  void* ksp;
  float* K; float* V; float* W;
  float* dk; float* dv; float* dW; float* ck; float* cv;
  uint16_t* idx; float* ds; float* wtmp;
  PartParams part;
  size_t bytes;
};
OpLayout op_layout(void* ws, int B, int H, int N, int D, int M, int kind) {
  // kind 0: select_attend fwd, 1: select_attend bwd, 2: update fwd, 3: update bwd
  OpLayout L{};
  Carve c(ws);
  const size_t BH = (size_t)B * H, S = BH * M * D;
  L.idx = c.take<uint16_t>(BH * N * IDX_ROW);
  if (kind == 0 || kind == 1 || kind == 2) { L.sk = c.take<float>(S); L.sv = c.take<float>(S); }
  if (kind == 0) {
    L.wtmp = c.take<float>(BH * N * KN);  // weights scratch of the select-only entry
    L.ksp = c.take<uint16_t>(BH * ksplit_head_elems(M, pick_dp(D)));
  }
  if (kind == 1) { L.ds = c.take<float>(BH * N * KN); L.dk = c.take<float>(S); L.dv = c.take<float>(S); }
  if (kind == 2) { L.nk = c.take<float>(S); L.nv = c.take<float>(S); }
  if (kind == 3) {
    L.K = c.take<float>(S); L.V = c.take<float>(S); L.W = c.take<float>(BH * M);
    L.sk = c.take<float>(S); L.sv = c.take<float>(S);
    L.dk = c.take<float>(S); L.dv = c.take<float>(S); L.dW = c.take<float>(BH * M);
    L.ck = c.take<float>(S); L.cv = c.take<float>(S);
  }
  if (kind != 0) L.part = carve_parts(c, B, H, N, D, M, kind == 1 ? SEG_ATTBWD : SEG_UPDATE);
  L.bytes = c.off;
  return L;
}

int need_ws(const void* ws, size_t have, size_t need) {
  if (need > 0 && !ws) return fail(MURM_ERR_ARG, "workspace is NULL (%zu bytes needed)", need);
  if (have < need) return fail(MURM_ERR_ARG, "workspace too small: %zu < %zu bytes", have, need);
  return MURM_OK;
}

// split-key table for 16-bit tokens (the float32 select kernel reads float32 keys)
KeySplitOut ksplit_out(int dtype, void* p, int D) {
  KeySplitOut k{};
  if (dtype != MURM_F32) {
    k.p = p;
    k.dtype = dtype;
    k.DP = pick_dp(D);
  }
  return k;
}

SAParams sa_params(int B, int H, int N, int D, int M, TokView q, const float* sk, int em, int causal,
                   double scale) {
  SAParams p{};
  p.q = q; p.sk = sk;
  p.B = B; p.H = H; p.N = N; p.D = D; p.M = M;
  p.em = (em <= 0 || em > M) ? M : em;
  p.causal = causal ? 1 : 0;
  p.scale = scale > 0 ? (float)scale : (float)(1.0 / sqrt((double)D));
  key_masks(M, &p.hi_mask, &p.lo_mask);
  return p;
}

// Slot tensors of the token dtype (16-bit) with 16-byte rows and D % 8 == 0,
// under wide token rows: the select kernel reads them itself and writes the
// float32 state (no conversion launch); otherwise one conversion launch
// writes the state and the split keys.
bool slots_readable(int dtype, int slot_dtype, int D, const TokView& qv, const void* sk, int64_t sk_sb,
                    int64_t sk_sh, int64_t sk_sm, const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm) {
  return slot_dtype == dtype && dtype != DT_F32 && D % 8 == 0 && qv.vec &&
         aligned16(sk, sk_sb, sk_sh, sk_sm, esize(dtype)) && aligned16(sv, sv_sb, sv_sh, sv_sm, esize(dtype));
}
void raw_slots(SAParams& p, const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm, const void* sv,
               int64_t sv_sb, int64_t sv_sh, int64_t sv_sm, float* st_k, float* st_v) {
  p.raw_k = sk; p.rk_sb = sk_sb; p.rk_sh = sk_sh; p.rk_sm = sk_sm;
  p.raw_v = sv; p.rv_sb = sv_sb; p.rv_sh = sv_sh; p.rv_sm = sv_sm;
  p.st_k = st_k; p.st_v = st_v;
  p.ksplit = nullptr;
  p.keys_hi_only = 1;
}

SegParams seg_base(int B, int H, int N, int D, int M) {
  SegParams p{};
  p.B = B; p.H = H; p.N = N; p.D = D; p.M = M; p.K = KN;
  p.eps = 1e-8f;
  return p;
}

// Largest M whose slot keys the select kernels stage in one CU's LDS.
int select_max_m(int dtype, int D) {
  if (!dtype_ok(dtype) || D < 1 || D > 128) return 0;
  const int DP = pick_dp(D);
  int M = 65535 & ~15;
  while (M >= KN && sa_lds_bytes(dtype, DP, M) > 160 * 1024) M -= 16;
  return M >= KN ? M : 0;
}

int select_fits(int dtype, int D, int M) {
  const int mx = select_max_m(dtype, D);
  if (M > mx)
    return fail(MURM_ERR_UNSUPPORTED,
                "slot keys (M=%d, D=%d) exceed the 160 KiB LDS of one CU: the select kernels take M <= %d here",
                M, D, mx);
  return MURM_OK;
}

int stencil_check(int dt, int B, int H, int M, int D) {
  if (!dtype_ok(dt)) return fail(MURM_ERR_ARG, "unknown dtype code");
  if (B < 1 || H < 1 || M < 1 || D < 1) return fail(MURM_ERR_ARG, "B, H, M, D must be >= 1");
  return MURM_OK;
}

// MFMA layout self-test kernel (see header)
__global__ void selftest_mfma_kernel(float* out) {
  const int l = threadIdx.x;
  const int row = l & 15, kq = l >> 4;  // A row / B col = l&15, k = 8*kq + i
  for (int test = 0; test < 3; ++test) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
      const int k = 8 * kq + i;
      float av = 0.f, bv = 0.f;
      if (test == 0) { av = k < 16 ? (float)(16 * row + k) : 0.f; bv = (k == row) ? 1.f : 0.f; }
      if (test == 1) { av = (k == row) ? 1.f : 0.f; bv = k < 16 ? (float)(16 * k + row) : 0.f; }
      if (test == 2) { av = (k == row + 16) ? 1.f : 0.f; bv = k >= 16 ? (float)(16 * (k - 16) + row) : 0.f; }
      a[i] = (__bf16)av;
      b[i] = (__bf16)bv;
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mfma_16x16x32(a, b, acc);
    for (int r = 0; r < 4; ++r) out[test * 256 + l * 4 + r] = acc[r];
  }
}

// ------------------------------------------------------- graph replay ---
// Opt-in (murm_graph_replay): the fused rounds' launch sequence of each
// distinct argument set (every pointer, size and scalar, and the stream) is
// captured once into a hipGraph and replayed with one hipGraphLaunch after
// that.  Skipped when timing is on, on the null stream, and when the stream
// is already capturing (the launches then join the caller's graph).
struct GraphCache {
  std::mutex mu;
  bool on = false;
  struct Entry {
    std::string key;
    hipGraphExec_t exec;
  };
  std::vector<Entry> entries;  // most recent last
  static constexpr size_t CAP = 16;
};
GraphCache& graphs() {
  static GraphCache g;
  return g;
}

template <typename... A>
std::string graph_key(char tag, const A&... args) {
  std::string k(1, tag);
  (k.append(reinterpret_cast<const char*>(&args), sizeof(args)), ...);
  return k;
}

// Runs `enqueue` on st directly, or through a cached (or newly captured) graph.
template <typename F>
int with_graph(hipStream_t st, const std::string& key, F&& enqueue) {
  GraphCache& G = graphs();
  bool on;
  {
    std::lock_guard<std::mutex> lk(G.mu);
    on = G.on;
  }
  {
    std::lock_guard<std::mutex> lk(timing().mu);
    on = on && !timing().on;
  }
  if (on && st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) on = false;
  }
  if (!on || !st) return enqueue();
  hipGraphExec_t exec = nullptr;
  {
    std::lock_guard<std::mutex> lk(G.mu);
    for (size_t i = 0; i < G.entries.size(); ++i) {
      if (G.entries[i].key == key) {
        GraphCache::Entry e = G.entries[i];
        G.entries.erase(G.entries.begin() + i);
        G.entries.push_back(e);
        exec = e.exec;
        break;
      }
    }
  }
  if (!exec) {
    hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(MURM_ERR_HIP, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    const int rc = enqueue();
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(st, &g);
    if (rc != MURM_OK) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess || !g) return fail(MURM_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail(MURM_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(G.mu);
    if (G.entries.size() >= GraphCache::CAP) {
      (void)hipGraphExecDestroy(G.entries.front().exec);
      G.entries.erase(G.entries.begin());
    }
    G.entries.push_back({key, exec});
  }
  const hipError_t e = hipGraphLaunch(exec, st);
  return e == hipSuccess ? MURM_OK : fail(MURM_ERR_HIP, "hipGraphLaunch: %s", hipGetErrorString(e));
}

}  // namespace

namespace murm {
LaunchEvents& launch_events() { return g_launch_events; }

int set_error(int code, const char* msg) {
  g_err = msg;
  return code;
}
}  // namespace murm

extern "C" {

const char* murm_version(void) { return "murmurative_hip 0.1.0 (gfx950)"; }
const char* murm_last_error(void) { return g_err.c_str(); }

void murm_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(timing().mu);
  timing().on = on != 0;
}
void murm_timing_reset(void) {
  Timing& T = timing();
  std::lock_guard<std::mutex> lk(T.mu);
  for (auto& v : T.rec) {
    for (auto& pr : v) {
      T.pool.push_back(pr.first);
      T.pool.push_back(pr.second);
    }
    v.clear();
  }
}
int murm_timing_read(int cls, double* total_ms, int64_t* launches) {
  if (cls < 0 || cls >= MURM_TIMING_CLASSES) return fail(MURM_ERR_ARG, "timing class %d", cls);
  Timing& T = timing();
  std::lock_guard<std::mutex> lk(T.mu);
  double tot = 0.0;
  for (auto& pr : T.rec[cls]) {
    if (!pr.first || !pr.second) continue;
    if (hipEventSynchronize(pr.second) != hipSuccess) return fail(MURM_ERR_HIP, "event sync failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, pr.first, pr.second) != hipSuccess) return fail(MURM_ERR_HIP, "elapsed failed");
    tot += ms;
  }
  if (total_ms) *total_ms = tot;
  if (launches) *launches = (int64_t)T.rec[cls].size();
  return MURM_OK;
}
const char* murm_timing_name(int cls) {
  return (cls >= 0 && cls < MURM_TIMING_CLASSES) ? kClassNames[cls] : "";
}

int murm_selftest_mfma(float* out, void* stream) {
  if (!out) return fail(MURM_ERR_ARG, "out is NULL");
  hipStream_t st = (hipStream_t)stream;
  MURM_LAUNCH(selftest_mfma_kernel, dim3(1), dim3(64), 0, st, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MURM_OK : fail(MURM_ERR_HIP, "selftest: %s", hipGetErrorString(e));
}

// ----------------------------------------------------------- select+attend
size_t murm_select_attend_workspace_bytes(int B, int H, int N, int D, int M) {
  return op_layout(nullptr, B, H, N, D, M, 0).bytes;
}

int murm_select_attend_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, const void* q,
                           int64_t q_sb, int64_t q_sh, int64_t q_sn, const void* sk, int64_t sk_sb,
                           int64_t sk_sh, int64_t sk_sm, const void* sv, int64_t sv_sb, int64_t sv_sh,
                           int64_t sv_sm, const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn,
                           int64_t mk_sm, const float* bias, int64_t bs_sb, int64_t bs_sh, int64_t bs_sn,
                           int64_t bs_sm, int causal, double scale, int effective_M, void* out,
                           int64_t out_sb, int64_t out_sh, int64_t out_sn, float* weights, int64_t* indices,
                           void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (!q || !sk || !sv || !out || !weights || !indices) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  if ((rc = select_fits(dtype, D, M))) return rc;
  OpLayout L = op_layout(workspace, B, H, N, D, M, 0);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  const TokView qv = tv_of(q, q_sb, q_sh, q_sn, dtype);
  const bool raw = slots_readable(dtype, slot_dtype, D, qv, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm);
  if (!raw) {
    const SlotConv<const void*, float*> ca{sk, sk_sb, sk_sh, sk_sm, L.sk};
    const SlotConv<const void*, float*> cb{sv, sv_sb, sv_sh, sv_sm, L.sv};
    const KeySplitOut ks = ksplit_out(dtype, L.ksp, D);
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, &cb, B, H, M, D, st, &ks));
  }
  SAParams p = sa_params(B, H, N, D, M, qv, L.sk, effective_M, causal, scale);
  p.mask = mask; p.mk_sb = mk_sb; p.mk_sh = mk_sh; p.mk_sn = mk_sn; p.mk_sm = mk_sm;
  p.bias = bias; p.bs_sb = bs_sb; p.bs_sh = bs_sh; p.bs_sn = bs_sn; p.bs_sm = bs_sm;
  p.idx16 = L.idx; p.idx64 = indices; p.w = weights;
  if (raw) {
    raw_slots(p, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm, L.sk, L.sv);
  } else {
    p.ksplit = ksplit_out(dtype, L.ksp, D).p;
    p.keys_hi_only = slot_dtype == dtype;  // keys exact in the token dtype: zero lo halves
  }
  RUN(C_SA, "select_attend", launch_select_attend(dtype, DP, p, st));
  OutParams o{};
  o.base = none_tv();
  o.out = tvm_of(out, out_sb, out_sh, out_sn, dtype);
  o.B = B; o.H = H; o.N = N; o.D = D; o.M = M; o.R = 1;
  o.rp.idx[0] = L.idx; o.rp.w[0] = weights; o.rp.a[0] = L.sv;
  RUN(C_OUT, "gather_out", launch_gather_out(dtype, DP, o, st));
  return MURM_OK;
}

int murm_select_max_m(int dtype, int D) { return select_max_m(dtype, D); }

int murm_select_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, const void* q, int64_t q_sb,
                    int64_t q_sh, int64_t q_sn, const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                    const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm,
                    const float* bias, int64_t bs_sb, int64_t bs_sh, int64_t bs_sn, int64_t bs_sm, int causal,
                    int effective_M, int64_t* indices, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (!q || !sk || !indices) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  if ((rc = select_fits(dtype, D, M))) return rc;
  OpLayout L = op_layout(workspace, B, H, N, D, M, 0);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  {
    const SlotConv<const void*, float*> ca{sk, sk_sb, sk_sh, sk_sm, L.sk};
    const KeySplitOut ks = ksplit_out(dtype, L.ksp, D);
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, nullptr, B, H, M, D, st, &ks));
  }
  SAParams p = sa_params(B, H, N, D, M, tv_of(q, q_sb, q_sh, q_sn, dtype), L.sk, effective_M, causal, 0.0);
  p.ksplit = ksplit_out(dtype, L.ksp, D).p;
  p.keys_hi_only = slot_dtype == dtype;  // keys exact in the token dtype: zero lo halves
  p.mask = mask; p.mk_sb = mk_sb; p.mk_sh = mk_sh; p.mk_sn = mk_sn; p.mk_sm = mk_sm;
  p.bias = bias; p.bs_sb = bs_sb; p.bs_sh = bs_sh; p.bs_sn = bs_sn; p.bs_sm = bs_sm;
  p.idx16 = nullptr; p.idx64 = indices;
  p.w = L.wtmp;  // weights are not returned
  RUN(C_SA, "select_attend", launch_select_attend(dtype, DP, p, st));
  return MURM_OK;
}

int murm_attend_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, const void* q, int64_t q_sb,
                    int64_t q_sh, int64_t q_sn, const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm,
                    const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm, const int64_t* indices,
                    double scale, void* out, int64_t out_sb, int64_t out_sh, int64_t out_sn, float* weights,
                    void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (!q || !sk || !sv || !indices || !out || !weights) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  OpLayout L = op_layout(workspace, B, H, N, D, M, 0);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  RUN(C_CONV, "idx_pack", launch_idx_pack(indices, L.idx, (int64_t)B * H * N, KN, M, st));
  {
    const SlotConv<const void*, float*> ca{sk, sk_sb, sk_sh, sk_sm, L.sk};
    const SlotConv<const void*, float*> cb{sv, sv_sb, sv_sh, sv_sm, L.sv};
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  AttendIdxParams a{};
  a.B = B; a.H = H; a.N = N; a.D = D; a.M = M;
  a.q = tv_of(q, q_sb, q_sh, q_sn, dtype); a.sk = L.sk; a.idx = L.idx;
  a.scale = scale > 0 ? (float)scale : (float)(1.0 / sqrt((double)D));
  a.w = weights;
  RUN(C_SA, "attend_idx", launch_attend_idx(dtype, DP, a, st));
  OutParams o{};
  o.base = none_tv();
  o.out = tvm_of(out, out_sb, out_sh, out_sn, dtype);
  o.B = B; o.H = H; o.N = N; o.D = D; o.M = M; o.R = 1;
  o.rp.idx[0] = L.idx; o.rp.w[0] = weights; o.rp.a[0] = L.sv;
  RUN(C_OUT, "gather_out", launch_gather_out(dtype, DP, o, st));
  return MURM_OK;
}

size_t murm_select_attend_bwd_workspace_bytes(int B, int H, int N, int D, int M) {
  return op_layout(nullptr, B, H, N, D, M, 1).bytes;
}

int murm_select_attend_bwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, const void* grad_out,
                           int64_t g_sb, int64_t g_sh, int64_t g_sn, const float* grad_weights, const void* q,
                           int64_t q_sb, int64_t q_sh, int64_t q_sn, const void* sk, int64_t sk_sb,
                           int64_t sk_sh, int64_t sk_sm, const void* sv, int64_t sv_sb, int64_t sv_sh,
                           int64_t sv_sm, const int64_t* indices, const float* weights, double scale,
                           void* grad_q, void* grad_sk, void* grad_sv, void* workspace, size_t workspace_bytes,
                           void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (!grad_out || !q || !sk || !sv || !indices || !weights || !grad_q || !grad_sk || !grad_sv)
    return fail(MURM_ERR_ARG, "NULL tensor pointer");
  OpLayout L = op_layout(workspace, B, H, N, D, M, 1);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  const float c = scale > 0 ? (float)scale : (float)(1.0 / sqrt((double)D));
  const int64_t rows = (int64_t)B * H * N;
  RUN(C_CONV, "idx_pack", launch_idx_pack(indices, L.idx, rows, KN, M, st));
  {
    const SlotConv<const void*, float*> ca{sk, sk_sb, sk_sh, sk_sm, L.sk};
    const SlotConv<const void*, float*> cb{sv, sv_sb, sv_sh, sv_sm, L.sv};
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  const TokView g = tv_of(grad_out, g_sb, g_sh, g_sn, dtype);
  const TokView qv = tv_of(q, q_sb, q_sh, q_sn, dtype);
  TokBwdParams t{};
  t.B = B; t.H = H; t.N = N; t.D = D; t.M = M;
  t.g = g; t.idx = L.idx; t.w = weights; t.sv = L.sv; t.gw = grad_weights; t.ds_out = L.ds;
  RUN(C_TOKB, "tok_bwd", launch_tok_bwd(dtype, DP, t, st));
  SegParams s = seg_base(B, H, N, D, M);
  s.idx = L.idx; s.wgt = weights; s.ds = L.ds; s.ds_scale = c; s.va = qv; s.vb = g;
  s.final_out = 1; s.gk_out = L.dk; s.gv_out = L.dv;
  RUN(C_SEGB, "seg_attbwd", launch_seg(dtype, DP, SEG_ATTBWD, s, &L.part, 0, st));
  if (seg_two_stage(dtype, DP, SEG_ATTBWD, s, &L.part))
    RUN(C_SEGBR, "seg_attbwd_reduce", launch_seg(dtype, DP, SEG_ATTBWD, s, &L.part, 1, st));
  const int64_t ssb = (int64_t)H * M * D, ssh = (int64_t)M * D, ssm = D;
  {
    const SlotConv<const float*, void*> ca{L.dk, ssb, ssh, ssm, grad_sk};
    const SlotConv<const float*, void*> cb{L.dv, ssb, ssh, ssm, grad_sv};
    RUN(C_CONV, "from_state", launch_from_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  TokGradParams tg{};
  tg.B = B; tg.H = H; tg.N = N; tg.D = D; tg.M = M; tg.R = 1; tg.c = c;
  tg.g = none_tv();
  tg.dq = tvm_of(grad_q, (int64_t)H * N * D, (int64_t)N * D, D, dtype);
  tg.dtk = none_tvm(); tg.dtv = none_tvm();
  tg.idx[0] = L.idx; tg.w[0] = weights; tg.ds[0] = L.ds; tg.sk[0] = L.sk;
  RUN(C_TOKG, "tok_grad", launch_tok_grad(dtype, DP, tg, st));
  return MURM_OK;
}

// ------------------------------------------------------------ slot update
size_t murm_slot_update_workspace_bytes(int B, int H, int N, int D, int M) {
  return op_layout(nullptr, B, H, N, D, M, 2).bytes;
}

static int update_common(int dtype, int slot_dtype, int B, int H, int N, int D, int M, void* sk, int64_t sk_sb,
                         int64_t sk_sh, int64_t sk_sm, void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                         const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn, const void* tv,
                         int64_t tv_sb, int64_t tv_sh, int64_t tv_sn, const int64_t* indices, const float* weights,
                         double alpha, double gamma, int diffuse, void* workspace, size_t workspace_bytes,
                         void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (!sk || !sv || !tk || !tv || !indices || !weights) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  OpLayout L = op_layout(workspace, B, H, N, D, M, 2);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  RUN(C_CONV, "idx_pack", launch_idx_pack(indices, L.idx, (int64_t)B * H * N, KN, M, st));
  {
    const SlotConv<const void*, float*> ca{sk, sk_sb, sk_sh, sk_sm, L.sk};
    const SlotConv<const void*, float*> cb{sv, sv_sb, sv_sh, sv_sm, L.sv};
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  SegParams s = seg_base(B, H, N, D, M);
  s.idx = L.idx; s.wgt = weights;
  s.va = tv_of(tk, tk_sb, tk_sh, tk_sn, dtype);
  s.vb = tv_of(tv, tv_sb, tv_sh, tv_sn, dtype);
  s.b_same_as_a = 0;
  s.sk_old = L.sk; s.sv_old = L.sv; s.sk_new = L.nk; s.sv_new = L.nv;
  s.alpha = (float)alpha; s.gamma = (float)gamma; s.diffuse = diffuse;
  RUN(C_SEGU, "seg_update", launch_seg(dtype, DP, SEG_UPDATE, s, &L.part, 0, st));
  if (seg_two_stage(dtype, DP, SEG_UPDATE, s, &L.part))
    RUN(C_SEGUR, "seg_update_reduce", launch_seg(dtype, DP, SEG_UPDATE, s, &L.part, 1, st));
  {
    const SlotConv<const float*, void*> ca{L.nk, sk_sb, sk_sh, sk_sm, sk};
    const SlotConv<const float*, void*> cb{L.nv, sv_sb, sv_sh, sv_sm, sv};
    RUN(C_CONV, "from_state", launch_from_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  return MURM_OK;
}

int murm_slot_update_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, void* sk, int64_t sk_sb,
                         int64_t sk_sh, int64_t sk_sm, void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                         const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn, const void* tv,
                         int64_t tv_sb, int64_t tv_sh, int64_t tv_sn, const int64_t* indices,
                         const float* weights, double alpha, void* workspace, size_t workspace_bytes,
                         void* stream) {
  return update_common(dtype, slot_dtype, B, H, N, D, M, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm, tk,
                       tk_sb, tk_sh, tk_sn, tv, tv_sb, tv_sh, tv_sn, indices, weights, alpha, 0.0, 0, workspace,
                       workspace_bytes, stream);
}

int murm_slot_update_diffuse_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, void* sk,
                                 int64_t sk_sb, int64_t sk_sh, int64_t sk_sm, void* sv, int64_t sv_sb,
                                 int64_t sv_sh, int64_t sv_sm, const void* tk, int64_t tk_sb, int64_t tk_sh,
                                 int64_t tk_sn, const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                                 const int64_t* indices, const float* weights, double alpha, double gamma,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return update_common(dtype, slot_dtype, B, H, N, D, M, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm, tk,
                       tk_sb, tk_sh, tk_sn, tv, tv_sb, tv_sh, tv_sn, indices, weights, alpha, gamma, 1, workspace,
                       workspace_bytes, stream);
}

size_t murm_slot_update_bwd_workspace_bytes(int B, int H, int N, int D, int M) {
  return op_layout(nullptr, B, H, N, D, M, 3).bytes;
}

int murm_slot_update_bwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, const void* gk,
                         int64_t gk_sb, int64_t gk_sh, int64_t gk_sm, const void* gv, int64_t gv_sb,
                         int64_t gv_sh, int64_t gv_sm, const void* tk, int64_t tk_sb, int64_t tk_sh,
                         int64_t tk_sn, const void* tv, int64_t tv_sb, int64_t tv_sh, int64_t tv_sn,
                         const int64_t* indices, const float* weights, double alpha, void* grad_tk,
                         void* grad_tv, void* grad_old_sk, void* grad_old_sv, float* grad_w, void* workspace,
                         size_t workspace_bytes, void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (!gk || !gv || !tk || !tv || !indices || !weights || !grad_tk || !grad_tv || !grad_old_sk ||
      !grad_old_sv || !grad_w)
    return fail(MURM_ERR_ARG, "NULL tensor pointer");
  OpLayout L = op_layout(workspace, B, H, N, D, M, 3);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  RUN(C_CONV, "idx_pack", launch_idx_pack(indices, L.idx, (int64_t)B * H * N, KN, M, st));
  {
    const SlotConv<const void*, float*> ca{gk, gk_sb, gk_sh, gk_sm, L.sk};
    const SlotConv<const void*, float*> cb{gv, gv_sb, gv_sh, gv_sm, L.sv};
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  const TokView tkv = tv_of(tk, tk_sb, tk_sh, tk_sn, dtype);
  const TokView tvv = tv_of(tv, tv_sb, tv_sh, tv_sn, dtype);
  SegParams s = seg_base(B, H, N, D, M);
  s.idx = L.idx; s.wgt = weights; s.va = tkv; s.vb = tvv; s.b_same_as_a = 0;
  s.ksum = L.K; s.vsum = L.V; s.wsum = L.W;
  RUN(C_SEGU, "seg_update", launch_seg(dtype, DP, SEG_UPDATE, s, &L.part, 0, st));
  if (seg_two_stage(dtype, DP, SEG_UPDATE, s, &L.part))
    RUN(C_SEGUR, "seg_update_reduce", launch_seg(dtype, DP, SEG_UPDATE, s, &L.part, 1, st));
  DuParams d{};
  d.B = B; d.H = H; d.M = M; d.D = D;
  d.Gk = L.sk; d.Gv = L.sv; d.K = L.K; d.V = L.V; d.W = L.W;
  d.alpha = (float)alpha; d.gamma = 0.f; d.eps = 1e-8f; d.transpose = 0; d.combine_dk = 0;
  d.dk_out = L.dk; d.dv_out = L.dv; d.dW_out = L.dW; d.carry_k = L.ck; d.carry_v = L.cv;
  RUN(C_DU, "du", launch_du(d, st));
  const int64_t ssb = (int64_t)H * M * D, ssh = (int64_t)M * D, ssm = D;
  {
    const SlotConv<const float*, void*> ca{L.ck, ssb, ssh, ssm, grad_old_sk};
    const SlotConv<const float*, void*> cb{L.cv, ssb, ssh, ssm, grad_old_sv};
    RUN(C_CONV, "from_state", launch_from_state2(slot_dtype, ca, &cb, B, H, M, D, st));
  }
  TokBwdParams t{};
  t.B = B; t.H = H; t.N = N; t.D = D; t.M = M;
  t.tk = tkv; t.tv = tvv; t.idx = L.idx; t.w = weights;
  t.dkk = L.dk; t.dkv = L.dv; t.dW = L.dW; t.dw_out = grad_w;
  RUN(C_TOKB, "tok_bwd", launch_tok_bwd(dtype, DP, t, st));
  TokGradParams tg{};
  tg.B = B; tg.H = H; tg.N = N; tg.D = D; tg.M = M; tg.R = 1; tg.c = 0.f;
  tg.g = none_tv(); tg.dq = none_tvm();
  tg.dtk = tvm_of(grad_tk, (int64_t)H * N * D, (int64_t)N * D, D, dtype);
  tg.dtv = tvm_of(grad_tv, (int64_t)H * N * D, (int64_t)N * D, D, dtype);
  tg.idx[0] = L.idx; tg.w[0] = weights; tg.dkk[0] = L.dk; tg.dkv[0] = L.dv;
  RUN(C_TOKG, "tok_grad", launch_tok_grad(dtype, DP, tg, st));
  return MURM_OK;
}

// -------------------------------------------------------------- diffusion
int murm_slot_diffusion_fwd(int slot_dtype, int B, int H, int M, int D, void* sk, int64_t sk_sb, int64_t sk_sh,
                            int64_t sk_sm, void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm, double gamma,
                            void* stream) {
  int rc = stencil_check(slot_dtype, B, H, M, D);
  if (rc) return rc;
  if (!sk || !sv) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  hipStream_t st = (hipStream_t)stream;
  RUN(C_CONV, "stencil", launch_stencil(slot_dtype, sk, sk_sb, sk_sh, sk_sm, sk, sk_sb, sk_sh, sk_sm, B, H, M,
                                        D, (float)gamma, 0, st));
  RUN(C_CONV, "stencil", launch_stencil(slot_dtype, sv, sv_sb, sv_sh, sv_sm, sv, sv_sb, sv_sh, sv_sm, B, H, M,
                                        D, (float)gamma, 0, st));
  return MURM_OK;
}

int murm_slot_diffusion_bwd(int slot_dtype, int B, int H, int M, int D, const void* gk, int64_t gk_sb,
                            int64_t gk_sh, int64_t gk_sm, const void* gv, int64_t gv_sb, int64_t gv_sh,
                            int64_t gv_sm, double gamma, void* grad_k, void* grad_v, void* stream) {
  int rc = stencil_check(slot_dtype, B, H, M, D);
  if (rc) return rc;
  if (!gk || !gv || !grad_k || !grad_v) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t ob = (int64_t)H * M * D, oh = (int64_t)M * D, om = D;
  RUN(C_CONV, "stencil", launch_stencil(slot_dtype, const_cast<void*>(gk), gk_sb, gk_sh, gk_sm, grad_k, ob, oh,
                                        om, B, H, M, D, (float)gamma, 1, st));
  RUN(C_CONV, "stencil", launch_stencil(slot_dtype, const_cast<void*>(gv), gv_sb, gv_sh, gv_sm, grad_v, ob, oh,
                                        om, B, H, M, D, (float)gamma, 1, st));
  return MURM_OK;
}

// ---------------------------------------------------------------- rounds
size_t murm_murmurate_workspace_bytes(int B, int H, int N, int D, int M, int rounds, int shared_kv) {
  if (rounds < 1 || rounds > MAX_ROUNDS) return 0;
  return fwd_layout(nullptr, B, H, N, D, M, rounds, shared_kv).bytes;
}

static int murmurate_fwd_enqueue(int dtype, int slot_dtype, int B, int H, int N, int D, int M, int rounds,
                       double alpha, double gamma, int causal, int effective_M, double scale, const void* q, int64_t q_sb,
                       int64_t q_sh, int64_t q_sn, const void* x, int64_t x_sb, int64_t x_sh, int64_t x_sn,
                       const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn, const void* tv,
                       int64_t tv_sb, int64_t tv_sh, int64_t tv_sn, const void* sk, int64_t sk_sb, int64_t sk_sh,
                       int64_t sk_sm, const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                       const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm, void* out,
                       int64_t out_sb, int64_t out_sh, int64_t out_sn, int64_t* indices_last,
                       float* weights_last, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (rounds < 1 || rounds > MAX_ROUNDS) return fail(MURM_ERR_ARG, "rounds=%d outside [1, 16]", rounds);
  if (!q || !sk || !sv || !out || !weights_last) return fail(MURM_ERR_ARG, "NULL tensor pointer");
  if ((tk == nullptr) != (tv == nullptr)) return fail(MURM_ERR_ARG, "tk and tv must both be given or both NULL");
  const int shared = tk == nullptr;
  if ((rc = select_fits(dtype, D, M))) return rc;
  FwdLayout L = fwd_layout(workspace, B, H, N, D, M, rounds, shared);
  if ((rc = need_ws(workspace, workspace_bytes, L.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  const TokView qv = tv_of(q, q_sb, q_sh, q_sn, dtype);
  const TokView kv = shared ? qv : tv_of(tk, tk_sb, tk_sh, tk_sn, dtype);
  const TokView vv = shared ? qv : tv_of(tv, tv_sb, tv_sh, tv_sn, dtype);
  const bool raw = slots_readable(dtype, slot_dtype, D, qv, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm);
  if (!raw) {
    const SlotConv<const void*, float*> ca{sk, sk_sb, sk_sh, sk_sm, L.sk[0]};
    const SlotConv<const void*, float*> cb{sv, sv_sb, sv_sh, sv_sm, L.sv[0]};
    const KeySplitOut ks = ksplit_out(dtype, L.ksp[0], D);
    RUN(C_CONV, "to_state", launch_to_state2(slot_dtype, ca, &cb, B, H, M, D, st, &ks));
  }
  for (int r = 0; r < rounds; ++r) {
    const bool last = r == rounds - 1;
    SAParams p = sa_params(B, H, N, D, M, qv, L.sk[r], effective_M, causal, scale);
    p.mask = mask; p.mk_sb = mk_sb; p.mk_sh = mk_sh; p.mk_sn = mk_sn; p.mk_sm = mk_sm;
    if (r == 0 && raw) {
      raw_slots(p, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm, L.sk[0], L.sv[0]);
    } else {
      p.ksplit = ksplit_out(dtype, L.ksp[r], D).p;
    }
    p.keys_hi_only = r == 0 && slot_dtype == dtype;  // the caller's keys: zero lo halves
    p.idx16 = L.idx[r];
    p.idx64 = last ? indices_last : nullptr;
    p.w = last ? weights_last : L.w[r];
    RUN(C_SA, "select_attend", launch_select_attend(dtype, DP, p, st));
    if (last) break;
    SegParams s = seg_base(B, H, N, D, M);
    s.idx = L.idx[r]; s.wgt = L.w[r]; s.va = kv; s.vb = vv; s.b_same_as_a = shared;
    s.uniq_idx = 1;  // the select kernel names 7 distinct slots per token
    s.sk_old = L.sk[r]; s.sv_old = L.sv[r]; s.sk_new = L.sk[r + 1]; s.sv_new = L.sv[r + 1];
    s.ksum = L.ksum[r]; s.vsum = shared ? nullptr : L.vsum[r]; s.wsum = L.wsum[r];
    s.alpha = (float)alpha; s.gamma = (float)gamma; s.diffuse = 1;
    s.ksplit_new = ksplit_out(dtype, L.ksp[r + 1], D);
    RUN(C_SEGU, "seg_update", launch_seg(dtype, DP, SEG_UPDATE, s, &L.part, 0, st));
    if (seg_two_stage(dtype, DP, SEG_UPDATE, s, &L.part))
      RUN(C_SEGUR, "seg_update_reduce", launch_seg(dtype, DP, SEG_UPDATE, s, &L.part, 1, st));
  }
  OutParams o{};
  o.base = x ? tv_of(x, x_sb, x_sh, x_sn, dtype) : qv;
  o.out = tvm_of(out, out_sb, out_sh, out_sn, dtype);
  o.B = B; o.H = H; o.N = N; o.D = D; o.M = M; o.R = rounds;
  for (int r = 0; r < rounds; ++r) {
    o.rp.idx[r] = L.idx[r];
    o.rp.w[r] = (r == rounds - 1) ? weights_last : L.w[r];
    o.rp.a[r] = L.sv[r];
  }
  RUN(C_OUT, "gather_out", launch_gather_out(dtype, DP, o, st));
  return MURM_OK;
}

int64_t murm_murmurate_workspace_offset(int B, int H, int N, int D, int M, int rounds, int shared_kv, int round,
                                        int field) {
  if (rounds < 1 || rounds > MAX_ROUNDS || round < 0 || round >= rounds) return -1;
  char* const base = reinterpret_cast<char*>(4096);  // any non-null origin
  FwdLayout L = fwd_layout(base, B, H, N, D, M, rounds, shared_kv);
  const void* p = nullptr;
  switch (field) {
    case 0: p = L.sk[round]; break;
    case 1: p = L.sv[round]; break;
    case 2: p = L.idx[round]; break;
    case 3: p = L.ksum[round]; break;
    case 4: p = L.vsum[round]; break;
    case 5: p = L.wsum[round]; break;
    case 6: p = L.w[round]; break;
    default: return -1;
  }
  return p ? (int64_t)(reinterpret_cast<const char*>(p) - base) : -1;
}

size_t murm_murmurate_bwd_workspace_bytes(int B, int H, int N, int D, int M, int rounds, int shared_kv) {
  if (rounds < 1 || rounds > MAX_ROUNDS) return 0;
  return bwd_layout(nullptr, B, H, N, D, M, rounds, shared_kv).bytes;
}

static int murmurate_bwd_enqueue(int dtype, int slot_dtype, int B, int H, int N, int D, int M, int rounds,
                       double alpha, double gamma, double scale, int x_given, const void* grad_out, int64_t g_sb, int64_t g_sh,
                       int64_t g_sn, const float* grad_weights_last, const void* q, int64_t q_sb, int64_t q_sh,
                       int64_t q_sn, const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn, const void* tv,
                       int64_t tv_sb, int64_t tv_sh, int64_t tv_sn, const float* weights_last,
                       const void* fwd_workspace, size_t fwd_workspace_bytes, void* grad_q, int64_t gq_sb,
                       int64_t gq_sh, int64_t gq_sn, void* grad_tk, int64_t gtk_sb, int64_t gtk_sh,
                       int64_t gtk_sn, void* grad_tv, int64_t gtv_sb, int64_t gtv_sh, int64_t gtv_sn,
                       void* grad_sk, void* grad_sv, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_geom(dtype, slot_dtype, B, H, N, D, M);
  if (rc) return rc;
  if (rounds < 1 || rounds > MAX_ROUNDS) return fail(MURM_ERR_ARG, "rounds=%d outside [1, 16]", rounds);
  if (!grad_out || !q || !weights_last || !grad_q || !grad_sk || !grad_sv)
    return fail(MURM_ERR_ARG, "NULL tensor pointer");
  if ((tk == nullptr) != (tv == nullptr)) return fail(MURM_ERR_ARG, "tk and tv must both be given or both NULL");
  const int shared = tk == nullptr;
  if (!shared && (!grad_tk || !grad_tv)) return fail(MURM_ERR_ARG, "grad_tk / grad_tv needed when tk / tv given");
  FwdLayout L = fwd_layout(const_cast<void*>(fwd_workspace), B, H, N, D, M, rounds, shared);
  if ((rc = need_ws(fwd_workspace, fwd_workspace_bytes, L.bytes))) return rc;
  BwdLayout G = bwd_layout(workspace, B, H, N, D, M, rounds, shared);
  if ((rc = need_ws(workspace, workspace_bytes, G.bytes))) return rc;
  const int DP = pick_dp(D);
  hipStream_t st = (hipStream_t)stream;
  const float c = scale > 0 ? (float)scale : (float)(1.0 / sqrt((double)D));
  const TokView gv = tv_of(grad_out, g_sb, g_sh, g_sn, dtype);
  const TokView qv = tv_of(q, q_sb, q_sh, q_sn, dtype);
  const TokView kv = shared ? qv : tv_of(tk, tk_sb, tk_sh, tk_sn, dtype);
  const TokView vv = shared ? qv : tv_of(tv, tv_sb, tv_sh, tv_sn, dtype);
  auto wr = [&](int r) { return (r == rounds - 1) ? weights_last : (const float*)L.w[r]; };

  for (int r = rounds - 1; r >= 0; --r) {
    const bool last = r == rounds - 1;
    TokBwdParams t{};
    t.B = B; t.H = H; t.N = N; t.D = D; t.M = M;
    t.g = gv; t.tk = kv; t.tv = vv; t.idx = L.idx[r]; t.w = wr(r); t.sv = L.sv[r];
    t.dkk = last ? nullptr : G.dk[r];
    t.dkv = (last || shared) ? nullptr : G.dv[r];
    t.dW = last ? nullptr : G.dW[r];
    t.gw = last ? grad_weights_last : nullptr;
    t.ds_out = G.ds[r];
    RUN(C_TOKB, "tok_bwd", launch_tok_bwd(dtype, DP, t, st));

    // slot side of round r; its epilogue runs round r-1's diffusion adjoint and
    // EMA backward (carries ping-pong: the halo rows read the other buffer)
    SegParams s = seg_base(B, H, N, D, M);
    s.idx = L.idx[r]; s.wgt = wr(r); s.ds = G.ds[r]; s.ds_scale = c; s.va = qv; s.vb = gv;
    s.uniq_idx = 1;  // the forward's select kernel named 7 distinct slots per token
    s.carry_k = last ? nullptr : G.ck[(r + 1) & 1];
    s.carry_v = last ? nullptr : G.cv[(r + 1) & 1];
    if (r > 0) {
      s.final_out = 0;
      s.Kp = L.ksum[r - 1]; s.Vp = L.vsum[r - 1]; s.Wp = L.wsum[r - 1];
      s.alpha = (float)alpha; s.gamma = (float)gamma;
      s.combine_dk = shared;
      s.dk_out = G.dk[r - 1]; s.dv_out = G.dv[r - 1]; s.dW_out = G.dW[r - 1];
      s.carry_k_out = G.ck[r & 1]; s.carry_v_out = G.cv[r & 1];
    } else {  // the first round's slot grads go straight to the caller's tensors
      s.final_out = 1;
      s.gk_out = G.Gk; s.gv_out = G.Gv;
      s.gk_t = grad_sk; s.gv_t = grad_sv;
      s.gt_sb = (int64_t)H * M * D; s.gt_sh = (int64_t)M * D; s.gt_sm = D;
      s.gt_dtype = slot_dtype;
    }
    RUN(C_SEGB, "seg_attbwd", launch_seg(dtype, DP, SEG_ATTBWD, s, &G.part, 0, st));
    if (seg_two_stage(dtype, DP, SEG_ATTBWD, s, &G.part))
      RUN(C_SEGBR, "seg_attbwd_reduce", launch_seg(dtype, DP, SEG_ATTBWD, s, &G.part, 1, st));
  }

  TokGradParams tg{};
  tg.B = B; tg.H = H; tg.N = N; tg.D = D; tg.M = M; tg.R = rounds; tg.c = c;
  tg.g = x_given ? none_tv() : gv;
  tg.dq = tvm_of(grad_q, gq_sb, gq_sh, gq_sn, dtype);
  tg.dtk = shared ? none_tvm() : tvm_of(grad_tk, gtk_sb, gtk_sh, gtk_sn, dtype);
  tg.dtv = shared ? none_tvm() : tvm_of(grad_tv, gtv_sb, gtv_sh, gtv_sn, dtype);
  tg.shared_kv = shared;
  for (int r = 0; r < rounds; ++r) {
    tg.idx[r] = L.idx[r]; tg.w[r] = wr(r); tg.ds[r] = G.ds[r]; tg.sk[r] = L.sk[r];
    tg.dkk[r] = (r < rounds - 1) ? G.dk[r] : nullptr;
    tg.dkv[r] = (r < rounds - 1 && !shared) ? G.dv[r] : nullptr;
  }
  RUN(C_TOKG, "tok_grad", launch_tok_grad(dtype, DP, tg, st));
  return MURM_OK;
}

int murm_murmurate_fwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, int rounds, double alpha,
                       double gamma, int causal, int effective_M, double scale, const void* q, int64_t q_sb,
                       int64_t q_sh, int64_t q_sn, const void* x, int64_t x_sb, int64_t x_sh, int64_t x_sn,
                       const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn, const void* tv,
                       int64_t tv_sb, int64_t tv_sh, int64_t tv_sn, const void* sk, int64_t sk_sb, int64_t sk_sh,
                       int64_t sk_sm, const void* sv, int64_t sv_sb, int64_t sv_sh, int64_t sv_sm,
                       const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm, void* out,
                       int64_t out_sb, int64_t out_sh, int64_t out_sn, int64_t* indices_last,
                       float* weights_last, void* workspace, size_t workspace_bytes, void* stream) {
  const std::string key =
      graph_key('f', dtype, slot_dtype, B, H, N, D, M, rounds, alpha, gamma, causal, effective_M, scale, q, q_sb,
                q_sh, q_sn, x, x_sb, x_sh, x_sn, tk, tk_sb, tk_sh, tk_sn, tv, tv_sb, tv_sh, tv_sn, sk, sk_sb, sk_sh,
                sk_sm, sv, sv_sb, sv_sh, sv_sm, mask, mk_sb, mk_sh, mk_sn, mk_sm, out, out_sb, out_sh, out_sn,
                indices_last, weights_last, workspace, workspace_bytes, stream);
  return with_graph((hipStream_t)stream, key, [&]() {
    return murmurate_fwd_enqueue(dtype, slot_dtype, B, H, N, D, M, rounds, alpha, gamma, causal, effective_M, scale,
                                 q, q_sb, q_sh, q_sn, x, x_sb, x_sh, x_sn, tk, tk_sb, tk_sh, tk_sn, tv, tv_sb, tv_sh,
                                 tv_sn, sk, sk_sb, sk_sh, sk_sm, sv, sv_sb, sv_sh, sv_sm, mask, mk_sb, mk_sh, mk_sn,
                                 mk_sm, out, out_sb, out_sh, out_sn, indices_last, weights_last, workspace,
                                 workspace_bytes, stream);
  });
}

int murm_murmurate_bwd(int dtype, int slot_dtype, int B, int H, int N, int D, int M, int rounds, double alpha,
                       double gamma, double scale, int x_given, const void* grad_out, int64_t g_sb, int64_t g_sh,
                       int64_t g_sn, const float* grad_weights_last, const void* q, int64_t q_sb, int64_t q_sh,
                       int64_t q_sn, const void* tk, int64_t tk_sb, int64_t tk_sh, int64_t tk_sn, const void* tv,
                       int64_t tv_sb, int64_t tv_sh, int64_t tv_sn, const float* weights_last,
                       const void* fwd_workspace, size_t fwd_workspace_bytes, void* grad_q, int64_t gq_sb,
                       int64_t gq_sh, int64_t gq_sn, void* grad_tk, int64_t gtk_sb, int64_t gtk_sh,
                       int64_t gtk_sn, void* grad_tv, int64_t gtv_sb, int64_t gtv_sh, int64_t gtv_sn,
                       void* grad_sk, void* grad_sv, void* workspace, size_t workspace_bytes, void* stream) {
  const std::string key =
      graph_key('b', dtype, slot_dtype, B, H, N, D, M, rounds, alpha, gamma, scale, x_given, grad_out, g_sb, g_sh,
                g_sn, grad_weights_last, q, q_sb, q_sh, q_sn, tk, tk_sb, tk_sh, tk_sn, tv, tv_sb, tv_sh, tv_sn,
                weights_last, fwd_workspace, fwd_workspace_bytes, grad_q, gq_sb, gq_sh, gq_sn, grad_tk, gtk_sb,
                gtk_sh, gtk_sn, grad_tv, gtv_sb, gtv_sh, gtv_sn, grad_sk, grad_sv, workspace, workspace_bytes,
                stream);
  return with_graph((hipStream_t)stream, key, [&]() {
    return murmurate_bwd_enqueue(dtype, slot_dtype, B, H, N, D, M, rounds, alpha, gamma, scale, x_given, grad_out,
                                 g_sb, g_sh, g_sn, grad_weights_last, q, q_sb, q_sh, q_sn, tk, tk_sb, tk_sh, tk_sn,
                                 tv, tv_sb, tv_sh, tv_sn, weights_last, fwd_workspace, fwd_workspace_bytes, grad_q,
                                 gq_sb, gq_sh, gq_sn, grad_tk, gtk_sb, gtk_sh, gtk_sn, grad_tv, gtv_sb, gtv_sh,
                                 gtv_sn, grad_sk, grad_sv, workspace, workspace_bytes, stream);
  });
}

void murm_graph_replay(int on) {
  GraphCache& G = graphs();
  std::lock_guard<std::mutex> lk(G.mu);
  G.on = on != 0;
  if (!G.on) {
    for (auto& e : G.entries) (void)hipGraphExecDestroy(e.exec);
    G.entries.clear();
  }
}

int murm_graph_cached(void) {
  GraphCache& G = graphs();
  std::lock_guard<std::mutex> lk(G.mu);
  return (int)G.entries.size();
}

}  // extern "C"
