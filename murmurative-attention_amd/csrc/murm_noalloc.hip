// Allocation-free entry point: murm_select_attend_fwd with its workspace in
// a fixed device array instead of a caller buffer, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops).  Nothing here
// calls hipMalloc / hipFree or any allocating routine.
//
// Every GPU the library runs on holds its own copy of `scratch` for the life
// of the process.  Calls on one GPU share it: calls that overlap in time on
// one GPU (different streams) race.  The select+attend workspace needs no
// clearing (every byte a call reads, it wrote first), so a call never relies
// on what an earlier call left there.

#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/murmurative_hip.h"
#include "murm_launch.h"

// In host code `scratch` names a host-side stand-in, not device memory: its
// device address (one per GPU) comes from hipGetSymbolAddress below and only
// that address reaches kernels.
static __device__ __align__(256) unsigned char scratch[MURM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEVICES] = {};

int err(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int err(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return murm::set_error(code, buf);
}

// Device address of `scratch` on the current device, which must own `st`;
// looked up on the first call on each device (that device current) and kept.
int scratch_address(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return err(MURM_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (st) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return err(MURM_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if ((int)sdev != dev)
      return err(MURM_ERR_ARG, "the stream belongs to device %d but device %d is current", (int)sdev, dev);
  }
  if (dev < 0 || dev >= MAX_DEVICES) return err(MURM_ERR_UNSUPPORTED, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return err(MURM_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return MURM_OK;
}

}  // namespace

extern "C" int murm_select_attend_fwd_noalloc(
    int dtype, int slot_dtype, int B, int H, int N, int D, int M, const void* q, int64_t q_sb, int64_t q_sh,
    int64_t q_sn, const void* sk, int64_t sk_sb, int64_t sk_sh, int64_t sk_sm, const void* sv, int64_t sv_sb,
    int64_t sv_sh, int64_t sv_sm, const uint8_t* mask, int64_t mk_sb, int64_t mk_sh, int64_t mk_sn, int64_t mk_sm,
    const float* bias, int64_t bs_sb, int64_t bs_sh, int64_t bs_sn, int64_t bs_sm, int causal, double scale,
    int effective_M, void* out, int64_t out_sb, int64_t out_sh, int64_t out_sn, float* weights, int64_t* indices,
    void* stream) {
  if (B < 1 || H < 1 || N < 1 || D < 1 || M < 1)
    return err(MURM_ERR_ARG, "B, H, N, D, M must be >= 1 (got %d, %d, %d, %d, %d)", B, H, N, D, M);
  const size_t need = murm_select_attend_workspace_bytes(B, H, N, D, M);
  if (need > (size_t)MURM_NOALLOC_SCRATCH_BYTES)
    return err(MURM_ERR_UNSUPPORTED,
               "B=%d H=%d N=%d D=%d M=%d needs %zu bytes of scratch but the allocation-free entry holds %zu; "
               "call murm_select_attend_fwd with a workspace",
               B, H, N, D, M, need, (size_t)MURM_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address((hipStream_t)stream, &ws);
  if (rc != MURM_OK) return rc;
  return murm_select_attend_fwd(dtype, slot_dtype, B, H, N, D, M, q, q_sb, q_sh, q_sn, sk, sk_sb, sk_sh, sk_sm, sv,
                                sv_sb, sv_sh, sv_sm, mask, mk_sb, mk_sh, mk_sn, mk_sm, bias, bs_sb, bs_sh, bs_sn,
                                bs_sm, causal, scale, effective_M, out, out_sb, out_sh, out_sn, weights, indices,
                                ws, (size_t)MURM_NOALLOC_SCRATCH_BYTES, stream);
}
