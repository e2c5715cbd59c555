// Tensor-level wrappers: checks, output allocation through the caching
// allocator, then one call into the C ABI of libmurmurative_hip on the
// current stream.  Shapes and error behaviour follow the reference launchers
// (src/murmurative/csrc/cuda/*.cu, launcher sections) with the dtype and size
// limits lifted: bf16 / fp16 / fp32, D <= 128, any M in [7, 65535].

#include <ATen/ATen.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/util/Exception.h>

#include <algorithm>

#include "murmurative_hip.h"
#include "torch_binding.h"

namespace {

constexpr int64_t KN = 7;

int dt_code(const at::Tensor& t, const char* name) {
  switch (t.scalar_type()) {
    case at::kFloat: return MURM_F32;
    case at::kHalf: return MURM_F16;
    case at::kBFloat16: return MURM_BF16;
    default: TORCH_CHECK(false, name, " must be float32, float16 or bfloat16, got ", t.scalar_type());
  }
  return -1;
}

void ok(int rc, const char* what) { TORCH_CHECK(rc == MURM_OK, what, ": ", murm_last_error()); }

hipStream_t stream_of(const at::Tensor& t) {
  return at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// 4-D device tensor with a unit-stride last dimension (copied otherwise).
at::Tensor rows4(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be on the GPU");
  TORCH_CHECK(t.dim() == 4, name, " must be 4-D, got ", t.dim(), "-D");
  return t.stride(3) == 1 ? t : t.contiguous();
}

void same_device(const at::Tensor& a, const at::Tensor& b, const char* name) {
  TORCH_CHECK(a.device() == b.device(), name, " is on ", b.device(), ", expected ", a.device());
}

at::Tensor idx_tensor(const at::Tensor& idx, int64_t B, int64_t H, int64_t N) {
  TORCH_CHECK(idx.is_cuda(), "indices must be on the GPU");
  TORCH_CHECK(idx.dim() == 4 && idx.size(0) == B && idx.size(1) == H && idx.size(2) == N,
              "indices must be [B,H,N,K] matching the tokens");
  TORCH_CHECK(idx.size(3) == KN, "indices must select exactly 7 slots per token, got ", idx.size(3));
  return idx.to(at::kLong).contiguous();
}

at::Tensor w_tensor(const at::Tensor& w, int64_t B, int64_t H, int64_t N) {
  TORCH_CHECK(w.is_cuda(), "weights must be on the GPU");
  TORCH_CHECK(w.dim() == 4 && w.size(0) == B && w.size(1) == H && w.size(2) == N && w.size(3) == KN,
              "weights must be [B,H,N,7]");
  return w.to(at::kFloat).contiguous();
}

void check_slots(const at::Tensor& sk, const at::Tensor& sv, int64_t B, int64_t H, int64_t D) {
  TORCH_CHECK(sk.size(0) == B && sk.size(1) == H && sk.size(3) == D,
              "slot_keys must be [B,H,M,D] with the tokens' B, H, D");
  TORCH_CHECK(sv.sizes() == sk.sizes(), "slot_values must have the shape of slot_keys");
  TORCH_CHECK(sv.scalar_type() == sk.scalar_type(), "slot_values must have the dtype of slot_keys");
}

// [B,H,N,M] view of an optional mask / bias with broadcast strides.
at::Tensor bhnm(const at::Tensor& t, at::ScalarType st, int64_t B, int64_t H, int64_t N, int64_t M,
                const at::Tensor& like, const char* name) {
  TORCH_CHECK(t.dim() <= 4, name, " must broadcast to [B,H,N,M]");
  at::Tensor u = t.to(like.device());
  u = (st == at::kByte) ? u.ne(0).to(at::kByte) : u.to(st);
  return u.expand({B, H, N, M});
}

}  // namespace

// ---------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor, at::Tensor> slot_select_attend(
    const at::Tensor& query_in, const at::Tensor& slot_keys_in, const at::Tensor& slot_values_in,
    const std::optional<at::Tensor>& mask, bool causal, const std::optional<at::Tensor>& position_bias,
    std::optional<double> scale, int64_t effective_M) {
  const at::Tensor q = rows4(query_in, "query");
  const at::Tensor sk = rows4(slot_keys_in, "slot_keys");
  const at::Tensor sv = rows4(slot_values_in, "slot_values");
  same_device(q, sk, "slot_keys");
  same_device(q, sv, "slot_values");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), M = sk.size(2);
  check_slots(sk, sv, B, H, D);
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  at::Tensor mk, bs;
  if (mask.has_value()) mk = bhnm(*mask, at::kByte, B, H, N, M, q, "mask");
  if (position_bias.has_value()) bs = bhnm(*position_bias, at::kFloat, B, H, N, M, q, "position_bias");
  auto out = at::empty({B, H, N, D}, q.options());
  auto weights = at::empty({B, H, N, KN}, q.options().dtype(at::kFloat));
  auto indices = at::empty({B, H, N, KN}, q.options().dtype(at::kLong));
  auto ws = workspace(murm_select_attend_workspace_bytes(B, H, N, D, M), q);
  ok(murm_select_attend_fwd(
         dt_code(q, "query"), dt_code(sk, "slot_keys"), B, H, N, D, M, q.data_ptr(), q.stride(0), q.stride(1),
         q.stride(2), sk.data_ptr(), sk.stride(0), sk.stride(1), sk.stride(2), sv.data_ptr(), sv.stride(0),
         sv.stride(1), sv.stride(2), mk.defined() ? (const uint8_t*)mk.data_ptr() : nullptr,
         mk.defined() ? mk.stride(0) : 0, mk.defined() ? mk.stride(1) : 0, mk.defined() ? mk.stride(2) : 0,
         mk.defined() ? mk.stride(3) : 0, bs.defined() ? bs.data_ptr<float>() : nullptr,
         bs.defined() ? bs.stride(0) : 0, bs.defined() ? bs.stride(1) : 0, bs.defined() ? bs.stride(2) : 0,
         bs.defined() ? bs.stride(3) : 0, causal ? 1 : 0, scale.has_value() ? *scale : 0.0, (int)effective_M,
         out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), weights.data_ptr<float>(),
         indices.data_ptr<int64_t>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(q)),
     "slot_select_attend");
  return {out, weights, indices};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> slot_select_attend_backward(
    const at::Tensor& grad_output_in, const at::Tensor& grad_weights_in, const at::Tensor& query_in,
    const at::Tensor& slot_keys_in, const at::Tensor& slot_values_in, const at::Tensor& indices_in,
    const at::Tensor& weights_in, std::optional<double> scale) {
  const at::Tensor q = rows4(query_in, "query");
  const at::Tensor go = rows4(grad_output_in, "grad_output");
  const at::Tensor sk = rows4(slot_keys_in, "slot_keys");
  const at::Tensor sv = rows4(slot_values_in, "slot_values");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), M = sk.size(2);
  check_slots(sk, sv, B, H, D);
  TORCH_CHECK(go.sizes() == q.sizes(), "grad_output must have the query's shape");
  TORCH_CHECK(go.scalar_type() == q.scalar_type(), "grad_output must have the query's dtype");
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  const at::Tensor idx = idx_tensor(indices_in, B, H, N);
  const at::Tensor w = w_tensor(weights_in, B, H, N);
  at::Tensor gw;
  if (grad_weights_in.defined() && grad_weights_in.numel() > 0) gw = w_tensor(grad_weights_in, B, H, N);
  auto gq = at::empty({B, H, N, D}, q.options());
  auto gsk = at::empty({B, H, M, D}, sk.options());
  auto gsv = at::empty({B, H, M, D}, sv.options());
  auto ws = workspace(murm_select_attend_bwd_workspace_bytes(B, H, N, D, M), q);
  ok(murm_select_attend_bwd(dt_code(q, "query"), dt_code(sk, "slot_keys"), B, H, N, D, M, go.data_ptr(),
                            go.stride(0), go.stride(1), go.stride(2), gw.defined() ? gw.data_ptr<float>() : nullptr,
                            q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), sk.data_ptr(), sk.stride(0),
                            sk.stride(1), sk.stride(2), sv.data_ptr(), sv.stride(0), sv.stride(1), sv.stride(2),
                            idx.data_ptr<int64_t>(), w.data_ptr<float>(), scale.has_value() ? *scale : 0.0,
                            gq.data_ptr(), gsk.data_ptr(), gsv.data_ptr(), ws.data_ptr(), (size_t)ws.numel(),
                            stream_of(q)),
     "slot_select_attend_backward");
  return {gq, gsk, gsv};
}

// ---------------------------------------------------------------------------
static void update_impl(at::Tensor& slot_keys, at::Tensor& slot_values, const at::Tensor& token_keys,
                        const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights,
                        double alpha, double gamma, bool diffuse, const char* what) {
  TORCH_CHECK(slot_keys.is_cuda() && slot_keys.dim() == 4 && slot_keys.stride(3) == 1,
              "slot_keys must be a 4-D GPU tensor with a contiguous last dimension");
  TORCH_CHECK(slot_values.is_cuda() && slot_values.dim() == 4 && slot_values.stride(3) == 1,
              "slot_values must be a 4-D GPU tensor with a contiguous last dimension");
  at::assert_no_internal_overlap(slot_keys);
  at::assert_no_internal_overlap(slot_values);
  const at::Tensor tk = rows4(token_keys, "token_keys");
  const at::Tensor tv = rows4(token_values, "token_values");
  const int64_t B = tk.size(0), H = tk.size(1), N = tk.size(2), D = tk.size(3), M = slot_keys.size(2);
  check_slots(slot_keys, slot_values, B, H, D);
  TORCH_CHECK(tv.sizes() == tk.sizes() && tv.scalar_type() == tk.scalar_type(),
              "token_values must match token_keys");
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(tk.device());
  const at::Tensor idx = idx_tensor(indices, B, H, N);
  const at::Tensor w = w_tensor(weights, B, H, N);
  auto ws = workspace(murm_slot_update_workspace_bytes(B, H, N, D, M), tk);
  const int dt = dt_code(tk, "token_keys"), sdt = dt_code(slot_keys, "slot_keys");
  int rc;
  if (diffuse) {
    rc = murm_slot_update_diffuse_fwd(dt, sdt, B, H, N, D, M, slot_keys.data_ptr(), slot_keys.stride(0),
                                      slot_keys.stride(1), slot_keys.stride(2), slot_values.data_ptr(),
                                      slot_values.stride(0), slot_values.stride(1), slot_values.stride(2),
                                      tk.data_ptr(), tk.stride(0), tk.stride(1), tk.stride(2), tv.data_ptr(),
                                      tv.stride(0), tv.stride(1), tv.stride(2), idx.data_ptr<int64_t>(),
                                      w.data_ptr<float>(), alpha, gamma, ws.data_ptr(), (size_t)ws.numel(),
                                      stream_of(tk));
  } else {
    rc = murm_slot_update_fwd(dt, sdt, B, H, N, D, M, slot_keys.data_ptr(), slot_keys.stride(0),
                              slot_keys.stride(1), slot_keys.stride(2), slot_values.data_ptr(),
                              slot_values.stride(0), slot_values.stride(1), slot_values.stride(2), tk.data_ptr(),
                              tk.stride(0), tk.stride(1), tk.stride(2), tv.data_ptr(), tv.stride(0), tv.stride(1),
                              tv.stride(2), idx.data_ptr<int64_t>(), w.data_ptr<float>(), alpha, ws.data_ptr(),
                              (size_t)ws.numel(), stream_of(tk));
  }
  ok(rc, what);
}

void slot_update(at::Tensor& slot_keys, at::Tensor& slot_values, const at::Tensor& token_keys,
                 const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights,
                 double alpha) {
  update_impl(slot_keys, slot_values, token_keys, token_values, indices, weights, alpha, 0.0, false,
              "slot_update");
}

void slot_update_diffuse(at::Tensor& slot_keys, at::Tensor& slot_values, const at::Tensor& token_keys,
                         const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights,
                         double alpha, double gamma) {
  update_impl(slot_keys, slot_values, token_keys, token_values, indices, weights, alpha, gamma, true,
              "slot_update_diffuse");
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> slot_update_backward(
    const at::Tensor& grad_new_sk_in, const at::Tensor& grad_new_sv_in, const at::Tensor& token_keys,
    const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights, double alpha) {
  const at::Tensor gk = rows4(grad_new_sk_in, "grad_new_sk");
  const at::Tensor gv = rows4(grad_new_sv_in, "grad_new_sv");
  const at::Tensor tk = rows4(token_keys, "token_keys");
  const at::Tensor tv = rows4(token_values, "token_values");
  const int64_t B = tk.size(0), H = tk.size(1), N = tk.size(2), D = tk.size(3), M = gk.size(2);
  check_slots(gk, gv, B, H, D);
  TORCH_CHECK(tv.sizes() == tk.sizes() && tv.scalar_type() == tk.scalar_type(),
              "token_values must match token_keys");
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(tk.device());
  const at::Tensor idx = idx_tensor(indices, B, H, N);
  const at::Tensor w = w_tensor(weights, B, H, N);
  auto gtk = at::empty({B, H, N, D}, tk.options());
  auto gtv = at::empty({B, H, N, D}, tv.options());
  auto gok = at::empty({B, H, M, D}, gk.options());
  auto gov = at::empty({B, H, M, D}, gv.options());
  auto gw = at::empty({B, H, N, KN}, tk.options().dtype(at::kFloat));
  auto ws = workspace(murm_slot_update_bwd_workspace_bytes(B, H, N, D, M), tk);
  ok(murm_slot_update_bwd(dt_code(tk, "token_keys"), dt_code(gk, "grad_new_sk"), B, H, N, D, M, gk.data_ptr(),
                          gk.stride(0), gk.stride(1), gk.stride(2), gv.data_ptr(), gv.stride(0), gv.stride(1),
                          gv.stride(2), tk.data_ptr(), tk.stride(0), tk.stride(1), tk.stride(2), tv.data_ptr(),
                          tv.stride(0), tv.stride(1), tv.stride(2), idx.data_ptr<int64_t>(), w.data_ptr<float>(),
                          alpha, gtk.data_ptr(), gtv.data_ptr(), gok.data_ptr(), gov.data_ptr(),
                          gw.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(tk)),
     "slot_update_backward");
  return {gtk, gtv, gok, gov, weights.scalar_type() == at::kFloat ? gw : gw.to(weights.scalar_type())};
}

// ---------------------------------------------------------------------------
void slot_diffusion(at::Tensor& slot_keys, at::Tensor& slot_values, double gamma) {
  TORCH_CHECK(slot_keys.is_cuda() && slot_keys.dim() == 4 && slot_keys.stride(3) == 1,
              "slot_keys must be a 4-D GPU tensor with a contiguous last dimension");
  TORCH_CHECK(slot_values.is_cuda() && slot_values.dim() == 4 && slot_values.stride(3) == 1,
              "slot_values must be a 4-D GPU tensor with a contiguous last dimension");
  TORCH_CHECK(slot_values.sizes() == slot_keys.sizes() && slot_values.scalar_type() == slot_keys.scalar_type(),
              "slot_values must match slot_keys");
  at::assert_no_internal_overlap(slot_keys);
  at::assert_no_internal_overlap(slot_values);
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(slot_keys.device());
  const int64_t B = slot_keys.size(0), H = slot_keys.size(1), M = slot_keys.size(2), D = slot_keys.size(3);
  ok(murm_slot_diffusion_fwd(dt_code(slot_keys, "slot_keys"), B, H, M, D, slot_keys.data_ptr(),
                             slot_keys.stride(0), slot_keys.stride(1), slot_keys.stride(2), slot_values.data_ptr(),
                             slot_values.stride(0), slot_values.stride(1), slot_values.stride(2), gamma,
                             stream_of(slot_keys)),
     "slot_diffusion");
}

std::tuple<at::Tensor, at::Tensor> slot_diffusion_backward(const at::Tensor& gk_in, const at::Tensor& gv_in,
                                                           double gamma) {
  const at::Tensor gk = rows4(gk_in, "grad_new_keys");
  const at::Tensor gv = rows4(gv_in, "grad_new_values");
  TORCH_CHECK(gv.sizes() == gk.sizes() && gv.scalar_type() == gk.scalar_type(),
              "grad_new_values must match grad_new_keys");
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(gk.device());
  const int64_t B = gk.size(0), H = gk.size(1), M = gk.size(2), D = gk.size(3);
  auto ok_ = at::empty({B, H, M, D}, gk.options());
  auto ov_ = at::empty({B, H, M, D}, gv.options());
  ok(murm_slot_diffusion_bwd(dt_code(gk, "grad_new_keys"), B, H, M, D, gk.data_ptr(), gk.stride(0), gk.stride(1),
                             gk.stride(2), gv.data_ptr(), gv.stride(0), gv.stride(1), gv.stride(2), gamma,
                             ok_.data_ptr(), ov_.data_ptr(), stream_of(gk)),
     "slot_diffusion_backward");
  return {ok_, ov_};
}

// ---------------------------------------------------------------------------
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> slot_murmurate_fwd(
    const at::Tensor& q_in, const std::optional<at::Tensor>& x_in, const std::optional<at::Tensor>& tk_in,
    const std::optional<at::Tensor>& tv_in, const at::Tensor& sk_in, const at::Tensor& sv_in, int64_t rounds,
    double alpha, double gamma, bool causal, int64_t effective_M, const std::optional<at::Tensor>& mask,
    std::optional<double> scale) {
  const at::Tensor q = rows4(q_in, "q");
  const at::Tensor sk = rows4(sk_in, "slots_k");
  const at::Tensor sv = rows4(sv_in, "slots_v");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), M = sk.size(2);
  check_slots(sk, sv, B, H, D);
  same_device(q, sk, "slots_k");
  TORCH_CHECK(tk_in.has_value() == tv_in.has_value(), "token_keys and token_values go together");
  at::Tensor x, tk, tv;
  auto tok = [&](const at::Tensor& t, const char* name) {
    at::Tensor r = rows4(t, name);
    TORCH_CHECK(r.sizes() == q.sizes() && r.scalar_type() == q.scalar_type(), name, " must match q");
    return r;
  };
  if (x_in.has_value()) x = tok(*x_in, "x");
  if (tk_in.has_value()) { tk = tok(*tk_in, "token_keys"); tv = tok(*tv_in, "token_values"); }
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  at::Tensor mk;
  if (mask.has_value()) mk = bhnm(*mask, at::kByte, B, H, N, M, q, "mask");
  const bool shared = !tk.defined();
  auto out = at::empty_like(x.defined() ? x : q);
  auto weights = at::empty({B, H, N, KN}, q.options().dtype(at::kFloat));
  auto indices = at::empty({B, H, N, KN}, q.options().dtype(at::kLong));
  auto ws = workspace(murm_murmurate_workspace_bytes(B, H, N, D, M, (int)rounds, shared ? 1 : 0), q);
  ok(murm_murmurate_fwd(
         dt_code(q, "q"), dt_code(sk, "slots_k"), B, H, N, D, M, (int)rounds, alpha, gamma, causal ? 1 : 0,
         (int)effective_M, scale.has_value() ? *scale : 0.0, q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
         x.defined() ? x.data_ptr() : nullptr, x.defined() ? x.stride(0) : 0, x.defined() ? x.stride(1) : 0,
         x.defined() ? x.stride(2) : 0, shared ? nullptr : tk.data_ptr(), shared ? 0 : tk.stride(0),
         shared ? 0 : tk.stride(1), shared ? 0 : tk.stride(2), shared ? nullptr : tv.data_ptr(),
         shared ? 0 : tv.stride(0), shared ? 0 : tv.stride(1), shared ? 0 : tv.stride(2), sk.data_ptr(),
         sk.stride(0), sk.stride(1), sk.stride(2), sv.data_ptr(), sv.stride(0), sv.stride(1), sv.stride(2),
         mk.defined() ? (const uint8_t*)mk.data_ptr() : nullptr, mk.defined() ? mk.stride(0) : 0,
         mk.defined() ? mk.stride(1) : 0, mk.defined() ? mk.stride(2) : 0, mk.defined() ? mk.stride(3) : 0,
         out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), indices.data_ptr<int64_t>(),
         weights.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(q)),
     "slot_murmurate");
  return {out, indices, weights, ws};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> slot_murmurate_bwd(
    const at::Tensor& go_in, const std::optional<at::Tensor>& gw_in, const at::Tensor& q_in,
    const std::optional<at::Tensor>& tk_in, const std::optional<at::Tensor>& tv_in, const at::Tensor& sk_in,
    const at::Tensor& weights_in, const at::Tensor& ws, int64_t rounds, double alpha, double gamma,
    std::optional<double> scale, bool x_given) {
  const at::Tensor q = rows4(q_in, "q");
  const at::Tensor go = rows4(go_in, "grad_out");
  TORCH_CHECK(go.sizes() == q.sizes() && go.scalar_type() == q.scalar_type(), "grad_out must match q");
  TORCH_CHECK(sk_in.dim() == 4, "slots_k must be 4-D");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), M = sk_in.size(2);
  TORCH_CHECK(tk_in.has_value() == tv_in.has_value(), "token_keys and token_values go together");
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  const bool shared = !tk_in.has_value();
  at::Tensor tk, tv;
  if (!shared) { tk = rows4(*tk_in, "token_keys"); tv = rows4(*tv_in, "token_values"); }
  const at::Tensor w = w_tensor(weights_in, B, H, N);
  at::Tensor gw;
  if (gw_in.has_value() && gw_in->defined()) gw = w_tensor(*gw_in, B, H, N);
  auto gq = at::empty_like(q);
  at::Tensor gtk = shared ? at::empty({0}, q.options()) : at::empty_like(tk);
  at::Tensor gtv = shared ? at::empty({0}, q.options()) : at::empty_like(tv);
  auto gsk = at::empty({B, H, M, D}, sk_in.options());
  auto gsv = at::empty({B, H, M, D}, sk_in.options());
  auto bws = workspace(murm_murmurate_bwd_workspace_bytes(B, H, N, D, M, (int)rounds, shared ? 1 : 0), q);
  ok(murm_murmurate_bwd(
         dt_code(q, "q"), dt_code(sk_in, "slots_k"), B, H, N, D, M, (int)rounds, alpha, gamma,
         scale.has_value() ? *scale : 0.0, x_given ? 1 : 0, go.data_ptr(), go.stride(0), go.stride(1),
         go.stride(2), gw.defined() ? gw.data_ptr<float>() : nullptr, q.data_ptr(), q.stride(0), q.stride(1),
         q.stride(2), shared ? nullptr : tk.data_ptr(), shared ? 0 : tk.stride(0), shared ? 0 : tk.stride(1),
         shared ? 0 : tk.stride(2), shared ? nullptr : tv.data_ptr(), shared ? 0 : tv.stride(0),
         shared ? 0 : tv.stride(1), shared ? 0 : tv.stride(2), w.data_ptr<float>(), ws.data_ptr(),
         (size_t)ws.numel(), gq.data_ptr(), gq.stride(0), gq.stride(1), gq.stride(2),
         shared ? nullptr : gtk.data_ptr(), shared ? 0 : gtk.stride(0), shared ? 0 : gtk.stride(1),
         shared ? 0 : gtk.stride(2), shared ? nullptr : gtv.data_ptr(), shared ? 0 : gtv.stride(0),
         shared ? 0 : gtv.stride(1), shared ? 0 : gtv.stride(2), gsk.data_ptr(), gsv.data_ptr(),
         bws.data_ptr(), (size_t)bws.numel(), stream_of(q)),
     "slot_murmurate backward");
  return {gq, gtk, gtv, gsk, gsv};
}

// ---------------------------------------------------------------------------
at::Tensor slot_select_fwd(const at::Tensor& query_in, const at::Tensor& slot_keys_in,
                           const std::optional<at::Tensor>& mask, bool causal,
                           const std::optional<at::Tensor>& position_bias, int64_t effective_M) {
  const at::Tensor q = rows4(query_in, "query");
  const at::Tensor sk = rows4(slot_keys_in, "slot_keys");
  same_device(q, sk, "slot_keys");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), M = sk.size(2);
  check_slots(sk, sk, B, H, D);
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  at::Tensor mk, bs;
  if (mask.has_value()) mk = bhnm(*mask, at::kByte, B, H, N, M, q, "mask");
  if (position_bias.has_value()) bs = bhnm(*position_bias, at::kFloat, B, H, N, M, q, "position_bias");
  auto indices = at::empty({B, H, N, KN}, q.options().dtype(at::kLong));
  auto ws = workspace(murm_select_attend_workspace_bytes(B, H, N, D, M), q);
  ok(murm_select_fwd(dt_code(q, "query"), dt_code(sk, "slot_keys"), B, H, N, D, M, q.data_ptr(), q.stride(0),
                     q.stride(1), q.stride(2), sk.data_ptr(), sk.stride(0), sk.stride(1), sk.stride(2),
                     mk.defined() ? (const uint8_t*)mk.data_ptr() : nullptr, mk.defined() ? mk.stride(0) : 0,
                     mk.defined() ? mk.stride(1) : 0, mk.defined() ? mk.stride(2) : 0,
                     mk.defined() ? mk.stride(3) : 0, bs.defined() ? bs.data_ptr<float>() : nullptr,
                     bs.defined() ? bs.stride(0) : 0, bs.defined() ? bs.stride(1) : 0,
                     bs.defined() ? bs.stride(2) : 0, bs.defined() ? bs.stride(3) : 0, causal ? 1 : 0,
                     (int)effective_M, indices.data_ptr<int64_t>(), ws.data_ptr(), (size_t)ws.numel(),
                     stream_of(q)),
     "slot_select");
  return indices;
}

std::tuple<at::Tensor, at::Tensor> slot_attend_fwd(const at::Tensor& query_in, const at::Tensor& slot_keys_in,
                                                   const at::Tensor& slot_values_in, const at::Tensor& indices_in,
                                                   std::optional<double> scale) {
  const at::Tensor q = rows4(query_in, "query");
  const at::Tensor sk = rows4(slot_keys_in, "slot_keys");
  const at::Tensor sv = rows4(slot_values_in, "slot_values");
  same_device(q, sk, "slot_keys");
  same_device(q, sv, "slot_values");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), M = sk.size(2);
  check_slots(sk, sv, B, H, D);
  at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(q.device());
  const at::Tensor idx = idx_tensor(indices_in, B, H, N);
  auto out = at::empty({B, H, N, D}, q.options());
  auto weights = at::empty({B, H, N, KN}, q.options().dtype(at::kFloat));
  auto ws = workspace(murm_select_attend_workspace_bytes(B, H, N, D, M), q);
  ok(murm_attend_fwd(dt_code(q, "query"), dt_code(sk, "slot_keys"), B, H, N, D, M, q.data_ptr(), q.stride(0),
                     q.stride(1), q.stride(2), sk.data_ptr(), sk.stride(0), sk.stride(1), sk.stride(2),
                     sv.data_ptr(), sv.stride(0), sv.stride(1), sv.stride(2), idx.data_ptr<int64_t>(),
                     scale.has_value() ? *scale : 0.0, out.data_ptr(), out.stride(0), out.stride(1),
                     out.stride(2), weights.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), stream_of(q)),
     "slot_attend");
  return {out, weights};
}
