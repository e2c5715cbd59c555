#include <torch/library.h>

#include "registration.h"
#include "torch_binding.h"

// The seven schemas of the reference namespace, unchanged
// (torch-ext/torch_binding.cpp:6-33 of beaglabs/murmurative-attention), plus
// the fused multi-round forward/backward pair used by slot_murmurate.
TORCH_LIBRARY(murmurative_attention, ops) {
  ops.def(
      "slot_select_attend(Tensor query, Tensor slot_keys, Tensor slot_values, "
      "Tensor? mask, bool causal, Tensor? position_bias, float? scale, int effective_M) -> "
      "(Tensor, Tensor, Tensor)");
  ops.def(
      "slot_select_attend_backward(Tensor grad_output, Tensor grad_weights, "
      "Tensor query, Tensor slot_keys, Tensor slot_values, Tensor indices, "
      "Tensor weights, float? scale) -> (Tensor, Tensor, Tensor)");
  ops.def(
      "slot_update(Tensor(a!) slot_keys, Tensor(b!) slot_values, "
      "Tensor token_keys, Tensor token_values, Tensor indices, "
      "Tensor weights, float alpha) -> ()");
  ops.def(
      "slot_update_backward(Tensor grad_new_sk, Tensor grad_new_sv, "
      "Tensor token_keys, Tensor token_values, Tensor indices, "
      "Tensor weights, float alpha) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  ops.def(
      "slot_diffusion(Tensor(a!) slot_keys, Tensor(b!) slot_values, "
      "float gamma) -> ()");
  ops.def(
      "slot_diffusion_backward(Tensor grad_new_keys, Tensor grad_new_values, "
      "float gamma) -> (Tensor, Tensor)");
  ops.def(
      "slot_update_diffuse(Tensor(a!) slot_keys, Tensor(b!) slot_values, "
      "Tensor token_keys, Tensor token_values, Tensor indices, "
      "Tensor weights, float alpha, float gamma) -> ()");
  ops.def(
      "slot_select_fwd(Tensor query, Tensor slot_keys, Tensor? mask, bool causal, "
      "Tensor? position_bias, int effective_M) -> Tensor");
  ops.def(
      "slot_attend_fwd(Tensor query, Tensor slot_keys, Tensor slot_values, Tensor indices, "
      "float? scale) -> (Tensor, Tensor)");
  ops.def(
      "slot_murmurate_fwd(Tensor q, Tensor? x, Tensor? token_keys, Tensor? token_values, "
      "Tensor slot_keys, Tensor slot_values, int rounds, float alpha, float gamma, bool causal, "
      "int effective_M, Tensor? mask, float? scale) -> (Tensor, Tensor, Tensor, Tensor)");
  ops.def(
      "slot_murmurate_bwd(Tensor grad_out, Tensor? grad_weights, Tensor q, Tensor? token_keys, "
      "Tensor? token_values, Tensor slot_keys, Tensor weights, Tensor workspace, int rounds, "
      "float alpha, float gamma, float? scale, bool x_given) -> "
      "(Tensor, Tensor, Tensor, Tensor, Tensor)");
}

// ROCm builds of PyTorch route HIP tensors through the CUDA dispatch key.
TORCH_LIBRARY_IMPL(murmurative_attention, CUDA, m) {
  m.impl("slot_select_attend", &slot_select_attend);
  m.impl("slot_select_attend_backward", &slot_select_attend_backward);
  m.impl("slot_update", &slot_update);
  m.impl("slot_update_backward", &slot_update_backward);
  m.impl("slot_diffusion", &slot_diffusion);
  m.impl("slot_diffusion_backward", &slot_diffusion_backward);
  m.impl("slot_update_diffuse", &slot_update_diffuse);
  m.impl("slot_select_fwd", &slot_select_fwd);
  m.impl("slot_attend_fwd", &slot_attend_fwd);
  m.impl("slot_murmurate_fwd", &slot_murmurate_fwd);
  m.impl("slot_murmurate_bwd", &slot_murmurate_bwd);
}

REGISTER_EXTENSION(TORCH_EXTENSION_NAME)
