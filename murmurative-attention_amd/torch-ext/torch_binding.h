#pragma once

#include <ATen/ATen.h>

#include <optional>
#include <tuple>

// Op implementations (wrappers.cpp).  The first seven keep the reference's
// schemas (torch-ext/torch_binding.cpp:7-32 of beaglabs/murmurative-attention);
// slot_murmurate_fwd / slot_murmurate_bwd are the fused multi-round pair.

std::tuple<at::Tensor, at::Tensor, at::Tensor> slot_select_attend(
    const at::Tensor& query, const at::Tensor& slot_keys, const at::Tensor& slot_values,
    const std::optional<at::Tensor>& mask, bool causal, const std::optional<at::Tensor>& position_bias,
    std::optional<double> scale, int64_t effective_M);

std::tuple<at::Tensor, at::Tensor, at::Tensor> slot_select_attend_backward(
    const at::Tensor& grad_output, const at::Tensor& grad_weights, const at::Tensor& query,
    const at::Tensor& slot_keys, const at::Tensor& slot_values, const at::Tensor& indices,
    const at::Tensor& weights, std::optional<double> scale);

void slot_update(at::Tensor& slot_keys, at::Tensor& slot_values, const at::Tensor& token_keys,
                 const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights,
                 double alpha);

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> slot_update_backward(
    const at::Tensor& grad_new_sk, const at::Tensor& grad_new_sv, const at::Tensor& token_keys,
    const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights, double alpha);

void slot_diffusion(at::Tensor& slot_keys, at::Tensor& slot_values, double gamma);

std::tuple<at::Tensor, at::Tensor> slot_diffusion_backward(const at::Tensor& grad_new_keys,
                                                           const at::Tensor& grad_new_values, double gamma);

void slot_update_diffuse(at::Tensor& slot_keys, at::Tensor& slot_values, const at::Tensor& token_keys,
                         const at::Tensor& token_values, const at::Tensor& indices, const at::Tensor& weights,
                         double alpha, double gamma);

at::Tensor slot_select_fwd(const at::Tensor& query, const at::Tensor& slot_keys,
                           const std::optional<at::Tensor>& mask, bool causal,
                           const std::optional<at::Tensor>& position_bias, int64_t effective_M);

std::tuple<at::Tensor, at::Tensor> slot_attend_fwd(const at::Tensor& query, const at::Tensor& slot_keys,
                                                   const at::Tensor& slot_values, const at::Tensor& indices,
                                                   std::optional<double> scale);

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> slot_murmurate_fwd(
    const at::Tensor& q, const std::optional<at::Tensor>& x, const std::optional<at::Tensor>& token_keys,
    const std::optional<at::Tensor>& token_values, const at::Tensor& slot_keys, const at::Tensor& slot_values,
    int64_t rounds, double alpha, double gamma, bool causal, int64_t effective_M,
    const std::optional<at::Tensor>& mask, std::optional<double> scale);

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> slot_murmurate_bwd(
    const at::Tensor& grad_out, const std::optional<at::Tensor>& grad_weights, const at::Tensor& q,
    const std::optional<at::Tensor>& token_keys, const std::optional<at::Tensor>& token_values,
    const at::Tensor& slot_keys, const at::Tensor& weights, const at::Tensor& workspace, int64_t rounds,
    double alpha, double gamma, std::optional<double> scale, bool x_given);
