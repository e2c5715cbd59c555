"""Python API and autograd for Murmurative Attention on MI355X.

Mirrors src/murmurative/ops.py of the reference: the same public functions,
arguments, defaults, autograd Functions and error types, dispatched to the
HIP kernels behind ``torch.ops.murmurative_attention``.  Differences:

* bf16, fp16 and fp32 tensors are accepted (the reference takes fp16 only,
  ops.py:41-48); other dtypes raise TypeError.
* ``slot_select`` / ``slot_attend`` run on the GPU kernels (the reference
  always evaluates them with ATen, ops.py:215-244); CPU tensors need
  ``use_reference=True``, which selects the eager path explicitly.
* ``slot_murmurate`` also accepts the README call form
  ``slot_murmurate(q, slots_k, slots_v, rounds=3, top_k=7, causal=False)
  -> (out, indices, weights)`` (README.md:61-69, 95-103), dispatched on
  ``q.dim() == 4``.  All rounds run in one fused forward op and one fused
  backward op; the gradient through the slot update into the softmax weights
  is included (the reference CUDA backward drops it).
* Diffusion after an update reads the post-update neighbours
  (reference.py:188-189) whichever update/diffuse entry is used.
"""

from typing import Callable, Optional, Tuple

import torch

from .reference import (  # noqa: F401  (re-exported names)
    slot_attend_reference,
    slot_diffusion_reference,
    slot_murmurate_reference,
    slot_select_reference,
    slot_update_reference,
)

K_NEIGHBORS = 7
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_has_hip_kernels = None


def _check_hip_kernels() -> bool:
    """Load the HIP extension once; raises RuntimeError without GPU or build."""
    global _has_hip_kernels
    if _has_hip_kernels is not None:
        return _has_hip_kernels
    from ._hip_kernels import ensure_compiled
    ensure_compiled()
    _has_hip_kernels = True
    return True


def _get_lib():
    _check_hip_kernels()
    try:
        return torch.ops.murmurative_attention
    except (AttributeError, RuntimeError) as e:
        raise ImportError(
            "HIP kernel namespace 'murmurative_attention' is not available; build the extension "
            "(murmurative-attention_amd/build.py) or use murmurative.reference.") from e


def _ensure_dtype(tensor: torch.Tensor, name: str) -> torch.Tensor:
    if tensor.dtype not in _DTYPES:
        raise TypeError(
            f"HIP kernels take float16, bfloat16 or float32 tensors, but {name} has dtype "
            f"{tensor.dtype}. Pass use_reference=True for other dtypes.")
    return tensor


def _ensure_gpu(tensor: torch.Tensor, name: str) -> torch.Tensor:
    if not tensor.is_cuda:
        raise RuntimeError(
            f"{name} is on {tensor.device}; the HIP kernels need GPU tensors "
            f"(use_reference=True selects the eager PyTorch path).")
    return tensor


def _gpu_inputs(**tensors):
    for name, t in tensors.items():
        if t is not None:
            _ensure_gpu(t, name)
            _ensure_dtype(t, name)


# ---------------------------------------------------------------------------
# Autograd Functions (reference ops.py:55-208)
# ---------------------------------------------------------------------------

class _SlotSelectAttend(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, slot_keys, slot_values, mask, causal, position_bias, scale, effective_M):
        lib = _get_lib()
        output, weights, indices = lib.slot_select_attend(
            query, slot_keys, slot_values, mask, causal, position_bias, scale, effective_M)
        ctx.save_for_backward(query, slot_keys, slot_values, indices, weights)
        ctx.scale = scale
        ctx.mark_non_differentiable(indices)
        return output, weights, indices

    @staticmethod
    def backward(ctx, grad_output, grad_weights, grad_indices):
        query, slot_keys, slot_values, indices, weights = ctx.saved_tensors
        lib = _get_lib()
        if grad_output is None:
            grad_output = torch.zeros_like(query)
        if grad_weights is None:
            grad_weights = torch.zeros_like(weights)
        gq, gsk, gsv = lib.slot_select_attend_backward(
            grad_output.contiguous(), grad_weights.contiguous(), query, slot_keys, slot_values,
            indices, weights, ctx.scale)
        return gq, gsk, gsv, None, None, None, None, None


class _SlotAttend(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, slot_keys, slot_values, indices, scale):
        lib = _get_lib()
        output, weights = lib.slot_attend_fwd(query, slot_keys, slot_values, indices, scale)
        ctx.save_for_backward(query, slot_keys, slot_values, indices, weights)
        ctx.scale = scale
        return output, weights

    @staticmethod
    def backward(ctx, grad_output, grad_weights):
        query, slot_keys, slot_values, indices, weights = ctx.saved_tensors
        lib = _get_lib()
        if grad_output is None:
            grad_output = torch.zeros_like(query)
        if grad_weights is None:
            grad_weights = torch.zeros_like(weights)
        gq, gsk, gsv = lib.slot_select_attend_backward(
            grad_output.contiguous(), grad_weights.contiguous(), query, slot_keys, slot_values,
            indices, weights, ctx.scale)
        return gq, gsk, gsv, None, None


class _SlotUpdate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, token_keys, token_values, slot_keys, slot_values, indices, weights, alpha):
        lib = _get_lib()
        ctx.save_for_backward(token_keys, token_values, indices, weights)
        ctx.alpha = alpha
        ctx.mark_dirty(slot_keys, slot_values)
        lib.slot_update(slot_keys, slot_values, token_keys, token_values, indices, weights, alpha)
        return slot_keys, slot_values

    @staticmethod
    def backward(ctx, grad_new_sk, grad_new_sv):
        token_keys, token_values, indices, weights = ctx.saved_tensors
        lib = _get_lib()
        gtk, gtv, gsk, gsv, gw = lib.slot_update_backward(
            grad_new_sk.contiguous(), grad_new_sv.contiguous(), token_keys, token_values, indices,
            weights, ctx.alpha)
        return gtk, gtv, gsk, gsv, None, gw, None


class _SlotDiffusion(torch.autograd.Function):
    @staticmethod
    def forward(ctx, slot_keys, slot_values, gamma):
        lib = _get_lib()
        ctx.gamma = gamma
        ctx.mark_dirty(slot_keys, slot_values)
        lib.slot_diffusion(slot_keys, slot_values, gamma)
        return slot_keys, slot_values

    @staticmethod
    def backward(ctx, grad_new_sk, grad_new_sv):
        lib = _get_lib()
        gk, gv = lib.slot_diffusion_backward(grad_new_sk.contiguous(), grad_new_sv.contiguous(), ctx.gamma)
        return gk, gv, None


class _SlotUpdateDiffuse(torch.autograd.Function):
    """Update then diffusion in place; backward chains the two adjoints (ops.py:157-208)."""

    @staticmethod
    def forward(ctx, token_keys, token_values, slot_keys, slot_values, indices, weights, alpha, gamma):
        lib = _get_lib()
        ctx.save_for_backward(token_keys, token_values, indices, weights)
        ctx.alpha = alpha
        ctx.gamma = gamma
        ctx.mark_dirty(slot_keys, slot_values)
        lib.slot_update_diffuse(slot_keys, slot_values, token_keys, token_values, indices, weights,
                                alpha, gamma)
        return slot_keys, slot_values

    @staticmethod
    def backward(ctx, grad_new_sk, grad_new_sv):
        token_keys, token_values, indices, weights = ctx.saved_tensors
        lib = _get_lib()
        gk, gv = lib.slot_diffusion_backward(grad_new_sk.contiguous(), grad_new_sv.contiguous(), ctx.gamma)
        gtk, gtv, gsk, gsv, gw = lib.slot_update_backward(
            gk, gv, token_keys, token_values, indices, weights, ctx.alpha)
        return gtk, gtv, gsk, gsv, None, gw, None, None


class _SlotMurmurate(torch.autograd.Function):
    """All rounds in one fused forward and one fused backward op.

    Inputs: q (selection queries), x (residual base or None = q), token keys
    and values (None = q), slots.  Outputs: (out, last indices, last weights).
    """

    @staticmethod
    def forward(ctx, q, x, tk, tv, slot_keys, slot_values, rounds, alpha, gamma, causal, effective_M,
                mask, scale):
        lib = _get_lib()
        out, indices, weights, ws = lib.slot_murmurate_fwd(
            q, x, tk, tv, slot_keys, slot_values, rounds, alpha, gamma, causal, effective_M, mask, scale)
        ctx.set_materialize_grads(False)  # unused outputs need no zero-filled gradients
        ctx.save_for_backward(q, tk, tv, slot_keys, weights)
        ctx.ws = ws
        ctx.cfg = (rounds, alpha, gamma, scale, x is not None)
        ctx.mark_non_differentiable(indices)
        return out, indices, weights

    @staticmethod
    def backward(ctx, grad_out, grad_indices, grad_weights):
        q, tk, tv, slot_keys, weights = ctx.saved_tensors
        rounds, alpha, gamma, scale, x_given = ctx.cfg
        lib = _get_lib()
        if grad_out is None:
            grad_out = torch.zeros_like(q)
        gq, gtk, gtv, gsk, gsv = lib.slot_murmurate_bwd(
            grad_out, grad_weights, q, tk, tv, slot_keys, weights, ctx.ws, rounds, alpha, gamma, scale,
            x_given)
        gx = grad_out if x_given else None
        if tk is None:
            gtk = gtv = None
        return gq, gx, gtk, gtv, gsk, gsv, None, None, None, None, None, None, None


# ---------------------------------------------------------------------------
# Python API (reference ops.py:215-422)
# ---------------------------------------------------------------------------

def slot_select(query: torch.Tensor, slot_keys: torch.Tensor, mask: Optional[torch.Tensor] = None,
                causal: bool = False, position_bias: Optional[torch.Tensor] = None,
                use_reference: bool = False) -> torch.Tensor:
    """Top-7 slot indices per token, sorted by descending score (int64 [B,H,N,7])."""
    if use_reference:
        return slot_select_reference(query, slot_keys, mask, causal, position_bias)
    _gpu_inputs(query=query, slot_keys=slot_keys)
    return _get_lib().slot_select_fwd(query, slot_keys, mask, causal, position_bias, 0)


def slot_attend(query: torch.Tensor, slot_keys: torch.Tensor, slot_values: torch.Tensor,
                indices: torch.Tensor, scale: Optional[float] = None,
                use_reference: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax attention over the given 7 slots per token; returns (out, float32 weights)."""
    if use_reference:
        return slot_attend_reference(query, slot_keys, slot_values, indices, scale)
    _gpu_inputs(query=query, slot_keys=slot_keys, slot_values=slot_values)
    return _SlotAttend.apply(query, slot_keys, slot_values, indices, scale)


def slot_select_attend(query: torch.Tensor, slot_keys: torch.Tensor, slot_values: torch.Tensor,
                       mask: Optional[torch.Tensor] = None, causal: bool = False,
                       position_bias: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                       effective_M: int = 0, use_reference: bool = False
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused selection + attention; returns (out, weights, indices) like ops.py:247-278."""
    M = slot_keys.shape[2]
    em = effective_M if effective_M > 0 else M
    em = min(em, M)
    if use_reference:
        indices = slot_select_reference(query, slot_keys, mask=mask, causal=causal,
                                        position_bias=position_bias,
                                        effective_M=em if effective_M > 0 else None)
        output, weights = slot_attend_reference(query, slot_keys, slot_values, indices, scale)
        return output, weights, indices
    _check_hip_kernels()
    _gpu_inputs(query=query, slot_keys=slot_keys, slot_values=slot_values, position_bias=position_bias)
    return _SlotSelectAttend.apply(query, slot_keys, slot_values, mask, causal, position_bias, scale, em)


def slot_update(token_keys: torch.Tensor, token_values: torch.Tensor, slot_keys: torch.Tensor,
                slot_values: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor,
                alpha: float = 0.9, use_reference: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """EMA write-back into the selected slots (in place on the HIP path)."""
    if use_reference:
        return slot_update_reference(token_keys, token_values, slot_keys, slot_values, indices, weights, alpha)
    _check_hip_kernels()
    _gpu_inputs(token_keys=token_keys, token_values=token_values, slot_keys=slot_keys,
                slot_values=slot_values)
    if slot_keys.requires_grad and slot_keys.is_leaf:
        slot_keys = slot_keys.clone()
    if slot_values.requires_grad and slot_values.is_leaf:
        slot_values = slot_values.clone()
    return _SlotUpdate.apply(token_keys, token_values, slot_keys, slot_values, indices, weights, alpha)


def slot_diffusion(slot_keys: torch.Tensor, slot_values: torch.Tensor, gamma: float = 0.1,
                   use_reference: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tridiagonal Laplace diffusion along the slot axis (in place on the HIP path)."""
    if use_reference:
        return slot_diffusion_reference(slot_keys, slot_values, gamma)
    _check_hip_kernels()
    _gpu_inputs(slot_keys=slot_keys, slot_values=slot_values)
    if slot_keys.requires_grad and slot_keys.is_leaf:
        slot_keys = slot_keys.clone()
    if slot_values.requires_grad and slot_values.is_leaf:
        slot_values = slot_values.clone()
    return _SlotDiffusion.apply(slot_keys, slot_values, gamma)


def _readme_reference(q, slots_k, slots_v, rounds, causal, alpha, gamma):
    x, idx, w = q, None, None
    sk, sv = slots_k, slots_v
    for _ in range(rounds):
        idx = slot_select_reference(q, sk, causal=causal)
        a, w = slot_attend_reference(q, sk, sv, idx)
        x = x + a
        sk, sv = slot_update_reference(q, q, sk, sv, idx, w, alpha)
        sk, sv = slot_diffusion_reference(sk, sv, gamma)
    return x, idx, w


def _slot_murmurate_readme(q, slots_k, slots_v=None, rounds=3, top_k=K_NEIGHBORS, causal=False, alpha=0.9,
                           gamma=0.15, use_reference=False):
    if top_k != K_NEIGHBORS:
        raise ValueError(f"top_k must be {K_NEIGHBORS} (got {top_k})")
    if slots_v is None:
        # README.md:64-67 calls slot_murmurate(x, slots, rounds=3): the slot
        # values start at zero, as the README layer passes them (README.md:99)
        slots_v = torch.zeros_like(slots_k)
    if q.dim() != 4 or slots_k.dim() != 4 or slots_v.dim() != 4:
        raise ValueError("q, slots_k and slots_v must be 4-D ([B,H,N,D] and [B,H,M,D])")
    if use_reference:
        return _readme_reference(q, slots_k, slots_v, rounds, causal, alpha, gamma)
    _check_hip_kernels()
    _gpu_inputs(q=q, slots_k=slots_k, slots_v=slots_v)
    return _SlotMurmurate.apply(q, None, None, None, slots_k, slots_v, int(rounds), float(alpha),
                                float(gamma), bool(causal), 0, None, None)


def _slot_murmurate_legacy(x, q_proj, k_proj, v_proj, slot_k_emb, slot_v_emb, num_heads=8, rounds=3,
                           alpha=0.9, gamma=0.15, causal=False, mask=None, position_bias_fn=None,
                           use_reference=False, use_dynamic_m=True, slot_ratio=8,
                           use_fused_update_diffuse=True):
    if not use_reference:
        _check_hip_kernels()
    B, N, D = x.shape
    H = num_heads
    if D % H != 0:
        raise ValueError(f"Embedding dimension D ({D}) must be divisible by num_heads ({H})")
    Dh = D // H
    M = slot_k_emb.shape[1]
    effective_M = M
    if use_dynamic_m:
        effective_M = min(M, max(32, (N + slot_ratio - 1) // slot_ratio))
    if use_reference:
        return slot_murmurate_reference(x, q_proj, k_proj, v_proj, slot_k_emb, slot_v_emb, num_heads=H,
                                        rounds=rounds, alpha=alpha, gamma=gamma, causal=causal, mask=mask,
                                        position_bias_fn=position_bias_fn, use_dynamic_m=use_dynamic_m,
                                        slot_ratio=slot_ratio)
    _gpu_inputs(x=x, q_proj=q_proj, k_proj=k_proj, v_proj=v_proj, slot_k_emb=slot_k_emb,
                slot_v_emb=slot_v_emb)

    def heads(t):
        return t.view(B, N, H, Dh).permute(0, 2, 1, 3)

    x_h, q_h, k_h, v_h = heads(x), heads(q_proj), heads(k_proj), heads(v_proj)
    slot_k = slot_k_emb.unsqueeze(0).expand(B, H, M, Dh)
    slot_v = slot_v_emb.unsqueeze(0).expand(B, H, M, Dh)
    if position_bias_fn is None:
        out_h, _, _ = _SlotMurmurate.apply(q_h, x_h, k_h, v_h, slot_k, slot_v, int(rounds), float(alpha),
                                           float(gamma), bool(causal), int(effective_M), mask, None)
    else:
        # a bias recomputed from x every round cannot live inside the fused op:
        # run the rounds here, one fused select+attend and one update+diffuse each
        out_h = x_h
        slot_k, slot_v = slot_k.clone(), slot_v.clone()
        for _ in range(rounds):
            pb = position_bias_fn(out_h)
            attn_out, attn_w, indices = _SlotSelectAttend.apply(
                q_h, slot_k, slot_v, mask, causal, pb.contiguous() if pb is not None else None, None,
                effective_M)
            out_h = out_h + attn_out
            slot_k, slot_v = _SlotUpdateDiffuse.apply(k_h, v_h, slot_k.clone(), slot_v.clone(), indices,
                                                      attn_w, alpha, gamma)
    return out_h.permute(0, 2, 1, 3).reshape(B, N, D)


def slot_murmurate(*args, **kwargs):
    """Murmurative Attention: R rounds of select -> attend -> update -> diffuse.

    README form (q.dim() == 4):
        slot_murmurate(q, slots_k, slots_v=None, rounds=3, top_k=7, causal=False,
                       alpha=0.9, gamma=0.15, use_reference=False)
        -> (out [B,H,N,D], indices int64 [B,H,N,7], weights float32 [B,H,N,7])
    with out = q + sum over rounds of the attention output, and indices and
    weights of the last round.  slots_v=None starts the slot values at zero
    (the README's verify call, slot_murmurate(x, slots, rounds=3)).

    Projection form (x.dim() == 3, reference ops.py:330-348):
        slot_murmurate(x, q_proj, k_proj, v_proj, slot_k_emb, slot_v_emb,
                       num_heads=8, rounds=3, alpha=0.9, gamma=0.15, causal=False,
                       mask=None, position_bias_fn=None, use_reference=False,
                       use_dynamic_m=True, slot_ratio=8, use_fused_update_diffuse=True)
        -> [B,N,D]
    """
    first = args[0] if args else kwargs.get("q", kwargs.get("x"))
    if first is None:
        raise TypeError("slot_murmurate needs a query / input tensor")
    if first.dim() == 4:
        if "q" not in kwargs and args:
            return _slot_murmurate_readme(*args, **kwargs)
        return _slot_murmurate_readme(**kwargs)
    return _slot_murmurate_legacy(*args, **kwargs)
