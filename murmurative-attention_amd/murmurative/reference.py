"""Eager PyTorch formulation of Murmurative Attention (the ``*_reference`` API).

Same names, arguments and results as src/murmurative/reference.py of the
reference project.  These run on whatever device their inputs live on, with
ATen ops; the package uses them only when a caller passes
``use_reference=True`` or calls a ``*_reference`` function directly.  The HIP
path never falls back to them.
"""

import math
from typing import Callable, Optional, Tuple

import torch

_K = 7


def _selection_scores(query, slot_keys, mask, causal, position_bias, effective_M):
    N, M = query.shape[2], slot_keys.shape[2]
    em = M if effective_M is None else min(int(effective_M), M)
    s = torch.matmul(query, slot_keys.transpose(-1, -2))
    if position_bias is not None:
        s = s + position_bias
    if mask is not None:
        s = s.masked_fill(mask == 0, float("-inf"))
    slots = torch.arange(M, device=query.device)
    if causal:
        s = s.masked_fill(slots.view(1, M) > torch.arange(N, device=query.device).view(N, 1), float("-inf"))
    if em < M:
        s = s.masked_fill(slots >= em, float("-inf"))
    return s


def slot_select_reference(query: torch.Tensor, slot_keys: torch.Tensor, mask: Optional[torch.Tensor] = None,
                          causal: bool = False, position_bias: Optional[torch.Tensor] = None,
                          effective_M: Optional[int] = None) -> torch.Tensor:
    """Top-7 slots per token by unscaled q.sk (+bias), masked, sorted descending (reference.py:6-39)."""
    s = _selection_scores(query, slot_keys, mask, causal, position_bias, effective_M)
    return torch.topk(s, k=_K, dim=-1, sorted=True).indices.to(torch.int64)


def slot_attend_reference(query: torch.Tensor, slot_keys: torch.Tensor, slot_values: torch.Tensor,
                          indices: torch.Tensor, scale: Optional[float] = None
                          ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax over the selected slots' scaled scores; returns (out, float32 weights) (reference.py:42-68)."""
    B, H, N, D = query.shape
    M, k = slot_keys.shape[2], indices.shape[-1]
    c = 1.0 / math.sqrt(D) if scale is None else scale
    flat = indices.clamp(0, M - 1).reshape(B, H, N * k, 1).expand(-1, -1, -1, D)
    keys = torch.gather(slot_keys, 2, flat).reshape(B, H, N, k, D)
    w = torch.softmax(torch.matmul(keys, query.unsqueeze(-1)).squeeze(-1) * c, dim=-1)
    vals = torch.gather(slot_values, 2, flat).reshape(B, H, N, k, D)
    out = torch.matmul(w.unsqueeze(-2), vals).squeeze(-2)
    return out, w.to(torch.float32)


def slot_update_reference(token_keys: torch.Tensor, token_values: torch.Tensor, slot_keys: torch.Tensor,
                          slot_values: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor,
                          alpha: float = 0.9) -> Tuple[torch.Tensor, torch.Tensor]:
    """EMA of the weighted token mean into every used slot, float32 sums (reference.py:71-115)."""
    B, H, N, D = token_keys.shape
    M, k = slot_keys.shape[2], indices.shape[-1]
    flat = indices.clamp(0, M - 1).reshape(B, H, N * k)
    w = weights.float().reshape(B, H, N * k, 1)

    def sums(t):
        rep = t.float().unsqueeze(3).expand(B, H, N, k, D).reshape(B, H, N * k, D)
        z = torch.zeros(B, H, M, D, device=t.device, dtype=torch.float32)
        return z.scatter_add_(2, flat.unsqueeze(-1).expand(-1, -1, -1, D), rep * w)

    K, V = sums(token_keys), sums(token_values)
    W = torch.zeros(B, H, M, 1, device=token_keys.device, dtype=torch.float32).scatter_add_(
        2, flat.unsqueeze(-1), w)
    used = W > 0
    old_k, old_v = slot_keys.float(), slot_values.float()
    new_k = torch.where(used, alpha * old_k + (1.0 - alpha) * K / (W + 1e-8), old_k)
    new_v = torch.where(used, alpha * old_v + (1.0 - alpha) * V / (W + 1e-8), old_v)
    return new_k.type_as(slot_keys), new_v.type_as(slot_values)


def slot_diffusion_reference(slot_keys: torch.Tensor, slot_values: torch.Tensor, gamma: float = 0.1
                             ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Jacobi tridiagonal stencil on rows 1..M-2, endpoints copied (reference.py:118-135)."""
    def step(x):
        M = x.shape[2]
        y = x.clone()
        if M >= 3:
            y[:, :, 1:M - 1] += gamma * (x[:, :, :M - 2] + x[:, :, 2:] - 2 * x[:, :, 1:M - 1])
        return y
    return step(slot_keys), step(slot_values)


def slot_murmurate_reference(x: torch.Tensor, q_proj: torch.Tensor, k_proj: torch.Tensor, v_proj: torch.Tensor,
                             slot_k_emb: torch.Tensor, slot_v_emb: torch.Tensor, num_heads: int = 8,
                             rounds: int = 3, alpha: float = 0.9, gamma: float = 0.15, causal: bool = False,
                             mask: Optional[torch.Tensor] = None,
                             position_bias_fn: Optional[Callable[[torch.Tensor], torch.Tensor]] = None,
                             use_dynamic_m: bool = False, slot_ratio: int = 8) -> torch.Tensor:
    """R rounds of select/attend/residual/update/diffuse on [B,N,D] inputs (reference.py:138-192)."""
    B, N, D = x.shape
    H = num_heads
    if D % H != 0:
        raise ValueError(f"Embedding dimension D ({D}) must be divisible by num_heads ({H})")
    Dh = D // H

    def heads(t):
        return t.view(B, N, H, Dh).permute(0, 2, 1, 3)

    xh, qh, kh, vh = heads(x), heads(q_proj), heads(k_proj), heads(v_proj)
    M = slot_k_emb.shape[1]
    sk = slot_k_emb.unsqueeze(0).expand(B, -1, -1, -1).contiguous()
    sv = slot_v_emb.unsqueeze(0).expand(B, -1, -1, -1).contiguous()
    em = min(M, max(32, (N + slot_ratio - 1) // slot_ratio)) if use_dynamic_m else None
    for _ in range(rounds):
        pb = position_bias_fn(xh) if position_bias_fn is not None else None
        idx = slot_select_reference(qh, sk, mask=mask, causal=causal, position_bias=pb, effective_M=em)
        a, w = slot_attend_reference(qh, sk, sv, idx)
        xh = xh + a
        sk, sv = slot_update_reference(kh, vh, sk, sv, idx, w, alpha)
        sk, sv = slot_diffusion_reference(sk, sv, gamma)
    return xh.permute(0, 2, 1, 3).contiguous().view(B, N, D)
