"""CPU oracle for the ``slot_murmurate`` hot path -- TEST INFRASTRUCTURE ONLY.

This module is the parity checker.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only to check
or time the HIP path against it.  No product code imports it; the HIP path
raises when its extension is missing instead of falling back to this file.

It is a plain-PyTorch CPU restatement of the reference's algorithm
(``src/murmurative/reference.py`` in beaglabs/murmurative-attention), written
from the maths.  Every function evaluates in the dtype of its inputs; callers
upcast to float64 (parity) or float32 (golden comparison, CPU baseline).
Gradients are PyTorch autograd through these functions; ``murmurate_backward``
restates the same gradients in closed form so that the per-phase quantities of
the HIP backward (ds, dK, dW, G') can be compared one by one.

How each function is pinned (tests/test_oracle.py):
  select      -- argsort brute force on tiny inputs, special case em == 7,
                 invariants (distinct, in range, sorted), golden tie order.
  attend      -- closed-form softmax loop, sum(w) == 1, gradcheck.
  update      -- explicit per-slot loop, alpha == 1 identity, untouched slots.
  diffusion   -- explicit matrix form, gamma == 0 identity, fixed endpoints.
  murmurate_* -- golden fixtures written by tests/golden/make_golden.py from
                 the reference's own functions; gradcheck of the composite.
  murmurate_backward -- equality with autograd of murmurate_readme, which is
                 itself pinned by gradcheck.
"""

from __future__ import annotations

import math
from typing import Callable, Optional, Tuple

import torch

K_NEIGHBORS = 7  # reference.py:38 (topk k=7)


# ---------------------------------------------------------------------------
# Single-round phases (reference.py:6-135)
# ---------------------------------------------------------------------------

def masked_scores(
    q: torch.Tensor,
    sk: torch.Tensor,
    mask: Optional[torch.Tensor] = None,
    causal: bool = False,
    position_bias: Optional[torch.Tensor] = None,
    effective_M: Optional[int] = None,
) -> torch.Tensor:
    """Selection scores [B,H,N,M] with every -inf the reference applies.

    reference.py:19 (unscaled q.sk), :21-22 (+bias), :24-25 (mask==0 -> -inf),
    :27-31 (causal: slot m > token n -> -inf), :34-36 (m >= em -> -inf).
    """
    N = q.shape[2]
    M = sk.shape[2]
    em = M if effective_M is None else min(int(effective_M), M)
    s = torch.matmul(q, sk.transpose(-1, -2))
    if position_bias is not None:
        s = s + position_bias
    if mask is not None:
        s = s.masked_fill(mask == 0, float("-inf"))
    if causal:
        cm = torch.arange(M).view(1, M) > torch.arange(N).view(N, 1)
        s = s.masked_fill(cm, float("-inf"))
    if em < M:
        s = s.masked_fill(torch.arange(M) >= em, float("-inf"))
    return s


def select(q, sk, mask=None, causal=False, position_bias=None, effective_M=None,
           k: int = K_NEIGHBORS) -> torch.Tensor:
    """Top-k slot indices per token, sorted by descending masked score, int64.

    reference.py:6-39 (torch.topk(scores, k=7, sorted=True)).
    """
    s = masked_scores(q, sk, mask, causal, position_bias, effective_M)
    _, idx = torch.topk(s, k=k, dim=-1, sorted=True)
    return idx.to(torch.int64)


def attend(q, sk, sv, idx, scale: Optional[float] = None):
    """Softmax over the k gathered slot scores; returns (out, w float32-or-wider).

    reference.py:42-68: indices clamped to [0, M-1] (:56); scores use the real
    (unmasked, unbiased) q.sk times scale (default 1/sqrt(D), :53-54, :61);
    softmax over k (:63); out = sum_j w_j sv[idx_j] (:65-66).
    """
    B, H, N, D = q.shape
    M = sk.shape[2]
    k = idx.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ii = idx.clamp(0, M - 1).reshape(B, H, N * k, 1).expand(-1, -1, -1, D)
    gk = torch.gather(sk, 2, ii).reshape(B, H, N, k, D)
    logits = (gk * q.unsqueeze(3)).sum(-1) * scale
    w = torch.softmax(logits, dim=-1)
    gv = torch.gather(sv, 2, ii).reshape(B, H, N, k, D)
    out = (w.unsqueeze(-1) * gv).sum(3)
    wdt = torch.promote_types(w.dtype, torch.float32)
    return out, w.to(wdt)


def slot_sums(tk, tv, idx, w, M: int):
    """Per-slot weighted sums (K, V [B,H,M,D]) and weight totals W [B,H,M].

    reference.py:86-103: accumulate w*tk, w*tv, w into the selected slot of
    every (token, j) pair, in float32 or wider; indices clamped (:84).
    """
    B, H, N, D = tk.shape
    acc = torch.promote_types(tk.dtype, torch.float32)
    ii = idx.clamp(0, M - 1).reshape(B, H, -1)
    ww = w.to(acc).reshape(B, H, -1)
    k = idx.shape[-1]
    tk_rep = tk.to(acc).unsqueeze(3).expand(B, H, N, k, D).reshape(B, H, N * k, D)
    tv_rep = tv.to(acc).unsqueeze(3).expand(B, H, N, k, D).reshape(B, H, N * k, D)
    K = torch.zeros(B, H, M, D, dtype=acc).scatter_add(
        2, ii.unsqueeze(-1).expand(-1, -1, -1, D), tk_rep * ww.unsqueeze(-1))
    V = torch.zeros(B, H, M, D, dtype=acc).scatter_add(
        2, ii.unsqueeze(-1).expand(-1, -1, -1, D), tv_rep * ww.unsqueeze(-1))
    W = torch.zeros(B, H, M, dtype=acc).scatter_add(2, ii, ww)
    return K, V, W


def update(tk, tv, sk, sv, idx, w, alpha: float = 0.9, eps: float = 1e-8):
    """EMA write-back of the weighted token mean into every used slot.

    reference.py:71-115: mean = sum/(W + 1e-8) (:106-107); slots with W > 0
    become alpha*old + (1-alpha)*mean, the others keep their value (:105,
    :109-113); the result is cast back to the slot dtype (:115).
    """
    M = sk.shape[2]
    K, V, W = slot_sums(tk, tv, idx, w, M)
    valid = (W > 0).unsqueeze(-1)
    Wd = W.unsqueeze(-1) + eps
    skf = sk.to(K.dtype)
    svf = sv.to(V.dtype)
    nk = torch.where(valid, alpha * skf + (1.0 - alpha) * (K / Wd), skf)
    nv = torch.where(valid, alpha * svf + (1.0 - alpha) * (V / Wd), svf)
    return nk.to(sk.dtype), nv.to(sv.dtype)


def diffusion(sk, sv, gamma: float = 0.1):
    """Tridiagonal Laplace stencil on the slot axis (Jacobi form).

    reference.py:118-135: rows 1..M-2 become x_m + gamma*(x_{m-1} + x_{m+1}
    - 2 x_m) with the right-hand side read before the write; rows 0 and M-1
    are copied.
    """
    def one(x):
        M = x.shape[2]
        if M < 3:
            return x.clone()
        mid = x[:, :, 1:M - 1] + gamma * (x[:, :, 0:M - 2] + x[:, :, 2:M] - 2 * x[:, :, 1:M - 1])
        return torch.cat([x[:, :, :1], mid, x[:, :, M - 1:]], dim=2)
    return one(sk), one(sv)


def diffusion_transpose(g, gamma: float):
    """Adjoint of ``diffusion`` for one tensor [B,H,M,D] (any M >= 1)."""
    M = g.shape[2]
    if M < 3:
        return g.clone()
    out = g.clone()
    inner = g[:, :, 1:M - 1]
    out[:, :, 1:M - 1] = out[:, :, 1:M - 1] - 2 * gamma * inner
    out[:, :, 0:M - 2] = out[:, :, 0:M - 2] + gamma * inner
    out[:, :, 2:M] = out[:, :, 2:M] + gamma * inner
    return out


# ---------------------------------------------------------------------------
# Composite (reference.py:138-192 and the README call form README.md:61-69)
# ---------------------------------------------------------------------------

def dynamic_m(N: int, M: int, slot_ratio: int = 8, m_min: int = 32) -> int:
    """effective_M = min(M, max(32, ceil(N / slot_ratio))) (reference.py:172-175)."""
    return min(M, max(m_min, (N + slot_ratio - 1) // slot_ratio))


def murmurate_legacy(x, q_proj, k_proj, v_proj, slot_k_emb, slot_v_emb, num_heads=8,
                     rounds=3, alpha=0.9, gamma=0.15, causal=False, mask=None,
                     position_bias_fn: Optional[Callable] = None, use_dynamic_m=False,
                     slot_ratio=8, forced_idx=None):
    """reference.py:138-192: x, q, k, v are [B,N,D]; slot embeddings [H,M,Dh].

    Per round: select on q (:182-185), attend on q (:186), residual x += a
    (:187), update with the k and v projections (:188), diffusion of the
    post-update slots (:189).  Output [B,N,D] (:191).  ``forced_idx`` replays
    given per-round selections (see murmurate_readme).
    """
    B, N, D = x.shape
    H = num_heads
    if D % H != 0:
        raise ValueError(f"Embedding dimension D ({D}) must be divisible by num_heads ({H})")
    Dh = D // H

    def heads(t):
        return t.reshape(B, N, H, Dh).permute(0, 2, 1, 3)

    xh, qh, kh, vh = heads(x), heads(q_proj), heads(k_proj), heads(v_proj)
    M = slot_k_emb.shape[1]
    sk = slot_k_emb.unsqueeze(0).expand(B, -1, -1, -1)
    sv = slot_v_emb.unsqueeze(0).expand(B, -1, -1, -1)
    em = dynamic_m(N, M, slot_ratio) if use_dynamic_m else None
    for r in range(rounds):
        pb = position_bias_fn(xh) if position_bias_fn is not None else None
        if forced_idx is not None:
            idx = forced_idx[r].to(torch.int64)
        else:
            idx = select(qh, sk, mask=mask, causal=causal, position_bias=pb, effective_M=em)
        a, w = attend(qh, sk, sv, idx)
        xh = xh + a
        sk, sv = update(kh, vh, sk, sv, idx, w, alpha)
        sk, sv = diffusion(sk, sv, gamma)
    return xh.permute(0, 2, 1, 3).reshape(B, N, D)


def murmurate_readme(q, sk, sv, rounds=3, top_k=K_NEIGHBORS, causal=False, alpha=0.9,
                     gamma=0.15, return_trace=False, forced_idx=None):
    """README call form: slot_murmurate(q, slots_k, slots_v, rounds, top_k, causal).

    q [B,H,N,D]; slots [B,H,M,D].  This is reference.py:177-189 with
    x = q_proj = k_proj = v_proj = q per head and effective_M = M (the
    reference.py:152 default).  Returns (x_R, indices of the last round,
    weights of the last round) as README.md:67 documents.  With
    ``return_trace`` it also returns the per-round (sk, sv, idx, w, scores).
    ``forced_idx`` (one [B,H,N,7] tensor per round) replaces the top-k of each
    round: the kernel's own selections replayed, so that every other quantity
    can be compared tightly while selection is checked on its own.
    """
    if top_k != K_NEIGHBORS:
        raise ValueError("top_k must be 7")
    x = q
    trace = []
    idx = w = None
    for r in range(rounds):
        s = masked_scores(q, sk, causal=causal)
        if forced_idx is not None:
            idx = forced_idx[r].to(torch.int64)
        else:
            idx = torch.topk(s, k=top_k, dim=-1, sorted=True)[1]
        a, w = attend(q, sk, sv, idx)
        if return_trace:
            trace.append((sk, sv, idx, w, s.detach()))
        x = x + a
        sk, sv = update(q, q, sk, sv, idx, w, alpha)
        sk, sv = diffusion(sk, sv, gamma)
    if return_trace:
        return x, idx, w, trace
    return x, idx, w


def murmurate_backward(q, sk0, sv0, grad_out, grad_w_last=None, rounds=3, causal=False,
                       alpha=0.9, gamma=0.15, eps=1e-8, forced_idx=None):
    """Closed-form backward of ``murmurate_readme`` (token and slot sides).

    Per round r, with c = 1/sqrt(D), I = idx_r, g = grad_out:
      diffusion adjoint   G'  = D^T G''
      update, slot side   dK = (1-a)/(W+eps) (G'k + G'v) on used slots
                          dW = -(1-a)(K.G'k + V.G'v)/(W+eps)^2 on used slots
                          carry = a G' (used) or G' (unused)
      token side          dw_j = g.sv[I_j] + q.dK[I_j] + dW[I_j] (+ grad_w)
                          ds_j = w_j (dw_j - sum_i w_i dw_i)
                          dq  += c sum_j ds_j sk[I_j] + sum_j w_j dK[I_j]
      slot side           dsk[m] = carry_k + c sum ds q ; dsv[m] = carry_v + sum w g
    and dq gets the residual term g.  Returns (dq, dsk0, dsv0, per-round dict).
    """
    B, H, N, D = q.shape
    M = sk0.shape[2]
    c = 1.0 / math.sqrt(D)
    _, _, _, trace = murmurate_readme(q, sk0, sv0, rounds, causal=causal, alpha=alpha,
                                      gamma=gamma, return_trace=True, forced_idx=forced_idx)
    dq = grad_out.clone()
    Gk = torch.zeros_like(sk0)
    Gv = torch.zeros_like(sv0)
    per_round = []
    bidx = torch.arange(B).view(B, 1, 1, 1)
    hidx = torch.arange(H).view(1, H, 1, 1)
    for r in reversed(range(rounds)):
        sk, sv, idx, w, _ = trace[r]
        K, V, W = slot_sums(q, q, idx, w, M)
        if r == rounds - 1:
            dKk = torch.zeros_like(sk)
            dKv = torch.zeros_like(sk)
            dW = torch.zeros(B, H, M, dtype=sk.dtype)
            carry_k, carry_v = Gk, Gv
        else:
            Gpk = diffusion_transpose(Gk, gamma)
            Gpv = diffusion_transpose(Gv, gamma)
            used = (W > 0)
            inv = (1.0 - alpha) / (W + eps)
            dKk = torch.where(used.unsqueeze(-1), inv.unsqueeze(-1) * Gpk, torch.zeros_like(Gpk))
            dKv = torch.where(used.unsqueeze(-1), inv.unsqueeze(-1) * Gpv, torch.zeros_like(Gpv))
            dW = torch.where(used, -(1.0 - alpha) * ((K * Gpk).sum(-1) + (V * Gpv).sum(-1))
                             / (W + eps) ** 2, torch.zeros_like(W))
            carry_k = torch.where(used.unsqueeze(-1), alpha * Gpk, Gpk)
            carry_v = torch.where(used.unsqueeze(-1), alpha * Gpv, Gpv)
        gsv = sv[bidx, hidx, idx]          # [B,H,N,7,D]
        gsk = sk[bidx, hidx, idx]
        gdk = (dKk + dKv)[bidx, hidx, idx]
        dw = (grad_out.unsqueeze(3) * gsv).sum(-1) + (q.unsqueeze(3) * gdk).sum(-1) + dW[bidx, hidx, idx]
        if r == rounds - 1 and grad_w_last is not None:
            dw = dw + grad_w_last.to(dw.dtype)
        ds = w * (dw - (w * dw).sum(-1, keepdim=True))
        dq = dq + c * (ds.unsqueeze(-1) * gsk).sum(3) + (w.unsqueeze(-1) * gdk).sum(3)
        ii = idx.reshape(B, H, -1)
        e = ii.unsqueeze(-1).expand(-1, -1, -1, D)
        qrep = q.unsqueeze(3).expand(B, H, N, 7, D).reshape(B, H, N * 7, D)
        grep = grad_out.unsqueeze(3).expand(B, H, N, 7, D).reshape(B, H, N * 7, D)
        dsk = carry_k.clone().scatter_add_(2, e, c * ds.reshape(B, H, -1, 1) * qrep)
        dsv = carry_v.clone().scatter_add_(2, e, w.reshape(B, H, -1, 1) * grep)
        per_round.append(dict(r=r, ds=ds, dKk=dKk, dKv=dKv, dW=dW, dsk=dsk, dsv=dsv))
        Gk, Gv = dsk, dsv
    return dq, Gk, Gv, per_round[::-1]


# ---------------------------------------------------------------------------
# Parity helpers: which index positions are decided by more than `rel` of score
# ---------------------------------------------------------------------------

def decided_positions(scores: torch.Tensor, k: int = K_NEIGHBORS, rel: float = 1e-3):
    """Masks over [.., k] index positions that a correct kernel must reproduce.

    ``set_ok[..., 0]`` is True for tokens whose k-th/(k+1)-th score gap
    exceeds ``rel`` relative (the top-k *set* is decided).  ``pos_ok[..., j]``
    is True where position j's neighbours in the sorted order are both further
    than ``rel`` relative, so the index at j is decided.  Scores at -inf are
    ties by construction and decide nothing.
    """
    top = torch.topk(scores.to(torch.float64), k=min(k + 1, scores.shape[-1]), dim=-1,
                     sorted=True)[0]
    if top.shape[-1] == k:  # M == k: the set is everything
        top = torch.cat([top, torch.full_like(top[..., :1], float("-inf"))], dim=-1)

    def gap(a, b):
        den = torch.maximum(a.abs(), b.abs()).clamp_min(1e-30)
        g = (a - b) / den
        g = torch.where(torch.isfinite(a) & torch.isinf(b) & (b < 0), torch.ones_like(g), g)
        g = torch.where(torch.isinf(a) & (a < 0), torch.zeros_like(g), g)
        return g

    gaps = gap(top[..., :-1], top[..., 1:])  # [.., k]
    set_ok = gaps[..., k - 1] > rel
    left = torch.cat([torch.ones_like(gaps[..., :1]), gaps[..., :k - 1]], dim=-1)
    right = gaps[..., :k]
    pos_ok = (left > rel) & (right > rel) & set_ok.unsqueeze(-1)
    return set_ok, pos_ok
