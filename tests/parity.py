"""Parity helpers shared by the GPU tests.

Protocol for multi-round results: the GPU forward runs first; its per-round
selections are read back from the forward workspace; the oracle (float64)
then replays exactly those selections (``forced_idx``) so that outputs,
weights and gradients can be compared tightly, while each round's selection
is checked on its own against the top-7 of the replayed oracle scores at
every position the scores decide (1e-3 relative gap, oracle.decided_positions).
"""

import math
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (ROOT, os.path.join(ROOT, "murmurative-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from oracle import murm_oracle as O  # noqa: E402

# 1e-5 abs (fp32), 2e-2 abs (fp16/bf16).  A 16-bit
# output cannot hold more than its own rounding, so the 16-bit bound also
# allows one half-ulp of the value (rtol 2^-11 fp16, 2^-8 bf16).
TOL = {
    torch.float32: (1e-5, 1e-6),
    torch.float16: (2e-2, 2.0 ** -11),
    torch.bfloat16: (2e-2, 2.0 ** -8),
}
GAP = 1e-3


def seeded(shape_list, seed=42, stds=None):
    """fp32 draws on a CPU generator in the order given (BASELINE convention)."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for i, shp in enumerate(shape_list):
        t = torch.randn(*shp, generator=g)
        if stds is not None and stds[i] is not None:
            t = t * stds[i]
        out.append(t)
    return out


def assert_close(name, got, ref, dtype, mask=None, extra=None):
    """|got - ref| <= atol + rtol*|ref| (+ extra, a per-element bound where the
    quantity is ill-conditioned in float32)."""
    atol, rtol = TOL[dtype]
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, (name, g.shape, r.shape)
    diff = (g - r).abs()
    tol = atol + rtol * r.abs()
    if extra is not None:
        tol = tol + extra.double().cpu()
    bad = diff > tol
    if mask is not None:
        bad = bad & mask
    if bad.any():
        i = int(torch.argmax((diff - tol).flatten()))
        raise AssertionError(
            f"{name}: {int(bad.sum())} of {bad.numel()} elements outside atol={atol} rtol={rtol}; "
            f"worst |d|={diff.flatten()[i].item():.3e} at {i} (got {g.flatten()[i].item():.6g}, "
            f"ref {r.flatten()[i].item():.6g})")
    return diff.max().item()


def check_selection(name, gpu_idx, scores, k=7):
    """Indices must equal the oracle's top-k wherever the scores decide them."""
    gi = gpu_idx.detach().cpu().to(torch.int64)
    top = torch.topk(scores.double(), k=k, dim=-1, sorted=True).indices
    set_ok, pos_ok = O.decided_positions(scores, k=k, rel=GAP)
    pos_bad = (gi != top) & pos_ok
    assert not pos_bad.any(), f"{name}: {int(pos_bad.sum())} decided index positions differ"
    set_bad = (gi.sort(-1).values != top.sort(-1).values).any(-1) & set_ok
    assert not set_bad.any(), f"{name}: {int(set_bad.sum())} decided top-7 sets differ"
    # structural: distinct, in range
    M = scores.shape[-1]
    assert int(gi.min()) >= 0 and int(gi.max()) < M, f"{name}: index out of range"
    assert (gi.sort(-1).values.diff(dim=-1) > 0).all(), f"{name}: repeated index"
    return float(set_ok.double().mean())


# Unit roundoff of the slot sums behind the update's weight gradient, per
# token dtype: float32 tokens sum in float32 (2^-24 per add, 2^-20 covers the
# sums' length); 16-bit tokens multiply hi + lo halves of the coefficients on
# MFMA, which represent a float32 coefficient to 2^-17 (bf16) or 2^-22
# (fp16) relative, on top of the float32 accumulation.  Pinned on the CPU in
# tests/test_parity_bounds.py.
U_GRADW = {torch.float32: 2.0 ** -20, torch.float16: 2.0 ** -20, torch.bfloat16: 2.0 ** -17}


def grad_w_bound(tk, tv, gk, gv, idx, w, alpha, dtype=torch.bfloat16, eps=1e-8):
    """Error bound of the update's weight gradient evaluated with the slot
    sums at the precision of `dtype`'s kernel path (U_GRADW).

    dw_nj = (1-a)/(W_m+eps) [(tk_n - K_m/(W_m+eps)).G'k_m + (tv_n - V_m/(W_m+eps)).G'v_m],
    m = idx_nj: the two halves cancel on slots whose total weight W_m is small,
    so a relative error u in the sums K, V, W becomes an absolute error of
    about u * cond with cond = (1-a)/W_m * (|tk|+|mean|).|G'| -- whoever
    evaluates it (a float32 evaluation of the reference's maths included)."""
    M = gk.shape[2]
    tk, tv, gk, gv = (t.double() for t in (tk, tv, gk, gv))
    K, V, W = O.slot_sums(tk, tv, idx, w.double(), M)
    mk, mv = K / (W.unsqueeze(-1) + eps), V / (W.unsqueeze(-1) + eps)
    B, H, N, _ = tk.shape
    b = torch.arange(B).view(B, 1, 1, 1)
    h = torch.arange(H).view(1, H, 1, 1)
    ag = lambda t: t.abs()[b, h, idx]  # noqa: E731
    mag = ((tk.abs().unsqueeze(3) + ag(mk)) * ag(gk)).sum(-1) + ((tv.abs().unsqueeze(3) + ag(mv)) * ag(gv)).sum(-1)
    cond = (1.0 - alpha) / (W[b, h, idx] + eps) * mag
    return cond * U_GRADW[dtype]


def round_indices(ws, B, H, N, D, M, R, shared, r):
    from murmurative import capi
    off = capi.load().murm_murmurate_workspace_offset(B, H, N, D, M, R, 1 if shared else 0, r, 2)
    assert off >= 0
    n = B * H * N * 8 * 2
    raw = ws[off:off + n].view(torch.int16).view(B, H, N, 8)[..., :7]
    return raw.to(torch.int64) & 0xFFFF


def default_scale(D):
    return 1.0 / math.sqrt(D)
