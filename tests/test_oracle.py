"""Pins for the CPU oracle (oracle/murm_oracle.py): golden vectors from the
reference's own functions, brute force on tiny inputs, closed forms and
finite-difference gradients.  CPU only."""

import math
import os

import numpy as np
import pytest
import torch

from oracle import murm_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _g(seed=0):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- select ---

def _brute_select(s, k=7):
    """Stable argsort of the masked scores, descending (ties by lower index)."""
    B, H, N, M = s.shape
    out = torch.empty(B, H, N, k, dtype=torch.int64)
    for b in range(B):
        for h in range(H):
            for n in range(N):
                row = s[b, h, n].tolist()
                order = sorted(range(M), key=lambda m: (-row[m], m))
                out[b, h, n] = torch.tensor(order[:k])
    return out


@pytest.mark.parametrize("kw", [dict(), dict(causal=True), dict(effective_M=19),
                                dict(mask="tok"), dict(bias=True)])
def test_select_matches_bruteforce(kw):
    g = _g(1)
    B, H, N, M, D = 1, 2, 12, 24, 8
    q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    sk = torch.randn(B, H, M, D, generator=g, dtype=torch.float64)
    mask = None
    if kw.get("mask") == "tok":
        mask = torch.ones(B, 1, N, M)
        mask[..., 3, :] = 0  # token 3 sees nothing
        mask[..., 5, 10:] = 0
    pb = torch.randn(B, H, N, M, generator=g, dtype=torch.float64) if kw.get("bias") else None
    causal = kw.get("causal", False)
    em = kw.get("effective_M")
    s = (q @ sk.transpose(-1, -2)).clone()
    if pb is not None:
        s = s + pb
    if mask is not None:
        s = s.masked_fill(mask == 0, -math.inf)
    for n in range(N):
        for m in range(M):
            if causal and m > n:
                s[:, :, n, m] = -math.inf
            if em is not None and m >= em:
                s[:, :, n, m] = -math.inf
    idx = O.select(q, sk, mask=mask, causal=causal, position_bias=pb, effective_M=em)
    ref = _brute_select(s)
    assert idx.dtype == torch.int64 and idx.shape == (B, H, N, 7)
    fin = torch.gather(s, -1, ref).isfinite()
    # finite positions are decided; -inf positions are ties (any masked slot)
    assert torch.equal(idx[fin], ref[fin])
    picked = torch.gather(s, -1, idx)
    assert torch.equal(picked.isfinite(), fin)
    assert (idx.sort(-1)[0].diff(dim=-1) > 0).all()  # distinct


def test_select_em_equals_k_is_all_slots():
    g = _g(2)
    q = torch.randn(1, 1, 16, 16, generator=g)
    sk = torch.randn(1, 1, 7, 16, generator=g)
    idx = O.select(q, sk)
    assert torch.equal(idx.sort(-1)[0], torch.arange(7).expand(1, 1, 16, 7))
    s = q @ sk.transpose(-1, -2)
    assert (torch.gather(s, -1, idx).diff(dim=-1) <= 0).all()


def test_select_tie_fixture():
    d = np.load(os.path.join(GOLD, "select_ties.npz"))
    q, sk = torch.from_numpy(d["causal__q"]), torch.from_numpy(d["causal__sk"])
    for key, kw in (("causal__idx", dict(causal=True)), ("em4__idx", dict(effective_M=4)),
                    ("em7__idx", dict(effective_M=7))):
        gold = torch.from_numpy(d[key])
        mine = O.select(q, sk, **kw)
        s = O.masked_scores(q, sk, **kw)
        fin = torch.gather(s, -1, gold).isfinite()
        assert torch.equal(mine[fin], gold[fin]), key
        assert torch.equal(torch.gather(s, -1, mine).isfinite(), fin), key


# ---------------------------------------------------------------- attend ---

def test_attend_closed_form_loop():
    g = _g(3)
    B, H, N, M, D = 1, 2, 5, 16, 8
    q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    sk = torch.randn(B, H, M, D, generator=g, dtype=torch.float64)
    sv = torch.randn(B, H, M, D, generator=g, dtype=torch.float64)
    idx = torch.stack([torch.randperm(M, generator=g)[:7] for _ in range(B * H * N)]).view(B, H, N, 7)
    out, w = O.attend(q, sk, sv, idx)
    c = 1 / math.sqrt(D)
    for b in range(B):
        for h in range(H):
            for n in range(N):
                z = [c * float(q[b, h, n] @ sk[b, h, int(m)]) for m in idx[b, h, n]]
                zmax = max(z)
                e = [math.exp(t - zmax) for t in z]
                tot = sum(e)
                ww = [t / tot for t in e]
                o = sum(ww[j] * sv[b, h, int(idx[b, h, n, j])] for j in range(7))
                assert torch.allclose(w[b, h, n], torch.tensor(ww, dtype=torch.float64), atol=1e-14)
                assert torch.allclose(out[b, h, n], o, atol=1e-14)
    assert torch.allclose(w.sum(-1), torch.ones(B, H, N, dtype=w.dtype))


def test_attend_clamps_indices_and_scale():
    g = _g(4)
    q = torch.randn(1, 1, 3, 4, generator=g, dtype=torch.float64)
    sk = torch.randn(1, 1, 9, 4, generator=g, dtype=torch.float64)
    sv = torch.randn(1, 1, 9, 4, generator=g, dtype=torch.float64)
    idx = torch.tensor([[[[-3, 0, 1, 2, 3, 4, 40]] * 3]])
    out, w = O.attend(q, sk, sv, idx, scale=0.5)
    out2, w2 = O.attend(q, sk, sv, idx.clamp(0, 8), scale=0.5)
    assert torch.equal(out, out2) and torch.equal(w, w2)


def test_attend_gradcheck():
    g = _g(5)
    B, H, N, M, D = 1, 2, 6, 16, 8
    q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64, requires_grad=True)
    sk = torch.randn(B, H, M, D, generator=g, dtype=torch.float64, requires_grad=True)
    sv = torch.randn(B, H, M, D, generator=g, dtype=torch.float64, requires_grad=True)
    idx = O.select(q.detach(), sk.detach())
    assert torch.autograd.gradcheck(lambda a, b, c: O.attend(a, b, c, idx), (q, sk, sv))


# ---------------------------------------------------------------- update ---

def test_update_matches_per_slot_loop():
    g = _g(6)
    B, H, N, M, D = 1, 2, 9, 12, 4
    tk = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    tv = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    sk = torch.randn(B, H, M, D, generator=g, dtype=torch.float64)
    sv = torch.randn(B, H, M, D, generator=g, dtype=torch.float64)
    idx = torch.stack([torch.randperm(M - 3, generator=g)[:7] for _ in range(B * H * N)]).view(B, H, N, 7)
    w = torch.rand(B, H, N, 7, generator=g, dtype=torch.float64)
    a = 0.8
    nk, nv = O.update(tk, tv, sk, sv, idx, w, alpha=a)
    for b in range(B):
        for h in range(H):
            for m in range(M):
                K = torch.zeros(D, dtype=torch.float64)
                V = torch.zeros(D, dtype=torch.float64)
                W = 0.0
                for n in range(N):
                    for j in range(7):
                        if int(idx[b, h, n, j]) == m:
                            K += w[b, h, n, j] * tk[b, h, n]
                            V += w[b, h, n, j] * tv[b, h, n]
                            W += float(w[b, h, n, j])
                if W > 0:
                    ek = a * sk[b, h, m] + (1 - a) * K / (W + 1e-8)
                    ev = a * sv[b, h, m] + (1 - a) * V / (W + 1e-8)
                else:  # slots M-3..M-1 are never selected: untouched
                    ek, ev = sk[b, h, m], sv[b, h, m]
                assert torch.allclose(nk[b, h, m], ek, atol=1e-13)
                assert torch.allclose(nv[b, h, m], ev, atol=1e-13)


def test_update_alpha_one_is_identity_and_dtype_kept():
    g = _g(7)
    tk = torch.randn(1, 2, 10, 8, generator=g).half()
    sk = torch.randn(1, 2, 16, 8, generator=g).half()
    idx = O.select(tk.float(), sk.float())
    _, w = O.attend(tk.float(), sk.float(), sk.float(), idx)
    nk, nv = O.update(tk, tk, sk, sk, idx, w, alpha=1.0)
    assert nk.dtype == torch.float16 and torch.equal(nk, sk) and torch.equal(nv, sk)


# ------------------------------------------------------------- diffusion ---

def _stencil_matrix(M, gamma):
    A = torch.eye(M, dtype=torch.float64)
    for m in range(1, M - 1):
        A[m, m - 1] = gamma
        A[m, m] = 1 - 2 * gamma
        A[m, m + 1] = gamma
    return A


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 32])
def test_diffusion_matrix_form_and_adjoint(M):
    g = _g(8)
    x = torch.randn(2, 3, M, 5, generator=g, dtype=torch.float64)
    y = torch.randn(2, 3, M, 5, generator=g, dtype=torch.float64)
    A = _stencil_matrix(M, 0.3)
    dk, dv = O.diffusion(x, y, 0.3)
    assert torch.allclose(dk, torch.einsum("ij,bhjd->bhid", A, x), atol=1e-14)
    assert torch.allclose(dv, torch.einsum("ij,bhjd->bhid", A, y), atol=1e-14)
    assert torch.allclose(O.diffusion_transpose(y, 0.3),
                          torch.einsum("ji,bhjd->bhid", A, y), atol=1e-14)
    z0, _ = O.diffusion(x, y, 0.0)
    assert torch.equal(z0, x)
    if M >= 1:
        assert torch.equal(dk[:, :, 0], x[:, :, 0]) and torch.equal(dk[:, :, -1], x[:, :, -1])


# ------------------------------------------------------------- composite ---

LEGACY = ["plain", "causal", "dynm", "alpha_gamma"]


@pytest.mark.parametrize("name", LEGACY)
def test_legacy_composite_golden(name):
    d = np.load(os.path.join(GOLD, "legacy_composite.npz"))
    B, N, H, Dh, M, R = [int(v) for v in d[name + "__meta"]]
    kw = dict(plain={}, causal=dict(causal=True), dynm=dict(use_dynamic_m=True),
              alpha_gamma=dict(alpha=0.5, gamma=0.3))[name]
    t = {k: torch.from_numpy(d[f"{name}__{k}"]) for k in ("x", "q", "k", "v", "ske", "sve", "out")}
    out = O.murmurate_legacy(t["x"], t["q"], t["k"], t["v"], t["ske"], t["sve"],
                             num_heads=H, rounds=R, **kw)
    assert torch.allclose(out, t["out"], atol=2e-5, rtol=1e-5)


def test_legacy_composite_golden_mask_and_bias():
    d = np.load(os.path.join(GOLD, "legacy_composite.npz"))
    B, N, H, Dh, M, R = [int(v) for v in d["maskbias__meta"]]
    t = {k: torch.from_numpy(d[f"maskbias__{k}"]) for k in
         ("x", "q", "k", "v", "ske", "sve", "mask", "out")}
    ramp = torch.linspace(-1.0, 1.0, M)
    out = O.murmurate_legacy(t["x"], t["q"], t["k"], t["v"], t["ske"], t["sve"], num_heads=H,
                             rounds=R, mask=t["mask"],
                             position_bias_fn=lambda xh: 0.25 * torch.tanh(xh[..., :1]) * ramp)
    fin = torch.ones(B, N, dtype=torch.bool)
    fin[:, 5:9] = False  # fully masked tokens attend to -inf ties: not decided
    assert torch.allclose(out[fin], t["out"][fin], atol=2e-5, rtol=1e-5)


def test_legacy_composite_golden_partial_mask_and_bias():
    d = np.load(os.path.join(GOLD, "legacy_composite.npz"))
    B, N, H, Dh, M, R = [int(v) for v in d["maskpart__meta"]]
    t = {k: torch.from_numpy(d[f"maskpart__{k}"]) for k in
         ("x", "q", "k", "v", "ske", "sve", "mask", "out")}
    ramp = torch.linspace(-1.0, 1.0, M)
    out = O.murmurate_legacy(t["x"], t["q"], t["k"], t["v"], t["ske"], t["sve"], num_heads=H,
                             rounds=R, mask=t["mask"],
                             position_bias_fn=lambda xh: 0.25 * torch.tanh(xh[..., :1]) * ramp)
    assert torch.allclose(out, t["out"], atol=2e-5, rtol=1e-5)


def test_readme_form_golden_config1():
    d = np.load(os.path.join(GOLD, "legacy_composite.npz"))
    B, N, H, Dh, M, R = [int(v) for v in d["readme_cfg1__meta"]]
    q = torch.from_numpy(d["readme_cfg1__q"])
    sk = torch.from_numpy(d["readme_cfg1__ske"]).unsqueeze(0).expand(B, -1, -1, -1)
    sv = torch.from_numpy(d["readme_cfg1__sve"]).unsqueeze(0).expand(B, -1, -1, -1)
    out, idx, w = O.murmurate_readme(q, sk, sv, rounds=R)
    assert torch.allclose(out, torch.from_numpy(d["readme_cfg1__out"]), atol=2e-5, rtol=1e-5)
    assert idx.shape == (B, H, N, 7) and w.dtype == torch.float32


def test_readme_form_equals_legacy_with_shared_projections():
    g = _g(9)
    B, H, N, Dh, M = 2, 2, 16, 8, 24
    q = torch.randn(B, H, N, Dh, generator=g, dtype=torch.float64)
    ske = torch.randn(H, M, Dh, generator=g, dtype=torch.float64)
    sve = torch.randn(H, M, Dh, generator=g, dtype=torch.float64)
    out, _, _ = O.murmurate_readme(q, ske.expand(B, -1, -1, -1), sve.expand(B, -1, -1, -1),
                                   rounds=3, causal=True)
    x = q.permute(0, 2, 1, 3).reshape(B, N, H * Dh)
    ref = O.murmurate_legacy(x, x, x, x, ske, sve, num_heads=H, rounds=3, causal=True)
    assert torch.allclose(out.permute(0, 2, 1, 3).reshape(B, N, H * Dh), ref, atol=1e-13)


def test_readme_composite_gradcheck():
    g = _g(10)
    B, H, N, D, M = 1, 2, 10, 8, 16
    q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64, requires_grad=True)
    sk = torch.randn(B, H, M, D, generator=g, dtype=torch.float64, requires_grad=True)
    sv = torch.randn(B, H, M, D, generator=g, dtype=torch.float64, requires_grad=True)

    def f(a, b, c):
        out, _, w = O.murmurate_readme(a, b, c, rounds=3)
        return out, w
    assert torch.autograd.gradcheck(f, (q, sk, sv), eps=1e-6, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_closed_form_backward_equals_autograd(causal):
    g = _g(11)
    B, H, N, D, M = 2, 2, 24, 8, 20
    q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64, requires_grad=True)
    sk = torch.randn(B, H, M, D, generator=g, dtype=torch.float64, requires_grad=True)
    sv = torch.randn(B, H, M, D, generator=g, dtype=torch.float64, requires_grad=True)
    go = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    gw = torch.randn(B, H, N, 7, generator=g, dtype=torch.float64)
    out, _, w = O.murmurate_readme(q, sk, sv, rounds=3, causal=causal)
    dq, dsk, dsv = torch.autograd.grad((out, w), (q, sk, sv), (go, gw))
    cq, csk, csv, _ = O.murmurate_backward(q.detach(), sk.detach(), sv.detach(), go,
                                           grad_w_last=gw, rounds=3, causal=causal)
    assert torch.allclose(cq, dq, atol=1e-12)
    assert torch.allclose(csk, dsk, atol=1e-12)
    assert torch.allclose(csv, dsv, atol=1e-12)


def test_decided_positions():
    s = torch.tensor([[[[9.0, 8.0, 7.0, 6.0, 5.0, 4.0, 3.0, 2.999, 1.0]]]])
    set_ok, pos_ok = O.decided_positions(s, rel=1e-3)
    assert not bool(set_ok.all())  # 3.0 vs 2.999 is 3.3e-4 relative
    s2 = torch.tensor([[[[9.0, 8.0, 7.0, 6.0, 5.0, 4.0, 3.0, 2.0, 1.0]]]])
    set_ok, pos_ok = O.decided_positions(s2, rel=1e-3)
    assert bool(set_ok.all()) and bool(pos_ok.all())
    s3 = torch.tensor([[[[9.0, 8.0, 8.0, 6.0, 5.0, 4.0, 3.0, 2.0, 1.0]]]])
    _, pos_ok = O.decided_positions(s3, rel=1e-3)
    assert pos_ok.tolist() == [[[[True, False, False, True, True, True, True]]]]
