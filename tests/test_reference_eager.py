"""The package's eager ``*_reference`` path (use_reference=True) equals the
oracle on CPU.  Product API, checked against the test oracle."""

import torch

import murmurative as M
from oracle import murm_oracle as O


def _g(s):
    return torch.Generator().manual_seed(s)


def test_eager_single_round_functions_match_oracle():
    g = _g(1)
    B, H, N, Mm, D = 2, 3, 20, 24, 8
    q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    sk = torch.randn(B, H, Mm, D, generator=g, dtype=torch.float64)
    sv = torch.randn(B, H, Mm, D, generator=g, dtype=torch.float64)
    pb = torch.randn(B, H, N, Mm, generator=g, dtype=torch.float64)
    mask = torch.ones(B, 1, N, 1)
    mask[:, :, 3] = 0
    for kw in (dict(), dict(causal=True), dict(position_bias=pb), dict(effective_M=9), dict(mask=mask)):
        a = M.slot_select_reference(q, sk, **kw)
        b = O.select(q, sk, **kw)
        s = O.masked_scores(q, sk, **kw)
        fin = torch.gather(s, -1, b).isfinite()
        assert torch.equal(a[fin], b[fin])
    idx = O.select(q, sk)
    o1, w1 = M.slot_attend_reference(q, sk, sv, idx, scale=0.3)
    o2, w2 = O.attend(q, sk, sv, idx, scale=0.3)
    assert torch.allclose(o1, o2, atol=1e-12) and torch.allclose(w1, w2.float(), atol=1e-6)
    _, w = O.attend(q, sk, sv, idx)
    # the eager path sums in float32 as reference.py:86-89 does; the oracle
    # keeps float64 inputs in float64
    u1 = M.slot_update_reference(q, q * 2, sk, sv, idx, w, 0.7)
    u2 = O.update(q, q * 2, sk, sv, idx, w, 0.7)
    assert all(torch.allclose(a, b, atol=1e-5) for a, b in zip(u1, u2))
    d1 = M.slot_diffusion_reference(sk, sv, 0.2)
    d2 = O.diffusion(sk, sv, 0.2)
    assert all(torch.allclose(a, b, atol=1e-12) for a, b in zip(d1, d2))


def test_eager_composites_match_oracle():
    g = _g(2)
    B, N, H, Dh, Mm = 2, 24, 2, 8, 32
    D = H * Dh
    x, q, k, v = (torch.randn(B, N, D, generator=g, dtype=torch.float64) for _ in range(4))
    ske = torch.randn(H, Mm, Dh, generator=g, dtype=torch.float64)
    sve = torch.randn(H, Mm, Dh, generator=g, dtype=torch.float64)
    for kw in (dict(), dict(causal=True), dict(use_dynamic_m=True)):
        a = M.slot_murmurate(x, q, k, v, ske, sve, num_heads=H, rounds=3, use_reference=True,
                             use_dynamic_m=kw.get("use_dynamic_m", False), causal=kw.get("causal", False))
        b = O.murmurate_legacy(x, q, k, v, ske, sve, num_heads=H, rounds=3, **kw)
        assert torch.allclose(a, b, atol=1e-5)
    qh = torch.randn(B, H, N, Dh, generator=g, dtype=torch.float64)
    out, idx, w = M.slot_murmurate(qh, ske.expand(B, -1, -1, -1), sve.expand(B, -1, -1, -1), rounds=3,
                                   use_reference=True)
    o2, i2, w2 = O.murmurate_readme(qh, ske.expand(B, -1, -1, -1), sve.expand(B, -1, -1, -1), rounds=3)
    assert torch.allclose(out, o2, atol=1e-5) and torch.equal(idx, i2)


def test_readme_verify_call_on_the_eager_path():
    # README.md:64-67: slot_murmurate(x, slots, rounds=3), slot values zero;
    # the fixture was written by the reference's own function (config-1 shapes)
    import os
    import numpy as np
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "legacy_composite.npz"))
    B, N, H, Dh, Mm, R = [int(v) for v in d["readme_cfg1__meta"]]
    x = torch.from_numpy(d["readme_cfg1__q"])
    slots = torch.from_numpy(d["readme_cfg1__ske"]).unsqueeze(0).expand(B, -1, -1, -1)
    out, idx, w = M.slot_murmurate(x, slots, rounds=3, use_reference=True)
    assert out.shape == (B, H, N, Dh) and idx.shape == (B, H, N, 7) and w.shape == (B, H, N, 7)
    assert torch.allclose(out, torch.from_numpy(d["readme_cfg1__out"]), atol=2e-5, rtol=1e-5)
    out2, idx2, _ = M.slot_murmurate(x, slots, torch.zeros_like(slots), rounds=3, use_reference=True)
    assert torch.equal(out, out2) and torch.equal(idx, idx2)
