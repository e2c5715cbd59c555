"""Write golden input/output vectors from the reference's own PyTorch functions.

Run once, in the build container only (the reference tree does not exist on
the GPU box):  python tests/golden/make_golden.py [/root/reference]

It imports ``src/murmurative/reference.py`` of beaglabs/murmurative-attention
and records, as small .npz fixtures next to this script:

* legacy_composite.npz -- ``slot_murmurate_reference`` (reference.py:138-192)
  on seeded fp32 inputs for several flag combinations (plain, causal, dynamic
  M, token mask + position-bias callable, partial mask + bias callable, and
  x = q = k = v, which is the README call form), and the config-1 shapes
  (B=2, H=4, N=128, d=64, M=256).
  The composition of the four phases (which tensor feeds which phase, residual
  placement, post-update diffusion neighbours) is what no closed form pins.
* select_ties.npz -- ``slot_select_reference`` (reference.py:6-39) on inputs
  whose masked scores tie at -inf (causal prefix n < 6, effective_M < 7), which
  records torch.topk's CPU order among tied scores.

Every other phase of the oracle is pinned by closed forms and brute force in
tests/test_oracle.py; nothing else is recorded here.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load_reference(root):
    sys.path.insert(0, os.path.join(root, "src"))
    from murmurative import reference as ref  # noqa: E402  (reference package)
    return ref


def _t(a):
    return a.detach().cpu().numpy()


def legacy_cases(ref):
    cases = {}
    g = torch.Generator().manual_seed(42)

    def rn(*shape, std=1.0):
        return torch.randn(*shape, generator=g, dtype=torch.float32) * std

    # (name, B, N, H, Dh, M, rounds, kwargs)
    specs = [
        ("plain", 2, 24, 4, 16, 32, 3, dict()),
        ("causal", 2, 24, 4, 16, 32, 3, dict(causal=True)),
        ("dynm", 1, 64, 2, 16, 64, 2, dict(use_dynamic_m=True)),
        ("alpha_gamma", 1, 40, 2, 32, 48, 4, dict(alpha=0.5, gamma=0.3)),
    ]
    for name, B, N, H, Dh, M, R, kw in specs:
        D = H * Dh
        x, q, k, v = rn(B, N, D), rn(B, N, D), rn(B, N, D), rn(B, N, D)
        ske, sve = rn(H, M, Dh), rn(H, M, Dh, std=0.5)
        out = ref.slot_murmurate_reference(x, q, k, v, ske, sve, num_heads=H, rounds=R, **kw)
        p = f"{name}__"
        cases.update({p + "x": _t(x), p + "q": _t(q), p + "k": _t(k), p + "v": _t(v),
                      p + "ske": _t(ske), p + "sve": _t(sve), p + "out": _t(out)})
        cases[p + "meta"] = np.array([B, N, H, Dh, M, R], dtype=np.int64)

    # token mask [B,1,N,1] (some tokens fully masked) plus a bias callable
    B, N, H, Dh, M, R = 1, 20, 2, 16, 32, 2
    D = H * Dh
    x, q, k, v = rn(B, N, D), rn(B, N, D), rn(B, N, D), rn(B, N, D)
    ske, sve = rn(H, M, Dh), rn(H, M, Dh, std=0.5)
    mask = torch.ones(B, 1, N, 1)
    mask[:, :, 5:9] = 0.0
    ramp = torch.linspace(-1.0, 1.0, M)

    def bias_fn(xh):
        return 0.25 * torch.tanh(xh[..., :1]) * ramp

    out = ref.slot_murmurate_reference(x, q, k, v, ske, sve, num_heads=H, rounds=R,
                                       mask=mask, position_bias_fn=bias_fn)
    p = "maskbias__"
    cases.update({p + "x": _t(x), p + "q": _t(q), p + "k": _t(k), p + "v": _t(v),
                  p + "ske": _t(ske), p + "sve": _t(sve), p + "mask": _t(mask),
                  p + "out": _t(out)})
    cases[p + "meta"] = np.array([B, N, H, Dh, M, R], dtype=np.int64)

    # partial [B,H,N,M] mask (every token keeps >= 7 slots, so no -inf ties)
    # plus the same bias callable: comparable on a device whose tie order
    # differs from torch.topk's
    B, N, H, Dh, M, R = 2, 24, 2, 16, 32, 3
    D = H * Dh
    x, q, k, v = rn(B, N, D), rn(B, N, D), rn(B, N, D), rn(B, N, D)
    ske, sve = rn(H, M, Dh), rn(H, M, Dh, std=0.5)
    gm = torch.Generator().manual_seed(3)
    mask = (torch.rand(B, H, N, M, generator=gm) > 0.4).float()
    mask[..., :8] = 1.0
    ramp = torch.linspace(-1.0, 1.0, M)
    out = ref.slot_murmurate_reference(x, q, k, v, ske, sve, num_heads=H, rounds=R,
                                       mask=mask, position_bias_fn=bias_fn)
    p = "maskpart__"
    cases.update({p + "x": _t(x), p + "q": _t(q), p + "k": _t(k), p + "v": _t(v),
                  p + "ske": _t(ske), p + "sve": _t(sve), p + "mask": _t(mask),
                  p + "out": _t(out)})
    cases[p + "meta"] = np.array([B, N, H, Dh, M, R], dtype=np.int64)

    # README call form (x = q = k = v), config-1 shapes: B=2, H=4, N=128, d=64, M=256,
    # q ~ N(0,1), slots_k ~ N(0,1), slots_v = 0.  The reference composite shares
    # one [H,M,d] slot set over the batch, so the fixture does the same.
    B, N, H, Dh, M, R = 2, 128, 4, 64, 256, 3
    gq = torch.Generator().manual_seed(42)
    qh = torch.randn(B, H, N, Dh, generator=gq)
    ske = torch.randn(H, M, Dh, generator=gq)
    sve = torch.zeros(H, M, Dh)
    xin = qh.permute(0, 2, 1, 3).reshape(B, N, H * Dh)
    out = ref.slot_murmurate_reference(xin, xin, xin, xin, ske, sve, num_heads=H, rounds=R)
    p = "readme_cfg1__"
    cases.update({p + "q": _t(qh), p + "ske": _t(ske), p + "sve": _t(sve),
                  p + "out": _t(out.reshape(B, N, H, Dh).permute(0, 2, 1, 3))})
    cases[p + "meta"] = np.array([B, N, H, Dh, M, R], dtype=np.int64)
    return cases


def tie_cases(ref):
    g = torch.Generator().manual_seed(7)
    cases = {}
    q = torch.randn(1, 2, 12, 16, generator=g)
    sk = torch.randn(1, 2, 24, 16, generator=g)
    cases["causal__q"], cases["causal__sk"] = _t(q), _t(sk)
    cases["causal__idx"] = _t(ref.slot_select_reference(q, sk, causal=True))
    cases["em4__idx"] = _t(ref.slot_select_reference(q, sk, effective_M=4))
    cases["em7__idx"] = _t(ref.slot_select_reference(q, sk, effective_M=7))
    return cases


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = _load_reference(root)
    torch.set_num_threads(1)
    np.savez_compressed(os.path.join(HERE, "legacy_composite.npz"), **legacy_cases(ref))
    np.savez_compressed(os.path.join(HERE, "select_ties.npz"), **tie_cases(ref))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
