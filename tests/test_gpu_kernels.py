"""GPU parity of the single-round ops against the CPU oracle (float64).

Selection: exact at every index position the oracle's scores decide (1e-3
relative gap); numerics: the oracle replays the kernel's indices and every
output and gradient must agree within the dtype's tolerance (tests/parity.py).
"""

import ctypes
import math

import pytest
import torch

import murmurative as MA
from murmurative import capi
from oracle import murm_oracle as O
from parity import TOL, assert_close, check_selection, grad_w_bound, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _print_case(*a):
    print("case", *a, flush=True)


def test_mfma_lane_layout_selftest():
    _print_case("mfma selftest")
    lib = capi.load()
    out = torch.zeros(768, device=DEV)
    capi.check(lib.murm_selftest_mfma(ctypes.c_void_p(out.data_ptr()), None), "selftest")
    torch.cuda.synchronize()
    lane = torch.arange(64).view(64, 1)
    r = torch.arange(4).view(1, 4)
    expect = (16 * (4 * (lane // 16) + r) + (lane % 16)).float().flatten()
    got = out.cpu().view(3, 256)
    for t in range(3):
        assert torch.equal(got[t], expect), f"layout test {t}: {got[t][:8]} vs {expect[:8]}"


def _inputs(B, H, N, D, M, dtype, seed=42, sv_std=1.0):
    q, sk, sv, go = seeded([(B, H, N, D), (B, H, M, D), (B, H, M, D), (B, H, N, D)], seed,
                           [None, None, sv_std, None])
    gw = seeded([(B, H, N, 7)], seed + 1)[0]
    q, sk, sv, go = (t.to(dtype) for t in (q, sk, sv, go))
    return q, sk, sv, go, gw


SA_CASES = [
    # (B, H, N, D, M, flags)
    (1, 2, 300, 64, 256, {}),
    (2, 3, 64, 32, 64, {}),
    (1, 2, 50, 16, 7, {}),
    (1, 2, 130, 128, 256, {}),
    (1, 1, 70, 64, 512, {}),
    (1, 2, 40, 48, 40, {}),
    (1, 2, 33, 64, 64, {"causal": True}),
    (1, 2, 64, 32, 64, {"effective_M": 20}),
    (1, 2, 64, 32, 64, {"effective_M": 5}),
    (2, 2, 48, 32, 64, {"mask": True}),
    (1, 2, 48, 32, 64, {"bias": True}),
    # a grid that fills the device: full-size select blocks (the small cases
    # above take the half-size blocks of small grids)
    (1, 16, 4096, 64, 64, {}),
    (1, 2, 64, 64, 128, {"scale": 0.3}),
]


def _slot_rows(t, pad):
    """t on the device as a leaf; with pad > 0 a view whose rows are pad
    elements longer than D (a slice of a wider zero tensor)."""
    if pad == 0:
        return t.to(DEV).requires_grad_(True)
    wide = torch.zeros(*t.shape[:-1], t.shape[-1] + pad, dtype=t.dtype, device=DEV)
    wide[..., :t.shape[-1]] = t.to(DEV)
    leaf = wide.requires_grad_(True)
    return leaf, leaf[..., :t.shape[-1]]


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", SA_CASES, ids=[f"c{i}" for i in range(len(SA_CASES))])
def test_select_attend_op(dtype, case):
    _check_select_attend(dtype, case)


# bf16 tokens: 16-byte bf16 slot rows are read by the select kernel itself;
# float32 slots and rows of 68 elements take the conversion launch
@pytest.mark.parametrize("layout", [(None, 8), (torch.float32, 0), (None, 4)], ids=["pad8", "f32slots", "pad4"])
def test_select_attend_op_slot_layouts(layout):
    _check_select_attend(torch.bfloat16, (1, 2, 300, 64, 256, {}), *layout)


def _check_select_attend(dtype, case, slot_dtype=None, slot_pad=0):
    B, H, N, D, M, fl = case
    _print_case("select_attend", dtype, case, slot_dtype, slot_pad)
    q, sk, sv, go, gw = _inputs(B, H, N, D, M, dtype)
    if slot_dtype is not None:
        sk, sv = sk.to(slot_dtype), sv.to(slot_dtype)
    mask = bias = None
    if fl.get("mask"):
        mask = torch.ones(B, 1, N, 1)
        mask[:, :, 5:9] = 0
        mask[1:, :, 20:30] = 0
    if fl.get("bias"):
        bias = (seeded([(B, H, N, M)], 7)[0] * 2.0).to(dtype)
    em = fl.get("effective_M", 0)
    scale = fl.get("scale")
    causal = fl.get("causal", False)
    qd = q.to(DEV).requires_grad_(True)
    if slot_pad:
        (skl, skd), (svl, svd) = _slot_rows(sk, slot_pad), _slot_rows(sv, slot_pad)
    else:
        skd, svd = _slot_rows(sk, 0), _slot_rows(sv, 0)
    out, w, idx = MA.slot_select_attend(qd, skd, svd, mask=None if mask is None else mask.to(DEV),
                                        causal=causal, position_bias=None if bias is None else bias.to(DEV),
                                        scale=scale, effective_M=em)
    (out.float() * go.to(DEV).float()).sum().add((w * gw.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    assert idx.dtype == torch.int64 and w.dtype == torch.float32 and out.dtype == dtype
    q64, sk64, sv64 = (t.double().requires_grad_(True) for t in (q, sk, sv))
    scores = O.masked_scores(q64.detach(), sk64.detach(), mask=mask, causal=causal,
                             position_bias=None if bias is None else bias.double(),
                             effective_M=em if em > 0 else None)
    check_selection("indices", idx, scores)
    o_out, o_w = O.attend(q64, sk64, sv64, idx.cpu(), scale=scale)
    assert_close("out", out, o_out, dtype)
    assert_close("weights", w, o_w, dtype)
    ((o_out * go.double()).sum() + (o_w * gw.double()).sum()).backward()
    assert_close("grad_q", qd.grad, q64.grad, dtype)
    gsk, gsv = (skl.grad[..., :D], svl.grad[..., :D]) if slot_pad else (skd.grad, svd.grad)
    assert_close("grad_slot_keys", gsk, sk64.grad, dtype)
    assert_close("grad_slot_values", gsv, sv64.grad, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16", "bf16"])
def test_slot_select_and_attend(dtype):
    _print_case("select/attend", dtype)
    B, H, N, D, M = 2, 2, 100, 64, 96
    q, sk, sv, go, gw = _inputs(B, H, N, D, M, dtype)
    idx = MA.slot_select(q.to(DEV), sk.to(DEV))
    scores = O.masked_scores(q.double(), sk.double())
    check_selection("slot_select", idx, scores)
    idx_c = MA.slot_select(q.to(DEV), sk.to(DEV), causal=True)
    check_selection("slot_select causal", idx_c, O.masked_scores(q.double(), sk.double(), causal=True))
    given = torch.stack([torch.randperm(M, generator=torch.Generator().manual_seed(i))[:7]
                         for i in range(B * H * N)]).view(B, H, N, 7)
    given[0, 0, 0, 0] = M + 5  # clamped to M-1 like reference.py:56
    qd, skd, svd = (t.to(DEV).requires_grad_(True) for t in (q, sk, sv))
    out, w = MA.slot_attend(qd, skd, svd, given.to(DEV))
    (out.float() * go.to(DEV).float()).sum().add((w * gw.to(DEV)).sum()).backward()
    q64, sk64, sv64 = (t.double().requires_grad_(True) for t in (q, sk, sv))
    o_out, o_w = O.attend(q64, sk64, sv64, given)
    ((o_out * go.double()).sum() + (o_w * gw.double()).sum()).backward()
    assert_close("attend out", out, o_out, dtype)
    assert_close("attend w", w, o_w, dtype)
    assert_close("attend dq", qd.grad, q64.grad, dtype)
    assert_close("attend dsk", skd.grad, sk64.grad, dtype)
    assert_close("attend dsv", svd.grad, sv64.grad, dtype)


def test_zero_scores_keep_distinct_indices():
    # all scores exactly 0: the packed keys are denormals and must survive max/med3
    _print_case("zero scores")
    q = torch.zeros(1, 1, 64, 64, device=DEV, dtype=torch.bfloat16)
    sk = torch.randn(1, 1, 256, 64, device=DEV, dtype=torch.bfloat16)
    out, w, idx = MA.slot_select_attend(q, sk, sk)
    torch.cuda.synchronize()
    i = idx.cpu()
    assert int(i.min()) >= 0 and int(i.max()) < 256
    assert (i.sort(-1).values.diff(dim=-1) > 0).all()
    assert torch.allclose(w.cpu(), torch.full_like(w.cpu(), 1 / 7))


# (B, H, N, D, M, duplicates): the token-chunk reduction serves M padded to 64
# times the per-slot threads up to 1024; (1, 2, 500, 96, 520) takes the
# per-slot-group kernels instead.  With duplicates a token names a slot twice
# (caller-given indices; the reference's index_add counts both).
UPD_CASES = [(1, 2, 40, 16, 64, 0), (2, 2, 300, 64, 256, 0), (1, 1, 1500, 128, 48, 0), (1, 2, 64, 32, 3 + 4, 0),
             (1, 2, 500, 96, 520, 0), (1, 2, 700, 64, 32, 1)]


def _update_inputs(B, H, N, D, M, dtype, seed=5, dup=False):
    tk, tv, sk, sv, gk, gv = seeded([(B, H, N, D), (B, H, N, D), (B, H, M, D), (B, H, M, D), (B, H, M, D),
                                     (B, H, M, D)], seed)
    g = torch.Generator().manual_seed(seed)
    used = M - 3 if M > 10 else M  # with M > 10 the last three slots stay unused (W = 0)
    if dup:
        idx = torch.randint(0, used, (B, H, N, 7), generator=g)
    else:
        idx = torch.stack([torch.randperm(used, generator=g)[:7] for _ in range(B * H * N)]).view(B, H, N, 7)
    w = torch.rand(B, H, N, 7, generator=g)
    w = w / w.sum(-1, keepdim=True)
    cast = lambda t: t.to(dtype)  # noqa: E731
    return cast(tk), cast(tv), cast(sk), cast(sv), cast(gk), cast(gv), idx, w


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("case", UPD_CASES, ids=[f"u{i}" for i in range(len(UPD_CASES))])
def test_update_and_diffusion_ops(dtype, case):
    B, H, N, D, M, dup = case
    _print_case("update/diffusion", dtype, case)
    tk, tv, sk, sv, gk, gv, idx, w = _update_inputs(B, H, N, D, M, dtype, dup=bool(dup))
    a, gm = 0.8, 0.15
    # forward, in place
    skd, svd = sk.to(DEV).clone(), sv.to(DEV).clone()
    r1 = MA.slot_update(tk.to(DEV), tv.to(DEV), skd, svd, idx.to(DEV), w.to(DEV), alpha=a)
    assert r1[0].data_ptr() == skd.data_ptr()
    e_k, e_v = O.update(tk.double(), tv.double(), sk.double(), sv.double(), idx, w.double(), a)
    assert_close("update k", skd, e_k, dtype)
    assert_close("update v", svd, e_v, dtype)
    skd2, svd2 = sk.to(DEV).clone(), sv.to(DEV).clone()
    MA.slot_diffusion(skd2, svd2, gamma=gm)
    f_k, f_v = O.diffusion(sk.double(), sv.double(), gm)
    assert_close("diffusion k", skd2, f_k, dtype)
    assert_close("diffusion v", svd2, f_v, dtype)
    lib = MA.ops._get_lib()
    skd3, svd3 = sk.to(DEV).clone(), sv.to(DEV).clone()
    lib.slot_update_diffuse(skd3, svd3, tk.to(DEV), tv.to(DEV), idx.to(DEV), w.to(DEV), a, gm)
    h_k, h_v = O.diffusion(e_k, e_v, gm)  # post-update neighbours
    assert_close("update_diffuse k", skd3, h_k, dtype)
    assert_close("update_diffuse v", svd3, h_v, dtype)
    # update backward op, given the gradient it receives (ops.py:117-130)
    gtk, gtv, gok, gov, gw_ = lib.slot_update_backward(gk.to(DEV), gv.to(DEV), tk.to(DEV), tv.to(DEV),
                                                       idx.to(DEV), w.to(DEV), a)
    tk64, tv64, sk64, sv64 = (t.double().requires_grad_(True) for t in (tk, tv, sk, sv))
    w64 = w.double().requires_grad_(True)
    ok_, ov_ = O.update(tk64, tv64, sk64, sv64, idx, w64, a)
    ((ok_ * gk.double()).sum() + (ov_ * gv.double()).sum()).backward()
    assert_close("update bwd token keys", gtk, tk64.grad, dtype)
    assert_close("update bwd token values", gtv, tv64.grad, dtype)
    assert_close("update bwd slot keys", gok, sk64.grad, dtype)
    assert_close("update bwd slot values", gov, sv64.grad, dtype)
    assert_close("update bwd weights", gw_, w64.grad, dtype, extra=grad_w_bound(tk, tv, gk, gv, idx, w, a, dtype))
    # update + diffusion through autograd: the adjoint crosses the op boundary
    # in the slot dtype (ops.py:188-208), so the oracle rounds it there too
    tkd, tvd, skg, svg = (t.to(DEV).requires_grad_(True) for t in (tk, tv, sk, sv))
    wd = w.to(DEV).requires_grad_(True)
    nk, nv = MA.ops._SlotUpdateDiffuse.apply(tkd, tvd, skg.clone(), svg.clone(), idx.to(DEV), wd, a, gm)
    (nk.float() * gk.to(DEV).float()).sum().add((nv.float() * gv.to(DEV).float()).sum()).backward()
    gpk = O.diffusion_transpose(gk.double(), gm).to(dtype)
    gpv = O.diffusion_transpose(gv.double(), gm).to(dtype)
    tk64, tv64, sk64, sv64 = (t.double().requires_grad_(True) for t in (tk, tv, sk, sv))
    w64 = w.double().requires_grad_(True)
    ok_, ov_ = O.update(tk64, tv64, sk64, sv64, idx, w64, a)
    ((ok_ * gpk.double()).sum() + (ov_ * gpv.double()).sum()).backward()
    assert_close("chain bwd token keys", tkd.grad, tk64.grad, dtype)
    assert_close("chain bwd token values", tvd.grad, tv64.grad, dtype)
    assert_close("chain bwd slot keys", skg.grad, sk64.grad, dtype)
    assert_close("chain bwd slot values", svg.grad, sv64.grad, dtype)
    assert_close("chain bwd weights", wd.grad, w64.grad, dtype, extra=grad_w_bound(tk, tv, gpk, gpv, idx, w, a, dtype))
    # diffusion backward op alone
    gdk, gdv = lib.slot_diffusion_backward(gk.to(DEV), gv.to(DEV), gm)
    assert_close("diffusion adjoint k", gdk, O.diffusion_transpose(gk.double(), gm), dtype)
    assert_close("diffusion adjoint v", gdv, O.diffusion_transpose(gv.double(), gm), dtype)


def test_update_is_deterministic():
    _print_case("update determinism")
    tk, tv, sk, sv, gk, gv, idx, w = _update_inputs(1, 4, 4096, 64, 256, torch.bfloat16, seed=9)
    outs = []
    for _ in range(3):
        k, v = sk.to(DEV).clone(), sv.to(DEV).clone()
        MA.slot_update(tk.to(DEV), tv.to(DEV), k, v, idx.to(DEV), w.to(DEV), alpha=0.9)
        outs.append((k.cpu(), v.cpu()))
    for k, v in outs[1:]:
        assert torch.equal(k, outs[0][0]) and torch.equal(v, outs[0][1])


def test_errors_are_raised_on_the_host():
    _print_case("errors")
    q = torch.randn(1, 1, 8, 200, device=DEV, dtype=torch.bfloat16)
    sk = torch.randn(1, 1, 16, 200, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="D=200"):
        MA.slot_select_attend(q, sk, sk)
    q = torch.randn(1, 1, 8, 16, device=DEV, dtype=torch.bfloat16)
    sk = torch.randn(1, 1, 5, 16, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="M=5"):
        MA.slot_select_attend(q, sk, sk)
    with pytest.raises(TypeError):
        MA.slot_select_attend(q.double(), sk.double(), sk.double())
    e = torch.randn(1, 16, device=DEV).expand(4, 1, 16, 16)
    with pytest.raises(RuntimeError):
        MA.ops._get_lib().slot_diffusion(e, e, 0.1)
