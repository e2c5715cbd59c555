"""CPU checks of the drop-in boundary: the C ABI library loads and exports
every symbol the header declares, the torch extension registers the
reference's op schemas verbatim, and the Python API raises the reference's
error types without a GPU.  No kernel runs here."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

import murmurative
from murmurative import capi, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "murmurative_hip.h")

REFERENCE_SCHEMAS = {
    "slot_select_attend": "slot_select_attend(Tensor query, Tensor slot_keys, Tensor slot_values, "
                          "Tensor? mask, bool causal, Tensor? position_bias, float? scale, int effective_M) -> "
                          "(Tensor, Tensor, Tensor)",
    "slot_select_attend_backward": "slot_select_attend_backward(Tensor grad_output, Tensor grad_weights, "
                                   "Tensor query, Tensor slot_keys, Tensor slot_values, Tensor indices, "
                                   "Tensor weights, float? scale) -> (Tensor, Tensor, Tensor)",
    "slot_update": "slot_update(Tensor(a!) slot_keys, Tensor(b!) slot_values, Tensor token_keys, "
                   "Tensor token_values, Tensor indices, Tensor weights, float alpha) -> ()",
    "slot_update_backward": "slot_update_backward(Tensor grad_new_sk, Tensor grad_new_sv, Tensor token_keys, "
                            "Tensor token_values, Tensor indices, Tensor weights, float alpha) -> "
                            "(Tensor, Tensor, Tensor, Tensor, Tensor)",
    "slot_diffusion": "slot_diffusion(Tensor(a!) slot_keys, Tensor(b!) slot_values, float gamma) -> ()",
    "slot_diffusion_backward": "slot_diffusion_backward(Tensor grad_new_keys, Tensor grad_new_values, "
                               "float gamma) -> (Tensor, Tensor)",
    "slot_update_diffuse": "slot_update_diffuse(Tensor(a!) slot_keys, Tensor(b!) slot_values, "
                           "Tensor token_keys, Tensor token_values, Tensor indices, Tensor weights, "
                           "float alpha, float gamma) -> ()",
}


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(murm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_ctypes_table_agree():
    assert header_functions() == sorted(capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (murm_[a-z0-9_]+)$", out, flags=re.M))
    assert set(header_functions()) <= exported
    assert lib.murm_version().startswith(b"murmurative_hip")


def test_workspace_queries_without_gpu():
    lib = capi.load()
    B, H, N, D, M, R = 1, 16, 8192, 64, 256, 3
    ws = lib.murm_murmurate_workspace_bytes(B, H, N, D, M, R, 1)
    S = B * H * M * D * 4
    assert ws >= R * 2 * S + R * B * H * N * 16
    offs = [lib.murm_murmurate_workspace_offset(B, H, N, D, M, R, 1, r, 2) for r in range(R)]
    assert all(o >= 0 and o % 256 == 0 for o in offs) and len(set(offs)) == R
    assert lib.murm_murmurate_workspace_offset(B, H, N, D, M, R, 1, R - 1, 6) == -1
    # argument errors are reported before anything is enqueued
    rc = lib.murm_slot_diffusion_fwd(7, 1, 1, 8, 8, None, 0, 0, 0, None, 0, 0, 0, 0.1, None)
    assert rc == capi.ERR_ARG and b"dtype" in lib.murm_last_error()


def test_torch_ops_keep_reference_schemas():
    from murmurative import murmurative_attention_ops  # noqa: F401  (registration only)
    ns = torch.ops.murmurative_attention
    for name, schema in REFERENCE_SCHEMAS.items():
        got = str(getattr(ns, name).default._schema)
        assert got == "murmurative_attention::" + schema, (name, got)
    for extra in ("slot_murmurate_fwd", "slot_murmurate_bwd", "slot_select_fwd", "slot_attend_fwd"):
        assert hasattr(ns, extra)


def test_public_names():
    assert sorted(murmurative.__all__) == sorted([
        "slot_select", "slot_attend", "slot_select_attend", "slot_update", "slot_diffusion", "slot_murmurate",
        "slot_select_reference", "slot_attend_reference", "slot_update_reference",
        "slot_diffusion_reference", "slot_murmurate_reference"])


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_hip_path_raises_without_gpu():
    q = torch.randn(1, 2, 16, 8)
    s = torch.randn(1, 2, 16, 8)
    ops._has_hip_kernels = None
    with pytest.raises(RuntimeError, match="GPU"):
        murmurative.slot_murmurate(q, s, s)
    with pytest.raises(RuntimeError):
        murmurative.slot_select_attend(q, s, s)
    x = torch.randn(1, 16, 8)
    with pytest.raises(RuntimeError):
        murmurative.slot_murmurate(x, x, x, x, torch.randn(2, 16, 4), torch.randn(2, 16, 4), num_heads=2)


def test_api_value_errors():
    x = torch.randn(1, 16, 10)
    e = torch.randn(3, 16, 3)
    with pytest.raises(ValueError, match="divisible"):
        murmurative.slot_murmurate(x, x, x, x, e, e, num_heads=3, use_reference=True)
    q = torch.randn(1, 2, 16, 8)
    s = torch.randn(1, 2, 16, 8)
    with pytest.raises(ValueError, match="top_k"):
        murmurative.slot_murmurate(q, s, s, rounds=2, top_k=5, use_reference=True)


def test_select_lds_bound_without_gpu():
    # the selecting entry points bound M by the LDS staging of one head's keys
    lib = capi.load()
    expect = {(capi.BF16, 32): 1024, (capi.BF16, 64): 560, (capi.BF16, 128): 288,
              (capi.F16, 64): 560, (capi.F32, 32): 1136, (capi.F32, 64): 592, (capi.F32, 128): 304}
    for (dt, D), m in expect.items():
        assert lib.murm_select_max_m(dt, D) == m, (dt, D)
    assert lib.murm_select_max_m(capi.BF16, 129) == 0 and lib.murm_select_max_m(9, 64) == 0
    # one slot past the bound is refused on the host, before any launch
    # (the tensor pointers are never dereferenced on this path)
    P = ctypes.c_void_p
    fake = P(4096)
    for dt, D in ((capi.BF16, 128), (capi.F32, 64)):
        M = lib.murm_select_max_m(dt, D) + 1
        rc = lib.murm_select_attend_fwd(dt, dt, 1, 1, 16, D, M, fake, 0, 0, D, fake, 0, 0, D, fake, 0, 0, D,
                                        None, 0, 0, 0, 0, None, 0, 0, 0, 0, 0, 0.0, 0, fake, 0, 0, D, fake, fake,
                                        fake, 1 << 40, None)
        assert rc == capi.ERR_UNSUPPORTED and b"LDS" in lib.murm_last_error(), (dt, D)
        rc = lib.murm_murmurate_fwd(dt, dt, 1, 1, 16, D, M, 3, 0.9, 0.15, 0, 0, 0.0, fake, 0, 0, D,
                                    None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0, fake, 0, 0, D, fake, 0, 0, D,
                                    None, 0, 0, 0, 0, fake, 0, 0, D, fake, fake, fake, 1 << 40, None)
        assert rc == capi.ERR_UNSUPPORTED and b"LDS" in lib.murm_last_error(), (dt, D)


def test_token_count_bound_without_gpu():
    # B*H*N of 2^31 tokens or more is refused on the host (the kernels number
    # token rows with 32 bits), before any launch
    lib = capi.load()
    P = ctypes.c_void_p
    fake = P(4096)
    B, H, N, D, M = 1, 128, 1 << 24, 64, 256
    rc = lib.murm_murmurate_fwd(capi.BF16, capi.BF16, B, H, N, D, M, 3, 0.9, 0.15, 0, 0, 0.0, fake, 0, 0, D,
                                None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0, fake, 0, 0, D, fake, 0, 0, D,
                                None, 0, 0, 0, 0, fake, 0, 0, D, fake, fake, fake, 1 << 40, None)
    assert rc == capi.ERR_UNSUPPORTED and b"tokens" in lib.murm_last_error()
