"""The allocation-free entry point murm_select_attend_fwd_noalloc against the
workspace entry point murm_select_attend_fwd it shares its kernels with:
bit-identical outputs on two calls in a row (the second smaller, so the
device scratch holds the first call's larger contents), for 16-bit and
float32 tokens; shapes beyond the scratch are refused on the host."""

import ctypes

import pytest
import torch

from murmurative import capi
from parity import seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = ctypes.c_void_p


def _s3(t):
    return t.stride(0), t.stride(1), t.stride(2)


def _run(lib, noalloc, code, q, sk, sv, causal):
    B, H, N, D = q.shape
    M = sk.shape[2]
    out = torch.full_like(q, float("nan"))
    w = torch.full((B, H, N, 7), float("nan"), device=DEV)
    idx = torch.full((B, H, N, 7), -1, dtype=torch.int64, device=DEV)
    st = P(torch.cuda.current_stream().cuda_stream)
    head = [code, code, B, H, N, D, M, P(q.data_ptr()), *_s3(q), P(sk.data_ptr()), *_s3(sk),
            P(sv.data_ptr()), *_s3(sv), None, 0, 0, 0, 0, None, 0, 0, 0, 0, int(causal), 0.0, 0,
            P(out.data_ptr()), *_s3(out), P(w.data_ptr()), P(idx.data_ptr())]
    if noalloc:
        rc = lib.murm_select_attend_fwd_noalloc(*head, st)
    else:
        n = lib.murm_select_attend_workspace_bytes(B, H, N, D, M)
        ws = torch.empty(n, dtype=torch.uint8, device=DEV)
        rc = lib.murm_select_attend_fwd(*head, P(ws.data_ptr()), n, st)
    capi.check(rc, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return out.cpu(), w.cpu(), idx.cpu()


@pytest.mark.parametrize("dtype,code", [(torch.bfloat16, capi.BF16), (torch.float32, capi.F32)],
                         ids=["bf16", "f32"])
def test_noalloc_matches_workspace_entry(dtype, code):
    lib = capi.load()
    # (B, H, N, D, M, causal): the second call is smaller than the first
    for i, (B, H, N, D, M, causal) in enumerate([(2, 4, 1000, 64, 256, False), (1, 2, 300, 32, 96, True)]):
        print("case noalloc", dtype, i, (B, H, N, D, M, causal), flush=True)
        q, sk, sv = seeded([(B, H, N, D), (B, H, M, D), (B, H, M, D)], 61 + i, [None, None, 0.1])
        q, sk, sv = (t.to(dtype).to(DEV) for t in (q, sk, sv))
        ref = _run(lib, False, code, q, sk, sv, causal)
        got = _run(lib, True, code, q, sk, sv, causal)
        for name, a, b in zip(("out", "weights", "indices"), got, ref):
            assert torch.equal(a, b), f"call {i}: {name} differs from the workspace entry point"
        assert int(got[2].min()) >= 0 and int(got[2].max()) < M


def test_noalloc_refuses_shapes_beyond_its_scratch():
    lib = capi.load()
    B, H, N, D, M = 1, 64, 65536, 128, 256
    need = lib.murm_select_attend_workspace_bytes(B, H, N, D, M)
    assert need > capi.NOALLOC_SCRATCH_BYTES
    fake = P(4096)  # never dereferenced: the size check comes first
    rc = lib.murm_select_attend_fwd_noalloc(capi.BF16, capi.BF16, B, H, N, D, M, fake, 0, 0, D, fake, 0, 0, D,
                                            fake, 0, 0, D, None, 0, 0, 0, 0, None, 0, 0, 0, 0, 0, 0.0, 0,
                                            fake, 0, 0, D, fake, fake, None)
    assert rc == capi.ERR_UNSUPPORTED
    assert b"scratch" in lib.murm_last_error()
