"""Graph replay of the fused rounds (murm_graph_replay): every replay must
give the bits of the direct launches, with the program's own eager work and
synchronisations between replays, also after an input changes in place (a
graph holds pointers, not data).  One graph is captured per distinct
argument set and reused."""

import ctypes

import pytest
import torch

import murmurative as MA
from murmurative import capi
from parity import seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = ctypes.c_void_p


def _s3(t):
    return t.stride(0), t.stride(1), t.stride(2)


def _fwd(lib, q, sk, sv, out, idx, w, ws, R):
    B, H, N, D = q.shape
    M = sk.shape[2]
    st = P(torch.cuda.current_stream().cuda_stream)
    rc = lib.murm_murmurate_fwd(capi.BF16, capi.BF16, B, H, N, D, M, R, 0.9, 0.15, 0, 0, 0.0,
                                P(q.data_ptr()), *_s3(q), None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0,
                                P(sk.data_ptr()), *_s3(sk), P(sv.data_ptr()), *_s3(sv), None, 0, 0, 0, 0,
                                P(out.data_ptr()), *_s3(out), P(idx.data_ptr()), P(w.data_ptr()),
                                P(ws.data_ptr()), ws.numel(), st)
    capi.check(rc, "murm_murmurate_fwd")


# Capture needs a real stream (not the legacy null stream torch uses by
# default); default priority.
def _side_stream():
    return torch.cuda.Stream()


def test_graph_replay_matches_direct_launches():
    print("case graph replay (C ABI, fixed buffers)", flush=True)
    with torch.cuda.stream(_side_stream()):
        _replay_c_abi()


def _replay_c_abi():
    lib = capi.load()
    B, H, N, D, M, R = 1, 4, 700, 64, 256, 3
    q, sk, sv = seeded([(B, H, N, D), (B, H, M, D), (B, H, M, D)], 91, [None, None, 0.02])
    q, sk, sv = (t.to(torch.bfloat16).to(DEV) for t in (q, sk, sv))
    ws = torch.empty(lib.murm_murmurate_workspace_bytes(B, H, N, D, M, R, 1), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    idx = torch.empty(B, H, N, 7, dtype=torch.int64, device=DEV)
    w = torch.empty(B, H, N, 7, dtype=torch.float32, device=DEV)

    def direct():
        capi.graph_replay(False)
        _fwd(lib, q, sk, sv, out, idx, w, ws, R)
        torch.cuda.synchronize()
        return out.clone(), idx.clone(), w.clone()

    ref = direct()
    try:
        capi.graph_replay(True)
        for rep in range(4):
            for t in (out, w):
                t.fill_(float("nan"))  # eager work on the same stream between replays
            idx.fill_(-1)
            torch.cuda.synchronize()
            _fwd(lib, q, sk, sv, out, idx, w, ws, R)
            torch.cuda.synchronize()
            assert torch.equal(out, ref[0]) and torch.equal(idx, ref[1]) and torch.equal(w, ref[2]), rep
        assert lib.murm_graph_cached() == 1
        # same pointers, new data: the replay reads the new values
        q.mul_(-1.0)
        torch.cuda.synchronize()
        _fwd(lib, q, sk, sv, out, idx, w, ws, R)
        torch.cuda.synchronize()
        got = (out.clone(), idx.clone(), w.clone())
        assert lib.murm_graph_cached() == 1
    finally:
        capi.graph_replay(False)
    ref2 = direct()
    for a, b in zip(got, ref2):
        assert torch.equal(a, b)
    assert lib.murm_graph_cached() == 0


def test_graph_replay_through_autograd():
    # forward + backward through the public API: the caching allocator hands
    # the op the same buffers call after call, so the graphs are replayed
    print("case graph replay (autograd)", flush=True)
    B, H, N, D, M = 1, 4, 900, 64, 256
    q, sk, sv, go = seeded([(B, H, N, D), (B, H, M, D), (B, H, M, D), (B, H, N, D)], 93, [None, None, 0.02, None])
    q, sk, sv, go = (t.to(torch.bfloat16).to(DEV) for t in (q, sk, sv, go))

    def step():
        qa, ska, sva = (t.clone().requires_grad_(True) for t in (q, sk, sv))
        out, idx, w = MA.slot_murmurate(qa, ska, sva, rounds=3)
        out.backward(go)
        torch.cuda.synchronize()
        return [t.detach().clone() for t in (out, idx, w, qa.grad, ska.grad, sva.grad)]

    torch.cuda.synchronize()  # inputs were made on the default stream
    with torch.cuda.stream(_side_stream()):
        capi.graph_replay(False)
        ref = step()
        try:
            capi.graph_replay(True)
            for rep in range(4):
                got = step()
                for a, b in zip(got, ref):
                    assert torch.equal(a, b), rep
            assert capi.load().murm_graph_cached() >= 2
        finally:
            capi.graph_replay(False)
