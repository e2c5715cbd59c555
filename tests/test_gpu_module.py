"""The README's MurmurativeAttention nn.Module (README.md:77-101) trained one
step on the GPU: projections, slot_murmurate over an expanded slot-embedding
parameter with zero slot values, MSE loss, backward, AdamW.

The slot_murmurate call inside the module is checked against the CPU oracle
replaying the kernel's per-round selections (tests/parity.py protocol): the
attention output, the gradient reaching q, and the slot-embedding gradient
summed over the batch through expand().  The step then has to move every
parameter by a finite amount.  M = 512 also exercises the kernels' large-M
paths (per-slot-group reductions, L2 gathers)."""

import pytest
import torch
import torch.nn as nn

import murmurative as MA
from murmurative import slot_murmurate
from oracle import murm_oracle as O
from parity import assert_close, check_selection, round_indices

pytestmark = pytest.mark.gpu
DEV = "cuda"


class MurmurativeAttention(nn.Module):
    """The module of README.md:82-101, unchanged."""

    def __init__(self, dim=256, heads=4, slots=256, rounds=3, top_k=7):
        super().__init__()
        self.heads = heads
        self.slots = slots
        self.rounds = rounds
        self.top_k = top_k
        self.dim = dim
        self.head_dim = dim // heads
        self.q_proj = nn.Linear(dim, dim, bias=False)
        self.o_proj = nn.Linear(dim, dim, bias=False)
        self.slot_embeddings = nn.Parameter(torch.randn(heads, slots, self.head_dim))

    def forward(self, x):
        B, N, D = x.shape
        q = self.q_proj(x).view(B, N, self.heads, self.head_dim).transpose(1, 2)
        slots_k = self.slot_embeddings.unsqueeze(0).expand(B, -1, -1, -1)
        slots_v = torch.zeros_like(slots_k)
        attn_out, _, _ = slot_murmurate(q, slots_k, slots_v, rounds=self.rounds)
        attn_out = attn_out.transpose(1, 2).contiguous().view(B, N, D)
        return self.o_proj(attn_out)


class _Recorder:
    """Delegates to the op library and records slot_murmurate_fwd's inputs and outputs."""

    def __init__(self, lib):
        self._lib = lib
        self.calls = []

    def __getattr__(self, name):
        return getattr(self._lib, name)

    def slot_murmurate_fwd(self, *args):
        res = self._lib.slot_murmurate_fwd(*args)
        self.calls.append((args, res))
        return res


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_module_training_step(dtype, monkeypatch):
    print("case module", dtype, flush=True)
    torch.manual_seed(42)
    dim, heads, slots, B, N, R = 256, 4, 512, 2, 256, 3
    model = MurmurativeAttention(dim=dim, heads=heads, slots=slots, rounds=R)
    with torch.no_grad():  # Linear ~ N(0, 0.02), slot embeddings ~ N(0, 1)
        model.q_proj.weight.normal_(0.0, 0.02)
        model.o_proj.weight.normal_(0.0, 0.02)
    model = model.to(DEV, dtype)
    g = torch.Generator().manual_seed(43)
    x = torch.randn(B, N, dim, generator=g).to(DEV, dtype)
    target = torch.randn(B, N, dim, generator=g).to(DEV, dtype)

    rec = _Recorder(MA.ops._get_lib())
    monkeypatch.setattr(MA.ops, "_get_lib", lambda: rec)
    attn = {}
    model.o_proj.register_forward_hook(lambda m, i, o: attn.__setitem__("in", i[0].detach()))
    model.o_proj.register_full_backward_hook(lambda m, gi, go: attn.__setitem__("grad", gi[0].detach()))
    qgrad = {}

    def grab_q(mod, inp, out):
        out.register_hook(lambda gr: qgrad.__setitem__("q", gr.detach()))
    model.q_proj.register_forward_hook(grab_q)

    opt = torch.optim.AdamW(model.parameters(), lr=5e-4, eps=1e-4)
    before = [p.detach().clone() for p in model.parameters()]
    loss = torch.nn.functional.mse_loss(model(x).float(), target.float())
    loss.backward()
    g_slots = model.slot_embeddings.grad.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    assert torch.isfinite(loss)
    for p0, p in zip(before, model.parameters()):
        assert torch.isfinite(p).all()
        assert not torch.equal(p0, p.detach()), "AdamW left a parameter unchanged"

    # the fused op inside the module, replayed by the oracle
    assert len(rec.calls) == 1
    args, (out, idx, w, ws) = rec.calls[0]
    q, sk = args[0], args[4]
    D, M = dim // heads, slots
    per_round = [round_indices(ws, B, heads, N, D, M, R, True, r) for r in range(R - 1)] + [idx]
    q64 = q.detach().cpu().double().requires_grad_(True)
    emb64 = sk.detach()[0].cpu().double().requires_grad_(True)  # the op's input, not the post-step parameter
    sk64 = emb64.unsqueeze(0).expand(B, -1, -1, -1)
    out64, _, _, trace = O.murmurate_readme(q64, sk64, torch.zeros_like(sk64), R, return_trace=True,
                                            forced_idx=[t.cpu() for t in per_round])
    for r in range(R):
        check_selection(f"round {r} indices", per_round[r], trace[r][4])
    got_attn = attn["in"].view(B, N, heads, D).transpose(1, 2)
    assert_close("attention output", got_attn, out64, dtype)
    g_attn = attn["grad"].view(B, N, heads, D).transpose(1, 2).cpu().double()
    out64.backward(g_attn)
    got_gq = qgrad["q"].view(B, N, heads, D).transpose(1, 2)
    assert_close("grad q", got_gq, q64.grad, dtype)
    assert_close("grad slot embeddings", g_slots, emb64.grad, dtype)


@pytest.mark.timeout(600)
def test_module_training_step_config5_full_size(monkeypatch):
    # BASELINE configs[4] at full size: dim 1024, heads 16 (head_dim 64),
    # slots 512, B 8, N 4096, bf16, AdamW.  Heads are independent, so the
    # oracle replays heads 0 and 15 over the whole batch (the slot-embedding
    # gradient of a head sums over the batch).
    print("case module config 5 full size", flush=True)
    dtype = torch.bfloat16
    dim, heads, slots, B, N, R = 1024, 16, 512, 8, 4096, 3
    g = torch.Generator().manual_seed(42)
    model = MurmurativeAttention(dim=dim, heads=heads, slots=slots, rounds=R)
    with torch.no_grad():  # Linear ~ N(0, 0.02), slot embeddings ~ N(0, 1), drawn in that order
        model.q_proj.weight.copy_(torch.randn(model.q_proj.weight.shape, generator=g) * 0.02)
        model.o_proj.weight.copy_(torch.randn(model.o_proj.weight.shape, generator=g) * 0.02)
        model.slot_embeddings.copy_(torch.randn(model.slot_embeddings.shape, generator=g))
    x = torch.randn(B, N, dim, generator=g).to(DEV, dtype)
    target = torch.randn(B, N, dim, generator=g).to(DEV, dtype)
    model = model.to(DEV, dtype)

    rec = _Recorder(MA.ops._get_lib())
    monkeypatch.setattr(MA.ops, "_get_lib", lambda: rec)
    attn = {}
    model.o_proj.register_forward_hook(lambda m, i, o: attn.__setitem__("in", i[0].detach()))
    model.o_proj.register_full_backward_hook(lambda m, gi, go: attn.__setitem__("grad", gi[0].detach()))
    qgrad = {}

    def grab_q(mod, inp, out):
        out.register_hook(lambda gr: qgrad.__setitem__("q", gr.detach()))
    model.q_proj.register_forward_hook(grab_q)

    opt = torch.optim.AdamW(model.parameters(), lr=5e-4, eps=1e-4)
    before = [p.detach().clone() for p in model.parameters()]
    loss = torch.nn.functional.mse_loss(model(x).float(), target.float())
    loss.backward()
    g_slots = model.slot_embeddings.grad.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    assert torch.isfinite(loss)
    for p0, p in zip(before, model.parameters()):
        assert torch.isfinite(p).all()
        assert not torch.equal(p0, p.detach()), "AdamW left a parameter unchanged"

    assert len(rec.calls) == 1
    args, (out, idx, w, ws) = rec.calls[0]
    q, sk = args[0], args[4]
    D, M = dim // heads, slots
    per_round = [round_indices(ws, B, heads, N, D, M, R, True, r) for r in range(R - 1)] + [idx.cpu()]
    got_attn = attn["in"].view(B, N, heads, D).transpose(1, 2)
    g_attn = attn["grad"].view(B, N, heads, D).transpose(1, 2)
    got_gq = qgrad["q"].view(B, N, heads, D).transpose(1, 2)
    for h in (0, heads - 1):
        sl = slice(h, h + 1)
        q64 = q.detach()[:, sl].cpu().float().requires_grad_(True)
        emb64 = sk.detach()[0, h].cpu().float().requires_grad_(True)  # the op's input for head h
        sk64 = emb64.view(1, 1, M, D).expand(B, 1, M, D)
        forced = [p[:, sl].cpu() for p in per_round]
        out64, _, _, trace = O.murmurate_readme(q64, sk64, torch.zeros_like(sk64), R, return_trace=True,
                                                forced_idx=forced)
        for r in range(R):
            check_selection(f"head {h} round {r} indices", forced[r], trace[r][4])
        assert_close(f"head {h} attention output", got_attn[:, sl], out64, dtype)
        out64.backward(g_attn[:, sl].cpu().float())
        assert_close(f"head {h} grad q", got_gq[:, sl], q64.grad, dtype)
        assert_close(f"head {h} grad slot embeddings", g_slots[h], emb64.grad, dtype)
