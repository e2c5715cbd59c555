"""Benchmark: slot_murmurate forward+backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu]

--config 1/2/3/4 run the op on BASELINE.json configs[0..3] (config 1, the
README verify call, forward + backward here); --config 5 runs the README
MurmurativeAttention layer's training step.

A step is one forward+backward of the README-form slot_murmurate over one
synthetic batch (seeded N(0,1) draws), inputs resident
in HBM.  `value` is tokens/s over exactly K timed steps (HIP-synchronised on
both sides).  A second pass over the same K steps has every kernel launch
record start/stop HIP events from its own dispatch (hipExtLaunchKernel, on
the stream the kernels run on) for the per-kernel durations behind the
roofline fraction.  The CPU baseline times the CPU oracle (a PyTorch
restatement of the reference's reference.py) on the host's CPU share.
`measured_peaks` puts a streaming copy's GB/s and a large bf16 GEMM's TFLOP/s
beside the spec peaks.  Prints one JSON line.
"""

import argparse
import contextlib
import json
import math
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "murmurative-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "tokens/sec fwd+bwd slot_murmurate H=16 N=8192 d=64 bf16; % of roofline"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

CONFIGS = {
    # name: (B, H, N, D, M, rounds, causal, dtype, slots_k std, slots_v std)
    # config 1 is the README verify call (forward, fp32); here it is timed
    # forward + backward like the others
    "1": (2, 4, 128, 64, 256, 3, False, "float32", 1.0, 0.0),
    "2": (4, 8, 2048, 64, 256, 3, False, "float16", 1.0, 0.02),
    "3": (1, 16, 8192, 64, 256, 3, False, "bfloat16", 1.0, 0.02),
    "4": (1, 16, 65536, 128, 256, 3, True, "bfloat16", 1.0, 0.02),
}


def byte_model(B, H, N, D, M, R, e):
    """Algorithmic HBM bytes per launch of each kernel class (README form).

    Every tensor is counted once per launch: tokens q / grad_out / out (T*D*e),
    u16 index rows (T*16), float32 weights and softmax grads (T*28), float32
    slot tables [B*H,M,D] (S), weight sums (B*H*M*4)."""
    T = B * H * N
    tok = T * D * e
    S = B * H * M * D * 4
    idx, w = T * 16, T * 28
    Wb = B * H * M * 4
    per_launch = {
        # q + slot keys in; u16 indices and weights out (+ int64 indices in the last round)
        "select_attend": (R * (tok + S + idx + w) + T * 56) / R,
        # q, R rounds of (indices, weights, value table) in; out written
        "gather_out": tok + R * (idx + w + S) + tok,
        # token-chunk partial sums of the update: q, indices, weights in (the
        # partials themselves are scratch, not algorithmic traffic)
        "seg_update": tok + idx + w,
        # chunk reduction + EMA + diffusion: 2 old slot tables in; 2 new tables,
        # key sums, weight sums out
        "seg_update_reduce": 2 * S + 2 * S + S + Wb,
        # partial sums of the slot-side attend backward: q, grad_out, ds, weights, indices in
        "seg_attbwd": 2 * tok + w + w + idx,
        # reduction + carry + previous round's diffusion adjoint / EMA backward:
        # 2 carries, key sums, weight sums in; dK, 2 carries, dW out
        "seg_attbwd_reduce": 2 * S + S + Wb + 3 * S + Wb,
        # 2 grads, key sums, weight sums in; dK, 2 carries, dW out
        "du": 2 * S + S + Wb + 3 * S + Wb,
        # grad_out, q, indices, weights, value table, dK, dW in; ds out (external grad_w once)
        "tok_bwd": 2 * tok + idx + w + 2 * S + Wb + w,
        # grad_out in; R rounds of (indices, weights, ds, key table, dK) in; dq out
        "tok_grad": tok + R * (idx + 2 * w + 2 * S) + tok,
        # input slots in (2 tables, 16-bit) + fp32 states out, and fp32 grads -> 16-bit slot grads
        "conversions": 2 * (B * H * M * D * e) + 2 * S,
    }
    flops = {"select_attend": 2.0 * T * M * D}
    return per_launch, flops


def call_bytes(B, H, N, D, M, R, e):
    """Algorithmic HBM bytes of one whole fwd+bwd call (one read of every input
    and one write of every output per phase, fp32 slot state, int32-sized
    indices): select+attend 2q+2s+i+w in round 0 and 3q+2s+i+w after it,
    update+diffuse q+i+w+4s, int64 API indices i; backward per round token side
    4q+i+w+2s, slot side 2q+i+w+2s, EMA/diffusion 6s, minus the first round's
    dq read."""
    T = B * H * N
    q, s, i, w = T * D * e, B * H * M * D * 4, T * 7 * 4, T * 7 * 4
    fwd = (2 * q + 2 * s + i + w) + (R - 1) * (3 * q + 2 * s + i + w) + R * (q + i + w + 4 * s) + i
    bwd = R * ((4 * q + i + w + 2 * s) + (2 * q + i + w + 2 * s) + 6 * s) - q
    return fwd + bwd


TRAFFIC_FILES = {
    "3": "slot_murmurate_fwd_bwd_headline_hbm_traffic.md",
    "4": "slot_murmurate_fwd_bwd_config4_hbm_traffic.md",
    "5": "murmurative_attention_layer_config5_hbm_traffic.md",
}


def traffic_file(config):
    name = TRAFFIC_FILES.get(config)
    return os.path.join(ROOT, "profiles", name) if name else None


def measured_traffic(config):
    """HBM bytes per launch of each timing class, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this configuration (copy-kernel
    calibrated); {} when there is none."""
    path = traffic_file(config)
    if not path or not os.path.exists(path):
        return {}
    out = {}
    for line in open(path):
        if line.startswith("traffic: "):
            _, cls, val = line.split()
            out[cls] = int(val)
    return out


# config 5: the README's MurmurativeAttention layer (README.md:82-101) trained one step
MODULE_CONFIGS = {
    "5": {"dim": 1024, "heads": 16, "slots": 512, "B": 8, "N": 4096, "rounds": 3, "dtype": "bfloat16",
          "lr": 5e-4, "eps": 1e-4},
}


def readme_module(torch, murmurate):
    """The layer of README.md:82-101 over a given slot_murmurate implementation."""
    nn = torch.nn

    class MurmurativeAttention(nn.Module):
        def __init__(self, dim, heads, slots, rounds=3):
            super().__init__()
            self.heads, self.slots, self.rounds = heads, slots, rounds
            self.dim, self.head_dim = dim, dim // heads
            self.q_proj = nn.Linear(dim, dim, bias=False)
            self.o_proj = nn.Linear(dim, dim, bias=False)
            self.slot_embeddings = nn.Parameter(torch.randn(heads, slots, self.head_dim))

        def forward(self, x):
            B, N, D = x.shape
            q = self.q_proj(x).view(B, N, self.heads, self.head_dim).transpose(1, 2)
            slots_k = self.slot_embeddings.unsqueeze(0).expand(B, -1, -1, -1)
            slots_v = torch.zeros_like(slots_k)
            attn_out = murmurate(q, slots_k, slots_v, self.rounds)[0]
            return self.o_proj(attn_out.transpose(1, 2).contiguous().view(B, N, D))

    return MurmurativeAttention


def make_module(mc, device, batch=None, seed=42):
    """Seeded layer + input + target: Linear weights ~ N(0, 0.02), slot embeddings
    ~ N(0, 1), x and target ~ N(0, 1), drawn in fp32 on the CPU in that order."""
    import torch
    import murmurative
    if device.type == "cuda":
        fn = lambda q, k, v, r: murmurative.slot_murmurate(q, k, v, rounds=r)
    else:
        from oracle import murm_oracle as O
        fn = lambda q, k, v, r: O.murmurate_readme(q, k, v, rounds=r)
    dt = getattr(torch, mc["dtype"])
    B = mc["B"] if batch is None else batch
    g = torch.Generator().manual_seed(seed)
    model = readme_module(torch, fn)(mc["dim"], mc["heads"], mc["slots"], mc["rounds"])
    with torch.no_grad():
        model.q_proj.weight.copy_(torch.randn(model.q_proj.weight.shape, generator=g) * 0.02)
        model.o_proj.weight.copy_(torch.randn(model.o_proj.weight.shape, generator=g) * 0.02)
        model.slot_embeddings.copy_(torch.randn(model.slot_embeddings.shape, generator=g))
    x = torch.randn(B, mc["N"], mc["dim"], generator=g)
    target = torch.randn(B, mc["N"], mc["dim"], generator=g)
    model = model.to(device=device, dtype=dt)
    opt = torch.optim.AdamW(model.parameters(), lr=mc["lr"], eps=mc["eps"])
    return model, opt, x.to(device=device, dtype=dt), target.to(device=device, dtype=dt)


def module_step(torch, model, opt, x, target):
    opt.zero_grad(set_to_none=True)
    loss = torch.nn.functional.mse_loss(model(x).float(), target.float())
    loss.backward()
    opt.step()
    return loss


def host_cpu():
    """The host cores the CPU baseline may use and how they were counted.

    threads = the process's CPU share: the cgroup quota when one is set, else
    the CPUs in its affinity mask, capped by OMP_NUM_THREADS when that is set
    (one GPU's share of the box's host cores)."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        info["affinity_cpus"] = os.cpu_count()
    share = info["affinity_cpus"] or 1
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            info["cgroup_cpu_quota"] = round(int(quota) / int(period), 2)
            share = min(share, max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        info["OMP_NUM_THREADS"] = int(omp)
        share = min(share, int(omp))
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                info["model"] = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return share, info


def cpu_baseline_module(mc, budget_s=20.0):
    """Time the same training step on the host with the CPU oracle in place of
    the kernels: batch 1, the sequence length cut to fit the time budget."""
    import torch
    threads, host = host_cpu()
    torch.set_num_threads(threads)
    cpu = torch.device("cpu")

    def run(n):
        m = dict(mc, N=n)
        model, opt, x, target = make_module(m, cpu, batch=1)
        t0 = time.perf_counter()
        module_step(torch, model, opt, x, target)
        return time.perf_counter() - t0

    run(256)  # warm-up
    n = 256
    while n < mc["N"] and run(n) * 2 * 3 < budget_s:
        n *= 2
    times = sorted(run(n) for _ in range(3))
    med = times[1]
    return {"value": round(n / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "host": host,
            "sample": (f"README layer training step (MSE, AdamW) with oracle/murm_oracle.py murmurate_readme "
                       f"in place of the kernels, {mc['dtype']}, B=1, N={n}, dim={mc['dim']}, heads={mc['heads']}, "
                       f"slots={mc['slots']}, R={mc['rounds']}; median of 3, {med:.3f} s; tokens/s = N / time")}


def make_inputs(cfg, device, seed=42):
    import torch
    B, H, N, D, M, R, causal, dt, sk_std, sv_std = cfg
    dtype = getattr(torch, dt)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, D, generator=g)
    sk = torch.randn(B, H, M, D, generator=g) * sk_std
    sv = torch.randn(B, H, M, D, generator=g) * sv_std
    go = torch.randn(B, H, N, D, generator=g)
    return [t.to(dtype).to(device) for t in (q, sk, sv, go)]


def cpu_baseline(cfg, budget_s=20.0):
    """Time the CPU oracle's forward+backward (autograd) on a bounded head sample."""
    import torch
    from oracle import murm_oracle as O
    B, H, N, D, M, R, causal, dt, _, _ = cfg
    threads, host = host_cpu()
    torch.set_num_threads(threads)
    q, sk, sv, go = make_inputs(cfg, "cpu", seed=42)

    def run(h):
        qq, kk, vv = (t[:, :h].detach().clone().requires_grad_(True) for t in (q, sk, sv))
        t0 = time.perf_counter()
        out, _, _ = O.murmurate_readme(qq, kk, vv, rounds=R, causal=causal)
        torch.autograd.grad(out, (qq, kk, vv), go[:, :h])
        return time.perf_counter() - t0

    run(1)  # warm-up
    t1 = run(1)
    heads = max(1, min(H, int(budget_s / 3.0 / max(t1, 1e-3))))
    times = sorted(run(heads) for _ in range(3))
    med = times[1]
    # heads are independent: the full call costs H/heads times the sample
    tok_s = B * N * heads / (H * med)
    return {"value": round(tok_s, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "host": host,
            "sample": (f"oracle/murm_oracle.py murmurate_readme fwd+bwd (autograd), {dt} inputs, "
                       f"B={B}, {heads} of {H} heads, N={N}, d={D}, M={M}, R={R}; median of 3 after "
                       f"1 warm-up, {med:.3f} s; tokens/s = B*N*(heads/H) / time")}


def measured_peaks(torch, dev):
    """Achievable HBM bandwidth and dense bf16 matrix rate on this GPU, beside
    the spec peaks: a 1 GiB device-to-device copy (torch copy kernel; bytes
    read + written) and an 8192^3 bf16 GEMM (torch.matmul -> hipBLASLt)."""
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    n = (1 << 30) // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    e0, e1 = ev(), ev()
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 10 * 2 * n * 4 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    K = 8192
    x = torch.randn(K, K, device=dev, dtype=torch.bfloat16)
    y = torch.randn(K, K, device=dev, dtype=torch.bfloat16)
    for _ in range(3):
        z = torch.matmul(x, y)
    e0, e1 = ev(), ev()
    e0.record()
    for _ in range(10):
        z = torch.matmul(x, y)
    e1.record()
    torch.cuda.synchronize()
    gemm_tf = 10 * 2 * K ** 3 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    del x, y, z
    return {"copy_GB_s": round(copy_gbs, 1), "hbm_spec_GB_s": HBM_PEAK_GBS,
            "copy_frac_of_spec": round(copy_gbs / HBM_PEAK_GBS, 4),
            "bf16_gemm_TFLOP_s": round(gemm_tf, 1), "bf16_dense_spec_TFLOP_s": MFMA_BF16_PEAK_TFLOPS,
            "gemm_frac_of_spec": round(gemm_tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "how": "1 GiB float32 copy_ x10 (read + write bytes); 8192^3 bf16 torch.matmul x10; HIP events"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="3", choices=sorted(list(CONFIGS) + list(MODULE_CONFIGS)))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-peaks", action="store_true", help="skip the copy / GEMM peak measurement")
    ap.add_argument("--graphs", action="store_true",
                    help="replay the fused rounds' kernels from captured hipGraphs (murm_graph_replay)")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the timed passes, copy a MIB-MiB tensor 3 times (a plain copy kernel of known "
                         "size, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {a.gpus}); the kernels run per (b,h) "
              f"with no cross-GPU work in this build.", file=sys.stderr)
        return 2

    import torch
    import murmurative
    from murmurative import capi

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    capi.graph_replay(a.graphs)
    module = a.config in MODULE_CONFIGS
    if module:
        mc = MODULE_CONFIGS[a.config]
        B, N, M, R, dt = mc["B"], mc["N"], mc["slots"], mc["rounds"], mc["dtype"]
        H, D, causal = mc["heads"], mc["dim"] // mc["heads"], False
        model, opt, x, target = make_module(mc, dev)

        def step():
            return module_step(torch, model, opt, x, target)
    else:
        cfg = CONFIGS[a.config]
        B, H, N, D, M, R, causal, dt, _, _ = cfg
        q, sk, sv, go = make_inputs(cfg, dev)
        for t in (q, sk, sv):
            t.requires_grad_(True)

        def step():
            out, idx, w = murmurative.slot_murmurate(q, sk, sv, rounds=R, causal=causal)
            return torch.autograd.grad(out, (q, sk, sv), go)

    # graph capture needs a stream other than the legacy null stream torch
    # runs on by default (default priority)
    side = torch.cuda.Stream() if a.graphs else None
    with torch.cuda.stream(side) if side is not None else contextlib.nullcontext():
        for _ in range(a.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    ms_per_step = 1e3 * elapsed / a.steps
    value = B * N * a.steps / elapsed

    # second pass: HIP events around every launch, same K steps
    capi.timing_reset()
    capi.timing_enable(True)
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    capi.timing_enable(False)
    kt = capi.timing_read()
    capi.timing_reset()

    e = 2 if dt in ("bfloat16", "float16") else 4
    per_launch, flops = byte_model(B, H, N, D, M, R, e)
    kernels = {}
    for name, (ms, n) in kt.items():
        avg_us = 1e3 * ms / n
        gbs = per_launch.get(name, 0.0) / (avg_us * 1e-6) / 1e9
        kernels[name] = {"launches_per_step": n / a.steps, "avg_us": round(avg_us, 2),
                         "ms_per_step": round(ms / a.steps, 4), "GB_s": round(gbs, 1),
                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    dom = max(kt, key=lambda k: kt[k][0])
    dk = kernels[dom]
    traffic = measured_traffic(a.config)
    roofline = {"kernel": dom, "bound": "hbm", "achieved": dk["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dk["GB_s"] / HBM_PEAK_GBS, 4), "traffic": traffic.get(dom),
                "bytes_per_launch": int(per_launch[dom]), "avg_us": dk["avg_us"],
                "timing": (f"HIP start/stop events recorded by every launch's own dispatch "
                           f"(hipExtLaunchKernel) on the kernels' stream, over {a.steps} steps")}
    if traffic.get(dom) is not None:
        roofline["traffic_source"] = os.path.relpath(traffic_file(a.config), ROOT)
    if "select_attend" in kt:
        # algorithmic score-GEMM FLOPs over the launch time (the MFMA busy
        # fraction from hardware counters is in profiles/)
        tf = flops["select_attend"] / (kernels["select_attend"]["avg_us"] * 1e-6) / 1e12
        kernels["select_attend"]["score_gemm_TFLOPs"] = round(tf, 2)
        kernels["select_attend"]["score_gemm_frac_of_bf16_peak"] = round(tf / MFMA_BF16_PEAK_TFLOPS, 4)
    device_ms = sum(ms for ms, _ in kt.values()) / a.steps
    # the whole call against the HBM floor of its algorithmic bytes (slot_murmurate only)
    cb = call_bytes(B, H, N, D, M, R, e)
    t_roof_us = cb / (HBM_PEAK_GBS * 1e9) * 1e6
    call_roofline = {"bytes": int(cb), "t_roof_us": round(t_roof_us, 2),
                     "kernel_us_per_step": round(1e3 * device_ms, 2),
                     "frac_of_kernel_time": round(t_roof_us / (1e3 * device_ms), 4)}
    if not module:
        call_roofline["frac_of_step_time"] = round(t_roof_us / (1e3 * ms_per_step), 4)

    dname = {"bfloat16": "bf16", "float16": "fp16", "float32": "fp32"}[dt]
    if module:
        metric = f"tokens/sec MurmurativeAttention layer training step dim={mc['dim']} heads={H} slots={M} {dname}"
        data = "synthetic: seeded N(0,1) input and target, Linear weights ~ N(0,0.02), slot embeddings ~ N(0,1)"
        config = {"workload": "README MurmurativeAttention layer: fwd + MSE + bwd + AdamW, BASELINE configs[4]",
                  "B": B, "N": N, "dim": mc["dim"], "heads": H, "head_dim": D, "slots": M, "top_k": 7,
                  "rounds": R, "lr": mc["lr"], "adam_eps": mc["eps"], "tokens_per_step": B * N}
    else:
        metric = METRIC if a.config == "3" else (
            f"tokens/sec fwd+bwd slot_murmurate B={B} H={H} N={N} d={D} M={M}{' causal' if causal else ''} {dname}")
        data = "synthetic: seeded N(0,1) draws shaped as BASELINE.json configs (slots_v ~ N(0,0.02))"
        config = {"workload": f"slot_murmurate README form fwd+bwd, BASELINE configs[{int(a.config) - 1}]",
                  "B": B, "H": H, "N": N, "head_dim": D, "M": M, "top_k": 7, "rounds": R, "causal": causal,
                  "tokens_per_step": B * N}
    res = {
        "metric": metric, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dname, "data": data, "config": config,
        "launches": "hipGraph replay (murm_graph_replay)" if a.graphs else "direct kernel launches",
        "roofline": roofline,
        "call_roofline": call_roofline,
        "kernels": kernels,
        "device_ms_per_step_in_kernels": round(device_ms, 4),
    }
    if not a.no_peaks:
        res["measured_peaks"] = measured_peaks(torch, dev)
    if a.copy_calibration > 0:
        n = a.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_calibration_bytes_each_way"] = n * 4
        del src, dst
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline_module(mc, a.cpu_budget) if module else cpu_baseline(cfg, a.cpu_budget)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
