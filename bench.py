"""Benchmark: causal polynomial attention fwd+bwd TFLOP/s on one MI355X (BASELINE.json headline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1b] [--cpu-seconds S] [--no-cpu-baseline]

A step is one forward + backward of the polynomial attention operator (kind "power", degree 2, which equals the
reference's signed_product with shared pairs) over one batch of seeded synthetic bf16 inputs resident in HBM:
q, k ~ N(0,1)/D^(1/4), v, dO ~ N(0,1), one causal document per row, row scale (t+1)^-1/2.

FLOP convention (exact causal pairs, power and mask not counted): Npairs = T(T+1)/2,
fwd = 4*B*H*Npairs*D, fwd+bwd = 14*B*H*Npairs*D. Peak: MI355X dense bf16 MFMA, 2.5 PFLOP/s.
Prints one JSON line (rank 0). The CPU baseline times the CPU oracle (oracle/, float32 numpy) on a bounded
sample of (b, h) slices of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = "poly-attn fwd+bwd TFLOP/s at B8 H16 T2048 D128 bf16; % of MI355X MFMA peak"

CONFIGS = {  # name: (B, H, T, D, degree, boost_rows, seed) -- BASELINE.json configs[1..4]
    "100m": (16, 12, 1024, 64, 2, 0.0, 1),
    "1b": (8, 16, 2048, 128, 2, 0.0, 2),
    "p4": (4, 16, 2048, 128, 4, 0.01, 3),
    "7b": (2, 32, 4096, 128, 2, 0.0, 4),
}


def npairs(T):
    return T * (T + 1) // 2


def make_inputs(B, H, T, D, boost, seed, device):
    import torch
    g = torch.Generator().manual_seed(seed)
    mk = lambda s: (torch.randn(B, H, T, D, generator=g) * s)  # noqa: E731
    q, k = mk(D ** -0.25), mk(D ** -0.25)
    if boost:
        for x in (q, k):
            rows = torch.rand(B, T, generator=g) < boost
            x.mul_(torch.where(rows, 4.0, 1.0)[:, None, :, None])
    v, do = mk(1.0), mk(1.0)
    q, k, v, do = (x.to(torch.bfloat16).to(device) for x in (q, k, v, do))
    doc = torch.zeros(B, T, dtype=torch.long, device=device)
    rs = (torch.arange(T, device=device, dtype=torch.float32) + 1).pow(-0.5).expand(B, T).contiguous()
    return q, k, v, do, doc, rs


def time_events(fn, reps):
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


def kernel_times(q, k, v, do, doc, rs, degree, reps):
    """Average duration (ms) of each launch of the fwd, dV, dK and dQ kernels (and of the dO pre-scaling pass when the
    operator uses it), timed with HIP events on the stream the library launches on (torch's current stream)."""
    import torch
    from tensor_train_ing_amd import _abi
    from tensor_train_ing_amd.poly_attn import _desc, _problem, _stream, doc_bounds
    lib = _abi.load()
    dstart, qend = doc_bounds(doc)
    prob = _problem(_abi.POWER, degree, q, k, q, k, v, dstart, qend, rs, None, None)
    o = torch.empty_like(v)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    # the row-scaled dO workspace, passed exactly when the operator passes it
    dos = torch.empty_like(do) if lib.tnpa_dout_scaled_helps(ctypes.byref(prob)) else None
    grads = _abi.Grads(_desc(do), _desc(dq), _desc(dk), _desc(dq), _desc(dk), _desc(dv), None, None,
                       _desc(dos) if dos is not None else _abi.Tensor())
    st = _stream(q.device)
    od = _desc(o)
    def phase(ph, name):
        return lambda: _abi.check(lib.tnpa_backward_phase(ctypes.byref(prob), ctypes.byref(grads), ph, st), name)
    fwd = lambda: _abi.check(lib.tnpa_forward(ctypes.byref(prob), ctypes.byref(od), st), "fwd")  # noqa: E731
    out = {}
    runs = [("fwd", fwd)] + ([("bwd_scale", phase(_abi.PHASE_KV_SCALE, "scale"))] if dos is not None else []) + [
        ("bwd_dv", phase(_abi.PHASE_KV_DV, "dv")), ("bwd_dk", phase(_abi.PHASE_KV_DK, "dk")),
        ("bwd_q", phase(_abi.PHASE_Q, "q"))]
    for name, fn in runs:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        out[name] = time_events(fn, reps)
    return out


def measured_traffic(config, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/hbm_traffic_<config>.txt, counters scaled by a plain-copy calibration), or None if not profiled."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"hbm_traffic_{config}.txt")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 4 and parts[0] == "k_" + kernel:
                    return int(parts[3])
    except OSError:
        pass
    return None


def cpu_baseline(B, H, T, D, degree, seconds):
    """Times the CPU oracle (float32 numpy dense restatement) fwd+bwd over (b, h) slices until `seconds` pass."""
    import numpy as np
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import polynomial_attention, polynomial_attention_backward, row_scale_mask, visible_mask
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("internal_api") == "openblas"]
                      or [1])
    except Exception:  # threadpoolctl missing: report the affinity size numpy's BLAS defaults to
        threads = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    C = row_scale_mask(visible_mask(np.zeros((1, T), dtype=np.int64)), 0.5, np.float32)
    done, t0 = 0, time.perf_counter()
    while done < B * H:
        q, k = (rng.standard_normal((1, 1, T, D), dtype=np.float32) * D ** -0.25 for _ in range(2))
        v, do = (rng.standard_normal((1, 1, T, D), dtype=np.float32) for _ in range(2))
        polynomial_attention("power", q, k, None, None, v, C, degree=degree)
        polynomial_attention_backward("power", q, k, None, None, v, C, do, degree=degree)
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    flops = 14.0 * done * npairs(T) * D
    return {"value": round(flops / el / 1e12, 6), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": f"{done} of {B * H} (b,h) slices of the same workload, T={T} D={D}, fwd+bwd of the CPU oracle "
                      f"(oracle/poly_attention.py, float32 numpy dense) in {el:.1f} s"}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="1b", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device-to-device copy of this many MiB (3 times) and exit: the known-size "
                         "kernel that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    a = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}, WORLD_SIZE {world}); "
              "the path shards over (b, h) with no exchange, so there is no multi-GPU figure to report.",
              file=sys.stderr)
        return 2

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.copy_probe_mib:
        src = torch.ones(a.copy_probe_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4, "dispatches": 3}), flush=True)
        return 0

    from tensor_train_ing_amd import poly_attention_hip
    B, H, T, D, degree, boost, seed = CONFIGS[a.config]
    q, k, v, do, doc, rs = make_inputs(B, H, T, D, boost, seed, dev)
    q.requires_grad_(); k.requires_grad_(); v.requires_grad_()  # noqa: E702

    def step():
        out = poly_attention_hip("power", q, k, None, None, v, doc, rs, degree=degree)
        return torch.autograd.grad(out, (q, k, v), do)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()  # one process, one GPU: the synchronize is the whole barrier
    t0 = time.perf_counter()
    ms_ev = time_events(step, a.steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / a.steps
    ms = max(ms_ev, 0.0)

    fl_fwd = 4.0 * B * H * npairs(T) * D
    fl_step = 3.5 * fl_fwd
    value = fl_step / (ms * 1e-3) / 1e12

    kt = kernel_times(q.detach(), k.detach(), v.detach(), do, doc, rs, degree, a.kernel_reps)
    # matmul units of 2*B*H*Npairs*D each kernel executes: fwd QK^T + PV; dV pass S + dV; dK pass S + dP + dK;
    # dQ pass S + dP + dQ (the row-scaling pass, when used, is a bandwidth kernel with no matrix work)
    units = {"fwd": 2, "bwd_dv": 2, "bwd_dk": 3, "bwd_q": 3}
    dom = max(units, key=lambda n: kt[n])
    ach = units[dom] * 2.0 * B * H * npairs(T) * D / (kt[dom] * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"polynomial attention fwd+bwd, BASELINE config '{a.config}': B{B} H{H} T{T} D{D} "
                               f"degree {degree}, causal, one document, row scale (t+1)^-1/2",
                   "B": B, "H": H, "T": T, "D": D, "degree": degree},
        "pct_of_peak": round(100 * value / PEAK_TFLOPS, 2),
        "fwd_tflops": round(fl_fwd / (kt["fwd"] * 1e-3) / 1e12, 2),
        "fwd_pct_of_peak": round(100 * fl_fwd / (kt["fwd"] * 1e-3) / 1e12 / PEAK_TFLOPS, 2),
        "wall_ms_per_step": round(wall_ms, 4),
        "kernel_ms": {n: round(t, 4) for n, t in kt.items()},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(ach / PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(a.config, dom)},
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(B, H, T, D, degree, a.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
