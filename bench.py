"""Benchmark: causal polynomial attention fwd+bwd TFLOP/s on one MI355X (BASELINE.json headline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1b] [--kind power] [--cpu-seconds S]
                    [--no-cpu-baseline]

A step is one forward + backward of the polynomial attention operator (default kind "power" at the config's
degree; degree 2 equals the reference's signed_product with shared pairs) over one batch of seeded synthetic bf16
inputs resident in HBM: q, k ~ N(0,1)/D^(1/4), v, dO ~ N(0,1), one causal document per row, row scale
(t+1)^-1/2. --kind signed_product / lower_degree_mix draw a second q/k pair the same way (the reference model's
default kind); those lines count 11 matmul units per step instead of 7 and carry no CPU baseline.

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

KIND_CODES = {"signed_product": 0, "offset_square": 1, "lower_degree_mix": 2, "power": 3}
TWO_PAIR_KINDS = ("signed_product", "lower_degree_mix")
CONFIGS = {  # name: (B, H, T, D, degree, boost_rows, seed) -- BASELINE.json configs[1..4]
    "100m": (16, 12, 1024, 64, 2, 0.0, 1),
    "1b": (8, 16, 2048, 128, 2, 0.0, 2),
    "p4": (4, 16, 2048, 128, 4, 0.01, 3),
    "7b": (2, 32, 4096, 128, 2, 0.0, 4),
}


def npairs(T, doc_len=0):
    """Visible (query, key) pairs of one row: causal, within contiguous documents of doc_len tokens (0: one)."""
    if not doc_len or doc_len >= T:
        return T * (T + 1) // 2
    full, rest = divmod(T, doc_len)
    return full * doc_len * (doc_len + 1) // 2 + rest * (rest + 1) // 2


def make_inputs(B, H, T, D, boost, seed, device, two_pairs=False, doc_len=0):
    """Seeded CPU draws cast to bf16 on the CPU: q, k (and q2, k2 for the two-pair kinds, drawn after dO so the
    one-pair inputs do not change), v, dO; one document per row; row scale (t+1)^-1/2."""
    import torch
    g = torch.Generator().manual_seed(seed)
    mk = lambda s: (torch.randn(B, H, T, D, generator=g) * s)  # noqa: E731
    q, k = mk(D ** -0.25), mk(D ** -0.25)
    if boost:
        for x in (q, k):
            rows = torch.rand(B, T, generator=g) < boost
            x.mul_(torch.where(rows, 4.0, 1.0)[:, None, :, None])
    v, do = mk(1.0), mk(1.0)
    q2, k2 = (mk(D ** -0.25), mk(D ** -0.25)) if two_pairs else (None, None)
    cast = lambda x: None if x is None else x.to(torch.bfloat16).to(device)  # noqa: E731
    q, k, v, do, q2, k2 = (cast(x) for x in (q, k, v, do, q2, k2))
    if doc_len:  # contiguous documents of doc_len tokens; row scale (position in document + 1)^-1/2
        t = torch.arange(T, device=device)
        doc = (t // doc_len).expand(B, T).contiguous()
        rs = ((t % doc_len).float() + 1).pow(-0.5).expand(B, T).contiguous()
    else:
        doc = torch.zeros(B, T, dtype=torch.long, device=device)
        rs = (torch.arange(T, device=device, dtype=torch.float32) + 1).pow(-0.5).expand(B, T).contiguous()
    if two_pairs:
        return q, k, v, do, doc, rs, q2, k2
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


def kernel_times(kind, q, k, q2, k2, v, do, doc, rs, degree, reps):
    """Average duration (ms) of each launch of the fwd, dV, dK and dQ kernels (one dK/dV kernel for the two-pair
    kinds and for head dims up to 64; plus the dO pre-scaling pass when the operator uses it), timed with HIP events
    on the stream the library launches on (torch's current stream)."""
    import torch
    from tensor_train_ing_amd import _abi
    from tensor_train_ing_amd.poly_attn import _desc, _problem, _stream, doc_bounds
    lib = _abi.load()
    K = KIND_CODES[kind]
    two = kind in TWO_PAIR_KINDS
    H, D = q.shape[1], q.shape[-1]
    coef = torch.tensor([[0.1, 0.2, -0.3, 1.0]], device=q.device).repeat(H, 1) if kind == "lower_degree_mix" else None
    b = torch.full((H,), 0.5, device=q.device) if kind == "offset_square" else None
    dstart, qend = doc_bounds(doc)
    prob = _problem(K, degree if kind == "power" else None, q, k, q2 if two else q, k2 if two else k, v, dstart, qend,
                    rs, coef, b)
    o = torch.empty_like(v)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dq2, dk2 = (torch.empty_like(q), torch.empty_like(k)) if two else (dq, dk)
    par = kind in ("offset_square", "lower_degree_mix")
    ws = torch.empty(max(1, lib.tnpa_dpar_workspace_floats(ctypes.byref(prob))), device=q.device) if par else None
    dpar = torch.empty(H, 4, device=q.device) if par else None
    # the row-scaled dO workspace, passed exactly when the operator passes it
    dos = torch.empty_like(do) if lib.tnpa_dout_scaled_helps(ctypes.byref(prob)) else None
    grads = _abi.Grads(_desc(do), _desc(dq), _desc(dk), _desc(dq2), _desc(dk2), _desc(dv),
                       ws.data_ptr() if par else None, dpar.data_ptr() if par else None,
                       _desc(dos) if dos is not None else _abi.Tensor())
    st = _stream(q.device)
    od = _desc(o)
    def phase(ph, name):
        return lambda: _abi.check(lib.tnpa_backward_phase(ctypes.byref(prob), ctypes.byref(grads), ph, st), name)
    fwd = lambda: _abi.check(lib.tnpa_forward(ctypes.byref(prob), ctypes.byref(od), st), "fwd")  # noqa: E731
    out = {}
    scale = [("bwd_scale", phase(_abi.PHASE_KV_SCALE, "scale"))] if dos is not None else []
    # the key side is one dK/dV kernel for the two-pair kinds and for head dims up to 64 (it writes the scaled dO
    # itself when given the workspace), separate dV and dK passes otherwise
    if two or D <= 64:
        kv = [("bwd_kv", phase(_abi.PHASE_KV, "kv"))]
        scale = []
    else:
        kv = [("bwd_dv", phase(_abi.PHASE_KV_DV, "dv")), ("bwd_dk", phase(_abi.PHASE_KV_DK, "dk"))]
    runs = [("fwd", fwd)] + scale + kv + [("bwd_q", phase(_abi.PHASE_Q, "q"))]
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
    ap.add_argument("--kind", default="power", choices=sorted(KIND_CODES),
                    help="polynomial family (default: power, the degree-p kind BASELINE.json's configs name; "
                         "signed_product with distinct q2/k2 is the reference model's default)")
    ap.add_argument("--doc-len", type=int, default=0,
                    help="contiguous documents of this many tokens per row (0: one document; FLOPs count only the "
                         "visible pairs, so the rate shows how well invisible tiles are skipped)")
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
    kind = a.kind
    two = kind in TWO_PAIR_KINDS
    if two:
        q, k, v, do, doc, rs, q2, k2 = make_inputs(B, H, T, D, boost, seed, dev, two_pairs=True, doc_len=a.doc_len)
    else:
        q, k, v, do, doc, rs = make_inputs(B, H, T, D, boost, seed, dev, doc_len=a.doc_len)
        q2 = k2 = None
    coef = torch.tensor([[0.1, 0.2, -0.3, 1.0]], device=dev).repeat(H, 1) if kind == "lower_degree_mix" else None
    bias = torch.full((H,), 0.5, device=dev) if kind == "offset_square" else None
    leaves = [q, k] + ([q2, k2] if two else []) + [v]
    for x in leaves:
        x.requires_grad_()

    def step():
        out = poly_attention_hip(kind, q, k, q2, k2, v, doc, rs, coef=coef, b=bias,
                                 degree=degree if kind == "power" else None)
        return torch.autograd.grad(out, leaves, do)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()  # one process, one GPU: the synchronize is the whole barrier
    t0 = time.perf_counter()
    ms_ev = time_events(step, a.steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / a.steps
    ms = max(ms_ev, 0.0)

    # counted FLOPs (exact causal pairs): one q/k pair fwd 2 matmul units of 2*B*H*Npairs*D, fwd+bwd 7; two pairs
    # fwd 3 (S1, S2, PV), fwd+bwd 11
    unit = 2.0 * B * H * npairs(T, a.doc_len) * D
    fl_fwd = (3 if two else 2) * unit
    fl_step = (11 if two else 7) * unit
    value = fl_step / (ms * 1e-3) / 1e12

    kt = kernel_times(kind, q.detach(), k.detach(), q2.detach() if two else None, k2.detach() if two else None,
                      v.detach(), do, doc, rs, degree, a.kernel_reps)
    docs = f", documents of {a.doc_len} tokens" if a.doc_len else ", one document"
    # matmul units each kernel executes: fwd QK^T + PV; dV pass S + dV; dK pass S + dP + dK; dQ pass S + dP + dQ;
    # two pairs: fwd S1 + S2 + PV, dK/dV kernel S1 + S2 + dP + dV + dK1 + dK2, dQ S1 + S2 + dP + dQ1 + dQ2 (the
    # row-scaling pass, when used, is a bandwidth kernel with no matrix work)
    # (one pair, head dims up to 64: one dK/dV kernel, S + dP + dV + dK)
    units = ({"fwd": 3, "bwd_kv": 6, "bwd_q": 5} if two else {"fwd": 2, "bwd_kv": 4, "bwd_q": 3} if D <= 64
             else {"fwd": 2, "bwd_dv": 2, "bwd_dk": 3, "bwd_q": 3})
    dom = max(units, key=lambda n: kt[n])
    ach = units[dom] * unit / (kt[dom] * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"polynomial attention fwd+bwd, BASELINE config '{a.config}': B{B} H{H} T{T} D{D} "
                               + (f"degree {degree}" if kind == "power" else f"kind {kind}")
                               + f", causal{docs}, row scale (position in document + 1)^-1/2",
                   "B": B, "H": H, "T": T, "D": D, "kind": kind, "degree": degree if kind == "power" else None,
                   "doc_len": a.doc_len or T},
        "pct_of_peak": round(100 * value / PEAK_TFLOPS, 2),
        "fwd_tflops": round(fl_fwd / (kt["fwd"] * 1e-3) / 1e12, 2),
        "fwd_pct_of_peak": round(100 * fl_fwd / (kt["fwd"] * 1e-3) / 1e12 / PEAK_TFLOPS, 2),
        "wall_ms_per_step": round(wall_ms, 4),
        "kernel_ms": {n: round(t, 4) for n, t in kt.items()},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(ach / PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(a.config, dom) if kind == "power" and not a.doc_len else None},
    }
    if not a.no_cpu_baseline and kind == "power" and not a.doc_len:
        line["cpu_baseline"] = cpu_baseline(B, H, T, D, degree, a.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
