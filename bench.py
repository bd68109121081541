"""Benchmark: causal polynomial attention fwd+bwd TFLOP/s on one MI355X (BASELINE.json headline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1b] [--kind power] [--dtype bf16]
                    [--doc-len L] [--head-dim D] [--rope] [--cpu-seconds S] [--no-cpu-baseline]

A step is one forward + backward of the polynomial attention operator (default kind "power" at the config's
degree; degree 2 equals the reference's signed_product with shared pairs) over one batch of seeded synthetic inputs
resident in HBM: q, k ~ N(0,1)/D^(1/4), v, dO ~ N(0,1), one causal document per row, row scale (t+1)^-1/2.
--kind signed_product / lower_degree_mix draw a second q/k pair the same way (the reference model's default kind);
those lines count 11 matmul units per step instead of 7. --dtype f32 runs the fp32 path (the reference's "ieee"
precision) against the fp32 MFMA peak.

Timing: W untimed steps, then K steps with a HIP event recorded on the launch stream (torch's current stream)
between consecutive steps; ms_per_step is the K-step total over K (the whole-job rate), ms_per_step_median the
median of the K intervals. Each kernel of the step is then timed alone (median of --kernel-reps launches, an event
pair around each), and the forward alone likewise (fwd_ms_median).

FLOP convention (exact causal pairs, power and mask not counted): Npairs = T(T+1)/2,
fwd = 4*B*H*Npairs*D, fwd+bwd = 14*B*H*Npairs*D. Peaks: MI355X dense bf16 MFMA 2.5 PFLOP/s, fp32 157.3 TFLOP/s.
Prints one JSON line (rank 0). The CPU baseline times the dense restatement of the reference attention in float32
torch (oracle/torch_dense.py; backward by autograd) on the host's cores, on a bounded sample of (b, h) slices of
the same inputs.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import subprocess
import sys
import time

PEAKS = {"bf16": 2500.0, "f32": 157.3}  # MI355X dense MFMA, TFLOP/s
METRIC = "poly-attn fwd+bwd TFLOP/s at B8 H16 T2048 D128 bf16; % of MI355X MFMA peak"

KIND_CODES = {"signed_product": 0, "offset_square": 1, "lower_degree_mix": 2, "power": 3}
TWO_PAIR_KINDS = ("signed_product", "lower_degree_mix")
CONFIGS = {  # name: (B, H, T, D, degree, boost_rows, seed) -- BASELINE.json configs[1..4]
    "100m": (16, 12, 1024, 64, 2, 0.0, 1),
    "1b": (8, 16, 2048, 128, 2, 0.0, 2),
    "p4": (4, 16, 2048, 128, 4, 0.01, 3),
    "7b": (2, 32, 4096, 128, 2, 0.0, 4),
}
# matrix units (of 2*B*H*Npairs*D FLOP) each launch executes: fwd QK^T + PV; dv pass S + dV; dk pass S + dP + dK;
# combined key side S + dP + dV + dK; dq pass S + dP + dQ; dQ from the stored dS tiles (qds) dQ only; with two
# pairs one more S, dK and dQ each (and one more S in the dv pass). The dO row-scaling pass, the dpar reduction and
# the rotary pass are bandwidth kernels with no matrix work.
UNITS_ONE = {"fwd": 2, "dv": 2, "dk": 3, "kv": 4, "q": 3, "qds": 1, "scale": 0, "dpar": 0, "rope": 0}
UNITS_TWO = {"fwd": 3, "dv": 3, "dk": 5, "kv": 6, "q": 5, "qds": 2, "scale": 0, "dpar": 0, "rope": 0}


def npairs(T, doc_len=0):
    """Visible (query, key) pairs of one row: causal, within contiguous documents of doc_len tokens (0: one)."""
    if not doc_len or doc_len >= T:
        return T * (T + 1) // 2
    full, rest = divmod(T, doc_len)
    return full * doc_len * (doc_len + 1) // 2 + rest * (rest + 1) // 2


def make_inputs(B, H, T, D, boost, seed, device, two_pairs=False, doc_len=0, dtype=None):
    """Seeded CPU draws cast to the dtype (bf16 by default) on the CPU: q, k (and q2, k2 for the two-pair kinds,
    drawn after dO so the one-pair inputs do not change), v, dO; one document per row; row scale (t+1)^-1/2."""
    import torch
    dtype = dtype or torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    mk = lambda s: (torch.randn(B, H, T, D, generator=g) * s)  # noqa: E731
    q, k = mk(D ** -0.25), mk(D ** -0.25)
    if boost:
        for x in (q, k):
            rows = torch.rand(B, T, generator=g) < boost
            x.mul_(torch.where(rows, 4.0, 1.0)[:, None, :, None])
    v, do = mk(1.0), mk(1.0)
    q2, k2 = (mk(D ** -0.25), mk(D ** -0.25)) if two_pairs else (None, None)
    cast = lambda x: None if x is None else x.to(dtype).to(device)  # noqa: E731
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


def rope_tables_for(doc, D, base=10000.0):
    """Rotary tables (B, 1, T, D/2) fp32 from positions within documents, built as the reference model builds them
    once per batch (ref: tnlm/attention.py:41-45 on doc positions, ref: tnlm/model.py:205-210): caller-side setup,
    not part of the timed step."""
    import torch
    B, T = doc.shape
    ar = torch.arange(T, device=doc.device).expand(B, T)
    start = torch.ones_like(doc, dtype=torch.bool)
    start[:, 1:] = doc[:, 1:] != doc[:, :-1]
    pos = ar - torch.where(start, ar, torch.zeros_like(ar)).cummax(-1).values
    inv = 1.0 / (base ** (torch.arange(0, D, 2, device=doc.device, dtype=torch.float32) / D))
    ang = pos.float()[..., None] * inv
    return ang.cos()[:, None], ang.sin()[:, None]


def torch_apply_rope(x, cos, sin):
    """The reference's rotation as separate tensor operations (ref: tnlm/attention.py:48-51): the unfused step that
    --rope compares against."""
    import torch
    x1, x2 = x.to(torch.promote_types(x.dtype, torch.float32)).chunk(2, dim=-1)
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).to(x.dtype)


def event_intervals(fn, reps):
    """Runs fn reps times back to back with a HIP event between consecutive runs on the current stream; returns
    the reps intervals (ms)."""
    import torch
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    evs[0].record()
    for i in range(reps):
        fn()
        evs[i + 1].record()
    evs[-1].synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(reps)]


def median_back_to_back(fn, reps):
    """Median interval (ms) of fn run reps times back to back, a HIP event between consecutive runs (after 3 untimed
    runs): each launch's time in the steady state of a busy GPU, as inside the step."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    return statistics.median(event_intervals(fn, reps))


def median_each(fn, reps):
    """Median duration (ms) of fn over reps runs, each bracketed by its own event pair (after 3 untimed runs)."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    times = []
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(reps):
        s.record()
        fn()
        e.record()
        e.synchronize()
        times.append(s.elapsed_time(e))
    return statistics.median(times)


def kernel_times(kind, q, k, q2, k2, v, do, doc, rs, degree, reps):
    """Median duration (ms) of each launch of the step, repeated back to back with HIP events on the stream the
    library launches on (torch's current stream): the forward, then each launch of the backward plan in order (the
    library's internal launch-level entry point; a launch run alone reads what the earlier ones wrote)."""
    import torch
    from tensor_train_ing_amd import _abi
    from tensor_train_ing_amd.poly_attn import _desc, _problem, _stream, doc_bounds
    lib = _abi.load()
    K = KIND_CODES[kind]
    two = kind in TWO_PAIR_KINDS
    H = q.shape[1]
    coef = torch.tensor([[0.1, 0.2, -0.3, 1.0]], device=q.device).repeat(H, 1) if kind == "lower_degree_mix" else None
    b = torch.full((H,), 0.5, device=q.device) if kind == "offset_square" else None
    dstart, qend = doc_bounds(doc)
    prob = _problem(K, degree if kind == "power" else None, q, k, q2 if two else q, k2 if two else k, v, dstart, qend,
                    rs, coef, b)
    o = torch.empty_like(v)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dq2, dk2 = (torch.empty_like(q), torch.empty_like(k)) if two else (dq, dk)
    dpar = torch.empty(H, 4, device=q.device)
    nbytes = lib.tnpa_backward_workspace_bytes(ctypes.byref(prob))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    grads = _abi.Grads(_desc(do), _desc(dq), _desc(dk), _desc(dq2), _desc(dk2), _desc(dv), dpar.data_ptr(),
                       ws.data_ptr(), nbytes)
    st = _stream(q.device)
    od = _desc(o)
    out = {"fwd": median_back_to_back(
        lambda: _abi.check(lib.tnpa_forward(ctypes.byref(prob), ctypes.byref(od), st), "fwd"), reps)}
    _abi.check(lib.tnpa_backward(ctypes.byref(prob), ctypes.byref(grads), st), "bwd")  # fills the workspace
    for i in range(lib.tnpa_x_launches(ctypes.byref(prob), 0)):
        name = lib.tnpa_x_launch_name(ctypes.byref(prob), 0, i).decode()
        out[name] = median_back_to_back(
            lambda: _abi.check(lib.tnpa_x_backward(ctypes.byref(prob), ctypes.byref(grads), 0, i, st), name), reps)
    return out


# kernel symbol names (as the rocprofv3 summaries list them) of each backward-plan launch
LAUNCH_KERNELS = {"fwd": ("k_fwd",), "kv": ("k_bwd_kv_pair", "k_bwd_kv"), "dv": ("k_bwd_kv",), "dk": ("k_bwd_kv",),
                  "q": ("k_bwd_q",), "qds": ("k_bwd_q_ds",)}


def measured_traffic(config, launch):
    """HBM bytes per dispatch of the kernel behind backward-plan launch `launch` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic_<config>.txt, counters scaled by a plain-copy
    calibration), or None if not profiled."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"hbm_traffic_{config}.txt")
    names = LAUNCH_KERNELS.get(launch, (launch,))
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 4 and parts[0] in names:
                    return int(parts[3])
    except OSError:
        pass
    return None


def cpu_model():
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(q, k, v, do, rs, degree, seconds):
    """Times the dense restatement of the reference attention (oracle/torch_dense.py) in float32 torch on the host's
    cores over (b, h) slices of the GPU run's own inputs (copied to the host and upcast), until `seconds` pass:
    the forward alone, then forward + backward (autograd). Returns the cpu_baseline object."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import causal_row_scale, dense_attention
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    B, H, T, D = q.shape
    slices = [(b, h) for b in range(B) for h in range(H)]
    host = [x.detach().float().cpu() for x in (q, k, v, do)]
    rsh = rs.detach().float().cpu()
    fwd_t, step_t = [], []
    t0 = time.perf_counter()
    for b, h in slices:
        qs, ks, vs, ds = (x[b, h].contiguous() for x in host)
        C = causal_row_scale(rsh[b])
        t1 = time.perf_counter()
        with torch.no_grad():
            dense_attention("power", qs, ks, None, None, vs, C, degree=degree)
        t2 = time.perf_counter()
        ins = [x.clone().requires_grad_() for x in (qs, ks, vs)]
        y = dense_attention("power", ins[0], ins[1], None, None, ins[2], C, degree=degree)
        torch.autograd.grad(y, ins, ds)
        t3 = time.perf_counter()
        fwd_t.append(t2 - t1)
        step_t.append(t3 - t2)
        if t3 - t0 >= seconds:
            break
    n = len(step_t)
    unit = 2.0 * npairs(T) * D  # one matrix unit of one (b, h) slice
    fwd_med, step_med = statistics.median(fwd_t), statistics.median(step_t)
    return {"value": round(7 * unit / step_med / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "fwd_tflops": round(2 * unit / fwd_med / 1e12, 6),
            "ms_per_slice_fwd": round(fwd_med * 1e3, 3), "ms_per_slice_fwd_bwd": round(step_med * 1e3, 3),
            "cpu": cpu_model(), "threads": torch.get_num_threads(),
            "sample": f"{n} of {B * H} (b,h) slices of the GPU run's inputs, T={T} D={D} degree {degree}: dense "
                      f"float32 torch restatement of the reference attention (oracle/torch_dense.py), fwd alone and "
                      f"fwd+bwd by autograd, median per slice, {threads} threads"}


CE_CONFIG = {"N": 8192, "d": 2048, "V": 50304, "chunk": 4096, "seed": 7}  # pilot_1b: 4 x 2048 tokens per microbatch


def bench_linear_ce(a):
    """The fused linear + cross-entropy (tensor_train_ing_amd.fused_ce) at the pilot-1B unembedding shape: N tokens,
    d_model, padded vocab, the reference's loss_chunk_tokens (ref: configs/pilot_1b.yaml:21,27,33). A step is the
    forward and backward (bf16 matmuls, fp32 log-sum-exp). FLOPs: 8 N V d (forward GEMM; backward recompute, dX and
    dW GEMMs). The roofline object covers this build's dominant HIP kernel, the backward epilogue, which is
    HBM-bound: it reads and writes each chunk's bf16 logits once (4 n V bytes per launch)."""
    import torch
    from tensor_train_ing_amd import _abi, linear_cross_entropy_sum
    from tensor_train_ing_amd.fused_ce import IGNORE_INDEX, _ptr, _stream
    dev = torch.device("cuda:0")
    c = CE_CONFIG
    N, d, V, chunk = c["N"], c["d"], c["V"], c["chunk"]
    g = torch.Generator().manual_seed(c["seed"])
    x = (torch.randn(N, d, generator=g) * 0.02).to(dev, torch.bfloat16).requires_grad_()
    w = (torch.randn(V, d, generator=g) * 0.02).to(dev, torch.bfloat16).requires_grad_()
    t = torch.randint(0, 50257, (N,), generator=g).to(dev)

    def step():
        total = linear_cross_entropy_sum(x, w, t, chunk=chunk)
        return torch.autograd.grad(total, (x, w))

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    iv = event_intervals(step, a.steps)
    ms = sum(iv) / len(iv)
    flops = 8.0 * N * V * d
    value = flops / (ms * 1e-3) / 1e12
    # the epilogues alone, on one chunk of logits
    lib = _abi.load()
    n = chunk
    lg = (x[:n].detach() @ w.detach().t())
    lse = torch.empty(n, device=dev)
    rl = torch.empty(n, device=dev)
    tot = torch.zeros((), device=dev)
    one = torch.ones(1, device=dev)
    st = _stream(dev)
    fwd_k = median_each(lambda: _abi.check(lib.tnce_forward_chunk(_ptr(lg), _abi.CE_BF16, n, V, V, _ptr(t[:n]),
                                                                  IGNORE_INDEX, _ptr(lse), _ptr(rl), _ptr(tot), st),
                                           "ce fwd"), a.kernel_reps)
    work = lg.clone()
    bwd_k = median_each(lambda: (work.copy_(lg), _abi.check(lib.tnce_backward_chunk(
        _ptr(work), _abi.CE_BF16, n, V, V, _ptr(t[:n]), IGNORE_INDEX, _ptr(lse), _ptr(one), st), "ce bwd")),
        a.kernel_reps)
    copy_k = median_each(lambda: work.copy_(lg), a.kernel_reps)
    bwd_only = max(bwd_k - copy_k, 1e-6)
    bwd_bytes = 4.0 * n * V  # bf16 read + write
    fwd_bytes = 2.0 * n * V
    gemm_ms = median_each(lambda: torch.matmul(x[:n].detach(), w.detach().t(), out=lg), a.kernel_reps)
    line = {
        "metric": "fused linear + cross-entropy fwd+bwd TFLOP/s at the pilot-1B unembedding (N8192 d2048 V50304, "
                  "chunk 4096, bf16)",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "chunked linear + cross-entropy (ref: tnlm/kernels/fused_ce.py), pilot_1b shape",
                   **c},
        "pct_of_peak": round(100 * value / PEAKS["bf16"], 2),
        "kernel_ms": {"ce_forward_chunk": round(fwd_k, 4), "ce_backward_chunk": round(bwd_only, 4),
                      "gemm_chunk_logits": round(gemm_ms, 4)},
        "roofline": {"bound": "hbm", "kernel": "ce_backward_chunk", "achieved": round(bwd_bytes / (bwd_only * 1e-3) / 1e9, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(bwd_bytes / (bwd_only * 1e-3) / 1e9 / 8000.0, 4),
                     "traffic": None},
        "ce_forward_chunk_gbs": round(fwd_bytes / (fwd_k * 1e-3) / 1e9, 1),
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = ce_cpu_baseline(x, w, t, chunk, a.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


def ce_cpu_baseline(x, w, t, chunk, seconds):
    """The CPU oracle of the fused linear + cross-entropy (oracle/fused_ce.py: numpy, float64, the reference's chunked
    algorithm) on a bounded sample of the same rows (the full weight matrix), forward and backward; the rate is
    scaled to the metric's FLOP convention (8 rows V d per sample)."""
    import numpy as np
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import linear_cross_entropy
    rows = 64
    xs = x[:rows].detach().float().cpu().numpy()
    ws = w.detach().float().cpu().numpy()
    ts = t[:rows].cpu().numpy()
    done, t0 = 0, time.perf_counter()
    while True:
        linear_cross_entropy(xs, ws, ts, chunk=chunk)
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = (time.perf_counter() - t0) / done
    V, d = ws.shape
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = len(os.sched_getaffinity(0))
    return {"value": round(8.0 * rows * V * d / el / 1e12, 6), "unit": "TFLOP/s", "cores": int(threads),
            "kind": "port", "cpu": cpu_model(),
            "sample": f"{rows} of {x.shape[0]} rows (full {V} x {d} weight) through the CPU oracle "
                      f"(oracle/fused_ce.py, numpy float64, forward + backward), {el * 1e3:.0f} ms per sample, "
                      f"{done} repetitions"}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # a fresh process reaches its steady step time only after ~70 steps (0.74 ms per step at steps 10-19, 0.67 from
    # step 80 on, at the headline), so the default warmup covers that
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="1b", choices=sorted(CONFIGS))
    ap.add_argument("--kind", default="power", choices=sorted(KIND_CODES),
                    help="polynomial family (default: power, the degree-p kind BASELINE.json's configs name; "
                         "signed_product with distinct q2/k2 is the reference model's default)")
    ap.add_argument("--dtype", default="bf16", choices=sorted(PEAKS))
    ap.add_argument("--doc-len", type=int, default=0,
                    help="contiguous documents of this many tokens per row (0: one document; FLOPs count only the "
                         "visible pairs, so the rate shows how well invisible tiles are skipped)")
    ap.add_argument("--rope", action="store_true",
                    help="q/k enter unrotated with rotary tables (positions within documents): the step includes the "
                         "one-pass rotation and the rotation's gradient inside the backward; also times the "
                         "reference's way (torch apply_rope, then the operator, autograd through both)")
    ap.add_argument("--head-dim", type=int, default=0,
                    help="run the config's B, H, T at this q/k and v head dim instead (16..256; a side line, not the "
                         "headline)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--workload", default="attention", choices=["attention", "linear_ce"],
                    help="attention: the headline polynomial attention step (default); linear_ce: the fused linear + "
                         "cross-entropy at the pilot-1B unembedding shape")
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

    if a.workload == "linear_ce":
        return bench_linear_ce(a)
    from tensor_train_ing_amd import poly_attention_hip
    B, H, T, D, degree, boost, seed = CONFIGS[a.config]
    D = a.head_dim or D
    kind = a.kind
    two = kind in TWO_PAIR_KINDS
    tdt = torch.bfloat16 if a.dtype == "bf16" else torch.float32
    ins = make_inputs(B, H, T, D, boost, seed, dev, two_pairs=two, doc_len=a.doc_len, dtype=tdt)
    q, k, v, do, doc, rs = ins[:6]
    q2, k2 = (ins[6], ins[7]) if two else (None, None)
    coef = torch.tensor([[0.1, 0.2, -0.3, 1.0]], device=dev).repeat(H, 1) if kind == "lower_degree_mix" else None
    bias = torch.full((H,), 0.5, device=dev) if kind == "offset_square" else None
    leaves = [q, k] + ([q2, k2] if two else []) + [v]
    for x in leaves:
        x.requires_grad_()
    deg = degree if kind == "power" else None

    rope = rope_tables_for(doc, D) if a.rope else None

    def step():
        out = poly_attention_hip(kind, q, k, q2, k2, v, doc, rs, coef=coef, b=bias, degree=deg, rope=rope)
        return torch.autograd.grad(out, leaves, do)

    def step_torch_rope():
        rot = lambda x: None if x is None else torch_apply_rope(x, *rope)  # noqa: E731
        out = poly_attention_hip(kind, rot(q), rot(k), rot(q2), rot(k2), v, doc, rs, coef=coef, b=bias, degree=deg)
        return torch.autograd.grad(out, leaves, do)

    def fwd_only():
        with torch.no_grad():
            return poly_attention_hip(kind, q, k, q2, k2, v, doc, rs, coef=coef, b=bias, degree=deg, rope=rope)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()  # one process, one GPU: the synchronize is the whole barrier
    t0 = time.perf_counter()
    iv = event_intervals(step, a.steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / a.steps
    ms = sum(iv) / len(iv)
    fwd_iv = event_intervals(fwd_only, a.steps)
    rope_info = None
    if a.rope:
        for _ in range(a.warmup):
            step_torch_rope()
        torch.cuda.synchronize()
        trope = event_intervals(step_torch_rope, a.steps)
        from tensor_train_ing_amd.poly_attn import rope_rotate, rope_tables_of
        cs, sn = rope_tables_of(rope, q)
        qd = q.detach()
        rope_info = {"ms_per_step_fused": round(statistics.median(iv), 4),
                     "ms_per_step_torch_apply_rope": round(statistics.median(trope), 4),
                     "rope_kernel_ms_per_tensor": round(median_each(lambda: rope_rotate(qd, cs, sn), a.kernel_reps),
                                                        4)}

    kt = kernel_times(kind, q.detach(), k.detach(), q2.detach() if two else None, k2.detach() if two else None,
                      v.detach(), do, doc, rs, degree, a.kernel_reps)

    # counted FLOPs (exact causal pairs): one q/k pair fwd 2 matmul units of 2*B*H*Npairs*D, fwd+bwd 7; two pairs
    # fwd 3 (S1, S2, PV), fwd+bwd 11
    unit = 2.0 * B * H * npairs(T, a.doc_len) * D
    fl_fwd = (3 if two else 2) * unit
    fl_step = (11 if two else 7) * unit
    value = fl_step / (ms * 1e-3) / 1e12
    peak = PEAKS[a.dtype]

    units = UNITS_TWO if two else UNITS_ONE
    if two and D > 128:  # the dk and q launches run once per pair, each with S1, S2 and dP
        units = {**units, "dk": 8, "q": 8}
    dom = max(kt, key=lambda n: kt[n])
    ach = units[dom] * unit / (kt[dom] * 1e-3) / 1e12
    docs = f", documents of {a.doc_len} tokens" if a.doc_len else ", one document"
    fwd_med = statistics.median(fwd_iv)
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": a.dtype, "data": "synthetic",
        "config": {"workload": f"polynomial attention fwd+bwd, BASELINE config '{a.config}'"
                               + (f" at head dim {D}" if a.head_dim else "") + f": B{B} H{H} T{T} D{D} "
                               + (f"degree {degree}" if kind == "power" else f"kind {kind}")
                               + f", causal{docs}, row scale (position in document + 1)^-1/2"
                               + (", rotary embedding of q/k inside the operator" if a.rope else ""),
                   "B": B, "H": H, "T": T, "D": D, "kind": kind, "degree": deg, "doc_len": a.doc_len or T,
                   "rope": a.rope},
        "pct_of_peak": round(100 * value / peak, 2),
        "ms_per_step_median": round(statistics.median(iv), 4),
        "fwd_ms_median": round(fwd_med, 4),
        "fwd_tflops": round(fl_fwd / (fwd_med * 1e-3) / 1e12, 2),
        "fwd_pct_of_peak": round(100 * fl_fwd / (fwd_med * 1e-3) / 1e12 / peak, 2),
        "wall_ms_per_step": round(wall_ms, 4),
        "kernel_ms": {n: round(t, 4) for n, t in kt.items()},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                     "traffic": (measured_traffic(a.config, dom)
                                 if kind == "power" and not a.doc_len and a.dtype == "bf16" and not a.head_dim
                                 else None)},
    }
    if rope_info is not None:
        line["rope"] = rope_info
    if not a.no_cpu_baseline and kind == "power" and not a.doc_len and not a.rope and not a.head_dim:
        line["cpu_baseline"] = cpu_baseline(q, k, v, do, rs, degree, a.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
