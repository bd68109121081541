"""Chunked linear + cross-entropy on MI355X: library GEMMs and fused HIP epilogues (libtnpa.so, include/tnce.h).

Drop-in for ref: tnlm/kernels/fused_ce.py (LinearCrossEntropy / linear_cross_entropy_sum): the same signature,
chunking, recomputation and precision policy -- the logits of one chunk of rows exist at a time; matmuls run in the
autocast dtype when autocast is active (as nn.Linear would), log-sum-exp and softmax in the accumulation type
(float32, or float64 for float64 inputs), dW accumulated in that type. Per chunk the matmuls are plain library GEMMs
(hipBLASLt / rocBLAS through torch.matmul) writing into one reused logits buffer, and everything the reference does
to the logits between them is one HIP pass:
    forward : logsumexp per row, the target logit, the masked loss sum       (tnce_forward_chunk)
    backward: exp(logit - lse) - onehot(target), times valid * g, downcast   (tnce_backward_chunk, in place)
There is no CPU path: the epilogues run only as HIP kernels.
"""
from __future__ import annotations

import ctypes

import torch

from . import _abi

IGNORE_INDEX = -100
_DTYPES = {torch.bfloat16: _abi.CE_BF16, torch.float16: _abi.CE_F16, torch.float32: _abi.CE_F32,
           torch.float64: _abi.CE_F64}


def _compute_dtype(x):
    """ref: tnlm/kernels/fused_ce.py:11-14"""
    if torch.is_autocast_enabled(x.device.type):
        return torch.get_autocast_dtype(x.device.type)
    return x.dtype


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _check(x, w, targets, cdtype):
    if not (x.is_cuda and w.is_cuda and targets.is_cuda):
        raise ValueError("linear_cross_entropy_sum (HIP) needs x, w and targets on a ROCm device")
    if x.dim() != 2 or w.dim() != 2 or targets.dim() != 1 or x.shape[1] != w.shape[1] or targets.shape[0] != x.shape[0]:
        raise ValueError(f"expected x (N, d), w (V, d), targets (N,); got {tuple(x.shape)}, {tuple(w.shape)}, "
                         f"{tuple(targets.shape)}")
    if cdtype not in _DTYPES:
        raise ValueError(f"unsupported compute dtype {cdtype}")


class LinearCrossEntropy(torch.autograd.Function):
    """ref: tnlm/kernels/fused_ce.py:18-55"""

    @staticmethod
    def forward(ctx, x, w, targets, chunk, cdtype):
        _check(x, w, targets, cdtype)
        N, V = x.shape[0], w.shape[0]
        chunk = max(1, int(chunk))
        xc, wc = x.to(cdtype), w.to(cdtype)
        acc = torch.promote_types(cdtype, torch.float32)
        lse = torch.empty(N, device=x.device, dtype=acc)
        total = torch.zeros((), device=x.device, dtype=acc)
        tg = targets.to(torch.int64).contiguous()
        rows = min(chunk, N)
        logits = torch.empty(rows, V, device=x.device, dtype=cdtype)
        row_loss = torch.empty(max(rows, 1), device=x.device, dtype=acc)
        lib = _abi.load()
        code = _DTYPES[cdtype]
        with torch.cuda.device(x.device):
            st = _stream(x.device)
            for s in range(0, N, chunk):
                n = min(chunk, N - s)
                lg = logits[:n]
                torch.matmul(xc[s:s + n], wc.t(), out=lg)
                _abi.check(lib.tnce_forward_chunk(_ptr(lg), code, n, V, V, _ptr(tg[s:s + n]), IGNORE_INDEX,
                                                  _ptr(lse[s:s + n]), _ptr(row_loss), _ptr(total), st),
                           "linear cross-entropy forward")
        ctx.save_for_backward(x, w, targets, lse)
        ctx.chunk, ctx.cdtype = chunk, cdtype
        return total

    @staticmethod
    def backward(ctx, g):
        x, w, targets, lse = ctx.saved_tensors
        chunk, cdtype = ctx.chunk, ctx.cdtype
        N, V = x.shape[0], w.shape[0]
        xc, wc = x.to(cdtype), w.to(cdtype)
        dx = torch.empty_like(x)
        acc = lse.dtype
        dw = torch.zeros(w.shape, device=w.device, dtype=acc)
        tg = targets.to(torch.int64).contiguous()
        gd = g.detach().to(device=x.device, dtype=acc).reshape(1).contiguous()
        rows = min(chunk, N)
        logits = torch.empty(rows, V, device=x.device, dtype=cdtype)
        part = torch.empty(w.shape, device=x.device, dtype=cdtype)  # one chunk's dW product, reused
        lib = _abi.load()
        code = _DTYPES[cdtype]
        with torch.cuda.device(x.device):
            st = _stream(x.device)
            for s in range(0, N, chunk):
                n = min(chunk, N - s)
                p = logits[:n]
                torch.matmul(xc[s:s + n], wc.t(), out=p)
                _abi.check(lib.tnce_backward_chunk(_ptr(p), code, n, V, V, _ptr(tg[s:s + n]), IGNORE_INDEX,
                                                   _ptr(lse[s:s + n]), _ptr(gd), st), "linear cross-entropy backward")
                if x.dtype == cdtype:
                    torch.matmul(p, wc, out=dx[s:s + n])
                else:
                    dx[s:s + n] = (p @ wc).to(x.dtype)
                # dw += (p^T x).to(acc): the product in cdtype, then one HIP pass adds it to the fp32/fp64 dW
                torch.matmul(p.t(), xc[s:s + n], out=part)
                _abi.check(lib.tnce_accumulate(_ptr(dw), _ptr(part), code, part.numel(), st),
                           "linear cross-entropy dW")
        return dx, dw.to(w.dtype), None, None, None


def linear_cross_entropy_sum(x, w, targets, chunk=4096):
    """sum over valid targets of CE(x @ w.T, target); x: (N, d), w: (V, d), targets: (N,) with -100 ignored.
    ref: tnlm/kernels/fused_ce.py:58-60"""
    return LinearCrossEntropy.apply(x, w, targets, chunk, _compute_dtype(x))
