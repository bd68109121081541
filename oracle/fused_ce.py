"""CPU oracle for the chunked linear + cross-entropy (test infrastructure only; nothing in the product imports it).

Restates ref: tnlm/kernels/fused_ce.py:18-55 in numpy, chunk by chunk, with the reference's rounding points made
explicit: the logits of a chunk are the matmul's output in the compute dtype (`round_to`), log-sum-exp and softmax
are taken in the accumulation type (float64 here), the softmax gradient p is rounded to the compute dtype before the
two matmuls, dx is rounded to x's dtype and dW accumulates each chunk's product (rounded to the compute dtype) in the
accumulation type. With round_to=None every step is float64: the dense cross-entropy of x @ w.T.
"""
from __future__ import annotations

import numpy as np

IGNORE_INDEX = -100


def _logsumexp(a: np.ndarray) -> np.ndarray:
    m = a.max(axis=1, keepdims=True)
    return (m + np.log(np.exp(a - m).sum(axis=1, keepdims=True)))[:, 0]


def linear_cross_entropy(x, w, targets, chunk=4096, g=1.0, round_to=None):
    """Returns (total, dx, dw, lse) for sum_i [t_i != -100] CE(x_i w^T, t_i) and its gradients times g.
    round_to: None (float64 throughout) or a function rounding an array to the compute dtype (e.g. round_to_bf16)."""
    rnd = round_to or (lambda a: a)
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    t = np.asarray(targets, dtype=np.int64)
    N = x.shape[0]
    xc, wc = rnd(x), rnd(w)
    valid = t != IGNORE_INDEX
    safe = np.where(valid, t, 0)
    lse = np.empty(N)
    total = 0.0
    for s in range(0, N, chunk):
        sl = slice(s, s + chunk)
        lg = rnd(xc[sl] @ wc.T)
        lse[sl] = _logsumexp(lg)
        tl = lg[np.arange(lg.shape[0]), safe[sl]]
        total += float(((lse[sl] - tl) * valid[sl]).sum())
    dx = np.empty_like(x)
    dw = np.zeros_like(w)
    for s in range(0, N, chunk):
        sl = slice(s, s + chunk)
        p = np.exp(rnd(xc[sl] @ wc.T) - lse[sl, None])
        p[np.arange(p.shape[0]), safe[sl]] -= 1.0
        p = rnd(p * (valid[sl, None] * g))
        dx[sl] = rnd(p @ wc)
        dw += rnd(p.T @ xc[sl])
    return total, dx, dw, lse
