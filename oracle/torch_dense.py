"""Dense causal polynomial attention in torch, for the CPU baseline (test infrastructure only).

The same dense form as oracle/poly_attention.py -- ref: tnlm/attention.py:54-77: S = q k^T / sqrt(dk), A = A(S1, S2)
(ref: tnlm/kernels/poly_attn.py:26-34, plus the degree-p power), P = C * A with C = visible * row scale applied
after the polynomial, y = P v -- restated with torch tensor ops so that `bench.py` can time it in float32 on the
host's cores with autograd providing the backward (a float32 torch CPU baseline). It is pinned against the numpy
oracle in tests/test_oracle.py. Nothing in the product package imports it.
"""
from __future__ import annotations

import math

import torch


def dense_attention(kind, q1, k1, q2, k2, v, C, coef=None, b=None, degree=None):
    """One (b, h) slice: q*/k* (T, dk), v (T, dv), C (T, T) = visible * row_scale[query]. Returns y (T, dv) in the
    inputs' dtype; differentiable in q*, k*, v (and coef / b)."""
    sm = 1.0 / math.sqrt(q1.shape[-1])
    S1 = (q1 @ k1.transpose(0, 1)) * sm
    if kind == "power":
        A = S1 ** degree
    elif kind == "offset_square":
        A = (S1 + b) ** 2
    else:
        S2 = (q2 @ k2.transpose(0, 1)) * sm
        A = S1 * S2 if kind == "signed_product" else coef[0] + coef[1] * S1 + coef[2] * S2 + coef[3] * S1 * S2
    return (C * A) @ v


def causal_row_scale(row_scale):
    """C for one row of one document: lower-triangular ones times the per-query row scale (T,) -> (T, T)."""
    T = row_scale.shape[0]
    return torch.ones(T, T, dtype=row_scale.dtype).tril() * row_scale[:, None]
