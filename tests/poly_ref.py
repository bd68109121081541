"""Test-side helpers: seeded inputs and a float64 torch restatement of the dense operator for GPU-sized checks.

`dense_reference` runs the dense form of ref: tnlm/attention.py:22-38,54-77 and the analytic backward of
ref: tensor_network_research_brief.md:321-329 in float64 on the inputs' device, one (b, h) slice at a time so that
memory stays O(T^2). It is itself pinned against the numpy oracle (oracle/poly_attention.py) in
tests/test_oracle.py::test_torch_reference_matches_oracle, and only serves as the checker where the numpy oracle
would be too slow (the full BASELINE configurations).
"""
from __future__ import annotations

import math

import torch


def visible(doc: torch.Tensor) -> torch.Tensor:
    """(T, T) bool for one row of doc ids: causal, same id, both >= 0."""
    T = doc.shape[0]
    causal = torch.ones(T, T, dtype=torch.bool, device=doc.device).tril()
    return causal & (doc[:, None] == doc[None, :]) & (doc[:, None] >= 0) & (doc[None, :] >= 0)


def _poly(kind, S1, S2, c, bh, degree):
    if kind == "signed_product":
        return S1 * S2, S2, S1
    if kind == "offset_square":
        t = S1 + bh
        return t * t, 2 * t, None
    if kind == "lower_degree_mix":
        return c[0] + c[1] * S1 + c[2] * S2 + c[3] * S1 * S2, c[1] + c[3] * S2, c[2] + c[3] * S1
    if kind == "power":
        return S1 ** degree, degree * S1 ** (degree - 1), None
    raise ValueError(kind)


@torch.no_grad()
def dense_reference(kind, q1, k1, q2, k2, v, dout, doc_ids, row_scale, coef=None, b=None, degree=None,
                    grads=True):
    """Returns dict(out, dq1, dk1, dv[, dq2, dk2][, dcoef][, db]) in float64. C = visible * row_scale[query]."""
    two = kind in ("signed_product", "lower_degree_mix")
    B, H, T, dk = q1.shape
    f = lambda x: None if x is None else x.to(torch.float64)  # noqa: E731
    q1, k1, v = f(q1), f(k1), f(v)
    q2, k2 = (f(q2), f(k2)) if two else (None, None)
    dout = f(dout)
    sm = 1.0 / math.sqrt(dk)
    res = {"out": torch.empty(B, H, T, v.shape[-1], dtype=torch.float64, device=q1.device)}
    if grads:
        for n, x in (("dq1", q1), ("dk1", k1), ("dv", v)) + ((("dq2", q2), ("dk2", k2)) if two else ()):
            res[n] = torch.empty_like(x)
        if kind == "lower_degree_mix":
            res["dcoef"] = torch.zeros(H, 4, dtype=torch.float64, device=q1.device)
        if kind == "offset_square":
            res["db"] = torch.zeros(H, dtype=torch.float64, device=q1.device)
    for bb in range(B):
        C = visible(doc_ids[bb]).to(torch.float64) * row_scale[bb].to(torch.float64)[:, None]
        for hh in range(H):
            S1 = (q1[bb, hh] @ k1[bb, hh].t().contiguous()) * sm
            S2 = (q2[bb, hh] @ k2[bb, hh].t().contiguous()) * sm if two else None
            c = coef[hh].to(torch.float64) if coef is not None else None
            bh = float(b[hh]) if b is not None else 0.0
            A, dA1, dA2 = _poly(kind, S1, S2, c, bh, degree)
            P = C * A
            res["out"][bb, hh] = P @ v[bb, hh]
            if not grads:
                continue
            U = dout[bb, hh]
            res["dv"][bb, hh] = P.t().contiguous() @ U
            Hm = C * (U @ v[bb, hh].t().contiguous())
            g1 = Hm * dA1
            res["dq1"][bb, hh] = (g1 @ k1[bb, hh]) * sm
            res["dk1"][bb, hh] = (g1.t().contiguous() @ q1[bb, hh]) * sm
            if two:
                g2 = Hm * dA2
                res["dq2"][bb, hh] = (g2 @ k2[bb, hh]) * sm
                res["dk2"][bb, hh] = (g2.t().contiguous() @ q2[bb, hh]) * sm
            if kind == "lower_degree_mix":
                res["dcoef"][hh] += torch.stack([Hm.sum(), (Hm * S1).sum(), (Hm * S2).sum(), (Hm * S1 * S2).sum()])
            if kind == "offset_square":
                res["db"][hh] += (Hm * dA1).sum()
    return res


def doc_positions(doc: torch.Tensor) -> torch.Tensor:
    B, T = doc.shape
    ar = torch.arange(T, device=doc.device).expand(B, T)
    start = torch.ones_like(doc, dtype=torch.bool)
    start[:, 1:] = doc[:, 1:] != doc[:, :-1]
    first = torch.where(start, ar, torch.zeros_like(ar)).cummax(-1).values
    return ar - first


def rope_tables(positions: torch.Tensor, dim: int, base: float = 10000.0):
    """(cos, sin), each (B, 1, T, dim/2) fp32, of per-token positions (B, T): ref: tnlm/attention.py:41-45."""
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, device=positions.device, dtype=torch.float32) / dim))
    ang = positions.float()[..., None] * inv
    return ang.cos()[:, None], ang.sin()[:, None]


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The reference's unfused rotary embedding as separate tensor operations (ref: tnlm/attention.py:48-51): the
    checker of the one-pass kernel and, through autograd, of its inverse."""
    x1, x2 = x.to(torch.promote_types(x.dtype, torch.float32)).chunk(2, dim=-1)
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1).to(x.dtype)


def row_scale(doc: torch.Tensor, power: float) -> torch.Tensor:
    """(pos + 1)^-power for real tokens, 0 for padding (ref: tests/test_kernels.py:30-32, tnlm/model.py:217-221)."""
    pos = doc_positions(doc)
    return torch.where(doc >= 0, (pos + 1).double().pow(-power), torch.zeros((), dtype=torch.float64,
                                                                              device=doc.device)).float()


def rel_fro(x: torch.Tensor, ref: torch.Tensor) -> float:
    """Frobenius relative error, the reference's metric (ref: tests/test_kernels.py:14-15)."""
    x, ref = x.double(), ref.double()
    return float((x - ref).norm() / ref.norm().clamp_min(1e-300))


def rel_max(x: torch.Tensor, ref: torch.Tensor) -> float:
    """max|x - ref| / max|ref|: the tolerance BASELINE.json states for bf16 (<= 2e-2)."""
    x, ref = x.double(), ref.double()
    return float((x - ref).abs().max() / ref.abs().max().clamp_min(1e-300))


def gaussian_inputs(B, H, T, dk, dv, dtype, seed, qk_scale=1.0, boost_rows=0.0, two_pairs=False, layout="bhtd"):
    """Seeded CPU draws (torch.Generator), rounded to `dtype` on the CPU, so every machine sees the same bits.
    boost_rows: fraction of token rows of q and of k (independently) multiplied by 4."""
    g = torch.Generator().manual_seed(seed)

    def mk(d, scale):
        x = torch.randn(B, T, H, d, generator=g) * scale
        return x.transpose(1, 2) if layout == "bthd" else x.permute(0, 2, 1, 3).contiguous()

    q1, k1 = mk(dk, qk_scale), mk(dk, qk_scale)
    if boost_rows:
        for x in (q1, k1):
            rows = torch.rand(B, T, generator=g) < boost_rows
            x.mul_(torch.where(rows, 4.0, 1.0)[:, None, :, None])
    q2, k2 = (mk(dk, qk_scale), mk(dk, qk_scale)) if two_pairs else (None, None)
    v, dout = mk(dv, 1.0), mk(dv, 1.0)
    cast = lambda x: None if x is None else x.to(dtype)  # noqa: E731
    return tuple(cast(x) for x in (q1, k1, q2, k2, v, dout))
