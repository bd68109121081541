"""FP64 dense CPU restatement of tnlm's causal polynomial attention, forward and analytic backward.

TEST INFRASTRUCTURE ONLY. This module is the oracle that the HIP kernels are checked against. The product package
(`tensor_train_ing_amd`) never imports it; only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` do.

Semantics follow the reference's single authoritative implementation:

* `doc_positions`         ref: tnlm/attention.py:12-19
* `visible_mask`          ref: tnlm/attention.py:22-32   (causal, same document, both tokens real)
* `row_scale_mask`        ref: tnlm/attention.py:35-38   (C = visible * n_visible^-power, empty rows zero)
* `scores`                ref: tnlm/attention.py:54-55   (q k^T / sqrt(dk), each pair with its own dk)
* `polynomial_attention`  ref: tnlm/attention.py:58-77   (mask applied AFTER the polynomial; no softmax)
* `polynomial_attention_recurrent` ref: tnlm/attention.py:80-95
* analytic backward       ref: tensor_network_research_brief.md:319-329 (grad_V = P^T U, H = C*(U V^T),
                          grad_S1 = H*dA/dS1, grad_S2 = H*dA/dS2), and for the learned head scalars the
                          per-block partial sums of ref: tnlm/kernels/poly_attn.py:123-135,143-148,304-306.
* `row_scale_from_docs`   ref: tnlm/model.py:217-221 (n_visible = doc position + 1, 0 for padding)
* `block_bounds_reference` ref: tnlm/kernels/poly_attn.py:205-218 (LO/HI tile bounds), restated by brute force.

The build adds one kind the reference does not name: ``"power"`` with ``degree=p``, A = S^p over a single q/k pair.
It is pinned by the reference's own kinds through the identities S^2 = signed_product(q,k,q,k),
S^3 = signed_product(q,k,q(x)q,k(x)k) and S^4 = signed_product(q(x)q,k(x)k,q(x)q,k(x)k)
(tests/test_oracle.py checks all three).

Arrays are numpy; shapes are q*, k*: (B, H, T, dk), v: (B, H, T, dv), C: (B, 1|H, T, T), doc_ids: (B, T).
"""
from __future__ import annotations

import math

import numpy as np

KINDS = ("signed_product", "offset_square", "lower_degree_mix", "power")


# ------------------------------------------------------------------ masks and row scale
def doc_positions(doc_ids: np.ndarray) -> np.ndarray:
    """Position of each token within its (contiguous) document.  ref: tnlm/attention.py:12-19"""
    doc_ids = np.asarray(doc_ids)
    B, T = doc_ids.shape
    ar = np.broadcast_to(np.arange(T), (B, T))
    start = np.ones((B, T), dtype=bool)
    start[:, 1:] = doc_ids[:, 1:] != doc_ids[:, :-1]
    first = np.maximum.accumulate(np.where(start, ar, 0), axis=1)
    return ar - first


def visible_mask(doc_ids: np.ndarray) -> np.ndarray:
    """(B, 1, T, T) bool: causal, same document id, and both tokens real (id >= 0).  ref: tnlm/attention.py:22-32"""
    doc_ids = np.asarray(doc_ids)
    T = doc_ids.shape[1]
    causal = np.tril(np.ones((T, T), dtype=bool))
    same = doc_ids[:, :, None] == doc_ids[:, None, :]
    valid = doc_ids >= 0
    return (causal[None] & same & valid[:, :, None] & valid[:, None, :])[:, None]


def row_scale_mask(visible: np.ndarray, power: float, dtype=np.float64) -> np.ndarray:
    """C = visible * n_visible^-power; rows with no visible key are all zero.  ref: tnlm/attention.py:35-38"""
    n = np.maximum(visible.sum(-1, keepdims=True), 1).astype(dtype)
    return visible.astype(dtype) * n ** (-power)


def row_scale_from_docs(doc_ids: np.ndarray, power: float) -> np.ndarray:
    """(B, T) float32 row scale the tiled operator takes: (doc position + 1)^-power, 0 for padding.

    ref: tnlm/model.py:217-221 and ref: tests/test_kernels.py:30-32. For contiguous documents this equals the
    n_visible^-power factor of `row_scale_mask` on every real row."""
    pos = doc_positions(doc_ids)
    n = (pos + 1).astype(np.float64)
    return np.where(np.asarray(doc_ids) >= 0, n ** (-power), 0.0).astype(np.float32)


def doc_bounds(doc_ids: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token visibility bounds used by the tiled kernels (brute force, O(T^2) per row).

    doc_start[b, q] = smallest key visible from query q (q + 1 when q sees nothing, i.e. padding), so that
    visible(q, k) <=> doc_start[q] <= k <= q for contiguous documents.
    query_end[b, k] = one past the last query that can see key k (k when no query sees it).
    These restate the reference's LO/HI scans (ref: tnlm/kernels/poly_attn.py:205-218) at token granularity."""
    vis = visible_mask(doc_ids)[:, 0]
    B, T, _ = vis.shape
    start = np.empty((B, T), dtype=np.int32)
    qend = np.empty((B, T), dtype=np.int32)
    for b in range(B):
        for t in range(T):
            ks = np.nonzero(vis[b, t])[0]
            start[b, t] = ks[0] if len(ks) else t + 1
            qs = np.nonzero(vis[b, :, t])[0]
            qend[b, t] = qs[-1] + 1 if len(qs) else t
    return start, qend


def block_bounds_reference(doc_ids: np.ndarray, BM: int, BN: int) -> tuple[np.ndarray, np.ndarray]:
    """LO[b, mb] = document start of the first query of block mb; HI[b, nb] = exclusive end of the document run
    holding the last key of block nb.  Brute-force restatement of ref: tnlm/kernels/poly_attn.py:205-218 (a run
    of equal ids, padding included, counts as one document there)."""
    doc_ids = np.asarray(doc_ids)
    B, T = doc_ids.shape
    nmb, nnb = -(-T // BM), -(-T // BN)
    lo = np.empty((B, nmb), dtype=np.int32)
    hi = np.empty((B, nnb), dtype=np.int32)
    for b in range(B):
        for mb in range(nmb):
            t = mb * BM
            while t > 0 and doc_ids[b, t - 1] == doc_ids[b, mb * BM]:
                t -= 1
            lo[b, mb] = t
        for nb in range(nnb):
            last = min(nb * BN + BN - 1, T - 1)
            t = last
            while t + 1 < T and doc_ids[b, t + 1] == doc_ids[b, last]:
                t += 1
            hi[b, nb] = t + 1
    return lo, hi


# ------------------------------------------------------------------ forward
def scores(q: np.ndarray, k: np.ndarray) -> np.ndarray:
    """S = q k^T / sqrt(dk) with dk = q.shape[-1].  ref: tnlm/attention.py:54-55"""
    return q @ np.swapaxes(k, -1, -2) / math.sqrt(q.shape[-1])


def _poly(kind, S1, S2, coef, b, degree):
    """A(S1, S2) and its partial derivatives.  ref: tnlm/attention.py:66-75, ref: tnlm/kernels/poly_attn.py:26-34"""
    if kind == "signed_product":
        return S1 * S2, S2, S1
    if kind == "offset_square":
        t = S1 + np.asarray(b).reshape(1, -1, 1, 1)
        return t * t, 2.0 * t, None
    if kind == "lower_degree_mix":
        c = np.asarray(coef).reshape(1, -1, 4, 1, 1)
        c0, c1, c2, c12 = (c[:, :, i] for i in range(4))
        return c0 + c1 * S1 + c2 * S2 + c12 * S1 * S2, c1 + c12 * S2, c2 + c12 * S1
    if kind == "power":
        p = int(degree)
        if p < 1:
            raise ValueError(f"power kind needs degree >= 1, got {degree}")
        return S1 ** p, p * S1 ** (p - 1), None
    raise ValueError(kind)


def _pair_scores(kind, q1, k1, q2, k2):
    S1 = scores(q1, k1)
    S2 = scores(q2, k2) if kind in ("signed_product", "lower_degree_mix") else None
    return S1, S2


def polynomial_attention(kind, q1, k1, q2, k2, v, C, coef=None, b=None, degree=None):
    """Dense forward y = (C * A(S1, S2)) @ v.  ref: tnlm/attention.py:58-77 (plus the degree-p `power` kind)."""
    S1, S2 = _pair_scores(kind, q1, k1, q2, k2)
    A, _, _ = _poly(kind, S1, S2, coef, b, degree)
    P = C * A  # zero masking after the polynomial (ref: tnlm/attention.py:76)
    return P @ v


def polynomial_attention_backward(kind, q1, k1, q2, k2, v, C, dout, coef=None, b=None, degree=None):
    """Analytic gradients of `polynomial_attention` for upstream gradient U = dout.

    grad_V = P^T U; H = C * (U V^T); grad_S1 = H * dA/dS1; grad_S2 = H * dA/dS2
    (ref: tensor_network_research_brief.md:321-329); grad_q = grad_S k / sqrt(dk), grad_k = grad_S^T q / sqrt(dk).
    Head-scalar gradients are the sums the reference reduces from per-block partials
    (ref: tnlm/kernels/poly_attn.py:123-135,304-306): dcoef[h] = sum(H, H S1, H S2, H S1 S2), db[h] = sum(H * 2(S1+b)).

    Returns dict with dq1, dk1, dv and, where the kind uses them, dq2, dk2, dcoef, db."""
    S1, S2 = _pair_scores(kind, q1, k1, q2, k2)
    A, dA1, dA2 = _poly(kind, S1, S2, coef, b, degree)
    P = C * A
    U = dout
    out = {"dv": np.swapaxes(P, -1, -2) @ U}
    Hm = C * (U @ np.swapaxes(v, -1, -2))
    g1 = Hm * dA1
    out["dq1"] = g1 @ k1 / math.sqrt(q1.shape[-1])
    out["dk1"] = np.swapaxes(g1, -1, -2) @ q1 / math.sqrt(q1.shape[-1])
    if dA2 is not None:
        g2 = Hm * dA2
        out["dq2"] = g2 @ k2 / math.sqrt(q2.shape[-1])
        out["dk2"] = np.swapaxes(g2, -1, -2) @ q2 / math.sqrt(q2.shape[-1])
    if kind == "lower_degree_mix":
        red = lambda x: x.sum(axis=(0, 2, 3))  # noqa: E731  (B, H, T, T) -> (H,)
        out["dcoef"] = np.stack([red(Hm), red(Hm * S1), red(Hm * S2), red(Hm * S1 * S2)], axis=1)
    if kind == "offset_square":
        out["db"] = (Hm * dA1).sum(axis=(0, 2, 3))
    return out


def polynomial_attention_recurrent(q1, k1, q2, k2, v, scale):
    """Exact causal recurrent form of signed_product for one document.  ref: tnlm/attention.py:80-95

    state_t = state_{t-1} + (k1_t (x) k2_t) v_t^T;  y_t = scale_t (q1_t (x) q2_t)^T state_t / dk.
    Shapes (H, T, d); scale: (T,)."""
    H, T, dk = q1.shape
    dv = v.shape[-1]
    state = np.zeros((H, dk * dk, dv))
    ys = np.empty((H, T, dv))
    for t in range(T):
        kk = (k1[:, t, :, None] * k2[:, t, None, :]).reshape(H, -1)
        state = state + kk[:, :, None] * v[:, t, None, :]
        qq = (q1[:, t, :, None] * q2[:, t, None, :]).reshape(H, -1)
        ys[:, t] = np.einsum("hs,hsv->hv", qq, state) * scale[t] / dk
    return ys


def polynomial_attention_loops(kind, q1, k1, q2, k2, v, doc_ids, row_power, coef=None, b=None, degree=None):
    """Pure-Python triple loop over (b, h, i, j) for tiny inputs: an independent evaluation of the forward.

    Visibility and row scale are recomputed per query from the raw doc ids (ref: tnlm/attention.py:22-38)."""
    B, H, T, dk = q1.shape
    dv = v.shape[-1]
    y = np.zeros((B, H, T, dv))
    for bb in range(B):
        for hh in range(H):
            for i in range(T):
                vis = [j for j in range(i + 1) if doc_ids[bb][i] >= 0 and doc_ids[bb][j] == doc_ids[bb][i]]
                if not vis:
                    continue
                sc = len(vis) ** (-row_power)
                for j in vis:
                    s1 = sum(q1[bb, hh, i, d] * k1[bb, hh, j, d] for d in range(dk)) / math.sqrt(dk)
                    if kind == "signed_product":
                        d2 = q2.shape[-1]
                        s2 = sum(q2[bb, hh, i, d] * k2[bb, hh, j, d] for d in range(d2)) / math.sqrt(d2)
                        a = s1 * s2
                    elif kind == "offset_square":
                        a = (s1 + b[hh]) ** 2
                    elif kind == "lower_degree_mix":
                        d2 = q2.shape[-1]
                        s2 = sum(q2[bb, hh, i, d] * k2[bb, hh, j, d] for d in range(d2)) / math.sqrt(d2)
                        c = coef[hh]
                        a = c[0] + c[1] * s1 + c[2] * s2 + c[3] * s1 * s2
                    elif kind == "power":
                        a = s1 ** int(degree)
                    else:
                        raise ValueError(kind)
                    for e in range(dv):
                        y[bb, hh, i, e] += sc * a * v[bb, hh, j, e]
    return y


# ------------------------------------------------------------------ helpers
def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float values to the nearest bfloat16 (round-to-nearest-even), returned as float32."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(f.shape)
