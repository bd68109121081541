"""Pins the CPU oracle (oracle/poly_attention.py) without trusting its own formulas.

Each check is an independent route to the same quantity, chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails at least one of them:
  * forward vs a pure-Python (b, h, i, j) loop over visible pairs (ref: tnlm/attention.py:22-38,54-77);
  * forward vs the exact recurrent form (ref: tnlm/attention.py:80-95; equal at 1e-12 per ref: tests/test_math.py:142-149);
  * the degree-p kind vs the reference's signed_product on tensor-squared inputs (S^2, S^3, S^4 identities);
  * analytic backward vs central finite differences and vs torch autograd of the dense forward
    (ref: tests/test_math.py:113-139);
  * masking / padding special cases (ref: tests/test_math.py:152-162,285-297; tests/test_kernels.py:84-93);
  * the per-token document bounds vs brute force and vs the reference's LO/HI block bounds
    (ref: tnlm/kernels/poly_attn.py:205-218);
  * the committed golden fixtures regenerate bit for bit, and the float64 torch checker used by the GPU tests
    agrees with the oracle.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import (block_bounds_reference, doc_bounds, doc_positions, polynomial_attention,
                    polynomial_attention_backward, polynomial_attention_loops, polynomial_attention_recurrent,
                    round_to_bf16, row_scale_from_docs, row_scale_mask, scores, visible_mask)

KINDS = ["signed_product", "offset_square", "lower_degree_mix", "power"]
ROW_POWER = {"signed_product": 0.5, "offset_square": 1.0, "lower_degree_mix": 0.5, "power": 0.5}


def _inputs(B=2, H=3, T=7, dk=4, dv=5, seed=0):
    rng = np.random.default_rng(seed)
    q1, k1, q2, k2 = (rng.standard_normal((B, H, T, dk)) for _ in range(4))
    v = rng.standard_normal((B, H, T, dv))
    coef = rng.standard_normal((H, 4))
    b = rng.standard_normal(H)
    return q1, k1, q2, k2, v, coef, b


DOCS = np.array([[0, 0, 0, 1, 1, 1, 1], [0, 0, -1, 2, 2, -1, -1]])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("degree", [None, 3])
def test_forward_matches_python_loops(kind, degree):
    if kind == "power" and degree is None:
        degree = 2
    q1, k1, q2, k2, v, coef, b = _inputs()
    p = ROW_POWER[kind]
    C = row_scale_mask(visible_mask(DOCS), p)
    y = polynomial_attention(kind, q1, k1, q2, k2, v, C, coef=coef, b=b, degree=degree)
    y_loop = polynomial_attention_loops(kind, q1, k1, q2, k2, v, DOCS, p, coef=coef, b=b, degree=degree)
    np.testing.assert_allclose(y, y_loop, rtol=1e-12, atol=1e-12)


def test_recurrent_equals_direct():
    q1, k1, q2, k2, v, _, _ = _inputs(B=1, T=9)
    q1, k1, q2, k2, v = (x[0] for x in (q1, k1, q2, k2, v))
    C = row_scale_mask(visible_mask(np.zeros((1, 9), dtype=np.int64)), 0.5)
    direct = polynomial_attention("signed_product", q1[None], k1[None], q2[None], k2[None], v[None], C)[0]
    rec = polynomial_attention_recurrent(q1, k1, q2, k2, v, np.arange(1, 10, dtype=np.float64) ** -0.5)
    np.testing.assert_allclose(rec, direct, rtol=1e-12, atol=1e-12)


def _tsq(x):
    """Row-wise tensor square: (..., d) -> (..., d*d)."""
    return (x[..., :, None] * x[..., None, :]).reshape(*x.shape[:-1], -1)


def test_power_kind_equals_reference_kinds():
    """S^2 = signed_product(q,k,q,k) = offset_square(b=0); S^3 = signed_product(q,k,q(x)q,k(x)k);
    S^4 = signed_product(q(x)q,k(x)k,q(x)q,k(x)k) (tensor squares have head dim d^2, so 1/sqrt(d^2) = 1/d)."""
    q, k, _, _, v, _, _ = _inputs(dk=3)
    C = row_scale_mask(visible_mask(DOCS), 0.5)
    P = lambda deg: polynomial_attention("power", q, k, None, None, v, C, degree=deg)  # noqa: E731
    sp = lambda a1, b1, a2, b2: polynomial_attention("signed_product", a1, b1, a2, b2, v, C)  # noqa: E731
    np.testing.assert_allclose(P(2), sp(q, k, q, k), rtol=1e-12)
    np.testing.assert_allclose(P(2), polynomial_attention("offset_square", q, k, None, None, v, C,
                                                          b=np.zeros(q.shape[1])), rtol=1e-12)
    np.testing.assert_allclose(P(3), sp(q, k, _tsq(q), _tsq(k)), rtol=1e-11)
    np.testing.assert_allclose(P(4), sp(_tsq(q), _tsq(k), _tsq(q), _tsq(k)), rtol=1e-11)
    # the gradients of the identity hold too: d/dq of S^2 equals dq1 + dq2 of signed_product(q,k,q,k)
    U = np.random.default_rng(3).standard_normal(v.shape)
    gp = polynomial_attention_backward("power", q, k, None, None, v, C, U, degree=2)
    gs = polynomial_attention_backward("signed_product", q, k, q, k, v, C, U)
    np.testing.assert_allclose(gp["dq1"], gs["dq1"] + gs["dq2"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gp["dk1"], gs["dk1"] + gs["dk2"], rtol=1e-12, atol=1e-12)


def _loss(kind, args, U, degree):
    q1, k1, q2, k2, v, coef, b = args
    C = row_scale_mask(visible_mask(DOCS), ROW_POWER[kind])
    return float((polynomial_attention(kind, q1, k1, q2, k2, v, C, coef=coef, b=b, degree=degree) * U).sum())


@pytest.mark.parametrize("kind", KINDS)
def test_backward_matches_finite_differences(kind):
    degree = 3 if kind == "power" else None
    args = list(_inputs(seed=1))
    U = np.random.default_rng(2).standard_normal((2, 3, 7, 5))
    C = row_scale_mask(visible_mask(DOCS), ROW_POWER[kind])
    g = polynomial_attention_backward(kind, *args[:5], C, U, coef=args[5], b=args[6], degree=degree)
    names = {"signed_product": ["dq1", "dk1", "dq2", "dk2", "dv"], "offset_square": ["dq1", "dk1", "dv", "db"],
             "lower_degree_mix": ["dq1", "dk1", "dq2", "dk2", "dv", "dcoef"], "power": ["dq1", "dk1", "dv"]}[kind]
    index = {"dq1": 0, "dk1": 1, "dq2": 2, "dk2": 3, "dv": 4, "dcoef": 5, "db": 6}
    rng = np.random.default_rng(4)
    eps = 1e-6
    for n in names:
        x = args[index[n]]
        for _ in range(6):  # random coordinates of each gradient
            idx = tuple(rng.integers(0, s) for s in x.shape)
            old = x[idx]
            x[idx] = old + eps
            lp = _loss(kind, args, U, degree)
            x[idx] = old - eps
            lm = _loss(kind, args, U, degree)
            x[idx] = old
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - g[n][idx]) <= 1e-6 * max(1.0, abs(fd)), (n, idx, fd, g[n][idx])


@pytest.mark.parametrize("kind", KINDS)
def test_backward_matches_torch_autograd(kind):
    degree = 4 if kind == "power" else None
    args = _inputs(seed=5)
    U = np.random.default_rng(6).standard_normal((2, 3, 7, 5))
    C = row_scale_mask(visible_mask(DOCS), ROW_POWER[kind])
    g = polynomial_attention_backward(kind, *args[:5], C, U, coef=args[5], b=args[6], degree=degree)
    t = [torch.tensor(a, requires_grad=True) for a in args]
    q1, k1, q2, k2, v, coef, b = t
    S1 = q1 @ k1.transpose(-1, -2) / math.sqrt(q1.shape[-1])
    S2 = q2 @ k2.transpose(-1, -2) / math.sqrt(q2.shape[-1])
    A = {"signed_product": lambda: S1 * S2, "offset_square": lambda: (S1 + b.view(1, -1, 1, 1)) ** 2,
         "lower_degree_mix": lambda: (coef[:, 0].view(1, -1, 1, 1) + coef[:, 1].view(1, -1, 1, 1) * S1
                                      + coef[:, 2].view(1, -1, 1, 1) * S2 + coef[:, 3].view(1, -1, 1, 1) * S1 * S2),
         "power": lambda: S1 ** degree}[kind]()
    y = (torch.tensor(C) * A) @ v
    y.backward(torch.tensor(U))
    for n, x in zip(["dq1", "dk1", "dq2", "dk2", "dv", "dcoef", "db"], t):
        if n in g:
            np.testing.assert_allclose(g[n], x.grad.numpy(), rtol=1e-10, atol=1e-10, err_msg=n)
        else:
            assert x.grad is None or float(x.grad.abs().max()) == 0.0, n


def test_masked_entries_zero_after_polynomial():
    """Offset/constant terms must not leak through future or other-document entries."""
    q1, k1, q2, k2, v, _, _ = _inputs(B=1, T=6)
    doc = np.array([[0, 0, 1, 1, 1, 1]])
    C = row_scale_mask(visible_mask(doc), 1.0)
    b = np.full(q1.shape[1], 5.0)
    y = polynomial_attention("offset_square", q1, k1, q2, k2, v, C, b=b)
    v2 = v.copy()
    v2[:, :, 4:] += 100  # future positions
    v2[:, :, :2] += 100  # other document
    y2 = polynomial_attention("offset_square", q1, k1, q2, k2, v2, C, b=b)
    np.testing.assert_allclose(y[:, :, 2:4], y2[:, :, 2:4], rtol=1e-12)


def test_padding_rows_zero_and_never_attended():
    doc = np.array([[0, 0, -1, -1]])
    vis = visible_mask(doc)[0, 0]
    assert not vis[2:].any() and not vis[:, 2:].any()
    q1, k1, q2, k2, v, coef, b = _inputs(B=1, T=4)
    for kind in KINDS:
        C = row_scale_mask(visible_mask(doc), ROW_POWER[kind])
        y = polynomial_attention(kind, q1, k1, q2, k2, v, C, coef=np.ones((3, 4)), b=np.ones(3), degree=2)
        assert np.abs(y[:, :, 2:]).max() == 0


def test_zero_query_gives_zero_output_and_large_inputs_finite():
    q1, k1, q2, k2, v, _, _ = _inputs(B=1, T=8)
    C = row_scale_mask(visible_mask(np.zeros((1, 8), dtype=np.int64)), 0.5)
    assert np.abs(polynomial_attention("signed_product", 0 * q1, k1, q2, k2, v, C)).max() == 0
    assert np.abs(polynomial_attention("power", 0 * q1, k1, None, None, v, C, degree=4)).max() == 0
    assert np.isfinite(polynomial_attention("signed_product", 30 * q1, 30 * k1, q2, k2, v, C)).all()


def test_row_scale_from_docs_equals_visible_count():
    """n_visible = doc position + 1 for contiguous documents (ref: tnlm/model.py:217-221)."""
    doc = np.array([[0, 0, 0, 1, 1, -1, -1, 2], [5, 5, 5, 5, 5, 5, 5, 5]])
    for p in (0.5, 1.0):
        C = row_scale_mask(visible_mask(doc), p)[:, 0]
        rs = row_scale_from_docs(doc, p).astype(np.float64)
        real = doc >= 0
        np.testing.assert_allclose(rs[real], C.max(-1)[real], rtol=1e-6)
        assert (rs[~real] == 0).all()
    np.testing.assert_array_equal(doc_positions(doc)[0], [0, 1, 2, 0, 1, 0, 1, 0])


def _random_docs(rng, B, T):
    doc = np.zeros((B, T), dtype=np.int64)
    for bb in range(B):
        cuts = np.sort(rng.choice(np.arange(1, T), size=min(int(rng.integers(0, 6)), T - 1), replace=False))
        ids = np.searchsorted(cuts, np.arange(T), side="right")
        pad = rng.random(len(cuts) + 1) < 0.3
        doc[bb] = np.where(pad[ids], -1, ids)
    return doc


def test_doc_bounds_bruteforce_and_reference_block_bounds():
    rng = np.random.default_rng(7)
    for _ in range(20):
        B, T = 3, int(rng.integers(1, 90))
        doc = _random_docs(rng, B, T)
        start, qend = doc_bounds(doc)
        vis = visible_mask(doc)[:, 0]
        ar = np.arange(T)
        for bb in range(B):
            expect = (start[bb][:, None] <= ar[None, :]) & (ar[None, :] <= ar[:, None])
            np.testing.assert_array_equal(expect, vis[bb])
            # query_end: visible(q, k) implies q < query_end[k]; and query_end is monotone in k
            qs, ks = np.nonzero(vis[bb])
            assert (qs < qend[bb][ks]).all()
            assert (np.diff(qend[bb]) >= 0).all() and (np.diff(start[bb]) >= 0).all()
        # the reference's LO/HI tile bounds contain every visible pair of their tiles
        for BM, BN in ((16, 16), (32, 64)):
            lo, hi = block_bounds_reference(doc, BM, BN)
            for bb in range(B):
                qs, ks = np.nonzero(vis[bb])
                assert (ks >= lo[bb][qs // BM]).all() and (qs < hi[bb][ks // BN]).all()
                # per-token bounds are never looser than the reference's tile bounds
                assert (start[bb][::BM] >= lo[bb]).all()


# hand-derived bounds (ids, doc_start, query_end, {(BM, BN): (LO, HI)}): exact values, so a bound that is too loose
# or too tight fails, not only one that misses a visible pair
HAND = [
    ([0, 0, 0, 1, 1, -1, -1, 2], [0, 0, 0, 3, 3, 6, 7, 7], [3, 3, 3, 5, 5, 5, 6, 8],
     {(4, 4): ([0, 3], [5, 8]), (2, 2): ([0, 0, 3, 5], [3, 5, 7, 8]), (3, 3): ([0, 3, 5], [3, 7, 8])}),
    ([0, 0, 0, 0, 0], [0, 0, 0, 0, 0], [5, 5, 5, 5, 5], {(2, 2): ([0, 0, 0], [5, 5, 5])}),
    ([-1, -1, -1], [1, 2, 3], [0, 1, 2], {(2, 2): ([0, 0], [3, 3])}),
    ([0, 1, 2, 3], [0, 1, 2, 3], [1, 2, 3, 4], {(2, 2): ([0, 2], [2, 4])}),
    ([5, 5, -1, 7, 7, 7], [0, 0, 3, 3, 3, 3], [2, 2, 2, 6, 6, 6], {(2, 4): ([0, 2, 3], [6, 6])}),
]


@pytest.mark.parametrize("case", range(len(HAND)))
def test_doc_bounds_and_block_bounds_hand_derived(case):
    ids, start, qend, blocks = HAND[case]
    ds, qe = doc_bounds(np.array([ids]))
    assert ds.tolist() == [start] and qe.tolist() == [qend]
    for (BM, BN), (lo, hi) in blocks.items():
        rl, rh = block_bounds_reference(np.array([ids]), BM, BN)
        assert rl.tolist() == [lo] and rh.tolist() == [hi], (BM, BN)


def test_round_to_bf16_matches_torch():
    x = np.random.default_rng(8).standard_normal(10000).astype(np.float32) * 100
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_to_bf16(x), ref)


def test_golden_fixtures_regenerate_exactly():
    import json
    from pathlib import Path

    import importlib.util
    here = Path(__file__).resolve().parent / "golden"
    spec = importlib.util.spec_from_file_location("gen_golden", here / "gen_golden.py")
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    for name in gen.CASES:
        arrays, meta = gen.make_case(name)
        z = np.load(here / f"{name}.npz")
        assert json.loads(str(z["meta"])) == json.loads(json.dumps(meta))
        for k, v in arrays.items():
            np.testing.assert_array_equal(z[k], v, err_msg=f"{name}:{k}")


@pytest.mark.parametrize("kind", KINDS)
def test_torch_reference_matches_oracle(kind):
    """The float64 torch checker used by the GPU tests (tests/poly_ref.py) agrees with the oracle."""
    from poly_ref import dense_reference
    degree = 4 if kind == "power" else None
    q1, k1, q2, k2, v, coef, b = _inputs(seed=9)
    q2 = q2 if kind in ("signed_product", "lower_degree_mix") else None
    k2 = k2 if q2 is not None else None
    U = np.random.default_rng(10).standard_normal(v.shape)
    p = ROW_POWER[kind]
    C = row_scale_mask(visible_mask(DOCS), p)
    exp = polynomial_attention_backward(kind, q1, k1, q2, k2, v, C, U, coef=coef, b=b, degree=degree)
    exp["out"] = polynomial_attention(kind, q1, k1, q2, k2, v, C, coef=coef, b=b, degree=degree)
    tt = lambda x: None if x is None else torch.from_numpy(np.asarray(x))  # noqa: E731
    rs = torch.from_numpy(row_scale_from_docs(DOCS, p).astype(np.float64))
    got = dense_reference(kind, tt(q1), tt(k1), tt(q2), tt(k2), tt(v), tt(U), tt(DOCS), rs, tt(coef), tt(b), degree)
    for n, e in exp.items():
        # the row scale the operator takes is fp32, so agreement is to fp32 rounding of the largest entries
        np.testing.assert_allclose(got[n].numpy(), e, rtol=1e-6, atol=1e-6 * np.abs(e).max(), err_msg=n)


@pytest.mark.parametrize("kind,degree", [("power", 2), ("power", 4), ("signed_product", None),
                                         ("offset_square", None), ("lower_degree_mix", None)])
def test_torch_dense_baseline_matches_oracle(kind, degree):
    """The torch restatement bench.py times as the CPU baseline equals the numpy oracle, forward and (through
    autograd) backward, in float64 on one document with the (t+1)^-1/2 row scale."""
    from oracle import causal_row_scale, dense_attention
    rng = np.random.default_rng(31)
    T, D = 40, 16
    q1, k1, q2, k2, v, do = (rng.standard_normal((1, 1, T, D)) for _ in range(6))
    coef, b = np.array([[0.3, -0.5, 0.7, 1.1]]), np.array([0.25])
    rs = (np.arange(T) + 1.0) ** -0.5
    C = np.tril(np.ones((T, T)))[None, None] * rs[None, None, :, None]
    ref = polynomial_attention(kind, q1, k1, q2, k2, v, C, coef=coef, b=b, degree=degree)
    g = polynomial_attention_backward(kind, q1, k1, q2, k2, v, C, do, coef=coef, b=b, degree=degree)
    t = lambda x: torch.from_numpy(x[0, 0]).requires_grad_()  # noqa: E731
    ins = [t(x) for x in (q1, k1, q2, k2, v)]
    y = dense_attention(kind, *ins, causal_row_scale(torch.from_numpy(rs)), coef=torch.from_numpy(coef[0]),
                        b=float(b[0]), degree=degree)
    np.testing.assert_allclose(y.detach().numpy(), ref[0, 0], rtol=1e-10, atol=1e-10)
    y.backward(torch.from_numpy(do[0, 0]))
    for name, x in zip(("dq1", "dk1", "dq2", "dk2", "dv"), ins):
        if name in g and g[name] is not None:
            np.testing.assert_allclose(x.grad.numpy(), g[name][0, 0], rtol=1e-9, atol=1e-9)


# ------------------------------------------------------------------ fused linear + cross-entropy oracle
def _ce_fixture(noncontiguous=False, all_ignored=False):
    """The reference's CPU acceptance fixture (ref: tests/test_scaling_loss.py:9-23), float64."""
    g = torch.Generator().manual_seed(1407)
    if noncontiguous:
        x = torch.randn(7, 22, generator=g, dtype=torch.float64).T[::2]
        w = torch.randn(7, 26, generator=g, dtype=torch.float64).T[::2]
        t = torch.randint(0, 13, (22,), generator=g)[::2]
    else:
        x = torch.randn(11, 7, generator=g, dtype=torch.float64)
        w = torch.randn(13, 7, generator=g, dtype=torch.float64)
        t = torch.randint(0, 13, (11,), generator=g)
    t = t.clone()
    t[::3] = -100
    if all_ignored:
        t.fill_(-100)
    return x, w, t


@pytest.mark.parametrize("chunk", [1, 2, 4, 11, 30])
@pytest.mark.parametrize("noncontiguous", [False, True])
@pytest.mark.parametrize("scale", [1.0, -2.75, 0.0])
def test_linear_ce_oracle_matches_dense_cross_entropy(chunk, noncontiguous, scale):
    """The chunked oracle equals torch's dense F.cross_entropy (sum, ignore_index -100) and its autograd gradients,
    in float64, for every chunking (ref: tests/test_scaling_loss.py:26-57)."""
    import torch.nn.functional as F
    from oracle import linear_cross_entropy
    x, w, t = _ce_fixture(noncontiguous)
    xr, wr = x.detach().clone().requires_grad_(), w.detach().clone().requires_grad_()
    ref = F.cross_entropy(xr @ wr.T, t, ignore_index=-100, reduction="sum")
    gx, gw = torch.autograd.grad(ref, (xr, wr), grad_outputs=torch.tensor(scale, dtype=torch.float64))
    total, dx, dw, _ = linear_cross_entropy(x.numpy(), w.numpy(), t.numpy(), chunk=chunk, g=scale)
    np.testing.assert_allclose(total, ref.item(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dx, gx.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(dw, gw.numpy(), rtol=1e-11, atol=1e-12)


def test_linear_ce_oracle_all_ignored_and_finite_differences():
    from oracle import linear_cross_entropy
    x, w, t = _ce_fixture(all_ignored=True)
    total, dx, dw, _ = linear_cross_entropy(x.numpy(), w.numpy(), t.numpy(), chunk=4)
    assert total == 0.0 and not dx.any() and not dw.any()
    # central differences of the total in a few coordinates of x and w
    x, w, t = _ce_fixture()
    xn, wn, tn = x.numpy().copy(), w.numpy().copy(), t.numpy()
    _, dx, dw, _ = linear_cross_entropy(xn, wn, tn, chunk=3)
    eps = 1e-6
    for arr, grad in ((xn, dx), (wn, dw)):
        for idx in [(0, 0), (2, 5), (arr.shape[0] - 1, arr.shape[1] - 1)]:
            old = arr[idx]
            arr[idx] = old + eps
            up = linear_cross_entropy(xn, wn, tn, chunk=3)[0]
            arr[idx] = old - eps
            dn = linear_cross_entropy(xn, wn, tn, chunk=3)[0]
            arr[idx] = old
            np.testing.assert_allclose((up - dn) / (2 * eps), grad[idx], rtol=1e-6, atol=1e-8)


def test_linear_ce_oracle_bf16_rounding_points():
    """With bf16 rounding the oracle stays within bf16 distance of the float64 result, and rounds exactly where the
    reference does: its logits are bf16 values, so lse - logit[t] of a row uses those values."""
    from oracle import linear_cross_entropy, round_to_bf16
    rng = np.random.default_rng(5)
    x, w = rng.standard_normal((40, 16)), rng.standard_normal((30, 16)) * 0.5
    t = rng.integers(0, 30, 40)
    t[::4] = -100
    ex = linear_cross_entropy(x, w, t, chunk=7)
    bf = linear_cross_entropy(x, w, t, chunk=7, round_to=round_to_bf16)
    assert abs(bf[0] - ex[0]) <= 2e-2 * abs(ex[0])
    for a, b in zip(bf[1:3], ex[1:3]):
        assert np.abs(a - b).max() <= 3e-2 * np.abs(b).max()
    lg = round_to_bf16(round_to_bf16(x[:7]) @ round_to_bf16(w).T)
    m = lg.max(1, keepdims=True)
    np.testing.assert_allclose(bf[3][:7], (m + np.log(np.exp(lg - m).sum(1, keepdims=True)))[:, 0], rtol=1e-14)
