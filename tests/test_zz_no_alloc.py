"""tnpa_backward_noalloc (the allocation-free backward, with its scratch in a fixed device array) against
tnpa_backward (caller-allocated workspace), called through the C ABI, on two calls in a row, the second on a smaller
problem, so stale scratch from the first call cannot leak into the second: bit-identical dK, dV and dcoef/db, and
bit-identical dQ except where tnpa_backward computes dQ from stored dS tiles (16-bit, one q/k pair, head dim 128),
which its fixed scratch cannot hold: there both dQ agree to 5e-3 relative Frobenius (S rounded inside a different
pair of products), within the bf16 tolerance of the reference."""
from __future__ import annotations

import ctypes

import pytest
import torch

from poly_ref import gaussian_inputs, rel_fro, row_scale

pytestmark = pytest.mark.gpu


def _run(entry, kind, B, H, T, D, seed, rope=False):
    from tensor_train_ing_amd import _abi
    from tensor_train_ing_amd.poly_attn import KINDS, _desc, _problem, _stream, doc_bounds
    lib = _abi.load()
    two = kind in ("signed_product", "lower_degree_mix")
    q1, k1, q2, k2, v, dout = (None if x is None else x.cuda() for x in gaussian_inputs(
        B, H, T, D, D, torch.bfloat16, seed, qk_scale=D ** -0.25, two_pairs=two))
    doc = torch.zeros(B, T, dtype=torch.long, device="cuda")
    doc[0, T // 3:] = 1
    doc[-1, T - T // 5:] = -1
    dstart, qend = doc_bounds(doc)
    rs = row_scale(doc, 0.5).float().contiguous()
    coef = torch.tensor([[0.3, -0.5, 0.7, 1.1]], device="cuda").repeat(H, 1).contiguous()
    bb = torch.linspace(-1, 1.5, H, device="cuda").contiguous()
    tabs = None
    if rope:  # q/k stand for rotated inputs; the backward applies the rotation's gradient to dq / dk
        from poly_ref import doc_positions, rope_tables
        cos, sin = rope_tables(doc_positions(doc), D)
        tabs = (cos[:, 0].contiguous(), sin[:, 0].contiguous())
    prob = _problem(KINDS[kind], 2, q1, k1, q2 if two else q1, k2 if two else k1, v, dstart, qend, rs,
                    coef if kind == "lower_degree_mix" else None, bb if kind == "offset_square" else None, rope=tabs)
    out = {n: torch.full_like(x, float("nan")) for n, x in (("dq1", q1), ("dk1", k1), ("dv", v), ("dq2", q1),
                                                              ("dk2", k1))}
    out["dpar"] = torch.full((H, 4), float("nan"), device="cuda")
    nbytes = lib.tnpa_backward_workspace_bytes(ctypes.byref(prob))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device="cuda") if entry == "tnpa_backward" else None
    g = _abi.Grads(_desc(dout), _desc(out["dq1"]), _desc(out["dk1"]), _desc(out["dq2"] if two else out["dq1"]),
                   _desc(out["dk2"] if two else out["dk1"]), _desc(out["dv"]), out["dpar"].data_ptr(),
                   ws.data_ptr() if ws is not None else None, nbytes if ws is not None else 0)
    _abi.check(getattr(lib, entry)(ctypes.byref(prob), ctypes.byref(g), _stream(q1.device)), entry)
    torch.cuda.synchronize()
    keep = ["dq1", "dk1", "dv"] + (["dq2", "dk2"] if two else []) + (
        ["dpar"] if kind in ("offset_square", "lower_degree_mix") else [])
    return {n: out[n] for n in keep}


@pytest.mark.parametrize("kind,D,rope", [("offset_square", 64, False), ("lower_degree_mix", 64, False),
                                         ("offset_square", 128, False), ("power", 128, False), ("power", 128, True),
                                         ("signed_product", 64, True), ("power", 256, True)])
def test_noalloc_backward_equals_workspace_backward(kind, D, rope):
    print(f"[noalloc] kind={kind} D={D} rope={rope}", flush=True)
    for B, H, T, seed in ((2, 4, 700, 1), (1, 2, 190, 2)):  # the second call is smaller
        a = _run("tnpa_backward", kind, B, H, T, D, seed, rope)
        b = _run("tnpa_backward_noalloc", kind, B, H, T, D, seed, rope)
        for n in a:
            assert torch.isfinite(a[n]).all(), n
            if n == "dq1" and D == 128 and kind in ("power", "offset_square"):
                assert rel_fro(a[n], b[n]) < 5e-3, (kind, D, T, n)
            else:
                assert torch.equal(a[n], b[n]), (kind, D, T, n)


def test_noalloc_rejects_problems_beyond_its_scratch():
    """A problem whose dcoef/db partials exceed the 1 MiB array is refused before anything is enqueued (checked
    with fake, never dereferenced addresses)."""
    from tensor_train_ing_amd import _abi
    lib = _abi.load()
    t = _abi.Tensor(4096, 64 * 4096 * 64, 4096 * 64, 64)
    p = _abi.Problem(64, 64, 4096, 64, 64, _abi.OFFSET_SQUARE, 2, _abi.BF16, t, t, t, t, t, 4096, 4096, 4096, None,
                     4096)
    g = _abi.Grads(t, t, t, t, t, t, 4096, None, 0)
    assert lib.tnpa_backward_noalloc(ctypes.byref(p), ctypes.byref(g), None) == _abi.ERR_UNSUPPORTED
    assert "scratch" in lib.tnpa_last_error().decode()
