"""Rotary position embedding on the HIP path: the one-pass rotation (tnpa_rope) against the reference's unfused
apply_rope and its autograd (ref: tnlm/attention.py:41-51), and poly_attention_hip(..., rope=...) against rotating
with the reference's tensor operations first (ref: tnlm/model.py:70-71,81-82): the same bits for the output and every
gradient, since both paths feed the kernels the same rotated q/k and apply the same fp32 gradient arithmetic."""
from __future__ import annotations

import pytest
import torch

from poly_ref import apply_rope, doc_positions, gaussian_inputs, rope_tables, row_scale

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _native():
    from tensor_train_ing_amd import _abi
    _abi.load()  # no fallback: a missing libtnpa.so fails here
    assert torch.cuda.is_available()


def _docs(B, T):
    doc = torch.zeros(B, T, dtype=torch.long)
    doc[0, T // 3:] = 1
    doc[-1, T - T // 5:] = -1
    return doc.cuda()


@pytest.mark.parametrize("dtype,D,layout", [(torch.bfloat16, 128, "bhtd"), (torch.bfloat16, 64, "bthd"),
                                             (torch.float16, 32, "bhtd"), (torch.float32, 16, "bthd"),
                                             (torch.float32, 128, "bhtd")])
def test_rope_kernel_matches_reference_apply_rope(dtype, D, layout):
    """Forward rotation bit-identical to apply_rope; inverse bit-identical to autograd's gradient of apply_rope
    (inputs with magnitudes up to ~30 so that products round; positions within documents as the reference's
    doc_positions gives them; strided (B, T, H, d) views are read in place)."""
    from tensor_train_ing_amd.poly_attn import rope_rotate, rope_tables_of
    print(f"[rope kernel] dtype={dtype} D={D} layout={layout}", flush=True)
    B, H, T = 2, 3, 333
    x, g, _, _, _, _ = (None if t is None else t.cuda()
                        for t in gaussian_inputs(B, H, T, D, D, dtype, 5, qk_scale=10.0, layout=layout))
    cos, sin = rope_tables(doc_positions(_docs(B, T)), D)
    cs, sn = rope_tables_of((cos, sin), x)
    y = rope_rotate(x, cs, sn)
    xr = x.detach().clone().requires_grad_()
    yr = apply_rope(xr, cos, sin)
    assert torch.equal(y, yr.detach())
    yr.backward(g)
    assert torch.equal(rope_rotate(g, cs, sn, inverse=True), xr.grad)
    # in place (out = x)
    z = x.contiguous()
    rope_rotate(z, cs, sn, out=z)
    assert torch.equal(z, y)


@pytest.mark.parametrize("kind,dtype,D,T", [("power", torch.bfloat16, 128, 300), ("power", torch.bfloat16, 64, 200),
                                             ("offset_square", torch.float16, 128, 160),
                                             ("signed_product", torch.bfloat16, 128, 250),
                                             ("lower_degree_mix", torch.bfloat16, 64, 130),
                                             ("power", torch.float32, 32, 100), ("power", torch.bfloat16, 16, 90),
                                             ("power", torch.bfloat16, 256, 150), ("power", torch.float32, 256, 80),
                                             ("signed_product", torch.bfloat16, 256, 120),
                                             ("lower_degree_mix", torch.float16, 256, 100)])
def test_fused_rope_matches_reference_rotation(kind, dtype, D, T):
    """poly_attention_hip(..., rope=(cos, sin)) on unrotated q/k against apply_rope + poly_attention_hip + autograd:
    output, dq, dk, dv (and dcoef / db) bit-identical. One q/k pair with head dims >= 32 applies the rotation's
    gradient in the dQ / dK epilogues; two pairs, head dim 16 and fp32 at head dim 256 in a pass after the
    backward."""
    from tensor_train_ing_amd import poly_attention_hip
    print(f"[rope fused] kind={kind} dtype={dtype} D={D} T={T}", flush=True)
    B, H = 2, 3
    two = kind in ("signed_product", "lower_degree_mix")
    q1, k1, q2, k2, v, dout = (None if t is None else t.cuda() for t in gaussian_inputs(
        B, H, T, D, D, dtype, 9, qk_scale=D ** -0.25, two_pairs=two))
    doc = _docs(B, T)
    rs = row_scale(doc, 0.5).float().contiguous()
    cos, sin = rope_tables(doc_positions(doc), D)
    coef = torch.tensor([[0.3, -0.5, 0.7, 1.1]], device="cuda").repeat(H, 1)
    bb = torch.linspace(-1, 1.5, H, device="cuda")
    deg = 2 if kind == "power" else None

    def run(fused):
        leaves = [t.detach().clone().requires_grad_() for t in (q1, k1, v) + ((q2, k2) if two else ())]
        cf = coef.clone().requires_grad_() if kind == "lower_degree_mix" else None
        b = bb.clone().requires_grad_() if kind == "offset_square" else None
        a1, b1, vv = leaves[:3]
        a2, b2 = (leaves[3], leaves[4]) if two else (None, None)
        if fused:
            o = poly_attention_hip(kind, a1, b1, a2, b2, vv, doc, rs, coef=cf, b=b, degree=deg, rope=(cos, sin))
        else:
            rot = lambda t: None if t is None else apply_rope(t, cos, sin)  # noqa: E731
            o = poly_attention_hip(kind, rot(a1), rot(b1), rot(a2), rot(b2), vv, doc, rs, coef=cf, b=b, degree=deg)
        o.backward(dout)
        res = [o.detach()] + [t.grad for t in leaves]
        res += [cf.grad] if cf is not None else []
        res += [b.grad] if b is not None else []
        return res

    for a, r in zip(run(True), run(False)):
        assert torch.equal(a, r)


def test_rope_with_shared_signed_product_pairs():
    """signed_product(q, k, q, k) runs as degree 2 with one rotation per tensor: the summed gradient equals the
    reference rotation's."""
    from tensor_train_ing_amd import poly_attention_hip
    B, H, T, D = 1, 2, 96, 64
    q, k, _, _, v, dout = (None if t is None else t.cuda()
                           for t in gaussian_inputs(B, H, T, D, D, torch.bfloat16, 3, qk_scale=D ** -0.25))
    doc = torch.zeros(B, T, dtype=torch.long, device="cuda")
    rs = row_scale(doc, 0.5).float().contiguous()
    cos, sin = rope_tables(doc_positions(doc), D)
    res = []
    for fused in (True, False):
        a, b, vv = (t.detach().clone().requires_grad_() for t in (q, k, v))
        if fused:
            o = poly_attention_hip("signed_product", a, b, a, b, vv, doc, rs, rope=(cos, sin))
        else:
            ra, rb = apply_rope(a, cos, sin), apply_rope(b, cos, sin)
            o = poly_attention_hip("signed_product", ra, rb, ra, rb, vv, doc, rs)
        o.backward(dout)
        res.append([o.detach(), a.grad, b.grad, vv.grad])
    for x, y in zip(*res):
        assert torch.equal(x, y)
