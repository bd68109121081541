"""Full-model parity through the "hip" backend, and the compiled (custom-op) path.

Mirrors ref: tests/test_kernels.py:106-125: the same two-layer model with the dense reference attention and with
the fast operator, documents and padding in the batch, loss within 1e-4 * |loss| and every parameter gradient
within 1e-3 (relative Frobenius norm), float32.
"""
from __future__ import annotations

import pytest
import torch

from mini_lm import MiniLM

pytestmark = pytest.mark.gpu


def _rel(x, ref):
    return ((x.float() - ref.float()).norm() / ref.float().norm().clamp(min=1e-30)).item()


def _batch(dev):
    g = torch.Generator().manual_seed(0)
    idx = torch.randint(0, 97, (2, 100), generator=g).to(dev)
    doc = torch.zeros(2, 100, dtype=torch.long, device=dev)
    doc[0, 30:] = 1
    doc[1, 90:] = -1
    tgt = idx.roll(-1, 1).masked_fill(doc < 0, -100)
    return idx, doc, tgt


def _pair(kind, mlp, dev, degree=2):
    torch.manual_seed(0)
    ref = MiniLM(kind, mlp, backend="reference", degree=degree).to(dev)
    hip = MiniLM(kind, mlp, backend="hip", degree=degree).to(dev)
    hip.load_state_dict(ref.state_dict())
    return ref, hip


@pytest.mark.parametrize("kind,mlp,degree", [("signed_product", "bilinear", 2), ("offset_square", "bilinear", 2),
                                             ("lower_degree_mix", "affine_bilinear", 2), ("power", "bilinear", 2),
                                             ("power", "bilinear", 4)])
def test_model_hip_backend_matches_reference(kind, mlp, degree):
    dev = torch.device("cuda:0")
    print(f"[model parity] kind={kind} mlp={mlp} degree={degree} B2 T100 fp32", flush=True)
    ref, hip = _pair(kind, mlp, dev, degree)
    idx, doc, tgt = _batch(dev)
    _, lr = ref(idx, doc, tgt)
    lr.backward()
    _, lh = hip(idx, doc, tgt)
    lh.backward()
    torch.cuda.synchronize()
    assert abs(lr.item() - lh.item()) < 1e-4 * abs(lr.item())
    for (n, a), (_, b) in zip(ref.named_parameters(), hip.named_parameters()):
        assert b.grad is not None, n
        assert _rel(b.grad, a.grad) < 1e-3, (n, _rel(b.grad, a.grad))


@pytest.mark.parametrize("kind,backend", [("signed_product", "aot_eager"), ("offset_square", "aot_eager"),
                                          ("lower_degree_mix", "aot_eager"), ("power", "aot_eager"),
                                          ("power", "inductor")])
def test_compiled_model_matches_eager(kind, backend):
    """torch.compile(fullgraph=True) traces the model with the operator as opaque tnpa:: custom ops (a graph break
    would raise); loss and gradients equal the eager run's. "inductor" is torch.compile's default backend, the one
    the reference trains with (ref: tnlm/train.py:353); it regenerates the model's other ops, so its tolerance is
    that of the model parity test rather than the bitwise-level 1e-5 of aot_eager."""
    dev = torch.device("cuda:0")
    print(f"[compiled model] kind={kind} backend={backend}", flush=True)
    torch._dynamo.reset()
    _, eager = _pair(kind, "bilinear", dev)
    _, comp = _pair(kind, "bilinear", dev)
    idx, doc, tgt = _batch(dev)
    _, le = eager(idx, doc, tgt)
    le.backward()
    fn = torch.compile(comp, backend=backend, fullgraph=True)
    _, lc = fn(idx, doc, tgt)
    lc.backward()
    torch.cuda.synchronize()
    ltol, gtol = (1e-6, 1e-5) if backend == "aot_eager" else (1e-4, 1e-3)
    assert abs(le.item() - lc.item()) <= ltol * abs(le.item())
    for (n, a), (_, b) in zip(eager.named_parameters(), comp.named_parameters()):
        assert _rel(b.grad, a.grad) < gtol, (n, _rel(b.grad, a.grad))


def test_document_bounds_computed_once_per_forward(monkeypatch):
    """A four-layer model runs the document-bounds prepass once per forward (the model context computes it and
    every layer's call receives it), and the backward reuses the forward's bounds."""
    import tensor_train_ing_amd.poly_attn as pa
    dev = torch.device("cuda:0")
    calls = []
    orig = pa.doc_bounds

    def counting(doc_ids):
        calls.append(tuple(doc_ids.shape))
        return orig(doc_ids)

    monkeypatch.setattr(pa, "doc_bounds", counting)
    torch.manual_seed(0)
    model = MiniLM("power", "bilinear", layers=4, backend="hip").to(dev)
    idx, doc, tgt = _batch(dev)
    _, loss = model(idx, doc, tgt)
    loss.backward()
    torch.cuda.synchronize()
    assert calls == [(2, 100)]


@pytest.mark.parametrize("kind", ["signed_product", "offset_square", "lower_degree_mix", "power"])
def test_custom_op_equals_autograd_function(kind):
    """The custom-op path launches the same kernels: bit-identical output and gradients (bf16, documents)."""
    from poly_ref import gaussian_inputs, row_scale
    from tensor_train_ing_amd import poly_attention_hip, poly_attention_op
    dev = torch.device("cuda:0")
    print(f"[custom op] kind={kind}", flush=True)
    two = kind in ("signed_product", "lower_degree_mix")
    q1, k1, q2, k2, v, do = (x.to(dev) for x in gaussian_inputs(2, 3, 200, 64, 64, torch.bfloat16, 5,
                                                                 qk_scale=64 ** -0.25, two_pairs=True))
    doc = torch.zeros(2, 200, dtype=torch.long, device=dev)
    doc[0, 70:] = 1
    doc[1, 150:] = -1
    rs = row_scale(doc, 0.5)
    coef = torch.tensor([[0.1, 0.2, -0.3, 1.0]], device=dev).repeat(3, 1) if kind == "lower_degree_mix" else None
    b = torch.full((3,), 0.5, device=dev) if kind == "offset_square" else None
    outs = []
    for fn in (poly_attention_hip, poly_attention_op):
        ins = [x.detach().clone().requires_grad_() for x in (q1, k1, q2, k2, v)]
        par = [t.detach().clone().requires_grad_() if t is not None else None for t in (coef, b)]
        o = fn(kind, ins[0], ins[1], ins[2] if two else None, ins[3] if two else None, ins[4], doc, rs,
               coef=par[0], b=par[1], degree=2 if kind == "power" else None)
        o.backward(do)
        grads = [t.grad for t in ins if t.grad is not None] + [t.grad for t in par if t is not None]
        outs.append([o.detach()] + grads)
    torch.cuda.synchronize()
    assert len(outs[0]) == len(outs[1])
    for a, b_ in zip(*outs):
        assert torch.equal(a, b_)


@pytest.mark.parametrize("kind", ["power", "signed_product"])
def test_custom_op_with_rope_equals_autograd_function(kind):
    """With rotary tables the custom-op path rotates through tnpa::rope (gradient: the inverse rotation op) and the
    autograd Function applies the inverse inside the backward: the same arithmetic, bit-identical results."""
    from poly_ref import doc_positions, gaussian_inputs, rope_tables, row_scale
    from tensor_train_ing_amd import poly_attention_hip, poly_attention_op
    dev = torch.device("cuda:0")
    print(f"[custom op rope] kind={kind}", flush=True)
    two = kind == "signed_product"
    q1, k1, q2, k2, v, do = (x.to(dev) for x in gaussian_inputs(2, 3, 160, 128, 128, torch.bfloat16, 7,
                                                                 qk_scale=128 ** -0.25, two_pairs=True))
    doc = torch.zeros(2, 160, dtype=torch.long, device=dev)
    doc[0, 50:] = 1
    rs = row_scale(doc, 0.5)
    rope = rope_tables(doc_positions(doc), 128)
    outs = []
    for fn in (poly_attention_hip, poly_attention_op):
        ins = [x.detach().clone().requires_grad_() for x in (q1, k1, q2, k2, v)]
        o = fn(kind, ins[0], ins[1], ins[2] if two else None, ins[3] if two else None, ins[4], doc, rs,
               degree=2 if kind == "power" else None, rope=rope)
        o.backward(do)
        outs.append([o.detach()] + [t.grad for t in ins if t.grad is not None])
    torch.cuda.synchronize()
    assert len(outs[0]) == len(outs[1])
    for a, b_ in zip(*outs):
        assert torch.equal(a, b_)
