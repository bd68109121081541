"""The polynomial attention as registered torch custom ops, for callers that compile their model.

The reference trains a compiled model (ref: tnlm/train.py:353); its Triton operator is traced through. A ctypes
call cannot be traced, so the same HIP kernels are registered here as three opaque custom ops with fake (shape)
implementations and an autograd formula:

    tnpa::doc_bounds               (doc_ids) -> (doc_start, query_end)
    tnpa::poly_attention           (kind, degree, q1, k1, q2?, k2?, v, doc_start, query_end, row_scale, coef?, b?,
                                    want_norms) -> (o, score_norms)   (score_norms empty unless want_norms)
    tnpa::poly_attention_backward  (kind, degree, q1, k1, q2?, k2?, v, doc_start, query_end, row_scale, coef?, b?, dO)
                                   -> (dq1, dk1, dq2, dk2, dv, dpar)
    tnpa::rope                     (x, cos, sin, inverse) -> rotated x   (its gradient: the same op, inverted)

Outputs and gradients are contiguous (B, H, T, d); dq2/dk2 are empty for one-pair kinds and dpar is empty unless the
kind has head parameters. The document bounds are an input of the attention op: computed once per batch by a model
(or once per call when the caller passes none) and handed to the backward, as the reference's autograd.Function
saves its LO/HI (ref: tnlm/kernels/poly_attn.py:281). `poly_attention_hip` switches to these ops by itself while
torch.compile traces it.
"""
from typing import Optional

import torch

from . import _abi
from .poly_attn import _canonical, _prep, _run_backward, _run_forward, doc_bounds, rope_rotate, rope_tables_of

_PAR_KINDS = (_abi.OFFSET_SQUARE, _abi.LOWER_DEGREE_MIX)
_TWO_PAIRS = (_abi.SIGNED_PRODUCT, _abi.LOWER_DEGREE_MIX)


@torch.library.custom_op("tnpa::doc_bounds", mutates_args=())
def doc_bounds_op(doc_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return doc_bounds(doc_ids)


@doc_bounds_op.register_fake
def _bounds_fake(doc_ids):
    B, T = doc_ids.shape
    return doc_ids.new_empty((B, T), dtype=torch.int32), doc_ids.new_empty((B, T), dtype=torch.int32)


@torch.library.custom_op("tnpa::rope", mutates_args=())
def rope_op(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool) -> torch.Tensor:
    return rope_rotate(x, cos, sin, inverse)


@rope_op.register_fake
def _rope_fake(x, cos, sin, inverse):
    return x.new_empty(x.shape)


def _rope_setup(ctx, inputs, output):
    _x, cos, sin, inverse = inputs
    ctx.inverse = inverse
    ctx.save_for_backward(cos, sin)


def _rope_backward(ctx, g):
    cos, sin = ctx.saved_tensors
    return rope_op(g.contiguous(), cos, sin, not ctx.inverse), None, None, None


rope_op.register_autograd(_rope_backward, setup_context=_rope_setup)


def _norms_shape(kind, H, want):
    return ((2 if kind in _TWO_PAIRS else 1), 2, H) if want else (0,)


@torch.library.custom_op("tnpa::poly_attention", mutates_args=())
def _fwd(kind: int, degree: int, q1: torch.Tensor, k1: torch.Tensor, q2: Optional[torch.Tensor],
         k2: Optional[torch.Tensor], v: torch.Tensor, doc_start: torch.Tensor, query_end: torch.Tensor,
         row_scale: torch.Tensor, coef: Optional[torch.Tensor], b: Optional[torch.Tensor],
         want_norms: bool) -> tuple[torch.Tensor, torch.Tensor]:
    norms = torch.zeros(_norms_shape(kind, q1.shape[1], want_norms), dtype=torch.float32, device=q1.device)
    o, *_ = _run_forward(kind, degree if degree > 0 else None, q1, k1, q2, k2, v, doc_start, row_scale, coef, b,
                         out_like_v=False, bounds=(doc_start, query_end), score_norms=norms if want_norms else None)
    return o, norms


@_fwd.register_fake
def _fwd_fake(kind, degree, q1, k1, q2, k2, v, doc_start, query_end, row_scale, coef, b, want_norms):
    return v.new_empty(v.shape), q1.new_empty(_norms_shape(kind, q1.shape[1], want_norms), dtype=torch.float32)


@torch.library.custom_op("tnpa::poly_attention_backward", mutates_args=())
def _bwd(kind: int, degree: int, q1: torch.Tensor, k1: torch.Tensor, q2: Optional[torch.Tensor],
         k2: Optional[torch.Tensor], v: torch.Tensor, doc_start: torch.Tensor, query_end: torch.Tensor,
         row_scale: torch.Tensor, coef: Optional[torch.Tensor], b: Optional[torch.Tensor],
         dout: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                      torch.Tensor]:
    two = kind in _TWO_PAIRS
    q1, k1, v = _prep(q1), _prep(k1), _prep(v)
    q2, k2 = (_prep(q2), _prep(k2)) if two else (q1, k1)
    sc = row_scale.detach().float().contiguous()
    coef_f = coef.detach().float().contiguous() if kind == _abi.LOWER_DEGREE_MIX else None
    b_f = b.detach().float().contiguous() if kind == _abi.OFFSET_SQUARE else None
    dq1, dk1, dq2, dk2, dv, dpar = _run_backward(kind, degree if degree > 0 else None, q1, k1, q2, k2, v,
                                                 doc_start, query_end, sc, coef_f, b_f, dout,
                                                 grads_like_inputs=False)
    # one-pair kinds: distinct empty tensors (custom-op outputs may not alias each other)
    return (dq1, dk1, dq2 if two else q1.new_empty(0), dk2 if two else q1.new_empty(0), dv,
            dpar if dpar is not None else q1.new_empty(0, dtype=torch.float32))


@_bwd.register_fake
def _bwd_fake(kind, degree, q1, k1, q2, k2, v, doc_start, query_end, row_scale, coef, b, dout):
    two = kind in _TWO_PAIRS
    H = q1.shape[1]
    return (q1.new_empty(q1.shape), k1.new_empty(k1.shape), q2.new_empty(q2.shape) if two else q1.new_empty(0),
            k2.new_empty(k2.shape) if two else q1.new_empty(0), v.new_empty(v.shape),
            q1.new_empty((H, 4), dtype=torch.float32) if kind in _PAR_KINDS else q1.new_empty(0, dtype=torch.float32))


def _setup_context(ctx, inputs, output):
    kind, degree, q1, k1, q2, k2, v, dstart, qend, row_scale, coef, b, _want = inputs
    ctx.kind, ctx.degree = kind, degree
    ctx.coef_dtype = coef.dtype if coef is not None else None
    ctx.b_dtype = b.dtype if b is not None else None
    ctx.save_for_backward(q1, k1, q2, k2, v, dstart, qend, row_scale, coef, b)


def _backward(ctx, do, _dnorms):
    q1, k1, q2, k2, v, dstart, qend, row_scale, coef, b = ctx.saved_tensors
    kind = ctx.kind
    dq1, dk1, dq2, dk2, dv, dpar = _bwd(kind, ctx.degree, q1, k1, q2, k2, v, dstart, qend, row_scale, coef, b,
                                        do.contiguous())
    two = kind in _TWO_PAIRS
    dcoef = dpar.to(ctx.coef_dtype) if (kind == _abi.LOWER_DEGREE_MIX and coef is not None) else None
    db = dpar[:, 0].to(ctx.b_dtype) if (kind == _abi.OFFSET_SQUARE and b is not None) else None
    return (None, None, dq1, dk1, dq2 if two else None, dk2 if two else None, dv, None, None, None, dcoef, db, None)


_fwd.register_autograd(_backward, setup_context=_setup_context)


def poly_attention_op(kind, q1, k1, q2, k2, v, doc_ids, row_scale, coef=None, b=None, *, degree=None, bounds=None,
                      score_norms=None, rope=None):
    """poly_attention_hip through the registered custom ops (same arguments, same results; contiguous output).
    Unknown kinds raise KeyError, as the reference. With rotary tables, q/k are rotated by tnpa::rope (whose
    gradient is the inverse rotation, the same arithmetic the eager backward applies in the library)."""
    K, degree = _canonical(kind, q1, k1, q2, k2, degree)
    two = K in _TWO_PAIRS
    if rope is not None:
        cs, sn = rope_tables_of(rope, q1)
        q1, k1 = rope_op(q1, cs, sn, False), rope_op(k1, cs, sn, False)
        if two:
            q2, k2 = rope_op(q2, cs, sn, False), rope_op(k2, cs, sn, False)
    dstart, qend = doc_bounds_op(doc_ids) if bounds is None else bounds
    o, norms = _fwd(K, int(degree) if degree is not None else 0, q1, k1, q2 if two else None, k2 if two else None,
                    v, dstart, qend, row_scale, coef if K == _abi.LOWER_DEGREE_MIX else None,
                    b if K == _abi.OFFSET_SQUARE else None, score_norms is not None)
    if score_norms is not None:
        score_norms.copy_(torch.maximum(score_norms, norms))
    return o
