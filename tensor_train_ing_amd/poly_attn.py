"""Tiled causal polynomial attention on MI355X: forward and backward through libtnpa.so (HIP, gfx950).

Drop-in for the reference operator ref: tnlm/kernels/poly_attn.py (PolyAttention / poly_attention_triton):
same argument order, layouts, masking, row normalisation, dtype contract and gradient tuple. Computes, without
materialising any T x T matrix,
    y_i = scale_i * sum_{j visible from i} A(S1_ij, S2_ij) v_j,   S_ij = q_i . k_j / sqrt(dk)
with A one of
    signed_product   : S1 * S2
    offset_square    : (S1 + b_h)^2                (q2/k2 unused)
    lower_degree_mix : c0 + c1 S1 + c2 S2 + c12 S1 S2
    power            : S1^degree                   (this build's degree-p kind; q2/k2 unused)
"visible" = causal and same document (doc ids >= 0, contiguous per row); the mask is applied after the
polynomial; scale_i = n_visible_i^-p is precomputed by the caller (0 for padding queries).

signed_product called with q2 is q1 and k2 is k1 is recognised as degree 2 and computes one QK^T product.
The only numerical work on the host is argument checking; everything else runs in the HIP kernels.
"""
from __future__ import annotations

import ctypes

import torch

from . import _abi

KINDS = {"signed_product": _abi.SIGNED_PRODUCT, "offset_square": _abi.OFFSET_SQUARE,
         "lower_degree_mix": _abi.LOWER_DEGREE_MIX, "power": _abi.POWER}
_DTYPES = {torch.bfloat16: _abi.BF16, torch.float32: _abi.F32, torch.float16: _abi.F16}
_TWO_PAIRS = (_abi.SIGNED_PRODUCT, _abi.LOWER_DEGREE_MIX)


def _aligned_rows(x: torch.Tensor) -> bool:
    """Unit stride on the head dim, rows that do not overlap (a time stride of at least the head dim: a dO reduced
    or broadcast over time has stride 0) and 16-byte aligned rows, as the kernels' 128-bit loads require."""
    es = x.element_size()
    if x.stride(-1) != 1 or x.stride(2) < x.shape[-1] or x.data_ptr() % 16 or (x.stride(2) * es) % 16:
        return False
    if x.shape[0] > 1 and (x.stride(0) * es) % 16:
        return False
    if x.shape[1] > 1 and (x.stride(1) * es) % 16:
        return False
    return True


def _prep(x: torch.Tensor) -> torch.Tensor:
    """x itself when the kernels can index it in place, else a contiguous copy (ref: poly_attn.py:262-270)."""
    return x if _aligned_rows(x) else x.contiguous()


def _desc(x: torch.Tensor) -> _abi.Tensor:
    return _abi.Tensor(x.data_ptr(), x.stride(0), x.stride(1), x.stride(2))


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def doc_bounds(doc_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(doc_start, query_end) int32 (B, T): first key visible from each query (q + 1 for padding) and one past the
    last query that sees each key. Replaces ref: tnlm/kernels/poly_attn.py:205-218 (_block_bounds); int64 ids are
    read as int64 (no narrowing). A model computes them once per batch and hands them to every layer's call
    (`bounds=`), instead of each layer recomputing them from the same ids."""
    if torch.compiler.is_compiling():
        from .ops import doc_bounds_op
        return doc_bounds_op(doc_ids)
    doc = doc_ids
    if doc.dtype not in (torch.int32, torch.int64):
        doc = doc.long()
    if doc.dim() != 2:
        raise ValueError(f"doc_ids must be (B, T), got {tuple(doc.shape)}")
    if not doc.is_cuda:
        raise ValueError("poly_attention_hip needs tensors on a ROCm device (doc_ids is on the CPU)")
    B, T = doc.shape
    if doc.stride(1) != 1 or (B > 1 and doc.stride(0) < T):  # e.g. ids expanded over the batch (stride 0)
        doc = doc.contiguous()
    dstart = torch.empty(B, T, dtype=torch.int32, device=doc.device)
    qend = torch.empty(B, T, dtype=torch.int32, device=doc.device)
    lib = _abi.load()
    with torch.cuda.device(doc.device):
        _abi.check(lib.tnpa_doc_bounds(ctypes.c_void_p(doc.data_ptr()), int(doc.dtype == torch.int64),
                                       doc.stride(0), B, T, ctypes.c_void_p(dstart.data_ptr()),
                                       ctypes.c_void_p(qend.data_ptr()), _stream(doc.device)), "doc_bounds")
    return dstart, qend


def rope_tables_of(rope, q1: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) as the kernels read them: fp32 (B, T, dk/2) contiguous, from the reference's rope_tables layout
    (B, 1, T, dk/2) or from (B, T, dk/2) (ref: tnlm/attention.py:41-45)."""
    if not (isinstance(rope, (tuple, list)) and len(rope) == 2):
        raise ValueError("rope must be the (cos, sin) pair of rotary tables")
    B, _, T, DK = q1.shape
    out = []
    for name, t in zip(("cos", "sin"), rope):
        if t.dim() == 4 and t.shape[1] == 1:
            t = t[:, 0]
        if tuple(t.shape) != (B, T, DK // 2):
            raise ValueError(f"rope {name}: shape {tuple(t.shape)}, expected {(B, T, DK // 2)} or {(B, 1, T, DK // 2)}")
        if t.device != q1.device:
            raise ValueError(f"rope {name} must be on the same device as q1")
        if t.requires_grad and torch.is_grad_enabled():
            raise ValueError("rope tables are fixed position-only factors; differentiable tables are not supported")
        out.append(t.detach().float().contiguous())
    return out[0], out[1]


def rope_rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, inverse: bool = False,
                out: torch.Tensor = None) -> torch.Tensor:
    """One-pass rotary embedding of a (B, H, T, d) tensor (tnpa_rope): the reference's apply_rope
    (ref: tnlm/attention.py:48-51), bit-identical, or with inverse=True the gradient of that rotation. cos / sin as
    rope_tables_of returns them. Writes `out` (a new tensor by default; may be x)."""
    x = _prep(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    B, H, T, D = x.shape
    lib = _abi.load()
    with torch.cuda.device(x.device):
        _abi.check(lib.tnpa_rope(ctypes.byref(_desc(x)), ctypes.byref(_desc(out)), B, H, T, D, _DTYPES[x.dtype],
                                 ctypes.c_void_p(cos.data_ptr()), ctypes.c_void_p(sin.data_ptr()), int(inverse),
                                 _stream(x.device)), "rope")
    return out


def _validate(K, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, degree):
    if q1.dim() != 4 or v.dim() != 4:
        raise ValueError("q*, k*, v must be (B, H, T, d)")
    B, H, T, DK = q1.shape
    DV = v.shape[-1]
    assert DK >= 16 and DK & (DK - 1) == 0 and DV >= 16 and DV & (DV - 1) == 0, "head dims: powers of 2 >= 16"
    if not q1.is_cuda:
        raise ValueError("poly_attention_hip needs tensors on a ROCm device")
    if q1.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {q1.dtype}; expected bfloat16, float16 or float32")
    used = [("k1", k1), ("v", v)] + ([("q2", q2), ("k2", k2)] if K in _TWO_PAIRS else [])
    for name, t in used:
        if t is None:
            raise ValueError(f"{name} is required for this kind")
        if t.dtype != q1.dtype or t.device != q1.device:
            raise ValueError(f"{name}: dtype/device {t.dtype}/{t.device} differs from q1 {q1.dtype}/{q1.device}")
    for name, t in used[:1] + used[2:]:
        if tuple(t.shape) != (B, H, T, DK):
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {(B, H, T, DK)}")
    if tuple(v.shape[:3]) != (B, H, T):
        raise ValueError(f"v: shape {tuple(v.shape)}, expected {(B, H, T, DV)}")
    if tuple(doc_ids.shape) != (B, T) or tuple(row_scale.shape) != (B, T):
        raise ValueError(f"doc_ids and row_scale must be (B, T) = {(B, T)}")
    if doc_ids.device != q1.device or row_scale.device != q1.device:
        raise ValueError("doc_ids and row_scale must be on the same device as q1")
    if row_scale.requires_grad and torch.is_grad_enabled():
        raise ValueError("row_scale is a fixed position-only factor; a differentiable row_scale is not supported")
    if K == _abi.LOWER_DEGREE_MIX and (coef is None or tuple(coef.shape) != (H, 4)):
        raise ValueError("lower_degree_mix needs coef of shape (H, 4)")
    if K == _abi.OFFSET_SQUARE and (b is None or tuple(b.shape) != (H,)):
        raise ValueError("offset_square needs b of shape (H,)")
    if K == _abi.POWER and (degree is None or not 1 <= int(degree) <= 8):
        raise ValueError("power kind needs degree in 1..8")


def _canonical(kind, q1, k1, q2, k2, degree):
    """(kind code, degree): signed_product with shared pairs (q2 is q1 and k2 is k1) is degree-2 power."""
    K = KINDS[kind]  # unknown kind -> KeyError, as the reference
    if K == _abi.SIGNED_PRODUCT and q2 is q1 and k2 is k1:
        return _abi.POWER, 2
    return K, degree


def _check_bounds(bounds, doc_ids):
    """(doc_start, query_end) as doc_bounds(doc_ids) returns them: int32 (B, T), contiguous, on doc_ids' device."""
    if not (isinstance(bounds, (tuple, list)) and len(bounds) == 2):
        raise ValueError("bounds must be the (doc_start, query_end) pair from doc_bounds(doc_ids)")
    for t in bounds:
        if (t.dtype != torch.int32 or tuple(t.shape) != tuple(doc_ids.shape) or not t.is_contiguous()
                or t.device != doc_ids.device):
            raise ValueError("bounds must be the (doc_start, query_end) pair from doc_bounds(doc_ids): int32 (B, T) "
                             "contiguous tensors on doc_ids' device")
    return bounds[0], bounds[1]


def _run_forward(K, degree, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, out_like_v=True, bounds=None,
                 score_norms=None, rope=None):
    """Validates, computes the document bounds (unless given), rotates q/k by the rotary tables (if given) and
    launches the forward. Returns (o, dstart, qend, (q1, k1, q2, k2, v) as the kernels read them (rotated), sc,
    coef_f, b_f). o has v's strides (out_like_v) or is contiguous."""
    _validate(K, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, degree)
    q1, k1, v = _prep(q1), _prep(k1), _prep(v)
    if K in _TWO_PAIRS:
        q2, k2 = _prep(q2), _prep(k2)
    if rope is not None:
        cs, sn = rope
        q1, k1 = rope_rotate(q1, cs, sn), rope_rotate(k1, cs, sn)
        if K in _TWO_PAIRS:
            q2, k2 = rope_rotate(q2, cs, sn), rope_rotate(k2, cs, sn)
    if K not in _TWO_PAIRS:
        q2, k2 = q1, k1
    dstart, qend = doc_bounds(doc_ids) if bounds is None else _check_bounds(bounds, doc_ids)
    sc = row_scale.detach().float().contiguous()
    coef_f = coef.detach().float().contiguous() if K == _abi.LOWER_DEGREE_MIX else None
    b_f = b.detach().float().contiguous() if K == _abi.OFFSET_SQUARE else None
    o = torch.empty_like(v) if out_like_v else None
    if o is None or not _aligned_rows(o):
        o = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    if score_norms is not None:
        pairs = 2 if K in _TWO_PAIRS else 1
        if (score_norms.dtype != torch.float32 or tuple(score_norms.shape) != (pairs, 2, q1.shape[1])
                or not score_norms.is_contiguous() or score_norms.device != q1.device):
            raise ValueError(f"score_norms must be a contiguous float32 ({pairs}, 2, H) tensor on q1's device")
    prob = _problem(K, degree, q1, k1, q2, k2, v, dstart, qend, sc, coef_f, b_f, score_norms, rope)
    lib = _abi.load()
    with torch.cuda.device(q1.device):
        _abi.check(lib.tnpa_forward(ctypes.byref(prob), ctypes.byref(_desc(o)), _stream(q1.device)),
                   "poly_attention forward")
    return o, dstart, qend, (q1, k1, q2, k2, v), sc, coef_f, b_f


def _run_backward(K, degree, q1, k1, q2, k2, v, dstart, qend, sc, coef_f, b_f, do, grads_like_inputs=True,
                  rope=None):
    """Launches the backward on tensors prepared by _run_forward. Returns (dq1, dk1, dq2, dk2, dv, dpar), with
    dq2/dk2 None for one-pair kinds and dpar the (H, 4) fp32 head-parameter gradient or None. With the rotary tables
    (q/k then being the rotated tensors) dq/dk are with respect to the unrotated q/k."""
    H = q1.shape[1]
    do = _prep(do.to(v.dtype))
    alloc = _alloc_like if grads_like_inputs else (lambda x: torch.empty(x.shape, dtype=x.dtype, device=x.device))
    dq1, dk1, dv = alloc(q1), alloc(k1), alloc(v)
    two = K in _TWO_PAIRS
    dq2, dk2 = (alloc(q2), alloc(k2)) if two else (dq1, dk1)
    prob = _problem(K, degree, q1, k1, q2, k2, v, dstart, qend, sc, coef_f, b_f, rope=rope)
    lib = _abi.load()
    par = K in (_abi.OFFSET_SQUARE, _abi.LOWER_DEGREE_MIX)
    dpar = torch.empty(H, 4, dtype=torch.float32, device=q1.device) if par else None
    # the library's scratch (dcoef/db partials; the row-scaled dO where the plan streams it), caller-allocated
    nbytes = lib.tnpa_backward_workspace_bytes(ctypes.byref(prob))
    if nbytes < 0:
        _abi.check(_abi.ERR_INVALID, "poly_attention backward")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q1.device) if nbytes > 0 else None
    g = _abi.Grads(_desc(do), _desc(dq1), _desc(dk1), _desc(dq2), _desc(dk2), _desc(dv),
                   dpar.data_ptr() if par else None, ws.data_ptr() if ws is not None else None, nbytes)
    with torch.cuda.device(q1.device):
        _abi.check(lib.tnpa_backward(ctypes.byref(prob), ctypes.byref(g), _stream(q1.device)),
                   "poly_attention backward")
    if not two:
        dq2 = dk2 = None
    return dq1, dk1, dq2, dk2, dv, dpar


class PolyAttention(torch.autograd.Function):
    """ref: tnlm/kernels/poly_attn.py:255-309, with an appended `degree` argument for kind="power"."""

    @staticmethod
    def forward(ctx, kind, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, degree=None, bounds=None,
                score_norms=None, rope=None):
        shared = KINDS[kind] == _abi.SIGNED_PRODUCT and q2 is q1 and k2 is k1
        K, degree = _canonical(kind, q1, k1, q2, k2, degree)
        tabs = rope_tables_of(rope, q1) if rope is not None else None
        o, dstart, qend, (q1, k1, q2, k2, v), sc, coef_f, b_f = _run_forward(
            K, degree, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, bounds=bounds, score_norms=score_norms,
            rope=tabs)
        cs, sn = tabs if tabs is not None else (None, None)
        ctx.save_for_backward(q1, k1, q2, k2, v, dstart, qend, sc, coef_f, b_f, cs, sn)
        ctx.K, ctx.degree, ctx.shared = K, degree, shared
        ctx.has_coef, ctx.has_b = coef is not None, b is not None
        ctx.coef_dtype = coef.dtype if coef is not None else None
        ctx.b_dtype = b.dtype if b is not None else None
        return o

    @staticmethod
    def backward(ctx, do):
        q1, k1, q2, k2, v, dstart, qend, sc, coef_f, b_f, cs, sn = ctx.saved_tensors
        K = ctx.K
        dq1, dk1, dq2, dk2, dv, dpar = _run_backward(K, ctx.degree, q1, k1, q2, k2, v, dstart, qend, sc, coef_f,
                                                      b_f, do, rope=(cs, sn) if cs is not None else None)
        dcoef = dpar.to(ctx.coef_dtype) if (K == _abi.LOWER_DEGREE_MIX and ctx.has_coef) else None
        db = dpar[:, 0].to(ctx.b_dtype) if (K == _abi.OFFSET_SQUARE and ctx.has_b) else None
        return None, dq1, dk1, dq2, dk2, dv, None, None, dcoef, db, None, None, None, None


def _alloc_like(x: torch.Tensor) -> torch.Tensor:
    y = torch.empty_like(x)
    return y if _aligned_rows(y) else torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _problem(K, degree, q1, k1, q2, k2, v, dstart, qend, sc, coef_f, b_f, score_norms=None,
             rope=None) -> _abi.Problem:
    B, H, T, DK = q1.shape
    return _abi.Problem(B, H, T, DK, v.shape[-1], K, int(degree) if degree is not None else 0, _DTYPES[q1.dtype],
                        _desc(q1), _desc(k1), _desc(q2), _desc(k2), _desc(v),
                        dstart.data_ptr(), qend.data_ptr(), sc.data_ptr(),
                        coef_f.data_ptr() if coef_f is not None else None,
                        b_f.data_ptr() if b_f is not None else None,
                        score_norms.data_ptr() if score_norms is not None else None,
                        rope[0].data_ptr() if rope is not None else None,
                        rope[1].data_ptr() if rope is not None else None)


def score_norm_buffer(kind, q1, k1, q2=None, k2=None) -> torch.Tensor:
    """A zeroed fp32 (pairs, 2, H) buffer for the forward's score-bound factors: pairs = 2 for the two-pair kinds,
    1 for the others and for signed_product with shared pairs (which runs as degree 2)."""
    K, _ = _canonical(kind, q1, k1, q2, k2, 2)
    return torch.zeros(2 if K in _TWO_PAIRS else 1, 2, q1.shape[1], dtype=torch.float32, device=q1.device)


def score_bound(score_norms: torch.Tensor, d_key: int) -> dict:
    """{"S1": (H,), ["S2": (H,)]} = max|q| * max|k| / sqrt(dk) per head from the forward's score_norms: the reference's
    Cauchy-Schwarz bound on max |S| (ref: tnlm/model.py:33-38), without a separate pass over q and k."""
    names = ("S1", "S2")
    return {names[i]: score_norms[i, 0] * score_norms[i, 1] / d_key ** 0.5 for i in range(score_norms.shape[0])}


def poly_attention_hip(kind, q1, k1, q2, k2, v, doc_ids, row_scale, coef=None, b=None, *, degree=None,
                       bounds=None, score_norms=None, rope=None):
    """q*, k*: (B, H, T, dk); v: (B, H, T, dv); doc_ids: (B, T) contiguous ids, < 0 = padding;
    row_scale: (B, T) = n_visible^-p for real queries, 0 for padding. kind="power" takes degree=p and ignores
    q2/k2. bounds: optional doc_bounds(doc_ids), computed once per batch by a caller with many layers.
    score_norms: optional zeroed float32 (pairs, 2, H) tensor (score_norm_buffer) that the forward fills with the
    per-head max |q| and max |k| of each pair, for score_bound(). rope: optional (cos, sin) rotary tables
    (rope_tables layout, ref: tnlm/attention.py:41-45): q*/k* are then the unrotated projections, rotated here in one
    pass each exactly as the reference's apply_rope (ref: tnlm/model.py:70-71,81-82), and the backward returns their
    gradients with the rotation's gradient applied inside the library. Every gradient is reduced in a fixed order
    (deterministic).  ref: tnlm/kernels/poly_attn.py:312-315"""
    if torch.compiler.is_compiling():
        # under torch.compile the same kernels run behind registered custom ops (opaque to the compiler)
        from .ops import poly_attention_op
        return poly_attention_op(kind, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, degree=degree, bounds=bounds,
                                 score_norms=score_norms, rope=rope)
    return PolyAttention.apply(kind, q1, k1, q2, k2, v, doc_ids, row_scale, coef, b, degree, bounds, score_norms,
                               rope)
