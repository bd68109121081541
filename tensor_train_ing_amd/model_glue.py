"""Model-side hooks for the "hip" attention backend.

The reference model prepares its fast path in `make_ctx` (ref: tnlm/model.py:205-227): with a fast backend it builds
no T x T mask, only the per-query row scales n_visible^-p (n_visible = position in document + 1, 0 for padding;
ref: tnlm/model.py:217-221), and `Attention.forward` hands them to the operator (ref: tnlm/model.py:86-91). These
functions do the same for "hip", so the reference's model code needs only its backend test widened to accept
"hip". `source_sha256` extends the checkpoint's source identity
(ref: tnlm/checkpoint.py:54) with this package's kernel sources.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import torch

from .config import poly_attention_for

PKG = Path(__file__).resolve().parent


def row_scales(doc_ids: torch.Tensor, positions: torch.Tensor, powers) -> dict:
    """{p: (B, T) float32}: (position + 1)^-p for real tokens (doc id >= 0), 0 for padding. `positions` is the
    model's position within document (ref: tnlm/attention.py:12-19). This equals n_visible^-p for contiguous
    documents, which the kernels assume.  ref: tnlm/model.py:217-221"""
    n = (positions + 1).float()
    valid = doc_ids >= 0
    return {p: torch.where(valid, n.pow(-p), torch.zeros_like(n)) for p in powers}


def fast_context(doc_ids: torch.Tensor, positions: torch.Tensor, powers, backend: str = "hip") -> dict:
    """The fast-path part of the model context: doc ids, backend name, row scales (no visibility mask) and the
    per-token document bounds, computed here once for every layer of the forward (one prepass launch per batch)."""
    from .poly_attn import doc_bounds
    return {"doc_ids": doc_ids, "backend": backend, "row_scale": row_scales(doc_ids, positions, powers),
            "bounds": doc_bounds(doc_ids)}


def attention(kind: str, q1, k1, q2, k2, v, ctx: dict, row_power: float, coef=None, b=None, degree=None,
              rope=None):
    """Attention.forward's fast-path call (ref: tnlm/model.py:86-91) for ctx["backend"] == "hip": (B, H, T, dv).
    rope: ctx["rope"] when q/k are the unrotated projections (ref: tnlm/model.py:69-71,81-82 then run inside the
    operator), None when the caller has rotated them."""
    fn = poly_attention_for(ctx["backend"])
    kw = {"degree": degree} if kind == "power" else {}
    if rope is not None:
        kw["rope"] = rope
    return fn(kind, q1, k1, q2, k2, v, ctx["doc_ids"], ctx["row_scale"][row_power], coef=coef, b=b,
              bounds=ctx.get("bounds"), **kw)


def source_files() -> list[Path]:
    """Every source file the operators are built from or run: the Python package, the HIP kernels and the C ABI
    headers (the built library is excluded)."""
    files = (sorted(PKG.rglob("*.py")) + sorted((PKG / "csrc").glob("*.hip")) + sorted((PKG / "csrc").glob("*.hpp"))
             + sorted((PKG / "csrc").glob("*.h")))
    files += sorted((PKG.parent / "include").glob("*.h"))
    return [f for f in files if "_build" not in f.parts and "__pycache__" not in f.parts]


def source_sha256() -> dict:
    """{"tensor_train_ing_amd/<path>": sha256 hex} for source_files(), in the form of the reference checkpoint's
    `source_sha256` entries (ref: tnlm/checkpoint.py:54), to be merged into them."""
    root = PKG.parent
    return {f.relative_to(root).as_posix(): hashlib.sha256(f.read_bytes()).hexdigest() for f in source_files()}
