"""The `attention_backend` selection key, extended with "hip".

Mirrors ref: tnlm/config.py:53-56,93 (allowed values) and the resolution in ref: tnlm/model.py:211-216 and
ref: tnlm/cli.py:67-71: "auto" picks the fast path on a GPU and the dense reference elsewhere. On a ROCm build of
PyTorch the fast path is "hip" (this package); on CUDA it stays "triton". The softmax control maps any fast path
to "flex" and the reference path to "softmax", as the reference does.
"""
from __future__ import annotations

import torch

ATTENTION_BACKENDS = ("reference", "triton", "hip", "auto")


def validate_attention_backend(backend: str) -> str:
    """Raises AssertionError for an unknown value, like ModelConfig.__post_init__ (ref: tnlm/config.py:93)."""
    assert backend in ATTENTION_BACKENDS, backend
    return backend


def resolve_attention_backend(backend: str, device: torch.device | str, attention: str = "signed_product") -> str:
    """Concrete backend for a model on `device`."""
    validate_attention_backend(backend)
    device = torch.device(device)
    if backend == "auto":
        if device.type == "cuda":
            backend = "hip" if torch.version.hip is not None else "triton"
        else:
            backend = "reference"
    if attention == "softmax":
        return "flex" if backend in ("triton", "hip") else "softmax"
    return backend


def poly_attention_for(backend: str):
    """The polynomial attention callable a resolved backend dispatches to (one lookup per model build, no
    per-call dispatch). Only "hip" is served by this package."""
    if backend != "hip":
        raise ValueError(f"backend {backend!r} is not provided by tensor_train_ing_amd")
    from .poly_attn import poly_attention_hip
    return poly_attention_hip
