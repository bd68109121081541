"""MI355X-native causal polynomial attention (gfx950 HIP kernels behind a C ABI), a drop-in for the Triton
operator of tnlm (ref: tnlm/kernels/poly_attn.py)."""
from .config import ATTENTION_BACKENDS, poly_attention_for, resolve_attention_backend  # noqa: F401
from .poly_attn import KINDS, PolyAttention, doc_bounds, poly_attention_hip, score_bound, score_norm_buffer  # noqa: F401
from .ops import poly_attention_op  # noqa: F401  (registers the tnpa:: custom ops)
from . import model_glue  # noqa: F401
from .fused_ce import LinearCrossEntropy, linear_cross_entropy_sum  # noqa: F401

__all__ = ["KINDS", "PolyAttention", "poly_attention_hip", "poly_attention_op", "doc_bounds", "score_bound",
           "score_norm_buffer",
           "ATTENTION_BACKENDS", "resolve_attention_backend", "poly_attention_for", "model_glue",
           "LinearCrossEntropy", "linear_cross_entropy_sum"]
