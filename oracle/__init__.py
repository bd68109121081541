"""CPU oracle for causal polynomial attention (test infrastructure only).

Nothing in the product package imports this directory. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may use it, and only as the checker or as the timed CPU baseline.
"""
from .poly_attention import (  # noqa: F401
    KINDS,
    block_bounds_reference,
    doc_bounds,
    doc_positions,
    polynomial_attention,
    polynomial_attention_backward,
    polynomial_attention_loops,
    polynomial_attention_recurrent,
    round_to_bf16,
    row_scale_from_docs,
    row_scale_mask,
    scores,
    visible_mask,
)
from .torch_dense import causal_row_scale, dense_attention  # noqa: F401
from .fused_ce import linear_cross_entropy  # noqa: F401
