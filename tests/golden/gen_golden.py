"""Writes the committed FP64 golden fixtures under tests/golden/ from the CPU oracle (oracle/poly_attention.py).

    python tests/golden/gen_golden.py

Inputs are drawn from seeded numpy generators and rounded to bfloat16-representable float32 values, so a bf16
or fp32 run on any machine reads identical input bits. Outputs (out, dq*, dk*, dv, dcoef, db) are FP64 from the
dense restatement of ref: tnlm/attention.py:54-77 and the analytic backward of
ref: tensor_network_research_brief.md:321-329. The reference ships no golden vectors of its own (its tests
recompute the dense FP64 form at test time), so these files are this build's own.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import (polynomial_attention, polynomial_attention_backward, round_to_bf16,  # noqa: E402
                    row_scale_mask, visible_mask)

HERE = Path(__file__).resolve().parent

# name: (kind, B, H, T, dk, dv, degree, row_power, seed, docs)
CASES = {
    # B2 H4 T128 D32, degree 2, scale 1/sqrt(D), row power 0.5, one document
    "config1_power2_b2h4t128d32": ("power", 2, 4, 128, 32, 32, 2, 0.5, 0, None),
    # degree 4 at a tiny size (pins the p=4 kernel path; q,k scaled by D^-1/4, 1% of rows x4 like config 4)
    "power4_b1h2t40d16": ("power", 1, 2, 40, 16, 16, 4, 0.5, 1, None),
    # the reference's three kinds with documents and padding (ref: tests/test_kernels.py:71-81 pattern)
    "signed_product_docs_b2h2t50": ("signed_product", 2, 2, 50, 16, 32, None, 0.5, 2, "docs"),
    "offset_square_docs_b2h2t50": ("offset_square", 2, 2, 50, 32, 16, None, 1.0, 3, "docs"),
    "lower_degree_mix_docs_b2h2t50": ("lower_degree_mix", 2, 2, 50, 16, 16, None, 0.5, 4, "docs"),
}


def _docs(B, T, kind):
    if kind is None:
        return np.zeros((B, T), dtype=np.int64)
    d = np.zeros((B, T), dtype=np.int64)
    d[0, 13:] = 1
    d[0, 31:] = 2
    d[0, 44:] = -1
    if B > 1:
        d[1, 1:] = 1
        d[1, 2:] = 2
        d[1, 40:] = 3
    return d


def make_case(name):
    kind, B, H, T, dk, dv, degree, row_power, seed, docs = CASES[name]
    rng = np.random.default_rng(seed)
    qk_scale = dk ** -0.25 if degree == 4 else 1.0
    q1, k1, q2, k2 = (round_to_bf16(rng.standard_normal((B, H, T, dk)) * qk_scale) for _ in range(4))
    if degree == 4:
        for x in (q1, k1):
            rows = rng.random((B, T)) < 0.05
            x *= np.where(rows, 4.0, 1.0)[:, None, :, None].astype(np.float32)
    v = round_to_bf16(rng.standard_normal((B, H, T, dv)))
    dout = round_to_bf16(rng.standard_normal((B, H, T, dv)))
    coef = round_to_bf16(np.tile(np.array([[0.3, -0.5, 0.7, 1.1]]), (H, 1)) + 0.1 * rng.standard_normal((H, 4)))
    b = round_to_bf16(np.linspace(-1, 1.5, H))
    doc = _docs(B, T, docs)
    C = row_scale_mask(visible_mask(doc), row_power)
    f64 = lambda x: x.astype(np.float64)  # noqa: E731
    args = (kind, f64(q1), f64(k1), f64(q2), f64(k2), f64(v), C)
    kw = dict(coef=f64(coef), b=f64(b), degree=degree)
    out = polynomial_attention(*args, **kw)
    grads = polynomial_attention_backward(*args, f64(dout), **kw)
    arrays = dict(q1=q1, k1=k1, q2=q2, k2=k2, v=v, dout=dout, coef=coef.astype(np.float32), b=b.astype(np.float32),
                  doc_ids=doc, out=out, **grads)
    meta = dict(kind=kind, B=B, H=H, T=T, dk=dk, dv=dv, degree=degree, row_power=row_power, seed=seed,
                docs=docs, inputs="bf16-representable float32", outputs="float64 dense oracle")
    return arrays, meta


def main():
    for name in CASES:
        arrays, meta = make_case(name)
        np.savez_compressed(HERE / f"{name}.npz", meta=json.dumps(meta), **arrays)
        print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
