"""Host-side integration pieces (no GPU): the registered custom ops and their shape functions, the model-side
row scales, the source identity, and that nothing falls back to the CPU."""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from oracle import row_scale_from_docs


def test_custom_ops_are_registered_with_the_reference_argument_order():
    import tensor_train_ing_amd  # noqa: F401  (registers tnpa::*)
    fwd = str(torch.ops.tnpa.poly_attention.default._schema)
    bwd = str(torch.ops.tnpa.poly_attention_backward.default._schema)
    bounds = str(torch.ops.tnpa.doc_bounds.default._schema)
    assert "Tensor q1, Tensor k1, Tensor? q2, Tensor? k2, Tensor v, Tensor doc_start, Tensor query_end, " \
           "Tensor row_scale, Tensor? coef, Tensor? b, bool want_norms" in fwd
    assert fwd.endswith("-> (Tensor, Tensor)")
    assert "Tensor doc_ids" in bounds and bounds.endswith("-> (Tensor, Tensor)")
    assert "Tensor dout" in bwd and bwd.endswith("-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")


@pytest.mark.parametrize("kind,two,par", [(0, True, False), (1, False, True), (2, True, True), (3, False, False)])
def test_fake_shapes(kind, two, par):
    """Shape functions (what torch.compile plans with) match what the kernels write."""
    import tensor_train_ing_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(2, 3, 40, 32, dtype=torch.bfloat16)
        v = torch.empty(2, 3, 40, 16, dtype=torch.bfloat16)
        doc = torch.zeros(2, 40, dtype=torch.long)
        rs = torch.ones(2, 40)
        ds, qe = torch.ops.tnpa.doc_bounds(doc)
        assert ds.shape == qe.shape == (2, 40) and ds.dtype == torch.int32
        o, nrm = torch.ops.tnpa.poly_attention(kind, 2, q, q, q if two else None, q if two else None, v, ds, qe, rs,
                                               None, None, True)
        assert tuple(nrm.shape) == ((2 if two else 1), 2, 3) and nrm.dtype == torch.float32
        assert o.shape == v.shape and o.dtype == v.dtype and o.is_contiguous()
        g = torch.ops.tnpa.poly_attention_backward(kind, 2, q, q, q if two else None, q if two else None, v, ds, qe,
                                                   rs, None, None, v)
        assert [tuple(x.shape) for x in g[:2]] == [tuple(q.shape)] * 2
        assert tuple(g[2].shape) == (tuple(q.shape) if two else (0,))
        assert tuple(g[4].shape) == tuple(v.shape)
        assert tuple(g[5].shape) == ((3, 4) if par else (0,))


def test_row_scales_match_the_visible_count():
    """(position + 1)^-p, 0 for padding, equals n_visible^-p of the dense mask for contiguous documents."""
    from tensor_train_ing_amd import model_glue
    from mini_lm import doc_positions
    doc = np.zeros((3, 50), dtype=np.int64)
    doc[0, 17:] = 1
    doc[1, 5:9] = 1
    doc[1, 9:] = 2
    doc[2, 44:] = -1
    d = torch.from_numpy(doc)
    got = model_glue.row_scales(d, doc_positions(d), (0.5, 1.0))
    for p in (0.5, 1.0):
        np.testing.assert_allclose(got[p].numpy(), row_scale_from_docs(doc, p), rtol=1e-6, atol=0)
    assert (got[0.5][2, 44:] == 0).all()


def test_source_identity_covers_the_kernels():
    """Every kernel source and the C ABI headers are in the identity, hashed like ref: tests/test_checkpoint.py:305."""
    from tensor_train_ing_amd import model_glue
    ident = model_glue.source_sha256()
    root = model_glue.PKG.parent
    for f in list((model_glue.PKG / "csrc").iterdir()) + sorted((root / "include").glob("*.h")):
        key = f.relative_to(root).as_posix()
        assert ident[key] == hashlib.sha256(f.read_bytes()).hexdigest(), key
    assert "tensor_train_ing_amd/poly_attn.py" in ident
    assert not any(k.endswith(".so") for k in ident)


def test_no_cpu_fallback():
    """CPU tensors are rejected by both entry points (the HIP kernels are the only implementation)."""
    from tensor_train_ing_amd import poly_attention_hip, poly_attention_op
    q = torch.randn(1, 1, 32, 16)
    doc = torch.zeros(1, 32, dtype=torch.long)
    rs = torch.ones(1, 32)
    for fn in (poly_attention_hip, poly_attention_op):
        with pytest.raises(ValueError, match="ROCm device"):
            fn("power", q, q, None, None, q, doc, rs, degree=2)


@pytest.mark.parametrize("T,L", [(128, 0), (128, 128), (100, 30), (97, 7), (64, 1), (50, 200)])
def test_bench_counts_exactly_the_visible_pairs(T, L):
    """bench.py's FLOP count uses the number of visible (query, key) pairs; brute force over the dense mask."""
    import bench
    from oracle import visible_mask
    doc = (np.arange(T) // L if L else np.zeros(T, dtype=np.int64))[None].astype(np.int64)
    assert bench.npairs(T, L) == int(visible_mask(doc).sum())


def test_bench_refuses_more_than_one_gpu(capsys):
    """This build measures one GPU: --gpus N > 1 exits with status 2 and says why (no torch or GPU touched)."""
    import bench
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_bench_cpu_baseline_runs_on_a_small_sample():
    """The CPU-baseline leg (the float32 torch restatement timed on host cores) on a tiny workload drawn as the GPU
    run draws it: positive fwd and fwd+bwd rates, the CPU model and the sample."""
    import bench
    q, k, v, do, doc, rs = bench.make_inputs(1, 2, 64, 16, 0.0, 0, "cpu")
    r = bench.cpu_baseline(q, k, v, do, rs, 2, 0.5)
    assert r["value"] > 0 and r["fwd_tflops"] > 0 and r["kind"] == "port" and r["cores"] >= 1
    assert "slices" in r["sample"] and r["cpu"]
