"""GPU parity of the chunked linear + cross-entropy (library GEMMs + HIP epilogues) against the CPU oracle.

Mirrors the reference's acceptance checks (ref: tests/test_scaling_loss.py:26-90): float64 and float32 sums and
gradients for many chunkings and non-contiguous inputs, arbitrary upstream scales, all-ignored targets, float64
gradcheck, a tied embedding / output weight; plus the bf16 autocast path against the oracle with the reference's
rounding points, and a pilot-1B-sized chunk against a float32 torch reference of the same chunk.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _native():
    from tensor_train_ing_amd import _abi
    _abi.load()
    assert torch.cuda.is_available()


def _fixture(dtype=torch.float64, noncontiguous=False, all_ignored=False):
    g = torch.Generator().manual_seed(1407)
    if noncontiguous:
        x = torch.randn(7, 22, generator=g, dtype=dtype).T[::2]
        w = torch.randn(7, 26, generator=g, dtype=dtype).T[::2]
        t = torch.randint(0, 13, (22,), generator=g)[::2]
    else:
        x = torch.randn(11, 7, generator=g, dtype=dtype)
        w = torch.randn(13, 7, generator=g, dtype=dtype)
        t = torch.randint(0, 13, (11,), generator=g)
    t = t.clone()
    t[::3] = -100
    if all_ignored:
        t.fill_(-100)
    return x, w, t


def _hip(x, w, t, chunk, scale=1.0):
    from tensor_train_ing_amd import linear_cross_entropy_sum
    dev = torch.device("cuda:0")
    xd = x.to(dev).requires_grad_()
    wd = w.to(dev).requires_grad_()
    total = linear_cross_entropy_sum(xd, wd, t.to(dev), chunk=chunk)
    gx, gw = torch.autograd.grad(total, (xd, wd), grad_outputs=torch.tensor(scale, dtype=total.dtype, device=dev))
    return total.detach().cpu(), gx.cpu(), gw.cpu()


@pytest.mark.parametrize("chunk", [1, 2, 4, 11, 30])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("noncontiguous", [False, True])
def test_sum_and_gradients_match_oracle(chunk, dtype, noncontiguous):
    from oracle import linear_cross_entropy
    x, w, t = _fixture(dtype, noncontiguous)
    total, gx, gw = _hip(x, w, t, chunk)
    ref = linear_cross_entropy(x.double().numpy(), w.double().numpy(), t.numpy(), chunk=chunk)
    tol = dict(rtol=2e-5, atol=2e-6) if dtype == torch.float32 else dict(rtol=5e-12, atol=5e-12)
    np.testing.assert_allclose(total.double().numpy(), ref[0], **tol)
    np.testing.assert_allclose(gx.double().numpy(), ref[1], **tol)
    np.testing.assert_allclose(gw.double().numpy(), ref[2], **tol)


@pytest.mark.parametrize("chunk", [1, 3, 30])
@pytest.mark.parametrize("scale", [-2.75, 0.0, 0.125, 3.5])
@pytest.mark.parametrize("all_ignored", [False, True])
def test_upstream_scale_and_ignored_targets(chunk, scale, all_ignored):
    from oracle import linear_cross_entropy
    x, w, t = _fixture(all_ignored=all_ignored)
    total, gx, gw = _hip(x, w, t, chunk, scale)
    ref = linear_cross_entropy(x.numpy(), w.numpy(), t.numpy(), chunk=chunk, g=scale)
    np.testing.assert_allclose(total.numpy(), ref[0], rtol=5e-12, atol=5e-12)
    np.testing.assert_allclose(gx.numpy(), ref[1], rtol=5e-12, atol=5e-12)
    np.testing.assert_allclose(gw.numpy(), ref[2], rtol=5e-12, atol=5e-12)
    if all_ignored:
        assert total.item() == 0.0 and not gx.any() and not gw.any()


@pytest.mark.parametrize("chunk", [1, 2, 8])
def test_fp64_gradcheck(chunk):
    from tensor_train_ing_amd import linear_cross_entropy_sum
    g = torch.Generator().manual_seed(23)
    dev = torch.device("cuda:0")
    x = torch.randn(4, 3, dtype=torch.float64, generator=g).to(dev).requires_grad_()
    w = torch.randn(5, 3, dtype=torch.float64, generator=g).to(dev).requires_grad_()
    t = torch.tensor([0, -100, 4, 2], device=dev)
    assert torch.autograd.gradcheck(lambda a, b: linear_cross_entropy_sum(a, b, t, chunk=chunk), (x, w), eps=1e-6,
                                    atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("chunk", [1, 4, 30])
def test_tied_embedding_and_output_weight_accumulate_both_paths(chunk):
    import torch.nn.functional as F
    from tensor_train_ing_amd import linear_cross_entropy_sum
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(67)
    weight = torch.randn(9, 5, dtype=torch.float64, generator=g).to(dev).requires_grad_()
    transform = torch.randn(5, 5, dtype=torch.float64, generator=g).to(dev).requires_grad_()
    rw, rt = weight.detach().cpu().requires_grad_(), transform.detach().cpu().requires_grad_()
    ids = torch.tensor([1, 2, 1, 7, 4, 2])
    t = torch.tensor([2, 1, -100, 4, 2, 8])
    x = F.embedding(ids.to(dev), weight) @ transform
    total = linear_cross_entropy_sum(x, weight, t.to(dev), chunk=chunk)
    gw, gt = torch.autograd.grad(total * 1.75, (weight, transform))
    # the CPU float64 dense reference (torch on the host): same model, dense logits
    xr = F.embedding(ids, rw) @ rt
    ref = F.cross_entropy(xr @ rw.T, t, reduction="sum")
    rgw, rgt = torch.autograd.grad(ref * 1.75, (rw, rt))
    torch.testing.assert_close(total.cpu(), ref.detach(), rtol=5e-12, atol=5e-12)
    torch.testing.assert_close(gw.cpu(), rgw, rtol=5e-12, atol=5e-12)
    torch.testing.assert_close(gt.cpu(), rgt, rtol=5e-12, atol=5e-12)


@pytest.mark.parametrize("chunk", [64, 1000])
def test_bf16_autocast_matches_oracle_rounding(chunk):
    """x, w in float32 under bf16 autocast: matmuls in bf16 (logits and p rounded to bf16 as in the reference),
    log-sum-exp in float32; against the oracle with the same rounding points, at bf16 tolerance."""
    from oracle import linear_cross_entropy, round_to_bf16
    from tensor_train_ing_amd import linear_cross_entropy_sum
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    N, d, V = 1000, 128, 3000
    x = torch.randn(N, d, generator=g) * 0.5
    w = torch.randn(V, d, generator=g) * 0.1
    t = torch.randint(0, V, (N,), generator=g)
    t[::7] = -100
    xd, wd = x.to(dev).requires_grad_(), w.to(dev).requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        total = linear_cross_entropy_sum(xd, wd, t.to(dev), chunk=chunk)
    assert total.dtype == torch.float32
    gx, gw = torch.autograd.grad(total, (xd, wd))
    ref = linear_cross_entropy(x.numpy(), w.numpy(), t.numpy(), chunk=chunk, round_to=round_to_bf16)
    assert abs(total.item() - ref[0]) <= 1e-3 * abs(ref[0])
    for got, r in ((gx, ref[1]), (gw, ref[2])):
        err = np.abs(got.double().cpu().numpy() - r).max() / np.abs(r).max()
        assert err <= 2e-2, err


def test_pilot_1b_chunk_against_torch_float32():
    """One pilot-1B-sized chunk (4096 rows, d_model 2048, padded vocab 50304; ref: configs/pilot_1b.yaml:21,27) in
    bf16: the HIP epilogues against the same chunk done with float32 torch ops on the bf16 logits; loss and
    gradients finite."""
    from tensor_train_ing_amd import linear_cross_entropy_sum
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(11)
    N, d, V = 4096, 2048, 50304
    x = (torch.randn(N, d, generator=g) * 0.02).to(dev, torch.bfloat16).requires_grad_()
    w = (torch.randn(V, d, generator=g) * 0.02).to(dev, torch.bfloat16).requires_grad_()
    t = torch.randint(0, 50257, (N,), generator=g).to(dev)
    t[::9] = -100
    total = linear_cross_entropy_sum(x, w, t, chunk=4096)
    gx, gw = torch.autograd.grad(total, (x, w))
    with torch.no_grad():
        lg = (x @ w.t()).float()
        lse = torch.logsumexp(lg, -1)
        valid = t != -100
        ref = ((lse - lg.gather(1, t.clamp_min(0)[:, None])[:, 0]) * valid).sum()
        p = torch.exp(lg - lse[:, None])
        p[torch.arange(N, device=dev), t.clamp_min(0)] -= 1
        p = (p * valid[:, None]).to(torch.bfloat16)
        rgx = p @ w
        rgw = (p.t() @ x).float()
    assert torch.isfinite(total) and torch.isfinite(gx).all() and torch.isfinite(gw).all()
    assert abs(total.item() - ref.item()) <= 1e-4 * abs(ref.item())
    assert ((gx.float() - rgx.float()).abs().max() / rgx.float().abs().max()).item() <= 1e-2
    assert ((gw.float() - rgw).abs().max() / rgw.abs().max()).item() <= 1e-2


@pytest.mark.parametrize("dtype,n", [(torch.bfloat16, 1 << 20), (torch.float16, 999), (torch.float32, 12345),
                                     (torch.float64, 77)])
def test_dw_accumulate_matches_reference_upcast_add(dtype, n):
    """tnce_accumulate(acc, part) against the reference's `dw += part.to(acc)`: bit-identical (one addition per
    element in the accumulation type), twice in a row, with a length that is not a multiple of the 16-byte step."""
    import ctypes
    from tensor_train_ing_amd import _abi
    from tensor_train_ing_amd.fused_ce import _DTYPES
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    acc_t = torch.float64 if dtype == torch.float64 else torch.float32
    acc = (torch.randn(n, generator=g, dtype=torch.float64) * 3).to(dev, acc_t)
    ref = acc.clone()
    lib = _abi.load()
    for _ in range(2):
        part = (torch.randn(n, generator=g, dtype=torch.float64) * 7).to(dev, dtype)
        ref += part.to(acc_t)
        _abi.check(lib.tnce_accumulate(ctypes.c_void_p(acc.data_ptr()), ctypes.c_void_p(part.data_ptr()),
                                       _DTYPES[dtype], n, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                   "accumulate")
    torch.cuda.synchronize()
    assert torch.equal(acc, ref)
