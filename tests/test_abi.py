"""CPU checks of the C ABI (include/tnpa.h) and the host-side operator logic; no GPU compute is launched.

Failure handling forced on the CPU: malformed shapes/strides/dtypes/head dims return an error code
and message before anything is enqueued; a differentiable row_scale is rejected; a missing library fails loudly.
"""
from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tnpa.h"
INTERNAL = ROOT / "tensor_train_ing_amd" / "csrc" / "tnpa_internal.h"


@pytest.fixture(scope="module")
def lib():
    from tensor_train_ing_amd import _abi
    return _abi.load()


def _declared_functions(header=HEADER):
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[\w\s\*]+?\b(tn(?:pa|ce)_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_reports_abi_version(lib):
    from tensor_train_ing_amd import _abi
    assert lib.tnpa_abi_version() == _abi.ABI_VERSION == 4


def test_every_declared_symbol_is_exported(lib):
    names = sorted({n for h in sorted((ROOT / "include").glob("*.h")) for n in _declared_functions(h)})
    assert len(names) >= 9 and "tnce_forward_chunk" in names, names
    for n in names:
        assert hasattr(lib, n), n
    from tensor_train_ing_amd import _abi
    assert set(_abi._SIGNATURES) == set(names)
    # the launch-level entry points the benchmark and the tests use stay out of the public header
    internal = _declared_functions(INTERNAL)
    assert internal and not set(internal) & set(names)
    for n in internal:
        assert hasattr(lib, n), n
    assert set(_abi._INTERNAL) == set(internal)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_struct_layout_matches_header(tmp_path):
    from tensor_train_ing_amd import _abi
    src = tmp_path / "layout.c"
    src.write_text(r'''
#include <stdio.h>
#include <stddef.h>
#include "tnpa.h"
int main(void) {
  printf("%zu %zu %zu\n", sizeof(tnpa_tensor_t), sizeof(tnpa_problem_t), sizeof(tnpa_grads_t));
  printf("%zu %zu %zu %zu\n", offsetof(tnpa_problem_t, q1), offsetof(tnpa_problem_t, v),
         offsetof(tnpa_problem_t, doc_start), offsetof(tnpa_problem_t, offset));
  printf("%zu %zu %zu %zu\n", offsetof(tnpa_grads_t, dv), offsetof(tnpa_grads_t, dpar),
         offsetof(tnpa_grads_t, workspace), offsetof(tnpa_grads_t, workspace_bytes));
  printf("%zu %zu %zu\n", offsetof(tnpa_problem_t, score_norms), offsetof(tnpa_problem_t, rope_cos),
         offsetof(tnpa_problem_t, rope_sin));
  return 0;
}''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                   check=True)
    got = [list(map(int, line.split())) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                     check=True).stdout.splitlines()]
    P, G = _abi.Problem, _abi.Grads
    assert got[0] == [ctypes.sizeof(_abi.Tensor), ctypes.sizeof(P), ctypes.sizeof(G)]
    assert got[1] == [P.q1.offset, P.v.offset, P.doc_start.offset, P.offset.offset]
    assert got[2] == [G.dv.offset, G.dpar.offset, G.workspace.offset, G.workspace_bytes.offset]
    assert got[3] == [P.score_norms.offset, P.rope_cos.offset, P.rope_sin.offset]


def _problem(**kw):
    from tensor_train_ing_amd import _abi
    t = _abi.Tensor(4096, 2 * 128 * 64, 128 * 64, 64)  # an aligned (never dereferenced) fake address
    p = _abi.Problem(2, 2, 128, 64, 64, _abi.POWER, 2, _abi.BF16, t, t, t, t, t, 4096, 4096, 4096, None, None)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("field,value,code,msg", [
    ("batch", 0, 1, "positive"),
    ("head_dim_k", 24, 1, "powers of 2"),
    ("head_dim_v", 8, 1, "powers of 2"),
    ("head_dim_k", 512, 2, "above 256"),
    ("head_dim_v", 512, 2, "above 256"),
    ("kind", 7, 1, "unknown kind"),
    ("degree", 0, 1, "degree"),
    ("dtype", 9, 1, "dtype"),
    ("rope_cos", 4096, 1, "both or neither"),
    ("doc_start", None, 1, "tnpa_doc_bounds"),
    ("row_scale", None, 1, "row_scale"),
])
def test_forward_rejects_bad_arguments_before_launch(lib, field, value, code, msg):
    from tensor_train_ing_amd import _abi
    p = _problem(**{field: value})
    out = _abi.Tensor(4096, 2 * 128 * 64, 128 * 64, 64)
    assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == code
    assert msg in lib.tnpa_last_error().decode()


def test_fp32_two_pairs_above_head_dim_128_unsupported(lib):
    """fp32 with two q/k pairs is built up to head dim 128 (its tiles would not fit LDS): TNPA_ERR_UNSUPPORTED
    (ValueError) before anything is launched; one pair, or 16-bit, at 256 is accepted."""
    from tensor_train_ing_amd import _abi
    for kind in (_abi.SIGNED_PRODUCT, _abi.LOWER_DEGREE_MIX):
        p = _problem(kind=kind, dtype=_abi.F32, head_dim_k=256, coef=4096)
        assert lib.tnpa_x_launches(ctypes.byref(p), 0) == -1
        out = _abi.Tensor(4096, 2 * 128 * 64, 128 * 64, 64)
        assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == _abi.ERR_UNSUPPORTED
        assert "up to 128" in lib.tnpa_last_error().decode()
    assert lib.tnpa_x_launches(ctypes.byref(_problem(kind=_abi.SIGNED_PRODUCT, head_dim_k=256)), 0) == 4
    assert lib.tnpa_x_launches(ctypes.byref(_problem(dtype=_abi.F32, head_dim_k=256, head_dim_v=256)), 0) == 4


def test_misaligned_views_and_missing_parameters_are_rejected(lib):
    from tensor_train_ing_amd import _abi
    out = _abi.Tensor(4096, 2 * 128 * 64, 128 * 64, 64)
    p = _problem(q1=_abi.Tensor(4098, 2 * 128 * 64, 128 * 64, 64))
    assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == _abi.ERR_INVALID
    assert "aligned" in lib.tnpa_last_error().decode()
    p = _problem(v=_abi.Tensor(4096, 2 * 128 * 64, 128 * 64, 60))
    assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == _abi.ERR_INVALID
    p = _problem(kind=_abi.LOWER_DEGREE_MIX)
    assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == _abi.ERR_INVALID
    assert "coef" in lib.tnpa_last_error().decode()
    p = _problem(rope_cos=4096 + 8, rope_sin=8192)
    assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == _abi.ERR_INVALID
    assert "aligned" in lib.tnpa_last_error().decode()
    assert lib.tnpa_rope(ctypes.byref(out), ctypes.byref(out), 2, 2, 128, 64, _abi.BF16, ctypes.c_void_p(4100),
                         ctypes.c_void_p(4096), 0, None) == _abi.ERR_INVALID
    assert "aligned" in lib.tnpa_last_error().decode()
    p = _problem(kind=_abi.OFFSET_SQUARE)
    assert lib.tnpa_forward(ctypes.byref(p), ctypes.byref(out), None) == _abi.ERR_INVALID
    assert "offset" in lib.tnpa_last_error().decode()
    assert lib.tnpa_forward(None, ctypes.byref(out), None) == _abi.ERR_INVALID
    # backward: the two head-scalar kinds need dpar and a workspace of the size the library asks for
    p = _problem(kind=_abi.OFFSET_SQUARE, offset=4096)
    t = _abi.Tensor(4096, 2 * 128 * 64, 128 * 64, 64)
    need = lib.tnpa_backward_workspace_bytes(ctypes.byref(p))
    assert need > 0
    g = _abi.Grads(t, t, t, t, t, t, None, 4096, need)
    assert lib.tnpa_backward(ctypes.byref(p), ctypes.byref(g), None) == _abi.ERR_INVALID
    assert "dpar" in lib.tnpa_last_error().decode()
    g = _abi.Grads(t, t, t, t, t, t, 4096, 4096, need - 1)
    assert lib.tnpa_backward(ctypes.byref(p), ctypes.byref(g), None) == _abi.ERR_INVALID
    assert "workspace" in lib.tnpa_last_error().decode()
    g = _abi.Grads(t, t, t, t, t, t, 4096, 4096 + 16, need)
    assert lib.tnpa_backward(ctypes.byref(p), ctypes.byref(g), None) == _abi.ERR_INVALID
    assert "aligned" in lib.tnpa_last_error().decode()
    g = _abi.Grads(t, t, t, t, t, t, None, None, 0)
    assert lib.tnpa_backward_workspace_bytes(None) == -1
    assert lib.tnpa_backward(None, ctypes.byref(g), None) == _abi.ERR_INVALID
    # internal launch-level entry: options and launch index are checked
    assert lib.tnpa_x_backward(ctypes.byref(_problem()), ctypes.byref(g), 3, -1, None) == _abi.ERR_INVALID
    assert lib.tnpa_x_backward(ctypes.byref(_problem()), ctypes.byref(g), 0, 7, None) == _abi.ERR_INVALID
    assert lib.tnpa_x_launches(ctypes.byref(_problem()), 8) == -1
    assert lib.tnpa_doc_bounds(None, 1, 128, 2, 128, None, None, None) == _abi.ERR_INVALID
    assert lib.tnpa_doc_bounds(ctypes.c_void_p(4096), 1, 64, 2, 128, ctypes.c_void_p(4096), ctypes.c_void_p(4096),
                               None) == _abi.ERR_INVALID


def test_backward_workspace_size(lib):
    """The workspace holds the fixed-order dcoef/db partials (one float4 per (b, h, key block)), where the plan
    streams it row_scale * dO in the problem dtype, and where dQ is computed from stored dS the dS tiles (one
    32x32 tile of the input dtype per sub-block on or below the diagonal); each part rounded up to 256 bytes."""
    from tensor_train_ing_amd import _abi
    r = lambda n: -(-n // 256) * 256  # noqa: E731
    assert lib.tnpa_backward_workspace_bytes(ctypes.byref(_problem())) == 0
    p = _problem(kind=_abi.OFFSET_SQUARE, offset=4096, seq_len=300)  # bf16, head dim 64: four-wave 128-key blocks
    assert lib.tnpa_backward_workspace_bytes(ctypes.byref(p)) == r(2 * 2 * 3 * 4 * 4)
    p = _problem(kind=_abi.OFFSET_SQUARE, offset=4096, seq_len=300, head_dim_k=128, head_dim_v=128)  # 128-key pairs
    tiles = 10 * 11 // 2  # 32-row sub-blocks of T=300: 10, tiles on or below the diagonal: 55
    assert lib.tnpa_backward_workspace_bytes(ctypes.byref(p)) == r(2 * 2 * 3 * 4 * 4) + r(2 * 2 * tiles * 1024 * 2)
    assert lib.tnpa_x_workspace_bytes(ctypes.byref(p), _abi.X_DS_OFF) == r(2 * 2 * 3 * 4 * 4)
    p = _problem(kind=_abi.OFFSET_SQUARE, offset=4096, seq_len=300, head_dim_k=128, head_dim_v=64)  # 256-key passes
    assert lib.tnpa_x_workspace_bytes(ctypes.byref(p), _abi.X_DS_OFF) == r(2 * 2 * 2 * 4 * 4)
    # lower_degree_mix (two pairs) streams the row-scaled dO: partials, then (B, H, T, dv) bf16
    p = _problem(kind=_abi.LOWER_DEGREE_MIX, coef=4096, seq_len=300)
    assert lib.tnpa_backward_workspace_bytes(ctypes.byref(p)) == r(2 * 2 * 3 * 4 * 4) + r(2 * 2 * 300 * 64 * 2)
    # at key head dim 128 the two-pair kinds add one set of dS tiles per pair (dS1, dS2)
    p = _problem(kind=_abi.LOWER_DEGREE_MIX, coef=4096, seq_len=300, head_dim_k=128, head_dim_v=128)
    assert lib.tnpa_backward_workspace_bytes(ctypes.byref(p)) == (r(2 * 2 * 3 * 4 * 4) + r(2 * 2 * 300 * 128 * 2)
                                                                   + 2 * r(2 * 2 * tiles * 1024 * 2))
    assert lib.tnpa_x_workspace_bytes(ctypes.byref(p), _abi.X_DS_OFF) == r(2 * 2 * 3 * 4 * 4) + r(2 * 2 * 300 * 128 * 2)
    p = _problem(kind=_abi.SIGNED_PRODUCT, seq_len=300, head_dim_k=128, head_dim_v=64)
    assert lib.tnpa_backward_workspace_bytes(ctypes.byref(p)) == r(2 * 2 * 300 * 64 * 2) + 2 * r(2 * 2 * tiles * 1024 * 2)
    # forcing the row-scaled dO on or off changes only that part
    p = _problem()
    assert lib.tnpa_x_workspace_bytes(ctypes.byref(p), _abi.X_PRESCALE_ON) == r(2 * 2 * 128 * 64 * 2)
    p = _problem(dtype=_abi.F32)
    assert lib.tnpa_x_workspace_bytes(ctypes.byref(p), _abi.X_PRESCALE_OFF) == 0
    assert lib.tnpa_x_workspace_bytes(ctypes.byref(p), 0) == r(2 * 2 * 128 * 64 * 4)


def _launches(lib, p, opts=0):
    return [lib.tnpa_x_launch_name(ctypes.byref(p), opts, i).decode() for i in range(lib.tnpa_x_launches(
        ctypes.byref(p), opts))]


def test_backward_plan(lib):
    """Which launches tnpa_backward makes: the row-scaled dO only where the key side cannot scale dO for free (fp32,
    two q/k pairs, or a head dim too small for the three-buffer tile split); separate dV and dK passes for 16-bit one
    q/k pair at a head dim above 64, except head dims 128 / 128, whose key side is the one wave-pair kernel; dQ from
    the dS tiles at key head dim 128 for 16-bit inputs, one pair or two (dQ recomputing S and dP otherwise, or with
    X_DS_OFF); the dpar reduction for the kinds with head parameters."""
    from tensor_train_ing_amd import _abi
    assert _launches(lib, _problem()) == ["kv", "q"]
    assert _launches(lib, _problem(head_dim_k=128, head_dim_v=128)) == ["kv", "qds"]
    assert _launches(lib, _problem(dtype=_abi.F16, head_dim_k=128, head_dim_v=128)) == ["kv", "qds"]
    assert _launches(lib, _problem(head_dim_k=128, head_dim_v=128), _abi.X_DS_OFF) == ["kv", "q"]
    assert _launches(lib, _problem(head_dim_k=64, head_dim_v=128)) == ["dv", "dk", "q"]
    assert _launches(lib, _problem(dtype=_abi.F32, head_dim_k=128, head_dim_v=128)) == ["scale", "kv", "q"]
    assert _launches(lib, _problem(dtype=_abi.F32)) == ["scale", "kv", "q"]
    assert _launches(lib, _problem(kind=_abi.SIGNED_PRODUCT)) == ["scale", "kv", "q"]
    assert _launches(lib, _problem(head_dim_v=16)) == ["scale", "kv", "q"]
    assert _launches(lib, _problem(head_dim_k=128, head_dim_v=32)) == ["scale", "dv", "dk", "qds"]
    assert _launches(lib, _problem(head_dim_v=32)) == ["kv", "q"]
    assert _launches(lib, _problem(kind=_abi.OFFSET_SQUARE, offset=4096)) == ["kv", "q", "dpar"]
    assert _launches(lib, _problem(kind=_abi.LOWER_DEGREE_MIX, coef=4096)) == ["scale", "kv", "q", "dpar"]
    assert _launches(lib, _problem(kind=_abi.SIGNED_PRODUCT, head_dim_k=128, head_dim_v=128)) == ["scale", "kv", "qds"]
    assert _launches(lib, _problem(kind=_abi.LOWER_DEGREE_MIX, coef=4096, head_dim_k=128, head_dim_v=64)) == [
        "scale", "kv", "qds", "dpar"]
    assert _launches(lib, _problem(kind=_abi.SIGNED_PRODUCT, head_dim_k=128, head_dim_v=128), _abi.X_DS_OFF) == [
        "scale", "kv", "q"]
    assert _launches(lib, _problem(kind=_abi.SIGNED_PRODUCT, dtype=_abi.F32, head_dim_k=128, head_dim_v=128)) == [
        "scale", "kv", "q"]
    assert _launches(lib, _problem(), _abi.X_PRESCALE_ON) == ["scale", "kv", "q"]
    assert _launches(lib, _problem(dtype=_abi.F32), _abi.X_PRESCALE_OFF) == ["kv", "q"]
    # rotary tables: the rotation's gradient goes into the dQ epilogues and, for one q/k pair with head dims >= 32,
    # the dK epilogue; otherwise dK gets it in one pass at the end
    for kw in ({}, dict(head_dim_k=128, head_dim_v=128), dict(dtype=_abi.F32, head_dim_k=32, head_dim_v=64)):
        assert _launches(lib, _problem(rope_cos=4096, rope_sin=8192, **kw)) == _launches(lib, _problem(**kw))
    for kw in (dict(head_dim_k=16, head_dim_v=16), dict(kind=_abi.LOWER_DEGREE_MIX, coef=4096),
               dict(kind=_abi.SIGNED_PRODUCT, head_dim_k=128, head_dim_v=128)):
        assert _launches(lib, _problem(rope_cos=4096, rope_sin=8192, **kw)) == _launches(lib, _problem(**kw)) + ["rope"]
    # head dims above 128: the row-scaled dO, then separate dV and dK passes of 128 keys, for every dtype and kind;
    # dQ from dS tiles for one 16-bit pair at key head dim 128 (the dK pass stores them), else recomputing S and dP;
    # the dK epilogue rotates except for fp32 (a pass after)
    for kw in (dict(head_dim_k=256, head_dim_v=256), dict(head_dim_k=256, head_dim_v=64),
               dict(dtype=_abi.F32, head_dim_k=16, head_dim_v=256), dict(dtype=_abi.F32, head_dim_k=128, head_dim_v=256),
               dict(kind=_abi.SIGNED_PRODUCT, head_dim_k=256, head_dim_v=128),
               dict(kind=_abi.SIGNED_PRODUCT, head_dim_k=128, head_dim_v=256)):
        assert _launches(lib, _problem(**kw)) == ["scale", "dv", "dk", "q"]
    assert _launches(lib, _problem(head_dim_k=128, head_dim_v=256)) == ["scale", "dv", "dk", "qds"]
    assert _launches(lib, _problem(kind=_abi.OFFSET_SQUARE, offset=4096, head_dim_k=256)) == [
        "scale", "dv", "dk", "q", "dpar"]
    assert _launches(lib, _problem(rope_cos=4096, rope_sin=8192, head_dim_k=256, head_dim_v=256)) == [
        "scale", "dv", "dk", "q"]
    assert _launches(lib, _problem(rope_cos=4096, rope_sin=8192, dtype=_abi.F32, head_dim_k=256)) == [
        "scale", "dv", "dk", "q", "rope"]
    assert lib.tnpa_x_launch_name(ctypes.byref(_problem()), 0, 5) == b""


def test_python_operator_errors_mirror_the_reference():
    from tensor_train_ing_amd import poly_attention_hip
    x = torch.zeros(1, 1, 8, 16)
    doc, rs = torch.zeros(1, 8, dtype=torch.long), torch.ones(1, 8)
    with pytest.raises(KeyError):
        poly_attention_hip("softmax", x, x, x, x, x, doc, rs)
    with pytest.raises(AssertionError, match="powers of 2"):
        y = torch.zeros(1, 1, 8, 24)
        poly_attention_hip("signed_product", y, y, y, y, y, doc, rs)
    with pytest.raises(ValueError, match="ROCm device"):
        poly_attention_hip("signed_product", x, x, x, x, x, doc, rs)


def test_differentiable_row_scale_is_rejected():
    from tensor_train_ing_amd.poly_attn import _abi as abi_mod, _validate
    x = torch.zeros(1, 1, 8, 16)
    rs = torch.ones(1, 8, requires_grad=True)
    with pytest.raises(ValueError):
        _validate(abi_mod.POWER, x, x, None, None, x, torch.zeros(1, 8, dtype=torch.long), rs, None, None, 2)


def test_missing_library_fails_loudly(tmp_path):
    from tensor_train_ing_amd import _abi
    with pytest.raises(RuntimeError, match="missing"):
        _abi.load(tmp_path / "libtnpa.so")


def test_backend_resolution_mirrors_reference():
    from tensor_train_ing_amd import ATTENTION_BACKENDS, resolve_attention_backend
    assert ATTENTION_BACKENDS == ("reference", "triton", "hip", "auto")
    assert resolve_attention_backend("auto", "cpu") == "reference"
    assert resolve_attention_backend("auto", "cpu", "softmax") == "softmax"
    expect = "hip" if torch.version.hip is not None else "triton"
    assert resolve_attention_backend("auto", "cuda:0") == expect
    assert resolve_attention_backend("hip", "cuda:0", "softmax") == "flex"
    assert resolve_attention_backend("reference", "cuda:0") == "reference"
    with pytest.raises(AssertionError):
        resolve_attention_backend("cuda", "cpu")


def test_product_never_imports_the_oracle():
    for f in (ROOT / "tensor_train_ing_amd").rglob("*.py"):
        src = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", src, flags=re.M), f


def test_rope_tables_are_checked():
    """rope=(cos, sin): the reference's (B, 1, T, dk/2) layout or (B, T, dk/2), fp32 after conversion, no gradient."""
    from tensor_train_ing_amd.poly_attn import rope_tables_of
    q = torch.zeros(2, 3, 10, 16)
    cs, sn = rope_tables_of((torch.ones(2, 1, 10, 8), torch.zeros(2, 10, 8, dtype=torch.float64)), q)
    assert cs.shape == sn.shape == (2, 10, 8) and cs.dtype == sn.dtype == torch.float32 and sn.is_contiguous()
    with pytest.raises(ValueError, match="expected"):
        rope_tables_of((torch.ones(2, 10, 16), torch.ones(2, 10, 8)), q)
    with pytest.raises(ValueError, match="pair"):
        rope_tables_of(torch.ones(2, 10, 8), q)
    with pytest.raises(ValueError, match="differentiable"):
        rope_tables_of((torch.ones(2, 10, 8, requires_grad=True), torch.ones(2, 10, 8)), q)
