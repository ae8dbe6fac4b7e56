"""The C ABI and the drop-in Python surface, checked without a GPU.

* libukv.so loads and exports every function include/ukv.h declares, and the
  ctypes table in unifiedkv_amd/_ext.py binds exactly those names.
* page16_native.page16_decode_attention raises the reference's RuntimeError
  strings, in the reference's order (core/page16_native.py:101-124).
"""
import re
import subprocess
from pathlib import Path

import pytest
import torch

from unifiedkv_amd import _ext, page16_native

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(ukv_\w+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"ukv_version", "ukv_status_string", "ukv_page16_workspace_bytes", "ukv_page16_decode"} <= names


def test_library_exports_every_declared_symbol():
    lib = _ext.load()
    names = declared_functions()
    for n in names:
        assert hasattr(lib, n), n
    assert names == set(_ext.SIGNATURES), "ctypes table and header disagree"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_ext.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (ukv_\w+)", out))
    assert names <= exported


def test_status_strings_and_version():
    lib = _ext.load()
    assert lib.ukv_version() >= 0x000100
    assert _ext.status_string(_ext.UKV_OK) == "ok"
    assert _ext.status_string(_ext.UKV_ERR_GQA) == "gqa"
    assert _ext.status_string(-999) == "unknown"


def test_has_triton_flag_reflects_library():
    assert page16_native.HAS_TRITON is True


def _t(*shape, dtype=torch.float16):
    return torch.zeros(shape, dtype=dtype)


def _call(q, k, v, bt, lens, n_rep=4):
    return page16_native.page16_decode_attention(q, k, v, bt, lens, softmax_scale=0.1, n_rep=n_rep)


GOOD = dict(q=(2, 8, 64), k=(10, 16, 2, 64), v=(10, 16, 2, 64), bt=(2, 3), lens=(2,))


def _args(**over):
    shapes = dict(GOOD)
    shapes.update(over)
    q = _t(*shapes["q"])
    k = _t(*shapes["k"])
    v = _t(*shapes["v"])
    bt = torch.zeros(shapes["bt"], dtype=torch.int32)
    lens = torch.ones(shapes["lens"], dtype=torch.int32)
    return q, k, v, bt, lens


@pytest.mark.parametrize("over,msg", [
    (dict(q=(2, 8)), "page16_native_shape_unsupported:q_dim_2"),
    (dict(q=(2, 8, 64, 1)), "page16_native_shape_unsupported:q_dim_4"),
    (dict(k=(10, 16, 2)), "page16_native_shape_unsupported:cache_rank"),
    (dict(v=(10, 16, 2, 64, 1)), "page16_native_shape_unsupported:cache_rank"),
    (dict(k=(10, 32, 2, 64)), "page16_native_shape_unsupported:block_size_32"),
    (dict(bt=(2,)), "page16_native_shape_unsupported:block_table_rank"),
    (dict(q=(0, 8, 64), bt=(0, 3), lens=(0,)), "page16_native_shape_unsupported:empty"),
    (dict(v=(10, 8, 2, 64)), "page16_native_shape_unsupported:v_cache"),
    (dict(v=(10, 16, 4, 64)), "page16_native_shape_unsupported:v_cache"),
    (dict(v=(10, 16, 2, 32)), "page16_native_shape_unsupported:v_cache"),
    (dict(k=(10, 16, 3, 64), v=(10, 16, 3, 64)), "page16_native_shape_unsupported:gqa"),
    (dict(bt=(3, 3)), "page16_native_shape_unsupported:block_table_batch"),
    (dict(lens=(3,)), "page16_native_shape_unsupported:seqlens"),
    (dict(q=(2, 8, 320), k=(10, 16, 2, 320), v=(10, 16, 2, 320)), "page16_native_shape_unsupported:head_dim_320"),
    (dict(k=(10, 16, 2, 32)), "page16_native_shape_unsupported:k_cache"),
    # the order of the reference's checks: q rank before cache rank before block size
    (dict(q=(2, 8), k=(10, 16, 2)), "page16_native_shape_unsupported:q_dim_2"),
    (dict(k=(10, 32, 2), bt=(2,)), "page16_native_shape_unsupported:cache_rank"),
    (dict(k=(10, 32, 2, 64), bt=(2,)), "page16_native_shape_unsupported:block_size_32"),
])
def test_reference_error_strings(over, msg):
    with pytest.raises(RuntimeError) as ei:
        _call(*_args(**over))
    assert str(ei.value) == msg


def test_dtype_mismatch_and_cpu_tensors_are_rejected():
    q, k, v, bt, lens = _args()
    with pytest.raises(RuntimeError, match="page16_native_shape_unsupported:dtype"):
        _call(q.float(), k, v, bt, lens)
    with pytest.raises(RuntimeError, match="page16_native_shape_unsupported:dtype"):
        _call(q, k.to(torch.bfloat16), v, bt, lens)
    with pytest.raises(RuntimeError, match="page16_native_unavailable:device"):
        _call(q, k, v, bt, lens)


def test_unavailable_library_message(monkeypatch):
    monkeypatch.setattr(page16_native, "HAS_TRITON", False)
    with pytest.raises(RuntimeError) as ei:
        _call(*_args())
    assert str(ei.value) == "page16_native_unavailable:triton_not_available"


def test_engine_error_classification_substrings():
    # core/engine.py:2862-2869 classifies by substring; every shape error must carry "shape".
    for over, _ in [(dict(q=(2, 8)), 0), (dict(bt=(3, 3)), 0)]:
        with pytest.raises(RuntimeError) as ei:
            _call(*_args(**over))
        assert "shape" in str(ei.value).lower()


def test_flat_dropin_import_for_unchanged_scheduler():
    """core/scheduler.py:14 imports `page16_native` flat; the dropin dir must satisfy it."""
    import importlib
    import sys

    dropin = str(ROOT / "unifiedkv_amd" / "dropin")
    sys.path.insert(0, dropin)
    try:
        sys.modules.pop("page16_native", None)
        mod = importlib.import_module("page16_native")
        from page16_native import HAS_TRITON as HAS_PAGE16_NATIVE, page16_decode_attention  # noqa: F401

        assert HAS_PAGE16_NATIVE is True
        assert mod.page16_decode_attention is page16_native.page16_decode_attention
    finally:
        sys.path.remove(dropin)
        sys.modules.pop("page16_native", None)
