"""Flat-import shim of the MI355X Page16 decode for BP-KV's unchanged scheduler.

core/scheduler.py:14 does ``from page16_native import HAS_TRITON, page16_decode_attention``
with core/ on sys.path. Putting this directory ahead of core/ on sys.path makes
that import resolve to libukv.so's kernels (see unifiedkv_amd.page16_native).
"""
import sys
from pathlib import Path

_ROOT = str(Path(__file__).resolve().parents[2])
if _ROOT not in sys.path:
    sys.path.append(_ROOT)

from unifiedkv_amd.page16_native import HAS_TRITON, HAS_UKV, page16_decode_attention  # noqa: E402,F401

__all__ = ["HAS_TRITON", "HAS_UKV", "page16_decode_attention"]
