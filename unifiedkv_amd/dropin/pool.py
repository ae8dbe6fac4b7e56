"""Flat-import shim of the MI355X paged pool for BP-KV's unchanged modules.

core/scheduler.py:9 and core/offload.py:8 do ``from pool import PagedKVPool`` with
core/ on sys.path; with this directory ahead of core/ that resolves here.
"""
import sys
from pathlib import Path

_ROOT = str(Path(__file__).resolve().parents[2])
if _ROOT not in sys.path:
    sys.path.append(_ROOT)

from unifiedkv_amd.pool import PagedKVPool, pack_block_table  # noqa: E402,F401

__all__ = ["PagedKVPool", "pack_block_table"]
