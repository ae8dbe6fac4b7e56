"""Seeded synthetic workloads for the Page16 hot path (the BASELINE configs).

Each decode case is a dict with 16-bit pools and int32 tables:

    q            [B, Hq, D]            uint16 bit patterns (numpy) / fp16|bf16 (torch)
    k_cache      [N, 16, Hkv, D]       one layer of the pool layout [L, N, 16, Hkv, D]
    v_cache      [N, 16, Hkv, D]       (core/pool.py:67-71)
    block_table  int32 [B, max_blocks] zero padded (core/pool.py:174-189)
    seqlens      int32 [B]             tokens attended, including the current one
    scale        1/sqrt(D);  n_rep = Hq // Hkv;  dtype "fp16" | "bf16"

``numpy_*`` builders are platform-stable (PCG64) and serve the CPU oracle and the
committed fixtures. ``torch_*`` builders create the same shapes directly on the
GPU (torch's Philox generator) for the full-size benchmark configs.
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np

PAGE = 16
DTYPE_CODES = {"fp16": 0, "bf16": 1}


def _round_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "fp16":
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def tables_from_pages(page_lists, max_blocks: Optional[int] = None) -> np.ndarray:
    """Zero-padded int32 [B, max_blocks] (the layout of PagedKVPool.build_block_table)."""
    mb = max(len(p) for p in page_lists) if max_blocks is None else max_blocks
    bt = np.zeros((len(page_lists), mb), dtype=np.int32)
    for i, ids in enumerate(page_lists):
        bt[i, : len(ids)] = ids
    return bt


# --------------------------------------------------------------------------
# Length / table layouts of the BASELINE decode configs
# --------------------------------------------------------------------------
def layout_tiny(rng: np.random.Generator):
    """Config 1: B=4, L ~ U{256..2048}, pool 1024 pages, one draw without replacement."""
    B, N = 4, 1024
    lens = rng.integers(256, 2048, size=B, endpoint=True).astype(np.int32)
    pages = [(int(L) + PAGE - 1) // PAGE for L in lens]
    draw = rng.permutation(N)[: sum(pages)]
    lists, o = [], 0
    for n in pages:
        lists.append(draw[o : o + n])
        o += n
    return dict(B=B, Hq=32, Hkv=8, D=128, dtype="fp16", N=N, seqlens=lens, block_table=tables_from_pages(lists))


def layout_longctx(rng: np.random.Generator, B: int = 16, ctx: int = 32768, spare: int = 8192):
    """Config 2: B=16 at ctx=32768 (2048 pages each), pool 40960 bf16 pages, permuted ids."""
    per = ctx // PAGE
    N = B * per + spare
    perm = rng.permutation(N)[: B * per].astype(np.int32)
    return dict(B=B, Hq=32, Hkv=8, D=128, dtype="bf16", N=N, seqlens=np.full(B, ctx, dtype=np.int32),
                block_table=perm.reshape(B, per))


def layout_ragged(rng: np.random.Generator, B: int = 64, median: int = 2048, sigma: float = 1.0):
    """Config 3: lognormal lengths (median 2048, sigma 1.0) clipped to [128, 32768],
    rounded up to a multiple of 16; pool = ceil(1.1 * pages) with interleaved ownership."""
    raw = rng.lognormal(mean=math.log(median), sigma=sigma, size=B)
    lens = np.clip(raw, 128, 32768)
    lens = (np.ceil(lens / PAGE) * PAGE).astype(np.int32)
    pages = [int(L) // PAGE for L in lens]
    total = sum(pages)
    N = int(math.ceil(1.1 * total))
    draw = rng.permutation(N)[:total].astype(np.int32)
    lists, o = [], 0
    for n in pages:
        lists.append(draw[o : o + n])
        o += n
    return dict(B=B, Hq=32, Hkv=8, D=128, dtype="bf16", N=N, seqlens=lens, block_table=tables_from_pages(lists),
                sigma=sigma)


LAYOUTS = {"tiny": layout_tiny, "longctx": layout_longctx, "ragged": layout_ragged}


# --------------------------------------------------------------------------
# Value generation
# --------------------------------------------------------------------------
def numpy_decode_case(layout: Dict, seed: int) -> Dict:
    """Fill a layout with N(0,1) q/K/V rounded to the dtype (uint16 bit patterns)."""
    rng = np.random.default_rng(seed + 1)
    B, Hq, Hkv, D, N, dt = (layout[k] for k in ("B", "Hq", "Hkv", "D", "N", "dtype"))
    case = dict(layout)
    case["q"] = _round_bits(rng.standard_normal((B, Hq, D), dtype=np.float32), dt)
    case["k_cache"] = _round_bits(rng.standard_normal((N, PAGE, Hkv, D), dtype=np.float32), dt)
    case["v_cache"] = _round_bits(rng.standard_normal((N, PAGE, Hkv, D), dtype=np.float32), dt)
    case["scale"] = 1.0 / math.sqrt(D)
    case["n_rep"] = Hq // Hkv
    case["seed"] = seed
    return case


def numpy_case(name: str, seed: int) -> Dict:
    rng = np.random.default_rng(seed)
    return numpy_decode_case(LAYOUTS[name](rng), seed)


def torch_decode_case(layout: Dict, seed: int, device="cuda"):
    """Same layout with q/K/V drawn on the device (torch generator), as torch tensors."""
    import torch

    tdt = torch.bfloat16 if layout["dtype"] == "bf16" else torch.float16
    gen = torch.Generator(device=device)
    gen.manual_seed(seed + 1)
    B, Hq, Hkv, D, N = (layout[k] for k in ("B", "Hq", "Hkv", "D", "N"))
    case = dict(layout)
    case["q"] = torch.randn((B, Hq, D), generator=gen, device=device, dtype=torch.float32).to(tdt)
    k = torch.empty((N, PAGE, Hkv, D), device=device, dtype=tdt)
    v = torch.empty_like(k)
    # fill in slabs to bound the fp32 temporary
    step = max(1, (1 << 27) // (PAGE * Hkv * D))
    for lo in range(0, N, step):
        hi = min(N, lo + step)
        k[lo:hi] = torch.randn((hi - lo, PAGE, Hkv, D), generator=gen, device=device, dtype=torch.float32).to(tdt)
        v[lo:hi] = torch.randn((hi - lo, PAGE, Hkv, D), generator=gen, device=device, dtype=torch.float32).to(tdt)
    case["k_cache"], case["v_cache"] = k, v
    case["block_table"] = torch.from_numpy(np.ascontiguousarray(layout["block_table"])).to(device)
    case["seqlens"] = torch.from_numpy(np.ascontiguousarray(layout["seqlens"])).to(device)
    case["scale"] = 1.0 / math.sqrt(D)
    case["n_rep"] = Hq // Hkv
    case["seed"] = seed
    return case


def to_torch(case: Dict, device="cuda") -> Dict:
    """Upload a numpy case (uint16 bit patterns) as fp16/bf16 device tensors."""
    import torch

    tdt = torch.bfloat16 if case["dtype"] == "bf16" else torch.float16
    out = dict(case)
    for key in ("q", "k_cache", "v_cache"):
        out[key] = torch.from_numpy(np.ascontiguousarray(case[key]).view(np.int16)).to(device).view(tdt)
    out["block_table"] = torch.from_numpy(np.ascontiguousarray(case["block_table"], dtype=np.int32)).to(device)
    out["seqlens"] = torch.from_numpy(np.ascontiguousarray(case["seqlens"], dtype=np.int32)).to(device)
    return out


def decode_bytes(seqlens, B: int, Hq: int, Hkv: int, D: int, max_blocks: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one decode call: K and V of every attended token once
    (independent of n_rep), plus q, out, the block table and the lengths."""
    kv = int(np.sum(np.asarray(seqlens, dtype=np.int64))) * Hkv * D * 2 * elem
    return kv + 2 * B * Hq * D * elem + 4 * B * max_blocks + 4 * B
