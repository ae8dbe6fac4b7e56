"""TEST INFRASTRUCTURE ONLY - CPU restatement of BP-KV's per-sequence offload / prefetch bookkeeping.

Only tests/ may import this module. It follows core/offload.py on host lists (no data): which
logical blocks move, the per-layer page maps (-1 = on the host), the states, the FIFO page
allocation and frees, and the CPU byte accounting.

* ``offload_blocks``     core/offload.py:547-599 (selection from the first layer's map, budget,
                         CPU-bytes check, pending map with -1 at the selected blocks)
* ``finalize_offload``   core/offload.py:362-397 (publish the pending map, free the old pages sorted)
* ``prefetch_blocks``    core/offload.py:620-691 (blocks with a host copy and no page, one FIFO
                         allocation shared by every layer, assigned in ascending block order)
* ``finalize_prefetch``  core/offload.py:399-449 (publish, release the CPU bytes)
* ``state_of``           core/offload.py:146-156
"""
from __future__ import annotations

from typing import Dict, List


def state_of(map0: List[int]) -> str:
    resident = sum(1 for b in map0 if b >= 0)
    return "ON_CPU" if resident <= 0 else ("ON_GPU" if resident >= len(map0) else "MIXED")


class OffloadOracle:
    def __init__(self, allocator, num_layers: int, block_size: int, heads: int, dim: int, cpu_budget: int):
        self.alloc = allocator
        self.L, self.B, self.H, self.D = num_layers, block_size, heads, dim
        self.cpu_budget = cpu_budget
        self.cpu_used = 0
        self.seqs: Dict[int, dict] = {}

    def add(self, seq, maps: List[List[int]], seq_len: int):
        self.seqs[seq] = dict(maps=[list(m) for m in maps], seq_len=seq_len, host=set(), pending=None,
                              pending_idx=None, state=state_of(maps[0]))

    def _bytes(self, s, idx):
        per = sum(2 * self.H * max(0, min(s["seq_len"], i * self.B + self.B) - i * self.B) * self.D * 2 for i in idx)
        return per * self.L

    def offload_blocks(self, seq, idx) -> bool:
        s = self.seqs[seq]
        if s["state"] not in ("ON_GPU", "MIXED"):
            return False
        m0 = s["maps"][0]
        sel = sorted({i for i in idx if 0 <= i < len(m0) and m0[i] >= 0})
        if not sel:
            return False
        need = self._bytes(s, sel)
        if self.cpu_used + need > self.cpu_budget:
            return False
        pend = [list(m) for m in s["maps"]]
        for m in pend:
            for i in sel:
                m[i] = -1
        s["pending"], s["pending_idx"], s["state"] = pend, sel, "OFFLOAD_INFLIGHT"
        self.cpu_used += need
        return True

    def finalize_offload(self, seq):
        s = self.seqs[seq]
        if s["state"] != "OFFLOAD_INFLIGHT":
            return
        freed = {o for old, new in zip(s["maps"], s["pending"]) for o, n in zip(old, new) if o >= 0 and n < 0}
        s["host"] |= set(s["pending_idx"])
        s["maps"], s["pending"], s["pending_idx"] = s["pending"], None, None
        s["state"] = state_of(s["maps"][0])
        if freed:
            self.alloc.free_blocks_by_ids(sorted(freed))

    def prefetch_blocks(self, seq, idx) -> bool:
        """True: nothing to do; False: issued (or failed)."""
        s = self.seqs[seq]
        if s["state"] not in ("ON_CPU", "MIXED"):
            return True
        m0 = s["maps"][0]
        sel = sorted({i for i in idx if 0 <= i < len(m0) and m0[i] < 0 and i in s["host"]})
        if not sel:
            return True
        ids = self.alloc.allocate_blocks(len(sel))
        if len(ids) != len(sel):
            if ids:
                self.alloc.free_blocks_by_ids(ids)
            return False
        pend = [list(m) for m in s["maps"]]
        for m in pend:
            for i, b in zip(sel, ids):
                m[i] = b
        s["pending"], s["pending_idx"], s["state"] = pend, sel, "PREFETCH_INFLIGHT"
        s["host"] -= set(sel)
        return False

    def finalize_prefetch(self, seq):
        s = self.seqs[seq]
        if s["state"] != "PREFETCH_INFLIGHT":
            return
        self.cpu_used = max(0, self.cpu_used - self._bytes(s, s["pending_idx"]))
        s["maps"], s["pending"], s["pending_idx"] = s["pending"], None, None
        s["state"] = state_of(s["maps"][0])
