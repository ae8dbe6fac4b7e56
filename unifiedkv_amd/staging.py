"""Offload / prefetch page movement between the paged pool and pinned host memory (row a8).

The reference moves one (layer, page) at a time: a transposed device copy, a
fresh pinned host tensor per K and per V block, and a small async copy on a
high-priority transfer stream (core/offload.py:547-599 offload, 620-691
prefetch, 163-179 per-page transposes); the page ids change across a round
trip, the contents do not (finalize: core/offload.py:362-449).

Here a round trip moves whole pages of every layer in large chunks:

* offload: the side stream waits for the compute stream (the reference's
  transfer stream does not, core/offload.py:578), gathers a chunk of pages of
  all layers into a device staging buffer with the gfx950 page-copy kernel, and
  DMAs the contiguous chunk into pinned host memory (hipMemcpyAsync D2H);
* prefetch: DMA host -> staging, then the page-copy kernel scatters the chunk to
  the newly allocated page ids.

Both return a ``torch.cuda.Event``; ``wait`` makes the current stream depend
on it. The side stream runs at the default priority.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Sequence

import torch

from . import page_ops


@dataclass
class HostPages:
    """Pinned host copy of n pages of every layer, in chunks of [layers, c, block, heads, dim]."""
    n_pages: int
    k_chunks: List[torch.Tensor] = field(default_factory=list)
    v_chunks: List[torch.Tensor] = field(default_factory=list)
    event: torch.cuda.Event = None

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.k_chunks + self.v_chunks)


class PageStager:
    """Chunked pool <-> pinned-host page mover on its own stream."""

    def __init__(self, pool, chunk_pages: int = 512):
        self.pool = pool
        self.dev = pool.device
        self.chunk = int(chunk_pages)
        self.stream = torch.cuda.Stream(device=self.dev)  # default priority
        shape = (pool.num_layers, self.chunk, pool.B, pool.num_kv_heads, pool.head_dim)
        self.stage_k = torch.empty(shape, dtype=pool.dtype, device=self.dev)
        self.stage_v = torch.empty_like(self.stage_k)
        self._iota = torch.arange(self.chunk, dtype=torch.int32, device=self.dev)

    def _ids(self, page_ids) -> torch.Tensor:
        """int32 device ids: [n] shared by all layers, or [layers, n] per layer."""
        if torch.is_tensor(page_ids):
            return page_ids.to(device=self.dev, dtype=torch.int32).contiguous()
        host = torch.tensor(page_ids if not isinstance(page_ids, list) or not page_ids or
                            not isinstance(page_ids[0], (list, tuple)) else [list(r) for r in page_ids],
                            dtype=torch.int32)
        return host.pin_memory().to(self.dev, non_blocking=True)

    def offload(self, page_ids, host: HostPages = None) -> HostPages:
        """Copy pages (all layers, K and V) to pinned host memory; asynchronous.

        page_ids: [n] ids shared by every layer, or [layers, n] per-layer ids (the pages a
        per-layer selection evicted). Pass a HostPages from an earlier call of the same size to
        reuse its pinned buffers. The pages must not be rewritten before ``host.event``."""
        n = int(page_ids.shape[-1]) if torch.is_tensor(page_ids) else (
            len(page_ids[0]) if page_ids and isinstance(page_ids[0], (list, tuple)) else len(page_ids))
        pool = self.pool
        if host is None or host.n_pages != n:
            host = HostPages(n_pages=n)
            for c0 in range(0, n, self.chunk):
                c = min(self.chunk, n - c0)
                shape = (pool.num_layers, c, pool.B, pool.num_kv_heads, pool.head_dim)
                host.k_chunks.append(torch.empty(shape, dtype=pool.dtype, pin_memory=True))
                host.v_chunks.append(torch.empty(shape, dtype=pool.dtype, pin_memory=True))
        cur = torch.cuda.current_stream(self.dev)
        self.stream.wait_stream(cur)
        with torch.cuda.stream(self.stream):
            ids = self._ids(page_ids)
            # A caller's int32 device tensor comes back as itself: mark its use on this stream, so
            # that the caching allocator does not hand its memory to the compute stream while the
            # copies below still read it.
            ids.record_stream(self.stream)
            for i, c0 in enumerate(range(0, n, self.chunk)):
                c = min(self.chunk, n - c0)
                page_ops.page_copy([pool.k_cache, pool.v_cache], [self.stage_k, self.stage_v], ids[..., c0:c0 + c],
                                   self._iota[:c])
                host.k_chunks[i].copy_(self.stage_k[:, :c], non_blocking=True)
                host.v_chunks[i].copy_(self.stage_v[:, :c], non_blocking=True)
            host.event = torch.cuda.Event()
            host.event.record(self.stream)
        return host

    def prefetch(self, host: HostPages, new_page_ids) -> torch.cuda.Event:
        """Write a HostPages back into pages `new_page_ids` ([n] shared or [layers, n]); asynchronous.

        Wait on the returned event (``wait``) before reading the pages."""
        ids_probe = self._ids(new_page_ids)
        if int(ids_probe.shape[-1]) != host.n_pages:
            raise ValueError("prefetch: one new page id per offloaded page")
        pool = self.pool
        cur = torch.cuda.current_stream(self.dev)
        self.stream.wait_stream(cur)
        with torch.cuda.stream(self.stream):
            if host.event is not None:
                self.stream.wait_event(host.event)
            ids = ids_probe
            ids.record_stream(self.stream)  # made on the compute stream, read on this one
            for i, c0 in enumerate(range(0, host.n_pages, self.chunk)):
                c = min(self.chunk, host.n_pages - c0)
                self.stage_k[:, :c].copy_(host.k_chunks[i], non_blocking=True)
                self.stage_v[:, :c].copy_(host.v_chunks[i], non_blocking=True)
                page_ops.page_copy([self.stage_k, self.stage_v], [pool.k_cache, pool.v_cache], self._iota[:c],
                                   ids[..., c0:c0 + c])
            ev = torch.cuda.Event()
            ev.record(self.stream)
        return ev

    def wait(self, event: torch.cuda.Event) -> None:
        torch.cuda.current_stream(self.dev).wait_event(event)
