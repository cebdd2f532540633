"""Block prefetch prediction and the KV page warm-up launch.

Interface of the reference's prefetch.py: ``BlockPrefetcher`` (:21-58, the
frequency heuristic the KV memory manager uses to predict next-step pages),
the module-level ``get_prefetcher`` / ``reset_prefetcher`` /
``get_prefetch_stream`` (:61-87) and ``launch_prefetch_pages`` (:183-261),
whose Triton kernel (:111-170) reads the K and V rows of the given pages with
an L2 cache hint and copies K into a scratch buffer. Here the warm-up is
libiak's ``iak_prefetch_pages``: it reads the pages' K and V rows with plain
(cached) loads so that they stay in the L2 / Infinity Cache for the next
step's decode, and folds them into per-wave checksums (so the loads are not
removed) instead of copying K. It is correctness-neutral, as in the
reference: nothing reads the checksum but tests.
"""
from __future__ import annotations

from collections import Counter, deque
from typing import List, Optional

import torch

from . import _native as N

__all__ = ["BlockPrefetcher", "get_prefetcher", "reset_prefetcher", "get_prefetch_stream", "launch_prefetch_pages"]


class BlockPrefetcher:
    """Predicts the blocks of the next decode step: an id is predicted when it
    appears in at least ``min_frequency`` of the last ``history_size`` recorded
    steps plus the current one."""

    def __init__(self, history_size: int = 4, min_frequency: int = 3) -> None:
        self.history_size = history_size
        self.min_frequency = min_frequency
        self._history: deque = deque(maxlen=history_size)

    def predict_next(self, current_selected: List[int]) -> List[int]:
        window = list(self._history) + [frozenset(current_selected)]
        if len(window) < self.min_frequency:
            return []
        counter: Counter = Counter()
        for s in window:
            counter.update(s)
        return sorted(bid for bid, cnt in counter.items() if cnt >= self.min_frequency)

    def record(self, selected: List[int]) -> None:
        self._history.append(frozenset(selected))

    def reset(self) -> None:
        self._history.clear()


_prefetcher: Optional[BlockPrefetcher] = None
_prefetch_stream = None


def get_prefetcher() -> BlockPrefetcher:
    global _prefetcher
    if _prefetcher is None:
        _prefetcher = BlockPrefetcher()
    return _prefetcher


def reset_prefetcher() -> None:
    if _prefetcher is not None:
        _prefetcher.reset()


def get_prefetch_stream():
    """A second stream for warm-ups (default priority), created on first use."""
    global _prefetch_stream
    if _prefetch_stream is None and torch.cuda.is_available():
        _prefetch_stream = torch.cuda.Stream()
    return _prefetch_stream


def launch_prefetch_pages(k: torch.Tensor, v: torch.Tensor, page_ids: torch.Tensor, stream=None,
                          page_size: int = 128) -> Optional[torch.Tensor]:
    """Warm the K and V rows of ``page_ids`` (pages of ``page_size`` tokens of
    k, v [batch, heads, kv_len, d_head]) into the caches, every (batch, head).
    Returns the per-wave checksums (int32 [batch * heads * len(page_ids) * 4],
    laid out as iak_prefetch_pages documents) of the data read, or None when
    there is nothing to do; a no-op on host tensors, as in the reference."""
    if not (k.is_cuda and v.is_cuda and page_ids.is_cuda) or page_ids.numel() == 0:
        return None
    if k.shape != v.shape or k.dim() != 4:
        raise ValueError(f"k and v must be [batch, heads, kv_len, d_head] of one shape, got {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    if k.dtype != v.dtype or k.element_size() != 2:
        raise ValueError("k and v must be 16-bit tensors of one dtype")
    B, H, T, D = k.shape
    ids = page_ids.to(torch.int32).contiguous()
    sink = torch.empty(B * H * ids.numel() * 4, dtype=torch.int32, device=k.device)
    a = N.PrefetchArgs()
    a.batch, a.heads, a.kv_len, a.head_dim = B, H, T, D
    a.page_size, a.num_ids = page_size, ids.numel()
    a.page_ids = ids.data_ptr()
    a.k, a.v = k.data_ptr(), v.data_ptr()
    a.k_stride_b, a.k_stride_h, a.k_stride_t = k.stride(0), k.stride(1), k.stride(2)
    a.v_stride_b, a.v_stride_h, a.v_stride_t = v.stride(0), v.stride(1), v.stride(2)
    a.checksum = sink.data_ptr()
    if k.stride(3) != 1 or v.stride(3) != 1:
        raise ValueError("k and v need a unit last stride")
    cur = torch.cuda.current_stream(k.device)
    s = stream if stream is not None else cur
    if s != cur:
        # the ids (and k, v) are written on the current stream; the allocator
        # must not hand the ids or the checksums to other work before s is done
        s.wait_stream(cur)
        ids.record_stream(s)
        sink.record_stream(s)
    N.prefetch_pages(a, s.cuda_stream)
    return sink
