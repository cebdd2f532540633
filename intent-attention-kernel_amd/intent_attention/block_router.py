"""Block router: semantic layout -> selected pages, precisions, prefetch hints.

Interface of the reference's block_router.py:18-421 (``BlockDecision``,
``RoutedBlock``, ``RouterConfig``, ``compute_block_scores``, ``BlockRouter``,
``routing_to_kernel_metadata``); outputs are identical to the reference's,
list order included.

Page arithmetic is done on intervals instead of token by token: a block
[start, end) covers pages start//ps .. (end-1)//ps, so the first-seen page
order, the first-occurrence precision and the prefetch candidates follow from
O(blocks + pages) work, which matters for 64k-131k token layouts.

Two reference behaviours are kept on purpose:
* ``routing_to_kernel_metadata`` computes prefetch hints with a default
  ``RouterConfig()``, not the router's own config (block_router.py:398).
* ``prefetch_page_ids`` returns the distinct best SCORES of the candidate
  pages, highest first: the reference's dedupe loop unpacks its
  ``(page_id, score)`` items as ``score, pid`` (:329-335), so it keeps and
  returns the score field.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import auto
from typing import Dict, Iterator, List, Optional, Tuple

import torch

from ._enum import StrEnum
from .block_metadata import BlockLayout, BlockPolicy, SemanticBlock
from .intent_quant import _BYTES_PER_VALUE, IntentQuantizer, KVPrecision


class BlockDecision(StrEnum):
    SELECT = auto()
    SKIP = auto()
    PREFETCH = auto()
    QUANTIZE = auto()
    PIN_HIGH_PRECISION = auto()


@dataclass
class RoutedBlock:
    name: str
    start: int
    end: int
    policy: BlockPolicy
    score: Optional[float]
    decision: BlockDecision
    precision: KVPrecision
    reason: str


@dataclass
class RouterConfig:
    top_k_blocks: int = 8
    score_threshold: float = 0.35
    recent_window_tokens: int = 2048
    memory_pressure: float = 0.5
    prefetch_top_k: int = 4
    preserve_system_prompt: bool = True
    preserve_recent: bool = True


_SELECTING = (BlockDecision.SELECT, BlockDecision.PIN_HIGH_PRECISION, BlockDecision.QUANTIZE)


def compute_block_scores(query_vector: torch.Tensor,
                         block_representations: Dict[str, torch.Tensor]) -> Dict[str, float]:
    """Cosine similarity of the query with each block representation, clipped to [0, 1]."""
    q = query_vector.flatten().float()
    q = q / (q.norm(p=2) + 1e-10)
    out: Dict[str, float] = {}
    for name, rep in block_representations.items():
        r = rep.flatten().float()
        r = r / (r.norm(p=2) + 1e-10)
        out[name] = min(1.0, max(0.0, float(torch.dot(q, r).item())))
    return out


def _pages(start: int, end: int, ps: int) -> range:
    """The distinct ``t // ps`` of tokens ``start <= t < end`` in increasing
    order (the reference walks the tokens, block_router.py:291-295): empty
    when ``end <= start``."""
    if end <= start:
        return range(0)
    return range(start // ps, (end - 1) // ps + 1)


class BlockRouter:
    """Policy layer: semantic blocks -> routing decisions -> kernel metadata."""

    def __init__(self, config: RouterConfig, quantizer: Optional[IntentQuantizer] = None) -> None:
        self.config = config
        self.quantizer = quantizer or IntentQuantizer(
            memory_pressure=config.memory_pressure, preserve_recent=config.preserve_recent,
            preserve_global=config.preserve_system_prompt)

    def _routed(self, b: SemanticBlock, decision: BlockDecision, precision: KVPrecision,
                reason: str) -> RoutedBlock:
        return RoutedBlock(b.name, b.start, b.end, b.policy, b.score, decision, precision, reason)

    def route_layout(self, layout: BlockLayout, total_tokens: int,
                     query_vector: Optional[torch.Tensor] = None,
                     block_representations: Optional[Dict[str, torch.Tensor]] = None) -> List[RoutedBlock]:
        """One RoutedBlock per block: pinned/recent blocks in layout order, then the
        top-k ATTEND blocks by score (stable), the rest of ATTEND, then SKIP blocks."""
        layout.validate(total_tokens)
        cfg = self.config
        scores = (compute_block_scores(query_vector, block_representations)
                  if query_vector is not None and block_representations is not None else {})
        pinned = [b for b in layout.blocks
                  if b.policy in (BlockPolicy.ALWAYS, BlockPolicy.GLOBAL, BlockPolicy.RECENT)]
        attend = []
        for b in layout.blocks:
            if b.policy == BlockPolicy.ATTEND:
                if b.score is None and b.name in scores:
                    b = SemanticBlock(b.name, b.start, b.end, b.policy, scores[b.name])
                attend.append(b)
        skip = [b for b in layout.blocks if b.policy not in
                (BlockPolicy.ALWAYS, BlockPolicy.GLOBAL, BlockPolicy.RECENT, BlockPolicy.ATTEND)]
        ranked = sorted((b for b in attend if b.score is not None), key=lambda b: b.score or 0.0,
                        reverse=True)   # stable: ties keep layout order
        prec = lambda b: self.quantizer.assign_block_precision(b).precision  # noqa: E731

        out: List[RoutedBlock] = []
        for b in pinned:
            if b.policy == BlockPolicy.RECENT:
                out.append(self._routed(b, BlockDecision.SELECT, prec(b), "recent context, always selected"))
            else:
                out.append(self._routed(b, BlockDecision.PIN_HIGH_PRECISION, prec(b),
                                        f"{b.policy.value} block, always selected"))
        for b in ranked[:cfg.top_k_blocks]:
            p = prec(b)
            if p == KVPrecision.SKIP:
                out.append(self._routed(b, BlockDecision.SKIP, p,
                                        "low-score attend, skipped under memory pressure"))
            else:
                out.append(self._routed(b, BlockDecision.SELECT if p == KVPrecision.FP16 else BlockDecision.QUANTIZE,
                                        p, f"attend score={b.score:.3f} >= threshold={cfg.score_threshold}"))
        for b in ranked[cfg.top_k_blocks:]:
            low = cfg.memory_pressure > 0.5 and b.score is not None and b.score < cfg.score_threshold
            out.append(self._routed(b, BlockDecision.SKIP, prec(b),
                                    "below top-k" + (", low score with pressure" if low else "")))
        for b in skip:
            p = prec(b)
            if b.score is not None and b.score >= cfg.score_threshold:
                out.append(self._routed(b, BlockDecision.SELECT, p,
                                        "SKIP block with unexpectedly high score, selected"))
            else:
                out.append(self._routed(b, BlockDecision.SKIP, KVPrecision.SKIP, "SKIP block, not selected"))
        return out

    def selected_blocks(self, routed_blocks: List[RoutedBlock]) -> List[RoutedBlock]:
        return [b for b in routed_blocks if b.decision in _SELECTING]

    def skipped_blocks(self, routed_blocks: List[RoutedBlock]) -> List[RoutedBlock]:
        return [b for b in routed_blocks if b.decision == BlockDecision.SKIP]

    def selected_token_indices(self, routed_blocks: List[RoutedBlock]) -> List[int]:
        return [t for b in self.selected_blocks(routed_blocks) for t in range(b.start, b.end)]

    def _first_seen_pages(self, routed_blocks: List[RoutedBlock], page_size: int) -> Iterator[Tuple[int, RoutedBlock]]:
        seen = set()
        for b in self.selected_blocks(routed_blocks):
            for pid in _pages(b.start, b.end, page_size):
                if pid not in seen:
                    seen.add(pid)
                    yield pid, b

    def selected_page_ids(self, routed_blocks: List[RoutedBlock], page_size: int) -> List[int]:
        return [pid for pid, _ in self._first_seen_pages(routed_blocks, page_size)]

    def prefetch_page_ids(self, routed_blocks: List[RoutedBlock], page_size: int) -> List[float]:
        thr = self.config.score_threshold
        best: Dict[int, float] = {}

        def offer(pid: int, score: float) -> None:
            if pid not in best or score > best[pid]:
                best[pid] = score

        for b in routed_blocks:
            if b.decision == BlockDecision.SKIP and b.score is not None and b.score >= thr:
                for pid in _pages(b.start, b.end, page_size):
                    offer(pid, b.score)
        for b in self.selected_blocks(routed_blocks):
            for pid in range(max(0, b.start // page_size - 1), (b.end + page_size - 1) // page_size + 1):
                offer(pid, 1.0)
        distinct = sorted(set(best.values()), reverse=True)
        return distinct[: self.config.prefetch_top_k]

    def routing_summary(self, routed_blocks: List[RoutedBlock]) -> Dict:
        """Counts and fp16 vs quantised byte estimates (head_dim 64, K+V), as the reference."""
        sel = self.selected_blocks(routed_blocks)
        total = sum(b.end - b.start for b in routed_blocks)
        sel_tok = sum(b.end - b.start for b in sel)
        dist: Dict[str, int] = {}
        fp16_b, q_b = 0, 0.0
        for b in sel:
            n = b.end - b.start
            fp16_b += 2 * n * 64 * 2
            q_b += 2 * n * 64 * _BYTES_PER_VALUE.get(b.precision, 2.0)
            dist[b.precision.value] = dist.get(b.precision.value, 0) + n
        pct = (1.0 - q_b / max(fp16_b, 1)) * 100.0 if fp16_b > 0 else 0.0
        return {"total_blocks": len(routed_blocks), "selected_blocks": len(sel),
                "skipped_blocks": len(self.skipped_blocks(routed_blocks)), "total_tokens": total,
                "selected_tokens": sel_tok, "skipped_tokens": total - sel_tok,
                "estimated_fp16_mb": round(fp16_b / (1024 * 1024), 3),
                "estimated_quant_mb": round(q_b / (1024 * 1024), 3),
                "bytes_saved_pct": round(pct, 2), "precision_distribution": dist}


def routing_to_kernel_metadata(routed_blocks: List[RoutedBlock], page_size: int) -> Dict:
    """Flat metadata for the kernel layer: page ids (routed order, first seen),
    prefetch hints, per-page precision names (first occurrence, numeric key
    order), block names and reasons."""
    router = BlockRouter(RouterConfig())
    by_page: Dict[int, str] = {}
    sel_ids: List[int] = []
    for pid, b in router._first_seen_pages(routed_blocks, page_size):
        sel_ids.append(pid)
        by_page[pid] = b.precision.value
    return {
        "selected_page_ids": sel_ids,
        "prefetch_page_ids": router.prefetch_page_ids(routed_blocks, page_size),
        "block_precision_by_page": {str(k): by_page[k] for k in sorted(by_page)},
        "selected_block_names": [b.name for b in router.selected_blocks(routed_blocks)],
        "skipped_block_names": [b.name for b in router.skipped_blocks(routed_blocks)],
        "reasons_by_block": {b.name: b.reason for b in routed_blocks},
    }
