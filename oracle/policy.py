"""Oracle: block policy, precision policy, router and kernel metadata.

Loop-faithful CPU restatement of the reference's decision logic (integer and
string work; the product must match it exactly, including list order).

Reference files (relative to ``src/intent_attention/``):
  _enum.py:5-13                    StrEnum: auto() value == member name
  block_metadata.py:10-93          BlockPolicy, SELECTED_POLICIES, SemanticBlock, BlockLayout
  intent_quant.py:14-131           KVPrecision, _BYTES_PER_VALUE, QuantPolicy, IntentQuantizer
  block_router.py:18-421           BlockDecision, RoutedBlock, RouterConfig, BlockRouter,
                                   routing_to_kernel_metadata
  fused_selected_quant_decode.py:29-34, 344-400   FusedKVPrecision, metadata_to_kernel_tensors
  triton_intent_quant_attention.py:40-48, 126-203, 499-536

Pinned by: the hand-derived known answer of the reference's basic router
layout (tests/test_oracle_policy.py), the reference tests' own facts
(test_block_router.py, test_end_to_end_router.py,
test_fused_selected_quant_decode.py:258-286, test_triton_intent_quant_attention.py:28-101)
and golden vectors written by running the reference in the build container
(tests/golden/).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

# --------------------------------------------------------------------------- #
# String enums. The reference's StrEnum (_enum.py:5-7) makes auto() return the
# member name, so every value below equals its name.
# --------------------------------------------------------------------------- #


class _Names:
    @classmethod
    def all(cls) -> List[str]:
        return [v for k, v in vars(cls).items() if not k.startswith("_") and isinstance(v, str)]


class BlockPolicy(_Names):          # block_metadata.py:10-15
    ALWAYS = "ALWAYS"
    ATTEND = "ATTEND"
    SKIP = "SKIP"
    RECENT = "RECENT"
    GLOBAL = "GLOBAL"


SELECTED_POLICIES = frozenset({"ALWAYS", "ATTEND", "RECENT", "GLOBAL"})   # block_metadata.py:18-25


class KVPrecision(_Names):          # intent_quant.py:14-20
    FP16 = "FP16"
    FP8 = "FP8"
    INT8 = "INT8"
    INT4 = "INT4"
    INT4_RESIDUAL = "INT4_RESIDUAL"
    SKIP = "SKIP"


BYTES_PER_VALUE = {                 # intent_quant.py:23-30
    "FP16": 2.0, "FP8": 1.0, "INT8": 1.0, "INT4": 0.5, "INT4_RESIDUAL": 1.0, "SKIP": 0.0,
}


class BlockDecision(_Names):        # block_router.py:18-23
    SELECT = "SELECT"
    SKIP = "SKIP"
    PREFETCH = "PREFETCH"
    QUANTIZE = "QUANTIZE"
    PIN_HIGH_PRECISION = "PIN_HIGH_PRECISION"


FUSED_TAG = {"FP16": 0, "INT8": 1, "SKIP": 2}                     # fused_selected_quant_decode.py:29-34
TRITON_TAG = {"FP16": 0, "FP8": 1, "INT8": 2, "INT4": 3,          # triton_intent_quant_attention.py:40-48
              "INT4_RESIDUAL": 4, "SKIP": 5}


@dataclass
class SemanticBlock:                # block_metadata.py:28-34
    name: str
    start: int
    end: int
    policy: str
    score: Optional[float] = None


@dataclass
class BlockLayout:                  # block_metadata.py:37-93
    blocks: List[SemanticBlock] = field(default_factory=list)

    def validate(self, total_tokens: int) -> None:
        """block_metadata.py:41-70 (same checks, same order, same messages)."""
        for i, block in enumerate(self.blocks):
            if not block.name:
                raise ValueError(f"Block at index {i} has empty name")
            if block.start < 0:
                raise ValueError(f"Block '{block.name}' has start={block.start} < 0")
            if block.end <= block.start:
                raise ValueError(
                    f"Block '{block.name}' has end={block.end} <= start={block.start}")
            if block.end > total_tokens:
                raise ValueError(
                    f"Block '{block.name}' has end={block.end} > total_tokens={total_tokens}")
            if block.policy == BlockPolicy.ATTEND and block.score is None:
                raise ValueError(f"Block '{block.name}' has policy ATTEND but score is None")
            if i > 0:
                prev = self.blocks[i - 1]
                if block.start < prev.start:
                    raise ValueError(
                        f"Blocks not sorted: '{block.name}' start={block.start} "
                        f"< '{prev.name}' start={prev.start}")
                if block.start < prev.end:
                    raise ValueError(
                        f"Blocks overlap: '{prev.name}' end={prev.end} "
                        f"> '{block.name}' start={block.start}")

    def selected_blocks(self) -> List[SemanticBlock]:
        """block_metadata.py:72-73."""
        return [b for b in self.blocks if b.policy in SELECTED_POLICIES]

    def selected_token_count(self) -> int:
        return sum(b.end - b.start for b in self.selected_blocks())

    def total_token_count(self) -> int:
        return sum(b.end - b.start for b in self.blocks)


@dataclass
class QuantPolicy:                  # intent_quant.py:33-48
    precision: str
    reason: str = ""

    @property
    def estimated_bytes_per_value(self) -> float:
        return BYTES_PER_VALUE[self.precision]

    @property
    def requires_scale(self) -> bool:
        return self.precision in ("INT8", "INT4", "INT4_RESIDUAL")

    @property
    def uses_residual(self) -> bool:
        return self.precision == "INT4_RESIDUAL"


class IntentQuantizer:
    """intent_quant.py:51-131 (precision policy only)."""

    def __init__(self, memory_pressure: float = 0.0, preserve_recent: bool = True,
                 preserve_global: bool = True, high_score_threshold: float = 0.75,
                 medium_score_threshold: float = 0.40) -> None:
        if not 0.0 <= memory_pressure <= 1.0:          # :67-70
            raise ValueError(f"memory_pressure must be in [0, 1], got {memory_pressure}")
        self.memory_pressure = memory_pressure
        self.preserve_recent = preserve_recent
        self.preserve_global = preserve_global
        self.high_score_threshold = high_score_threshold
        self.medium_score_threshold = medium_score_threshold

    def assign_block_precision(self, block: SemanticBlock) -> QuantPolicy:
        """intent_quant.py:77-131: the decision tree, branch for branch."""
        pol, score, mp = block.policy, block.score, self.memory_pressure
        if pol in ("ALWAYS", "GLOBAL"):                                   # :83-92
            if pol == "GLOBAL" and self.preserve_global:
                if mp > 0.8:
                    return QuantPolicy("INT8", "global, extreme pressure")
                return QuantPolicy("FP16", "global, preserved")
            if mp > 0.9:
                return QuantPolicy("INT8", "always, extreme pressure")
            if mp > 0.7:
                return QuantPolicy("FP8", "always, high pressure")
            return QuantPolicy("FP16", "always, full precision")
        if pol == "RECENT":                                               # :95-106
            if self.preserve_recent:
                if mp > 0.8:
                    return QuantPolicy("INT8", "recent, extreme pressure")
                if mp > 0.5:
                    return QuantPolicy("FP8", "recent, moderate pressure")
                return QuantPolicy("FP8", "recent, preserved")
            if mp > 0.6:
                return QuantPolicy("INT4_RESIDUAL", "recent, high pressure, not preserved")
            return QuantPolicy("INT8", "recent, not preserved")
        if pol == "ATTEND":                                               # :109-125
            if score is None:
                return QuantPolicy("INT8" if mp > 0.5 else "FP16", "attend, no score")
            if score >= self.high_score_threshold:
                if mp > 0.8:
                    return QuantPolicy("INT8", "high-score, extreme pressure")
                if mp > 0.5:
                    return QuantPolicy("FP8", "high-score, moderate pressure")
                return QuantPolicy("INT8", "high-score attend")
            if score >= self.medium_score_threshold:
                if mp > 0.6:
                    return QuantPolicy("INT4", "medium-score, high pressure")
                return QuantPolicy("INT4_RESIDUAL", "medium-score attend")
            if mp > 0.3:
                return QuantPolicy("SKIP", "low-score, pressure")
            return QuantPolicy("INT4", "low-score attend")
        if pol == "SKIP":                                                 # :128-129
            return QuantPolicy("SKIP", "skipped block")
        return QuantPolicy("FP16", "default")                             # :131


@dataclass
class RouterConfig:                 # block_router.py:38-46
    top_k_blocks: int = 8
    score_threshold: float = 0.35
    recent_window_tokens: int = 2048
    memory_pressure: float = 0.5
    prefetch_top_k: int = 4
    preserve_system_prompt: bool = True
    preserve_recent: bool = True


@dataclass
class RoutedBlock:                  # block_router.py:26-35
    name: str
    start: int
    end: int
    policy: str
    score: Optional[float]
    decision: str
    precision: str
    reason: str


class BlockRouter:
    """block_router.py:80-337 (query-vector scoring, :49-77, is not on the path)."""

    def __init__(self, config: RouterConfig, quantizer: Optional[IntentQuantizer] = None):
        self.config = config
        self.quantizer = quantizer or IntentQuantizer(                    # :95-99
            memory_pressure=config.memory_pressure,
            preserve_recent=config.preserve_recent,
            preserve_global=config.preserve_system_prompt)

    def route_layout(self, layout: BlockLayout, total_tokens: int) -> List[RoutedBlock]:
        """block_router.py:101-266."""
        layout.validate(total_tokens)
        cfg = self.config
        high, attend, skip = [], [], []
        for b in layout.blocks:                                           # :126-132
            if b.policy in ("ALWAYS", "GLOBAL", "RECENT"):
                high.append(b)
            elif b.policy == "ATTEND":
                attend.append(b)
            else:
                skip.append(b)
        # :146-152 -- Python's sorted() is stable: equal scores keep layout order.
        scored = sorted([b for b in attend if b.score is not None],
                        key=lambda b: (b.score or 0.0), reverse=True)
        top_k, bottom = scored[:cfg.top_k_blocks], scored[cfg.top_k_blocks:]
        out: List[RoutedBlock] = []
        for b in high:                                                    # :157-184
            prec = self.quantizer.assign_block_precision(b).precision
            if b.policy in ("ALWAYS", "GLOBAL"):
                out.append(RoutedBlock(b.name, b.start, b.end, b.policy, b.score,
                                       "PIN_HIGH_PRECISION", prec,
                                       f"{b.policy} block, always selected"))
            else:
                out.append(RoutedBlock(b.name, b.start, b.end, b.policy, b.score,
                                       "SELECT", prec, "recent context, always selected"))
        for b in top_k:                                                   # :186-215
            if b.score is None:
                continue
            prec = self.quantizer.assign_block_precision(b).precision
            if prec == "SKIP":
                out.append(RoutedBlock(b.name, b.start, b.end, b.policy, b.score, "SKIP", prec,
                                       "low-score attend, skipped under memory pressure"))
                continue
            out.append(RoutedBlock(
                b.name, b.start, b.end, b.policy, b.score,
                "QUANTIZE" if prec != "FP16" else "SELECT", prec,
                f"attend score={b.score:.3f} >= threshold={cfg.score_threshold}"))
        for b in bottom:                                                  # :217-233
            prec = self.quantizer.assign_block_precision(b).precision
            reason = "below top-k"
            if cfg.memory_pressure > 0.5 and b.score is not None and b.score < cfg.score_threshold:
                reason += ", low score with pressure"
            out.append(RoutedBlock(b.name, b.start, b.end, b.policy, b.score, "SKIP", prec, reason))
        for b in skip:                                                    # :235-264
            prec = self.quantizer.assign_block_precision(b).precision
            if b.score is not None and b.score >= cfg.score_threshold:
                out.append(RoutedBlock(b.name, b.start, b.end, b.policy, b.score, "SELECT", prec,
                                       "SKIP block with unexpectedly high score, selected"))
            else:
                out.append(RoutedBlock(b.name, b.start, b.end, b.policy, b.score, "SKIP", "SKIP",
                                       "SKIP block, not selected"))
        return out

    @staticmethod
    def selected_blocks(routed: List[RoutedBlock]) -> List[RoutedBlock]:
        """block_router.py:268-272."""
        return [b for b in routed if b.decision in ("SELECT", "PIN_HIGH_PRECISION", "QUANTIZE")]

    @staticmethod
    def skipped_blocks(routed: List[RoutedBlock]) -> List[RoutedBlock]:
        """block_router.py:274-275."""
        return [b for b in routed if b.decision == "SKIP"]

    def selected_page_ids(self, routed: List[RoutedBlock], page_size: int) -> List[int]:
        """block_router.py:283-296: token by token, first-seen dedupe, routed order."""
        ids, seen = [], set()
        for b in self.selected_blocks(routed):
            for t in range(b.start, b.end):
                pid = t // page_size
                if pid not in seen:
                    seen.add(pid)
                    ids.append(pid)
        return ids

    def prefetch_page_ids(self, routed: List[RoutedBlock], page_size: int) -> List[int]:
        """block_router.py:298-337."""
        cfg = self.config
        cands: List[Tuple[float, int]] = []
        for b in routed:
            if b.decision == "SKIP" and b.score is not None and b.score >= cfg.score_threshold:
                for t in range(b.start, b.end):
                    cands.append((b.score, t // page_size))
        for b in self.selected_blocks(routed):
            left = max(0, b.start // page_size - 1)
            right = (b.end + page_size - 1) // page_size
            for pid in range(left, right + 1):
                cands.append((1.0, pid))
        if not cands:
            return []
        best: Dict[int, float] = {}
        for score, pid in cands:
            if pid not in best or score > best[pid]:
                best[pid] = score
        order = sorted(best.items(), key=lambda x: (-x[1], x[0]))
        out, seen = [], set()
        # :329-335 iterates ``(page_id, score)`` items as ``for score, pid in``:
        # the names are swapped, so the list is deduplicated on, and holds, the
        # SCORE values (distinct scores, highest first), not page ids. Kept as
        # the reference computes it.
        for _page_id, score in order:
            if score not in seen:
                seen.add(score)
                out.append(score)
        return out[: cfg.prefetch_top_k]


def routing_to_kernel_metadata(routed: List[RoutedBlock], page_size: int) -> Dict:
    """block_router.py:383-421. Prefetch uses a default RouterConfig() (:398)."""
    router = BlockRouter(RouterConfig())
    selected = router.selected_blocks(routed)
    skipped = router.skipped_blocks(routed)
    sel_ids = router.selected_page_ids(routed, page_size)
    pre_ids = router.prefetch_page_ids(routed, page_size)
    prec_by_page: Dict[int, str] = {}
    for b in selected:                                                    # :405-410
        for t in range(b.start, b.end):
            pid = t // page_size
            if pid not in prec_by_page:
                prec_by_page[pid] = b.precision
    return {
        "selected_page_ids": sel_ids,
        "prefetch_page_ids": pre_ids,
        "block_precision_by_page": {str(k): v for k, v in sorted(prec_by_page.items())},
        "selected_block_names": [b.name for b in selected],
        "skipped_block_names": [b.name for b in skipped],
        "reasons_by_block": {b.name: b.reason for b in routed},
    }


def metadata_to_kernel_tensors(meta: Dict, num_pages: int, B: int = 1, H: int = 1,
                               max_selected: int = 64, native_precisions: bool = False):
    """fused_selected_quant_decode.py:344-400 as numpy int32 arrays.

    Reference mapping (native_precisions=False, :379-389): "SKIP"->2, "INT8",
    "INT4", "INT4_RESIDUAL"->1, any other string (incl. "FP8")->0; keys that
    are not integers are skipped; default tag FP16 (0); the same id list is
    broadcast to every (b, h) and truncated to max_selected.

    native_precisions=True is this build's opt-in extension: FP8->3, INT4->4,
    INT4_RESIDUAL->5 (the fused numbering with new tags appended).
    """
    table = np.zeros((B, H, max_selected), dtype=np.int32)
    counts = np.zeros((B, H), dtype=np.int32)
    prec = np.full((num_pages,), 0, dtype=np.int32)
    for k, v in meta.get("block_precision_by_page", {}).items():
        try:
            pid = int(k)
        except ValueError:
            continue
        if v == "SKIP":
            prec[pid] = 2
        elif v == "INT8":
            prec[pid] = 1
        elif v in ("INT4", "INT4_RESIDUAL"):
            prec[pid] = (4 if v == "INT4" else 5) if native_precisions else 1
        elif v == "FP8" and native_precisions:
            prec[pid] = 3
        else:
            prec[pid] = 0
    ids = meta.get("selected_page_ids", [])
    n = min(len(ids), max_selected)
    for b in range(B):
        for h in range(H):
            for p in range(n):
                table[b, h, p] = ids[p]
            counts[b, h] = n
    return table, prec, counts


def make_page_tables_from_selected_pages(selected, batch: int, heads: int,
                                         max_selected_pages: Optional[int] = None):
    """triton_intent_quant_attention.py:126-203 (numpy; -1 padding)."""
    selected = np.asarray(selected)
    if selected.ndim == 1:
        n = selected.size
        width = max_selected_pages or n
        if n > width:
            raise ValueError("selected_pages length exceeds max_selected_pages")
        ids = np.full((batch, heads, width), -1, dtype=np.int32)
        ids[:, :, :n] = selected.astype(np.int32).reshape(1, 1, n)
        return ids, np.full((batch, heads), n, dtype=np.int32)
    if selected.ndim == 3:
        if selected.shape[0] != batch or selected.shape[1] != heads:
            raise ValueError("selected_pages [B, H, N] must match batch and heads")
        n = selected.shape[2]
        width = max_selected_pages or n
        if n > width:
            raise ValueError("selected_pages width exceeds max_selected_pages")
        ids = np.full((batch, heads, width), -1, dtype=np.int32)
        ids[:, :, :n] = selected.astype(np.int32)
        return ids, np.full((batch, heads), n, dtype=np.int32)
    raise ValueError("selected_pages must have shape [N] or [B, H, N]")


def make_precision_tensor(num_pages: int, fp16_pages=None, int8_pages=None):
    """triton_intent_quant_attention.py:499-536 (default INT8 = 2)."""
    prec = np.full((num_pages,), TRITON_TAG["INT8"], dtype=np.int32)
    if fp16_pages is not None:
        prec[np.asarray(fp16_pages, dtype=np.int64)] = TRITON_TAG["FP16"]
    if int8_pages is not None:
        prec[np.asarray(int8_pages, dtype=np.int64)] = TRITON_TAG["INT8"]
    return prec


# --------------------------------------------------------------------------- #
# Page tables from routed spans: routing_to_kernel_metadata followed by
# metadata_to_kernel_tensors, generalised to one span list per group of rows,
# a logical -> physical block table and residency. Test infrastructure: the
# product computes this on the GPU (iak_build_page_tables).
# --------------------------------------------------------------------------- #

def reference_tag(name: str, native_precisions: bool = False) -> int:
    """The precision string -> fused tag mapping of metadata_to_kernel_tensors
    (fused_selected_quant_decode.py:379-389; native tags as above)."""
    if name == "SKIP":
        return 2
    if name == "INT8":
        return 1
    if name in ("INT4", "INT4_RESIDUAL"):
        return (4 if name == "INT4" else 5) if native_precisions else 1
    if name == "FP8" and native_precisions:
        return 3
    return 0


def routed_spans(routed: List[RoutedBlock], native_precisions: bool = False) -> List[Tuple[int, int, int]]:
    """(start, end, tag) of the selected blocks in routed order (the blocks
    whose tokens routing_to_kernel_metadata pages, block_router.py:400-410)."""
    return [(b.start, b.end, reference_tag(b.precision, native_precisions))
            for b in BlockRouter.selected_blocks(routed)]


def build_page_tables_oracle(lists, num_rows: int, table_width: int, page_size: int, num_pages: int, *,
                             rows_per_seq: int = 1, rows_per_list: Optional[int] = None, block_table=None,
                             dedupe: bool = True, default_tag: int = 0):
    """Loops over rows, spans and tokens; numpy int32 (page_table [R, W],
    page_precision [num_pages], page_counts [R]).

    ``lists[l]`` is a list of ``(start, end, tag)`` spans in routed order. Row
    ``r`` reads list ``r // rows_per_list`` (default: one list for every row,
    the reference's broadcast) and block-table row ``r // rows_per_seq``.
    Per row:
      * logical pages ``t // page_size`` of tokens ``start <= t < end``, span by
        span, first seen only (block_router.py:283-296, :405-410); with
        ``dedupe=False`` every page of every span, in order;
      * physical id ``block_table[seq][l]`` (``l`` outside the row or a negative
        entry: not resident, dropped), or ``l`` without a block table; ids
        outside ``[0, num_pages)`` are dropped;
      * ``page_table[r, :n]`` = the first ``min(n, W)`` ids, zeros after, and
        ``page_counts[r] = min(n, W)`` (fused_selected_quant_decode.py:394-400);
      * ``page_precision[q]`` = the tag of the span that emitted ``q``, taken
        from the lowest row that emits ``q`` (the smallest tag if that row
        emits ``q`` twice); pages no row emits keep ``default_tag``. Every page
        a row emits counts, also those past ``W`` (the reference tags every key
        of block_precision_by_page).
    """
    rpl = num_rows if rows_per_list is None else rows_per_list
    table = np.zeros((num_rows, table_width), dtype=np.int32)
    counts = np.zeros((num_rows,), dtype=np.int32)
    prec = np.full((num_pages,), default_tag, dtype=np.int32)
    owner_row = {}
    memo = {}
    for r in range(num_rows):
        key = (r // max(rpl, 1), r // rows_per_seq)
        if key in memo:                       # rows sharing list and block-table row
            ids, tags = memo[key]
            n = min(len(ids), table_width)
            table[r, :n] = ids[:n]
            counts[r] = n
            continue
        spans = lists[key[0]]
        seq = key[1]
        ids, tags, seen = [], [], set()
        for start, end, tag in spans:
            for t in range(start, end):
                lp = t // page_size
                if dedupe:
                    if lp in seen:
                        continue
                    seen.add(lp)
                if block_table is not None:
                    row = block_table[seq]
                    q = int(row[lp]) if 0 <= lp < len(row) else -1
                else:
                    q = lp
                if 0 <= q < num_pages and (dedupe or t == start or (t - 1) // page_size != lp):
                    ids.append(q)
                    tags.append(tag)
        memo[key] = (ids, tags)
        n = min(len(ids), table_width)
        table[r, :n] = ids[:n]
        counts[r] = n
        for q, tag in zip(ids, tags):
            if q not in owner_row or owner_row[q][0] == r and tag < prec[q]:
                owner_row[q] = (r, tag)
                prec[q] = tag
    return table, prec, counts
