"""Semantic block layout (policy input of the router).

Interface of the reference's block_metadata.py:10-93: ``BlockPolicy``,
``SELECTED_POLICIES``, ``SemanticBlock``, ``BlockLayout`` with the same
validation order and messages (:41-70).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import auto
from typing import Dict, List, Optional

from ._enum import StrEnum


class BlockPolicy(StrEnum):
    ALWAYS = auto()
    ATTEND = auto()
    SKIP = auto()
    RECENT = auto()
    GLOBAL = auto()


SELECTED_POLICIES = frozenset(p for p in BlockPolicy if p is not BlockPolicy.SKIP)


@dataclass
class SemanticBlock:
    name: str
    start: int
    end: int
    policy: BlockPolicy
    score: Optional[float] = None


@dataclass
class BlockLayout:
    blocks: List[SemanticBlock] = field(default_factory=list)

    def validate(self, total_tokens: int) -> None:
        prev: Optional[SemanticBlock] = None
        for i, b in enumerate(self.blocks):
            if not b.name:
                raise ValueError(f"Block at index {i} has empty name")
            if b.start < 0:
                raise ValueError(f"Block '{b.name}' has start={b.start} < 0")
            if b.end <= b.start:
                raise ValueError(f"Block '{b.name}' has end={b.end} <= start={b.start}")
            if b.end > total_tokens:
                raise ValueError(f"Block '{b.name}' has end={b.end} > total_tokens={total_tokens}")
            if b.policy == BlockPolicy.ATTEND and b.score is None:
                raise ValueError(f"Block '{b.name}' has policy ATTEND but score is None")
            if prev is not None:
                if b.start < prev.start:
                    raise ValueError(f"Blocks not sorted: '{b.name}' start={b.start} "
                                     f"< '{prev.name}' start={prev.start}")
                if b.start < prev.end:
                    raise ValueError(f"Blocks overlap: '{prev.name}' end={prev.end} "
                                     f"> '{b.name}' start={b.start}")
            prev = b

    def selected_blocks(self) -> List[SemanticBlock]:
        return [b for b in self.blocks if b.policy in SELECTED_POLICIES]

    def selected_token_indices(self) -> List[int]:
        return [t for b in self.selected_blocks() for t in range(b.start, b.end)]

    def selected_token_count(self) -> int:
        return sum(b.end - b.start for b in self.selected_blocks())

    def total_token_count(self) -> int:
        return sum(b.end - b.start for b in self.blocks)

    def summary(self) -> Dict[str, int]:
        return {"total_blocks": len(self.blocks), "selected_blocks": len(self.selected_blocks()),
                "total_token_count": self.total_token_count(),
                "selected_token_count": self.selected_token_count()}
