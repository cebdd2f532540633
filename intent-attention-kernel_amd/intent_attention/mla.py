"""Multi-head latent attention (DeepSeek-V2/V3 style) over semantic blocks,
with the reference's interface (src/intent_attention/mla.py).

``MLAConfig``, ``absorb_weights`` and ``MLABlockTable`` keep the reference's
definitions (mla.py:15-58). The two decode entry points run the latent
attention on libiak's float32 row kernel (``triton_mla_decode.mla_latent_context``,
the reference's arithmetic) and keep the reference's results:

* ``mla_sparse_decode_reference`` (mla.py:61-92): the selected blocks' latents
  concatenated, ``softmax(q_absorb C^T / sqrt(d_c)) C @ W_VO`` returned as
  float16 (zeros of ``[batch, q_len, d_model]`` float32 when nothing is selected);
* ``mla_triton_decode`` (mla.py:95-136): the same latents as pages of
  ``mla_decode_triton``, float32 result as the reference's GPU branch.

Both take device tensors; host tensors raise RuntimeError.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from .block_metadata import BlockLayout
from .triton_mla_decode import mla_decode_triton, mla_latent_context


@dataclass
class MLAConfig:
    d_model: int
    d_c: int
    n_heads: int
    d_head: int
    d_rope: int = 64


def absorb_weights(W_UQ: torch.Tensor, W_UK: torch.Tensor, W_UV: torch.Tensor,
                   W_O: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(W_QK_fused, W_VO_fused) as the reference forms them (mla.py:23-27)."""
    W_QK_fused = W_UQ.float().half()
    W_VO_fused = torch.mm(W_UV.float(), W_O.float()).half()
    return W_QK_fused, W_VO_fused


class MLABlockTable:
    """Latent (and RoPE) pages appended per block id (mla.py:30-58)."""

    def __init__(self, config: MLAConfig, page_size: int = 64):
        self.config = config
        self.page_size = page_size
        self._latent_pages: Dict[int, List[torch.Tensor]] = {}
        self._rope_pages: Dict[int, List[torch.Tensor]] = {}

    def append(self, block_id: int, c_page: torch.Tensor, rope_page: Optional[torch.Tensor] = None) -> None:
        self._latent_pages.setdefault(block_id, []).append(c_page)
        if rope_page is not None:
            self._rope_pages.setdefault(block_id, []).append(rope_page)

    def get_latent(self, block_id: int) -> Optional[torch.Tensor]:
        pages = self._latent_pages.get(block_id)
        return torch.cat(pages, dim=0) if pages else None

    def get_rope(self, block_id: int) -> Optional[torch.Tensor]:
        pages = self._rope_pages.get(block_id)
        return torch.cat(pages, dim=0) if pages else None

    def memory_bytes(self) -> int:
        total = 0
        for pages in (*self._latent_pages.values(), *self._rope_pages.values()):
            for p in pages:
                total += p.numel() * 2
        return total


def _absorbed_query(q: torch.Tensor, W_QK_fused: torch.Tensor) -> torch.Tensor:
    batch, n_heads, q_len, d_head = q.shape
    q_flat = q.permute(0, 2, 1, 3).reshape(batch, q_len, n_heads * d_head).float()
    return torch.matmul(q_flat, W_QK_fused.float())


def _selected_latents(block_table: MLABlockTable, layout: BlockLayout, threshold: float) -> Tuple[list, list]:
    selected = [b for b in layout.selected_blocks() if b.score is None or b.score >= threshold]
    parts = []
    for b in selected:
        c = block_table.get_latent(layout.blocks.index(b) if isinstance(b.name, str) else b.name)
        if c is not None:
            parts.append(c)
    return selected, parts


def _debug(selected, layout: BlockLayout, block_table: MLABlockTable, latent_tokens: int) -> Dict:
    return {"selected_block_names": [b.name for b in selected],
            "selected_latent_tokens": latent_tokens,
            "total_kv_tokens": sum(b.end - b.start for b in layout.blocks),
            "mla_memory_bytes": block_table.memory_bytes()}


def mla_sparse_decode_reference(q: torch.Tensor, block_table: MLABlockTable, W_QK_fused: torch.Tensor,
                                W_VO_fused: torch.Tensor, layout: BlockLayout, threshold: float = 0.5,
                                return_debug: bool = False):
    """Latent attention over the selected blocks (mla.py:61-92); returns (out, debug or None)."""
    batch, _, q_len, _ = q.shape
    config = block_table.config
    q_absorb = _absorbed_query(q, W_QK_fused)
    selected, parts = _selected_latents(block_table, layout, threshold)
    if not parts:
        out = torch.zeros(batch, q_len, config.d_model)
        return (out, {"selected_latent_tokens": 0}) if return_debug else (out, None)
    C = torch.cat(parts, dim=0).float()
    if C.shape[1] != config.d_c:
        raise ValueError(f"latent width {C.shape[1]} != config.d_c {config.d_c}")
    ctx = mla_latent_context(q_absorb, C, torch.arange(C.shape[0], device=C.device, dtype=torch.int32), 1)
    out = torch.matmul(ctx, W_VO_fused.float()).half()
    if not return_debug:
        return out, None
    return out, _debug(selected, layout, block_table, C.shape[0])


def mla_triton_decode(q: torch.Tensor, block_table: MLABlockTable, W_QK_fused: torch.Tensor,
                      W_VO_fused: torch.Tensor, layout: BlockLayout, threshold: float = 0.5,
                      return_debug: bool = False):
    """The selected blocks' latents as pages of ``mla_decode_triton`` (mla.py:95-136)."""
    batch, _, q_len, _ = q.shape
    config = block_table.config
    q_absorb = _absorbed_query(q, W_QK_fused)
    selected, parts = _selected_latents(block_table, layout, threshold)
    if not parts:
        out = torch.zeros(batch, q_len, config.d_model)
        return (out, {"selected_latent_tokens": 0}) if return_debug else (out, None)
    sizes = [c.shape[0] for c in parts]
    page_size = sizes[0] if len(set(sizes)) == 1 else min(sizes)
    C = torch.cat(parts, dim=0).float()
    page_table = torch.arange(len(parts), dtype=torch.int32, device=C.device)
    out = mla_decode_triton(q_absorb.float(), C, W_VO_fused.float(), page_table, page_size=page_size)
    if not return_debug:
        return out, None
    return out, _debug(selected, layout, block_table, sum(sizes))
