"""KV memory manager page store on the MI355X: FP16 <-> INT8 page transcoding
on the HIP kernels (iak_transcode_pages).

Interface of the reference's kv_memory_manager.py: ``PageStorageFormat``
(:23-27), ``PageState`` (:30-57), ``PageFormatPolicy`` (:60-84),
``_format_for_block`` / ``_page_page_mask`` (:87-108) and ``KVMemoryManager``
(:111-570) with the same page bookkeeping, format policy, self-tuning
thresholds, demotion / promotion rules, page selection and prefetch warm-up.

The page store differs in where the bytes live and what computes them:

* the FP16 and INT8 pools, and the float32 INT8 scales, are device tensors
  ([capacity, page_size * head_dim]); a page's ``kv_fp16`` / ``kv_int8`` is a
  view of its pool row, as in the reference;
* INT8 pages are written (demoted) and read back (promoted) by libiak's
  transcoding kernel with the reference's arithmetic (scale = max|x| / 127,
  codes = clamp(round(float16(x / scale)), -128, 127), read-back
  float16(code * scale)), bit-exact; ``demote_cold_pages``,
  ``promote_hot_pages`` and the prefetch warm-up transcode every page they
  pick in one launch; ``kv_int8_scale`` holds the float64 value of the scale;
* SPARSE pages keep the reference's top-k storage (torch ops on the device)
  and are interface-only, as in the reference's attention;
* ``step`` computes the attention the reference's step sets up
  (adaptive_format_attention.py:25-112 over the tensors of
  kv_memory_manager.py:444-479): every query head attends the page_size
  tokens of every selected page with K = V = the page's rows, FP16 rows as
  stored, INT8 rows as code * float16(scale), SPARSE rows filled at their
  index positions, pages without data as zero rows, and with ``mask=True``
  the rows outside a partial page's mask zeroed; on the paged-decode kernel.
  The reference's own step returns zeros for every input: the score and
  accumulator update (adaptive_format_attention.py:98-112) is indented under
  the unknown-format branch, so no page ever contributes. Its step also
  indexes page_counts [1, 1] by every (batch, head) and so takes B = H = 1
  only; here every (batch, head) attends the same pages.

Device tensors only: a manager on a non-ROCm device raises RuntimeError.
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass
from enum import IntEnum
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native as N
from .block_metadata import BlockLayout, BlockPolicy
from .decode_core import PagePools, current_stream_handle, paged_decode
from .prefetch import BlockPrefetcher


class PageStorageFormat(IntEnum):
    FP16 = 0
    INT8 = 1
    SPARSE = 2
    SKIP = 3


@dataclass
class PageState:
    page_id: int
    format: PageStorageFormat = PageStorageFormat.FP16
    access_count: int = 0
    last_access_step: int = -1
    block_name: str = ""
    block_policy: str = ""
    score: float = 0.0
    numa_hint: int = 0
    token_start: int = 0
    token_end: int = 0
    kv_fp16: Optional[torch.Tensor] = None
    kv_int8: Optional[torch.Tensor] = None
    kv_int8_scale: float = 1.0
    sp_k_indices: Optional[torch.Tensor] = None
    sp_k_values: Optional[torch.Tensor] = None
    sp_v_indices: Optional[torch.Tensor] = None
    sp_v_values: Optional[torch.Tensor] = None
    sp_nnz: int = 0
    partial_page_mask: Optional[torch.Tensor] = None

    def __post_init__(self):
        self.format = PageStorageFormat(self.format)


@dataclass
class PageFormatPolicy:
    """Block policy and access pattern -> storage format; the thresholds adapt
    when ``KVMemoryManager.adapt_policy_every`` > 0."""

    always_format: PageStorageFormat = PageStorageFormat.FP16
    global_format: PageStorageFormat = PageStorageFormat.FP16
    recent_format: PageStorageFormat = PageStorageFormat.FP16
    attend_high_format: PageStorageFormat = PageStorageFormat.FP16
    attend_low_format: PageStorageFormat = PageStorageFormat.INT8
    skip_format: PageStorageFormat = PageStorageFormat.SKIP
    score_threshold: float = 0.5
    demote_cold_after_steps: int = 10
    demote_cold_to: PageStorageFormat = PageStorageFormat.INT8
    promote_hot_after_accesses: int = 3
    promote_hot_to: PageStorageFormat = PageStorageFormat.FP16
    demote_step_min: int = 2
    demote_step_max: int = 50
    promote_access_min: int = 1
    promote_access_max: int = 20


def _format_for_block(policy: str, score: float, cfg: PageFormatPolicy) -> PageStorageFormat:
    by_policy = {BlockPolicy.ALWAYS.value: cfg.always_format, BlockPolicy.GLOBAL.value: cfg.global_format,
                 BlockPolicy.RECENT.value: cfg.recent_format, BlockPolicy.SKIP.value: cfg.skip_format}
    if policy in by_policy:
        return by_policy[policy]
    if policy == BlockPolicy.ATTEND.value:
        return cfg.attend_high_format if score >= cfg.score_threshold else cfg.attend_low_format
    return cfg.attend_low_format


def _page_page_mask(page_size: int, token_start: int, token_end: int) -> torch.Tensor:
    """Valid-token mask of one partial page: tokens token_start % page_size .. +(end - start)."""
    mask = torch.zeros(page_size, dtype=torch.bool)
    lo = token_start % page_size
    mask[lo:min(lo + (token_end - token_start), page_size)] = True
    return mask


class KVMemoryManager:
    """Per-page storage formats (FP16 / INT8 / SPARSE / SKIP) on device pools,
    with self-tuning demotion / promotion and prefetch warm-up."""

    def __init__(self, num_pages: int, page_size: int, head_dim: int, policy: Optional[PageFormatPolicy] = None,
                 device: str = "cuda", sparse_max_nnz: int = 8, adapt_policy_every: int = 5):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("KVMemoryManager keeps its pages on a ROCm device (the MI355X transcoding "
                               f"kernels); got device {self.device}")
        if (page_size * head_dim) % 8:
            raise ValueError(f"page_size * head_dim must be a multiple of 8, got {page_size * head_dim}")
        N.load()
        self.num_pages = num_pages
        self.page_size = page_size
        self.head_dim = head_dim
        self.policy = policy or PageFormatPolicy()
        self.sparse_max_nnz = sparse_max_nnz
        self.adapt_policy_every = adapt_policy_every
        self.step_count = 0
        self.pages: Dict[int, PageState] = {}
        self.block_name_to_page_ids: Dict[str, List[int]] = {}
        self._prefetcher = BlockPrefetcher()
        self._prefetch_predictions: List[int] = []
        self._demote_history: deque = deque(maxlen=50)
        self._hot_access_history: List[int] = []
        cap = max(1, num_pages)
        e = page_size * head_dim
        self._fp16_pool = torch.zeros((cap, e), dtype=torch.float16, device=self.device)
        self._int8_pool = torch.zeros((cap, e), dtype=torch.int8, device=self.device)
        self._scales = torch.ones(cap, dtype=torch.float32, device=self.device)

    # ---------------------------------------------------------------- pools

    @property
    def _elems(self) -> int:
        return self.page_size * self.head_dim

    def _grow_pool(self, needed: int) -> None:
        cap = self._fp16_pool.shape[0]
        if needed <= cap:
            return
        new = max(needed, 2 * cap)
        for name in ("_fp16_pool", "_int8_pool"):
            old = getattr(self, name)
            t = torch.zeros((new, self._elems), dtype=old.dtype, device=self.device)
            t[:cap] = old
            setattr(self, name, t)
        s = torch.ones(new, dtype=torch.float32, device=self.device)
        s[:cap] = self._scales
        self._scales = s
        # views of the old pools are stale: point every page at the new rows
        for st in self.pages.values():
            if st.kv_fp16 is not None:
                st.kv_fp16 = self._fp16_slice(st.page_id)
            if st.kv_int8 is not None:
                st.kv_int8 = self._int8_slice(st.page_id)

    def _fp16_slice(self, pid: int) -> torch.Tensor:
        return self._fp16_pool[pid].view(self.page_size, self.head_dim)

    def _int8_slice(self, pid: int) -> torch.Tensor:
        return self._int8_pool[pid].view(self.page_size, self.head_dim)

    def _transcode(self, pids: Sequence[int], mode: int, fp16: Optional[torch.Tensor] = None,
                   int8: Optional[torch.Tensor] = None, scales: Optional[torch.Tensor] = None) -> None:
        """One iak_transcode_pages launch over pool slots ``pids`` (default pools)."""
        if not pids:
            return
        fp16 = self._fp16_pool if fp16 is None else fp16
        int8 = self._int8_pool if int8 is None else int8
        scales = self._scales if scales is None else scales
        ids = torch.tensor(list(pids), dtype=torch.int32, device=self.device)
        a = N.TranscodeArgs()
        a.num_pages, a.page_elems, a.mode = len(pids), self._elems, mode
        a.pages, a.pool_pages = ids.data_ptr(), fp16.shape[0]
        a.fp16, a.int8, a.scales = fp16.data_ptr(), int8.data_ptr(), scales.data_ptr()
        N.transcode_pages(a, current_stream_handle(self.device))
        torch.autograd.graph.increment_version([fp16, int8, scales])   # written through raw pointers

    def _zero_rows(self, pids: Sequence[int]) -> None:
        """Pool rows of pages that hold no data: zero FP16 rows, zero codes, scale 1
        (what the reference's attention tensors hold for such pages)."""
        if not pids:
            return
        self._grow_pool(max(pids) + 1)
        idx = torch.tensor(list(pids), dtype=torch.long, device=self.device)
        self._fp16_pool[idx] = 0
        self._int8_pool[idx] = 0
        self._scales[idx] = 1.0

    def _scale_values(self, pids: Sequence[int]) -> List[float]:
        """The reference's float64 scales max_abs / 127 of pages whose float32
        scales the demote kernel stored: max_abs is a float16 value, and the
        float32 quotient is within 2^-24 (relative) of max_abs / 127, so
        float16(scale32 * 127) recovers max_abs exactly (0 and NaN pages hold
        scale 1.0 = 127 / 127; inf stays inf)."""
        s32 = self._scales[torch.tensor(list(pids), device=self.device, dtype=torch.long)].double().tolist()
        return [float(np.float16(v * 127.0)) / 127.0 for v in s32]

    # ----------------------------------------------------------- bookkeeping

    def register_layout(self, layout: BlockLayout) -> None:
        """Pages for every block of the layout (formats and token bounds)."""
        self.block_name_to_page_ids.clear()
        nxt = 0
        for block in layout.blocks:
            n = (block.end - block.start + self.page_size - 1) // self.page_size
            policy_str = str(getattr(block.policy, "value", block.policy))
            ids = []
            for i in range(n):
                pid = nxt + i
                lo = block.start + i * self.page_size
                hi = min(block.start + (i + 1) * self.page_size, block.end)
                full = hi - lo == self.page_size
                self.pages[pid] = PageState(
                    page_id=pid, format=_format_for_block(policy_str, block.score or 0.0, self.policy),
                    block_name=block.name, block_policy=policy_str, score=block.score or 0.0, token_start=lo,
                    token_end=hi, partial_page_mask=None if full else _page_page_mask(self.page_size, lo, hi))
                ids.append(pid)
            self.block_name_to_page_ids[block.name] = ids
            self._zero_rows(ids)
            nxt += n

    def allocate_pages(self, block_name: str, block_policy: str, num_pages: int, score: float = 0.0,
                       token_start: int = 0, token_end: int = 0) -> List[int]:
        first = len(self.pages)
        ids = []
        for i in range(num_pages):
            pid = first + i
            self.pages[pid] = PageState(page_id=pid, format=_format_for_block(block_policy, score, self.policy),
                                        block_name=block_name, block_policy=block_policy, score=score,
                                        token_start=token_start, token_end=token_end)
            ids.append(pid)
        self.block_name_to_page_ids.setdefault(block_name, []).extend(ids)
        self._zero_rows(ids)
        return ids

    # ------------------------------------------------------------ page data

    def write_page(self, page_id: int, kv: torch.Tensor) -> None:
        if page_id not in self.pages:
            raise ValueError(f"page_id {page_id} not allocated")
        st = self.pages[page_id]
        if st.format == PageStorageFormat.SKIP:
            return
        kv16 = kv.to(device=self.device, dtype=torch.float16).reshape(self.page_size, self.head_dim)
        if st.format in (PageStorageFormat.FP16, PageStorageFormat.INT8):
            self._grow_pool(page_id + 1)
            self._fp16_slice(page_id).copy_(kv16)
            if st.format == PageStorageFormat.FP16:
                st.kv_fp16 = self._fp16_slice(page_id)
            else:
                self._transcode([page_id], N.TRANSCODE_DEMOTE_INT8)
                st.kv_int8 = self._int8_slice(page_id)
                st.kv_int8_scale = self._scale_values([page_id])[0]
                st.kv_fp16 = None
        elif st.format == PageStorageFormat.SPARSE:
            flat = kv16.flatten()
            k = min(self.sparse_max_nnz, flat.numel())
            _, idx = flat.abs().topk(k)
            st.sp_k_indices = st.sp_v_indices = idx.to(torch.int64)
            st.sp_k_values = st.sp_v_values = flat[idx]
            st.sp_nnz = k

    def _read_page_data(self, page_id: int) -> Optional[torch.Tensor]:
        st = self.pages.get(page_id)
        if st is None:
            return None
        if st.format == PageStorageFormat.FP16 and st.kv_fp16 is not None:
            return st.kv_fp16.clone()
        if st.format == PageStorageFormat.INT8 and st.kv_int8 is not None:
            out = torch.empty((1, self._elems), dtype=torch.float16, device=self.device)
            self._transcode([0], N.TRANSCODE_PROMOTE_FP16, fp16=out, int8=self._int8_pool[page_id:page_id + 1],
                            scales=self._scales[page_id:page_id + 1])
            return out.view(self.page_size, self.head_dim)
        if st.format == PageStorageFormat.SPARSE and st.sp_k_values is not None:
            out = torch.zeros(self._elems, dtype=torch.float16, device=self.device)
            out[st.sp_k_indices] = st.sp_k_values
            return out.view(self.page_size, self.head_dim)
        if st.format == PageStorageFormat.SKIP:
            return torch.zeros(self.page_size, self.head_dim, dtype=torch.float16, device=self.device)
        return None

    def _clear(self, st: PageState) -> None:
        st.kv_fp16 = st.kv_int8 = None
        st.sp_k_indices = st.sp_k_values = st.sp_v_indices = st.sp_v_values = None
        st.sp_nnz = 0

    def set_page_formats(self, page_ids: Sequence[int], new_fmt: PageStorageFormat) -> None:
        """set_page_format for many pages: FP16 -> INT8 and INT8 -> FP16 pages are
        transcoded in one kernel launch each; other transitions go page by page."""
        new_fmt = PageStorageFormat(new_fmt)
        demote, promote = [], []
        for pid in page_ids:
            st = self.pages.get(pid)
            if st is None or st.format == new_fmt:
                continue
            if st.format == PageStorageFormat.FP16 and st.kv_fp16 is not None and new_fmt == PageStorageFormat.INT8:
                demote.append(pid)
            elif (st.format == PageStorageFormat.INT8 and st.kv_int8 is not None
                  and new_fmt == PageStorageFormat.FP16):
                promote.append(pid)
            else:
                data = self._read_page_data(pid)
                st.format = new_fmt
                self._clear(st)
                if data is not None:
                    self.write_page(pid, data)
                else:
                    self._zero_rows([pid])
        self._transcode(demote, N.TRANSCODE_DEMOTE_INT8)
        scales = self._scale_values(demote) if demote else []
        for pid, s in zip(demote, scales):
            st = self.pages[pid]
            self._clear(st)
            st.format, st.kv_int8, st.kv_int8_scale = new_fmt, self._int8_slice(pid), s
        self._transcode(promote, N.TRANSCODE_PROMOTE_FP16)
        for pid in promote:
            st = self.pages[pid]
            self._clear(st)
            st.format, st.kv_fp16 = new_fmt, self._fp16_slice(pid)

    def set_page_format(self, page_id: int, new_fmt: PageStorageFormat) -> None:
        self.set_page_formats([page_id], new_fmt)

    # ------------------------------------------------------ self-tuning policy

    def _adapt_policy(self) -> None:
        """Tune the demotion / promotion thresholds from the access history."""
        if self.step_count % self.adapt_policy_every != 0:
            return
        hit_rate = sum(self._demote_history) / max(len(self._demote_history), 1)
        fp16 = [s for s in self.pages.values() if s.format == PageStorageFormat.FP16]
        cold = sum(1 for s in fp16 if (self.step_count - s.last_access_step if s.last_access_step >= 0
                                       else self.step_count) >= self.policy.demote_cold_after_steps)
        cold_rate = cold / max(len(fp16), 1) if fp16 else 0.0
        p = self.policy
        if hit_rate > 0.30 and p.demote_cold_after_steps < p.demote_step_max:
            p.demote_cold_after_steps += 1
        if cold_rate > 0.50 and p.demote_cold_after_steps > p.demote_step_min:
            p.demote_cold_after_steps -= 1
        hot = sum(1 for s in self.pages.values()
                  if s.format == PageStorageFormat.INT8 and s.access_count >= p.promote_hot_after_accesses)
        if hot == 0 and fp16 and cold_rate < 0.2 and p.promote_hot_after_accesses < p.promote_access_max:
            p.promote_hot_after_accesses += 1

    def _prefetch_warmup(self) -> List[int]:
        """Promote the prefetch-predicted INT8 pages (one transcoding launch)."""
        warm = [pid for pid in self._prefetch_predictions
                if pid in self.pages and self.pages[pid].format == PageStorageFormat.INT8]
        self.set_page_formats(warm, self.policy.promote_hot_to)
        return warm

    def demote_cold_pages(self) -> List[int]:
        """Demote pages not accessed for demote_cold_after_steps steps (one launch)."""
        demoted = []
        for pid, st in list(self.pages.items()):
            if st.format in (PageStorageFormat.SKIP, PageStorageFormat.INT8, PageStorageFormat.SPARSE):
                continue
            since = self.step_count - st.last_access_step
            if st.last_access_step >= 0 and since >= self.policy.demote_cold_after_steps:
                demoted.append(pid)
                self._demote_history.append(since < self.policy.demote_cold_after_steps * 2)
        self.set_page_formats(demoted, self.policy.demote_cold_to)
        return demoted

    def promote_hot_pages(self) -> List[int]:
        """Promote INT8 pages accessed promote_hot_after_accesses times (one launch)."""
        promoted = [pid for pid, st in self.pages.items()
                    if st.format == PageStorageFormat.INT8 and st.access_count >= self.policy.promote_hot_after_accesses]
        self.set_page_formats(promoted, self.policy.promote_hot_to)
        return promoted

    # -------------------------------------------------------------- selection

    def select_pages(self) -> Tuple[List[int], torch.Tensor, torch.Tensor, Optional[Dict[int, torch.Tensor]]]:
        """(selected page ids, format tags [num_pages], page ids [1, 1, max_sel]
        padded with -1, partial-page masks or None)."""
        selected = [pid for pid, s in self.pages.items()
                    if s.format != PageStorageFormat.SKIP and s.block_policy != BlockPolicy.SKIP.value]
        fmts = torch.zeros(len(self.pages) or 1, dtype=torch.int32)
        for pid, s in self.pages.items():
            fmts[pid] = int(s.format)
        ids = torch.full((1, 1, max(len(selected), 1)), -1, dtype=torch.int32)
        ids[0, 0, :len(selected)] = torch.tensor(selected, dtype=torch.int32)
        masks = {pid: self.pages[pid].partial_page_mask for pid in selected
                 if self.pages[pid].partial_page_mask is not None} or None
        return selected, fmts, ids, masks

    def _kernel_layout(self) -> bool:
        """Pools in the decode kernel's own page layout (16 tokens, head_dim 64 / 128)."""
        return self.page_size == 16 and self.head_dim in (64, 128)

    def _pool_decode(self, query: torch.Tensor, selected: List[int], fmts: torch.Tensor,
                     ids: torch.Tensor) -> torch.Tensor:
        """Decode straight from the pools: FP16 rows and INT8 codes in place."""
        B, H, D = query.shape
        cap = self._fp16_pool.shape[0]
        s16 = self._scales.half()                 # the reference's attention takes float16 page scales
        pools = PagePools(k_fp16=self._fp16_pool.view(cap, 16, D), v_fp16=self._fp16_pool.view(cap, 16, D),
                          k_int8=self._int8_pool.view(cap, 16, D), v_int8=self._int8_pool.view(cap, 16, D),
                          k_int8_scale=s16, v_int8_scale=s16)
        tags = torch.full((cap,), int(PageStorageFormat.SKIP), dtype=torch.int32)
        tags[:fmts.numel()] = fmts[:cap]
        W = ids.shape[2]
        return paged_decode(query, pools, ids.to(self.device).expand(B, H, W).contiguous(),
                            torch.full((B, H), len(selected), dtype=torch.int32, device=self.device),
                            tags.to(self.device), tag_map=[N.TAG_FP16, N.TAG_INT8] + [N.TAG_SKIP] * 6,
                            sm_scale=1.0 / math.sqrt(D), out_dtype=torch.float16)

    def _staged_rows(self, selected: List[int], masks: Optional[Dict[int, torch.Tensor]]) -> torch.Tensor:
        """The selected pages' K (= V) rows [len(selected) * page_size, head_dim]
        float16, page by page as the reference's attention reconstructs them:
        FP16 rows; INT8 codes * float16(scale) (the transcoding kernel's promote
        with float16-rounded scales); SPARSE rows at positions ``indices < page_size``
        filled with their value; FP16 / INT8 rows outside a partial-page mask
        zeroed when ``masks`` is given; pages with no data are zero rows."""
        PS, D, n = self.page_size, self.head_dim, len(selected)
        rows = torch.zeros((n, PS, D), dtype=torch.float16, device=self.device)
        f16 = [(j, pid) for j, pid in enumerate(selected)
               if self.pages[pid].format == PageStorageFormat.FP16 and self.pages[pid].kv_fp16 is not None]
        i8 = [(j, pid) for j, pid in enumerate(selected)
              if self.pages[pid].format == PageStorageFormat.INT8 and self.pages[pid].kv_int8 is not None]
        if f16:
            pos = torch.tensor([j for j, _ in f16], dtype=torch.long, device=self.device)
            src = torch.tensor([p for _, p in f16], dtype=torch.long, device=self.device)
            rows[pos] = self._fp16_pool.index_select(0, src).view(-1, PS, D)
        if i8:
            pos = torch.tensor([j for j, _ in i8], dtype=torch.long, device=self.device)
            src = torch.tensor([p for _, p in i8], dtype=torch.long, device=self.device)
            codes = self._int8_pool.index_select(0, src)
            scales = self._scales.index_select(0, src).half().float()
            deq = torch.empty((len(i8), self._elems), dtype=torch.float16, device=self.device)
            self._transcode(list(range(len(i8))), N.TRANSCODE_PROMOTE_FP16, fp16=deq, int8=codes, scales=scales)
            rows[pos] = deq.view(-1, PS, D)
        for j, pid in enumerate(selected):
            st = self.pages[pid]
            if st.format == PageStorageFormat.SPARSE and st.sp_k_values is not None:
                # all sparse_max_nnz slots, in order; slots past sp_nnz hold (0, 0.0)
                nnz = min(st.sp_nnz, self.sparse_max_nnz)
                idx = st.sp_k_indices[:nnz].tolist() + [0] * (self.sparse_max_nnz - nnz)
                val = st.sp_k_values[:nnz].to(self.device)
                for k, r in enumerate(idx):
                    if 0 <= r < PS:
                        rows[j, r, :] = val[k] if k < nnz else 0
            elif masks and pid in masks and st.format in (PageStorageFormat.FP16, PageStorageFormat.INT8):
                rows[j, ~masks[pid].to(self.device)] = 0
        return rows.view(n * PS, D)

    def _staged_decode(self, query: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
        """Decode over staged rows [T, D]: 16-token FP16 pages of width 64 / 128,
        the last page bounded by the kernel's per-row token count."""
        B, H, D = query.shape
        T = rows.shape[0]
        width = 64 if D <= 64 else 128
        P = (T + 15) // 16
        pages = torch.zeros((P * 16, width), dtype=torch.float16, device=self.device)
        pages[:T, :D] = rows
        pages = pages.view(P, 16, width)
        q = torch.zeros((B, H, width), dtype=query.dtype, device=self.device)
        q[..., :D] = query
        table = torch.arange(P, dtype=torch.int32, device=self.device).expand(B, H, P).contiguous()
        out = paged_decode(q, PagePools(k_fp16=pages, v_fp16=pages), table,
                           torch.full((B, H), P, dtype=torch.int32, device=self.device),
                           torch.zeros(P, dtype=torch.int32, device=self.device),
                           sm_scale=1.0 / math.sqrt(D), out_dtype=torch.float16,
                           valid_tokens=torch.full((B, H), T, dtype=torch.int32, device=self.device))
        return out[..., :D].contiguous()

    def step(self, query: torch.Tensor, demote: bool = False, promote: bool = False, warmup: bool = False,
             adapt: bool = False, mask: bool = False) -> torch.Tensor:
        """One decode step over the selected pages: query [B, H, D] -> [B, H, D] float16.

        Every query head attends every selected page's page_size tokens (K = V =
        the page's rows) with softmax scale 1 / sqrt(head_dim). Pools in the
        kernel layout (16-token pages, head_dim 64 / 128) are decoded in place
        (FP16 and INT8 pages, no SPARSE selected, no masks applied); otherwise
        the rows are staged into 16-token pages first."""
        self.step_count += 1
        if warmup:
            self._prefetch_warmup()
        if demote:
            self.demote_cold_pages()
        if promote:
            self.promote_hot_pages()
        selected, fmts, ids, masks = self.select_pages()
        for pid in selected:
            st = self.pages[pid]
            st.access_count += 1
            st.last_access_step = self.step_count
        self._grow_pool(len(self.pages))
        if query.dim() != 3:
            raise ValueError(f"query must be [B, H, D], got {tuple(query.shape)}")
        B, H, D = query.shape
        if D != self.head_dim:
            raise ValueError(f"query head_dim {D} != {self.head_dim}")
        if D > 128:
            raise ValueError(f"head_dim {D} exceeds the decode kernel's widest (128)")
        query = query.to(self.device)
        if not selected or B * H == 0:
            out = torch.zeros((B, H, D), dtype=torch.float16, device=self.device)
        elif self._kernel_layout() and not (mask and masks) and all(
                self.pages[p].format != PageStorageFormat.SPARSE for p in selected):
            out = self._pool_decode(query, selected, fmts, ids)
        else:
            out = self._staged_decode(query, self._staged_rows(selected, masks if mask else None))
        self._prefetcher.record(selected)
        self._prefetch_predictions = self._prefetcher.predict_next(selected)
        if adapt:
            self._adapt_policy()
        return out

    def predict_prefetch(self) -> List[int]:
        return self._prefetch_predictions

    def page_summary(self) -> Dict:
        fmt_counts = {f.name: 0 for f in PageStorageFormat}
        accesses = cold = 0
        for s in self.pages.values():
            fmt_counts[PageStorageFormat(s.format).name] += 1
            accesses += s.access_count
            since = self.step_count - s.last_access_step if s.last_access_step >= 0 else self.step_count
            cold += since >= self.policy.demote_cold_after_steps
        return {"num_pages": len(self.pages), "step": self.step_count, "format_distribution": fmt_counts,
                "total_accesses": accesses, "cold_pages": cold, "prefetch_predictions": len(self._prefetch_predictions),
                "demote_after_steps": self.policy.demote_cold_after_steps,
                "promote_after_accesses": self.policy.promote_hot_after_accesses}
