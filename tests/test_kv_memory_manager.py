"""Host logic of the KV memory manager and the block prefetcher (no GPU).

Mirrors the reference's tests/test_kv_memory_manager.py (enum values, page
state, policy defaults, partial-page masks) and tests/test_prefetch.py
(BlockPrefetcher), plus the device requirement: the manager keeps its pages on
a ROCm device, and asking for a host one raises.
"""
import pytest
import torch

from intent_attention.block_metadata import BlockPolicy
from intent_attention.kv_memory_manager import (KVMemoryManager, PageFormatPolicy, PageState, PageStorageFormat,
                                                _format_for_block, _page_page_mask)
from intent_attention.prefetch import BlockPrefetcher, get_prefetcher, launch_prefetch_pages, reset_prefetcher


def test_enum_values_are_stable():
    assert [f.value for f in PageStorageFormat] == [0, 1, 2, 3]
    assert [f.name for f in PageStorageFormat] == ["FP16", "INT8", "SPARSE", "SKIP"]


def test_page_state_defaults_and_coercion():
    assert PageState(page_id=0).format == PageStorageFormat.FP16
    assert PageState(page_id=0, format=PageStorageFormat.INT8).format == PageStorageFormat.INT8
    assert PageState(page_id=0, format=2).format == PageStorageFormat.SPARSE


def test_policy_defaults():
    p = PageFormatPolicy()
    assert p.always_format == PageStorageFormat.FP16 and p.skip_format == PageStorageFormat.SKIP
    assert p.attend_low_format == PageStorageFormat.INT8
    assert (p.demote_cold_after_steps, p.promote_hot_after_accesses) == (10, 3)
    assert (p.demote_step_min, p.demote_step_max, p.promote_access_min, p.promote_access_max) == (2, 50, 1, 20)


def test_format_for_block():
    cfg = PageFormatPolicy()
    assert _format_for_block("ALWAYS", 0.0, cfg) == PageStorageFormat.FP16
    assert _format_for_block(BlockPolicy.SKIP.value, 0.0, cfg) == PageStorageFormat.SKIP
    assert _format_for_block("ATTEND", 0.5, cfg) == PageStorageFormat.FP16      # score >= threshold
    assert _format_for_block("ATTEND", 0.49, cfg) == PageStorageFormat.INT8
    assert _format_for_block("unknown", 1.0, cfg) == PageStorageFormat.INT8     # falls to attend_low


@pytest.mark.parametrize("start,end,lo,hi", [(0, 16, 0, 16), (4, 16, 4, 16), (0, 12, 0, 12), (4, 12, 4, 12),
                                             (20, 26, 4, 10), (30, 40, 14, 16)])
def test_page_page_mask(start, end, lo, hi):
    m = _page_page_mask(16, start, end)
    want = torch.zeros(16, dtype=torch.bool)
    want[lo:hi] = True
    assert torch.equal(m, want)


def test_manager_needs_a_rocm_device():
    with pytest.raises(RuntimeError, match="ROCm device"):
        KVMemoryManager(num_pages=4, page_size=4, head_dim=16, device="cpu")


def test_block_prefetcher():
    p = BlockPrefetcher(history_size=4, min_frequency=3)
    assert p.predict_next([1, 2, 3]) == []
    p.record([1])
    assert p.predict_next([1]) == []
    p.reset()
    for s in ([1, 2], [1, 3], [1, 4]):
        p.record(s)
    assert p.predict_next([1, 5]) == [1]
    p.reset()
    for _ in range(3):
        p.record([3, 1, 2])
    assert p.predict_next([3, 1, 2]) == [1, 2, 3]
    # the window is the last history_size steps plus the current one
    q = BlockPrefetcher(history_size=2, min_frequency=3)
    for s in ([7], [7], [8], [8]):
        q.record(s)
    assert q.predict_next([8]) == [8]
    reset_prefetcher()
    assert get_prefetcher().predict_next([1]) == []


def test_prefetch_is_a_no_op_on_host_tensors():
    k = torch.zeros(1, 1, 32, 16, dtype=torch.float16)
    assert launch_prefetch_pages(k, k, torch.tensor([0, 1])) is None
