"""Host logic of the adaptive-format decode API (no GPU): the reference's
test_triton_adaptive_format_attention.py cases that run on the CPU (enum
values, page-table helper, availability probes) and the device requirement."""
import pytest
import torch

from intent_attention.triton_adaptive_format_attention import (
    AdaptiveFormatKernelConfig, AdaptivePageFormat, adaptive_format_decode_attention_triton, is_cuda_available,
    is_triton_available, make_adaptive_page_tables)


def test_enum_and_config():
    assert [(f.name, f.value) for f in AdaptivePageFormat] == [("FP16", 0), ("INT8", 1), ("SPARSE", 2), ("SKIP", 3)]
    c = AdaptiveFormatKernelConfig()
    assert (c.page_size, c.head_dim, c.max_selected_pages, c.block_d, c.sparse_max_nnz) == (16, 64, 64, 64, 256)
    assert is_triton_available() is False and isinstance(is_cuda_available(), bool)


def test_make_adaptive_page_tables():
    ids, counts = make_adaptive_page_tables(torch.tensor([3, 1, 2], dtype=torch.int32), batch=1, heads=1)
    assert ids.tolist() == [[[3, 1, 2]]] and counts.tolist() == [[3]]
    ids, counts = make_adaptive_page_tables(torch.tensor([0], dtype=torch.int32), batch=2, heads=2,
                                            max_selected_pages=4)
    assert ids.shape == (2, 2, 4) and ids[0, 0].tolist() == [0, -1, -1, -1] and counts[1, 1].item() == 1
    sel = torch.arange(12, dtype=torch.int32).view(2, 3, 2)
    ids, counts = make_adaptive_page_tables(sel, batch=2, heads=3, max_selected_pages=3)
    assert ids[1, 2].tolist() == [10, 11, -1] and counts.tolist() == [[2, 2, 2], [2, 2, 2]]
    with pytest.raises(ValueError):
        make_adaptive_page_tables(torch.zeros(2, 3, 4, 5), batch=2, heads=3)
    with pytest.raises(ValueError):
        make_adaptive_page_tables(torch.zeros(5, dtype=torch.int32), batch=1, heads=1, max_selected_pages=4)
    with pytest.raises(ValueError):
        make_adaptive_page_tables(torch.zeros(2, 2, 3, dtype=torch.int32), batch=2, heads=3)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the error raised without a ROCm device")
def test_needs_a_device():
    q = torch.zeros(1, 1, 64, dtype=torch.float16)
    kv = torch.zeros(2, 16, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA is not available"):
        adaptive_format_decode_attention_triton(q, torch.zeros(1, 1, 64, dtype=torch.int32),
                                                torch.zeros(2, dtype=torch.int32), kv, kv)
