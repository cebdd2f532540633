"""MI355X-native selected-quant paged decode (drop-in for the hot path of
manishklach/intent-attention-kernel).

Host-side policy (router, precision policy, kernel metadata) runs on the CPU
as in the reference; the decode itself runs only in libiak.so, the HIP/gfx950
library behind the C ABI in include/iak.h.
"""
from .block_metadata import SELECTED_POLICIES, BlockLayout, BlockPolicy, SemanticBlock
from .block_router import (
    BlockDecision,
    BlockRouter,
    RoutedBlock,
    RouterConfig,
    compute_block_scores,
    routing_to_kernel_metadata,
)
from .fused_selected_quant_decode import (
    FusedDecodeConfig,
    FusedKVPrecision,
    fused_selected_quant_decode,
    fused_selected_quant_decode_reference,
    is_native_available,
    metadata_to_kernel_tensors,
)
from .intent_quant import (
    IntentQuantizer,
    KVPrecision,
    QuantPolicy,
    compute_quant_error,
    fake_dequantize_tensor,
    fake_quantize_tensor,
)
from .intent_quant_decode import (
    IntentQuantKernelConfig,
    TritonKVPrecision,
    fake_int8_pages_from_fp16,
    intent_quant_decode_attention_triton,
    make_page_tables_from_selected_pages,
    make_precision_tensor,
)
from .decode_core import PagePools, make_plan, pack_page_descriptors, paged_decode
from .reference import dense_attention, semantic_block_attention
from .intent_quant_attention import compare_intent_quant_to_fp16_selected, intent_quant_attention_reference
from .mla import MLABlockTable, MLAConfig, absorb_weights, mla_sparse_decode_reference, mla_triton_decode
from .mla_core import LatentPools, mla_paged_decode
from .triton_mla_decode import mla_decode_triton
from .quantize import fake_int8_pages_device, quantize_pages
from .page_tables import build_page_tables, routing_to_kernel_tensors
from .kv_memory_manager import KVMemoryManager, PageFormatPolicy, PageState, PageStorageFormat
from .prefetch import BlockPrefetcher, get_prefetch_stream, get_prefetcher, launch_prefetch_pages, reset_prefetcher
from .triton_adaptive_format_attention import (
    AdaptiveFormatKernelConfig,
    AdaptivePageFormat,
    adaptive_format_decode_attention_reference_dispatch,
    adaptive_format_decode_attention_triton,
    make_adaptive_page_tables,
)

__all__ = [
    "SELECTED_POLICIES", "BlockLayout", "BlockPolicy", "SemanticBlock",
    "BlockDecision", "BlockRouter", "RoutedBlock", "RouterConfig", "compute_block_scores",
    "routing_to_kernel_metadata",
    "FusedDecodeConfig", "FusedKVPrecision", "fused_selected_quant_decode", "fused_selected_quant_decode_reference",
    "is_native_available",
    "metadata_to_kernel_tensors",
    "IntentQuantizer", "KVPrecision", "QuantPolicy", "compute_quant_error", "fake_dequantize_tensor",
    "fake_quantize_tensor",
    "IntentQuantKernelConfig", "TritonKVPrecision", "fake_int8_pages_from_fp16",
    "intent_quant_decode_attention_triton", "make_page_tables_from_selected_pages", "make_precision_tensor",
    "PagePools", "make_plan", "pack_page_descriptors", "paged_decode",
    "dense_attention", "semantic_block_attention", "intent_quant_attention_reference",
    "compare_intent_quant_to_fp16_selected",
    "MLABlockTable", "MLAConfig", "absorb_weights", "mla_sparse_decode_reference", "mla_triton_decode",
    "LatentPools", "mla_paged_decode", "mla_decode_triton",
    "quantize_pages", "fake_int8_pages_device",
    "build_page_tables", "routing_to_kernel_tensors",
    "KVMemoryManager", "PageFormatPolicy", "PageState", "PageStorageFormat",
    "BlockPrefetcher", "get_prefetch_stream", "get_prefetcher", "launch_prefetch_pages", "reset_prefetcher",
    "AdaptiveFormatKernelConfig", "AdaptivePageFormat", "adaptive_format_decode_attention_reference_dispatch",
    "adaptive_format_decode_attention_triton", "make_adaptive_page_tables",
]
