"""Import-path alias of the reference's ``triton_intent_quant_attention`` module.

Reference code that does ``from intent_attention.triton_intent_quant_attention
import ...`` keeps working; every name is the HIP-backed implementation in
``intent_quant_decode`` (this build contains no Triton).
"""
from .intent_quant_decode import (  # noqa: F401
    IntentQuantKernelConfig,
    TritonKVPrecision,
    _validate_decode_inputs,
    fake_int8_pages_from_fp16,
    intent_quant_decode_attention_triton,
    is_cuda_available,
    is_triton_available,
    make_page_tables_from_selected_pages,
    make_precision_tensor,
)
