"""CPU oracle for the fused selected-quant paged decode path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the algorithm of
the reference prototype (``manishklach/intent-attention-kernel``) for the one
hot path this repository accelerates: router page selection -> kernel
metadata -> per-page quantised codes -> fused selected-page decode attention
(plus the MLA latent decode variant). Every function cites the reference
``file:line`` it follows (paths are relative to the reference's
``src/intent_attention/``).

Who may use it: ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and only as the checker (or the timed
CPU baseline). The shipped package (``intent-attention-kernel_amd/``) never
imports it; the product path fails loudly when its HIP library is missing.

Modules
-------
policy     BlockPolicy/SemanticBlock/BlockLayout, IntentQuantizer policy,
           BlockRouter.route_layout, routing_to_kernel_metadata,
           metadata_to_kernel_tensors (integer/decision logic; exact).
quant      fake_quantize_tensor arithmetic (fp16 and fp32 variants), the
           e4m3fn encoder, both fake_int8_pages_from_fp16 variants and the
           page-granule quantisers that produce the kernel's storage codes.
decode     fused_selected_quant_decode_reference (loop-faithful) and a
           vectorised restatement with the GQA / native-precision extension.
attention  dense_attention and intent_quant_attention_reference.
mla        _mla_decode_cpu / mla_sparse_decode_reference restatement.

Parity status of each function is recorded in its docstring ("pinned by: ...")
and summarised in the repository's design notes; a function without such a
pin says "parity unpinned".
"""
