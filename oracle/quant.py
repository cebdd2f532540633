"""Oracle: quantisation arithmetic (codes must be bit-exact).

Restates, in numpy, the arithmetic of

  intent_quant.py:221-226   _absmax_scale      scale = clamp(amax|x| / 127, min=1e-8), in x's dtype
  intent_quant.py:229-312   fake_quantize_tensor (FP16 / FP8 / INT8 / INT4 / INT4_RESIDUAL / SKIP)
  fused_selected_quant_decode.py:521-542          fake_int8_pages_from_fp16 (fp16 arithmetic)
  triton_intent_quant_attention.py:460-496        fake_int8_pages_from_fp16 (fp32 arithmetic)

Floating-point model. Every elementwise step of the reference is one IEEE
operation rounded to the dtype torch computes it in: for a float16 tensor
that is the float16 result of the exact operation (torch's CPU half kernels
compute in float32 and round once; float32 carries 24 >= 2*11+2 bits, so that
equals one correctly rounded float16 operation). Here each step is evaluated
exactly in float64 and rounded once to the storage dtype, which is the same
value. ``round`` is round-half-to-even (torch.round). The e4m3fn cast is
round-to-nearest-even with NaN (0x7F | sign) for magnitudes that round above
448, and for NaN inputs.

The page-granule quantisers at the bottom produce the kernel's storage: they
apply fake_quantize_tensor's arithmetic to one page (one KV head) of
``[page_size, D]`` values, exactly as the reference does when its tensor is a
single page (``page.reshape(-1, 1)``: the scale reduces over every element),
or to one 32-channel group of a page for INT4 (``page.view(PS, D//32, 32)
.permute(0, 2, 1).reshape(-1, D//32)``: one scale per group).

Pinned by: torch's own float8_e4m3fn cast over every float16 value
(tests/test_oracle_quant.py), closed-form checks (codes * scale reconstructs,
ties to even, clamps, saturation of INT4 at 7/127 of absmax, the all-zero
page), and golden vectors written by the reference's fake_quantize_tensor and
both fake_int8_pages_from_fp16 variants (tests/golden/).
"""
from __future__ import annotations

from typing import Dict, Tuple

import numpy as np

F16 = np.float16
F32 = np.float32
F64 = np.float64

E4M3_MAX = 448.0


def _r(x, dtype):
    """Round float64 values (exact results) once to ``dtype``."""
    with np.errstate(all="ignore"):
        return np.asarray(x, dtype=F64).astype(dtype)


def _div(a, b, dtype):
    with np.errstate(all="ignore"):
        return _r(np.asarray(a, F64) / np.asarray(b, F64), dtype)


def _mul(a, b, dtype):
    with np.errstate(all="ignore"):
        return _r(np.asarray(a, F64) * np.asarray(b, F64), dtype)


def _sub(a, b, dtype):
    with np.errstate(all="ignore"):
        return _r(np.asarray(a, F64) - np.asarray(b, F64), dtype)


def _add(a, b, dtype):
    with np.errstate(all="ignore"):
        return _r(np.asarray(a, F64) + np.asarray(b, F64), dtype)


def round_half_even(x):
    """torch.round: ties to even (numpy.rint is the same IEEE operation)."""
    with np.errstate(all="ignore"):
        return np.rint(np.asarray(x, F64))


def _clamp(x, lo, hi):
    """torch.clamp on floats: NaN propagates."""
    x = np.asarray(x, F64)
    with np.errstate(all="ignore"):
        return np.where(np.isnan(x), np.nan, np.minimum(np.maximum(x, lo), hi))


def to_int8(x) -> np.ndarray:
    """``.to(torch.int8)`` of values already rounded and clamped to [-128, 127].

    NaN (from a 0/0 on an all-zero block) has no defined integer value in C;
    torch on x86-64 yields 0 for it (cvttss2si returns INT_MIN, whose low byte
    is 0). That single case is mapped to 0 here and flagged by the tests.
    """
    x = np.asarray(x, F64)
    out = np.where(np.isnan(x), 0, x)
    return out.astype(np.int64).astype(np.int8)


# --------------------------------------------------------------------------- #
# e4m3fn (OCP FP8: 1 sign, 4 exponent (bias 7), 3 mantissa; no inf; NaN = S.1111.111)
# --------------------------------------------------------------------------- #


def e4m3fn_encode(x) -> np.ndarray:
    """Round-to-nearest-even cast of real values to e4m3fn codes (uint8).

    Binade [2^e, 2^(e+1)) for e >= -6 has quantum 2^(e-3); below 2^-6 the
    subnormal quantum is 2^-9. A magnitude that rounds above 448 is NaN.
    """
    x = np.asarray(x, F64)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    nan = np.isnan(a)
    a0 = np.where(nan | (a == 0), 1.0, a)
    _, e = np.frexp(a0)                  # a0 = m * 2**e, m in [0.5, 1)
    e = np.maximum(e - 1, -6)            # floor(log2 a), clamped to the subnormal binade
    quantum = np.ldexp(1.0, e - 3)
    n = np.rint(a0 / quantum)            # exact division by a power of two, then RNE
    val = np.where(a == 0, 0.0, n * quantum)
    over = val > E4M3_MAX
    vv = np.where((val == 0) | over | nan, 1.0, val)
    _, e2 = np.frexp(vv)
    e2 = e2 - 1
    sub = e2 < -6
    exp_field = np.where(sub, 0, e2 + 7)
    mant = np.where(sub, vv / 2.0 ** -9, vv / np.ldexp(1.0, e2 - 3) - 8.0)
    code = (exp_field.astype(np.int64) << 3) | mant.astype(np.int64)
    code = np.where(val == 0, 0, code)
    code = np.where(over | nan, 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


def e4m3fn_decode(code) -> np.ndarray:
    """e4m3fn code -> float64 value (NaN for 0x7F / 0xFF)."""
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    ef = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(ef == 0, m * 2.0 ** -9, (8 + m) * np.ldexp(1.0, ef - 7 - 3))
    val = np.where((ef == 0xF) & (m == 0x7), np.nan, val)
    return s * val


# --------------------------------------------------------------------------- #
# fake_quantize_tensor (intent_quant.py:221-312), arithmetic dtype = x.dtype
# --------------------------------------------------------------------------- #


def absmax_scale(x: np.ndarray, dtype) -> Tuple[np.ndarray, np.ndarray]:
    """intent_quant.py:221-226: per last-dim channel absmax over all other dims.

    ``clamp(min=1e-8)``: torch converts the bound to the tensor dtype first; in
    float16 1e-8 becomes 0, so an all-zero channel keeps scale 0 (and its
    quotient 0/0 is NaN), while in float32 the bound is fl32(1e-8).
    """
    x = np.asarray(x, dtype)
    axes = tuple(range(x.ndim - 1))
    amax = np.abs(x).max(axis=axes, keepdims=True).astype(dtype)
    scale = _div(amax, 127.0, dtype)
    lo = float(np.asarray(1e-8, dtype=dtype))
    scale = np.maximum(scale, np.asarray(lo, dtype)).astype(dtype)
    return scale, amax


def fake_quantize_codes(x: np.ndarray, precision: str) -> Dict[str, np.ndarray]:
    """Codes, scales and reconstruction of fake_quantize_tensor(x, precision).

    ``x`` is a float16 or float32 array; its dtype is the arithmetic dtype
    (intent_quant.py:229-312). Returns a dict with ``recon`` (the tensor the
    reference returns) and, per precision, ``codes``/``scale`` and for
    INT4_RESIDUAL ``codes2``/``scale2``.
    """
    dt = x.dtype
    assert dt in (F16, F32), dt
    if precision == "FP16":                                   # :238-239
        return {"recon": x.astype(F16)}
    if precision == "SKIP":                                   # :309-310
        return {"recon": np.zeros_like(x)}
    if precision == "FP8":                                    # :241-244
        scale, _ = absmax_scale(x, dt)
        q = e4m3fn_encode(_div(x, scale, dt))
        recon = _mul(e4m3fn_decode(q), scale.astype(F32), F32)   # q.float() * scale -> fp32
        return {"codes": q, "scale": scale, "recon": recon}
    if precision in ("INT8", "INT4"):                         # :260-265
        max_q = 127 if precision == "INT8" else 7
        scale, _ = absmax_scale(x, dt)
        q = to_int8(round_half_even(_clamp(_div(x, scale, dt), -max_q, max_q)))
        recon = _mul(q.astype(F64), scale.astype(F32), F32)
        return {"codes": q, "scale": scale, "recon": recon}
    if precision == "INT4_RESIDUAL":                          # :282-292
        scale, _ = absmax_scale(x, dt)
        q1 = to_int8(round_half_even(_clamp(_div(x, scale, dt), -7, 7)))
        base = _mul(q1.astype(F64), scale.astype(F32), F32)        # fp32
        resid = _sub(x.astype(F64), base, F32)                      # x - fp32 -> fp32
        s2, _ = absmax_scale(resid, F32)
        q2 = to_int8(round_half_even(_clamp(_div(resid, s2, F32), -7, 7)))
        res_recon = _mul(q2.astype(F64), s2, F32)
        recon = _add(base, res_recon, F32)
        return {"codes": q1, "scale": scale, "codes2": q2, "scale2": s2, "recon": recon}
    raise ValueError(f"Unknown precision: {precision}")


def fake_quantize_tensor(x: np.ndarray, precision: str) -> np.ndarray:
    """The reconstructed tensor returned by intent_quant.py:229-312."""
    return fake_quantize_codes(x, precision)["recon"]


# --------------------------------------------------------------------------- #
# The two fake_int8_pages_from_fp16 functions (same name, different arithmetic)
# --------------------------------------------------------------------------- #


def fake_int8_pages_fused(pages: np.ndarray, eps: float = 1e-6):
    """fused_selected_quant_decode.py:521-542, float16 arithmetic.

    absmax over each flattened page, clamp(min=eps) (eps converted to float16
    by torch's clamp), /127, round half-even, clamp(-128, 127), int8; scales
    float16 [num_pages].
    """
    p = np.asarray(pages, F16).reshape(pages.shape[0], -1)
    amax = np.abs(p).max(axis=1, keepdims=True).astype(F16)
    amax = np.maximum(amax, np.asarray(eps, F16)).astype(F16)
    scales = _div(amax, 127.0, F16)
    q = to_int8(_clamp(round_half_even(_div(p, scales, F16)), -128, 127))
    return q.reshape(pages.shape), scales.reshape(-1)


def fake_int8_pages_triton(pages: np.ndarray, eps: float = 1e-6):
    """triton_intent_quant_attention.py:460-496, float32 arithmetic.

    ``pages.float()``, amax per page, clamp_min(eps), /127, round, clamp(-127, 127);
    scales float32 [num_pages].
    """
    if pages.ndim != 3:
        raise ValueError("pages must have shape [num_pages, page_size, D]")
    p = np.asarray(pages).astype(F32).reshape(pages.shape[0], -1)
    amax = np.abs(p).max(axis=1)
    amax = np.maximum(amax, np.asarray(eps, F32)).astype(F32)
    scales = _div(amax, 127.0, F32)
    q = to_int8(_clamp(round_half_even(_div(p, scales[:, None], F32)), -127, 127))
    return q.reshape(pages.shape), scales.astype(F32)


# --------------------------------------------------------------------------- #
# Page-granule storage quantisers (the kernel's pools)
# --------------------------------------------------------------------------- #

INT4_GROUP = 32


def quantize_page(page: np.ndarray, precision: str, int4_group: int = INT4_GROUP):
    """Codes for ONE page of one KV head, ``page`` = float16 ``[PS, D]``.

    FP8 / INT8 / INT4_RESIDUAL: the scale reduces over the whole page
    (fake_quantize_tensor on ``page.reshape(-1, 1)``). INT4: one scale per
    ``int4_group`` channels (fake_quantize_tensor on the group view).
    Returns (codes, scales) with codes shaped ``[PS, D]`` (int8 / uint8 fp8)
    and scales a 1-D float array: FP8/INT8 -> [1] float16; INT4 -> [D//group]
    float16; INT4_RESIDUAL -> ([1] float16 base, [1] float32 residual) and
    codes (q1, q2).
    """
    page = np.asarray(page, F16)
    PS, D = page.shape
    if precision in ("FP8", "INT8", "INT4_RESIDUAL"):
        r = fake_quantize_codes(page.reshape(-1, 1), precision)
        if precision == "INT4_RESIDUAL":
            return ((r["codes"].reshape(PS, D), r["codes2"].reshape(PS, D)),
                    (r["scale"].reshape(1), r["scale2"].reshape(1)))
        return r["codes"].reshape(PS, D), r["scale"].reshape(1)
    if precision == "INT4":
        g = int4_group
        view = page.reshape(PS, D // g, g).transpose(0, 2, 1).reshape(-1, D // g)
        r = fake_quantize_codes(view, "INT4")
        codes = r["codes"].reshape(PS, g, D // g).transpose(0, 2, 1).reshape(PS, D)
        return codes, r["scale"].reshape(D // g)
    raise ValueError(precision)


def dequantize_page(codes, scales, precision: str, int4_group: int = INT4_GROUP) -> np.ndarray:
    """The reconstruction the reference computes from ``quantize_page``'s codes (float32)."""
    if precision == "FP8":
        return _mul(e4m3fn_decode(codes), np.asarray(scales, F32)[0], F32)
    if precision == "INT8":
        return _mul(np.asarray(codes, F64), np.asarray(scales, F32)[0], F32)
    if precision == "INT4":
        c = np.asarray(codes, F64)
        PS, D = c.shape
        s = np.repeat(np.asarray(scales, F32), int4_group)[None, :]
        return _mul(c, s, F32)
    if precision == "INT4_RESIDUAL":
        (q1, q2), (s1, s2) = codes, scales
        base = _mul(np.asarray(q1, F64), np.asarray(s1, F32)[0], F32)
        res = _mul(np.asarray(q2, F64), np.asarray(s2, F32)[0], F32)
        return _add(base, res, F32)
    raise ValueError(precision)


# Packed INT4 storage: two codes per byte, element 2j in the low nibble and
# 2j+1 in the high nibble of byte j, each nibble holding ``code + 8`` (codes
# are in [-7, 7], so nibbles are 1..15; 0 never occurs).

def pack_int4(codes: np.ndarray) -> np.ndarray:
    c = (np.asarray(codes, np.int16) + 8).astype(np.uint8)
    assert c.shape[-1] % 2 == 0
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    lo = (p & 0xF).astype(np.int16) - 8
    hi = (p >> 4).astype(np.int16) - 8
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


# INT4_RESIDUAL storage: one byte per element, base code + 8 in the low nibble,
# residual code + 8 in the high nibble.

def pack_int4_residual(q1: np.ndarray, q2: np.ndarray) -> np.ndarray:
    a = (np.asarray(q1, np.int16) + 8).astype(np.uint8)
    b = (np.asarray(q2, np.int16) + 8).astype(np.uint8)
    return (a | (b << 4)).astype(np.uint8)


def unpack_int4_residual(packed: np.ndarray):
    p = np.asarray(packed, np.uint8)
    return ((p & 0xF).astype(np.int16) - 8).astype(np.int8), ((p >> 4).astype(np.int16) - 8).astype(np.int8)
