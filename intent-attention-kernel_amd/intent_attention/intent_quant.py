"""Precision policy and fake-quantisation arithmetic.

Interface of the reference's intent_quant.py: ``KVPrecision`` (:14-20),
``_BYTES_PER_VALUE`` (:23-30), ``QuantPolicy`` (:33-48), ``IntentQuantizer``
(:51-213) and ``fake_quantize_tensor`` / ``fake_dequantize_tensor`` /
``compute_quant_error`` (:221-340).

The precision policy is expressed as ordered rule tables (first matching rule
wins); it yields the same decision as the reference's branch tree for every
(policy, score, pressure) input. The fake-quant arithmetic is the reference's
(absmax / 127 per last-dim channel in the input dtype, round half-even,
clamp to 127 or 7) written with torch ops that keep true division on every
device: a division by a Python scalar becomes a multiplication by its
reciprocal on GPU tensors, so the divisor is passed as a tensor.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import auto
from typing import Any, Callable, Dict, List, Sequence, Tuple

import torch

from ._enum import StrEnum
from .block_metadata import BlockLayout, BlockPolicy, SemanticBlock


class KVPrecision(StrEnum):
    FP16 = auto()
    FP8 = auto()
    INT8 = auto()
    INT4 = auto()
    INT4_RESIDUAL = auto()
    SKIP = auto()


_BYTES_PER_VALUE: Dict[KVPrecision, float] = {
    KVPrecision.FP16: 2.0, KVPrecision.FP8: 1.0, KVPrecision.INT8: 1.0,
    KVPrecision.INT4: 0.5, KVPrecision.INT4_RESIDUAL: 1.0, KVPrecision.SKIP: 0.0,
}

_SCALED = frozenset({KVPrecision.INT8, KVPrecision.INT4, KVPrecision.INT4_RESIDUAL})


@dataclass
class QuantPolicy:
    precision: KVPrecision
    reason: str = ""
    estimated_bytes_per_value: float = field(init=False)
    requires_scale: bool = field(init=False)
    uses_residual: bool = field(init=False)

    def __post_init__(self) -> None:
        self.estimated_bytes_per_value = _BYTES_PER_VALUE[self.precision]
        self.requires_scale = self.precision in _SCALED
        self.uses_residual = self.precision == KVPrecision.INT4_RESIDUAL


# A rule is (predicate(quantizer, score, pressure), precision, reason).
_Rule = Tuple[Callable[[Any, Any, float], bool], KVPrecision, str]
P = KVPrecision

_ALWAYS_RULES: Sequence[_Rule] = (
    (lambda s, sc, mp: mp > 0.9, P.INT8, "always, extreme pressure"),
    (lambda s, sc, mp: mp > 0.7, P.FP8, "always, high pressure"),
    (lambda s, sc, mp: True, P.FP16, "always, full precision"),
)
_GLOBAL_PRESERVED_RULES: Sequence[_Rule] = (
    (lambda s, sc, mp: mp > 0.8, P.INT8, "global, extreme pressure"),
    (lambda s, sc, mp: True, P.FP16, "global, preserved"),
)
_RECENT_RULES: Sequence[_Rule] = (
    (lambda s, sc, mp: s.preserve_recent and mp > 0.8, P.INT8, "recent, extreme pressure"),
    (lambda s, sc, mp: s.preserve_recent and mp > 0.5, P.FP8, "recent, moderate pressure"),
    (lambda s, sc, mp: s.preserve_recent, P.FP8, "recent, preserved"),
    (lambda s, sc, mp: mp > 0.6, P.INT4_RESIDUAL, "recent, high pressure, not preserved"),
    (lambda s, sc, mp: True, P.INT8, "recent, not preserved"),
)
_ATTEND_RULES: Sequence[_Rule] = (
    (lambda s, sc, mp: sc is None and mp > 0.5, P.INT8, "attend, no score"),
    (lambda s, sc, mp: sc is None, P.FP16, "attend, no score"),
    (lambda s, sc, mp: sc >= s.high_score_threshold and mp > 0.8, P.INT8, "high-score, extreme pressure"),
    (lambda s, sc, mp: sc >= s.high_score_threshold and mp > 0.5, P.FP8, "high-score, moderate pressure"),
    (lambda s, sc, mp: sc >= s.high_score_threshold, P.INT8, "high-score attend"),
    (lambda s, sc, mp: sc >= s.medium_score_threshold and mp > 0.6, P.INT4, "medium-score, high pressure"),
    (lambda s, sc, mp: sc >= s.medium_score_threshold, P.INT4_RESIDUAL, "medium-score attend"),
    (lambda s, sc, mp: mp > 0.3, P.SKIP, "low-score, pressure"),
    (lambda s, sc, mp: True, P.INT4, "low-score attend"),
)


class IntentQuantizer:
    """Mixed-precision policy from block policy, score and memory pressure."""

    def __init__(self, memory_pressure: float = 0.0, preserve_recent: bool = True,
                 preserve_global: bool = True, high_score_threshold: float = 0.75,
                 medium_score_threshold: float = 0.40) -> None:
        if not 0.0 <= memory_pressure <= 1.0:
            raise ValueError(f"memory_pressure must be in [0, 1], got {memory_pressure}")
        self.memory_pressure = memory_pressure
        self.preserve_recent = preserve_recent
        self.preserve_global = preserve_global
        self.high_score_threshold = high_score_threshold
        self.medium_score_threshold = medium_score_threshold

    def _rules(self, pol: BlockPolicy) -> Sequence[_Rule]:
        if pol == BlockPolicy.GLOBAL and self.preserve_global:
            return _GLOBAL_PRESERVED_RULES
        if pol in (BlockPolicy.ALWAYS, BlockPolicy.GLOBAL):
            return _ALWAYS_RULES
        if pol == BlockPolicy.RECENT:
            return _RECENT_RULES
        if pol == BlockPolicy.ATTEND:
            return _ATTEND_RULES
        if pol == BlockPolicy.SKIP:
            return ((lambda s, sc, mp: True, P.SKIP, "skipped block"),)
        return ((lambda s, sc, mp: True, P.FP16, "default"),)

    def assign_block_precision(self, block: SemanticBlock) -> QuantPolicy:
        mp = self.memory_pressure
        for pred, prec, reason in self._rules(block.policy):
            if pred(self, block.score, mp):
                return QuantPolicy(prec, reason)
        raise AssertionError("rule tables end with a catch-all")

    def assign_layout_precision(self, layout: BlockLayout) -> Dict[str, QuantPolicy]:
        return {b.name: self.assign_block_precision(b) for b in layout.blocks}

    def estimate_layout_bytes(self, layout: BlockLayout, heads: int, head_dim: int,
                              kv_tensors: int = 2) -> Dict[str, Any]:
        pols = self.assign_layout_precision(layout)
        dense, quant, fp16_tok = 0, 0.0, 0
        dist: Dict[str, int] = {}
        for b in layout.blocks:
            pol, n = pols[b.name], b.end - b.start
            dense += kv_tensors * n * head_dim * 2
            quant += kv_tensors * n * head_dim * pol.estimated_bytes_per_value
            dist[pol.precision.value] = dist.get(pol.precision.value, 0) + n
            fp16_tok += n if pol.precision == KVPrecision.FP16 else 0
        pct = (1.0 - quant / dense) * 100.0 if dense > 0 else 0.0
        return {"total_tokens": layout.total_token_count(), "dense_fp16_bytes": dense,
                "intent_quant_bytes": int(round(quant)), "bytes_saved": int(round(dense - quant)),
                "bytes_saved_pct": round(pct, 2), "precision_distribution": dist,
                "critical_full_precision_tokens": fp16_tok}

    def summary_table(self, layout: BlockLayout, heads: int, head_dim: int) -> List[Dict[str, Any]]:
        pols = self.assign_layout_precision(layout)
        rows = []
        for b in layout.blocks:
            pol, n = pols[b.name], b.end - b.start
            rows.append({"block": b.name, "policy": b.policy.value, "score": b.score, "tokens": n,
                         "precision": pol.precision.value, "reason": pol.reason,
                         "dense_fp16_bytes": 2 * n * head_dim * 2,
                         "quant_bytes": int(round(2 * n * head_dim * pol.estimated_bytes_per_value))})
        return rows


# --------------------------------------------------------------------------- #
# Fake quantisation (the reference's numerics, any device)
# --------------------------------------------------------------------------- #

def _tdiv(x: torch.Tensor, c: float) -> torch.Tensor:
    """x / c with a true division on every device (see module docstring)."""
    return x / torch.full((1,), c, dtype=x.dtype, device=x.device)


def _absmax_scale(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    absmax = x.abs().amax(dim=tuple(range(x.ndim - 1)), keepdim=True)
    return _tdiv(absmax, 127.0).clamp(min=1e-8), absmax


def _metrics(x: torch.Tensor, recon: torch.Tensor) -> Dict[str, float]:
    err = (x - recon).float()
    return {"mse": float(err.pow(2).mean()), "max_abs_error": float(err.abs().max()),
            "cosine_similarity": float(torch.nn.functional.cosine_similarity(
                x.flatten().unsqueeze(0), recon.flatten().unsqueeze(0)).item())}


def fake_quantize_tensor(x: torch.Tensor, precision: KVPrecision) -> Tuple[torch.Tensor, Dict[str, Any]]:
    """Reconstruction and metadata of a symmetric absmax fake quantisation."""
    if precision == KVPrecision.FP16:
        return x.half(), {"precision": "fp16", "scale": None}
    if precision == KVPrecision.SKIP:
        return torch.zeros_like(x), {"precision": "skip"}
    if precision == KVPrecision.FP8:
        scale, absmax = _absmax_scale(x)
        recon = (x / scale).to(torch.float8_e4m3fn).float() * scale
        return recon, {"precision": "fp8", "scale": scale, "absmax": absmax, **_metrics(x, recon)}
    if precision in (KVPrecision.INT8, KVPrecision.INT4):
        bits = 8 if precision == KVPrecision.INT8 else 4
        qmax = (1 << (bits - 1)) - 1
        scale, absmax = _absmax_scale(x)
        recon = (x / scale).clamp(-qmax, qmax).round().to(torch.int8).float() * scale
        return recon, {"precision": precision.value, "n_bits": bits, "scale": scale, "absmax": absmax,
                       **_metrics(x, recon)}
    if precision == KVPrecision.INT4_RESIDUAL:
        scale, absmax = _absmax_scale(x)
        base = (x / scale).clamp(-7, 7).round().to(torch.int8).float() * scale
        resid = x - base
        rscale, _ = _absmax_scale(resid)
        recon = base + (resid / rscale).clamp(-7, 7).round().to(torch.int8).float() * rscale
        return recon, {"precision": "int4_residual", "scale": scale, "residual_scale": rscale,
                       "absmax": absmax, **_metrics(x, recon)}
    raise ValueError(f"Unknown precision: {precision}")


def fake_dequantize_tensor(qx: torch.Tensor, metadata: Dict[str, Any]) -> torch.Tensor:
    """Identity: fake_quantize_tensor already returns the reconstruction."""
    return qx


def compute_quant_error(original: torch.Tensor, reconstructed: torch.Tensor) -> Dict[str, float]:
    return _metrics(original, reconstructed)
