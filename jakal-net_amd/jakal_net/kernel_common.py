"""Selection / mask / gather helpers and native kernel specs.

Helper semantics follow the reference's ``src/jakal_net/kernel_common.py``:
``masked_softmax`` (:420-423), ``select_topk`` (:426-430), ``build_topk_mask``
(:433-440), ``causal_window_mask`` (:443-456), ``gather_*_by_indices``
(:510-527) and the spec extractors ``pairwise_kernel_spec`` (:185-192) and
``pairwise_route_kernel_spec`` (:296-306) for the low-rank modules.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from jakal_net.modules import LowRankBilinearPairwise, LowRankBilinearRoute


@dataclass(frozen=True, slots=True)
class PairwiseKernelSpec:
    kind: str
    weight: Tensor
    bias: Tensor | None
    in_weight: Tensor | None = None
    in_bias: Tensor | None = None
    out_weight: Tensor | None = None
    out_bias: Tensor | None = None


@dataclass(frozen=True, slots=True)
class PairwiseRouteKernelSpec:
    kind: str
    source_weight: Tensor | None
    source_bias: Tensor | None
    target_weight: Tensor | None
    target_bias: Tensor | None
    core_weight: Tensor
    bias: Tensor | None
    hidden_weight: Tensor | None = None
    hidden_bias: Tensor | None = None
    out_weight: Tensor | None = None
    out_bias: Tensor | None = None
    temperature: float = 1.0


def supports_pairwise_kernel(pairwise_fn: object) -> bool:
    """True for pairwise modules the native hot path scores on the GPU."""
    return isinstance(pairwise_fn, LowRankBilinearPairwise)


def unwrap_temperature_scaled_route(route_fn: object) -> tuple[object, float]:
    return getattr(route_fn, "route_fn", route_fn), float(getattr(route_fn, "temperature", 1.0))


def supports_pairwise_route_kernel(route_fn: object) -> bool:
    inner, _ = unwrap_temperature_scaled_route(route_fn)
    return isinstance(inner, LowRankBilinearRoute)


def pairwise_kernel_spec(pairwise_fn: object) -> PairwiseKernelSpec:
    if isinstance(pairwise_fn, LowRankBilinearPairwise):
        return PairwiseKernelSpec(
            kind="low_rank_bilinear",
            weight=pairwise_fn.normalized_weight(),
            bias=pairwise_fn.bias,
            in_weight=pairwise_fn.source_proj.weight,
            out_weight=pairwise_fn.target_proj.weight,
        )
    raise TypeError("Unsupported pairwise_fn for native/kernel spec.")


def pairwise_route_kernel_spec(route_fn: object) -> PairwiseRouteKernelSpec:
    inner, temperature = unwrap_temperature_scaled_route(route_fn)
    if isinstance(inner, LowRankBilinearRoute):
        return PairwiseRouteKernelSpec(
            kind="low_rank_bilinear_route",
            source_weight=inner.source_proj.weight,
            source_bias=None,
            target_weight=inner.target_proj.weight,
            target_bias=None,
            core_weight=inner.weight,
            bias=inner.bias,
            temperature=temperature,
        )
    raise TypeError("Unsupported pairwise route_fn for native/kernel spec.")


def masked_softmax(logits: Tensor, mask: Tensor, dim: int = -1) -> Tensor:
    """Softmax over the entries where ``mask`` is true; masked logits get the dtype minimum."""
    floor = torch.finfo(logits.dtype).min
    return torch.softmax(logits.masked_fill(~mask, floor), dim=dim)


def entmax15(logits: Tensor, *, mask: Tensor | None = None) -> Tensor:
    """1.5-entmax over the last dimension (reference kernels.py:155-202):
    masked entries -> min, shift by the max, halve, sort-based threshold."""
    clean = torch.nan_to_num(logits)
    if mask is not None:
        clean = clean.masked_fill(~mask.to(dtype=torch.bool), torch.finfo(clean.dtype).min)
    x = (clean - clean.max(dim=-1, keepdim=True).values) / 2
    srt = torch.sort(x, dim=-1, descending=True).values
    rho = torch.arange(1, x.shape[-1] + 1, device=x.device, dtype=x.dtype)
    mean = srt.cumsum(-1) / rho
    mean_sq = (srt * srt).cumsum(-1) / rho
    delta = torch.clamp((1 - rho * (mean_sq - mean.square())) / rho, min=0)
    tau = mean - torch.sqrt(delta)
    support = (tau <= srt).sum(dim=-1, keepdim=True).clamp_min(1)
    p = torch.clamp(x - tau.gather(-1, support - 1), min=0).square()
    if mask is not None:
        p = p * mask.to(dtype=p.dtype)
    den = p.sum(dim=-1, keepdim=True)
    return torch.where(den > 0, p / den.clamp_min(torch.finfo(p.dtype).eps), torch.zeros_like(p))


def signed_entmax15(logits: Tensor, *, dim: int = -1, mask: Tensor | None = None) -> Tensor:
    """sign(l) * entmax15(|l|) (reference kernels.py:221-237)."""
    if dim != -1:
        raise ValueError("signed_entmax15 supports dim=-1 only.")
    clean = torch.nan_to_num(logits)
    out = torch.sign(clean) * entmax15(clean.abs(), mask=mask)
    if mask is not None:
        out = out * mask.to(dtype=out.dtype)
    return torch.nan_to_num(out)


def select_topk(scores: Tensor, topk: int, *, dim: int = -1) -> torch.return_types.topk:
    if topk <= 0:
        raise ValueError("topk must be positive.")
    return scores.topk(k=min(topk, scores.shape[dim]), dim=dim)


def build_topk_mask(scores: Tensor, topk: int, *, dim: int = -1) -> Tensor:
    if topk <= 0:
        raise ValueError("topk must be positive.")
    if topk >= scores.shape[dim]:
        return torch.ones_like(scores, dtype=torch.bool)
    picked = select_topk(scores, topk, dim=dim).indices
    return torch.zeros_like(scores, dtype=torch.bool).scatter(dim, picked, True)


def causal_window_mask(
    target_start: int,
    target_end: int,
    source_start: int,
    source_end: int,
    window: int,
    *,
    device: torch.device | None = None,
) -> Tensor:
    """``mask[i, j] = (j <= i) and (j >= i - window)`` over the given index ranges."""
    if window < 0:
        raise ValueError("window must be non-negative.")
    t = torch.arange(target_start, target_end, device=device).unsqueeze(-1)
    s = torch.arange(source_start, source_end, device=device).unsqueeze(0)
    return (s <= t) & (s >= t - window)


def gather_state_by_indices(projected_state: Tensor, indices: Tensor) -> Tensor:
    """``out[..., i, e] = projected_state[..., indices[..., i, e]]``."""
    expanded = projected_state.unsqueeze(-2).expand(*projected_state.shape[:-1], indices.shape[-2],
                                                    projected_state.shape[-1])
    return torch.take_along_dim(expanded, indices, dim=-1)


def gather_val_by_indices(projected_val: Tensor, indices: Tensor) -> Tensor:
    """``out[..., i, e, :] = projected_val[..., indices[..., i, e], :]``."""
    dim = projected_val.shape[-1]
    expanded = projected_val.unsqueeze(-3).expand(
        *projected_val.shape[:-2], indices.shape[-2], projected_val.shape[-2], dim
    )
    return torch.take_along_dim(expanded, indices.unsqueeze(-1).expand(*indices.shape, dim), dim=-2)
