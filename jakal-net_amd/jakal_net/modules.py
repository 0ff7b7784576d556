"""Score modules on the native hot path.

Only the low-rank families are hot-path modules:

* ``LowRankBilinearPairwise`` (reference ``src/jakal_net/modules.py:75-100``):
  ``s_ij = (U x_i) . (w_hat * (V x_j)) + b`` with ``w_hat = w / max(||w||, 1e-6)``.
* ``LowRankBilinearRoute`` (reference ``modules.py:415-441``):
  ``l_jk = (w * (Ws src_j)) . (Wt dst_k) + b`` with the raw ``w``.
* ``TemperatureScaledRoute`` (reference ``scripts/progressive_b_example.py:58-68``)
  divides the wrapped route's logits by a fixed temperature.
* ``MultiHeadPairwise`` / ``MultiHeadRoute`` (reference ``modules.py:259-301``,
  ``:470-529``) combine several heads' scores; the native path runs the
  max aggregation over low-rank heads.

Parameter creation order (source projection, target projection, weight, bias)
is the reference's, so a given torch seed yields the same initial parameters.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch
from torch import Tensor, nn


class LowRankBilinearPairwise(nn.Module):
    """Low-rank bilinear pairwise score with a unit-norm core weight."""

    def __init__(self, dim: int, rank: int, *, bias: bool = True) -> None:
        super().__init__()
        if rank <= 0:
            raise ValueError("rank must be positive.")
        self.source_proj = nn.Linear(dim, rank, bias=False)
        self.target_proj = nn.Linear(dim, rank, bias=False)
        self.weight = nn.Parameter(torch.ones(rank))
        self.bias = nn.Parameter(torch.zeros(())) if bias else None

    def normalized_weight(self) -> Tensor:
        return self.weight / self.weight.norm(p=2).clamp_min(1e-6)

    def effective_weight(self) -> Tensor:
        """Dense [dim, dim] matrix M with s_ij = x_i^T M x_j (+ b)."""
        scaled_target = self.target_proj.weight.t() * self.normalized_weight().unsqueeze(0)
        return scaled_target @ self.source_proj.weight

    def forward(self, target_val: Tensor, source_val: Tensor) -> Tensor:
        target = self.target_proj(target_val)
        source = self.source_proj(source_val) * self.normalized_weight()
        scores = target @ source.transpose(-1, -2)
        if self.bias is not None:
            scores = scores + self.bias
        return scores


class LowRankBilinearRoute(nn.Module):
    """Low-rank bilinear route logits from source rows to destination rows."""

    expects_pairwise_inputs = True

    def __init__(self, src_dim: int, dst_dim: int | None = None, *, rank: int, bias: bool = True) -> None:
        super().__init__()
        if rank <= 0:
            raise ValueError("rank must be positive.")
        self.source_proj = nn.Linear(src_dim, rank, bias=False)
        self.target_proj = nn.Linear(src_dim if dst_dim is None else dst_dim, rank, bias=False)
        self.weight = nn.Parameter(torch.ones(rank))
        self.bias = nn.Parameter(torch.zeros(())) if bias else None

    def forward(self, source_val: Tensor, target_val: Tensor) -> Tensor:
        source = self.source_proj(source_val) * self.weight
        target = self.target_proj(target_val)
        logits = source @ target.transpose(-1, -2)
        if self.bias is not None:
            logits = logits + self.bias
        return logits


class TemperatureScaledRoute(nn.Module):
    """Wraps a route module and divides its logits by ``temperature``."""

    def __init__(self, route_fn: nn.Module, temperature: float) -> None:
        super().__init__()
        if temperature <= 0.0:
            raise ValueError("temperature must be positive.")
        self.route_fn = route_fn
        self.temperature = float(temperature)
        self.expects_pairwise_inputs = getattr(route_fn, "expects_pairwise_inputs", False)

    def forward(self, *args: Tensor) -> Tensor:
        return self.route_fn(*args) / self.temperature


PAIRWISE_AGGREGATES = ("max", "mean", "sum", "head_mean", "smoothmax", "signed_smoothmax")
ROUTE_AGGREGATES = ("max", "mean", "sum", "head_mean")


def _combine_heads(scores: list[Tensor], aggregate: str) -> Tensor:
    """Combine per-head scores (reference modules.py:275-301, 497-529).

    max: elementwise maximum; mean: sum / H; sum and head_mean: sum;
    smoothmax: logsumexp - log H; signed_smoothmax: the heads weighted by
    softmax(|s_h|) over the heads."""
    if aggregate == "max":
        out = scores[0]
        for s in scores[1:]:
            out = torch.maximum(out, s)
        return out
    if aggregate in ("smoothmax", "signed_smoothmax"):
        stacked = torch.stack(scores, dim=-1)
        if aggregate == "smoothmax":
            return torch.logsumexp(stacked, dim=-1) - math.log(len(scores))
        return (stacked * torch.softmax(stacked.abs(), dim=-1)).sum(dim=-1)
    out = scores[0]
    for s in scores[1:]:
        out = out + s
    return out / len(scores) if aggregate == "mean" else out


class MultiHeadPairwise(nn.Module):
    """Several pairwise heads combined per pair by ``aggregate``."""

    def __init__(self, heads: Sequence[nn.Module], *, aggregate: str = "max") -> None:
        super().__init__()
        if len(heads) == 0:
            raise ValueError("heads must contain at least one pairwise module.")
        if aggregate not in PAIRWISE_AGGREGATES:
            raise ValueError(f"Unsupported aggregate mode: {aggregate!r}.")
        self.heads = nn.ModuleList(heads)
        self.aggregate = aggregate
        self.num_heads = len(self.heads)

    def head_scores(self, target_val: Tensor, source_val: Tensor) -> Tensor:
        """Per-head scores stacked on a trailing head axis."""
        return torch.stack([head(target_val, source_val) for head in self.heads], dim=-1)

    def forward(self, target_val: Tensor, source_val: Tensor) -> Tensor:
        return _combine_heads([head(target_val, source_val) for head in self.heads], self.aggregate)


class MultiHeadRoute(nn.Module):
    """Several route heads combined per (source, destination) by ``aggregate``."""

    def __init__(self, heads: Sequence[nn.Module], *, aggregate: str = "max") -> None:
        super().__init__()
        if len(heads) == 0:
            raise ValueError("heads must contain at least one route module.")
        if aggregate not in ROUTE_AGGREGATES:
            raise ValueError(f"Unsupported aggregate mode: {aggregate!r}.")
        self.heads = nn.ModuleList(heads)
        self.aggregate = aggregate
        self.num_heads = len(self.heads)
        self.expects_pairwise_inputs = any(getattr(h, "expects_pairwise_inputs", False) for h in self.heads)

    def _head(self, head: nn.Module, source_val: Tensor, target_val: Tensor | None) -> Tensor:
        if getattr(head, "expects_pairwise_inputs", False):
            if target_val is None:
                raise ValueError("target_val is required for MultiHeadRoute heads with pairwise inputs.")
            return head(source_val, target_val)
        return head(source_val)

    def head_logits(self, source_val: Tensor, target_val: Tensor | None = None) -> Tensor:
        """Per-head logits stacked on a trailing head axis."""
        return torch.stack([self._head(h, source_val, target_val) for h in self.heads], dim=-1)

    def forward(self, source_val: Tensor, target_val: Tensor | None = None) -> Tensor:
        return _combine_heads([self._head(h, source_val, target_val) for h in self.heads], self.aggregate)
