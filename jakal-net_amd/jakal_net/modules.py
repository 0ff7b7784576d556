"""Score modules on the native hot path.

Only the low-rank families are hot-path modules:

* ``LowRankBilinearPairwise`` (reference ``src/jakal_net/modules.py:75-100``):
  ``s_ij = (U x_i) . (w_hat * (V x_j)) + b`` with ``w_hat = w / max(||w||, 1e-6)``.
* ``LowRankBilinearRoute`` (reference ``modules.py:415-441``):
  ``l_jk = (w * (Ws src_j)) . (Wt dst_k) + b`` with the raw ``w``.
* ``TemperatureScaledRoute`` (reference ``scripts/progressive_b_example.py:58-68``)
  divides the wrapped route's logits by a fixed temperature.

Parameter creation order (source projection, target projection, weight, bias)
is the reference's, so a given torch seed yields the same initial parameters.
"""

from __future__ import annotations

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
