"""What the native ops need to know about a score or route module.

The native ops take a module's parameters as a flat positional list (the
pybind signatures of native/jakal_net_native.cpp:5962-6936).  The two spec
records below carry that list for the low-rank modules, which are the only
modules on the hot path (src/jakal_net/kernel_common.py:185-192, 296-306):

* ``LowRankBilinearPairwise``: weight = the normalised core weight w_hat,
  in_weight = V (source projection), out_weight = U (target projection);
* ``LowRankBilinearRoute``, optionally inside a ``TemperatureScaledRoute``:
  source / target projections, the raw core weight w, the bias and the
  temperature;
* ``MultiHeadPairwise`` / ``MultiHeadRoute`` with ``aggregate="max"`` over
  such heads: kind ``"multihead_max_" + the head kind`` and every field
  stacked over the heads on a leading axis (kernel_common.py:152-178,
  :240-270).  Heads must agree in shape and in whether they carry a bias.
  The route heads share one temperature; the spec's temperature is the
  product of an outer ``TemperatureScaledRoute``'s and the heads' own, which
  is what the module computes.

The compressions and keep-masks of the PyTorch forms are in
``jakal_net.compress``.
"""

from __future__ import annotations

from dataclasses import dataclass

from torch import Tensor

import torch

from jakal_net.modules import LowRankBilinearPairwise, LowRankBilinearRoute, MultiHeadPairwise, MultiHeadRoute


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


def _same_head_shapes(heads: list) -> bool:
    shapes = {(h.source_proj.weight.shape, h.target_proj.weight.shape, h.bias is None) for h in heads}
    return len(shapes) == 1


def _pairwise_heads(pairwise_fn: object) -> list[LowRankBilinearPairwise] | None:
    """The low-rank heads of a max-aggregated MultiHeadPairwise the library computes, else None."""
    if not isinstance(pairwise_fn, MultiHeadPairwise) or pairwise_fn.aggregate != "max":
        return None
    heads = list(pairwise_fn.heads)
    if not heads or not all(isinstance(h, LowRankBilinearPairwise) for h in heads) or not _same_head_shapes(heads):
        return None
    return heads


def supports_pairwise_kernel(pairwise_fn: object) -> bool:
    """True for score modules the HIP library computes."""
    return isinstance(pairwise_fn, LowRankBilinearPairwise) or _pairwise_heads(pairwise_fn) is not None


def _route_and_temperature(route_fn: object) -> tuple[object, float]:
    """The route module inside a TemperatureScaledRoute (with its temperature), else (route_fn, 1)."""
    inner = getattr(route_fn, "route_fn", None)
    if inner is None:
        return route_fn, 1.0
    return inner, float(getattr(route_fn, "temperature", 1.0))


def _route_heads(route_fn: object) -> tuple[list[LowRankBilinearRoute], float] | None:
    """(low-rank heads, temperature) of a max-aggregated MultiHeadRoute the library computes, else None."""
    inner, outer_temperature = _route_and_temperature(route_fn)
    if not isinstance(inner, MultiHeadRoute) or inner.aggregate != "max" or len(inner.heads) == 0:
        return None
    unwrapped = [_route_and_temperature(h) for h in inner.heads]
    heads = [r for r, _ in unwrapped]
    temperatures = {t for _, t in unwrapped}
    if not all(isinstance(h, LowRankBilinearRoute) for h in heads) or len(temperatures) != 1:
        return None
    if not _same_head_shapes(heads):
        return None
    return heads, outer_temperature * temperatures.pop()


def supports_pairwise_route_kernel(route_fn: object) -> bool:
    """True for route modules the HIP library computes."""
    return isinstance(_route_and_temperature(route_fn)[0], LowRankBilinearRoute) or _route_heads(route_fn) is not None


def _stack(values: list) -> torch.Tensor | None:
    return None if values[0] is None else torch.stack(values)


def pairwise_kernel_spec(pairwise_fn: object, unit_scale=None) -> PairwiseKernelSpec:
    """The kernel arguments of a score module.  unit_scale, when given, maps a
    raw [r] weight or [H, r] stack to w / max(||w||, 1e-6) per row (the native
    module's fused op); otherwise each module's normalized_weight() is used."""
    heads = _pairwise_heads(pairwise_fn)
    if heads is not None:
        weight = (torch.stack([h.normalized_weight() for h in heads]) if unit_scale is None
                  else unit_scale(torch.stack([h.weight for h in heads])))
        return PairwiseKernelSpec(
            kind="multihead_max_low_rank_bilinear",
            weight=weight,
            bias=_stack([h.bias for h in heads]),
            in_weight=_stack([h.source_proj.weight for h in heads]),
            out_weight=_stack([h.target_proj.weight for h in heads]),
        )
    if not isinstance(pairwise_fn, LowRankBilinearPairwise):
        raise TypeError(f"no native kernel spec for a {type(pairwise_fn).__name__} score module.")
    return PairwiseKernelSpec(
        kind="low_rank_bilinear",
        weight=pairwise_fn.normalized_weight() if unit_scale is None else unit_scale(pairwise_fn.weight),
        bias=pairwise_fn.bias,
        in_weight=pairwise_fn.source_proj.weight,
        out_weight=pairwise_fn.target_proj.weight,
    )


def pairwise_route_kernel_spec(route_fn: object) -> PairwiseRouteKernelSpec:
    multi = _route_heads(route_fn)
    if multi is not None:
        heads, temperature = multi
        specs = [pairwise_route_kernel_spec(h) for h in heads]
        return PairwiseRouteKernelSpec(
            kind="multihead_max_low_rank_bilinear_route",
            source_weight=_stack([p.source_weight for p in specs]),
            source_bias=None,
            target_weight=_stack([p.target_weight for p in specs]),
            target_bias=None,
            core_weight=_stack([p.core_weight for p in specs]),
            bias=_stack([p.bias for p in specs]),
            temperature=temperature,
        )
    route, temperature = _route_and_temperature(route_fn)
    if not isinstance(route, LowRankBilinearRoute):
        raise TypeError(f"no native kernel spec for a {type(route).__name__} route module.")
    return PairwiseRouteKernelSpec(
        kind="low_rank_bilinear_route",
        source_weight=route.source_proj.weight,
        source_bias=None,
        target_weight=route.target_proj.weight,
        target_bias=None,
        core_weight=route.weight,
        bias=route.bias,
        temperature=temperature,
    )
