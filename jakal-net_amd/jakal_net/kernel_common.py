"""What the native ops need to know about a score or route module.

The native ops take a module's parameters as a flat positional list (the
pybind signatures of native/jakal_net_native.cpp:5962-6936).  The two spec
records below carry that list for the low-rank modules, which are the only
modules on the hot path (src/jakal_net/kernel_common.py:185-192, 296-306):

* ``LowRankBilinearPairwise``: weight = the normalised core weight w_hat,
  in_weight = V (source projection), out_weight = U (target projection);
* ``LowRankBilinearRoute``, optionally inside a ``TemperatureScaledRoute``:
  source / target projections, the raw core weight w, the bias and the
  temperature.

The compressions and keep-masks of the PyTorch forms are in
``jakal_net.compress``.
"""

from __future__ import annotations

from dataclasses import dataclass

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
    """True for score modules the HIP library computes."""
    return isinstance(pairwise_fn, LowRankBilinearPairwise)


def _route_and_temperature(route_fn: object) -> tuple[object, float]:
    """The route module inside a TemperatureScaledRoute (with its temperature), else (route_fn, 1)."""
    inner = getattr(route_fn, "route_fn", None)
    if inner is None:
        return route_fn, 1.0
    return inner, float(getattr(route_fn, "temperature", 1.0))


def supports_pairwise_route_kernel(route_fn: object) -> bool:
    """True for route modules the HIP library computes."""
    return isinstance(_route_and_temperature(route_fn)[0], LowRankBilinearRoute)


def pairwise_kernel_spec(pairwise_fn: object) -> PairwiseKernelSpec:
    if not isinstance(pairwise_fn, LowRankBilinearPairwise):
        raise TypeError(f"no native kernel spec for a {type(pairwise_fn).__name__} score module.")
    return PairwiseKernelSpec(
        kind="low_rank_bilinear",
        weight=pairwise_fn.normalized_weight(),
        bias=pairwise_fn.bias,
        in_weight=pairwise_fn.source_proj.weight,
        out_weight=pairwise_fn.target_proj.weight,
    )


def pairwise_route_kernel_spec(route_fn: object) -> PairwiseRouteKernelSpec:
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
