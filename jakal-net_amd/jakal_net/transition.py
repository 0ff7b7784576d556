"""Cross-layer routing: dense ``Transition`` and top-k ``SparseTransition``.

Semantics of the reference operators (src/jakal_net/transition.py):

* route logits ``l[..., j, k] = route_fn(src.val, dst.val)`` for routes that
  take (source, destination) pairs, ``route_fn(src.val)`` otherwise
  (:168-173); with ``use_direction_only`` both value sets are first scaled to
  unit length (:163-166);
* route weights ``p`` per source row over the destinations: softmax,
  signed |l| softmax or signed entmax-1.5 (:187-194); the sparse form keeps
  each *source row's* k best destinations and normalises over those (:439-444);
* sender strength ``rho = state_activation_fn(src.state)`` (softplus);
* ``delta_state[k] = sum_j p_jk rho_j ps_j`` and ``delta_val[k] = sum_j p_jk
  rho_j pv_j`` with ``ps = state_proj_fn(src.state)``, ``pv =
  val_proj_fn(src.val)`` of shape [..., Ns, dst.dim] (:449-451); ``forward``
  merges the delta into ``dst`` (:389-392).

Backends as in ``jakal_net.propagation``; the HIP library takes
``LowRankBilinearRoute`` (optionally temperature-scaled) with any of the
three route compressions.
"""

from __future__ import annotations

import inspect
from typing import Callable

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from jakal_net.compress import ROUTE_COMPRESS_NAMES, compress_routes, topk_keep_mask
from jakal_net.core import (
    ImplementationMode,
    Layer,
    LayerDelta,
    MergeMode,
    accumulation_dtype,
    block_ranges,
    check_implementation,
    check_merge_mode,
    expect_shape,
    finish_layer,
)
from jakal_net.kernel_common import supports_pairwise_route_kernel
from jakal_net.native_backend import (
    native_disabled_by_env,
    native_supports,
    native_supports_device,
    require_native_for_device,
    transition_pairwise_dense_native,
    transition_pairwise_topk_native,
)

_POSITIONAL = (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)


def route_takes_pairs(route_fn: object) -> bool:
    """Whether ``route_fn`` scores (source, destination) pairs: it says so with
    ``expects_pairwise_inputs``, or its call takes two positional arguments."""
    if getattr(route_fn, "expects_pairwise_inputs", False):
        return True
    call = route_fn.forward if isinstance(route_fn, nn.Module) else route_fn
    try:
        params = inspect.signature(call).parameters.values()
    except (TypeError, ValueError):
        return False
    return sum(p.kind in _POSITIONAL for p in params) >= 2


def unit_directions(val: Tensor) -> Tensor:
    """Value rows scaled to unit L2 length (eps 1e-6), NaNs zeroed
    (src/jakal_net/_architectural_common.py:44-45, 227-228)."""
    return F.normalize(torch.nan_to_num(val), p=2.0, dim=-1, eps=1e-6)


def route_statistics(routes: Tensor, topk_index: Tensor | None = None) -> dict[str, float]:
    """Diagnostics of a route matrix [..., Ns, Nd] (reference transition.py:99-121):
    mean row entropy, variance of the per-destination load, the fraction of
    destinations receiving (almost) nothing, and -- for top-k routes -- how
    often a source row's destination also appears among the previous row's."""
    p = routes.clamp_min(1e-12)
    load = routes.sum(dim=-2)
    stats = {
        "entropy": float((-(p * p.log()).sum(dim=-1)).mean()),
        "destination_load_variance": float(load.var(unbiased=False)),
        "dead_slot_ratio": float((load <= 1e-6).float().mean()),
        "topk_overlap": 0.0,
    }
    if topk_index is not None and topk_index.shape[-2] > 1:
        shared = topk_index[..., 1:, :, None] == topk_index[..., :-1, None, :]
        stats["topk_overlap"] = float(shared.any(dim=-1).float().mean())
    return stats


class Transition(nn.Module):
    """Dense cross-layer routing (reference transition.py:124-392)."""

    def __init__(
        self,
        route_fn: Callable[..., Tensor] | nn.Module,
        *,
        norm_fn: Callable[[Layer], Layer] | None = None,
        state_activation_fn: Callable[[Tensor], Tensor] = F.softplus,
        route_compress_name: str = "softmax",
        val_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        state_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        merge_mode: MergeMode = "add",
        implementation: ImplementationMode = "streaming",
        src_block_size: int | None = 128,
        dst_block_size: int | None = 128,
        accumulator_dtype: torch.dtype | None = None,
        use_direction_only: bool = False,
    ) -> None:
        super().__init__()
        check_merge_mode(merge_mode)
        check_implementation(implementation)
        if route_compress_name not in ROUTE_COMPRESS_NAMES:
            raise ValueError(f"route_compress_name must be one of {ROUTE_COMPRESS_NAMES}, got "
                             f"{route_compress_name!r}.")
        self.route_fn = route_fn
        self.norm_fn = norm_fn
        self.state_activation_fn = state_activation_fn
        self.route_compress_name = route_compress_name
        self.val_proj_fn = val_proj_fn if val_proj_fn is not None else nn.Identity()
        self.state_proj_fn = state_proj_fn if state_proj_fn is not None else nn.Identity()
        self.merge_mode = merge_mode
        self.implementation = implementation
        self.src_block_size = src_block_size
        self.dst_block_size = dst_block_size
        self.accumulator_dtype = accumulator_dtype
        self.use_direction_only = use_direction_only
        self.track_stats = False
        self.last_stats: dict[str, float] | None = None
        self._pairs = route_takes_pairs(route_fn)

    # ---- logits, routes and what each source sends ----------------------------
    def _values(self, layer: Layer) -> Tensor:
        return unit_directions(layer.val) if self.use_direction_only else layer.val

    def _logits(self, src_val: Tensor, dst_val: Tensor) -> Tensor:
        return self.route_fn(src_val, dst_val) if self._pairs else self.route_fn(src_val)

    def compute_route_logits(self, src_layer: Layer, dst_layer: Layer) -> Tensor:
        logits = self._logits(self._values(src_layer), self._values(dst_layer))
        expect_shape(logits, (*src_layer.batch_shape, src_layer.num_nodes, dst_layer.num_nodes), "route_fn")
        return logits

    def _keep(self, logits: Tensor, dst_layer: Layer) -> Tensor | None:
        return None

    def _routes(self, logits: Tensor, dst_layer: Layer) -> Tensor:
        return compress_routes(logits, self.route_compress_name, mask=self._keep(logits, dst_layer))

    def compute_routes(self, src_layer: Layer, dst_layer: Layer) -> Tensor:
        logits = self.compute_route_logits(src_layer, dst_layer)
        return self._routes(logits, dst_layer)

    def _sender_terms(self, src_layer: Layer, dst_layer: Layer, src_val: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        """(rho, ps, pv): sender strength, projected state and values per source node."""
        pv = self.val_proj_fn(src_val)
        ps = self.state_proj_fn(src_layer.state)
        rho = self.state_activation_fn(src_layer.state)
        expect_shape(pv, (*src_layer.state.shape, dst_layer.dim), "val_proj_fn")
        expect_shape(ps, src_layer.state.shape, "state_proj_fn")
        expect_shape(rho, src_layer.state.shape, "state_activation_fn")
        return rho, ps, pv

    # ---- PyTorch forms -------------------------------------------------------
    @staticmethod
    def _sums(routes: Tensor, rho: Tensor, ps: Tensor, pv: Tensor) -> tuple[Tensor, Tensor]:
        weighted = routes * rho.unsqueeze(-1)  # [..., Ns, Nd]
        return (weighted * ps.unsqueeze(-1)).sum(dim=-2), weighted.transpose(-1, -2) @ pv

    def _compute_delta_reference(self, src_layer: Layer, dst_layer: Layer) -> LayerDelta:
        src_val = self._values(src_layer)
        logits = self._logits(src_val, self._values(dst_layer))
        expect_shape(logits, (*src_layer.batch_shape, src_layer.num_nodes, dst_layer.num_nodes), "route_fn")
        rho, ps, pv = self._sender_terms(src_layer, dst_layer, src_val)
        ds, dv = self._sums(self._routes(logits, dst_layer), rho, ps, pv)
        return LayerDelta(delta_state=ds, delta_val=dv)

    def _compute_delta_streaming(self, src_layer: Layer, dst_layer: Layer) -> LayerDelta:
        src_val, dst_val = self._values(src_layer), self._values(dst_layer)
        rho, ps, pv = self._sender_terms(src_layer, dst_layer, src_val)
        acc_s = accumulation_dtype(ps.dtype, self.accumulator_dtype)
        acc_v = accumulation_dtype(pv.dtype, self.accumulator_dtype)
        ds = torch.zeros(dst_layer.state.shape, dtype=acc_s, device=dst_layer.state.device)
        dv = torch.zeros(dst_layer.val.shape, dtype=acc_v, device=dst_layer.val.device)
        for s0, s1 in block_ranges(src_layer.num_nodes, self.src_block_size):
            logits = self._logits(src_val[..., s0:s1, :], dst_val)
            expect_shape(logits, (*src_layer.batch_shape, s1 - s0, dst_layer.num_nodes), "route_fn")
            weighted = self._routes(logits, dst_layer) * rho[..., s0:s1].unsqueeze(-1)
            ds = ds + (weighted.to(acc_s) * ps[..., s0:s1].unsqueeze(-1).to(acc_s)).sum(dim=-2)
            dv = dv + weighted.to(acc_v).transpose(-1, -2) @ pv[..., s0:s1, :].to(acc_v)
        return LayerDelta(delta_state=ds.to(ps.dtype), delta_val=dv.to(pv.dtype))

    # ---- the HIP library -----------------------------------------------------
    def _native_op_name(self) -> str:
        return "transition_pairwise_dense"

    def _on_native_path(self) -> bool:
        return self._pairs and supports_pairwise_route_kernel(self.route_fn)

    def _compute_delta_native(self, src_layer: Layer, dst_layer: Layer, *, strict: bool) -> LayerDelta | None:
        """The library's result, or None when this call is not the library's to
        run; strict: a GPU tensor the library cannot take raises instead."""
        if not self._on_native_path() or native_disabled_by_env():
            return None
        op, device_type = self._native_op_name(), src_layer.val.device.type
        if not (native_supports(op) and native_supports_device(device_type)):
            if strict:
                require_native_for_device(op, device_type)
            return None
        # unit directions are taken here, differentiably, and the library
        # scores the normalised values (reference transition.py:665-680)
        src_val, dst_val = self._values(src_layer), self._values(dst_layer)
        rho, ps, pv = self._sender_terms(src_layer, dst_layer, src_val)
        try:
            return self._call_native(src_layer, dst_layer, src_val, dst_val, rho, ps, pv)
        except NotImplementedError:  # outside the library's limits
            if strict:
                raise
            return None

    def _call_native(self, src_layer, dst_layer, src_val, dst_val, rho, ps, pv) -> LayerDelta:
        return transition_pairwise_dense_native(
            route_fn=self.route_fn,
            route_compress_name=self.route_compress_name,
            sender_strength=rho,
            src_val=src_val,
            dst_val=dst_val,
            projected_state=ps,
            projected_val=pv,
            src_block_size=self.src_block_size or src_layer.num_nodes,
            dst_block_size=self.dst_block_size or dst_layer.num_nodes,
        )

    # ---- dispatch ------------------------------------------------------------
    def _statistics(self, src_layer: Layer, dst_layer: Layer) -> dict[str, float]:
        with torch.no_grad():
            return route_statistics(self.compute_routes(src_layer, dst_layer))

    def compute_delta(self, src_layer: Layer, dst_layer: Layer) -> LayerDelta:
        if self.track_stats:
            self.last_stats = self._statistics(src_layer, dst_layer)
        impl = self.implementation
        # native calls stay native under graph capture (the reference's fall
        # back to PyTorch there, transition.py:332-333, 660-661; the HIP ops
        # only launch kernels)
        if impl == "reference":
            return self._compute_delta_reference(src_layer, dst_layer)
        if impl in ("native", "kernel"):
            delta = self._compute_delta_native(src_layer, dst_layer, strict=impl == "native")
            if delta is not None:
                return delta
        return self._compute_delta_streaming(src_layer, dst_layer)

    def forward(self, src_layer: Layer, dst_layer: Layer) -> Layer:
        delta = self.compute_delta(src_layer, dst_layer)
        return finish_layer(dst_layer.apply_delta(delta, self.merge_mode), self.norm_fn)


class SparseTransition(Transition):
    """Per-source top-k routing (reference transition.py:395-721)."""

    def __init__(
        self,
        route_fn: Callable[..., Tensor] | nn.Module,
        *,
        topk: int,
        norm_fn: Callable[[Layer], Layer] | None = None,
        state_activation_fn: Callable[[Tensor], Tensor] = F.softplus,
        route_compress_name: str = "softmax",
        val_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        state_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        merge_mode: MergeMode = "add",
        implementation: ImplementationMode = "streaming",
        src_block_size: int | None = 128,
        dst_block_size: int | None = 128,
        accumulator_dtype: torch.dtype | None = None,
        use_direction_only: bool = False,
    ) -> None:
        super().__init__(
            route_fn,
            norm_fn=norm_fn,
            state_activation_fn=state_activation_fn,
            route_compress_name=route_compress_name,
            val_proj_fn=val_proj_fn,
            state_proj_fn=state_proj_fn,
            merge_mode=merge_mode,
            implementation=implementation,
            src_block_size=src_block_size,
            dst_block_size=dst_block_size,
            accumulator_dtype=accumulator_dtype,
            use_direction_only=use_direction_only,
        )
        if topk < 1:
            raise ValueError(f"topk must be at least 1, got {topk}.")
        self.topk = topk

    def _keep(self, logits: Tensor, dst_layer: Layer) -> Tensor | None:
        if self.topk >= dst_layer.num_nodes:
            return None  # every destination (transition.py:437-440)
        return topk_keep_mask(logits, self.topk, dim=-1)

    def _statistics(self, src_layer: Layer, dst_layer: Layer) -> dict[str, float]:
        with torch.no_grad():
            logits = self.compute_route_logits(src_layer, dst_layer)
            if self.topk >= dst_layer.num_nodes:
                return route_statistics(self._routes(logits, dst_layer))
            best = torch.topk(logits, self.topk, dim=-1)
            routes = torch.zeros_like(logits).scatter_(
                -1, best.indices, compress_routes(best.values, self.route_compress_name))
            return route_statistics(routes, best.indices)

    def _native_op_name(self) -> str:
        return "transition_pairwise_topk"

    def _call_native(self, src_layer, dst_layer, src_val, dst_val, rho, ps, pv) -> LayerDelta:
        return transition_pairwise_topk_native(
            route_fn=self.route_fn,
            sender_strength=rho,
            src_val=src_val,
            dst_val=dst_val,
            projected_state=ps,
            projected_val=pv,
            topk=self.topk,
            src_block_size=self.src_block_size or src_layer.num_nodes,
            dst_block_size=self.dst_block_size or dst_layer.num_nodes,
            route_compress_name=self.route_compress_name,
        )
