"""Cross-layer routing: dense ``Transition`` and top-k ``SparseTransition``.

Operator semantics follow the reference's ``src/jakal_net/transition.py``:

* route logits ``l = route_fn(src.val, dst.val)`` ([..., Ns, Nd]) for pairwise
  routes, ``route_fn(src.val)`` otherwise (:168-173);
* routes ``p = softmax(l)`` over destinations (:187-194); for the sparse form
  each *source row* keeps its k best destinations and the softmax runs over
  those k only (:439-444);
* sender strength ``rho = state_activation_fn(src.state)`` (softplus by default);
* ``delta_state[k] = sum_j p_jk rho_j ps_j``, ``delta_val[k] = sum_j p_jk rho_j pv_j``
  (:449-451) and ``forward`` adds the delta to ``dst`` (:389-392).

Backends as in ``jakal_net.propagation``: the native path (HIP library) covers
``LowRankBilinearRoute`` (optionally temperature-wrapped) with softmax or signed |l| softmax routes.
"""

from __future__ import annotations

import inspect
from typing import Callable

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from jakal_net.core import (
    ImplementationMode,
    Layer,
    LayerDelta,
    MergeMode,
    apply_optional_layer_fn,
    iter_blocks,
    resolve_accumulator_dtype,
    validate_implementation,
    validate_merge_mode,
    validate_projected_state,
    validate_route_block_logits,
    validate_route_logits,
)
from jakal_net.kernel_common import build_topk_mask, masked_softmax, signed_entmax15, supports_pairwise_route_kernel
from jakal_net.native_backend import (
    native_disabled_by_env,
    native_supports,
    native_supports_device,
    require_native_for_device,
    transition_pairwise_dense_native,
    transition_pairwise_topk_native,
)


def _cuda_graph_capture_active(device_type: str) -> bool:
    if device_type != "cuda":
        return False
    try:
        return bool(torch.cuda.is_current_stream_capturing())
    except Exception:  # noqa: BLE001
        return False


def signed_abs_softmax(logits: Tensor, *, dim: int = -1, mask: Tensor | None = None) -> Tensor:
    """``sign(l) * softmax(|l|)`` over the unmasked entries (reference transition.py:53-67)."""
    clean = torch.nan_to_num(logits)
    signs = torch.sign(clean)
    magnitudes = clean.abs()
    if mask is not None:
        signs = signs * mask.to(dtype=signs.dtype)
        magnitudes = magnitudes.masked_fill(~mask, -torch.inf)
    return torch.nan_to_num(signs * torch.softmax(magnitudes, dim=dim))


def _route_uses_pairwise_inputs(route_fn: object) -> bool:
    if getattr(route_fn, "expects_pairwise_inputs", False):
        return True
    fn = route_fn.forward if isinstance(route_fn, nn.Module) else route_fn
    try:
        params = inspect.signature(fn).parameters.values()
    except (TypeError, ValueError):
        return False
    positional = [
        p for p in params if p.kind in (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)
    ]
    return len(positional) >= 2


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
        validate_merge_mode(merge_mode)
        validate_implementation(implementation)
        if route_compress_name not in {"softmax", "signed_abs_softmax", "signed_entmax15"}:
            raise ValueError(f"Unsupported route_compress_name: {route_compress_name!r}.")
        self.route_fn = route_fn
        self.norm_fn = norm_fn
        self.state_activation_fn = state_activation_fn
        self.route_compress_name = route_compress_name
        self.val_proj_fn = nn.Identity() if val_proj_fn is None else val_proj_fn
        self.state_proj_fn = nn.Identity() if state_proj_fn is None else state_proj_fn
        self.merge_mode = merge_mode
        self.implementation = implementation
        self.src_block_size = src_block_size
        self.dst_block_size = dst_block_size
        self.accumulator_dtype = accumulator_dtype
        self.use_direction_only = use_direction_only
        self.track_stats = False
        self.last_stats: dict[str, float] | None = None
        self._route_expects_pairwise_inputs = _route_uses_pairwise_inputs(route_fn)

    # ---- shared pieces -------------------------------------------------------
    def _directional_val(self, val: Tensor) -> Tensor:
        if not self.use_direction_only:
            return val
        # unit value directions (reference _architectural_common.py:44-45)
        return F.normalize(torch.nan_to_num(val), p=2.0, dim=-1, eps=1e-6)

    def _route_logits(self, src_val: Tensor, dst_val: Tensor) -> Tensor:
        if self._route_expects_pairwise_inputs:
            return self.route_fn(self._directional_val(src_val), self._directional_val(dst_val))
        return self.route_fn(self._directional_val(src_val))

    def compute_route_logits(self, src_layer: Layer, dst_layer: Layer) -> Tensor:
        logits = self._route_logits(src_layer.val, dst_layer.val)
        validate_route_logits(logits, src_layer, dst_layer)
        return logits

    def _compress_routes(self, logits: Tensor, mask: Tensor | None = None) -> Tensor:
        if self.route_compress_name == "signed_abs_softmax":
            return signed_abs_softmax(logits, dim=-1, mask=mask)
        if self.route_compress_name == "signed_entmax15":
            return signed_entmax15(logits, dim=-1, mask=mask)
        if mask is not None:
            return masked_softmax(logits, mask, dim=-1)
        return torch.softmax(logits, dim=-1)

    def compute_routes(self, src_layer: Layer, dst_layer: Layer) -> Tensor:
        return self._compress_routes(self.compute_route_logits(src_layer, dst_layer))

    def _project_inputs(self, src_layer: Layer, dst_layer: Layer) -> tuple[Tensor, Tensor, Tensor]:
        projected_val = self.val_proj_fn(self._directional_val(src_layer.val))
        projected_state = self.state_proj_fn(src_layer.state)
        sender_strength = self.state_activation_fn(src_layer.state)
        expected = (*src_layer.state.shape, dst_layer.dim)
        if tuple(projected_val.shape) != expected:
            raise ValueError(
                f"val_proj_fn must return [..., src_nodes, dst_dim], expected {expected}, "
                f"got {tuple(projected_val.shape)}."
            )
        validate_projected_state(projected_state, src_layer)
        if sender_strength.shape != src_layer.state.shape:
            raise ValueError("state_activation_fn must preserve the src_layer.state shape.")
        return projected_val, projected_state, sender_strength

    def _route_mask(self, logits: Tensor, dst_layer: Layer) -> Tensor | None:
        return None

    def _compute_delta_reference(self, src_layer: Layer, dst_layer: Layer) -> LayerDelta:
        logits = self.compute_route_logits(src_layer, dst_layer)
        routes = self._compress_routes(logits, mask=self._route_mask(logits, dst_layer))
        projected_val, projected_state, sender = self._project_inputs(src_layer, dst_layer)
        weighted = routes * sender.unsqueeze(-1)
        return LayerDelta(
            delta_state=torch.einsum("...jk,...j->...k", weighted, projected_state),
            delta_val=torch.einsum("...jk,...jd->...kd", weighted, projected_val),
        )

    def _compute_delta_streaming(self, src_layer: Layer, dst_layer: Layer) -> LayerDelta:
        projected_val, projected_state, sender = self._project_inputs(src_layer, dst_layer)
        state_dtype = resolve_accumulator_dtype(projected_state.dtype, self.accumulator_dtype)
        val_dtype = resolve_accumulator_dtype(projected_val.dtype, self.accumulator_dtype)
        delta_state = torch.zeros(dst_layer.state.shape, dtype=state_dtype, device=dst_layer.state.device)
        delta_val = torch.zeros(dst_layer.val.shape, dtype=val_dtype, device=dst_layer.val.device)
        for s0, s1 in iter_blocks(src_layer.num_nodes, self.src_block_size, name="src_block_size"):
            logits = self._route_logits(src_layer.val[..., s0:s1, :], dst_layer.val)
            validate_route_block_logits(
                logits, batch_shape=src_layer.batch_shape, source_nodes=s1 - s0, dst_nodes=dst_layer.num_nodes
            )
            routes = self._compress_routes(logits, mask=self._route_mask(logits, dst_layer))
            weighted = routes * sender[..., s0:s1].unsqueeze(-1)
            delta_state = delta_state + torch.einsum(
                "...jk,...j->...k", weighted.to(state_dtype), projected_state[..., s0:s1].to(state_dtype)
            )
            delta_val = delta_val + torch.einsum(
                "...jk,...jd->...kd", weighted.to(val_dtype), projected_val[..., s0:s1, :].to(val_dtype)
            )
        return LayerDelta(delta_state=delta_state.to(projected_state.dtype), delta_val=delta_val.to(projected_val.dtype))

    # ---- native dispatch -----------------------------------------------------
    def _native_op_name(self) -> str:
        return "transition_pairwise_dense"

    def _hot_path(self) -> bool:
        # the HIP dense route covers softmax and signed |l| softmax routes
        return (
            self._route_expects_pairwise_inputs
            and supports_pairwise_route_kernel(self.route_fn)
            and self.route_compress_name in ("softmax", "signed_abs_softmax", "signed_entmax15")
            and not self.use_direction_only
        )

    def _try_native(self, src_layer: Layer, dst_layer: Layer, *, strict: bool) -> LayerDelta | None:
        if not self._hot_path() or native_disabled_by_env():
            return None
        device_type = src_layer.val.device.type
        op = self._native_op_name()
        if native_supports(op) and native_supports_device(device_type):
            projected_val, projected_state, sender = self._project_inputs(src_layer, dst_layer)
            return self._call_native(src_layer, dst_layer, projected_val, projected_state, sender)
        if strict:
            require_native_for_device(op, device_type)
        return None

    def _call_native(self, src_layer, dst_layer, projected_val, projected_state, sender) -> LayerDelta:
        return transition_pairwise_dense_native(
            route_fn=self.route_fn,
            route_compress_name=self.route_compress_name,
            sender_strength=sender,
            src_val=src_layer.val,
            dst_val=dst_layer.val,
            projected_state=projected_state,
            projected_val=projected_val,
            src_block_size=self.src_block_size or src_layer.num_nodes,
            dst_block_size=self.dst_block_size or dst_layer.num_nodes,
        )

    def compute_delta(self, src_layer: Layer, dst_layer: Layer) -> LayerDelta:
        if self.track_stats:
            self.last_stats = self._route_stats(src_layer, dst_layer)
        impl = self.implementation
        if impl == "native" and _cuda_graph_capture_active(src_layer.val.device.type):
            return self._compute_delta_reference(src_layer, dst_layer)
        if impl == "reference":
            return self._compute_delta_reference(src_layer, dst_layer)
        if impl in ("native", "kernel"):
            delta = self._try_native(src_layer, dst_layer, strict=(impl == "native"))
            if delta is not None:
                return delta
        return self._compute_delta_streaming(src_layer, dst_layer)

    def _route_stats(self, src_layer: Layer, dst_layer: Layer) -> dict[str, float]:
        with torch.no_grad():
            logits = self.compute_route_logits(src_layer, dst_layer)
            routes = self._compress_routes(logits, mask=self._route_mask(logits, dst_layer))
            probs = routes.clamp_min(1e-12)
            load = routes.sum(dim=-2)
            return {
                "entropy": float(-(probs * probs.log()).sum(dim=-1).mean().item()),
                "destination_load_variance": float(load.var(unbiased=False).item()),
                "dead_slot_ratio": float(1.0 - (load > 1e-6).float().mean().item()),
            }

    def forward(self, src_layer: Layer, dst_layer: Layer) -> Layer:
        delta = self.compute_delta(src_layer, dst_layer)
        return apply_optional_layer_fn(dst_layer.apply_delta(delta, merge_mode=self.merge_mode), self.norm_fn)


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
            route_fn=route_fn,
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
        if topk <= 0:
            raise ValueError("topk must be positive.")
        self.topk = topk

    def _route_mask(self, logits: Tensor, dst_layer: Layer) -> Tensor | None:
        k = min(self.topk, dst_layer.num_nodes)
        if k == dst_layer.num_nodes:
            return None
        return build_topk_mask(logits, k, dim=-1)

    def _native_op_name(self) -> str:
        return "transition_pairwise_topk"

    def _hot_path(self) -> bool:
        # the HIP top-k route also covers signed |l| softmax routes
        return (
            self._route_expects_pairwise_inputs
            and supports_pairwise_route_kernel(self.route_fn)
            and self.route_compress_name in ("softmax", "signed_abs_softmax", "signed_entmax15")
            and not self.use_direction_only
        )

    def _call_native(self, src_layer, dst_layer, projected_val, projected_state, sender) -> LayerDelta:
        return transition_pairwise_topk_native(
            route_fn=self.route_fn,
            sender_strength=sender,
            src_val=src_layer.val,
            dst_val=dst_layer.val,
            projected_state=projected_state,
            projected_val=projected_val,
            topk=self.topk,
            src_block_size=self.src_block_size or src_layer.num_nodes,
            dst_block_size=self.dst_block_size or dst_layer.num_nodes,
            route_compress_name=self.route_compress_name,
        )
