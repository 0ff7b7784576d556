"""Same-layer message passing: dense ``Propagation`` and ``SparsePropagation``.

Operator semantics follow the reference's ``src/jakal_net/propagation.py``:

* scores ``s = pairwise_fn(val, val)`` over all (target i, source j) pairs;
* dense: ``e = compress(s)``; window: ``e = compress(s)`` on ``i-w <= j <= i``
  (:459-470); top-k: ``e = compress(s)`` on the k best sources of each target
  (:471), all other edges zero;
* ``delta_state = e @ projected_state``, ``delta_val = e @ projected_val``
  (:473-479), or with ``state_weight_edges`` the edges are multiplied by
  ``softplus(state_j)`` and ``delta_state = sum_j e`` (:474-478).

Backends (``implementation=``):

* ``"reference"`` -- dense masked PyTorch form (reference :207-220, :453-480);
* ``"streaming"`` -- blockwise PyTorch over target blocks;
* ``"native"``    -- the HIP library through ``jakal_net_native`` for the hot-path
  configuration (``LowRankBilinearPairwise`` with softsign or signed_abs_softmax
  edges).  On a GPU tensor a missing or disabled library is an error, never a
  silent CPU/PyTorch fallback.  Configurations outside the hot path (custom
  score callables, other compress functions) run the streaming path, as the
  reference runs them in its Python kernel backend;
* ``"kernel"``    -- the native op when it is available for the device, else streaming.
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from jakal_net.core import (
    ImplementationMode,
    Layer,
    LayerDelta,
    SparsePropagationType,
    apply_optional_layer_fn,
    iter_blocks,
    resolve_accumulator_dtype,
    validate_implementation,
    validate_pairwise_block_scores,
    validate_pairwise_scores,
    validate_projected_state,
    validate_projected_val,
)
from jakal_net.kernel_common import build_topk_mask, causal_window_mask, signed_entmax15, supports_pairwise_kernel
from jakal_net.native_backend import (
    native_disabled_by_env,
    native_supports,
    native_supports_device,
    propagation_dense_native,
    propagation_topk_native,
    propagation_window_native,
    require_native_for_device,
)


def _cuda_graph_capture_active(device_type: str) -> bool:
    if device_type != "cuda":
        return False
    try:
        return bool(torch.cuda.is_current_stream_capturing())
    except Exception:  # noqa: BLE001
        return False


def edge_compress_name(edge_compress_fn: Callable[[Tensor], Tensor]) -> str | None:
    """Canonical name of a compress function (reference propagation.py:56-64)."""
    name = getattr(edge_compress_fn, "__name__", "")
    if edge_compress_fn is F.softsign or name == "softsign":
        return "softsign"
    if name in {"signed_abs_softmax", "signed_abs_softmax_edges", "_signed_abs_softmax_edges"}:
        return "signed_abs_softmax"
    if name in {"signed_entmax15", "_signed_entmax15_edges"}:
        return "signed_entmax15"
    return None


_NATIVE_EDGE_COMPRESS = ("softsign", "signed_abs_softmax", "signed_entmax15")


def compress_edges(scores: Tensor, edge_compress_fn: Callable[[Tensor], Tensor], *, mask: Tensor | None = None) -> Tensor:
    """Apply the edge compression; masked edges are exactly zero.

    ``signed_abs_softmax`` normalises over the unmasked entries only
    (reference propagation.py:67-88)."""
    if edge_compress_name(edge_compress_fn) == "signed_abs_softmax":
        clean = torch.nan_to_num(scores)
        signs = torch.sign(clean)
        magnitudes = clean.abs()
        if mask is not None:
            signs = signs * mask.to(dtype=signs.dtype)
            magnitudes = magnitudes.masked_fill(~mask, -torch.inf)
        return torch.nan_to_num(signs * torch.softmax(magnitudes, dim=-1))
    if edge_compress_name(edge_compress_fn) == "signed_entmax15":
        return signed_entmax15(scores, mask=mask)
    edges = edge_compress_fn(scores)
    if mask is not None:
        edges = edges * mask.to(dtype=edges.dtype)
    return edges


class Propagation(nn.Module):
    """Dense same-layer propagation (reference propagation.py:108-404)."""

    def __init__(
        self,
        pairwise_fn: Callable[[Tensor, Tensor], Tensor] | nn.Module,
        *,
        edge_compress_fn: Callable[[Tensor], Tensor] = F.softsign,
        val_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        state_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        norm_fn: Callable[[Layer], Layer] | None = None,
        residual: bool = True,
        return_delta: bool = True,
        state_weight_edges: bool = False,
        implementation: ImplementationMode = "streaming",
        target_block_size: int | None = 128,
        source_block_size: int | None = 128,
        accumulator_dtype: torch.dtype | None = None,
        use_direction_only: bool = False,
    ) -> None:
        super().__init__()
        validate_implementation(implementation)
        self.pairwise_fn = pairwise_fn
        self.edge_compress_fn = edge_compress_fn
        self.val_proj_fn = nn.Identity() if val_proj_fn is None else val_proj_fn
        self.state_proj_fn = nn.Identity() if state_proj_fn is None else state_proj_fn
        self.norm_fn = norm_fn
        self.residual = residual
        self.return_delta = return_delta
        self.state_weight_edges = state_weight_edges
        self.implementation = implementation
        self.target_block_size = target_block_size
        self.source_block_size = source_block_size
        self.accumulator_dtype = accumulator_dtype
        self.use_direction_only = use_direction_only

    # ---- shared pieces -------------------------------------------------------
    def compute_scores(self, layer: Layer) -> Tensor:
        scores = self.pairwise_fn(layer.val, layer.val)
        validate_pairwise_scores(scores, layer)
        return scores

    def compute_edges(self, layer: Layer) -> Tensor:
        return self.edge_compress_fn(self.compute_scores(layer))

    def _edge_source_strength(self, source_state: Tensor) -> Tensor:
        return F.softplus(source_state)

    def _project_inputs(self, layer: Layer) -> tuple[Tensor, Tensor]:
        projected_state = self.state_proj_fn(layer.state)
        projected_val = self.val_proj_fn(layer.val)
        validate_projected_state(projected_state, layer)
        validate_projected_val(projected_val, layer)
        return projected_state, projected_val

    def _aggregation_inputs(self, layer: Layer) -> tuple[Tensor, Tensor]:
        """(per-source state weight, per-source value) so that delta = e @ each.

        With ``state_weight_edges`` the source strength softplus(state_j) is
        folded into both (reference propagation.py:165-174)."""
        projected_state, projected_val = self._project_inputs(layer)
        if not self.state_weight_edges:
            return projected_state, projected_val
        strength = self._edge_source_strength(layer.state)
        return strength, projected_val * strength.unsqueeze(-1)

    def _edge_mask(self, scores: Tensor, layer: Layer, target_start: int, target_end: int) -> Tensor | None:
        return None

    def _compute_delta_reference(self, layer: Layer) -> LayerDelta:
        scores = self.compute_scores(layer)
        mask = self._edge_mask(scores, layer, 0, layer.num_nodes)
        edges = compress_edges(scores, self.edge_compress_fn, mask=mask)
        weights, values = self._aggregation_inputs(layer)
        delta_state = torch.einsum("...ij,...j->...i", edges, weights)
        delta_val = torch.einsum("...ij,...jd->...id", edges, values)
        return LayerDelta(delta_state=delta_state, delta_val=delta_val)

    def _source_range(self, layer: Layer, target_start: int, target_end: int) -> tuple[int, int]:
        return 0, layer.num_nodes

    def _compute_delta_streaming(self, layer: Layer) -> LayerDelta:
        weights, values = self._aggregation_inputs(layer)
        state_dtype = resolve_accumulator_dtype(weights.dtype, self.accumulator_dtype)
        val_dtype = resolve_accumulator_dtype(values.dtype, self.accumulator_dtype)
        state_parts: list[Tensor] = []
        val_parts: list[Tensor] = []
        for t0, t1 in iter_blocks(layer.num_nodes, self.target_block_size, name="target_block_size"):
            s0, s1 = self._source_range(layer, t0, t1)
            scores = self.pairwise_fn(layer.val[..., t0:t1, :], layer.val[..., s0:s1, :])
            validate_pairwise_block_scores(
                scores, batch_shape=layer.batch_shape, target_nodes=t1 - t0, source_nodes=s1 - s0
            )
            mask = self._block_mask(scores, layer, t0, t1, s0, s1)
            edges = compress_edges(scores, self.edge_compress_fn, mask=mask)
            state_parts.append(
                torch.einsum("...ij,...j->...i", edges.to(state_dtype), weights[..., s0:s1].to(state_dtype))
            )
            val_parts.append(
                torch.einsum("...ij,...jd->...id", edges.to(val_dtype), values[..., s0:s1, :].to(val_dtype))
            )
        return LayerDelta(
            delta_state=torch.cat(state_parts, dim=-1).to(weights.dtype),
            delta_val=torch.cat(val_parts, dim=-2).to(values.dtype),
        )

    def _block_mask(self, scores: Tensor, layer: Layer, t0: int, t1: int, s0: int, s1: int) -> Tensor | None:
        return None

    # ---- native dispatch -----------------------------------------------------
    def _native_op_name(self) -> str:
        return "propagation_dense"

    def _hot_path_config(self) -> str | None:
        """Compress name when this operator is on the native hot path, else None."""
        name = edge_compress_name(self.edge_compress_fn)
        if name in _NATIVE_EDGE_COMPRESS and supports_pairwise_kernel(self.pairwise_fn):
            return name
        return None

    def _try_native(self, layer: Layer, *, strict: bool) -> LayerDelta | None:
        compress = self._hot_path_config()
        if compress is None or native_disabled_by_env():
            return None
        device_type = layer.val.device.type
        op = self._native_op_name()
        if native_supports(op) and native_supports_device(device_type):
            weights, values = self._aggregation_inputs(layer)
            return self._call_native(compress, layer, weights, values)
        if strict:
            require_native_for_device(op, device_type)
        return None

    def _call_native(self, compress: str, layer: Layer, weights: Tensor, values: Tensor) -> LayerDelta:
        return propagation_dense_native(
            pairwise_fn=self.pairwise_fn,
            edge_compress_name=compress,
            layer_val=layer.val,
            projected_state=weights,
            projected_val=values,
            source_state=None,
            target_block_size=self.target_block_size or layer.num_nodes,
            source_block_size=self.source_block_size or layer.num_nodes,
        )

    def compute_delta(self, layer: Layer) -> LayerDelta:
        impl = self.implementation
        if impl == "native" and _cuda_graph_capture_active(layer.val.device.type):
            return self._compute_delta_reference(layer)
        if impl == "reference":
            return self._compute_delta_reference(layer)
        if impl in ("native", "kernel"):
            delta = self._try_native(layer, strict=(impl == "native"))
            if delta is not None:
                return delta
        return self._compute_delta_streaming(layer)

    def forward(self, layer: Layer) -> LayerDelta | Layer:
        delta = self.compute_delta(layer)
        if self.return_delta:
            return delta
        updated = layer.apply_delta(delta, merge_mode="add" if self.residual else "replace")
        return apply_optional_layer_fn(updated, self.norm_fn)


class SparsePropagation(Propagation):
    """Window or top-k same-layer propagation (reference propagation.py:407-829)."""

    def __init__(
        self,
        pairwise_fn: Callable[[Tensor, Tensor], Tensor] | nn.Module,
        *,
        sparse_type: SparsePropagationType,
        edge_compress_fn: Callable[[Tensor], Tensor] = F.softsign,
        topk: int | None = None,
        window: int | None = None,
        val_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        state_proj_fn: Callable[[Tensor], Tensor] | nn.Module | None = None,
        norm_fn: Callable[[Layer], Layer] | None = None,
        residual: bool = True,
        return_delta: bool = True,
        state_weight_edges: bool = False,
        implementation: ImplementationMode = "streaming",
        target_block_size: int | None = 128,
        source_block_size: int | None = 128,
        accumulator_dtype: torch.dtype | None = None,
        use_direction_only: bool = False,
    ) -> None:
        super().__init__(
            pairwise_fn=pairwise_fn,
            edge_compress_fn=edge_compress_fn,
            val_proj_fn=val_proj_fn,
            state_proj_fn=state_proj_fn,
            norm_fn=norm_fn,
            residual=residual,
            return_delta=return_delta,
            state_weight_edges=state_weight_edges,
            implementation=implementation,
            target_block_size=target_block_size,
            source_block_size=source_block_size,
            accumulator_dtype=accumulator_dtype,
            use_direction_only=use_direction_only,
        )
        if sparse_type not in ("window", "topk"):
            raise ValueError(f"Unsupported sparse_type: {sparse_type!r}.")
        if sparse_type == "window" and window is None:
            raise ValueError("window sparse propagation requires window.")
        if sparse_type == "topk" and topk is None:
            raise ValueError("topk sparse propagation requires topk.")
        self.sparse_type = sparse_type
        self.topk = topk
        self.window = window

    def _edge_mask(self, scores: Tensor, layer: Layer, target_start: int, target_end: int) -> Tensor | None:
        if self.sparse_type == "window":
            mask = causal_window_mask(0, layer.num_nodes, 0, layer.num_nodes, self.window or 0, device=scores.device)
            return mask.view((1,) * (scores.ndim - 2) + tuple(mask.shape))
        return build_topk_mask(scores, self.topk or layer.num_nodes)

    def _source_range(self, layer: Layer, target_start: int, target_end: int) -> tuple[int, int]:
        if self.sparse_type == "window":
            return max(0, target_start - (self.window or 0)), target_end
        return 0, layer.num_nodes

    def _block_mask(self, scores: Tensor, layer: Layer, t0: int, t1: int, s0: int, s1: int) -> Tensor | None:
        if self.sparse_type == "window":
            mask = causal_window_mask(t0, t1, s0, s1, self.window or 0, device=scores.device)
            return mask.view((1,) * (scores.ndim - 2) + tuple(mask.shape))
        # each target block sees every source, so a row-wise top-k mask is exact
        return build_topk_mask(scores, self.topk or layer.num_nodes)

    def _native_op_name(self) -> str:
        if self.sparse_type == "window":
            return "propagation_window"
        return "propagation_topk"

    def _call_native(self, compress: str, layer: Layer, weights: Tensor, values: Tensor) -> LayerDelta:
        tbs = self.target_block_size or layer.num_nodes
        sbs = self.source_block_size or layer.num_nodes
        if self.sparse_type == "window":
            return propagation_window_native(
                pairwise_fn=self.pairwise_fn,
                edge_compress_name=compress,
                layer_val=layer.val,
                projected_state=weights,
                projected_val=values,
                window=self.window or 0,
                target_block_size=tbs,
                source_block_size=sbs,
            )
        return propagation_topk_native(
            pairwise_fn=self.pairwise_fn,
            edge_compress_name=compress,
            layer_val=layer.val,
            projected_state=weights,
            projected_val=values,
            topk=self.topk or layer.num_nodes,
            target_block_size=tbs,
            source_block_size=sbs,
        )
