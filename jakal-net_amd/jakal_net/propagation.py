"""Same-layer message passing: dense ``Propagation`` and ``SparsePropagation``.

Semantics of the reference operators (src/jakal_net/propagation.py):

* scores ``s[..., i, j] = pairwise_fn(val, val)`` for target i and source j;
* dense: every pair is an edge; window: the sources ``i - window <= j <= i``
  (:459-470); top-k: the k best sources of each target (:471);
* edge weights ``e = compress(s)`` on the kept pairs, 0 elsewhere;
* ``delta_state[i] = sum_j e_ij ps_j`` and ``delta_val[i] = sum_j e_ij pv_j``
  with ``ps = state_proj_fn(state)``, ``pv = val_proj_fn(val)`` (:473-479);
  with ``state_weight_edges`` every edge is scaled by ``softplus(state_j)``
  and ``delta_state[i] = sum_j e_ij`` (:474-478).

``implementation=``:

* ``"reference"`` -- the dense masked PyTorch form (:207-220, :453-480);
* ``"streaming"`` -- the same math over blocks of target rows;
* ``"native"`` -- the HIP library (``jakal_net_native``) for the hot-path
  configuration: ``LowRankBilinearPairwise`` with softsign,
  signed_abs_softmax or signed_entmax15 edges.  For GPU tensors a missing or
  disabled library, or a shape outside the library's limits, raises; other
  configurations (custom score callables or compressions) run the streaming
  form, as the reference runs them in its PyTorch backends;
* ``"kernel"`` -- the HIP library when it accepts the call, else streaming.
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from jakal_net.compress import compress_edges, edge_compress_name, topk_keep_mask, window_keep_mask
from jakal_net.core import (
    ImplementationMode,
    Layer,
    LayerDelta,
    SparsePropagationType,
    accumulation_dtype,
    block_ranges,
    check_implementation,
    expect_shape,
    finish_layer,
)
from jakal_net.kernel_common import supports_pairwise_kernel
from jakal_net.native_backend import (
    native_disabled_by_env,
    native_supports,
    native_supports_device,
    propagation_dense_native,
    propagation_topk_native,
    propagation_window_native,
    require_native_for_device,
)

NATIVE_EDGE_COMPRESSIONS = ("softsign", "signed_abs_softmax", "signed_entmax15")


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
        check_implementation(implementation)
        self.pairwise_fn = pairwise_fn
        self.edge_compress_fn = edge_compress_fn
        self.val_proj_fn = val_proj_fn if val_proj_fn is not None else nn.Identity()
        self.state_proj_fn = state_proj_fn if state_proj_fn is not None else nn.Identity()
        self.norm_fn = norm_fn
        self.residual = residual
        self.return_delta = return_delta
        self.state_weight_edges = state_weight_edges
        self.implementation = implementation
        self.target_block_size = target_block_size
        self.source_block_size = source_block_size
        self.accumulator_dtype = accumulator_dtype
        # kept for the constructor contract; same-layer scores use the values as they are
        self.use_direction_only = use_direction_only

    # ---- scores, edges and what each source carries --------------------------
    def compute_scores(self, layer: Layer) -> Tensor:
        scores = self.pairwise_fn(layer.val, layer.val)
        expect_shape(scores, (*layer.batch_shape, layer.num_nodes, layer.num_nodes), "pairwise_fn")
        return scores

    def compute_edges(self, layer: Layer) -> Tensor:
        return self.edge_compress_fn(self.compute_scores(layer))

    def _source_terms(self, layer: Layer) -> tuple[Tensor, Tensor]:
        """(w, v) per source node such that delta_state = e @ w and delta_val = e @ v."""
        state = self.state_proj_fn(layer.state)
        val = self.val_proj_fn(layer.val)
        expect_shape(state, layer.state.shape, "state_proj_fn")
        expect_shape(val, layer.val.shape, "val_proj_fn")
        if not self.state_weight_edges:
            return state, val
        strength = F.softplus(layer.state)  # edge scale softplus(state_j), reference propagation.py:157-174
        return strength, val * strength.unsqueeze(-1)

    # the kept pairs of target rows t0..t1 and source columns s0..s1 (None: all)
    def _keep(self, scores: Tensor, layer: Layer, t0: int, t1: int, s0: int, s1: int) -> Tensor | None:
        return None

    # the source columns target rows t0..t1 can reach
    def _source_span(self, layer: Layer, t0: int, t1: int) -> tuple[int, int]:
        return 0, layer.num_nodes

    # ---- PyTorch forms -------------------------------------------------------
    def _delta_from_scores(self, scores: Tensor, keep: Tensor | None, w: Tensor, v: Tensor,
                           acc: tuple[torch.dtype, torch.dtype] | None = None) -> tuple[Tensor, Tensor]:
        edges = compress_edges(scores, self.edge_compress_fn, mask=keep)
        if acc is None:
            return (edges * w.unsqueeze(-2)).sum(-1), edges @ v
        ds, dv = acc
        return (edges.to(ds) * w.unsqueeze(-2).to(ds)).sum(-1), edges.to(dv) @ v.to(dv)

    def _compute_delta_reference(self, layer: Layer) -> LayerDelta:
        n = layer.num_nodes
        scores = self.compute_scores(layer)
        w, v = self._source_terms(layer)
        ds, dv = self._delta_from_scores(scores, self._keep(scores, layer, 0, n, 0, n), w, v)
        return LayerDelta(delta_state=ds, delta_val=dv)

    def _compute_delta_streaming(self, layer: Layer) -> LayerDelta:
        w, v = self._source_terms(layer)
        acc = (accumulation_dtype(w.dtype, self.accumulator_dtype), accumulation_dtype(v.dtype, self.accumulator_dtype))
        parts_s, parts_v = [], []
        for t0, t1 in block_ranges(layer.num_nodes, self.target_block_size):
            s0, s1 = self._source_span(layer, t0, t1)
            scores = self.pairwise_fn(layer.val[..., t0:t1, :], layer.val[..., s0:s1, :])
            expect_shape(scores, (*layer.batch_shape, t1 - t0, s1 - s0), "pairwise_fn")
            ds, dv = self._delta_from_scores(scores, self._keep(scores, layer, t0, t1, s0, s1), w[..., s0:s1],
                                             v[..., s0:s1, :], acc)
            parts_s.append(ds)
            parts_v.append(dv)
        return LayerDelta(delta_state=torch.cat(parts_s, dim=-1).to(w.dtype),
                          delta_val=torch.cat(parts_v, dim=-2).to(v.dtype))

    # ---- the HIP library -----------------------------------------------------
    def _native_op_name(self) -> str:
        return "propagation_dense"

    def _native_compression(self) -> str | None:
        """The compression's name when this operator is on the native hot path, else None."""
        name = edge_compress_name(self.edge_compress_fn)
        if name in NATIVE_EDGE_COMPRESSIONS and supports_pairwise_kernel(self.pairwise_fn):
            return name
        return None

    def _compute_delta_native(self, layer: Layer, *, strict: bool) -> LayerDelta | None:
        """The library's result, or None when this call is not the library's to run.

        strict (implementation="native"): a GPU tensor the library cannot take
        raises instead of returning None."""
        compress = self._native_compression()
        if compress is None or native_disabled_by_env():
            return None
        op, device_type = self._native_op_name(), layer.val.device.type
        if not (native_supports(op) and native_supports_device(device_type)):
            if strict:
                require_native_for_device(op, device_type)
            return None
        w, v = self._source_terms(layer)
        try:
            return self._call_native(compress, layer, w, v)
        except NotImplementedError:  # outside the library's limits (k, rank, widths)
            if strict:
                raise
            return None

    def _call_native(self, compress: str, layer: Layer, w: Tensor, v: Tensor) -> LayerDelta:
        return propagation_dense_native(
            pairwise_fn=self.pairwise_fn,
            edge_compress_name=compress,
            layer_val=layer.val,
            projected_state=w,
            projected_val=v,
            source_state=None,
            target_block_size=self.target_block_size or layer.num_nodes,
            source_block_size=self.source_block_size or layer.num_nodes,
        )

    # ---- dispatch ------------------------------------------------------------
    def compute_delta(self, layer: Layer) -> LayerDelta:
        impl = self.implementation
        # The reference sends native calls made under graph capture to its
        # PyTorch form (propagation.py:356-357, 775-776).  The HIP ops launch
        # kernels only (no allocation, synchronisation or memset inside the
        # library), so a captured step keeps them.
        if impl == "reference":
            return self._compute_delta_reference(layer)
        if impl in ("native", "kernel"):
            delta = self._compute_delta_native(layer, strict=impl == "native")
            if delta is not None:
                return delta
        return self._compute_delta_streaming(layer)

    def forward(self, layer: Layer) -> LayerDelta | Layer:
        delta = self.compute_delta(layer)
        if self.return_delta:
            return delta
        return finish_layer(layer.apply_delta(delta, "add" if self.residual else "replace"), self.norm_fn)


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
            pairwise_fn,
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
        needed = {"topk": topk, "window": window}
        if sparse_type not in needed:
            raise ValueError(f"sparse_type must be 'window' or 'topk', got {sparse_type!r}.")
        if needed[sparse_type] is None:
            raise ValueError(f"sparse_type={sparse_type!r} needs the {sparse_type} argument.")
        self.sparse_type = sparse_type
        self.topk = topk
        self.window = window

    def _keep(self, scores: Tensor, layer: Layer, t0: int, t1: int, s0: int, s1: int) -> Tensor | None:
        if self.sparse_type == "window":
            return window_keep_mask(t0, t1, s0, s1, self.window or 0, device=scores.device)
        # every block of target rows sees all sources, so the row-wise top-k is exact
        return topk_keep_mask(scores, self.topk or layer.num_nodes)

    def _source_span(self, layer: Layer, t0: int, t1: int) -> tuple[int, int]:
        if self.sparse_type == "window":
            return max(0, t0 - (self.window or 0)), t1
        return 0, layer.num_nodes

    def _native_op_name(self) -> str:
        return "propagation_window" if self.sparse_type == "window" else "propagation_topk"

    def _call_native(self, compress: str, layer: Layer, w: Tensor, v: Tensor) -> LayerDelta:
        common = dict(
            pairwise_fn=self.pairwise_fn,
            edge_compress_name=compress,
            layer_val=layer.val,
            projected_state=w,
            projected_val=v,
            target_block_size=self.target_block_size or layer.num_nodes,
            source_block_size=self.source_block_size or layer.num_nodes,
        )
        if self.sparse_type == "window":
            return propagation_window_native(window=self.window or 0, **common)
        return propagation_topk_native(topk=self.topk or layer.num_nodes, **common)
