"""Layer containers and shape helpers of the Jakal-Net operator API.

Public surface follows the reference's ``src/jakal_net/core.py:9-260``: a
``Layer`` is a per-node scalar ``state [..., N]`` plus a value vector
``val [..., N, D]``; operators return a ``LayerDelta`` that ``apply_delta``
adds to (or substitutes for) a layer.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterator, Literal

import torch
from torch import Tensor

MergeMode = Literal["add", "replace"]
SparsePropagationType = Literal["window", "topk"]
ImplementationMode = Literal["reference", "streaming", "kernel", "native"]

_MERGE_MODES = ("add", "replace")
_IMPLEMENTATIONS = ("reference", "streaming", "kernel", "native")


@dataclass(frozen=True, slots=True)
class BlockSpan:
    """Half-open index range ``[start, end)`` (reference core.py:14-27)."""

    start: int
    end: int

    def __post_init__(self) -> None:
        if self.start < 0:
            raise ValueError("BlockSpan.start must be non-negative.")
        if self.end < self.start:
            raise ValueError("BlockSpan.end must be greater than or equal to start.")

    @property
    def size(self) -> int:
        return self.end - self.start


@dataclass(slots=True)
class LayerDelta:
    """Update produced by an operator (reference core.py:30-50)."""

    delta_state: Tensor
    delta_val: Tensor

    def __post_init__(self) -> None:
        if self.delta_state.ndim < 1:
            raise ValueError("delta_state must end with the node dimension.")
        if self.delta_val.ndim < 2:
            raise ValueError("delta_val must end with [num_nodes, dim].")
        if tuple(self.delta_val.shape[:-1]) != tuple(self.delta_state.shape):
            raise ValueError("delta_val must match delta_state on every dimension except value dim.")

    @classmethod
    def zeros_like(cls, layer: "Layer") -> "LayerDelta":
        return cls(delta_state=torch.zeros_like(layer.state), delta_val=torch.zeros_like(layer.val))


@dataclass(slots=True)
class Layer:
    """Graph layer: ``state [..., N]`` and ``val [..., N, dim]`` (reference core.py:53-131)."""

    dim: int
    num_nodes: int
    state: Tensor
    val: Tensor

    def __post_init__(self) -> None:
        if self.dim <= 0:
            raise ValueError("dim must be positive.")
        if self.num_nodes <= 0:
            raise ValueError("num_nodes must be positive.")
        if self.state.ndim < 1:
            raise ValueError("state must end with [num_nodes].")
        if self.val.ndim < 2:
            raise ValueError("val must end with [num_nodes, dim].")
        if self.state.shape[-1] != self.num_nodes:
            raise ValueError(f"state.shape[-1] must be {self.num_nodes}, got {self.state.shape[-1]}.")
        if self.val.shape[-2] != self.num_nodes:
            raise ValueError(f"val.shape[-2] must be {self.num_nodes}, got {self.val.shape[-2]}.")
        if self.val.shape[-1] != self.dim:
            raise ValueError(f"val.shape[-1] must be {self.dim}, got {self.val.shape[-1]}.")
        if tuple(self.val.shape[:-1]) != tuple(self.state.shape):
            raise ValueError("val must match state on every dimension except the trailing value dim.")

    @classmethod
    def zeros(
        cls,
        dim: int,
        num_nodes: int,
        batch_shape: tuple[int, ...] = (),
        *,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> "Layer":
        shape = (*batch_shape, num_nodes)
        return cls(
            dim=dim,
            num_nodes=num_nodes,
            state=torch.zeros(shape, device=device, dtype=dtype),
            val=torch.zeros((*shape, dim), device=device, dtype=dtype),
        )

    @property
    def batch_shape(self) -> torch.Size:
        return self.state.shape[:-1]

    def clone(self) -> "Layer":
        return Layer(dim=self.dim, num_nodes=self.num_nodes, state=self.state.clone(), val=self.val.clone())

    def with_tensors(self, *, state: Tensor | None = None, val: Tensor | None = None) -> "Layer":
        return Layer(
            dim=self.dim,
            num_nodes=self.num_nodes,
            state=self.state if state is None else state,
            val=self.val if val is None else val,
        )

    def apply_delta(self, delta: LayerDelta, merge_mode: MergeMode = "add") -> "Layer":
        validate_merge_mode(merge_mode)
        if self.state.shape != delta.delta_state.shape:
            raise ValueError("delta_state shape does not match the target layer.")
        if self.val.shape != delta.delta_val.shape:
            raise ValueError("delta_val shape does not match the target layer.")
        if merge_mode == "replace":
            return self.with_tensors(state=delta.delta_state, val=delta.delta_val)
        return self.with_tensors(state=self.state + delta.delta_state, val=self.val + delta.delta_val)


def validate_merge_mode(merge_mode: MergeMode) -> None:
    if merge_mode not in _MERGE_MODES:
        raise ValueError(f"Unsupported merge_mode: {merge_mode!r}.")


def validate_implementation(implementation: ImplementationMode) -> None:
    if implementation not in _IMPLEMENTATIONS:
        raise ValueError(f"Unsupported implementation: {implementation!r}.")


def apply_optional_layer_fn(layer: Layer, layer_fn: Callable[[Layer], Layer] | None) -> Layer:
    if layer_fn is None:
        return layer
    result = layer_fn(layer)
    if not isinstance(result, Layer):
        raise TypeError("layer_fn must return a Layer instance.")
    return result


def validate_projected_state(projected_state: Tensor, reference: Layer) -> None:
    if projected_state.shape != reference.state.shape:
        raise ValueError(
            "state_proj_fn must return a tensor shaped like layer.state, "
            f"expected {tuple(reference.state.shape)}, got {tuple(projected_state.shape)}."
        )


def validate_projected_val(projected_val: Tensor, reference: Layer) -> None:
    if projected_val.shape != reference.val.shape:
        raise ValueError(
            "val_proj_fn must return a tensor shaped like layer.val, "
            f"expected {tuple(reference.val.shape)}, got {tuple(projected_val.shape)}."
        )


def validate_pairwise_block_scores(
    scores: Tensor,
    *,
    batch_shape: torch.Size | tuple[int, ...],
    target_nodes: int,
    source_nodes: int,
) -> None:
    expected = (*batch_shape, target_nodes, source_nodes)
    if tuple(scores.shape) != expected:
        raise ValueError(
            "pairwise_fn must return scores shaped like [..., num_nodes, num_nodes], "
            f"expected {expected}, got {tuple(scores.shape)}."
        )


def validate_pairwise_scores(scores: Tensor, layer: Layer) -> None:
    validate_pairwise_block_scores(
        scores, batch_shape=layer.batch_shape, target_nodes=layer.num_nodes, source_nodes=layer.num_nodes
    )


def validate_route_block_logits(
    logits: Tensor,
    *,
    batch_shape: torch.Size | tuple[int, ...],
    source_nodes: int,
    dst_nodes: int,
) -> None:
    expected = (*batch_shape, source_nodes, dst_nodes)
    if tuple(logits.shape) != expected:
        raise ValueError(
            "route_fn must return logits shaped like [..., src_nodes, dst_nodes], "
            f"expected {expected}, got {tuple(logits.shape)}."
        )


def validate_route_logits(logits: Tensor, src_layer: Layer, dst_layer: Layer) -> None:
    validate_route_block_logits(
        logits, batch_shape=src_layer.batch_shape, source_nodes=src_layer.num_nodes, dst_nodes=dst_layer.num_nodes
    )


def resolve_block_size(block_size: int | None, total_size: int, *, name: str) -> int:
    if total_size <= 0:
        raise ValueError("total_size must be positive.")
    if block_size is None:
        return total_size
    if block_size <= 0:
        raise ValueError(f"{name} must be positive when provided.")
    return min(block_size, total_size)


def iter_block_spans(total_size: int, block_size: int | None, *, name: str) -> Iterator[BlockSpan]:
    step = resolve_block_size(block_size, total_size, name=name)
    start = 0
    while start < total_size:
        end = min(start + step, total_size)
        yield BlockSpan(start=start, end=end)
        start = end


def iter_blocks(total_size: int, block_size: int | None, *, name: str) -> Iterator[tuple[int, int]]:
    for span in iter_block_spans(total_size, block_size, name=name):
        yield span.start, span.end


def resolve_accumulator_dtype(tensor_dtype: torch.dtype, accumulator_dtype: torch.dtype | None) -> torch.dtype:
    """fp16/bf16 accumulate in fp32 unless told otherwise (reference core.py:242-249)."""
    if accumulator_dtype is not None:
        return accumulator_dtype
    if tensor_dtype in (torch.float16, torch.bfloat16):
        return torch.float32
    return tensor_dtype


def allocate_accumulator(
    shape: torch.Size | tuple[int, ...],
    *,
    device: torch.device | str,
    tensor_dtype: torch.dtype,
    accumulator_dtype: torch.dtype | None = None,
) -> Tensor:
    return torch.zeros(shape, device=device, dtype=resolve_accumulator_dtype(tensor_dtype, accumulator_dtype))
