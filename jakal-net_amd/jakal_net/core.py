"""Layers and layer deltas of the Jakal-Net operator API.

A layer is a batch of graphs with ``num_nodes`` nodes each.  Every node
carries a scalar state and a ``dim``-long value vector, held as ``state
[..., num_nodes]`` and ``val [..., num_nodes, dim]`` with the same leading
batch shape.  Operators return a ``LayerDelta`` of the same shapes, which a
layer takes in with ``apply_delta``: added to its tensors, or replacing them.

The public names (``Layer``, ``LayerDelta``, the ``MergeMode`` /
``SparsePropagationType`` / ``ImplementationMode`` literals) are the
operator API of the reference (src/jakal_net/core.py:9-131); the helpers
below them serve this package's operators only.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterator, Literal, get_args

import torch
from torch import Tensor

MergeMode = Literal["add", "replace"]
SparsePropagationType = Literal["window", "topk"]
ImplementationMode = Literal["reference", "streaming", "kernel", "native"]

MERGE_MODES = frozenset(get_args(MergeMode))
IMPLEMENTATIONS = frozenset(get_args(ImplementationMode))


def _node_axes(state: Tensor, val: Tensor, owner: str) -> tuple[int, int]:
    """(nodes, value dim) of a state / value pair; ValueError when the pair is malformed."""
    if state.dim() < 1:
        raise ValueError(f"{owner}: the state tensor has no node axis (a 0-d tensor was given).")
    if val.dim() < 2:
        raise ValueError(f"{owner}: the value tensor needs [..., nodes, dim] axes, got shape {tuple(val.shape)}.")
    if tuple(val.shape[:-1]) != tuple(state.shape):
        raise ValueError(
            f"{owner}: a value tensor of shape {tuple(val.shape)} does not pair with a state tensor of shape "
            f"{tuple(state.shape)} (values add one trailing axis to the state's shape)."
        )
    return int(state.shape[-1]), int(val.shape[-1])


@dataclass(slots=True)
class LayerDelta:
    """An operator's update: ``delta_state [..., N]`` and ``delta_val [..., N, D]``."""

    delta_state: Tensor
    delta_val: Tensor

    def __post_init__(self) -> None:
        _node_axes(self.delta_state, self.delta_val, "LayerDelta")

    @classmethod
    def zeros_like(cls, layer: "Layer") -> "LayerDelta":
        return cls(delta_state=layer.state.new_zeros(layer.state.shape), delta_val=layer.val.new_zeros(layer.val.shape))


@dataclass(slots=True)
class Layer:
    """A batch of node states ``state [..., N]`` and node values ``val [..., N, dim]``."""

    dim: int
    num_nodes: int
    state: Tensor
    val: Tensor

    def __post_init__(self) -> None:
        if self.dim < 1 or self.num_nodes < 1:
            raise ValueError(f"Layer: dim and num_nodes must be at least 1, got dim={self.dim}, "
                             f"num_nodes={self.num_nodes}.")
        nodes, dim = _node_axes(self.state, self.val, "Layer")
        if nodes != self.num_nodes or dim != self.dim:
            raise ValueError(f"Layer: declared {self.num_nodes} nodes of dim {self.dim}, but the tensors hold "
                             f"{nodes} nodes of dim {dim}.")

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
        val = torch.zeros((*batch_shape, num_nodes, dim), device=device, dtype=dtype)
        return cls(dim=dim, num_nodes=num_nodes, state=val.new_zeros(val.shape[:-1]), val=val)

    @property
    def batch_shape(self) -> torch.Size:
        return self.state.shape[:-1]

    def with_tensors(self, *, state: Tensor | None = None, val: Tensor | None = None) -> "Layer":
        """A layer of the same geometry with either tensor swapped (the other one shared)."""
        return Layer(self.dim, self.num_nodes, self.state if state is None else state, self.val if val is None else val)

    def clone(self) -> "Layer":
        return self.with_tensors(state=self.state.clone(), val=self.val.clone())

    def apply_delta(self, delta: LayerDelta, merge_mode: MergeMode = "add") -> "Layer":
        """``add``: state + delta_state, val + delta_val; ``replace``: the delta's tensors."""
        check_merge_mode(merge_mode)
        if delta.delta_state.shape != self.state.shape or delta.delta_val.shape != self.val.shape:
            raise ValueError(
                f"apply_delta: a delta of shapes {tuple(delta.delta_state.shape)} / {tuple(delta.delta_val.shape)} "
                f"does not fit a layer of shapes {tuple(self.state.shape)} / {tuple(self.val.shape)}."
            )
        if merge_mode == "replace":
            return self.with_tensors(state=delta.delta_state, val=delta.delta_val)
        return self.with_tensors(state=self.state + delta.delta_state, val=self.val + delta.delta_val)


# ---------------------------------------------------------------------------
# helpers of the operators in this package
# ---------------------------------------------------------------------------
def check_merge_mode(merge_mode: str) -> None:
    if merge_mode not in MERGE_MODES:
        raise ValueError(f"merge_mode must be one of {sorted(MERGE_MODES)}, got {merge_mode!r}.")


def check_implementation(implementation: str) -> None:
    if implementation not in IMPLEMENTATIONS:
        raise ValueError(f"implementation must be one of {sorted(IMPLEMENTATIONS)}, got {implementation!r}.")


def finish_layer(layer: Layer, layer_fn: Callable[[Layer], Layer] | None) -> Layer:
    """Run an operator's optional ``norm_fn`` on its output layer."""
    if layer_fn is None:
        return layer
    out = layer_fn(layer)
    if not isinstance(out, Layer):
        raise TypeError(f"norm_fn returned {type(out).__name__}, not a Layer.")
    return out


def expect_shape(tensor: Tensor, shape: tuple[int, ...] | torch.Size, produced_by: str) -> None:
    """ValueError naming the callable that produced ``tensor`` when its shape is not ``shape``."""
    if tuple(tensor.shape) != tuple(shape):
        raise ValueError(f"{produced_by} produced a tensor of shape {tuple(tensor.shape)}; expected {tuple(shape)}.")


def block_ranges(total: int, block: int | None) -> Iterator[tuple[int, int]]:
    """Consecutive ``[start, end)`` ranges of at most ``block`` (all of ``total`` when None)."""
    if total < 1:
        raise ValueError(f"block_ranges: nothing to split (total={total}).")
    if block is not None and block < 1:
        raise ValueError(f"block sizes must be at least 1, got {block}.")
    step = total if block is None else min(block, total)
    for start in range(0, total, step):
        yield start, min(total, start + step)


def accumulation_dtype(dtype: torch.dtype, override: torch.dtype | None) -> torch.dtype:
    """The dtype blockwise sums accumulate in: ``override`` if given, fp32 for
    half-precision inputs, else the input dtype (the reference's streaming
    backends accumulate fp16 / bf16 in fp32, src/jakal_net/core.py:242-249)."""
    if override is not None:
        return override
    return torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype
