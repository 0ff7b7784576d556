"""Native backend loader and hot-path dispatch.

Loader contract of the reference's ``src/jakal_net/native_backend.py:33-178``:
the native module is a Python module named ``jakal_net_native`` (override with
``JAKAL_NET_NATIVE_MODULE``), found on ``sys.path`` or in ``build_native/``,
``native/build/`` or the repository root; ``JAKAL_NET_DISABLE_NATIVE=1``
disables it; it reports ``supported_ops()``, ``supported_devices()`` and
``backend_name()``.  This build's module drives the HIP library through its C
ABI; on ROCm PyTorch reports GPU tensors as device type ``"cuda"``.

The hot-path wrappers pass the reference's positional argument lists
(``native_backend.py:5585-5643``, ``:5944-6021``, ``:5472-5582``,
``:5359-5423``, ``:5755-5822``) to the module's ops.
"""

from __future__ import annotations

import importlib
import os
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from torch import Tensor

from jakal_net.core import LayerDelta
from jakal_net.kernel_common import (
    pairwise_kernel_spec,
    pairwise_route_kernel_spec,
    supports_pairwise_kernel,
    supports_pairwise_route_kernel,
)

DEFAULT_NATIVE_MODULE = "jakal_net_native"
NATIVE_MODULE_ENV = "JAKAL_NET_NATIVE_MODULE"
DISABLE_NATIVE_ENV = "JAKAL_NET_DISABLE_NATIVE"

_TRUE_FLAGS = {"1", "true", "TRUE", "yes"}


@dataclass(frozen=True, slots=True)
class NativeStatus:
    available: bool
    module_name: str
    backend_name: str | None
    supported_ops: tuple[str, ...]
    supported_devices: tuple[str, ...]
    error: str | None


def _module_name() -> str:
    return os.environ.get(NATIVE_MODULE_ENV, DEFAULT_NATIVE_MODULE)


def native_disabled_by_env() -> bool:
    return os.environ.get(DISABLE_NATIVE_ENV, "").strip() in _TRUE_FLAGS


class _NativeLoader:
    """Finds, imports and describes the native module once per process (again
    on ``force_reload``); keeps the module and its status."""

    def __init__(self) -> None:
        self.module: Any | None = None
        self.status: NativeStatus | None = None

    @staticmethod
    def search_dirs() -> list[Path]:
        """Directories tried, in order, after a plain import fails."""
        root = Path(__file__).resolve().parents[2]
        return [root / "build_native", root / "native" / "build", root]

    def _locate(self, name: str) -> Any:
        failures: list[str] = []
        for where in [None, *(d for d in self.search_dirs() if d.is_dir())]:
            if where is not None and str(where) not in sys.path:
                sys.path.insert(0, str(where))
            try:
                return importlib.import_module(name)
            except Exception as exc:  # noqa: BLE001  (every failure is reported)
                failures.append(f"{where or 'sys.path'} -> {exc.__class__.__name__}: {exc}")
        raise ImportError(f"cannot import native module {name!r}: " + "; ".join(failures))

    @staticmethod
    def _describe(module: Any, name: str) -> NativeStatus:
        def listed(fn_name: str, const_name: str, fallback: tuple[str, ...]) -> tuple[str, ...]:
            source = getattr(module, fn_name, None)
            values = source() if callable(source) else getattr(module, const_name, fallback)
            return tuple(map(str, values))

        backend = getattr(module, "backend_name", None)
        backend = backend() if callable(backend) else backend
        return NativeStatus(
            available=True,
            module_name=name,
            backend_name=None if backend is None else str(backend),
            supported_ops=listed("supported_ops", "SUPPORTED_OPS", ()),
            supported_devices=listed("supported_devices", "SUPPORTED_DEVICES", ("cpu",)),
            error=None,
        )

    def load(self, force_reload: bool = False) -> NativeStatus:
        name = _module_name()
        if native_disabled_by_env():  # the switch wins over a module already loaded
            self.module = None
            self.status = NativeStatus(False, name, None, (), (),
                                       f"native backend switched off by {DISABLE_NATIVE_ENV}")
        elif self.status is None or force_reload:
            try:
                module = self._locate(name)
            except Exception as exc:  # noqa: BLE001
                self.module = None
                self.status = NativeStatus(False, name, None, (), (), f"{exc.__class__.__name__}: {exc}")
            else:
                self.module, self.status = module, self._describe(module, name)
        return self.status


_LOADER = _NativeLoader()


def native_status(*, force_reload: bool = False) -> NativeStatus:
    return _LOADER.load(force_reload=force_reload)


def native_available() -> bool:
    return native_status().available


def native_supports(op_name: str) -> bool:
    status = native_status()
    return status.available and op_name in status.supported_ops


def native_supports_device(device_type: str) -> bool:
    status = native_status()
    return status.available and device_type in status.supported_devices


def require_native_for_device(op_name: str, device_type: str) -> None:
    """Raise when a GPU tensor asks for the native hot path and it cannot run.

    CPU tensors fall back to the streaming PyTorch path (the library is GPU
    only); a GPU tensor never silently leaves the HIP path."""
    if device_type == "cpu":
        return
    status = native_status()
    if not status.available:
        raise RuntimeError(f"jakal_net native backend unavailable for {op_name} on {device_type}: {status.error}")
    if device_type not in status.supported_devices:
        raise RuntimeError(f"native backend {status.backend_name} does not support device {device_type!r}")
    raise RuntimeError(f"native backend {status.backend_name} does not implement {op_name!r}")


def _native_module() -> Any:
    status = native_status()
    if status.available and _LOADER.module is not None:
        return _LOADER.module
    raise RuntimeError(f"no native module to call: {status.error or 'not loaded'}")


def _as_layer_delta(result: Any) -> LayerDelta:
    if isinstance(result, LayerDelta):
        return result
    if isinstance(result, tuple) and len(result) == 2 and all(isinstance(t, Tensor) for t in result):
        delta_state, delta_val = result
        return LayerDelta(delta_state=delta_state, delta_val=delta_val)
    raise TypeError(f"a native op returned {type(result).__name__}; expected a LayerDelta or a "
                    f"(delta_state, delta_val) pair")


# ---------------------------------------------------------------------------
# Hot-path wrappers (argument lists of the reference's pybind ops).
# ---------------------------------------------------------------------------
def propagation_topk_native(
    *,
    pairwise_fn: object,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    topk: int,
    target_block_size: int,
    source_block_size: int,
) -> LayerDelta:
    if not supports_pairwise_kernel(pairwise_fn):
        raise TypeError("Unsupported pairwise_fn for native propagation.")
    spec = pairwise_kernel_spec(pairwise_fn, unit_scale=getattr(_native_module(), "unit_scale", None))
    return _as_layer_delta(
        _native_module().propagation_topk(
            spec.kind, spec.weight, spec.bias, spec.in_weight, spec.in_bias, spec.out_weight, spec.out_bias,
            edge_compress_name, layer_val, projected_state, projected_val, topk, target_block_size,
            source_block_size,
        )
    )


def propagation_window_native(
    *,
    pairwise_fn: object,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    window: int,
    target_block_size: int,
    source_block_size: int,
) -> LayerDelta:
    if not supports_pairwise_kernel(pairwise_fn):
        raise TypeError("Unsupported pairwise_fn for native propagation.")
    spec = pairwise_kernel_spec(pairwise_fn, unit_scale=getattr(_native_module(), "unit_scale", None))
    return _as_layer_delta(
        _native_module().propagation_window(
            spec.kind, spec.weight, spec.bias, spec.in_weight, spec.in_bias, spec.out_weight, spec.out_bias,
            edge_compress_name, layer_val, projected_state, projected_val, window, target_block_size,
            source_block_size,
        )
    )


def propagation_dense_native(
    *,
    pairwise_fn: object,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    source_state: Tensor | None = None,
    target_block_size: int,
    source_block_size: int,
) -> LayerDelta:
    if not supports_pairwise_kernel(pairwise_fn):
        raise TypeError("Unsupported pairwise_fn for native propagation.")
    spec = pairwise_kernel_spec(pairwise_fn, unit_scale=getattr(_native_module(), "unit_scale", None))
    return _as_layer_delta(
        _native_module().propagation_dense(
            spec.kind, spec.weight, spec.bias, spec.in_weight, spec.in_bias, spec.out_weight, spec.out_bias,
            edge_compress_name, layer_val, projected_state, projected_val, source_state, target_block_size,
            source_block_size,
        )
    )


def transition_pairwise_topk_native(
    *,
    route_fn: object,
    sender_strength: Tensor,
    src_val: Tensor,
    dst_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    topk: int,
    src_block_size: int,
    dst_block_size: int,
    route_compress_name: str = "softmax",
) -> LayerDelta:
    if not supports_pairwise_route_kernel(route_fn):
        raise TypeError("Unsupported pairwise route_fn for native sparse transition.")
    if route_compress_name not in ("softmax", "signed_abs_softmax", "signed_entmax15"):
        raise TypeError("Native sparse pairwise transition supports softmax, signed_abs_softmax and signed_entmax15 "
                        "routes.")
    spec = pairwise_route_kernel_spec(route_fn)
    return _as_layer_delta(
        _native_module().transition_pairwise_topk(
            spec.kind, spec.source_weight, spec.source_bias, spec.target_weight, spec.target_bias,
            spec.core_weight, spec.bias, spec.hidden_weight, spec.hidden_bias, spec.out_weight, spec.out_bias,
            float(spec.temperature), sender_strength, src_val, dst_val, projected_state, projected_val, topk,
            src_block_size, dst_block_size, route_compress_name=route_compress_name,
        )
    )


def transition_pairwise_dense_native(
    *,
    route_fn: object,
    route_compress_name: str = "softmax",
    sender_strength: Tensor,
    src_val: Tensor,
    dst_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    src_block_size: int,
    dst_block_size: int,
) -> LayerDelta:
    if not supports_pairwise_route_kernel(route_fn):
        raise TypeError("Unsupported pairwise route_fn for native dense transition.")
    spec = pairwise_route_kernel_spec(route_fn)
    return _as_layer_delta(
        _native_module().transition_pairwise_dense(
            spec.kind, spec.source_weight, spec.source_bias, spec.target_weight, spec.target_bias,
            spec.core_weight, spec.bias, spec.hidden_weight, spec.hidden_bias, spec.out_weight, spec.out_bias,
            route_compress_name, float(spec.temperature), sender_strength, src_val, dst_val, projected_state,
            projected_val, src_block_size, dst_block_size,
        )
    )
