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


_NATIVE_MODULE: Any | None = None
_NATIVE_STATUS: NativeStatus | None = None


def _module_name() -> str:
    return os.environ.get(NATIVE_MODULE_ENV, DEFAULT_NATIVE_MODULE)


def native_disabled_by_env() -> bool:
    return os.environ.get(DISABLE_NATIVE_ENV, "").strip() in _TRUE_FLAGS


def _candidate_module_paths() -> tuple[Path, ...]:
    repo_root = Path(__file__).resolve().parents[2]
    return (repo_root / "build_native", repo_root / "native" / "build", repo_root)


def _import_native_module(module_name: str) -> Any:
    try:
        return importlib.import_module(module_name)
    except Exception as first:  # noqa: BLE001
        errors = [f"default import: {type(first).__name__}: {first}"]
        for candidate in _candidate_module_paths():
            if not candidate.exists():
                continue
            if str(candidate) not in sys.path:
                sys.path.insert(0, str(candidate))
            try:
                return importlib.import_module(module_name)
            except Exception as exc:  # noqa: BLE001
                errors.append(f"{candidate}: {type(exc).__name__}: {exc}")
        raise ImportError("; ".join(errors)) from first


def _names(module: Any, fn_name: str, const_name: str, default: tuple[str, ...]) -> tuple[str, ...]:
    fn = getattr(module, fn_name, None)
    if callable(fn):
        return tuple(str(x) for x in fn())
    return tuple(str(x) for x in getattr(module, const_name, default))


def _load_native_module(force_reload: bool = False) -> NativeStatus:
    global _NATIVE_MODULE, _NATIVE_STATUS
    module_name = _module_name()
    if native_disabled_by_env():
        _NATIVE_MODULE = None
        _NATIVE_STATUS = NativeStatus(False, module_name, None, (), (), f"{DISABLE_NATIVE_ENV} is set.")
        return _NATIVE_STATUS
    if _NATIVE_STATUS is not None and not force_reload:
        return _NATIVE_STATUS
    try:
        module = _import_native_module(module_name)
    except Exception as exc:  # noqa: BLE001
        _NATIVE_MODULE = None
        _NATIVE_STATUS = NativeStatus(False, module_name, None, (), (), f"{type(exc).__name__}: {exc}")
        return _NATIVE_STATUS
    backend = getattr(module, "backend_name", None)
    if callable(backend):
        backend = backend()
    _NATIVE_MODULE = module
    _NATIVE_STATUS = NativeStatus(
        available=True,
        module_name=module_name,
        backend_name=None if backend is None else str(backend),
        supported_ops=_names(module, "supported_ops", "SUPPORTED_OPS", ()),
        supported_devices=_names(module, "supported_devices", "SUPPORTED_DEVICES", ("cpu",)),
        error=None,
    )
    return _NATIVE_STATUS


def native_status(*, force_reload: bool = False) -> NativeStatus:
    return _load_native_module(force_reload=force_reload)


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
    if not status.available or _NATIVE_MODULE is None:
        raise RuntimeError(status.error or "Native backend is unavailable.")
    return _NATIVE_MODULE


def _to_layer_delta(result: Any) -> LayerDelta:
    if isinstance(result, LayerDelta):
        return result
    if isinstance(result, tuple) and len(result) == 2 and all(isinstance(t, Tensor) for t in result):
        return LayerDelta(delta_state=result[0], delta_val=result[1])
    raise TypeError("Native backend must return LayerDelta or (delta_state, delta_val).")


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
    return _to_layer_delta(
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
    return _to_layer_delta(
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
    return _to_layer_delta(
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
    return _to_layer_delta(
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
    return _to_layer_delta(
        _native_module().transition_pairwise_dense(
            spec.kind, spec.source_weight, spec.source_bias, spec.target_weight, spec.target_bias,
            spec.core_weight, spec.bias, spec.hidden_weight, spec.hidden_bias, spec.out_weight, spec.out_bias,
            route_compress_name, float(spec.temperature), sender_strength, src_val, dst_val, projected_state,
            projected_val, src_block_size, dst_block_size,
        )
    )
