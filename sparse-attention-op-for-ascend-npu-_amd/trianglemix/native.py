"""Load the native libraries once per process and report their status.

Restates the part of the reference's native bootstrap that is not
Ascend-specific: load once under a lock, refuse a second adapter path, verify
the registration, keep a status object, strict vs fail-open
(package/src/vllm_ascend_trianglemix/native.py:602-678,
package/src/vllm_ascend_trianglemix/kernel.py:287-339).  The CANN runtime
fingerprint / SoC / OPP-path logic has no ROCm counterpart and is not kept.

There is no CPU fallback: when the libraries are missing or fail to load,
every call that needs them raises ``NativeUnavailable``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
HIP_LIBRARY = PKG_DIR / "libtrianglemix.so"
TORCH_ADAPTER = PKG_DIR / "_trianglemix_torch.so"

ABI_VERSION = 3

_LOCK = threading.Lock()
_LOADED_ADAPTER_PATH: str | None = None
_CDLL: ctypes.CDLL | None = None


class NativeUnavailable(RuntimeError):
    """The HIP library or the torch adapter is not built / not loadable."""


@dataclass(frozen=True)
class NativeStatus:
    ready: bool
    adapter_path: str | None
    library_path: str | None
    reason: str

    def to_dict(self) -> dict:
        return {"ready": self.ready, "adapter_path": self.adapter_path,
                "library_path": self.library_path, "reason": self.reason}


_STATUS = NativeStatus(False, None, None, "not_loaded")


def _normalise(path: str | os.PathLike[str] | None) -> str:
    if path is None or not os.fspath(path).strip():
        raise ValueError("TriangleMix adapter path is empty")
    resolved = os.path.realpath(os.path.abspath(os.path.expanduser(os.fspath(path))))
    if not os.path.isfile(resolved):
        raise FileNotFoundError(f"TriangleMix Torch adapter does not exist: {resolved}")
    return resolved


def _declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    i64, i32p, vp = ctypes.c_int64, ctypes.POINTER(ctypes.c_int32), ctypes.c_void_p
    lib.tm_abi_version.restype = ctypes.c_int
    lib.tm_abi_version.argtypes = []
    lib.tm_status_string.restype = ctypes.c_char_p
    lib.tm_status_string.argtypes = [ctypes.c_int]
    lib.tm_last_error.restype = ctypes.c_char_p
    lib.tm_last_error.argtypes = []
    lib.tm_triangle_paged_sparse_attention.restype = ctypes.c_int
    lib.tm_triangle_paged_sparse_attention.argtypes = [
        vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ctypes.c_float, vp, i64, vp]
    lib.tm_triangle_paged_sparse_attention_noalloc.restype = ctypes.c_int
    lib.tm_triangle_paged_sparse_attention_noalloc.argtypes = [
        vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ctypes.c_float, vp]
    lib.tm_triangle_paged_sparse_attention_workspace_size.restype = i64
    lib.tm_triangle_paged_sparse_attention_workspace_size.argtypes = [i64, i64, i64, i64]
    lib.tm_dense_paged_causal_attention.restype = ctypes.c_int
    lib.tm_dense_paged_causal_attention.argtypes = [
        vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_float, vp, i64, vp]
    lib.tm_dense_paged_causal_attention_workspace_size.restype = i64
    lib.tm_dense_paged_causal_attention_workspace_size.argtypes = [i64, i64, i64]
    lib.tm_chunk_plan.restype = ctypes.c_int
    lib.tm_chunk_plan.argtypes = [ctypes.c_int, i64, i64, i64, i64, ctypes.POINTER(ctypes.c_int32),
                                  ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)]
    lib.tm_reshape_and_cache.restype = ctypes.c_int
    lib.tm_reshape_and_cache.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, vp]
    del i32p
    return lib


def load_hip_library(path: str | os.PathLike[str] | None = None) -> ctypes.CDLL:
    """ctypes handle of ``libtrianglemix.so`` (loaded once per process)."""
    global _CDLL
    with _LOCK:
        if _CDLL is not None:
            return _CDLL
        target = Path(path) if path is not None else HIP_LIBRARY
        if not target.is_file():
            raise NativeUnavailable(f"HIP library is not built: {target}")
        lib = _declare(ctypes.CDLL(str(target)))
        version = lib.tm_abi_version()
        if version != ABI_VERSION:
            raise NativeUnavailable(f"HIP library ABI {version} != expected {ABI_VERSION}")
        _CDLL = lib
        return lib


def _out_op_registered() -> bool:
    import torch

    try:
        torch.ops.trianglemix.triangle_paged_sparse_attention.out  # noqa: B018
    except (AttributeError, RuntimeError):
        return False
    return True


def load_triangle_mix_adapter(path: str | os.PathLike[str] | None = None) -> str:
    """Load the torch adapter once; the same path again is a no-op.

    Mirrors kernel.py:296-322: a second, different path is refused because
    live operator registrations cannot be replaced.
    """
    import torch

    global _LOADED_ADAPTER_PATH, _STATUS
    resolved = _normalise(path if path is not None else TORCH_ADAPTER)
    with _LOCK:
        if _LOADED_ADAPTER_PATH is not None:
            if _LOADED_ADAPTER_PATH != resolved:
                raise RuntimeError(
                    f"TriangleMix adapter is already loaded from {_LOADED_ADAPTER_PATH}; refusing {resolved}")
            return resolved
        torch.ops.load_library(resolved)
        if not _out_op_registered():
            raise RuntimeError("TriangleMix adapter did not register trianglemix::triangle_paged_sparse_attention.out")
        _LOADED_ADAPTER_PATH = resolved
        _STATUS = NativeStatus(True, resolved, str(HIP_LIBRARY), "ready")
        return resolved


def triangle_mix_adapter_loaded() -> bool:
    with _LOCK:
        return _LOADED_ADAPTER_PATH is not None


def ensure_native_loaded(*, strict: bool = False) -> NativeStatus:
    """Load both libraries; fail open (status with a reason) unless strict."""
    global _STATUS
    try:
        load_hip_library()
        load_triangle_mix_adapter()
    except Exception as error:  # noqa: BLE001 - fail-open is the contract
        if strict:
            raise
        with _LOCK:
            _STATUS = NativeStatus(False, None, None, f"{type(error).__name__}: {error}")
    return native_status()


def native_status() -> NativeStatus:
    with _LOCK:
        return _STATUS


def require_adapter() -> None:
    """Raise ``NativeUnavailable`` unless the torch adapter is loaded."""
    if not triangle_mix_adapter_loaded():
        status = ensure_native_loaded(strict=False)
        if not status.ready:
            raise NativeUnavailable(f"TriangleMix native adapter unavailable: {status.reason}")


_ROUTED = None  # the adapter's routed-call module once imported, False when it cannot be


def routed_fast_path():
    """The torch adapter's routed-call entry points (``tensor_gate``, ``launch_sparse``, ``launch_dense``),
    or None.

    The adapter library is also a Python extension module: for the routing
    layer it gives the per-call tensor gates in one native call and the
    ``.out`` launches without the dispatcher's Python argument handling.  It
    is imported only once the adapter is loaded from this package's own file
    (importing another file would register the ops a second time).
    """
    global _ROUTED
    if _ROUTED is None:
        with _LOCK:
            own = _LOADED_ADAPTER_PATH is not None and _LOADED_ADAPTER_PATH == _normalise(TORCH_ADAPTER)
        if not own:
            return None
        try:
            import importlib

            _ROUTED = importlib.import_module(__package__ + "._trianglemix_torch")
        except ImportError:
            _ROUTED = False
    return _ROUTED or None
