"""ctypes binding of libackvq.so: device, buffers, transfers and errors.

The vq binding needs only the device/buffer/transfer part of the reference's
``ack`` module (src/alelyon_compute_kit/_kit/python/ack.py:599-1160): the same
error classes, the same ``Device``/``Buffer`` lifecycle (explicit ``free``,
``close`` refused while buffers live, every call serialised under the
device's ``RLock``) and the same return codes. The reference's ABI-14
handshake over every operator family does not apply: this library carries
the vq4/v1 extension only, and ``VQDevice`` checks its schema itself.

Loading the library never touches the GPU; ``Device()`` opens it.
"""
from __future__ import annotations

import ctypes
import operator
import os
import threading
import warnings
from pathlib import Path

import numpy as np

ACK_OK = 0
ACK_ERR_NULL = -1
ACK_ERR_DEVICE = -2          # the reference's ACK_ERR_VULKAN: the device runtime failed
ACK_ERR_VULKAN = ACK_ERR_DEVICE
ACK_ERR_SHAPE = -3
ACK_ERR_SIZE = -4
ACK_ERR_LIVE_BUFFERS = -5
ACK_ERR_CLOSED = -6
ACK_ERR_FOREIGN = -7
ACK_ERR_FREED = -8
ACK_ERR_ABI = -9
ACK_ERR_POISONED = -10
ACK_ERR_UNSUPPORTED_OP = -11

_MAX_NBYTES = 1 << 40
_POD_SIZES = {"b": (1,), "i": (1, 2, 4, 8), "u": (1, 2, 4, 8), "f": (2, 4, 8)}
_HERE = Path(__file__).resolve().parent
LIBRARY_NAME = "libackvq.so"


class AckError(RuntimeError):
    """A library call returned an error code; the message is the library's."""


class AckUnavailable(AckError):
    """No shared library, or no usable device."""


class AckShapeError(AckError):
    """The request's geometry is refused."""


class AckPoisoned(AckError):
    """The device's state is unknown after a failed device operation: every
    later call on it refuses; close it and start a new process."""


def _kit_error(what: str, rc: int, message: str) -> AckError:
    cls = AckPoisoned if rc == ACK_ERR_POISONED else AckError
    return cls(f"{what}: {message}")


def _is_bool(value) -> bool:
    return isinstance(value, (bool, np.bool_))


def _checked_nbytes(nbytes: int) -> int:
    if _is_bool(nbytes):
        raise AckError("nbytes must be a positive integer, not a boolean")
    try:
        count = operator.index(nbytes)
    except TypeError as exc:
        raise AckError("nbytes must be a positive integer") from exc
    if not 0 < count <= _MAX_NBYTES:
        raise AckError(f"nbytes must be in 1..{_MAX_NBYTES}")
    return count


def _pod_dtype(dtype) -> np.dtype:
    try:
        result = np.dtype(dtype)
    except (TypeError, ValueError) as exc:
        raise AckError("unsupported buffer dtype") from exc
    if (result.hasobject or result.fields is not None or result.subdtype is not None
            or result.itemsize not in _POD_SIZES.get(result.kind, ())):
        raise AckError(f"unsupported buffer dtype {result} is refused; use a plain "
                       "fixed-width numeric or bool dtype")
    return result


def library_path() -> Path | None:
    """``ACK_LIBRARY`` if set, else the library built into this package."""
    candidates = []
    if os.environ.get("ACK_LIBRARY"):
        candidates.append(Path(os.environ["ACK_LIBRARY"]))
    candidates.append(_HERE / "_lib" / LIBRARY_NAME)
    for candidate in candidates:
        if candidate.is_file():
            return candidate
    return None


_c = ctypes
_SIGNATURES = {
    "ack_vq_schema": ([], _c.c_uint32),
    "ack_vq": ([_c.c_void_p] * 7 + [_c.c_void_p, _c.c_size_t], _c.c_int32),
    "ack_vq_batch": ([_c.c_void_p] * 7 + [_c.c_void_p, _c.c_size_t, _c.c_uint32], _c.c_int32),
    "ack_open": ([], _c.c_void_p),
    "ack_close": ([_c.c_void_p], _c.c_int32),
    "ack_device_name": ([_c.c_void_p, _c.c_char_p, _c.c_size_t], _c.c_int32),
    "ack_last_error": ([_c.c_char_p, _c.c_size_t], _c.c_int32),
    "ack_buffer_alloc": ([_c.c_void_p, _c.c_uint64], _c.c_void_p),
    "ack_buffer_free": ([_c.c_void_p, _c.c_void_p], _c.c_int32),
    "ack_upload": ([_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_size_t], _c.c_int32),
    "ack_download": ([_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_size_t], _c.c_int32),
    "ack_vq_plan_query": ([_c.c_void_p, _c.c_size_t, _c.c_uint32, _c.c_void_p, _c.c_void_p,
                           _c.c_void_p], _c.c_int32),
    "ack_vq_plan_check_buffers": ([_c.c_void_p, _c.c_size_t, _c.c_void_p, _c.c_void_p],
                                  _c.c_int32),
    "ack_vq_adamw_step": ([_c.c_void_p] * 8 + [_c.c_void_p, _c.c_size_t, _c.c_uint32,
                                               _c.c_uint32], _c.c_int32),
    "ack_stream_timer": ([_c.c_void_p, _c.c_uint32, _c.POINTER(_c.c_float)], _c.c_int32),
    "ack_sync": ([_c.c_void_p], _c.c_int32),
    "ack_vq_path_name": ([_c.c_void_p, _c.c_size_t, _c.c_char_p, _c.c_size_t], _c.c_int32),
    "ack_vq_set_policy": ([_c.c_void_p, _c.c_uint32], _c.c_int32),
    "ack_vq_host_encode": ([_c.c_void_p, _c.c_uint64, _c.c_void_p, _c.c_uint32, _c.c_void_p],
                           _c.c_int32),
    "ack_vq_host_fit_codebook": ([_c.c_void_p, _c.c_uint64, _c.c_uint32, _c.c_uint32,
                                  _c.c_uint32, _c.c_void_p, _c.c_void_p], _c.c_int32),
    "ack_vq_fit_codebook": ([_c.c_void_p] * 5 + [_c.c_uint64, _c.c_uint32, _c.c_uint32,
                                                 _c.c_uint32], _c.c_int32),
    "ack_vq_matmul_dense": ([_c.c_void_p] * 6 + [_c.c_void_p, _c.c_size_t], _c.c_int32),
    "ack_vq_dense_path_name": ([_c.c_void_p, _c.c_size_t, _c.c_char_p, _c.c_size_t], _c.c_int32),
    "ack_buffer_copy": ([_c.c_void_p, _c.c_void_p, _c.c_uint64, _c.c_void_p, _c.c_uint64,
                         _c.c_uint64], _c.c_int32),
}


class _Lib:
    """The loaded library with every entry point declared."""

    def __init__(self, path: Path) -> None:
        self.path = path
        self.cdll = ctypes.CDLL(str(path))
        for name, (argtypes, restype) in _SIGNATURES.items():
            try:
                fn = getattr(self.cdll, name)
            except AttributeError as exc:
                raise AckUnavailable(f"{path} lacks {name}") from exc
            fn.argtypes, fn.restype = argtypes, restype

    def last_error(self) -> str:
        buf = ctypes.create_string_buffer(1024)
        self.cdll.ack_last_error(buf, len(buf))
        return buf.value.decode("utf-8", errors="replace")


_LIB: _Lib | None = None
_LIB_LOCK = threading.Lock()


def _lib() -> _Lib:
    global _LIB
    with _LIB_LOCK:
        if _LIB is None:
            path = library_path()
            if path is None:
                raise AckUnavailable(
                    f"{LIBRARY_NAME} is not built; run alelyon-compute-kit_amd/build.py")
            _LIB = _Lib(path)
        return _LIB


class Buffer:
    """A device buffer; explicit free() releases it."""

    def __init__(self, device: "Device", nbytes: int) -> None:
        self._device = device
        self._handle = None
        self._nbytes = _checked_nbytes(nbytes)
        with device._lock:
            device._require_open()
            handle = device._lib.cdll.ack_buffer_alloc(device._handle, self._nbytes)
            if not handle:
                raise AckError(f"buffer alloc: {device._lib.last_error()}")
            device._buffers.add(handle)
            self._handle = handle

    @property
    def nbytes(self) -> int:
        return self._nbytes

    def _require_live(self) -> None:
        if not self._handle:
            raise AckError("buffer has been freed")
        self._device._require_open()

    def upload(self, data) -> None:
        with self._device._lock:
            self._require_live()
            array = np.asarray(data)
            _pod_dtype(array.dtype)
            if array.nbytes != self.nbytes:
                raise AckError(f"upload of {array.nbytes} bytes into a {self.nbytes}-byte buffer")
            raw = np.ascontiguousarray(array)
            lib = self._device._lib
            rc = lib.cdll.ack_upload(self._device._handle, self._handle, raw.ctypes.data,
                                     raw.nbytes)
            if rc != ACK_OK:
                raise _kit_error("upload", rc, lib.last_error())

    def download(self, dtype) -> np.ndarray:
        with self._device._lock:
            self._require_live()
            dtype = _pod_dtype(dtype)
            if self.nbytes % dtype.itemsize:
                raise AckError(f"buffer size {self.nbytes} is not divisible by dtype itemsize "
                               f"{dtype.itemsize}; a transfer requires a whole number of elements")
            out = np.empty(self.nbytes // dtype.itemsize, dtype=dtype)
            lib = self._device._lib
            rc = lib.cdll.ack_download(self._device._handle, self._handle, out.ctypes.data,
                                       out.nbytes)
            if rc != ACK_OK:
                raise _kit_error("download", rc, lib.last_error())
            return out

    def copy_from(self, src: "Buffer", nbytes: int, *, offset: int = 0,
                  src_offset: int = 0) -> None:
        """Enqueue a device-to-device copy of ``nbytes`` from ``src``."""
        with self._device._lock:
            self._require_live()
            src._require_live()
            lib = self._device._lib
            rc = lib.cdll.ack_buffer_copy(self._device._handle, self._handle, offset,
                                          src._handle, src_offset, nbytes)
            if rc != ACK_OK:
                raise _kit_error("copy", rc, lib.last_error())

    def free(self) -> None:
        with self._device._lock:
            if self._handle:
                self._device._require_open()
                lib = self._device._lib
                rc = lib.cdll.ack_buffer_free(self._device._handle, self._handle)
                self._device._buffers.discard(self._handle)
                self._handle = None
                if rc != ACK_OK:
                    raise _kit_error("free", rc, lib.last_error())

    def __del__(self) -> None:
        try:
            self.free()
        except AckError as exc:
            try:
                warnings.warn(f"ack.Buffer finaliser: {exc}", ResourceWarning, stacklevel=2)
            except Exception:
                pass
        except Exception:
            pass


class Device:
    """One HIP device. Free its buffers before close(); calls are serialised."""

    def __init__(self) -> None:
        self._lock = threading.RLock()
        self._buffers: set[int] = set()
        self._handle = None
        self._lib = lib = _lib()
        self._handle = lib.cdll.ack_open()
        if not self._handle:
            raise AckUnavailable(f"ack_open: {lib.last_error()}")
        try:
            buf = ctypes.create_string_buffer(256)
            rc = lib.cdll.ack_device_name(self._handle, buf, len(buf))
            if rc != ACK_OK:
                raise AckError(f"device name: {lib.last_error()}")
            self.name = buf.value.decode("utf-8", errors="replace")
        except BaseException:
            self.close()
            raise

    def capability_record(self) -> dict:
        """What this device and library declare, JSON-serialisable."""
        with self._lock:
            self._require_open()
            return {"device": self.name, "library": str(self._lib.path),
                    "vq_schema": int(self._lib.cdll.ack_vq_schema())}

    def _require_open(self) -> None:
        if not self._handle:
            raise AckError("device is closed")

    def close(self) -> None:
        """Free the device only on ACK_OK; a refusal keeps the handle valid."""
        with self._lock:
            if self._handle:
                if self._buffers:
                    raise AckError("device has live buffers still allocated; free them before close")
                rc = self._lib.cdll.ack_close(self._handle)
                if rc == ACK_ERR_CLOSED:
                    self._handle = None
                    raise AckError(f"close: {self._lib.last_error()}")
                if rc != ACK_OK:
                    raise AckError(f"close: {self._lib.last_error()}")
                self._handle = None

    def __enter__(self) -> "Device":
        with self._lock:
            self._require_open()
            return self

    def __exit__(self, *exc) -> None:
        self.close()

    def buffer(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def synchronize(self) -> None:
        with self._lock:
            self._require_open()
            rc = self._lib.cdll.ack_sync(self._handle)
            if rc != ACK_OK:
                raise _kit_error("sync", rc, self._lib.last_error())

    def timer_start(self) -> None:
        """Record a start event on the device stream (benchmarks)."""
        with self._lock:
            self._require_open()
            rc = self._lib.cdll.ack_stream_timer(self._handle, 0, None)
            if rc != ACK_OK:
                raise _kit_error("timer", rc, self._lib.last_error())

    def timer_stop(self) -> float:
        """Record a stop event, wait for it, return milliseconds since start."""
        with self._lock:
            self._require_open()
            ms = ctypes.c_float()
            rc = self._lib.cdll.ack_stream_timer(self._handle, 1, ctypes.byref(ms))
            if rc != ACK_OK:
                raise _kit_error("timer", rc, self._lib.last_error())
            return float(ms.value)

    def set_policy(self, policy: int) -> None:
        """0: automatic kernel choice; 1: the general matmul kernel only."""
        with self._lock:
            self._require_open()
            rc = self._lib.cdll.ack_vq_set_policy(self._handle, policy)
            if rc != ACK_OK:
                raise _kit_error("policy", rc, self._lib.last_error())
