"""ctypes binding of libackvq.so: the device, its buffers, transfers, errors.

The vq4 path needs the device/buffer/transfer part of the reference's
``ack`` module (src/alelyon_compute_kit/_kit/python/ack.py:599-1160). What
callers can observe is kept: the error classes, the return codes, a
``Device`` that refuses to close while its buffers live, ``Buffer`` objects
with ``upload``/``download``/``free``, every call on a device serialised.
The reference's ABI-14 handshake over every operator family does not apply
to a library that carries the vq4/v1 extension only; ``VQDevice`` checks the
extension's schema itself.

Design here: one ``Library`` object holds the loaded shared library with
every entry point declared from a table; return codes map to exception
classes in one place (``Library.check``); a device keeps a registry of its
live buffer handles; a buffer dropped without ``free()`` is released by a
``weakref.finalize`` hook that reports any refusal as a ResourceWarning.

Loading the library never touches the GPU; ``Device()`` opens one.
"""
from __future__ import annotations

import ctypes
import numbers
import os
import threading
import warnings
import weakref
from pathlib import Path

import numpy as np

# Return codes of the C ABI (include/ack_vq.h; the reference's ffi.rs codes).
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

LIBRARY_NAME = "libackvq.so"
MAX_BUFFER_BYTES = 1 << 40


class AckError(RuntimeError):
    """A library call returned an error code; the message is the library's."""


class AckUnavailable(AckError):
    """No shared library, or no usable device."""


class AckShapeError(AckError):
    """The library refused the request's geometry (ACK_ERR_SHAPE)."""


class AckPoisoned(AckError):
    """The device's state is unknown after a failed device operation: every
    later call on it refuses; close it and start a new process."""


_EXCEPTION_FOR_CODE = {ACK_ERR_POISONED: AckPoisoned, ACK_ERR_SHAPE: AckShapeError}

# (kind, itemsize) of the element types a transfer accepts: plain
# fixed-width numbers and bool, never objects, records or sub-arrays.
_TRANSFER_TYPES = frozenset([("b", 1)] + [(k, s) for k in "iu" for s in (1, 2, 4, 8)]
                            + [("f", s) for s in (2, 4, 8)])

_P, _U32, _U64, _I32, _SZ = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32,
                             ctypes.c_size_t)


class AckAbiInfo(ctypes.Structure):
    """What ``ack_abi_info`` fills in: the layout of the reference's struct
    (src/alelyon_compute_kit/_kit/src/ffi.rs:1005-1060). This library holds
    the vq4/v1 entries only: its operator bits, operator schemas and
    capabilities are 0, which the reference defines as absent."""

    _fields_ = [("size", ctypes.c_uint32), ("version", ctypes.c_uint32),
                ("operators", ctypes.c_uint64), ("shaders", ctypes.c_uint64),
                ("build", ctypes.c_uint64)] + [
        (name, ctypes.c_uint32) for name in (
            "op_schema_matmul_bf16", "op_schema_cast", "capability_streams", "capability_rng",
            "capability_optimizer", "capability_serialization", "op_schema_matmul_f32",
            "op_schema_pointwise", "op_schema_reduce", "op_schema_rowwise", "op_schema_loss",
            "op_schema_embedding", "op_schema_matmul_f16", "op_schema_index",
            "op_schema_convert", "op_schema_intwise")]


class AckDeviceInfo(ctypes.Structure):
    """What ``ack_device_info`` fills in for an open device: the layout of the
    reference's struct (ffi.rs:1212-1250), its values from the HIP runtime."""

    _fields_ = [(name, ctypes.c_uint32) for name in (
        "size", "version", "api_version", "driver_version_raw", "driver_id", "vendor_id",
        "device_id", "device_type")] + [
        ("device_uuid", ctypes.c_uint8 * 16), ("driver_uuid", ctypes.c_uint8 * 16),
        ("features", ctypes.c_uint64), ("subgroup_size", ctypes.c_uint32),
        ("timestamp_valid_bits", ctypes.c_uint32), ("timestamp_period_ns", ctypes.c_float),
        ("max_push_constant_bytes", ctypes.c_uint32), ("device_local_bytes", ctypes.c_uint64),
        ("max_storage_buffer_bytes", ctypes.c_uint64),
        ("max_workgroup_invocations", ctypes.c_uint32),
        ("max_workgroup_count", ctypes.c_uint32 * 3), ("max_workgroup_size", ctypes.c_uint32 * 3)] + [
        (name, ctypes.c_uint32) for name in (
            "matmul_tile", "matmul_k_multiple", "matmul_layouts", "matmul_operand_dtype",
            "matmul_result_dtype", "cast_modes", "reserved")] + [
        ("identity", ctypes.c_uint64), ("device_name", ctypes.c_char * 256),
        ("driver_name", ctypes.c_char * 64), ("driver_info", ctypes.c_char * 128)]


# the reference's feature bits (ffi.rs:983-1000) and dtype codes (:1002-1003)
ACK_FEATURE_BITS = {
    "cooperative_matrix": 1, "bf16_type": 2, "bf16_dot_product": 4,
    "bf16_cooperative_matrix": 8, "subgroup_size_control": 16,
    "coopmat_bf16_16x16x16_subgroup": 32, "shader_int16": 64, "shader_float16": 128,
    "coopmat_f16_16x16x16_subgroup": 256,
}
ACK_DTYPE_NAMES = {1: "bf16", 2: "f32"}
# name: (argument types, result type), as include/ack_vq.h declares them
_ENTRY_POINTS = {
    "ack_vq_schema": ((), _U32),
    "ack_vq": ((_P,) * 8 + (_SZ,), _I32),
    "ack_vq_batch": ((_P,) * 8 + (_SZ, _U32), _I32),
    "ack_vq_noalloc": ((_P,) * 8 + (_SZ,), _I32),
    "ack_open": ((), _P),
    "ack_close": ((_P,), _I32),
    "ack_device_name": ((_P, ctypes.c_char_p, _SZ), _I32),
    "ack_last_error": ((ctypes.c_char_p, _SZ), _I32),
    "ack_buffer_alloc": ((_P, _U64), _P),
    "ack_buffer_free": ((_P, _P), _I32),
    "ack_upload": ((_P, _P, _P, _SZ), _I32),
    "ack_download": ((_P, _P, _P, _SZ), _I32),
    "ack_buffer_copy": ((_P, _P, _U64, _P, _U64, _U64), _I32),
    "ack_vq_sum_squares": ((_P, _P, _U64, _P), _I32),
    "ack_vq_scale": ((_P, _P, _U64, ctypes.c_float), _I32),
    "ack_sync": ((_P,), _I32),
    "ack_stream_timer": ((_P, _U32, ctypes.POINTER(ctypes.c_float)), _I32),
    "ack_vq_plan_query": ((_P, _SZ, _U32, _P, _P, _P), _I32),
    "ack_vq_plan_check_buffers": ((_P, _SZ, _P, _P), _I32),
    "ack_vq_path_name": ((_P, _SZ, ctypes.c_char_p, _SZ), _I32),
    "ack_vq_batch_path_name": ((_P, _SZ, ctypes.c_uint32, ctypes.c_char_p, _SZ), _I32),
    "ack_vq_dense_path_name": ((_P, _SZ, ctypes.c_char_p, _SZ), _I32),
    "ack_vq_set_policy": ((_P, _U32), _I32),
    "ack_vq_host_encode": ((_P, _U64, _P, _U32, _P), _I32),
    "ack_vq_host_fit_codebook": ((_P, _U64, _U32, _U32, _U32, _P, _P), _I32),
    "ack_vq_fit_codebook": ((_P,) * 5 + (_U64, _U32, _U32, _U32), _I32),
    "ack_vq_matmul_dense": ((_P,) * 7 + (_SZ,), _I32),
    "ack_vq_adamw_step": ((_P,) * 9 + (_SZ, _U32, _U32), _I32),
    "ack_abi_info": ((ctypes.POINTER(AckAbiInfo), _SZ), _I32),
    "ack_device_info": ((_P, ctypes.POINTER(AckDeviceInfo), _SZ), _I32),
}


def library_path() -> Path | None:
    """``ACK_LIBRARY`` if it names a file, else the library built into this
    package, else None."""
    here = Path(__file__).resolve().parent / "_lib" / LIBRARY_NAME
    for candidate in (os.environ.get("ACK_LIBRARY"), here):
        if candidate and Path(candidate).is_file():
            return Path(candidate)
    return None


class Library:
    """libackvq.so loaded once per process, every entry point declared."""

    def __init__(self, path: Path) -> None:
        self.path = Path(path)
        self.cdll = ctypes.CDLL(str(self.path))
        missing = [name for name in _ENTRY_POINTS if not hasattr(self.cdll, name)]
        if missing:
            raise AckUnavailable(f"{self.path} lacks {', '.join(missing)}; rebuild it")
        for name, (args, result) in _ENTRY_POINTS.items():
            entry = getattr(self.cdll, name)
            entry.argtypes, entry.restype = list(args), result

    def last_error(self) -> str:
        """This thread's last error message from the library."""
        text = ctypes.create_string_buffer(1024)
        self.cdll.ack_last_error(text, len(text))
        return text.value.decode("utf-8", errors="replace")

    def check(self, rc: int, context: str) -> None:
        """Raise the exception of a nonzero return code, with the message."""
        if rc != ACK_OK:
            raise _EXCEPTION_FOR_CODE.get(rc, AckError)(f"{context}: {self.last_error()}")


_loaded: Library | None = None
_load_guard = threading.Lock()


def library() -> Library:
    """The process's Library; AckUnavailable when nothing is built."""
    global _loaded
    with _load_guard:
        if _loaded is None:
            path = library_path()
            if path is None:
                raise AckUnavailable(
                    f"{LIBRARY_NAME} is not built; run alelyon-compute-kit_amd/build.py")
            _loaded = Library(path)
        return _loaded


_lib = library  # the name the tests' fixtures use


def _byte_count(nbytes) -> int:
    if isinstance(nbytes, (bool, np.bool_)):
        raise AckError("nbytes must be a positive integer, not a boolean")
    if not isinstance(nbytes, numbers.Integral):
        raise AckError("nbytes must be a positive integer")
    count = int(nbytes)
    if count < 1 or count > MAX_BUFFER_BYTES:
        raise AckError(f"nbytes must be in 1..{MAX_BUFFER_BYTES}")
    return count


def _transfer_dtype(dtype) -> np.dtype:
    try:
        dt = np.dtype(dtype)
    except (TypeError, ValueError) as exc:
        raise AckError("unsupported buffer dtype") from exc
    plain = dt.fields is None and dt.subdtype is None and not dt.hasobject
    if not plain or (dt.kind, dt.itemsize) not in _TRANSFER_TYPES:
        raise AckError(f"unsupported buffer dtype {dt} is refused; use a plain "
                       "fixed-width numeric or bool dtype")
    return dt


def _release_dropped(device: "Device", handle: int) -> None:
    """Finaliser of a Buffer that was never freed."""
    try:
        device._release(handle)
    except AckError as exc:
        warnings.warn(f"ack.Buffer finaliser: {exc}", ResourceWarning, stacklevel=2)


class Device:
    """One HIP device. Free its buffers before close(); calls are serialised
    under the device's re-entrant lock."""

    def __init__(self) -> None:
        self.lib = library()
        self.lock = threading.RLock()
        self._live: set[int] = set()
        self._handle = self.lib.cdll.ack_open()
        if not self._handle:
            raise AckUnavailable(f"ack_open: {self.lib.last_error()}")
        try:
            label = ctypes.create_string_buffer(256)
            self.lib.check(self.lib.cdll.ack_device_name(self._handle, label, len(label)),
                           "device name")
            self.name = label.value.decode("utf-8", errors="replace")
        except BaseException:
            self.close()
            raise

    # -- the handle every entry point takes ---------------------------------
    @property
    def handle(self) -> int:
        """The open device's handle; AckError once closed."""
        if not self._handle:
            raise AckError("device is closed")
        return self._handle

    def call(self, entry: str, *args, context: str | None = None) -> None:
        """Call a status-returning entry point on this device under its lock
        and raise on a nonzero code."""
        with self.lock:
            rc = getattr(self.lib.cdll, entry)(self.handle, *args)
            self.lib.check(rc, context or entry)

    # -- buffers -----------------------------------------------------------------
    def buffer(self, nbytes: int) -> "Buffer":
        return Buffer(self, nbytes)

    def _allocate(self, nbytes: int) -> int:
        with self.lock:
            handle = self.lib.cdll.ack_buffer_alloc(self.handle, nbytes)
            if not handle:
                raise AckError(f"buffer alloc: {self.lib.last_error()}")
            self._live.add(handle)
            return handle

    def _release(self, handle: int) -> None:
        with self.lock:
            if handle not in self._live:
                return
            self._live.discard(handle)  # whatever the library answers, it is gone here
            self.lib.check(self.lib.cdll.ack_buffer_free(self.handle, handle), "free")

    # -- lifetime ------------------------------------------------------------
    def close(self) -> None:
        """Free the device only on ACK_OK; a refusal keeps the handle valid,
        except when the library already considers it closed."""
        with self.lock:
            if not self._handle:
                return
            if self._live:
                raise AckError("device has live buffers still allocated; free them before close")
            rc = self.lib.cdll.ack_close(self._handle)
            if rc in (ACK_OK, ACK_ERR_CLOSED):
                self._handle = None
            if rc != ACK_OK:
                raise AckError(f"close: {self.lib.last_error()}")

    def __enter__(self) -> "Device":
        self.handle  # refuses a closed device
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    # -- stream control and diagnostics ----------------------------------------
    def info(self) -> AckDeviceInfo:
        """``ack_device_info`` of this device."""
        out = AckDeviceInfo()
        with self.lock:
            self.lib.check(self.lib.cdll.ack_device_info(self.handle, ctypes.byref(out),
                                                         ctypes.sizeof(out)), "device info")
        return out

    def capability_record(self) -> dict:
        """The record of what this run ran on, in the reference's shape
        (``capability_record(abi_info(), self.info())``)."""
        return capability_record(abi_info(self.lib), self.info())

    def synchronize(self) -> None:
        self.call("ack_sync", context="sync")

    def timer_start(self) -> None:
        """Record a start event on the device stream (benchmarks)."""
        self.call("ack_stream_timer", 0, None, context="timer")

    def timer_stop(self) -> float:
        """Record a stop event, wait for it, return milliseconds since start."""
        elapsed = ctypes.c_float()
        self.call("ack_stream_timer", 1, ctypes.byref(elapsed), context="timer")
        return float(elapsed.value)

    def set_policy(self, policy: int) -> None:
        """0: automatic kernel choice; 1: the general matmul kernel only;
        2: factorised paths at any size (tests of small shapes)."""
        self.call("ack_vq_set_policy", policy, context="policy")


class Buffer:
    """A device buffer of ``nbytes``; ``free()`` releases it explicitly."""

    def __init__(self, device: Device, nbytes: int) -> None:
        size = _byte_count(nbytes)
        self._device = device
        self._nbytes = size
        self._handle = device._allocate(size)
        self._finalizer = weakref.finalize(self, _release_dropped, device, self._handle)

    @property
    def nbytes(self) -> int:
        return self._nbytes

    @property
    def handle(self) -> int:
        """The live buffer's handle; AckError once freed or its device closed."""
        if not self._handle:
            raise AckError("buffer has been freed")
        self._device.handle
        return self._handle

    def upload(self, data) -> None:
        """Copy a host array of exactly ``nbytes`` into the buffer."""
        host = np.asarray(data)
        _transfer_dtype(host.dtype)
        if host.nbytes != self._nbytes:
            raise AckError(f"upload of {host.nbytes} bytes into a {self._nbytes}-byte buffer")
        host = np.ascontiguousarray(host)
        self._device.call("ack_upload", self.handle, host.ctypes.data, host.nbytes,
                          context="upload")

    def download(self, dtype) -> np.ndarray:
        """The buffer's bytes as a new 1-D host array of ``dtype`` (waits for
        the device stream)."""
        dt = _transfer_dtype(dtype)
        count, rest = divmod(self._nbytes, dt.itemsize)
        if rest:
            raise AckError(f"buffer size {self._nbytes} is not divisible by dtype itemsize "
                           f"{dt.itemsize}; a transfer requires a whole number of elements")
        host = np.empty(count, dtype=dt)
        self._device.call("ack_download", self.handle, host.ctypes.data, host.nbytes,
                          context="download")
        return host

    def copy_from(self, src: "Buffer", nbytes: int, *, offset: int = 0,
                  src_offset: int = 0) -> None:
        """Enqueue a device-to-device copy of ``nbytes`` from ``src``."""
        self._device.call("ack_buffer_copy", self.handle, offset, src.handle, src_offset, nbytes,
                          context="copy")

    def free(self) -> None:
        """Release the buffer; a second call does nothing."""
        if not self._handle:
            return
        self._device.handle  # freeing through a closed device is refused
        handle, self._handle = self._handle, None
        self._finalizer.detach()
        self._device._release(handle)


def abi_info(lib: Library | None = None) -> AckAbiInfo:
    """``ack_abi_info`` of the loaded library."""
    lib = lib or library()
    out = AckAbiInfo()
    lib.check(lib.cdll.ack_abi_info(ctypes.byref(out), ctypes.sizeof(out)), "abi info")
    return out


def _api_version_string(packed: int) -> str:
    return f"{(packed >> 22) & 0x7F}.{(packed >> 12) & 0x3FF}.{packed & 0xFFF}"


def capability_record(abi: AckAbiInfo, info: AckDeviceInfo) -> dict:
    """A JSON-serialisable record of what a run ran on, with the keys of the
    reference's record (src/alelyon_compute_kit/_kit/python/ack.py:527-596)
    plus ``abi.vq_schema`` (the vq4 schema this library serves). Every value
    is declared by this library and the HIP runtime; the operator families the
    reference lists are absent here (0)."""
    lib = library()
    return {
        "schema": 1,
        "abi": {
            "version": abi.version,
            "operators": abi.operators,
            "vq_schema": int(lib.cdll.ack_vq_schema()),
            "op_schema_matmul_bf16": abi.op_schema_matmul_bf16,
            "op_schema_cast": abi.op_schema_cast,
            "op_schema_matmul_f32": abi.op_schema_matmul_f32,
            "op_schema_matmul_f16": abi.op_schema_matmul_f16,
            "op_schema_index": abi.op_schema_index,
            "op_schema_convert": abi.op_schema_convert,
            "op_schema_intwise": abi.op_schema_intwise,
            "op_schema_pointwise": abi.op_schema_pointwise,
            "reserved_op_schemas": {
                "reduce": abi.op_schema_reduce,
                "rowwise": abi.op_schema_rowwise,
                "loss": abi.op_schema_loss,
                "embedding": abi.op_schema_embedding,
            },
            "shaders": f"{abi.shaders:016x}",
            "build": f"{abi.build:016x}",
            "capabilities": {
                "streams": abi.capability_streams,
                "rng": abi.capability_rng,
                "optimizer": abi.capability_optimizer,
                "serialization": abi.capability_serialization,
            },
        },
        "device": {
            "name": info.device_name.decode("utf-8", errors="replace"),
            "vendor_id": info.vendor_id,
            "device_id": info.device_id,
            "device_type": info.device_type,
            "device_uuid": bytes(info.device_uuid).hex(),
            "driver_uuid": bytes(info.driver_uuid).hex(),
            "driver_id": info.driver_id,
            "driver_version_raw": info.driver_version_raw,
            "driver_name": info.driver_name.decode("utf-8", errors="replace"),
            "driver_info": info.driver_info.decode("utf-8", errors="replace"),
            "api_version": _api_version_string(info.api_version),
            "features": sorted(name for name, bit in ACK_FEATURE_BITS.items()
                               if info.features & bit),
            "subgroup_size": info.subgroup_size,
            "timestamp_valid_bits": info.timestamp_valid_bits,
            "timestamp_period_ns": info.timestamp_period_ns,
            "device_local_bytes": info.device_local_bytes,
            "limits": {
                "max_storage_buffer_bytes": info.max_storage_buffer_bytes,
                "max_push_constant_bytes": info.max_push_constant_bytes,
                "max_workgroup_invocations": info.max_workgroup_invocations,
                "max_workgroup_count": list(info.max_workgroup_count),
                "max_workgroup_size": list(info.max_workgroup_size),
            },
            "matmul": {
                "tile": info.matmul_tile,
                "k_multiple": info.matmul_k_multiple,
                "layouts": [n for i, n in enumerate(("NN", "NT", "TN", "TT"))
                            if info.matmul_layouts & (1 << i)],
                "operand_dtype": ACK_DTYPE_NAMES.get(info.matmul_operand_dtype,
                                                     info.matmul_operand_dtype),
                "result_dtype": ACK_DTYPE_NAMES.get(info.matmul_result_dtype,
                                                    info.matmul_result_dtype),
            },
            "cast_modes": info.cast_modes,
            "identity": f"{info.identity:016x}",
        },
    }
