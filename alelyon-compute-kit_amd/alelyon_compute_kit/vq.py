"""vq4/v1 vector-coded tensors on AMD Instinct MI355X.

Each 4-bit index selects one of 16 FP32 vectors of 8, 16 or 32 values (one
codebook per tensor); eight indices share a little-endian u32 word. This
module keeps the reference's Python surface
(src/alelyon_compute_kit/_kit/python/vq.py:21-410) -- ``storage_layout``,
``VQArray`` with its ``ACKVQ4`` wire image, the CPU ``encode`` and
``fit_codebook``, ``VQDevice`` and ``VQAdamW`` -- with the same signatures,
refusals and results. Device work runs in libackvq.so's gfx950 kernels; the
CPU ``encode`` and ``fit_codebook`` run in the same library's native host
code. Nothing here computes a device result on the CPU: without the library
every device entry raises ``AckUnavailable``.
"""
from __future__ import annotations

import ctypes
import math
import operator
import struct
from contextlib import ExitStack

import numpy as np

from . import ack

SCHEMA = 1
GROUPS = (8, 16, 32)
ENTRIES = 16
MAX_ELEMENTS = 268_435_456
# The reference caps one product at 2^28 multiply-adds because its shader is
# a scalar loop (vq.py:25, vq4_ops.rs:21-23). This library's tiled kernels
# admit 2^38 (libackvq plan.hpp kMaxMatmulMacs).
REFERENCE_MAX_MATMUL_MACS = 268_435_456
MAX_MATMUL_MACS = 1 << 38
_HEADER = struct.Struct("<8sIIIIQQ")   # magic, schema, group, rank, reserved, elements, code bytes
_MAGIC = b"ACKVQ4\0\0"


def _integer(value, name: str, minimum: int, maximum: int) -> int:
    if isinstance(value, (bool, np.bool_)):
        raise ValueError(f"{name} must be an integer")
    try:
        result = operator.index(value)
    except TypeError as exc:
        raise ValueError(f"{name} must be an integer") from exc
    if not minimum <= result <= maximum:
        raise ValueError(f"{name} must be in {minimum}..{maximum}")
    return result


def _shape(shape) -> tuple[int, ...]:
    dims = tuple(_integer(x, "dimension", 1, MAX_ELEMENTS) for x in shape)
    if not 1 <= len(dims) <= 6 or math.prod(dims) > MAX_ELEMENTS:
        raise ValueError("vq shape requires rank 1..6 and a bounded element count")
    return dims


def _group(group) -> int:
    group = _integer(group, "group", 8, 32)
    if group not in GROUPS:
        raise ValueError("vq group must be 8, 16 or 32")
    return group


def _float_array(value, name: str) -> np.ndarray:
    array = np.asarray(value)
    if array.dtype != np.dtype("float32") or not np.isfinite(array).all():
        raise ValueError(f"{name} must contain finite float32 values")
    return np.ascontiguousarray(array)


def _book(value, group: int) -> np.ndarray:
    book = _float_array(value, "codebook")
    if book.shape != (ENTRIES, group):
        raise ValueError(f"codebook must have shape (16, {group})")
    return book


def storage_layout(shape, group: int = 16) -> dict:
    """Byte accounting of one tensor's image (vq.py:70-82)."""
    shape, group = _shape(shape), _group(group)
    elements = math.prod(shape)
    vectors = -(-elements // group)
    code_bytes = -(-vectors // 8) * 4
    book_bytes = ENTRIES * group * 4
    metadata = _HEADER.size + 8 * len(shape)
    total = code_bytes + book_bytes + metadata
    return {"elements": elements, "vectors": vectors, "code_bytes": code_bytes,
            "codebook_bytes": book_bytes, "metadata_bytes": metadata,
            "serialized_bytes": total, "payload_bytes": code_bytes + book_bytes,
            "bits_per_value": 8 * total / elements,
            "sub_bit": 8 * total < elements}


def _unpack_indices(codes: np.ndarray, vectors: int) -> np.ndarray:
    v = np.arange(vectors, dtype=np.int64)
    return (codes[v // 8] >> ((v % 8) * 4).astype(np.uint32)) & np.uint32(15)


class VQArray:
    """An owned, immutable wire image: shape, group, packed codes, codebook.

    No dense master tensor is kept (vq.py:85-151).
    """

    __slots__ = ("shape", "group", "codes", "codebook")

    def __init__(self, shape, group, codes, codebook):
        shape, group = _shape(shape), _group(group)
        layout = storage_layout(shape, group)
        raw = np.asarray(codes)
        if raw.dtype != np.dtype("uint32") or raw.shape != (layout["code_bytes"] // 4,):
            raise ValueError("vq codes must be the exact uint32 word image")
        book = _book(codebook, group)
        # One tensor, one image: nibbles past the last vector must be zero.
        tail = layout["vectors"] % 8
        if tail and int(raw[-1]) >> (4 * tail):
            raise ValueError("vq unused codeword bits must be zero")
        owned_codes, owned_book = raw.copy(), book.copy()
        owned_codes.flags.writeable = False
        owned_book.flags.writeable = False
        object.__setattr__(self, "shape", shape)
        object.__setattr__(self, "group", group)
        object.__setattr__(self, "codes", owned_codes)
        object.__setattr__(self, "codebook", owned_book)

    def __setattr__(self, name, value):
        raise AttributeError("VQArray is immutable")

    def __eq__(self, other):
        if not isinstance(other, VQArray):
            return NotImplemented
        return (self.shape == other.shape and self.group == other.group
                and np.array_equal(self.codes, other.codes)
                and np.array_equal(self.codebook, other.codebook))

    __hash__ = None

    def __repr__(self) -> str:
        return f"VQArray(shape={self.shape}, group={self.group})"

    @property
    def layout(self) -> dict:
        return storage_layout(self.shape, self.group)

    def decode(self) -> np.ndarray:
        """CPU gather of the image into a dense float32 array (vq.py:117-121)."""
        layout = self.layout
        idx = _unpack_indices(self.codes, layout["vectors"])
        dense = self.codebook[idx].reshape(-1)[:layout["elements"]]
        return dense.copy().reshape(self.shape)

    def to_bytes(self) -> bytes:
        layout = self.layout
        header = _HEADER.pack(_MAGIC, SCHEMA, self.group, len(self.shape), 0,
                              layout["elements"], layout["code_bytes"])
        dims = struct.pack(f"<{len(self.shape)}Q", *self.shape)
        return (header + dims + self.codebook.astype("<f4").tobytes()
                + self.codes.astype("<u4").tobytes())

    @classmethod
    def from_bytes(cls, data, *, max_bytes: int = 128 * 1024 * 1024) -> "VQArray":
        limit = _integer(max_bytes, "max_bytes", _HEADER.size, 1 << 32)
        view = memoryview(data).cast("B")
        if not _HEADER.size <= view.nbytes <= limit:
            raise ValueError("vq artifact byte limit or truncated header")
        magic, schema, group, rank, reserved, elements, code_bytes = _HEADER.unpack_from(view)
        if magic != _MAGIC or schema != SCHEMA or reserved or not 1 <= rank <= 6:
            raise ValueError("unsupported vq artifact header")
        dims_end = _HEADER.size + 8 * rank
        if view.nbytes < dims_end:
            raise ValueError("truncated vq dimensions")
        shape = struct.unpack_from(f"<{rank}Q", view, _HEADER.size)
        layout = storage_layout(shape, group)
        if elements != layout["elements"] or code_bytes != layout["code_bytes"]:
            raise ValueError("vq header disagrees with its dimensions")
        if view.nbytes != layout["serialized_bytes"]:
            raise ValueError("vq artifact length mismatch")
        book_end = dims_end + layout["codebook_bytes"]
        book = np.frombuffer(view[dims_end:book_end], dtype="<f4").reshape(ENTRIES, group)
        codes = np.frombuffer(view[book_end:], dtype="<u4")
        return cls(shape, group, codes.astype(np.uint32), book.astype(np.float32))


def _host_lib():
    return ack._lib()


def encode(values, codebook, *, group: int = 16) -> VQArray:
    """CPU reference encode (vq.py:154-179): nearest entry by float64 squared
    distance, lowest index on ties; native host code."""
    group = _group(group)
    x = _float_array(values, "values")
    shape = _shape(x.shape)
    book = _book(codebook, group)
    layout = storage_layout(shape, group)
    words = np.zeros(layout["code_bytes"] // 4, dtype=np.uint32)
    lib = _host_lib()
    rc = lib.cdll.ack_vq_host_encode(x.ctypes.data, x.size, book.ctypes.data, group,
                                     words.ctypes.data)
    if rc != ack.ACK_OK:
        raise ack._kit_error("encode", rc, lib.last_error())
    return VQArray(shape, group, words, book)


def fit_codebook(values, *, group: int = 16, iterations: int = 4,
                 sample_vectors: int = 4096, init=None) -> np.ndarray:
    """Bounded deterministic calibration (vq.py:182-257), native host code.

    Lloyd on a strided sample of at most ``sample_vectors`` complete vectors;
    an entry left empty is reseeded with the sample vector farthest from the
    book, unless a warm start (``init``) from a sample smaller than the
    tensor finds the whole tensor still selecting it.
    """
    group = _group(group)
    iterations = _integer(iterations, "iterations", 0, 32)
    sample_vectors = _integer(sample_vectors, "sample_vectors", ENTRIES, 65536)
    x = _float_array(values, "values").reshape(-1)
    if x.size < group:
        raise ValueError("codebook calibration needs at least one complete vector")
    warm = None if init is None else _book(init, group)
    book = np.empty((ENTRIES, group), dtype=np.float32)
    lib = _host_lib()
    rc = lib.cdll.ack_vq_host_fit_codebook(
        x.ctypes.data, x.size, group, iterations, sample_vectors,
        None if warm is None else warm.ctypes.data, book.ctypes.data)
    if rc != ack.ACK_OK:
        raise ack._kit_error("fit_codebook", rc, lib.last_error())
    return book


def _plan(words) -> bytes:
    return struct.pack("<8I", *words)


class VQDevice:
    """Synchronous, status-checked vq4 operations on an open ``ack.Device``.

    Each call uploads its packed operands, runs on the GPU, checks the status
    word and downloads the result (vq.py:260-365). ``run`` is the resident
    form for callers that keep operands in device buffers.
    """

    def __init__(self, device: ack.Device):
        self.device = device
        with device._lock:
            device._require_open()
            lib = device._lib.cdll
            if lib.ack_vq_schema() != SCHEMA:
                raise ack.AckUnavailable("incompatible vq4 extension schema")
            self._lib = device._lib

    # -- resident interface ------------------------------------------------
    def run(self, words, inputs, out: ack.Buffer, status: ack.Buffer, *, count: int = 1) -> None:
        """Enqueue one plan on resident buffers; does not wait or check status.

        ``inputs`` are 1-4 ``ack.Buffer``; missing slots alias the first, as
        the reference's ``_run`` does (vq.py:298-299). ``count`` > 1 runs the
        batched entry over back-to-back instances.
        """
        device = self.device
        with device._lock:
            device._require_open()
            slots = list(inputs)
            while len(slots) < 4:
                slots.append(slots[0])
            plan = _plan(words)
            if count == 1:
                rc = self._lib.cdll.ack_vq(device._handle, *(b._handle for b in slots),
                                           out._handle, status._handle, plan, len(plan))
            else:
                rc = self._lib.cdll.ack_vq_batch(device._handle, *(b._handle for b in slots),
                                                 out._handle, status._handle, plan, len(plan),
                                                 count)
            if rc != ack.ACK_OK:
                raise ack._kit_error("vq", rc, self._lib.last_error())

    def _run(self, words, arrays, output_bytes: int, dtype, *, count: int = 1):
        device = self.device
        with device._lock, ExitStack() as cleanup:
            device._require_open()
            buffers = []
            for array in arrays:
                b = device.buffer(array.nbytes)
                cleanup.callback(b.free)
                b.upload(array)
                buffers.append(b)
            out = device.buffer(output_bytes)
            cleanup.callback(out.free)
            status = device.buffer(4)
            cleanup.callback(status.free)
            status.upload(np.zeros(1, dtype=np.uint32))
            self.run(words, buffers, out, status, count=count)
            flags = int(status.download(np.uint32)[0])
            if flags:
                raise ack.AckError(f"vq device arithmetic refused: status={flags}")
            return out.download(dtype)

    def fit_resident(self, values: ack.Buffer, elements: int, book: ack.Buffer,
                     status: ack.Buffer, *, group: int = 16, iterations: int = 4,
                     sample_vectors: int = 4096, init: ack.Buffer | None = None) -> None:
        """Enqueue ``fit_codebook`` of ``elements`` FP32 values held in a device
        buffer; the 16 x group book lands in ``book``. Does not wait or check
        status (bit 1: a nonfinite sampled value or init entry)."""
        group = _group(group)
        iterations = _integer(iterations, "iterations", 0, 32)
        sample_vectors = _integer(sample_vectors, "sample_vectors", ENTRIES, 65536)
        device = self.device
        with device._lock:
            device._require_open()
            rc = self._lib.cdll.ack_vq_fit_codebook(
                device._handle, values._handle, None if init is None else init._handle,
                book._handle, status._handle, elements, group, iterations, sample_vectors)
            if rc != ack.ACK_OK:
                raise ack._kit_error("fit_codebook", rc, self._lib.last_error())

    def fit_codebook(self, values, *, group: int = 16, iterations: int = 4,
                     sample_vectors: int = 4096, init=None) -> np.ndarray:
        """``fit_codebook`` (vq.py:182-257) computed on the GPU: the same
        refusals and the same book, bit for bit."""
        group = _group(group)
        iterations = _integer(iterations, "iterations", 0, 32)
        sample_vectors = _integer(sample_vectors, "sample_vectors", ENTRIES, 65536)
        x = _float_array(values, "values").reshape(-1)
        if x.size < group:
            raise ValueError("codebook calibration needs at least one complete vector")
        warm = None if init is None else _book(init, group)
        device = self.device
        with device._lock, ExitStack() as cleanup:
            device._require_open()

            def upload(array):
                b = device.buffer(array.nbytes)
                cleanup.callback(b.free)
                b.upload(array)
                return b

            values_buf = upload(x)
            init_buf = None if warm is None else upload(warm)
            book = device.buffer(ENTRIES * group * 4)
            cleanup.callback(book.free)
            status = upload(np.zeros(1, dtype=np.uint32))
            self.fit_resident(values_buf, x.size, book, status, group=group,
                              iterations=iterations, sample_vectors=sample_vectors,
                              init=init_buf)
            flags = int(status.download(np.uint32)[0])
            if flags:
                raise ack.AckError(f"vq device arithmetic refused: status={flags}")
            return book.download(np.float32).reshape(ENTRIES, group)

    def path_name(self, words) -> str:
        """The kernel path the library takes for a plan."""
        buf = ctypes.create_string_buffer(64)
        plan = _plan(words)
        rc = self._lib.cdll.ack_vq_path_name(plan, len(plan), buf, len(buf))
        if rc != ack.ACK_OK:
            raise ack._kit_error("vq", rc, self._lib.last_error())
        return buf.value.decode()

    # -- the reference surface ---------------------------------------------
    def encode(self, values, codebook, *, group: int = 16) -> VQArray:
        group = _group(group)
        x = _float_array(values, "values")
        layout = storage_layout(x.shape, group)
        book = _book(codebook, group)
        codes = self._run((0, x.size, 1, 1, group, ENTRIES, 0, 0), (x, book),
                          layout["code_bytes"], np.uint32)
        return VQArray(x.shape, group, codes, book)

    def decode(self, value: VQArray) -> np.ndarray:
        layout = value.layout
        dense = self._run((1, layout["elements"], 1, 1, value.group, ENTRIES, 0, 0),
                          (value.codes, value.codebook), layout["elements"] * 4, np.float32)
        return dense.reshape(value.shape)

    @staticmethod
    def _matmul_geometry(a: VQArray, b: VQArray, transpose_a, transpose_b):
        if type(transpose_a) is not bool or type(transpose_b) is not bool:
            raise ValueError("transpose flags must be boolean")
        if len(a.shape) != 2 or len(b.shape) != 2 or a.group != b.group:
            raise ValueError("vq matmul requires two matrices using the same vector group")
        m, k = a.shape[::-1] if transpose_a else a.shape
        k2, n = b.shape[::-1] if transpose_b else b.shape
        if k != k2 or max(m, n, k) > 65536 or m * n > MAX_ELEMENTS:
            raise ValueError("vq matmul dimensions are incompatible or exceed bounds")
        if m * n * k > MAX_MATMUL_MACS:
            raise ValueError("vq-matmul-work-limit: split the product into bounded calls")
        return m, n, k, int(transpose_a) | (int(transpose_b) << 1)

    def matmul(self, a: VQArray, b: VQArray, *, transpose_a=False, transpose_b=False) -> np.ndarray:
        m, n, k, flags = self._matmul_geometry(a, b, transpose_a, transpose_b)
        out = self._run((2, m, n, k, a.group, ENTRIES, flags, 0),
                        (a.codes, a.codebook, b.codes, b.codebook), m * n * 4, np.float32)
        return out.reshape(m, n)

    def matmul_batch(self, a, b, *, transpose_a=False, transpose_b=False) -> np.ndarray:
        """``[op(a[i]) @ op(b[i]) for i]`` as one batched launch
        (``ack_vq_batch``): the operands of every instance share shapes and
        group, their packed images are laid back to back. Returns
        ``(count, m, n)`` float32."""
        a, b = list(a), list(b)
        if not a or len(a) != len(b):
            raise ValueError("vq batched matmul needs one right operand per left operand")
        if any(x.shape != a[0].shape or x.group != a[0].group for x in a) or \
                any(y.shape != b[0].shape or y.group != b[0].group for y in b):
            raise ValueError("vq batched matmul operands must share shapes and group")
        m, n, k, flags = self._matmul_geometry(a[0], b[0], transpose_a, transpose_b)
        arrays = (np.concatenate([x.codes for x in a]),
                  np.concatenate([x.codebook.reshape(-1) for x in a]),
                  np.concatenate([y.codes for y in b]),
                  np.concatenate([y.codebook.reshape(-1) for y in b]))
        out = self._run((2, m, n, k, a[0].group, ENTRIES, flags, 0), arrays,
                        len(a) * m * n * 4, np.float32, count=len(a))
        return out.reshape(len(a), m, n)

    @staticmethod
    def _dense_geometry(x: np.ndarray, b: VQArray, transpose_a, transpose_b):
        if type(transpose_a) is not bool or type(transpose_b) is not bool:
            raise ValueError("transpose flags must be boolean")
        if x.ndim != 2 or len(b.shape) != 2:
            raise ValueError("vq dense matmul requires a dense matrix and a vq matrix")
        m, k = x.shape[::-1] if transpose_a else x.shape
        k2, n = b.shape[::-1] if transpose_b else b.shape
        if k != k2 or max(m, n, k) > 65536 or m * n > MAX_ELEMENTS or m * k > MAX_ELEMENTS:
            raise ValueError("vq matmul dimensions are incompatible or exceed bounds")
        if m * n * k > MAX_MATMUL_MACS:
            raise ValueError("vq-matmul-work-limit: split the product into bounded calls")
        return m, n, k, int(transpose_a) | (int(transpose_b) << 1)

    def matmul_dense(self, x, b: VQArray, *, transpose_a=False, transpose_b=False) -> np.ndarray:
        """``op(x) @ op(b)`` with ``x`` a dense float32 matrix: the packed
        product without encoding the activations (an extension; ``matmul``
        keeps the reference's semantics)."""
        x = _float_array(x, "dense operand")
        m, n, k, flags = self._dense_geometry(x, b, transpose_a, transpose_b)
        device = self.device
        with device._lock, ExitStack() as cleanup:
            device._require_open()
            bufs = []
            for array in (x, b.codes, b.codebook):
                buf = device.buffer(array.nbytes)
                cleanup.callback(buf.free)
                buf.upload(array)
                bufs.append(buf)
            out = device.buffer(m * n * 4)
            cleanup.callback(out.free)
            status = device.buffer(4)
            cleanup.callback(status.free)
            status.upload(np.zeros(1, dtype=np.uint32))
            self.run_dense((2, m, n, k, b.group, ENTRIES, flags, 0), *bufs, out, status)
            flags_out = int(status.download(np.uint32)[0])
            if flags_out:
                raise ack.AckError(f"vq device arithmetic refused: status={flags_out}")
            return out.download(np.float32).reshape(m, n)

    def run_dense(self, words, x: ack.Buffer, b_codes: ack.Buffer, b_book: ack.Buffer,
                  out: ack.Buffer, status: ack.Buffer) -> None:
        """Enqueue the dense-activation product on resident buffers (an op-2
        plan; ``x`` holds m x k float32); does not wait or check status."""
        device = self.device
        with device._lock:
            device._require_open()
            plan = _plan(words)
            rc = self._lib.cdll.ack_vq_matmul_dense(device._handle, x._handle, b_codes._handle,
                                                    b_book._handle, out._handle, status._handle,
                                                    plan, len(plan))
            if rc != ack.ACK_OK:
                raise ack._kit_error("vq", rc, self._lib.last_error())

    def dense_path_name(self, words) -> str:
        """The kernel path the dense-activation product takes for an op-2 plan."""
        buf = ctypes.create_string_buffer(64)
        plan = _plan(words)
        rc = self._lib.cdll.ack_vq_dense_path_name(plan, len(plan), buf, len(buf))
        if rc != ack.ACK_OK:
            raise ack._kit_error("vq", rc, self._lib.last_error())
        return buf.value.decode()

    @staticmethod
    def _adamw_inputs(weight, momentum, variance, gradient, lr, beta1, beta2, eps,
                      weight_decay, step):
        states = (weight, momentum, variance, gradient)
        if any(s.shape != weight.shape or s.group != weight.group for s in states):
            raise ValueError("vq AdamW states must have identical shapes and groups")
        count = weight.layout["elements"]
        if count * 3 > MAX_ELEMENTS:
            raise ValueError("vq AdamW active scratch exceeds element bound")
        coefficients = VQDevice.adamw_coefficients(lr, beta1, beta2, eps, weight_decay, step)
        codes = np.concatenate([s.codes for s in states])
        books = np.concatenate([s.codebook.reshape(-1) for s in states])
        return count, codes, books, coefficients

    @staticmethod
    def adamw_coefficients(lr, beta1, beta2, eps, weight_decay, step) -> np.ndarray:
        """Op 3's seven float32 coefficients (vq.py:348-360), with the same
        refusals."""
        step = _integer(step, "step", 1, 1 << 53)
        values = (lr, beta1, beta2, eps, weight_decay)
        if any(isinstance(x, (bool, np.bool_)) or not math.isfinite(float(x)) for x in values):
            raise ValueError("vq AdamW coefficients must be finite numbers")
        if lr < 0 or not 0 <= beta1 < 1 or not 0 <= beta2 < 1 or eps <= 0 or weight_decay < 0:
            raise ValueError("vq AdamW coefficients outside their domains")
        # Bias corrections in Python float64, then rounded to float32 (vq.py:357-358).
        coefficients = np.array([lr, beta1, beta2, eps, weight_decay,
                                 1 - beta1 ** step, 1 - beta2 ** step], dtype=np.float32)
        if (not np.isfinite(coefficients).all() or coefficients[3] <= 0
                or (coefficients[5:] <= 0).any()):
            raise ValueError("vq AdamW coefficients are not representable in float32")
        return coefficients

    def adamw(self, weight: VQArray, momentum: VQArray, variance: VQArray,
              gradient: VQArray, *, lr: float, beta1: float, beta2: float,
              eps: float, weight_decay: float, step: int) -> tuple[np.ndarray, ...]:
        """Op 3: AdamW from four coded states into FP32 scratch [W', M', V']."""
        count, codes, books, coefficients = self._adamw_inputs(
            weight, momentum, variance, gradient, lr, beta1, beta2, eps, weight_decay, step)
        result = self._run((3, count, 1, 1, weight.group, ENTRIES, 0, 0),
                           (codes, books, coefficients), count * 3 * 4, np.float32)
        return tuple(x.reshape(weight.shape) for x in np.split(result, 3))

    def adamw_step_resident(self, codes: ack.Buffer, books: ack.Buffer, coefficients: ack.Buffer,
                            out_codes: ack.Buffer, out_books: ack.Buffer, changed: ack.Buffer,
                            status: ack.Buffer, *, count: int, group: int,
                            iterations: int = 4, sample_vectors: int = 4096) -> None:
        """Enqueue the fused step on resident buffers (the op-3 inputs as
        ``adamw`` lays them out); does not wait or check status."""
        group = _group(group)
        iterations = _integer(iterations, "iterations", 0, 32)
        sample_vectors = _integer(sample_vectors, "sample_vectors", ENTRIES, 65536)
        device = self.device
        with device._lock:
            device._require_open()
            plan = _plan((3, count, 1, 1, group, ENTRIES, 0, 0))
            rc = self._lib.cdll.ack_vq_adamw_step(
                device._handle, codes._handle, books._handle, coefficients._handle,
                out_codes._handle, out_books._handle, changed._handle, status._handle,
                plan, len(plan), iterations, sample_vectors)
            if rc != ack.ACK_OK:
                raise ack._kit_error("vq", rc, self._lib.last_error())

    def adamw_step(self, weight: VQArray, momentum: VQArray, variance: VQArray,
                   gradient: VQArray, *, lr: float, beta1: float, beta2: float,
                   eps: float, weight_decay: float, step: int, iterations: int = 4,
                   sample_vectors: int = 4096):
        """The fused optimizer step: op-3 arithmetic, warm-started refit of each
        state's book, and re-encode, with no dense scratch. Returns the new
        (weight, momentum, variance) images and the changed-weight count --
        the values ``VQAdamW.step`` would reach through ``adamw``,
        ``fit_codebook`` and ``encode``."""
        count, codes, books, coefficients = self._adamw_inputs(
            weight, momentum, variance, gradient, lr, beta1, beta2, eps, weight_decay, step)
        if count < weight.group:
            raise ValueError("codebook calibration needs at least one complete vector")
        iterations = _integer(iterations, "iterations", 0, 32)
        sample_vectors = _integer(sample_vectors, "sample_vectors", ENTRIES, 65536)
        words = weight.layout["code_bytes"] // 4
        group = weight.group
        device = self.device
        with device._lock, ExitStack() as cleanup:
            device._require_open()
            bufs = []
            for array in (codes, books, coefficients):
                b = device.buffer(array.nbytes)
                cleanup.callback(b.free)
                b.upload(array)
                bufs.append(b)
            out_codes = device.buffer(3 * words * 4)
            cleanup.callback(out_codes.free)
            out_books = device.buffer(3 * ENTRIES * group * 4)
            cleanup.callback(out_books.free)
            changed = device.buffer(4)
            cleanup.callback(changed.free)
            status = device.buffer(4)
            cleanup.callback(status.free)
            status.upload(np.zeros(1, dtype=np.uint32))
            self.adamw_step_resident(*bufs, out_codes, out_books, changed, status, count=count,
                                     group=group, iterations=iterations,
                                     sample_vectors=sample_vectors)
            flags = int(status.download(np.uint32)[0])
            if flags:
                raise ack.AckError(f"vq device arithmetic refused: status={flags}")
            new_codes = out_codes.download(np.uint32).reshape(3, words)
            new_books = out_books.download(np.float32).reshape(3, ENTRIES, group)
            moved = int(changed.download(np.uint32)[0])
        images = tuple(VQArray(weight.shape, group, new_codes[i], new_books[i]) for i in range(3))
        return images, moved


class VQAdamW:
    """AdamW whose persistent weight and both moments are vq4 images
    (vq.py:368-410). A failed step leaves the three images and the step
    counter unchanged; durable commits are the caller's.

    With a ``VQDevice`` backend the step runs fused (``VQDevice.adamw_step``);
    any other backend gets the reference's sequence ``adamw`` ->
    ``fit_codebook`` -> ``encode``, which keeps host-only fakes working.
    """

    def __init__(self, backend, weight: VQArray, *, lr=1e-3, betas=(0.9, 0.95), eps=1e-8,
                 weight_decay=0.0):
        self.backend = backend
        self.weight = weight
        zeros = np.zeros_like(weight.codes)
        zero_book = np.zeros((ENTRIES, weight.group), dtype=np.float32)
        self.momentum = VQArray(weight.shape, weight.group, zeros, zero_book)
        self.variance = VQArray(weight.shape, weight.group, zeros, zero_book)
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.steps = 0

    def step(self, gradient: VQArray) -> dict:
        next_step = self.steps + 1
        kwargs = dict(lr=self.lr, beta1=self.betas[0], beta2=self.betas[1], eps=self.eps,
                      weight_decay=self.weight_decay, step=next_step)
        if isinstance(self.backend, VQDevice):
            encoded, changed = self.backend.adamw_step(
                self.weight, self.momentum, self.variance, gradient, **kwargs)
            words = self.weight.layout["code_bytes"] + ENTRIES * self.weight.group * 4
            native_bytes = 3 * words + 4
            calibration = "device float64 fit on the strided sample (the host fit's books)"
        else:
            scratch = self.backend.adamw(self.weight, self.momentum, self.variance, gradient,
                                         **kwargs)
            # Each updated array warm-starts from its own state's book: the
            # pairing must be exact, so a wrong count is refused, not zipped.
            if len(scratch) != 3:
                raise ValueError(f"vq AdamW update returned {len(scratch)} arrays, not 3")
            encoded = []
            for value, state in zip(scratch, (self.weight, self.momentum, self.variance)):
                book = fit_codebook(value, group=self.weight.group, init=state.codebook)
                encoded.append(self.backend.encode(value, book, group=self.weight.group))
            changed = int(np.count_nonzero(encoded[0].decode() != self.weight.decode()))
            native_bytes = sum(s.nbytes for s in scratch)
            calibration = "native float64 fit of FP32 scratch"
        self.weight, self.momentum, self.variance = encoded
        self.steps = next_step
        return {"step": self.steps, "changed_weight_values": changed,
                "persistent_state_bytes": sum(s.layout["serialized_bytes"] for s in encoded),
                "gradient_bytes": gradient.layout["serialized_bytes"],
                "native_update_output_bytes": native_bytes,
                "calibration": calibration,
                "model_quality_validated": False}
