"""vq4/v1 vector-coded tensors on AMD Instinct MI355X.

A vq4 tensor stores one 4-bit index per group of 8, 16 or 32 FP32 values,
eight indices to a little-endian u32 word, and one 16-entry FP32 codebook.
This module is the drop-in Python surface of the reference's vq4 extension
(src/alelyon_compute_kit/_kit/python/vq.py:21-410): ``storage_layout``,
``VQArray`` and its ``ACKVQ4`` wire image, the CPU ``encode`` and
``fit_codebook``, ``VQDevice`` and ``VQAdamW``, with the reference's
signatures, refusal texts and results.

Device work runs in libackvq.so's gfx950 kernels and the CPU ``encode`` and
``fit_codebook`` in the same library's native host code; nothing here
computes a device result in Python. Without the library every entry raises
``ack.AckUnavailable``.
"""
from __future__ import annotations

import ctypes
import math
import operator
from dataclasses import dataclass

import numpy as np

from . import ack

SCHEMA = 1
GROUPS = (8, 16, 32)
ENTRIES = 16
MAX_ELEMENTS = 1 << 28
MAX_DIM = 65536
# The reference caps one product at 2^28 multiply-adds because its shader is
# a scalar loop (vq.py:25, vq4_ops.rs:21-23). This library's kernels admit
# 2^38 (libackvq plan.hpp kMaxMatmulMacs).
REFERENCE_MAX_MATMUL_MACS = 1 << 28
MAX_MATMUL_MACS = 1 << 38
MAX_IMAGE_BYTES = 128 * 1024 * 1024

_MAGIC = b"ACKVQ4\0\0"
# The 40-byte image header, little-endian (vq.py:26).
_HEADER = np.dtype([("magic", "V8"), ("schema", "<u4"), ("group", "<u4"), ("rank", "<u4"),
                    ("reserved", "<u4"), ("elements", "<u8"), ("code_bytes", "<u8")])


# ---- arguments ------------------------------------------------------------------
def _bounded_int(value, name: str, low: int, high: int) -> int:
    """An integer argument in low..high; booleans are not integers here."""
    if isinstance(value, (bool, np.bool_)):
        raise ValueError(f"{name} must be an integer")
    try:
        number = operator.index(value)
    except TypeError:
        raise ValueError(f"{name} must be an integer") from None
    if not low <= number <= high:
        raise ValueError(f"{name} must be in {low}..{high}")
    return number


def _checked_group(group) -> int:
    value = _bounded_int(group, "group", min(GROUPS), max(GROUPS))
    if value not in GROUPS:
        raise ValueError("vq group must be 8, 16 or 32")
    return value


def _checked_shape(shape) -> tuple[int, ...]:
    dims = tuple(_bounded_int(d, "dimension", 1, MAX_ELEMENTS) for d in shape)
    if len(dims) not in range(1, 7) or math.prod(dims) > MAX_ELEMENTS:
        raise ValueError("vq shape requires rank 1..6 and a bounded element count")
    return dims


def _finite_f32(value, name: str) -> np.ndarray:
    array = np.asarray(value)
    if array.dtype != np.float32 or not np.isfinite(array).all():
        raise ValueError(f"{name} must contain finite float32 values")
    return np.ascontiguousarray(array)


def _checked_book(value, group: int) -> np.ndarray:
    book = _finite_f32(value, "codebook")
    if book.shape != (ENTRIES, group):
        raise ValueError(f"codebook must have shape (16, {group})")
    return book


# ---- geometry of one image --------------------------------------------------------
@dataclass(frozen=True)
class _Geometry:
    """Byte accounting of one tensor's image (vq.py:70-82)."""

    shape: tuple[int, ...]
    group: int

    @classmethod
    def of(cls, shape, group) -> "_Geometry":
        return cls(_checked_shape(shape), _checked_group(group))

    @property
    def elements(self) -> int:
        return math.prod(self.shape)

    @property
    def vectors(self) -> int:
        return -(-self.elements // self.group)

    @property
    def words(self) -> int:
        return -(-self.vectors // 8)

    @property
    def code_bytes(self) -> int:
        return 4 * self.words

    @property
    def codebook_bytes(self) -> int:
        return 4 * ENTRIES * self.group

    @property
    def metadata_bytes(self) -> int:
        return _HEADER.itemsize + 8 * len(self.shape)

    @property
    def serialized_bytes(self) -> int:
        return self.metadata_bytes + self.codebook_bytes + self.code_bytes

    def as_dict(self) -> dict:
        total = self.serialized_bytes
        return {"elements": self.elements, "vectors": self.vectors,
                "code_bytes": self.code_bytes, "codebook_bytes": self.codebook_bytes,
                "metadata_bytes": self.metadata_bytes, "serialized_bytes": total,
                "payload_bytes": self.code_bytes + self.codebook_bytes,
                "bits_per_value": 8 * total / self.elements,
                "sub_bit": 8 * total < self.elements}


def storage_layout(shape, group: int = 16) -> dict:
    """Byte accounting of one tensor's vq4 image: elements, vectors, code,
    codebook and metadata bytes, the serialized total and its bits per value."""
    return _Geometry.of(shape, group).as_dict()


def _nibbles(codes: np.ndarray, vectors: int) -> np.ndarray:
    """One index per vector from the packed words: byte b of the
    little-endian words holds vector 2b in its low nibble and 2b + 1 in its
    high one."""
    octets = np.ascontiguousarray(codes, dtype="<u4").view(np.uint8)
    split = np.empty((octets.size, 2), dtype=np.uint8)
    np.bitwise_and(octets, 15, out=split[:, 0])
    np.right_shift(octets, 4, out=split[:, 1])
    return split.reshape(-1)[:vectors]


# ---- the wire image ----------------------------------------------------------------
class VQArray:
    """An owned, immutable vq4 image: shape, group, the packed uint32 words
    and the (16, group) float32 codebook. No dense master tensor is kept."""

    __slots__ = ("shape", "group", "codes", "codebook")

    def __init__(self, shape, group, codes, codebook):
        geometry = _Geometry.of(shape, group)
        words = np.asarray(codes)
        if words.dtype != np.uint32 or words.shape != (geometry.words,):
            raise ValueError("vq codes must be the exact uint32 word image")
        book = _checked_book(codebook, geometry.group)
        used = geometry.vectors - 8 * (geometry.words - 1)  # nibbles of the last word in use
        if used < 8 and int(words[-1]) >> (4 * used):
            raise ValueError("vq unused codeword bits must be zero")
        frozen_codes = np.array(words, dtype=np.uint32, copy=True)
        frozen_book = np.array(book, dtype=np.float32, copy=True)
        frozen_codes.setflags(write=False)
        frozen_book.setflags(write=False)
        for name, value in (("shape", geometry.shape), ("group", geometry.group),
                            ("codes", frozen_codes), ("codebook", frozen_book)):
            object.__setattr__(self, name, value)

    def __setattr__(self, name, value):
        raise AttributeError("VQArray is immutable")

    def __eq__(self, other):
        if not isinstance(other, VQArray):
            return NotImplemented
        return (self.shape, self.group) == (other.shape, other.group) and \
            np.array_equal(self.codes, other.codes) and \
            np.array_equal(self.codebook.view(np.uint32), other.codebook.view(np.uint32))

    __hash__ = None

    def __repr__(self) -> str:
        return f"VQArray(shape={self.shape}, group={self.group})"

    @property
    def layout(self) -> dict:
        return storage_layout(self.shape, self.group)

    def decode(self) -> np.ndarray:
        """The dense float32 tensor the image stands for (a CPU gather)."""
        geometry = _Geometry(self.shape, self.group)
        rows = self.codebook[_nibbles(self.codes, geometry.vectors)]
        return rows.reshape(-1)[:geometry.elements].reshape(self.shape)

    def to_bytes(self) -> bytes:
        """The ACKVQ4 image: header, u64 dims, the codebook, the code words."""
        geometry = _Geometry(self.shape, self.group)
        head = np.zeros((), dtype=_HEADER)
        head["magic"] = np.void(_MAGIC)
        head["schema"], head["group"], head["rank"] = SCHEMA, self.group, len(self.shape)
        head["elements"], head["code_bytes"] = geometry.elements, geometry.code_bytes
        parts = (head, np.asarray(self.shape, dtype="<u8"), self.codebook.astype("<f4"),
                 self.codes.astype("<u4"))
        return b"".join(part.tobytes() for part in parts)

    @classmethod
    def from_bytes(cls, data, *, max_bytes: int = MAX_IMAGE_BYTES) -> "VQArray":
        """Parse and validate an ACKVQ4 image of at most ``max_bytes``."""
        limit = _bounded_int(max_bytes, "max_bytes", _HEADER.itemsize, 1 << 32)
        raw = memoryview(data).cast("B")
        if not _HEADER.itemsize <= raw.nbytes <= limit:
            raise ValueError("vq artifact byte limit or truncated header")
        head = np.frombuffer(raw, dtype=_HEADER, count=1)[0]
        rank = int(head["rank"])
        if head["magic"].tobytes() != _MAGIC or int(head["schema"]) != SCHEMA \
                or int(head["reserved"]) != 0 or rank not in range(1, 7):
            raise ValueError("unsupported vq artifact header")
        start = _HEADER.itemsize + 8 * rank
        if raw.nbytes < start:
            raise ValueError("truncated vq dimensions")
        dims = np.frombuffer(raw, dtype="<u8", count=rank, offset=_HEADER.itemsize)
        geometry = _Geometry.of(tuple(int(d) for d in dims), int(head["group"]))
        if (int(head["elements"]), int(head["code_bytes"])) != (geometry.elements,
                                                                 geometry.code_bytes):
            raise ValueError("vq header disagrees with its dimensions")
        if raw.nbytes != geometry.serialized_bytes:
            raise ValueError("vq artifact length mismatch")
        book = np.frombuffer(raw, dtype="<f4", count=ENTRIES * geometry.group, offset=start)
        words = np.frombuffer(raw, dtype="<u4", offset=start + geometry.codebook_bytes)
        return cls(geometry.shape, geometry.group, words.astype(np.uint32),
                   book.reshape(ENTRIES, geometry.group).astype(np.float32))


# ---- CPU encode and calibration (native host code) -----------------------------
def encode(values, codebook, *, group: int = 16) -> VQArray:
    """The reference's CPU encode (vq.py:154-179): each vector takes the
    entry nearest by float64 squared distance, the lowest index on ties; a
    final partial vector compares its valid values only."""
    group = _checked_group(group)
    x = _finite_f32(values, "values")
    geometry = _Geometry.of(x.shape, group)
    book = _checked_book(codebook, group)
    words = np.zeros(geometry.words, dtype=np.uint32)
    lib = ack.library()
    lib.check(lib.cdll.ack_vq_host_encode(x.ctypes.data, x.size, book.ctypes.data, group,
                                          words.ctypes.data), "encode")
    return VQArray(geometry.shape, group, words, book)


def _fit_arguments(values, group, iterations, sample_vectors, init):
    group = _checked_group(group)
    iterations = _bounded_int(iterations, "iterations", 0, 32)
    sample_vectors = _bounded_int(sample_vectors, "sample_vectors", ENTRIES, 65536)
    x = _finite_f32(values, "values").reshape(-1)
    if x.size < group:
        raise ValueError("codebook calibration needs at least one complete vector")
    warm = None if init is None else _checked_book(init, group)
    return x, group, iterations, sample_vectors, warm


def fit_codebook(values, *, group: int = 16, iterations: int = 4,
                 sample_vectors: int = 4096, init=None) -> np.ndarray:
    """The reference's bounded deterministic calibration (vq.py:182-257) in
    native host code: Lloyd iterations on a strided sample of at most
    ``sample_vectors`` complete vectors, an emptied entry reseeded with the
    sample vector farthest from the book unless a warm start (``init``) on a
    sample smaller than the tensor finds the whole tensor still using it."""
    x, group, iterations, sample_vectors, warm = _fit_arguments(values, group, iterations,
                                                                sample_vectors, init)
    book = np.empty((ENTRIES, group), dtype=np.float32)
    lib = ack.library()
    lib.check(lib.cdll.ack_vq_host_fit_codebook(
        x.ctypes.data, x.size, group, iterations, sample_vectors,
        None if warm is None else warm.ctypes.data, book.ctypes.data), "fit_codebook")
    return book


def _plan(words) -> bytes:
    """The 32-byte plan block: eight little-endian u32."""
    return np.asarray(words, dtype="<u4").tobytes()


def adamw_coefficients(lr, beta1, beta2, eps, weight_decay, step) -> np.ndarray:
    """Op 3's seven float32 coefficients (vq.py:348-360): lr, beta1, beta2,
    eps, decay and the two bias corrections, taken in Python float64 and
    rounded to float32, with the reference's refusals."""
    step = _bounded_int(step, "step", 1, 1 << 53)
    hyper = (lr, beta1, beta2, eps, weight_decay)
    if any(isinstance(h, (bool, np.bool_)) or not math.isfinite(float(h)) for h in hyper):
        raise ValueError("vq AdamW coefficients must be finite numbers")
    if not (lr >= 0 and 0 <= beta1 < 1 and 0 <= beta2 < 1 and eps > 0 and weight_decay >= 0):
        raise ValueError("vq AdamW coefficients outside their domains")
    block = np.array([*hyper, 1 - beta1 ** step, 1 - beta2 ** step], dtype=np.float32)
    if not np.isfinite(block).all() or not block[3] > 0 or not (block[5:] > 0).all():
        raise ValueError("vq AdamW coefficients are not representable in float32")
    return block


# ---- device calls -----------------------------------------------------------------
class _Transient:
    """The device buffers of one synchronous call: staged host inputs,
    outputs and a zeroed status word, all freed when the call ends. Holds the
    device's lock for the whole call."""

    def __init__(self, device: ack.Device):
        self.device = device
        self.held: list[ack.Buffer] = []

    def __enter__(self) -> "_Transient":
        self.device.lock.acquire()
        try:
            self.device.handle
        except BaseException:
            self.device.lock.release()
            raise
        return self

    def __exit__(self, kind, error, trace) -> None:
        failure = None
        try:
            for buf in reversed(self.held):
                try:
                    buf.free()
                except ack.AckError as exc:
                    failure = failure or exc
        finally:
            self.device.lock.release()
        if failure is not None and kind is None:
            raise failure

    def empty(self, nbytes: int) -> ack.Buffer:
        buf = self.device.buffer(nbytes)
        self.held.append(buf)
        return buf

    def staged(self, array) -> ack.Buffer:
        host = np.ascontiguousarray(array)
        buf = self.empty(host.nbytes)
        buf.upload(host)
        return buf

    def status(self) -> ack.Buffer:
        return self.staged(np.zeros(1, dtype=np.uint32))

    @staticmethod
    def settle(status: ack.Buffer) -> None:
        """Read the status word: any set bit refuses the call's results."""
        flags = int(status.download(np.uint32)[0])
        if flags:
            raise ack.AckError(f"vq device arithmetic refused: status={flags}")


def _product_dims(a_shape, b_shape, transpose_a, transpose_b, what: str):
    if type(transpose_a) is not bool or type(transpose_b) is not bool:
        raise ValueError("transpose flags must be boolean")
    m, k = a_shape[::-1] if transpose_a else a_shape
    kb, n = b_shape[::-1] if transpose_b else b_shape
    if k != kb or max(m, n, k) > MAX_DIM or m * n > MAX_ELEMENTS or \
            (what == "dense" and m * k > MAX_ELEMENTS):
        raise ValueError("vq matmul dimensions are incompatible or exceed bounds")
    if m * n * k > MAX_MATMUL_MACS:
        raise ValueError("vq-matmul-work-limit: split the product into bounded calls")
    return m, n, k, int(transpose_a) | int(transpose_b) << 1


class VQDevice:
    """Synchronous, status-checked vq4 operations on an open ``ack.Device``.

    The reference's methods (``encode``, ``decode``, ``matmul``, ``adamw``)
    upload their packed operands, run on the GPU, read the status word and
    download the result (vq.py:260-365). The resident methods (``run``,
    ``run_dense``, ``fit_resident``, ``adamw_step_resident``) enqueue on
    buffers the caller keeps on the device and neither wait nor check.
    """

    def __init__(self, device: ack.Device):
        self.device = device
        with device.lock:
            device.handle
            if device.lib.cdll.ack_vq_schema() != SCHEMA:
                raise ack.AckUnavailable("incompatible vq4 extension schema")

    # -- resident interface --------------------------------------------------------
    def run(self, words, inputs, out: ack.Buffer, status: ack.Buffer, *, count: int = 1) -> None:
        """Enqueue one plan over 1-4 input buffers (unused slots take the
        first, as the reference's call does, vq.py:298-299); ``count`` > 1 runs
        ``ack_vq_batch`` over back-to-back instances."""
        slots = list(inputs) + [inputs[0]] * (4 - len(inputs))
        handles = [b.handle for b in slots] + [out.handle, status.handle]
        plan = _plan(words)
        if count == 1:
            self.device.call("ack_vq", *handles, plan, len(plan), context="vq")
        else:
            self.device.call("ack_vq_batch", *handles, plan, len(plan), count, context="vq")

    def run_dense(self, words, x: ack.Buffer, b_codes: ack.Buffer, b_book: ack.Buffer,
                  out: ack.Buffer, status: ack.Buffer) -> None:
        """Enqueue the dense-activation product: an op-2 plan whose A is the
        m x k float32 array in ``x``."""
        plan = _plan(words)
        self.device.call("ack_vq_matmul_dense", x.handle, b_codes.handle, b_book.handle,
                         out.handle, status.handle, plan, len(plan), context="vq")

    def fit_resident(self, values: ack.Buffer, elements: int, book: ack.Buffer,
                     status: ack.Buffer, *, group: int = 16, iterations: int = 4,
                     sample_vectors: int = 4096, init: ack.Buffer | None = None) -> None:
        """Enqueue ``fit_codebook`` of ``elements`` float32 values in a device
        buffer; the (16, group) book lands in ``book``. Status bit 1: a
        nonfinite sampled value or init entry."""
        group = _checked_group(group)
        iterations = _bounded_int(iterations, "iterations", 0, 32)
        sample_vectors = _bounded_int(sample_vectors, "sample_vectors", ENTRIES, 65536)
        self.device.call("ack_vq_fit_codebook", values.handle,
                         None if init is None else init.handle, book.handle, status.handle,
                         elements, group, iterations, sample_vectors, context="fit_codebook")

    def sum_squares_resident(self, values: ack.Buffer, count: int, out: ack.Buffer) -> None:
        """Enqueue the float64 sum of squares of ``count`` float32 values of a
        device buffer into the first 8 bytes of ``out``: a fixed order, within
        (count / 65536 + 15)·2^-53 of the exact sum, relatively."""
        count = _bounded_int(count, "count", 0, 2 ** 62)
        self.device.call("ack_vq_sum_squares", values.handle, count, out.handle,
                         context="sum_squares")

    def scale_resident(self, values: ack.Buffer, count: int, factor) -> None:
        """Enqueue ``values[i] *= float32(factor)`` for ``count`` float32 values
        of a device buffer, in place (numpy's float32 multiply, bit for bit)."""
        count = _bounded_int(count, "count", 0, 2 ** 62)
        self.device.call("ack_vq_scale", values.handle, count, float(np.float32(factor)),
                         context="scale")

    def adamw_step_resident(self, codes: ack.Buffer, books: ack.Buffer, coefficients: ack.Buffer,
                            out_codes: ack.Buffer, out_books: ack.Buffer, changed: ack.Buffer,
                            status: ack.Buffer, *, count: int, group: int,
                            iterations: int = 4, sample_vectors: int = 4096) -> None:
        """Enqueue the fused optimizer step on op 3's inputs as ``adamw``
        lays them out: [W|M|V|G] codes, their four books, seven coefficients."""
        group = _checked_group(group)
        iterations = _bounded_int(iterations, "iterations", 0, 32)
        sample_vectors = _bounded_int(sample_vectors, "sample_vectors", ENTRIES, 65536)
        plan = _plan((3, count, 1, 1, group, ENTRIES, 0, 0))
        self.device.call("ack_vq_adamw_step", codes.handle, books.handle, coefficients.handle,
                         out_codes.handle, out_books.handle, changed.handle, status.handle,
                         plan, len(plan), iterations, sample_vectors, context="vq")

    def _path(self, entry: str, words) -> str:
        name = ctypes.create_string_buffer(64)
        plan = _plan(words)
        lib = self.device.lib
        lib.check(getattr(lib.cdll, entry)(plan, len(plan), name, len(name)), "vq")
        return name.value.decode()

    def path_name(self, words, count: int = 1) -> str:
        """The kernel path ack_vq (count 1) or ack_vq_batch takes for a plan
        (automatic policy)."""
        name = ctypes.create_string_buffer(64)
        plan = _plan(words)
        lib = self.device.lib
        count = _bounded_int(count, "count", 1, 2**31)
        lib.check(lib.cdll.ack_vq_batch_path_name(plan, len(plan), count, name, len(name)), "vq")
        return name.value.decode()

    def dense_path_name(self, words) -> str:
        """The kernel path the dense-activation product takes for an op-2 plan."""
        return self._path("ack_vq_dense_path_name", words)

    # -- the reference's surface, host arrays in and out -----------------------
    def encode(self, values, codebook, *, group: int = 16) -> VQArray:
        """Op 0, the shader's FP32 argmin (vq4.comp:118-144)."""
        group = _checked_group(group)
        x = _finite_f32(values, "values")
        geometry = _Geometry.of(x.shape, group)
        book = _checked_book(codebook, group)
        with _Transient(self.device) as call:
            inputs, out, status = [call.staged(x), call.staged(book)], \
                call.empty(geometry.code_bytes), call.status()
            self.run((0, x.size, 1, 1, group, ENTRIES, 0, 0), inputs, out, status)
            call.settle(status)
            words = out.download(np.uint32)
        return VQArray(geometry.shape, group, words, book)

    def decode(self, value: VQArray) -> np.ndarray:
        """Op 1, the gather of every value from its vector's entry."""
        count = _Geometry(value.shape, value.group).elements
        with _Transient(self.device) as call:
            inputs, out, status = [call.staged(value.codes), call.staged(value.codebook)], \
                call.empty(4 * count), call.status()
            self.run((1, count, 1, 1, value.group, ENTRIES, 0, 0), inputs, out, status)
            call.settle(status)
            return out.download(np.float32).reshape(value.shape)

    @staticmethod
    def matmul_geometry(a: VQArray, b: VQArray, transpose_a=False, transpose_b=False):
        """(m, n, k, flags) of op(a) @ op(b), with the reference's refusals
        and this library's work bound."""
        if type(transpose_a) is not bool or type(transpose_b) is not bool:
            raise ValueError("transpose flags must be boolean")
        if len(a.shape) != 2 or len(b.shape) != 2 or a.group != b.group:
            raise ValueError("vq matmul requires two matrices using the same vector group")
        return _product_dims(a.shape, b.shape, transpose_a, transpose_b, "packed")

    @staticmethod
    def dense_geometry(x: np.ndarray, b: VQArray, transpose_a=False, transpose_b=False):
        """(m, n, k, flags) of op(x) @ op(b) for a dense float32 x."""
        if type(transpose_a) is not bool or type(transpose_b) is not bool:
            raise ValueError("transpose flags must be boolean")
        if np.ndim(x) != 2 or len(b.shape) != 2:
            raise ValueError("vq dense matmul requires a dense matrix and a vq matrix")
        return _product_dims(np.shape(x), b.shape, transpose_a, transpose_b, "dense")

    def _product(self, words, arrays, out_bytes: int, *, count: int = 1) -> np.ndarray:
        with _Transient(self.device) as call:
            inputs = [call.staged(a) for a in arrays]
            out, status = call.empty(out_bytes), call.status()
            self.run(words, inputs, out, status, count=count)
            call.settle(status)
            return out.download(np.float32)

    def matmul(self, a: VQArray, b: VQArray, *, transpose_a=False, transpose_b=False) -> np.ndarray:
        """Op 2: op(a) @ op(b) of two vq4 matrices of one group (vq4.comp:165-176)."""
        m, n, k, flags = self.matmul_geometry(a, b, transpose_a, transpose_b)
        out = self._product((2, m, n, k, a.group, ENTRIES, flags, 0),
                            (a.codes, a.codebook, b.codes, b.codebook), 4 * m * n)
        return out.reshape(m, n)

    def matmul_batch(self, a, b, *, transpose_a=False, transpose_b=False) -> np.ndarray:
        """``[op(a[i]) @ op(b[i]) for i]`` in one ``ack_vq_batch`` launch; every
        instance shares shapes and group. Returns (count, m, n) float32."""
        lefts, rights = list(a), list(b)
        if not lefts or len(lefts) != len(rights):
            raise ValueError("vq batched matmul needs one right operand per left operand")
        first_a, first_b = lefts[0], rights[0]
        if any((x.shape, x.group) != (first_a.shape, first_a.group) for x in lefts) or \
                any((y.shape, y.group) != (first_b.shape, first_b.group) for y in rights):
            raise ValueError("vq batched matmul operands must share shapes and group")
        m, n, k, flags = self.matmul_geometry(first_a, first_b, transpose_a, transpose_b)
        slots = [np.concatenate([getattr(v, part).reshape(-1) for v in side])
                 for side in (lefts, rights) for part in ("codes", "codebook")]
        out = self._product((2, m, n, k, first_a.group, ENTRIES, flags, 0), slots,
                            4 * m * n * len(lefts), count=len(lefts))
        return out.reshape(len(lefts), m, n)

    def matmul_dense(self, x, b: VQArray, *, transpose_a=False, transpose_b=False) -> np.ndarray:
        """op(x) @ op(b) with x a dense float32 matrix: op 2 without encoding
        the activations (an extension; ``matmul`` keeps the reference's
        semantics)."""
        x = _finite_f32(x, "dense operand")
        m, n, k, flags = self.dense_geometry(x, b, transpose_a, transpose_b)
        with _Transient(self.device) as call:
            xs, codes, book = (call.staged(v) for v in (x, b.codes, b.codebook))
            out, status = call.empty(4 * m * n), call.status()
            self.run_dense((2, m, n, k, b.group, ENTRIES, flags, 0), xs, codes, book, out, status)
            call.settle(status)
            return out.download(np.float32).reshape(m, n)

    def fit_codebook(self, values, *, group: int = 16, iterations: int = 4,
                     sample_vectors: int = 4096, init=None) -> np.ndarray:
        """``fit_codebook`` (vq.py:182-257) computed on the GPU: the same
        refusals and the same book, bit for bit."""
        x, group, iterations, sample_vectors, warm = _fit_arguments(values, group, iterations,
                                                                    sample_vectors, init)
        with _Transient(self.device) as call:
            xs = call.staged(x)
            init_buf = None if warm is None else call.staged(warm)
            book, status = call.empty(4 * ENTRIES * group), call.status()
            self.fit_resident(xs, x.size, book, status, group=group, iterations=iterations,
                              sample_vectors=sample_vectors, init=init_buf)
            call.settle(status)
            return book.download(np.float32).reshape(ENTRIES, group)

    adamw_coefficients = staticmethod(adamw_coefficients)

    @staticmethod
    def op3_inputs(weight, momentum, variance, gradient, lr, beta1, beta2, eps, weight_decay,
                   step):
        """(count, codes, books, coefficients): op 3's packed inputs, the four
        states' codes back to back, their books and the coefficient block."""
        states = (weight, momentum, variance, gradient)
        hyper = (lr, beta1, beta2, eps, weight_decay, step)
        first = states[0]
        if any((s.shape, s.group) != (first.shape, first.group) for s in states):
            raise ValueError("vq AdamW states must have identical shapes and groups")
        count = _Geometry(first.shape, first.group).elements
        if 3 * count > MAX_ELEMENTS:
            raise ValueError("vq AdamW active scratch exceeds element bound")
        block = adamw_coefficients(*hyper)
        return (count, np.concatenate([s.codes for s in states]),
                np.concatenate([s.codebook.reshape(-1) for s in states]), block)

    def adamw(self, weight: VQArray, momentum: VQArray, variance: VQArray,
              gradient: VQArray, *, lr: float, beta1: float, beta2: float,
              eps: float, weight_decay: float, step: int) -> tuple[np.ndarray, ...]:
        """Op 3: AdamW from four coded states into FP32 scratch [W', M', V']."""
        count, codes, books, block = self.op3_inputs(weight, momentum, variance, gradient, lr,
                                                     beta1, beta2, eps, weight_decay, step)
        dense = self._product((3, count, 1, 1, weight.group, ENTRIES, 0, 0), (codes, books, block),
                              12 * count)
        return tuple(part.reshape(weight.shape) for part in np.split(dense, 3))

    def adamw_step(self, weight: VQArray, momentum: VQArray, variance: VQArray,
                   gradient: VQArray, *, lr: float, beta1: float, beta2: float,
                   eps: float, weight_decay: float, step: int, iterations: int = 4,
                   sample_vectors: int = 4096):
        """The fused optimizer step: op 3's arithmetic, each state's book
        refitted warm from its old one, and the re-encode, with no dense
        scratch. Returns the new (weight, momentum, variance) images and the
        count of changed weight values: what ``adamw`` -> ``fit_codebook`` ->
        ``encode`` reach on the same inputs."""
        count, codes, books, block = self.op3_inputs(weight, momentum, variance, gradient, lr,
                                                     beta1, beta2, eps, weight_decay, step)
        if count < weight.group:
            raise ValueError("codebook calibration needs at least one complete vector")
        iterations = _bounded_int(iterations, "iterations", 0, 32)
        sample_vectors = _bounded_int(sample_vectors, "sample_vectors", ENTRIES, 65536)
        geometry = _Geometry(weight.shape, weight.group)
        with _Transient(self.device) as call:
            ins = [call.staged(v) for v in (codes, books, block)]
            out_codes = call.empty(3 * geometry.code_bytes)
            out_books = call.empty(3 * geometry.codebook_bytes)
            changed, status = call.empty(4), call.status()
            self.adamw_step_resident(*ins, out_codes, out_books, changed, status, count=count,
                                     group=weight.group, iterations=iterations,
                                     sample_vectors=sample_vectors)
            call.settle(status)
            new_codes = out_codes.download(np.uint32).reshape(3, geometry.words)
            new_books = out_books.download(np.float32).reshape(3, ENTRIES, weight.group)
            moved = int(changed.download(np.uint32)[0])
        images = tuple(VQArray(weight.shape, weight.group, c, b)
                       for c, b in zip(new_codes, new_books))
        return images, moved


class VQAdamW:
    """AdamW whose persistent weight and both moments are vq4 images
    (vq.py:368-410). A failed step leaves the three images and the step
    counter as they were; durable commits are the caller's.

    A ``VQDevice`` backend runs the fused step (``VQDevice.adamw_step``);
    any other backend gets the reference's sequence ``adamw`` ->
    ``fit_codebook`` -> ``encode``, which keeps host-only fakes working.
    """

    def __init__(self, backend, weight: VQArray, *, lr=1e-3, betas=(0.9, 0.95), eps=1e-8,
                 weight_decay=0.0):
        self.backend = backend
        self.weight = weight
        blank = VQArray(weight.shape, weight.group, np.zeros_like(weight.codes),
                        np.zeros((ENTRIES, weight.group), dtype=np.float32))
        self.momentum = self.variance = blank
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.steps = 0

    def _hyper(self, step: int) -> dict:
        return {"lr": self.lr, "beta1": self.betas[0], "beta2": self.betas[1], "eps": self.eps,
                "weight_decay": self.weight_decay, "step": step}

    def _stepwise(self, gradient: VQArray, hyper: dict):
        """The reference's sequence on any backend: dense update, each state
        refitted warm from its old book, then encoded."""
        olds = (self.weight, self.momentum, self.variance)
        dense = self.backend.adamw(*olds, gradient, **hyper)
        if len(dense) != len(olds):  # each update pairs with its own state's book
            raise ValueError(f"vq AdamW update returned {len(dense)} arrays, not 3")
        images = tuple(self.backend.encode(update, fit_codebook(update, group=old.group,
                                                                init=old.codebook),
                                           group=old.group)
                       for update, old in zip(dense, olds))
        moved = int(np.count_nonzero(images[0].decode() != self.weight.decode()))
        return images, moved

    def step(self, gradient: VQArray) -> dict:
        """One AdamW step from a vq4 gradient; returns the reference's report."""
        upcoming = self.steps + 1
        hyper = self._hyper(upcoming)
        if isinstance(self.backend, VQDevice):
            images, moved = self.backend.adamw_step(self.weight, self.momentum, self.variance,
                                                    gradient, **hyper)
            calibration = "device float64 fit of the update; no dense scratch written"
        else:
            images, moved = self._stepwise(gradient, hyper)
            calibration = "CPU float32/float64 temporary arrays"  # the reference's text
        self.weight, self.momentum, self.variance = images
        self.steps = upcoming
        elements = _Geometry(self.weight.shape, self.weight.group).elements
        return {"step": upcoming, "changed_weight_values": moved,
                "persistent_state_bytes": sum(s.layout["serialized_bytes"] for s in images),
                "gradient_bytes": gradient.layout["serialized_bytes"],
                # the dense [W'|M'|V'] update of op 3, in bytes (the fused step
                # evaluates it without storing it)
                "native_update_output_bytes": 12 * elements,
                "calibration": calibration,
                "model_quality_validated": False}
