"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for the vq4/v1 path.

Two halves:

* ``shader``: ctypes access to liboracle.so, the scalar C restatement of
  src/alelyon_compute_kit/_kit/kernels/vq4.comp (oracle/vq4_oracle.c). It is
  the checker for every GPU kernel result.
* numpy restatements of the reference's CPU functions in
  src/alelyon_compute_kit/_kit/python/vq.py -- the wire image (:70-151), the
  float64 ``encode`` (:154-179), ``fit_codebook``/``_reseed`` (:182-257), the
  AdamW coefficient block (:357-358) -- and of the seeded payload generator
  ``ExpertBank.initialize_expert`` (_kit/python/expert_bank.py:357-390) and
  the harness's gradient clip (src/alelyon_compute_kit/harness.py:196-200).

Pins, function by function (each test also plants a mistake that must fail):

* ShaderOracle.decode -- a gather, bitwise, NaN payloads kept
  (tests/test_oracle.py test_decode_is_a_bit_exact_gather).
* ShaderOracle.encode -- a numpy float32 brute force, bitwise; the reference's
  float64 CPU encode except at near-ties; planted nonfinite values for the
  status bits (test_encode_*).
* ShaderOracle.matmul -- the sequential FP32 sum by brute force on straddling
  groups in all four layouts, bitwise; a float64 GEMM within 1e-5; planted
  overflow (test_matmul_*). ShaderOracle.matmul_dense -- op 2 with A
  decoded first, bitwise (test_dense_matmul_reduces_to_op2_on_decoded_activations).
* ShaderOracle.adamw, adamw_coefficients, adamw64 -- numpy float32 step by
  step, bitwise; float64 within 1e-6; the status bits (test_adamw_*); the
  reference's VQAdamW orchestration on recorded steps
  (tests/test_host_calibration.py test_vqadamw_steps_match_the_reference_with_a_host_backend).
* image_bytes, pack_indices, unpack_indices, words_for -- the README's
  3,128-byte image and the config-1 image written by the reference, byte for
  byte (tests/test_format.py).
* encode64 -- the reference's CPU encode on recorded vectors
  (test_oracle_encode_matches_reference_vectors).
* fit_codebook, reseed, linspace_index -- the reference's fit on recorded
  vectors, and numpy's linspace (test_oracle_fit_matches_reference_vectors,
  test_linspace_sampling_matches_numpy).
* expert_payload -- the payloads the reference's ExpertBank.initialize_expert
  wrote (test_expert_payload_equals_the_reference_initializer).
* clip_scale -- closed forms on gradients of known norm, and the clip the
  reference harness applied on recorded steps
  (test_clip_scale_closed_forms, test_clip_scale_equals_the_reference_harness).
* matmul64, max_rel -- textbook float64 product and the north star's metric;
  checked against the brute-force sums above.

The shader's driver-precision division and square root are not pinned by
anything in the reference: AdamW parity against the reference itself is
"parity unpinned" beyond the stated FP32 tolerance.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.
"""
from __future__ import annotations

import ctypes
import math
import struct
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ENTRIES = 16
_HEADER = struct.Struct("<8sIIIIQQ")
_MAGIC = b"ACKVQ4\0\0"


# ---- the shader restatement (C) --------------------------------------------
def build_shader_oracle() -> Path:
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return HERE / "liboracle.so"


class ShaderOracle:
    """vq4.comp ops 0-3 on the CPU; each call returns (result, status bits)."""

    def __init__(self, path: Path | None = None):
        path = path or HERE / "liboracle.so"
        if not path.is_file():
            path = build_shader_oracle()
        lib = ctypes.CDLL(str(path))
        p, u32 = ctypes.c_void_p, ctypes.c_uint32
        lib.oracle_encode.argtypes = [p, u32, p, u32, p]
        lib.oracle_decode.argtypes = [p, p, u32, u32, p]
        lib.oracle_matmul.argtypes = [p, p, p, p, u32, u32, u32, u32, u32, p]
        lib.oracle_matmul_dense.argtypes = [p, p, p, u32, u32, u32, u32, u32, p]
        lib.oracle_adamw.argtypes = [p, p, p, u32, u32, p]
        for fn in (lib.oracle_encode, lib.oracle_decode, lib.oracle_matmul,
                   lib.oracle_matmul_dense, lib.oracle_adamw):
            fn.restype = u32
        self.lib = lib

    @staticmethod
    def _c(a, dtype):
        a = np.ascontiguousarray(a, dtype=dtype)
        return a, a.ctypes.data

    def encode(self, x, book, group):
        x, px = self._c(np.ravel(x), np.float32)
        book, pb = self._c(book, np.float32)
        out = np.zeros(words_for(x.size, group), dtype=np.uint32)
        status = self.lib.oracle_encode(px, x.size, pb, group, out.ctypes.data)
        return out, int(status)

    def decode(self, codes, book, m, group):
        codes, pc = self._c(codes, np.uint32)
        book, pb = self._c(book, np.float32)
        out = np.zeros(m, dtype=np.float32)
        status = self.lib.oracle_decode(pc, pb, m, group, out.ctypes.data)
        return out, int(status)

    def matmul(self, a_codes, a_book, b_codes, b_book, m, n, k, group, flags):
        a_codes, pac = self._c(a_codes, np.uint32)
        a_book, pab = self._c(a_book, np.float32)
        b_codes, pbc = self._c(b_codes, np.uint32)
        b_book, pbb = self._c(b_book, np.float32)
        out = np.zeros((m, n), dtype=np.float32)
        status = self.lib.oracle_matmul(pac, pab, pbc, pbb, m, n, k, group, flags,
                                        out.ctypes.data)
        return out, int(status)

    def matmul_dense(self, x, b_codes, b_book, m, n, k, group, flags):
        """The dense-activation product: op 2 with A read from dense x."""
        x, px = self._c(x, np.float32)
        b_codes, pbc = self._c(b_codes, np.uint32)
        b_book, pbb = self._c(b_book, np.float32)
        out = np.zeros((m, n), dtype=np.float32)
        status = self.lib.oracle_matmul_dense(px, pbc, pbb, m, n, k, group, flags,
                                              out.ctypes.data)
        return out, int(status)

    def adamw(self, codes4, books4, coefficients, m, group, fill=np.nan):
        codes4, pc = self._c(codes4, np.uint32)
        books4, pb = self._c(books4, np.float32)
        coefficients, pk = self._c(coefficients, np.float32)
        out = np.full(3 * m, fill, dtype=np.float32)
        status = self.lib.oracle_adamw(pc, pb, pk, m, group, out.ctypes.data)
        return out, int(status)


# ---- format -----------------------------------------------------------------
def words_for(values: int, group: int) -> int:
    """ceil(ceil(values / group) / 8) (vq4.comp:31)."""
    return -(-(-(-values // group)) // 8)


def image_bytes(shape, group, codes, book) -> bytes:
    """The ACKVQ4 wire image (vq.py:123-128)."""
    elements = math.prod(shape)
    code_bytes = words_for(elements, group) * 4
    header = _HEADER.pack(_MAGIC, 1, group, len(shape), 0, elements, code_bytes)
    return (header + struct.pack(f"<{len(shape)}Q", *shape)
            + np.asarray(book, dtype="<f4").tobytes() + np.asarray(codes, dtype="<u4").tobytes())


def unpack_indices(codes, vectors: int) -> np.ndarray:
    v = np.arange(vectors)
    return ((np.asarray(codes, dtype=np.uint32)[v // 8] >> (4 * (v % 8)).astype(np.uint32))
            & np.uint32(15)).astype(np.int64)


def pack_indices(idx) -> np.ndarray:
    idx = np.asarray(idx, dtype=np.uint32)
    words = np.zeros(-(-idx.size // 8), dtype=np.uint32)
    for lane in range(8):
        part = idx[lane::8]
        words[:part.size] |= part << np.uint32(4 * lane)
    return words


def decode(codes, book, m: int, group: int) -> np.ndarray:
    """out[i] = book[code(i // g)][i % g]."""
    idx = unpack_indices(codes, -(-m // group))
    return np.asarray(book, dtype=np.float32)[idx].reshape(-1)[:m].copy()


# ---- CPU encode and calibration (vq.py:154-257) -------------------------------
def encode64(values, book, group: int) -> np.ndarray:
    """Float64 nearest-entry indices, lowest index on ties; returns packed words."""
    x = np.asarray(values, dtype=np.float32).reshape(-1)
    vectors = -(-x.size // group)
    padded = np.zeros(vectors * group, dtype=np.float32)
    padded[:x.size] = x
    v = padded.reshape(vectors, group).astype(np.float64)
    b = np.asarray(book, dtype=np.float32).astype(np.float64)
    d = np.zeros((vectors, ENTRIES))
    tail = x.size % group
    for j in range(group):
        delta = v[:, j, None] - b[None, :, j]
        if tail and j >= tail:
            delta[-1] = 0.0
        d += delta * delta
    return pack_indices(np.argmin(d, axis=1))


def linspace_index(n: int, num: int) -> np.ndarray:
    return np.linspace(0, n - 1, num, dtype=np.int64)


def reseed(sample: np.ndarray, book: np.ndarray) -> np.ndarray:
    gap = ((sample.astype(np.float64)[:, None, :] - book.astype(np.float64)[None, :, :]) ** 2)
    return sample[int(gap.sum(-1).min(1).argmax())]


def fit_codebook(values, group: int, iterations: int = 4, sample_vectors: int = 4096,
                 init=None) -> np.ndarray:
    x = np.asarray(values, dtype=np.float32).reshape(-1)
    complete = x[:x.size // group * group].reshape(-1, group)
    sample = complete[linspace_index(len(complete), min(len(complete), sample_vectors))]
    if init is None:
        book = sample[linspace_index(len(sample), ENTRIES)].copy()
    else:
        book = np.array(init, dtype=np.float32, copy=True)
    for _ in range(iterations):
        idx = unpack_indices(encode64(sample, book, group), len(sample))
        empty = [e for e in range(ENTRIES) if not (idx == e).any()]
        reachable = [e for e in empty
                     if not any(np.array_equal(book[e], book[j]) for j in range(e))]
        kept = set()
        if init is not None and len(sample) < len(complete) and reachable:
            kept = set(unpack_indices(encode64(complete, book, group), len(complete)).tolist())
        for e in range(ENTRIES):
            rows = sample[idx == e]
            if len(rows):
                book[e] = rows.mean(axis=0, dtype=np.float64).astype(np.float32)
            elif e not in kept:
                book[e] = reseed(sample, book)
    return book


# ---- optimizer and callers ----------------------------------------------------
def adamw_coefficients(lr, beta1, beta2, eps, weight_decay, step) -> np.ndarray:
    """The seven FP32 coefficients (vq.py:357-358)."""
    return np.array([lr, beta1, beta2, eps, weight_decay, 1 - beta1 ** step,
                     1 - beta2 ** step], dtype=np.float32)


def adamw64(w, m, v, g, coefficients):
    """vq4.comp:98-104 evaluated in float64 (a closed form, not the shader's
    rounding) -- the tolerance reference for op 3."""
    lr, b1, b2, eps, decay, c1, c2 = (float(c) for c in coefficients)
    w, m, v, g = (np.asarray(a, dtype=np.float64) for a in (w, m, v, g))
    nm = b1 * m + (1 - b1) * g
    nv = b2 * v + (1 - b2) * g * g
    nw = w * (1 - lr * decay) - lr * (nm / c1) / (np.sqrt(nv / c2) + eps)
    return nw, nm, nv


def expert_payload(shape, group: int, seed: int, layer: int, expert: int, index: int):
    """ExpertBank.initialize_expert's seeded (codes, book) for one matrix."""
    vectors = -(-math.prod(shape) // group)
    words = -(-vectors // 8)
    rng = np.random.default_rng(np.random.SeedSequence([seed, layer, expert, index]))
    codes = rng.integers(0, 1 << 32, words, dtype=np.uint32)
    tail = vectors % 8
    if tail:
        codes[-1] &= np.uint32((1 << (tail * 4)) - 1)
    book = rng.standard_normal((ENTRIES, group), dtype=np.float32)
    book *= np.float32(1.0 / math.sqrt(shape[0]))
    return codes, book


def clip_scale(gradient, max_grad_norm: float) -> float:
    """harness.py:196-200: min(1, max_norm / (||g||_2 + 1e-6)), norm in float64."""
    norm = float(np.linalg.norm(np.asarray(gradient).astype(np.float64)))
    return min(1.0, max_grad_norm / (norm + 1e-6))


def matmul64(a, b, transpose_a=False, transpose_b=False) -> np.ndarray:
    """Float64 product of decoded operands: the tolerance reference for op 2."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return (a.T if transpose_a else a) @ (b.T if transpose_b else b)


def max_rel(y, ref) -> float:
    """max_i |y_i - ref_i| / max_i |ref_i| (the north star's metric)."""
    ref = np.asarray(ref, dtype=np.float64)
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref))) if ref.size else 0.0
    return err / scale if scale > 0 else err
