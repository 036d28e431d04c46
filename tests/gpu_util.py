"""Helpers for GPU tests: run one plan on resident buffers and return both
the output and the status word (VQDevice raises on a nonzero status before
downloading the output)."""
from __future__ import annotations

import sys

import numpy as np


def say(*parts) -> None:
    print("[gpu case]", *parts, flush=True)
    sys.stdout.flush()


def run_plan(vqdev, words, arrays, out_bytes, out_dtype, *, count=1, fill=0):
    """Upload `arrays`, run `words` (ack_vq, or ack_vq_batch when count > 1),
    download (output, status). The output buffer starts filled with `fill`
    bytes so unwritten elements are recognisable."""
    from alelyon_compute_kit import ack
    device = vqdev.device
    bufs = []
    try:
        for a in arrays:
            b = device.buffer(a.nbytes)
            bufs.append(b)
            b.upload(a)
        out = device.buffer(out_bytes)
        bufs.append(out)
        out.upload(np.full(out_bytes, fill, dtype=np.uint8))
        status = device.buffer(4)
        bufs.append(status)
        status.upload(np.zeros(1, np.uint32))
        vqdev.run(words, bufs[:len(arrays)], out, status, count=count)
        flags = int(status.download(np.uint32)[0])
        return out.download(out_dtype), flags
    finally:
        for b in bufs:
            try:
                b.free()
            except ack.AckError:
                pass


def image(rng, m, group, scale=1.0):
    """Random codes (tail nibbles zero) and a normal codebook."""
    vectors = -(-m // group)
    idx = rng.integers(0, 16, vectors).astype(np.uint32)
    words = np.zeros(-(-vectors // 8), np.uint32)
    for lane in range(8):
        part = idx[lane::8]
        words[:part.size] |= part << np.uint32(4 * lane)
    book = (rng.standard_normal((16, group)) * scale).astype(np.float32)
    return words, book


# The automatic choice for m <= 8 rows of A against B grouped along n (flags
# bit 1 clear): gemv-direct up to this many weights in all (n k count;
# kDirectMaxWeights and kDirectMaxRows in alelyon-compute-kit_amd/csrc/kernels.hpp),
# the bin kernels above it. The test policy (2) never takes gemv-direct.
DIRECT_MAX_WEIGHTS = 1 << 25


def onehot_auto(m, n, k, group, flags=0, count=1, dense=False):
    """Whether the automatic choice is onehot-mfma: one product with B grouped
    along n (flags 0), from 64 rows, or from 8 (packed A at g 16 / 32) or 9
    (dense A) rows with B of at least 2^20 values."""
    if count != 1 or flags != 0 or n % (8 * group) or k % 16:
        return False
    if not dense and (group not in (16, 32) or k % group):
        return False
    return m >= 64 or (m >= (9 if dense else 8) and n * k >= 1 << 20)


def small_auto_path(m, n, k, count=1, group=None, flags=0):
    """onehot-mfma where it applies (when `group` is given), else gemv-direct
    where it applies, else gemv-pairs (m = 1) or gemv-rows; a batch filling
    the chip with row instances is gemv-row-pairs, which this helper does not
    model (callers pass count 1 there)."""
    if group is not None and onehot_auto(m, n, k, group, flags, count):
        return "onehot-mfma"
    if m <= 8 and n * k * count <= DIRECT_MAX_WEIGHTS:
        return "gemv-direct"
    return "gemv-pairs" if m == 1 else "gemv-rows"


def binned_path(m):
    """The path the test policy takes for m <= 8 (B grouped along n)."""
    return "gemv-pairs" if m == 1 else "gemv-rows"


def m1_auto_path(n, k, count=1):
    return small_auto_path(1, n, k, count)
