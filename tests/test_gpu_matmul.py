"""GPU parity of the packed-pair product (op 2).

The general kernel keeps the shader's per-output order and must equal the
oracle bit for bit; the codebook-factorised paths reorder the sum and must
lie within the north star's FP32 tolerance: max|y - y_ref| / max|y_ref| <=
1e-5, against both the oracle and a float64 product of the decoded operands.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest

from gpu_util import (binned_path, image, m1_auto_path, onehot_auto, run_plan, say,
                      small_auto_path)

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _operands(rng, m, n, k, group, a_scale=1.0, b_scale=1.0):
    a_codes, a_book = image(rng, m * k, group, a_scale)
    b_codes, b_book = image(rng, k * n, group, b_scale)
    return a_codes, a_book, b_codes, b_book


def _dense(codes, book, count, shape, group):
    from oracle import vq4_numpy as o
    return o.decode(codes, book, count, group).reshape(shape)


def _ref64(ops, m, n, k, group, flags):
    from oracle import vq4_numpy as o
    a_codes, a_book, b_codes, b_book = ops
    a = _dense(a_codes, a_book, m * k, (k, m) if flags & 1 else (m, k), group)
    b = _dense(b_codes, b_book, k * n, (n, k) if flags & 2 else (k, n), group)
    return o.matmul64(a, b, bool(flags & 1), bool(flags & 2))


def _gpu(vqdev, ops, m, n, k, group, flags, count=1):
    out, status = run_plan(vqdev, (2, m, n, k, group, 16, flags, 0), ops, 4 * m * n * count,
                           np.float32, count=count)
    return out.reshape(count, m, n) if count > 1 else out.reshape(m, n), status


@pytest.fixture
def general(device):
    device.set_policy(1)
    yield
    device.set_policy(0)


@pytest.fixture
def any_size(device):
    """Factorised paths wherever their shape applies, also below the sizes
    at which the automatic choice keeps the general kernel."""
    device.set_policy(2)
    yield
    device.set_policy(0)


GENERAL_SHAPES = [(3, 5, 7, 8), (37, 53, 96, 16), (64, 64, 64, 32), (1, 256, 256, 16),
                  (130, 70, 33, 8)]


@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_general_kernel_is_bit_identical_to_the_shader(vqdev, oracle, general, flags):
    rng = np.random.default_rng(flags)
    for m, n, k, group in GENERAL_SHAPES:
        say("general", m, n, k, group, flags)
        ops = _operands(rng, m, n, k, group)
        out, status = _gpu(vqdev, ops, m, n, k, group, flags)
        ref, ref_status = oracle.matmul(*ops, m, n, k, group, flags)
        np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))
        assert status == ref_status == 0


def test_general_kernel_status_on_overflow(vqdev, oracle, general):
    from oracle import vq4_numpy as o
    codes = o.pack_indices(np.zeros(4, np.int64))
    book = np.full((16, 8), 3e19, np.float32)
    say("general overflow")
    _, status = _gpu(vqdev, (codes, book, codes, book), 4, 4, 8, 8, 0)
    assert status == oracle.matmul(codes, book, codes, book, 4, 4, 8, 8, 0)[1] == 1


GEMV_SHAPES = [(256, 256, 16), (4096, 4096, 16), (512, 1024, 8), (1024, 768, 32),
               (100, 512, 16), (3000, 2048, 8)]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8])
def test_gemv_within_tolerance(vqdev, oracle, m):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(50 + m)
    for (k, n, group), policy in itertools.product(GEMV_SHAPES, (0, 2)):
        words = (2, m, n, k, group, 16, 0, 0)
        auto = small_auto_path(m, n, k, group=group)
        assert vqdev.path_name(words) == auto
        say("gemv", m, k, n, group, auto if policy == 0 else binned_path(m))
        ops = _operands(rng, m, n, k, group, 1.0, 0.02)
        vqdev.device.set_policy(policy)   # 2: the bin kernels
        try:
            out, status = _gpu(vqdev, ops, m, n, k, group, 0)
        finally:
            vqdev.device.set_policy(0)
        assert status == 0
        if m * n * k <= 1 << 24:
            ref, _ = oracle.matmul(*ops, m, n, k, group, 0)
            assert o.max_rel(out, ref) <= TOL
        assert o.max_rel(out, _ref64(ops, m, n, k, group, 0)) <= TOL


# n, k, group, count: whole and ragged tiles of 256 columns (640 at g 16, 320
# at g 8), k below one group, k with a tail of rows, several slices and
# instances, and the size limit itself (2^25 weights)
DIRECT_SHAPES = [(4096, 4096, 16, 1), (4096, 4096, 16, 2), (1024, 1024, 8, 1),
                 (640, 1000, 16, 3), (320, 1000, 8, 1), (64, 4, 8, 1), (2048, 63, 16, 5),
                 (256, 8192, 16, 4), (8192, 4096, 8, 1), (512, 2048, 32, 2)]


@pytest.mark.parametrize("n,k,group,count", DIRECT_SHAPES)
def test_gemv_direct(vqdev, oracle, n, k, group, count):
    """m = 1 products of at most 2^25 weights in all take gemv-direct (decode
    per output, one launch): within 1e-5 of the oracle and of the float64
    product for every instance."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(n + k + group + count)
    m = 1
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == "gemv-direct"
    say("gemv-direct", n, k, group, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    out = out.reshape(count, m, n)
    for i in range(count):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, 0)
        assert o.max_rel(out[i], ref) <= TOL
        assert o.max_rel(out[i], _ref64(items[i], m, n, k, group, 0)) <= TOL


# m, n, k, group, flags (bit 0: A stored k x m), count
DIRECT_ROW_SHAPES = [(2, 4096, 4096, 16, 0, 1), (3, 1024, 1000, 8, 1, 1),
                     (4, 2048, 2048, 32, 0, 2), (5, 640, 1000, 16, 1, 3),
                     (6, 256, 63, 8, 0, 4), (7, 4096, 1024, 16, 1, 1),
                     (8, 4096, 4096, 8, 0, 1), (8, 2048, 2048, 8, 1, 2), (8, 64, 4, 8, 0, 1)]


@pytest.mark.parametrize("m,n,k,group,flags,count", DIRECT_ROW_SHAPES)
def test_gemv_direct_rows(vqdev, oracle, m, n, k, group, flags, count):
    """2..8 rows of A, row-major or stored k x m, over products of at most
    2^25 weights in all: one gemv-direct launch, each block holding 1, 2, 4
    or 8 rows; within 1e-5 of the oracle and of the float64 product, row by
    row, for every instance."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(m * 31 + n + k + group + flags + count)
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    words = (2, m, n, k, group, 16, flags, 0)
    assert vqdev.path_name(words, count=count) == "gemv-direct"
    say("gemv-direct rows", m, n, k, group, flags, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, flags, count=count)
    assert status == 0
    out = out.reshape(count, m, n)
    for i in range(count):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, flags)
        assert o.max_rel(out[i], ref) <= TOL
        _check_rows(out[i], _ref64(items[i], m, n, k, group, flags))


def test_gemv_direct_repeats_bit_for_bit(vqdev):
    """The slices' partial sums are added by the last block of each tile in
    slice order, counted through arrival counters that block resets: 96 calls
    in a row, cycling through three shapes with different row, tile and slice
    counts, give the same bits every time."""
    rng = np.random.default_rng(77)
    device = vqdev.device
    shapes = [(1, 4096, 4096, 16, 0), (1, 1280, 3000, 8, 0), (5, 1024, 2000, 8, 1)]
    runs = []
    try:
        for m, n, k, group, flags in shapes:
            ops = _operands(rng, m, n, k, group, 1.0, 0.02)
            bufs = [device.buffer(a.nbytes) for a in ops]
            for b, a in zip(bufs, ops):
                b.upload(a)
            out, status = device.buffer(4 * m * n), device.buffer(4)
            status.upload(np.zeros(1, np.uint32))
            words = (2, m, n, k, group, 16, flags, 0)
            assert vqdev.path_name(words) == "gemv-direct"
            runs.append((words, bufs, out, status))
        first = []
        for words, bufs, out, status in runs:
            vqdev.run(words, bufs, out, status)
            first.append(out.download(np.uint32).copy())
        say("gemv-direct repeats", 96)
        for i in range(96):
            words, bufs, out, status = runs[i % 3]
            vqdev.run(words, bufs, out, status)
            if i % 12 < 3:   # download now and then; the other calls queue back to back
                assert np.array_equal(out.download(np.uint32), first[i % 3]), i
        for (words, bufs, out, status), ref in zip(runs, first):
            assert np.array_equal(out.download(np.uint32), ref)
            assert int(status.download(np.uint32)[0]) == 0
    finally:
        for _, bufs, out, status in runs:
            for b in bufs + [out, status]:
                b.free()


def test_gemv_direct_on_two_handles_of_one_gpu(vqdev):
    """Each device handle has its own stream and its own arrival counters:
    products enqueued alternately on two handles of the same GPU, without
    waiting in between, each equal that handle's first result."""
    from alelyon_compute_kit import ack, vq
    rng = np.random.default_rng(78)
    n, k, group = 2048, 4096, 16
    ops = _operands(rng, 1, n, k, group, 1.0, 0.02)
    words = (2, 1, n, k, group, 16, 0, 0)
    with ack.Device() as other:
        devs = [vqdev, vq.VQDevice(other)]
        held = []
        try:
            runs = []
            for d in devs:
                bufs = [d.device.buffer(a.nbytes) for a in ops]
                for b, a in zip(bufs, ops):
                    b.upload(a)
                out, status = d.device.buffer(4 * n), d.device.buffer(4)
                status.upload(np.zeros(1, np.uint32))
                held.append((d, bufs + [out, status]))
                runs.append((d, bufs, out, status))
            say("gemv-direct two handles", 32)
            for i in range(32):
                d, bufs, out, status = runs[i % 2]
                d.run(words, bufs, out, status)
            first = runs[0][2].download(np.uint32)
            assert np.array_equal(runs[1][2].download(np.uint32), first)
            for d, bufs, out, status in runs:
                assert int(status.download(np.uint32)[0]) == 0
        finally:
            for d, bs in held:
                for b in bs:
                    b.free()


def _chunk_auto_path(m, n, k, group, flags):
    """The automatic choice for 9 <= m < 64 over at least 2^20 weights: the
    one-hot MFMA path for a row-major A at g 16/32, else the chunked row-pair
    GEMV."""
    return "onehot-mfma" if onehot_auto(m, n, k, group, flags) else "gemv-rows"


@pytest.mark.parametrize("m,flags", [(9, 0), (16, 0), (17, 1), (32, 0), (40, 1), (63, 0)])
def test_gemv_rows_in_chunks_of_eight(vqdev, oracle, any_size, m, flags):
    """9 <= m < 64 with a weight of at least 2^20 values runs, under the test
    policy, the row-pair kernel over consecutive chunks of 8 rows of A (the
    last one shorter), each written at its own output rows; A transposed
    interleaves every row along k. Smaller weights keep the general kernel."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(60 + m)
    for k, n, group in ((1024, 1024, 16), (2048, 512, 8), (512, 2048, 32)):
        words = (2, m, n, k, group, 16, flags, 0)
        assert vqdev.path_name(words) == _chunk_auto_path(m, n, k, group, flags)
        say("gemv-rows chunks", m, k, n, group, flags)
        ops = _operands(rng, m, n, k, group, 1.0, 0.02)
        out, status = _gpu(vqdev, ops, m, n, k, group, flags)
        assert status == 0
        ref, _ = oracle.matmul(*ops, m, n, k, group, flags)
        assert o.max_rel(out, ref) <= TOL
        assert o.max_rel(out, _ref64(ops, m, n, k, group, flags)) <= TOL
    assert vqdev.path_name((2, m, 512, 512, 16, 16, flags, 0)) == "general"


def test_gemv_rows_chunks_with_split_k(vqdev):
    """m = 24 over k = 20000 at g = 8: every chunk splits k and reuses the
    partials workspace in stream order."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(123)
    m, k, n, group = 24, 20000, 512, 8
    ops = _operands(rng, m, n, k, group, 1.0, 0.02)
    say("gemv-rows chunks split", m, k)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0)
    assert status == 0
    assert o.max_rel(out, _ref64(ops, m, n, k, group, 0)) <= TOL


def test_gemv_transposed_a(vqdev, oracle):
    """A stored (k, m): the activation decode follows the flat index."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(77)
    for m, k, n, group in ((1, 256, 256, 16), (4, 200, 512, 8), (3, 96, 1024, 32),
                           (8, 3000, 256, 16), (7, 1100, 512, 8)):
        say("gemv a^T", m, k, n, group)
        ops = _operands(rng, m, n, k, group)
        out, status = _gpu(vqdev, ops, m, n, k, group, 1)
        ref, _ = oracle.matmul(*ops, m, n, k, group, 1)
        assert status == 0 and o.max_rel(out, ref) <= TOL


def test_gemv_batched(vqdev, oracle):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(88)
    m, k, n, group, count = 1, 512, 512, 16, 6
    items = [_operands(rng, m, n, k, group) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    say("gemv batch", count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    for i, it in enumerate(items):
        ref, _ = oracle.matmul(*it, m, n, k, group, 0)
        assert o.max_rel(out[i], ref) <= TOL


@pytest.mark.parametrize("m", [1, 3, 5, 8])
def test_gemv_long_slices(vqdev, oracle, m):
    """256 instances fill the chip without splitting k, so each block walks
    all 2600 rows: several integer windows, and the staged activations are
    restaged at chunk ends that do not coincide with window ends."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(90 + m)
    k, n, group, count = 2600, 128, 16, 256
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    say("gemv long slices", m, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    for i in (0, 1, 128, 255):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, 0)
        assert o.max_rel(out[i], ref) <= TOL
        assert o.max_rel(out[i], _ref64(items[i], m, n, k, group, 0)) <= TOL


def test_gemv_pairs_restaged_activations(vqdev, oracle):
    """m = 1 over 9000 rows in one slice: three 4096-row integer windows and
    two restages of the 4096-row activation chunk."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(91)
    m, k, n, group, count = 1, 9000, 256, 16, 256
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == "gemv-pairs"
    say("gemv-pairs restaged", count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    for i in (0, 77, 255):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, 0)
        assert o.max_rel(out[i], ref) <= TOL
        assert o.max_rel(out[i], _ref64(items[i], m, n, k, group, 0)) <= TOL


@pytest.mark.parametrize("k,group", [(300, 16), (4352, 8), (7936, 32), (12500, 16)])
def test_gemv_pairs_padding_batches(vqdev, oracle, any_size, k, group):
    """m = 1 with slice lengths that are not a whole number of ring turns:
    the last turn carries padding batches past the slice, which must add
    nothing (and, past a restage, read no stale activations)."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(k)
    m, n, count = 1, 256, 256
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    # automatic choice: gemv-direct for the smallest batch; the test policy runs gemv-pairs
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == m1_auto_path(n, k, count)
    say("gemv-pairs padding", k, group, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    for i in (0, 100, 255):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, 0)
        assert o.max_rel(out[i], ref) <= TOL
        assert o.max_rel(out[i], _ref64(items[i], m, n, k, group, 0)) <= TOL


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_gemv_pairs_saturated_window(vqdev, sign):
    """Every row of a 4096-row window puts the same byte, with the largest
    activation, into one pair bin: the integer sum reaches 4096 * (2^19 - 1)
    (or -2^31) and must not wrap."""
    from oracle import vq4_numpy as o
    m, n, k, group = 1, 512, 4096, 16
    a_book = np.full((16, group), sign * np.nextafter(np.float32(1), np.float32(0)), np.float32)
    a_codes = o.pack_indices(np.zeros(k // group, np.int64))
    b_book = (np.arange(16 * group, dtype=np.float32).reshape(16, group) / 256.0).astype(np.float32)
    b_codes = o.pack_indices(np.full(k * n // group, 5, np.int64))
    one = (a_codes, a_book, b_codes, b_book)
    count = 256  # enough instances that no block splits k: one slice holds the window
    ops = tuple(np.tile(a.reshape(-1), count) for a in one)
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == "gemv-pairs"
    say("gemv-pairs saturated", sign)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    ref = _ref64(one, m, n, k, group, 0)
    for i in (0, 255):
        assert o.max_rel(out[i], ref) <= TOL


@pytest.mark.parametrize("n,k,group", [(512, 4096, 16), (4096, 512, 16), (4096, 512, 8),
                                       (1024, 1024, 8)])
def test_gemv_pairs_four_instances_per_block(vqdev, oracle, n, k, group):
    """1024 instances: each block walks four, and at groups 8 and 16 the bins
    are never cleared between them (each instance's sums are differences of
    cumulative bins). n = 512 (g16) and 1024 (g8) cover the one-word loads,
    n = 4096 the 16-byte loads of whole tiles (two tiles at g8); group 16
    takes the MFMA output product with deferred products and kept outputs,
    group 8 the S table."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(n + k + group)
    m, count = 1, 1024
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == "gemv-pairs"
    say("gemv-pairs four per block", n, k, group, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    for i in (0, 1, 255, 256, 511, 700, 1023):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, 0)
        assert o.max_rel(out[i], ref) <= TOL
        assert o.max_rel(out[i], _ref64(items[i], m, n, k, group, 0)) <= TOL


@pytest.mark.parametrize("count", [257, 1536])
def test_gemv_pairs_kept_outputs_across_instances(vqdev, oracle, count):
    """Blocks walking one to six instances: the batched decode path keeps an
    instance's outputs in registers and stores them during the next
    instance (or when the block ends). Neighbouring instances of a block use
    different operands, so an output stored for the wrong item fails."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(count)
    m, n, k, group = 1, 512, 4096, 16
    sets = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(7)]
    pick = [(i + i // 256) % 7 for i in range(count)]
    ops = tuple(np.concatenate([sets[p][s].reshape(-1) for p in pick]) for s in range(4))
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == "gemv-pairs"
    say("gemv-pairs kept outputs", count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    refs = [oracle.matmul(*st, m, n, k, group, 0)[0] for st in sets]
    for i in range(count):
        assert o.max_rel(out[i], refs[pick[i]]) <= TOL, i


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_gemv_pairs_saturated_windows_in_sequence(vqdev, sign):
    """The saturated window four times per block: the cumulative bins pass
    2^31 several times, and each instance's difference must still be exact."""
    from oracle import vq4_numpy as o
    m, n, k, group = 1, 4096, 4096, 16
    a_book = np.full((16, group), sign * np.nextafter(np.float32(1), np.float32(0)), np.float32)
    a_codes = o.pack_indices(np.zeros(k // group, np.int64))
    b_book = (np.arange(16 * group, dtype=np.float32).reshape(16, group) / 256.0).astype(np.float32)
    b_codes = o.pack_indices(np.full(k * n // group, 0x5A % 16, np.int64))
    one = (a_codes, a_book, b_codes, b_book)
    count = 1024
    ops = tuple(np.tile(a.reshape(-1), count) for a in one)
    say("gemv-pairs saturated sequence", sign)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    ref = _ref64(one, m, n, k, group, 0)
    for i in (0, 255, 256, 767, 1023):
        assert o.max_rel(out[i], ref) <= TOL


@pytest.mark.parametrize("m,k,group,flags", [(2, 20000, 8, 0), (8, 20000, 8, 0),
                                             (5, 12000, 16, 1), (6, 700, 32, 0)])
def test_gemv_rows_split_slices(vqdev, any_size, m, k, group, flags):
    """One product (no batch) over long k: k is split across blocks, and for
    g = 8, m = 8 the slices are also capped so one slice's A words fit the
    staging area; the split partials are summed by the finish kernel."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(k + m)
    n = 512
    ops = _operands(rng, m, n, k, group, 1.0, 0.02)
    # the automatic choice is gemv-direct at these sizes; the test policy runs gemv-rows
    assert vqdev.path_name((2, m, n, k, group, 16, flags, 0)) == small_auto_path(m, n, k,
                                                                                 group=group,
                                                                                 flags=flags)
    say("gemv-rows split", m, k, group, flags)
    out, status = _gpu(vqdev, ops, m, n, k, group, flags)
    assert status == 0
    assert o.max_rel(out, _ref64(ops, m, n, k, group, flags)) <= TOL


@pytest.mark.parametrize("m,n,k,group,flags,count", [
    (4, 4096, 512, 16, 0, 64),      # one tile
    (3, 2560, 384, 8, 0, 40),       # two tiles, the second 8 words wide
    (8, 4096, 1024, 32, 0, 70),     # a 16-word tile
    (2, 4096, 4224, 16, 0, 64),     # one row pair; two windows, restaged activations
    (4, 4096, 512, 16, 1, 64),      # A transposed
    (5, 12288, 256, 16, 0, 24),     # three tiles
])
def test_gemv_rows_batched_shapes(vqdev, oracle, m, n, k, group, flags, count):
    """The 2..8-row product over many instances: several tiles and partial
    ones, every group, two windows, A transposed, and instance counts that are
    not a multiple of the blocks per instance group."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(m * 1000 + n + k + group + flags)
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    say("gemv rows batched", m, n, k, group, flags, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, flags, count=count)
    assert status == 0
    for i in sorted({0, 1, count // 2, count - 1}):
        ref, _ = oracle.matmul(*items[i], m, n, k, group, flags)
        assert o.max_rel(out[i], ref) <= TOL
        assert o.max_rel(out[i], _ref64(items[i], m, n, k, group, flags)) <= TOL


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_gemv_rows_saturated_window(vqdev, sign):
    """Both rows of a 64-bit bin pair at the largest activation over a full
    4096-row window into one bin: each int32 half reaches 4096 * (2^19 - 1)
    (or -2^31) and the carry between the halves must stay exact."""
    from oracle import vq4_numpy as o
    m, n, k, group = 2, 512, 4096, 16
    a_book = np.full((16, group), sign * np.nextafter(np.float32(1), np.float32(0)), np.float32)
    a_book[1] = -a_book[1]
    # row 0 uses entry 0, row 1 entry 1: opposite signs in the two halves
    a_idx = np.concatenate([np.zeros(k // group, np.int64), np.ones(k // group, np.int64)])
    a_codes = o.pack_indices(a_idx)
    b_book = (np.arange(16 * group, dtype=np.float32).reshape(16, group) / 256.0).astype(np.float32)
    b_codes = o.pack_indices(np.full(k * n // group, 9, np.int64))
    one = (a_codes, a_book, b_codes, b_book)
    count = 64   # 128 row instances: too few for the row-pair kernel
    ops = tuple(np.tile(a.reshape(-1), count) for a in one)
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == "gemv-rows"
    say("gemv-rows saturated", sign)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    ref = _ref64(one, m, n, k, group, 0)
    for i in (0, count - 1):
        assert o.max_rel(out[i], ref) <= TOL


def test_config1_matmul(vqdev, oracle):
    """benchmark config 1: x (1x256) times W (256x256), group 16, both images
    recorded from the reference."""
    from alelyon_compute_kit import vq
    from conftest import golden
    from oracle import vq4_numpy as o
    g = golden("config1.npz")
    w = vq.VQArray.from_bytes(g["w_image"].tobytes())
    x = vq.VQArray.from_bytes(g["x_image"].tobytes())
    say("config1 matmul")
    y = vqdev.matmul(x, w)
    ref, _ = oracle.matmul(x.codes, x.codebook, w.codes, w.codebook, 1, 256, 256, 16, 0)
    assert o.max_rel(y, ref) <= TOL
    assert o.max_rel(y, g["x_decoded"].astype(np.float64) @ g["w_decoded"]) <= TOL


@pytest.mark.parametrize("m", [1, 4, 8])
def test_config3_decode_shaped_gemv(vqdev, m):
    """benchmark config 3 at full size: W 4096x4096 ~N(0, 0.02^2) fitted at
    group 16, X m x 4096 ~N(0,1) fitted and encoded; forward only."""
    from alelyon_compute_kit import vq
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    w_img = vq.encode(w, vq.fit_codebook(w, group=16), group=16)
    x = rng.standard_normal((m, 4096)).astype(np.float32)
    x_img = vq.encode(x, vq.fit_codebook(x, group=16), group=16)
    say("config3", m)
    y = vqdev.matmul(x_img, w_img)
    ref = x_img.decode().astype(np.float64) @ w_img.decode().astype(np.float64)
    assert o.max_rel(y, ref) <= TOL


def test_transposed_products_agree_with_float64(vqdev):
    """dY . W^T and A^T . B at moderate size through the automatic path."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(99)
    for m, n, k, group, flags in ((64, 96, 128, 32, 2), (33, 40, 64, 8, 1), (100, 64, 256, 16, 3)):
        say("auto", m, n, k, group, flags)
        ops = _operands(rng, m, n, k, group)
        out, status = _gpu(vqdev, ops, m, n, k, group, flags)
        assert status == 0
        assert o.max_rel(out, _ref64(ops, m, n, k, group, flags)) <= TOL


LARGE_M_SHAPES = [(64, 256, 64, 16), (100, 512, 96, 32), (130, 2048, 256, 16),
                  (255, 1024, 512, 32), (200, 768, 1024, 16)]


@pytest.mark.parametrize("m,n,k,group", LARGE_M_SHAPES)
def test_large_m_under_the_test_policy(vqdev, oracle, any_size, m, n, k, group):
    """Large-m products with B's groups along n take onehot-mfma by default
    and under the test policy alike (no bin kernel serves m >= 64); rows past
    m in the last block are masked."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(m + n + k)
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.path_name(words) == "onehot-mfma"
    say("onehot-mfma (test policy)", m, n, k, group)
    ops = _operands(rng, m, n, k, group, 1.0, 0.02)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0)
    assert status == 0
    ref, _ = oracle.matmul(*ops, m, n, k, group, 0)
    assert o.max_rel(out, ref) <= TOL
    assert o.max_rel(out, _ref64(ops, m, n, k, group, 0)) <= TOL


# (m, n, k, group): one 16-step of k, a last pass shorter than 8 groups of A
# (k not a multiple of 8 g), rows past m in the last block, 1 and 8 word
# columns; grids below 256 blocks of 256 rows run 64-row blocks, the last two
# shapes the 256-row blocks. 64-row grids of fewer than 256 blocks split k
# (4 ways at 16 x 1024 x 1024, 8 at 63 x 4096 x 4096 and at the 128-row
# chunk, 3 at 513 x 2048 x 4096; 48 x 2048 x 4112 into 11 parts of 3 passes,
# the last one 2 passes and a 16-step). The last two shapes have fewer 256-row
# blocks than the chip's 512 slots and take the mixed 256/192-row tiling: one
# column class (4 + 4 blocks per column) and two (5 + 4 and 2 + 8, as config 4)
ONEHOT_SHAPES = [(16, 1024, 1024, 16), (40, 2048, 512, 32), (63, 4096, 4096, 16),
                 (64, 256, 64, 16), (100, 512, 96, 32), (130, 2048, 256, 16),
                 (256, 1024, 512, 32), (333, 768, 1024, 16), (256, 256, 16, 16),
                 (300, 512, 1040, 16), (1000, 4096, 288, 32), (513, 2048, 4096, 32),
                 (48, 2048, 4112, 16), (128, 4096, 4096, 32),
                 (1000, 16384, 256, 32), (2100, 4096, 1040, 16),
                 (1792, 8192, 256, 16), (2048, 7168, 512, 16),
                 (8, 4096, 4096, 16), (9, 1024, 1024, 16), (12, 4096, 14336, 32)]


@pytest.mark.parametrize("m,n,k,group", ONEHOT_SHAPES)
def test_onehot_mfma_within_tolerance(vqdev, oracle, m, n, k, group):
    """m >= 64 rows of a packed A (or from 8 with B of at least 2^20 values;
    groups along k) times B grouped along n:
    A's book rows (scaled by a power of two and split into three bf16 terms,
    exact for every entry down to 2^-118 of the largest) times the one-hot of
    B's codes on bf16 MFMA, then the 16-term product with B's book. Within
    1e-5 of the oracle and of the float64 product, every row against its own
    largest output."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(m + n + k + group)
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.path_name(words) == "onehot-mfma"
    say("onehot-mfma", m, n, k, group)
    ops = _operands(rng, m, n, k, group, 1.0, 0.02)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0)
    assert status == 0
    if m * n * k <= 1 << 28:
        ref, _ = oracle.matmul(*ops, m, n, k, group, 0)
        assert o.max_rel(out, ref) <= TOL
    _check_rows(out, _ref64(ops, m, n, k, group, 0))


def test_onehot_mfma_rows_of_very_different_magnitude(vqdev):
    """A's book holds entries near 1 and near 2^-24: even rows use only the
    small ones. The book is split after one power-of-two scale, and every
    entry within 2^-40 of the largest keeps all its bits, so each row keeps
    the 1e-5 bar against its own largest output."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(77)
    m, n, k, group = 512, 1024, 1024, 32
    a_book = rng.standard_normal((16, group)).astype(np.float32)
    a_book[:8] *= np.float32(2.0 ** -24)
    idx = rng.integers(8, 16, (m, k // group))
    idx[0::2] = rng.integers(0, 8, (m // 2, k // group))
    a_codes = o.pack_indices(idx.reshape(-1))
    b_codes, b_book = image(rng, k * n, group, 0.02)
    ops = (a_codes, a_book, b_codes, b_book)
    assert vqdev.path_name((2, m, n, k, group, 16, 0, 0)) == "onehot-mfma"
    say("onehot-mfma magnitudes")
    out, status = _gpu(vqdev, ops, m, n, k, group, 0)
    assert status == 0
    exact = _ref64(ops, m, n, k, group, 0)
    assert np.abs(exact[0]).max() < 1e-5 < np.abs(exact[1]).max()
    _check_rows(out, exact)


def test_gram_mfma_rows_of_very_different_magnitude(vqdev):
    """B stored (n, k), both grouped along k; A's book holds entries near 1
    and near 2^-24 and even rows use only the small ones, so their Gram
    entries sit 2^-24 below the largest. The Gram table's three bf16 terms
    carry every entry exactly, so each row keeps the 1e-5 bar against its own
    largest output."""
    rng = np.random.default_rng(78)
    m, n, k, group = 512, 384, 2048, 16
    a_book = rng.standard_normal((16, group)).astype(np.float32)
    a_book[:8] *= np.float32(2.0 ** -24)
    from oracle import vq4_numpy as o
    idx = rng.integers(8, 16, (m, k // group))
    idx[0::2] = rng.integers(0, 8, (m // 2, k // group))
    a_codes = o.pack_indices(idx.reshape(-1))
    b_codes, b_book = image(rng, k * n, group, 0.02)
    ops = (a_codes, a_book, b_codes, b_book)
    assert vqdev.path_name((2, m, n, k, group, 16, 2, 0)) == "gram-mfma"
    say("gram-mfma magnitudes")
    out, status = _gpu(vqdev, ops, m, n, k, group, 2)
    assert status == 0
    exact = _ref64(ops, m, n, k, group, 2)
    assert np.abs(exact[0]).max() < 1e-5 < np.abs(exact[1]).max()
    _check_rows(out, exact)


def test_config4_forward_against_float64(vqdev):
    """benchmark config 4 forward at full size: X 2048x4096 . W 4096x14336 at
    group 32; every output against the float64 product of the decoded
    operands, over the whole matrix and row by row."""
    from alelyon_compute_kit import vq
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((4096, 14336)) * 0.02).astype(np.float32)
    w_img = vqdev.encode(w, vq.fit_codebook(w, group=32), group=32)
    x = rng.standard_normal((2048, 4096)).astype(np.float32)
    x_img = vqdev.encode(x, vq.fit_codebook(x, group=32), group=32)
    assert vqdev.path_name((2, 2048, 14336, 4096, 32, 16, 0, 0)) == "onehot-mfma"
    say("config4 forward")
    y = vqdev.matmul(x_img, w_img)
    ref = x_img.decode().astype(np.float64) @ w_img.decode().astype(np.float64)
    assert o.max_rel(y, ref) <= TOL
    row_err = np.abs(y - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert row_err.max() <= TOL, f"row {int(row_err.argmax())}"


# (m, n, k, group): k / group of 12, 17 and 33 start rows mid-word
GRAM_SHAPES = [(1, 256, 256, 16), (37, 53, 96, 8), (64, 96, 128, 32), (130, 200, 272, 16),
               (256, 384, 1024, 32), (100, 64, 264, 8), (300, 129, 512, 16)]


@pytest.mark.parametrize("m,n,k,group", GRAM_SHAPES)
def test_gram_mfma_within_tolerance(vqdev, oracle, any_size, m, n, k, group):
    """B stored (n, k) with both operands grouped along k: one-hot A times the
    codebooks' Gram table on bf16 MFMA (three bf16 terms hi + mid + lo, every
    entry down to 2^-118 of the largest exact). Products below
    2^22 multiply-adds take the general kernel by default; the test policy
    sends them through the Gram kernel."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(m * 7 + n + k)
    words = (2, m, n, k, group, 16, 2, 0)
    assert vqdev.path_name(words) == ("gram-mfma" if m * n * k >= 1 << 22 else "general")
    say("gram-mfma", m, n, k, group)
    ops = _operands(rng, m, n, k, group, 0.1, 0.02)
    out, status = _gpu(vqdev, ops, m, n, k, group, 2)
    assert status == 0
    ref, _ = oracle.matmul(*ops, m, n, k, group, 2)
    assert o.max_rel(out, ref) <= TOL
    assert o.max_rel(out, _ref64(ops, m, n, k, group, 2)) <= TOL


def test_gram_mfma_batched(vqdev, oracle, any_size):
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(123)
    m, n, k, group, count = 70, 96, 160, 16, 5
    items = [_operands(rng, m, n, k, group, 1.0 + i, 0.5) for i in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    say("gram-mfma batch", count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 2, count=count)
    assert status == 0
    for i, it in enumerate(items):
        ref, _ = oracle.matmul(*it, m, n, k, group, 2)
        assert o.max_rel(out[i], ref) <= TOL


def test_gram_mfma_status_on_overflow(vqdev, oracle, any_size):
    from oracle import vq4_numpy as o
    codes = o.pack_indices(np.zeros(4, np.int64))
    book = np.full((16, 8), 3e19, np.float32)
    say("gram-mfma overflow")
    _, status = _gpu(vqdev, (codes, book, codes, book), 4, 4, 8, 8, 2)
    assert status == oracle.matmul(codes, book, codes, book, 4, 4, 8, 8, 2)[1] == 1


def test_config4_backward_against_float64(vqdev):
    """benchmark config 4 backward at full size: dY 2048x14336 ~ N(0, 1e-2) .
    W^T with W 4096x14336 stored (n, k) at group 32; every output against the
    float64 product of the decoded operands, over the whole matrix and row by
    row."""
    from alelyon_compute_kit import vq
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((4096, 14336)) * 0.02).astype(np.float32)
    w_img = vqdev.encode(w, vq.fit_codebook(w, group=32), group=32)
    dy = (rng.standard_normal((2048, 14336)) * 0.1).astype(np.float32)
    dy_img = vqdev.encode(dy, vq.fit_codebook(dy, group=32), group=32)
    assert vqdev.path_name((2, 2048, 4096, 14336, 32, 16, 2, 0)) == "gram-mfma"
    say("config4 backward")
    y = vqdev.matmul(dy_img, w_img, transpose_b=True)
    assert y.shape == (2048, 4096)
    ref = dy_img.decode().astype(np.float64) @ w_img.decode().astype(np.float64).T
    assert o.max_rel(y, ref) <= TOL
    row_err = np.abs(y - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert row_err.max() <= TOL, f"row {int(row_err.argmax())}"


@pytest.mark.parametrize("m,flags", [(1, 0), (6, 2), (48, 1), (200, 0)])
def test_matmul_batch_method_matches_each_instance(vqdev, m, flags):
    """``VQDevice.matmul_batch`` (one ``ack_vq_batch`` launch) against a
    float64 product of each instance's decoded operands."""
    from alelyon_compute_kit import vq
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(100 + m)
    n, k, group, count = 384, 512, 16, 5
    a_shape = (k, m) if flags & 1 else (m, k)
    b_shape = (n, k) if flags & 2 else (k, n)
    a_vals = [rng.standard_normal(a_shape).astype(np.float32) for _ in range(count)]
    b_vals = [rng.standard_normal(b_shape).astype(np.float32) * 0.1 for _ in range(count)]
    a = [vq.encode(v, vq.fit_codebook(v, group=group), group=group) for v in a_vals]
    b = [vq.encode(v, vq.fit_codebook(v, group=group), group=group) for v in b_vals]
    say("matmul_batch", m, n, k, flags, count)
    got = vqdev.matmul_batch(a, b, transpose_a=bool(flags & 1), transpose_b=bool(flags & 2))
    assert got.shape == (count, m, n)
    for i in range(count):
        exact = o.matmul64(a[i].decode(), b[i].decode(), bool(flags & 1), bool(flags & 2))
        assert o.max_rel(got[i], exact) <= TOL
    with pytest.raises(ValueError, match="share shapes"):
        vqdev.matmul_batch(a[:2], [b[0], vq.encode(b_vals[1].T.copy(), b[1].codebook,
                                                    group=group)])


# ---- activations with outliers, rows of different magnitudes ------------------
def _outlier_a(rng, m, k, group, *, tiny_rows=False):
    """A (m x k, groups along k) whose codebook has one outlier entry, 7 =
    30.0 in every component, that each row uses exactly once; the other
    vectors draw from entries 4..15 ~ N(0,1). With tiny_rows the even rows use
    only entries 0..3, ~ 1e-6 N(0,1): rows 2^20 below their neighbours."""
    from oracle import vq4_numpy as o
    book = rng.standard_normal((16, group)).astype(np.float32)
    book[:4] *= np.float32(1e-6)
    book[7] = np.float32(30.0)
    per_row = k // group
    idx = rng.choice(np.r_[4:7, 8:16], size=(m, per_row))
    idx[np.arange(m), rng.integers(0, per_row, m)] = 7
    if tiny_rows:
        idx[0::2] = rng.integers(0, 4, size=idx[0::2].shape)
    return o.pack_indices(idx.reshape(-1)), book


def _check_rows(out, ref, tol=TOL):
    """max_rel over the whole output and row by row, each row against its own
    largest magnitude."""
    from oracle import vq4_numpy as o
    assert o.max_rel(out, ref) <= tol
    for r in range(ref.shape[0]):
        assert o.max_rel(out[r], ref[r]) <= tol, f"row {r}"


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("k,n", [(4096, 4096), (14336, 2048)])
@pytest.mark.parametrize("count", [1, 256])
def test_gemv_outlier_codebook_entry(vqdev, oracle, m, k, n, count):
    """One activation of 30 per row among N(0,1) ones: the fixed-point step
    follows the window's L1 norm, so the outlier costs no precision elsewhere.
    One product takes gemv-direct by default and, under the test policy, the
    fixed-point bins with k split over blocks (finish kernel); 256 instances
    run whole slices of one window per block (m = 1, the config-3 path) or the
    row instances (m > 1)."""
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(k + m + count)
    group = 16
    a_codes, a_book = _outlier_a(rng, m, k, group)
    b_codes, b_book = image(rng, k * n, group, 0.02)
    one = (a_codes, a_book, b_codes, b_book)
    ops = tuple(np.tile(a.reshape(-1), count) for a in one)
    if m == 1 or count == 1:
        auto = small_auto_path(m, n, k, count, group=group)
        assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == auto
    else:   # the batch of 256 takes the row instances
        auto = "gemv-row-pairs"
        assert vqdev.path_name((2, m, n, k, group, 16, 0, 0), count=count) == auto
    say("gemv outlier entry", m, k, n, count, auto)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    if auto == "gemv-direct":   # the fixed-point bins too, under the test policy
        vqdev.device.set_policy(2)
        try:
            pairs, pairs_status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
        finally:
            vqdev.device.set_policy(0)
        assert pairs_status == 0
        pairs = pairs.reshape(count, m, n)
        _check_rows(pairs[0], _ref64(one, m, n, k, group, 0))
    out = out.reshape(count, m, n)
    ref, ref_status = oracle.matmul(*one, m, n, k, group, 0)
    assert ref_status == 0
    exact = _ref64(one, m, n, k, group, 0)
    for i in sorted({0, count // 2, count - 1}):
        _check_rows(out[i], ref.reshape(m, n))
        _check_rows(out[i], exact)
    # every instance holds the same operands: the same bits
    assert (out.view(np.uint32) == out[0].view(np.uint32)).all()


@pytest.mark.parametrize("m", [2, 5, 8])
@pytest.mark.parametrize("count", [1, 256])
def test_gemv_rows_each_row_its_own_scale(vqdev, oracle, any_size, m, count):
    """Rows of A 2^20 apart in magnitude in one launch (even rows ~1e-6,
    odd rows ~1 with an outlier of 30): every row, checked against its own
    largest output, keeps the 1e-5 bar; a shared scale would round the small
    rows to zero."""
    rng = np.random.default_rng(300 + m + count)
    k, n, group = 4096, 4096, 16
    a_codes, a_book = _outlier_a(rng, m, k, group, tiny_rows=True)
    b_codes, b_book = image(rng, k * n, group, 0.02)
    one = (a_codes, a_book, b_codes, b_book)
    ops = tuple(np.tile(a.reshape(-1), count) for a in one)
    exact = _ref64(one, m, n, k, group, 0)
    assert np.abs(exact[0]).max() < 1e-3 < np.abs(exact[1]).max()
    # the test policy (bins), then one product on the automatic gemv-direct
    for policy in (2, 0) if count == 1 else (2,):
        vqdev.device.set_policy(policy)
        say("gemv-rows own scale", m, count, policy)
        out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
        assert status == 0
        out = out.reshape(count, m, n)
        for i in sorted({0, count - 1}):
            _check_rows(out[i], exact)



ROW_PAIR_SHAPES = [
    # m, n, k, group, count
    (2, 4096, 512, 16, 128),     # two rows, cumulative bins, MFMA output product
    (3, 4096, 512, 16, 90),      # 3 rows: an item's rows straddle the XCD groups of 32
    (7, 2048, 512, 8, 40),       # 7 rows at g = 8 (cumulative bins, scalar output product)
    (8, 4096, 1024, 32, 40),     # g = 32, a 16-word tile: one-word loads, bins cleared
    (4, 1024, 8192, 16, 64),     # two windows per row: x restaged, FP32 window sums
    (8, 65536, 576, 8, 1),       # one product whose rows alone fill the chip
]


@pytest.mark.parametrize("m,n,k,group,count", ROW_PAIR_SHAPES)
def test_gemv_row_pairs(vqdev, oracle, m, n, k, group, count):
    """2..8 rows of a row-major A over a batch (or a product wide enough)
    whose row instances fill the chip: each row runs as an m = 1 pair-bin
    instance, the rows of one product on one XCD. Every checked row is held
    to the 1e-5 bar against its own largest output; neighbouring instances
    have different operands, so a row or item mix-up fails."""
    rng = np.random.default_rng(m * 7 + n + k + group + count)
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.path_name(words, count=count) == "gemv-row-pairs"
    b_sets = [image(rng, k * n, group, 0.02) for _ in range(min(count, 3))]
    items = [image(rng, m * k, group, 1.0) + b_sets[i % len(b_sets)] for i in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in items]) for s in range(4))
    say("gemv-row-pairs", m, n, k, group, count)
    out, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    out = out.reshape(count, m, n)
    for i in sorted({0, 1 % count, count // 2, count - 1}):
        _check_rows(out[i], _ref64(items[i], m, n, k, group, 0))
    if m * n * k <= 1 << 24:
        ref, _ = oracle.matmul(*items[0], m, n, k, group, 0)
        _check_rows(out[0], ref.reshape(m, n))


def test_gemv_row_pairs_not_taken_where_rows_cannot_be_instances(vqdev):
    """A transposed, k not a multiple of 8 g, or too few row instances keep
    the row-pair-atomic kernel."""
    assert vqdev.path_name((2, 4, 4096, 512, 16, 16, 1, 0), count=64) == "gemv-rows"
    assert vqdev.path_name((2, 4, 4096, 520, 8, 16, 0, 0), count=64) == "gemv-rows"
    assert vqdev.path_name((2, 4, 4096, 512, 16, 16, 0, 0), count=63) == "gemv-rows"
    assert vqdev.path_name((2, 4, 4096, 512, 16, 16, 0, 0), count=64) == "gemv-row-pairs"
    assert vqdev.path_name((2, 4, 8192, 4160, 16, 16, 0, 0)) == "gemv-rows"
    # one small product: a single gemv-direct launch
    assert vqdev.path_name((2, 4, 4096, 512, 16, 16, 0, 0)) == "gemv-direct"

# ---- status word on the reordered paths ----------------------------------------
# path, m, n, k, group, flags: shapes each path takes
STATUS_PATHS = [("gemv-direct", 1, 512, 512, 16, 0), ("gemv-pairs", 1, 8192, 4160, 16, 0),
                ("gemv-direct", 4, 512, 512, 16, 0), ("gemv-direct", 7, 384, 1024, 8, 1),
                ("gemv-rows", 4, 8192, 4160, 16, 0),
                ("gemv-rows", 7, 8192, 4160, 8, 1), ("onehot-mfma", 128, 512, 256, 16, 0),
                ("onehot-mfma", 256, 512, 256, 16, 0), ("onehot-mfma", 300, 1024, 288, 32, 0),
                ("gram-mfma", 64, 96, 1024, 16, 2)]


def _status_case(rng, case, m, n, k, group):
    """Operands of one status case: a NaN in A's book, an Inf in B's, a
    product that overflows (3e19 * 3e19), or clean operands."""
    ops = list(_operands(rng, m, n, k, group, 1.0, 0.02))
    if case == "nan_a":
        ops[1] = ops[1].copy()
        ops[1][11, 3] = np.nan                 # an entry no code need select
    elif case == "inf_b":
        ops[3] = ops[3].copy()
        ops[3][2, 0] = np.inf
    elif case == "overflow":
        ops[1] = np.full_like(ops[1], 3e19)
        ops[3] = np.full_like(ops[3], 3e19)
    return tuple(ops)


@pytest.mark.parametrize("path,m,n,k,group,flags", STATUS_PATHS)
@pytest.mark.parametrize("case", ["clean", "nan_a", "inf_b", "overflow"])
def test_status_equals_the_shader_on_reordered_paths(vqdev, oracle, path, m, n, k, group,
                                                     flags, case):
    """Status bit 1 (vq4.comp:149-158 book sweep, :173 nonfinite product or
    total) of the reordered paths equals the shader's: nonfinite book
    entries, used or not, and an overflowing product set it; clean operands
    do not."""
    rng = np.random.default_rng([m, n, k, flags, ["clean", "nan_a", "inf_b", "overflow"].index(case)])
    assert vqdev.path_name((2, m, n, k, group, 16, flags, 0)) == path
    ops = _status_case(rng, case, m, n, k, group)
    say("status", path, m, n, k, group, flags, case)
    _, status = _gpu(vqdev, ops, m, n, k, group, flags)
    _, ref_status = oracle.matmul(*ops, m, n, k, group, flags)
    assert status == ref_status == (0 if case == "clean" else 1)


@pytest.mark.parametrize("m", [1, 4])
def test_status_of_batched_gemv_flags_the_bad_instance_only_once(vqdev, oracle, m):
    """ack_vq_batch shares one status word: one instance with a NaN in its
    B book among clean ones sets bit 1; all clean instances leave it 0."""
    rng = np.random.default_rng(40 + m)
    k, n, group, count = 4096, 4096, 16, 256
    items = [_operands(rng, m, n, k, group, 1.0, 0.02) for _ in range(4)]
    clean = [items[i % 4] for i in range(count)]
    ops = tuple(np.concatenate([it[s].reshape(-1) for it in clean]) for s in range(4))
    say("status batch clean", m)
    _, status = _gpu(vqdev, ops, m, n, k, group, 0, count=count)
    assert status == 0
    bad_book = ops[3].copy()
    bad_book[(count - 3) * 16 * group + 5] = np.nan
    say("status batch one bad", m)
    _, status = _gpu(vqdev, (ops[0], ops[1], ops[2], bad_book), m, n, k, group, 0, count=count)
    assert status == 1
