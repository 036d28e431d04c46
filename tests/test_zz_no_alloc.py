"""ack_vq_noalloc, the entry point that allocates nothing: through the C ABI
its results equal ack_vq's bit for bit (the same kernels, with their
workspace in the library's fixed scratch array instead of allocated memory),
on consecutive calls whose second input is smaller than the first, for
every path that uses a workspace; a plan needing more workspace than the
array holds is refused before anything is enqueued."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import image, say

pytestmark = pytest.mark.gpu


def _operands(rng, m, n, k, group, flags=0):
    a_codes, a_book = image(rng, m * k, group, 1.0)
    b_codes, b_book = image(rng, k * n, group, 0.02)
    return a_codes, a_book, b_codes, b_book


def _call(vqdev, entry, words, arrays, out_bytes):
    """Run `entry` (ack_vq or ack_vq_noalloc) through the C ABI on fresh
    buffers; returns (rc, output bytes as uint32, status word)."""
    device = vqdev.device
    held = []
    try:
        for a in arrays:
            b = device.buffer(a.nbytes)
            b.upload(a)
            held.append(b)
        out = device.buffer(out_bytes)
        out.upload(np.full(out_bytes, 0xA5, np.uint8))     # unwritten outputs are visible
        status = device.buffer(4)
        status.upload(np.zeros(1, np.uint32))
        held += [out, status]
        slots = held[:len(arrays)] + [held[0]] * (4 - len(arrays))
        plan = np.asarray(words, dtype="<u4").tobytes()
        with device.lock:
            rc = getattr(device.lib.cdll, entry)(device.handle, *(b.handle for b in slots),
                                                 out.handle, status.handle, plan, len(plan))
        if rc != 0:
            return rc, None, None
        return rc, out.download(np.uint32), int(status.download(np.uint32)[0])
    finally:
        for b in held:
            b.free()


# (m, n, k, group, flags, path): every path whose launch takes a workspace,
# the larger product first in each pair
PAIRS = [
    [(1, 8192, 8192, 16, 0, "gemv-pairs"), (1, 8192, 4160, 16, 0, "gemv-pairs")],
    [(1, 4096, 4096, 16, 0, "gemv-direct"), (1, 2048, 1024, 16, 0, "gemv-direct")],
    [(8, 4096, 4096, 8, 0, "gemv-direct"), (3, 1024, 2048, 8, 1, "gemv-direct")],
    [(8, 4096, 8320, 16, 1, "gemv-rows"), (3, 4096, 8320, 8, 0, "gemv-rows")],
    [(24, 2048, 8192, 8, 0, "gemv-rows"), (12, 1024, 4096, 16, 1, "gemv-rows")],
    [(16, 4096, 14336, 16, 0, "onehot-mfma"), (8, 4096, 4096, 32, 0, "onehot-mfma")],
    [(512, 4096, 4096, 32, 0, "onehot-mfma"), (64, 1024, 1024, 16, 0, "onehot-mfma")],
    [(2048, 8192, 512, 16, 0, "onehot-mfma"), (128, 4096, 4096, 32, 0, "onehot-mfma")],
]


@pytest.mark.parametrize("pair", PAIRS, ids=[p[0][5] + str(i) for i, p in enumerate(PAIRS)])
def test_noalloc_equals_ack_vq_on_consecutive_calls(vqdev, pair):
    rng = np.random.default_rng(len(pair[0]) + pair[0][0] + pair[0][1])
    for m, n, k, group, flags, path in pair:
        words = (2, m, n, k, group, 16, flags, 0)
        assert vqdev.path_name(words) == path
        ops = _operands(rng, m, n, k, group, flags)
        say("noalloc", path, m, n, k, group, flags)
        rc, got, status = _call(vqdev, "ack_vq_noalloc", words, ops, 4 * m * n)
        assert rc == 0 and status == 0
        rc, want, ref_status = _call(vqdev, "ack_vq", words, ops, 4 * m * n)
        assert rc == 0 and ref_status == 0
        np.testing.assert_array_equal(got, want)


def test_noalloc_scratch_belongs_to_one_handle_at_a_time(vqdev):
    """Two device handles on one GPU share its scratch. A handle's noalloc
    calls follow each other on its stream; a second handle's call while the
    first handle's noalloc work may still be running is refused with
    ACK_ERR_DEVICE naming the scratch (or, if that work has already finished,
    accepted), and once the first handle is synchronized the second handle's
    call runs: every accepted result equals ack_vq's bit for bit."""
    from alelyon_compute_kit import ack
    rng = np.random.default_rng(12)
    m, n, k, group = 512, 4096, 4096, 32
    words = (2, m, n, k, group, 16, 0, 0)
    assert vqdev.path_name(words) == "onehot-mfma"
    ops = _operands(rng, m, n, k, group)
    plan = np.asarray(words, dtype="<u4").tobytes()
    say("noalloc reference", m, n, k, group)
    rc, want, status = _call(vqdev, "ack_vq", words, ops, 4 * m * n)
    assert rc == 0 and status == 0
    first = vqdev.device
    with ack.Device() as second:
        held = {}
        try:
            for name, dev in (("first", first), ("second", second)):
                bufs = [dev.buffer(a.nbytes) for a in ops]
                for b, a in zip(bufs, ops):
                    b.upload(a)
                out, st = dev.buffer(4 * m * n), dev.buffer(4)
                st.upload(np.zeros(1, np.uint32))
                held[name] = (dev, bufs, out, st)

            def launch(name):
                dev, bufs, out, st = held[name]
                with dev.lock:
                    return dev.lib.cdll.ack_vq_noalloc(dev.handle, *(b.handle for b in bufs),
                                                       out.handle, st.handle, plan, len(plan))

            def result(name):
                dev, _, out, st = held[name]
                return out.download(np.uint32), int(st.download(np.uint32)[0])

            say("noalloc: second handle twice, then the first handle at once")
            assert launch("second") == 0
            assert launch("second") == 0                  # one handle: ordered on its stream
            rc = launch("first")
            if rc != 0:
                assert rc == ack.ACK_ERR_DEVICE
                assert "scratch" in first.lib.last_error()
            got, st = result("second")                   # synchronizes the second handle
            assert st == 0
            np.testing.assert_array_equal(got, want)
            if rc == 0:                                   # accepted: the earlier work had ended
                got, st = result("first")
                assert st == 0
                np.testing.assert_array_equal(got, want)
            say("noalloc: the first handle after the second synchronized")
            assert launch("first") == 0
            got, st = result("first")
            assert st == 0
            np.testing.assert_array_equal(got, want)
        finally:
            for dev, bufs, out, st in held.values():
                for b in bufs + [out, st]:
                    b.free()


def test_noalloc_other_ops_and_status(vqdev, oracle):
    """Ops without a workspace run unchanged; status bits still come back."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal(4096).astype(np.float32)
    book = rng.standard_normal((16, 16)).astype(np.float32)
    words = (0, x.size, 1, 1, 16, 16, 0, 0)
    say("noalloc encode")
    rc, codes, status = _call(vqdev, "ack_vq_noalloc", words, (x, book), x.size // 16 // 2)
    assert rc == 0 and status == 0
    np.testing.assert_array_equal(codes, oracle.encode(x, book, 16)[0])
    ops = list(_operands(rng, 1, 2048, 2048, 16))
    ops[3] = ops[3].copy()
    ops[3][4, 2] = np.nan
    say("noalloc status")
    rc, _, status = _call(vqdev, "ack_vq_noalloc", (2, 1, 2048, 2048, 16, 16, 0, 0), ops, 4 * 2048)
    assert rc == 0 and status == 1


def test_noalloc_refuses_a_workspace_past_the_scratch(vqdev):
    """8 activation rows stored k x m over a 16384 x 16384 weight at group
    16, one product: k splits 64 ways over 4 column tiles, 32 MiB of split-k
    partials. Refused with ACK_ERR_SIZE and a message naming the scratch;
    ack_vq would allocate them."""
    from alelyon_compute_kit import ack
    m, n, k, group = 8, 16384, 16384, 16
    words = (2, m, n, k, group, 16, 1, 0)
    assert vqdev.path_name(words) == "gemv-rows"
    rng = np.random.default_rng(8)
    ops = _operands(rng, m, n, k, group, 1)
    say("noalloc refusal")
    rc, _, _ = _call(vqdev, "ack_vq_noalloc", words, ops, 4 * m * n)
    assert rc == ack.ACK_ERR_SIZE
    assert "scratch" in vqdev.device.lib.last_error()
