"""The fused VQAdamW step on the GPU (ack_vq_adamw_step) against the same
step composed from op 3, the native fit and the GPU encode -- the sequence
the reference's VQAdamW.step runs (vq.py:388-410). Both must reach identical
images and the same changed-weight count."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu


class Unfused:
    """VQDevice's adamw and encode, without the fused entry: VQAdamW then
    takes the reference's unfused sequence."""

    def __init__(self, vqdev):
        self.vqdev = vqdev

    def adamw(self, *args, **kwargs):
        return self.vqdev.adamw(*args, **kwargs)

    def encode(self, values, codebook, *, group):
        return self.vqdev.encode(values, codebook, group=group)

    def decode(self, value):
        return self.vqdev.decode(value)


def _weight(rng, shape, group, scale=0.05):
    from alelyon_compute_kit import vq
    w = (rng.standard_normal(shape) * scale).astype(np.float32)
    return vq.encode(w, vq.fit_codebook(w, group=group), group=group)


def _check_report(fused, plain, opt, grad, step):
    """The report of the fused step carries the reference's keys with the
    reference's meanings (vq.py:405-410): the same values as the unfused
    sequence's, native_update_output_bytes the dense [W'|M'|V'] update's size
    (the fused step evaluates it without storing it); only the calibration
    text says where the fit ran."""
    keys = {"step", "changed_weight_values", "persistent_state_bytes", "gradient_bytes",
            "native_update_output_bytes", "calibration", "model_quality_validated"}
    assert set(fused) == set(plain) == keys
    elements = opt.weight.layout["elements"]
    assert fused["step"] == step and fused["native_update_output_bytes"] == 12 * elements
    assert fused["gradient_bytes"] == grad.layout["serialized_bytes"]
    assert fused["persistent_state_bytes"] == sum(
        s.layout["serialized_bytes"] for s in (opt.weight, opt.momentum, opt.variance))
    assert fused["model_quality_validated"] is False
    assert fused["calibration"] == "device float64 fit of the update; no dense scratch written"
    assert plain["calibration"] == "CPU float32/float64 temporary arrays"  # vq.py:409
    for key in keys - {"calibration"}:
        assert fused[key] == plain[key], key


@pytest.mark.parametrize("shape,group", [((64, 48), 16), ((40, 40), 8), ((3000, 32), 32),
                                         ((512, 512), 8), ((1000, 77), 16)])
def test_fused_step_equals_the_unfused_sequence(vqdev, shape, group):
    from alelyon_compute_kit import vq
    rng = np.random.default_rng(group + shape[0])
    weight = _weight(rng, shape, group)
    fused = vq.VQAdamW(vqdev, weight, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01)
    plain = vq.VQAdamW(Unfused(vqdev), weight, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01)
    for step in range(3):
        g = (rng.standard_normal(shape) * 1e-2).astype(np.float32)
        grad = vq.encode(g, vq.fit_codebook(g, group=group), group=group)
        say("adamw step", shape, group, step)
        r1 = fused.step(grad)
        r2 = plain.step(grad)
        _check_report(r1, r2, fused, grad, step + 1)
        for a, b in ((fused.weight, plain.weight), (fused.momentum, plain.momentum),
                     (fused.variance, plain.variance)):
            np.testing.assert_array_equal(a.codebook, b.codebook)
            np.testing.assert_array_equal(a.codes, b.codes)


@pytest.mark.parametrize("group", [8, 16, 32])
def test_fused_step_overflowing_gradient_entry_used_or_not(vqdev, group):
    """A gradient book entry whose square overflows FP32 (V' = inf for every
    element that reads it). No vector uses it: the fused step (whose encode
    pass forms V' per (V, G) code pair, that entry included) completes and
    equals the unfused sequence. One vector uses it: both refuse the step, as
    op 3 reports a nonfinite result."""
    from alelyon_compute_kit import ack, vq
    rng = np.random.default_rng(70 + group)
    shape = (256, 8 * group)
    weight = _weight(rng, shape, group)
    vectors = shape[0] * shape[1] // group
    book = (rng.standard_normal((16, group)) * 1e-2).astype(np.float32)
    book[15] = np.float32(3e19)
    idx = rng.integers(0, 15, vectors)
    unused = vq.VQArray(shape, group, o_pack(idx), book)
    fused = vq.VQAdamW(vqdev, weight, lr=1e-3, betas=(0.9, 0.999))
    plain = vq.VQAdamW(Unfused(vqdev), weight, lr=1e-3, betas=(0.9, 0.999))
    say("adamw overflow entry unused", group)
    r1, r2 = fused.step(unused), plain.step(unused)
    _check_report(r1, r2, fused, unused, 1)
    for a, b in ((fused.weight, plain.weight), (fused.momentum, plain.momentum),
                 (fused.variance, plain.variance)):
        np.testing.assert_array_equal(a.codebook, b.codebook)
        np.testing.assert_array_equal(a.codes, b.codes)
    idx[vectors // 3] = 15
    used = vq.VQArray(shape, group, o_pack(idx), book)
    say("adamw overflow entry used", group)
    for opt in (vq.VQAdamW(vqdev, weight, lr=1e-3, betas=(0.9, 0.999)),
                vq.VQAdamW(Unfused(vqdev), weight, lr=1e-3, betas=(0.9, 0.999))):
        with pytest.raises(ack.AckError):
            opt.step(used)


def o_pack(idx):
    from oracle import vq4_numpy as o
    return o.pack_indices(idx.astype(np.int64))


@pytest.mark.parametrize("group,rare_at", [(8, -1), (16, -1), (32, -1), (8, 1)])
def test_zero_gradient_moves_no_weight_on_the_gpu(vqdev, group, rare_at):
    from alelyon_compute_kit import vq
    vectors = 65536 // group
    atoms = np.random.default_rng(1).standard_normal((16, group)).astype(np.float32)
    index = np.insert(np.arange(vectors - 1) % 15, rare_at % vectors, 15)
    values = atoms[index].reshape(-1)
    weight = vq.encode(values, atoms, group=group)
    zero = vq.VQArray(weight.shape, group, np.zeros_like(weight.codes),
                      np.zeros((16, group), np.float32))
    opt = vq.VQAdamW(vqdev, weight, lr=1e-3, weight_decay=0.0)
    say("zero gradient", group, rare_at)
    report = opt.step(zero)
    assert report["changed_weight_values"] == 0
    assert np.array_equal(opt.weight.decode(), values)
    assert len(np.unique(opt.weight.codebook.round(6), axis=0)) == 16


def test_fused_step_refuses_bad_coefficients_and_keeps_state(vqdev):
    from alelyon_compute_kit import ack, vq
    rng = np.random.default_rng(3)
    weight = _weight(rng, (64, 64), 16)
    variance = vq.VQArray(weight.shape, 16, weight.codes, -np.abs(weight.codebook) - 1)
    opt = vq.VQAdamW(vqdev, weight)
    opt.variance = variance
    say("adamw step negative variance")
    with pytest.raises(ack.AckError, match="status=4"):
        opt.step(weight)
    assert opt.steps == 0 and opt.weight is weight


def _oracle_encode_threads(oracle, x, book, group, parts=16):
    """The shader oracle's encode over word-aligned chunks on host threads
    (the C oracle releases the GIL): the same words as one call."""
    from concurrent.futures import ThreadPoolExecutor
    step = -(-x.size // parts)
    step = -(-step // (8 * group)) * 8 * group      # chunks start on code-word boundaries
    chunks = [x[i:i + step] for i in range(0, x.size, step)]
    with ThreadPoolExecutor(len(chunks)) as pool:
        results = list(pool.map(lambda c: oracle.encode(c, book, group), chunks))
    return np.concatenate([r[0] for r in results]), max(r[1] for r in results)


def test_config5_at_full_size(vqdev, oracle):
    """benchmark config 5: W 8192 x 8192, rows ~ N(0,1) then L2-normalised,
    group 8, book = fit_codebook(W). The GPU encode picks the oracle's code
    for every one of the 8,388,608 vectors, decode is the exact gather, and
    one fused VQAdamW step with an N(0, 1e-3) gradient equals the unfused
    sequence (op 3, native fits, GPU encode) bit for bit at full size."""
    from alelyon_compute_kit import vq
    n, g = 8192, 8
    rng = np.random.default_rng(5)
    w = rng.standard_normal((n, n), dtype=np.float32)
    w /= np.linalg.norm(w, axis=1, keepdims=True).astype(np.float32)
    book = vq.fit_codebook(w, group=g)
    say("config5 encode", n, g)
    img = vqdev.encode(w, book, group=g)
    vectors = w.reshape(-1, g)
    ref_codes, status = _oracle_encode_threads(oracle, w.reshape(-1), book, g)
    assert status == 0
    from oracle import vq4_numpy as o
    np.testing.assert_array_equal(img.codes, ref_codes)
    say("config5 decode")
    dense = vqdev.decode(img)
    np.testing.assert_array_equal(dense.reshape(-1, g), book[o.unpack_indices(img.codes,
                                                                              vectors.shape[0])])
    del w, vectors, dense
    grad = rng.standard_normal((n, n), dtype=np.float32) * np.float32(np.sqrt(1e-3))
    g_img = vq.encode(grad, vq.fit_codebook(grad, group=g), group=g)
    del grad
    say("config5 fused step")
    fused = vq.VQAdamW(vqdev, img, lr=1e-3, betas=(0.9, 0.999))
    plain = vq.VQAdamW(Unfused(vqdev), img, lr=1e-3, betas=(0.9, 0.999))
    r1, r2 = fused.step(g_img), plain.step(g_img)
    assert r1["changed_weight_values"] == r2["changed_weight_values"]
    for a, b in ((fused.weight, plain.weight), (fused.momentum, plain.momentum),
                 (fused.variance, plain.variance)):
        np.testing.assert_array_equal(a.codebook, b.codebook)
        np.testing.assert_array_equal(a.codes, b.codes)
