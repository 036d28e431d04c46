"""The expert bank (on-disk generations) and the harness that trains through it.

CPU tests pin the bank's format against the reference's seeded payloads
(tests/golden/expert_payloads.npz, written from the reference's own
ExpertBank.initialize_expert), its commit counters and refusals, and the
harness flow with a host backend. GPU tests run the harness step and the
benchmark config-2 flow on the MI355X and require every committed image to be
byte-identical to the same flow computed by the CPU oracle.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from alelyon_compute_kit import expert_bank, harness, vq
from conftest import golden


class HostBackend:
    """numpy arithmetic on decoded operands (the reference's test fake,
    tests/test_harness.py:7-28, restated)."""

    def encode(self, values, codebook, *, group):
        return vq.encode(values, codebook, group=group)

    def decode(self, value):
        return value.decode()

    def matmul(self, left, right, *, transpose_a=False, transpose_b=False):
        a, b = left.decode(), right.decode()
        return (a.T if transpose_a else a) @ (b.T if transpose_b else b)

    def adamw(self, weight, momentum, variance, gradient, *, lr, beta1, beta2, eps,
              weight_decay, step):
        w, m, v, g = (s.decode() for s in (weight, momentum, variance, gradient))
        m = beta1 * m + (1.0 - beta1) * g
        v = beta2 * v + (1.0 - beta2) * np.square(g)
        w = w - lr * ((m / (1.0 - beta1 ** step)) / (np.sqrt(v / (1.0 - beta2 ** step)) + eps)
                      + weight_decay * w)
        return w.astype(np.float32), m.astype(np.float32), v.astype(np.float32)


def _small_bank(tmp_path, name="bank"):
    bank = expert_bank.ExpertBank.create(
        tmp_path / name, expert_bank.BankConfig(1, 1, ((4, 3), (4, 3), (4, 3)), 8))
    bank.initialize_expert(0, 0, seed=4, zero_optimizer_state=True)
    return bank


# ---- bank ----------------------------------------------------------------------
def test_bank_metadata_is_canonical_and_reopens(tmp_path):
    config = expert_bank.BankConfig(2, 3, ((8, 16), (16, 8)), 8)
    bank = expert_bank.ExpertBank.create(tmp_path / "b", config)
    data = (tmp_path / "b" / "bank.json").read_bytes()
    assert data == json.dumps({"schema": "ack-expert-bank/v1", "config": config.to_dict()},
                              sort_keys=True, separators=(",", ":")).encode()
    again = expert_bank.ExpertBank.open(tmp_path / "b")
    assert again.config == bank.config and again.config.parameters_per_expert == 256
    with pytest.raises(FileExistsError):
        expert_bank.ExpertBank.create(tmp_path / "b", config)
    (tmp_path / "b" / "bank.json").write_bytes(data.replace(b":", b": ", 1))
    with pytest.raises(expert_bank.ExpertBankError, match="noncanonical"):
        expert_bank.ExpertBank.open(tmp_path / "b")


@pytest.mark.parametrize("bad", [
    dict(layers=0, experts_per_layer=1, matrix_shapes=((4, 4),)),
    dict(layers=1, experts_per_layer=1, matrix_shapes=((4, 4),), group=12),
    dict(layers=1, experts_per_layer=1, matrix_shapes=()),
    dict(layers=1, experts_per_layer=1, matrix_shapes=((4, 4, 4),)),
    dict(layers=True, experts_per_layer=1, matrix_shapes=((4, 4),)),
])
def test_bank_config_refusals(bad):
    with pytest.raises(expert_bank.ExpertBankError):
        expert_bank.BankConfig(**bad)


def test_initialize_expert_matches_the_reference_payloads(tmp_path):
    g = golden("expert_payloads.npz")
    bank = expert_bank.ExpertBank.create(
        tmp_path / "c2", expert_bank.BankConfig(1, 1, ((128, 128),) * 3, 16))
    bank.initialize_expert(0, 0, seed=7)
    for i, t in enumerate(bank.read_expert(0, 0)):
        assert np.array_equal(t.codes, g[f"c2_{i}_codes"])
        assert np.array_equal(t.codebook.view(np.uint32), g[f"c2_{i}_book"].view(np.uint32))
    small = _small_bank(tmp_path)
    for i, t in enumerate(small.read_expert(0, 0)):
        assert np.array_equal(t.codes, g[f"h_{i}_codes"])
        assert np.array_equal(t.codebook.view(np.uint32), g[f"h_{i}_book"].view(np.uint32))
    with pytest.raises(expert_bank.ExpertBankError, match="already"):
        small.initialize_expert(0, 0, seed=4)


def test_write_counters_generations_and_refusals(tmp_path):
    bank = _small_bank(tmp_path)
    state = bank.read_expert_state(0, 0)
    assert (state.revision, state.optimizer_step, state.parameter_update_applications) == (1, 0, 0)
    receipt = bank.write_expert(0, 0, state.tensors, updated_count=12, optimizer_step=3)
    assert receipt["revision"] == 2 and receipt["parameter_update_applications"] == 12
    after = bank.read_expert_state(0, 0)
    assert (after.revision, after.optimizer_step) == (2, 3)
    pointer = json.loads((bank.root / "expert-0-0.json").read_bytes())
    assert pointer["update_commits"] == 1
    with pytest.raises(expert_bank.ExpertBankError, match="regress"):
        bank.write_expert(0, 0, state.tensors, optimizer_step=2)
    wrong = vq.VQArray((3, 4), 8, state.tensors[0].codes, state.tensors[0].codebook)
    with pytest.raises(expert_bank.ExpertBankError, match="geometry"):
        bank.write_expert(0, 0, (wrong,) + state.tensors[1:])
    with pytest.raises(expert_bank.ExpertBankError):
        bank.write_expert(0, 1, state.tensors)
    # refused writes leave no pending pointer and no new shards behind
    names = sorted(p.name for p in bank.root.iterdir())
    assert not any(n.startswith("pending-") for n in names)
    assert sum(n.endswith(".vq") for n in names) == 6  # two generations x three shards
    stats = bank.stats()
    assert stats["materialized_experts"] == 1 and stats["updated_experts"] == 1
    assert stats["committed_payload_bytes"] == sum(t.layout["serialized_bytes"]
                                                   for t in state.tensors)


def _reference_bank():
    """The files the reference's ExpertBank left after create, three seeded
    experts and two updates of expert (0, 1) (tests/golden/make_golden.py)."""
    g = golden("bank_files.npz")
    blob, off = g["blob"].tobytes(), g["offsets"]
    files = {str(n): blob[off[i]:off[i + 1]] for i, n in enumerate(g["names"])}
    return files, [str(h) for h in g["history_0_1"]], g["stats"].tobytes()


def test_a_reference_written_bank_opens_and_reads(tmp_path):
    files, _, stats = _reference_bank()
    root = tmp_path / "ref"
    root.mkdir()
    for name, data in files.items():
        (root / name).write_bytes(data)
    bank = expert_bank.ExpertBank.open(root)
    state = bank.read_expert_state(0, 1)
    assert (state.optimizer_step, state.revision, state.parameter_update_applications) == \
        (4, 3, 117)
    assert state.tensors == bank.read_expert(1, 1)       # the second update carried (1, 1)'s
    zero = bank.read_expert(1, 0)
    assert not zero[1].codes.any() and not zero[2].codebook.any()
    assert expert_bank.canonical_json(bank.stats()) == stats


def test_this_writer_leaves_the_reference_files(tmp_path):
    """The same operations write the same bytes: bank.json, every shard and
    every pointer, once generation ids (uuid4, random in both) are mapped."""
    files, history, stats = _reference_bank()
    root = tmp_path / "ours"
    bank = expert_bank.ExpertBank.create(
        root, expert_bank.BankConfig(2, 2, ((10, 13), (13, 10), (10, 13)), 8))
    ours = []

    def generation(base):
        return json.loads((root / f"{base}.json").read_text())["generation"]

    bank.initialize_expert(0, 1, seed=3)
    ours.append(generation("expert-0-1"))
    bank.initialize_expert(1, 0, seed=5, zero_optimizer_state=True)
    bank.initialize_expert(1, 1, seed=9)
    bank.write_expert(0, 1, bank.read_expert(1, 0), updated_count=100, optimizer_step=1)
    ours.append(generation("expert-0-1"))
    bank.write_expert(0, 1, bank.read_expert(1, 1), updated_count=17, optimizer_step=4)
    ours.append(generation("expert-0-1"))
    rename = dict(zip(ours, history))
    for base in ("expert-1-0", "expert-1-1"):
        rename[generation(base)] = json.loads(files[f"{base}.json"])["generation"]

    def mapped(text: str) -> str:
        for mine, theirs in rename.items():
            text = text.replace(mine, theirs)
        return text

    written = {mapped(p.name): p.read_bytes() for p in root.iterdir()}
    assert sorted(written) == sorted(files)
    for name, data in written.items():
        if name.endswith(".json"):
            data = mapped(data.decode()).encode()
        assert data == files[name], name
    assert expert_bank.canonical_json(bank.stats()) == stats


def test_this_writer_leaves_the_reference_files_at_full_size(tmp_path):
    """Full-size experts (three 4096x4096 group-16 matrices): the same seeded
    experts and committed update leave files of the same names (generation
    ids mapped), sizes and SHA-256 as the reference writer's, the same pointer
    and bank JSON, and the same stats (tests/golden/bank_scale.npz)."""
    import hashlib
    g = golden("bank_scale.npz")
    ref = {str(n): (int(sz), str(h)) for n, sz, h in zip(g["names"], g["sizes"], g["sha256"])}
    blob, off = g["json_blob"].tobytes(), g["json_offsets"]
    ref_json = {str(n): blob[off[i]:off[i + 1]] for i, n in enumerate(g["json_names"])}
    history = [str(h) for h in g["history_0_0"]]
    root = tmp_path / "scale"
    bank = expert_bank.ExpertBank.create(
        root, expert_bank.BankConfig(1, 2, ((4096, 4096),) * 3, 16))

    def generation(base):
        return json.loads((root / f"{base}.json").read_text())["generation"]

    ours = []
    bank.initialize_expert(0, 0, seed=11)
    ours.append(generation("expert-0-0"))
    bank.initialize_expert(0, 1, seed=12, zero_optimizer_state=True)
    bank.write_expert(0, 0, bank.read_expert(0, 1), updated_count=4096, optimizer_step=2)
    ours.append(generation("expert-0-0"))
    rename = dict(zip(ours, history))
    rename[generation("expert-0-1")] = json.loads(ref_json["expert-0-1.json"])["generation"]

    def mapped(text: str) -> str:
        for mine, theirs in rename.items():
            text = text.replace(mine, theirs)
        return text

    written = {mapped(p.name): p for p in root.iterdir()}
    assert sorted(written) == sorted(ref)
    for name, path in written.items():
        data = path.read_bytes()
        if name.endswith(".json"):
            data = mapped(data.decode()).encode()
            assert data == ref_json[name], name
        assert (len(data), hashlib.sha256(data).hexdigest()) == ref[name], name
    assert expert_bank.canonical_json(bank.stats()) == g["stats"].tobytes()


def test_a_changed_shard_is_refused(tmp_path):
    bank = _small_bank(tmp_path)
    pointer = json.loads((bank.root / "expert-0-0.json").read_bytes())
    shard = bank.root / f"expert-0-0-g{pointer['generation']}-t0.vq"
    data = bytearray(shard.read_bytes())
    data[-1] ^= 1
    shard.write_bytes(bytes(data))
    with pytest.raises(expert_bank.ExpertBankError, match="checksum"):
        bank.read_expert_state(0, 0)
    zero = vq.VQArray((4, 3), 8, np.zeros(1, np.uint32), np.zeros((16, 8), np.float32))
    with pytest.raises(expert_bank.ExpertBankError, match="checksum"):
        bank.write_expert(0, 0, (zero, zero, zero))  # never builds on corrupt state


# ---- harness with a host backend ------------------------------------------------
def test_forward_is_the_packed_product_and_checks_width(tmp_path):
    bank = _small_bank(tmp_path)
    runner = harness.VulkanExpertHarness(bank, backend=HostBackend())
    x = np.arange(8, dtype=np.float32).reshape(2, 4)
    expected = x @ bank.read_expert_state(0, 0).tensors[0].decode()
    np.testing.assert_array_equal(runner.forward(x), expected)
    with pytest.raises(harness.HarnessError, match="width"):
        runner.forward(np.zeros((2, 5), np.float32))
    with pytest.raises(harness.HarnessError, match="rank-2 float32"):
        runner.forward(np.zeros((2, 4), np.float64))


def test_train_step_commits_the_optimizer_state(tmp_path):
    bank = _small_bank(tmp_path)
    runner = harness.ExpertHarness(bank, backend=HostBackend())
    before = bank.read_expert_state(0, 0)
    step = runner.train_step(np.ones((2, 4), np.float32), np.zeros((2, 3), np.float32),
                             max_grad_norm=0.01)
    after = bank.read_expert_state(0, 0)
    assert (step.optimizer_step, step.revision) == (1, 2)
    assert after.optimizer_step == 1 and after.parameter_update_applications == 12
    assert step.clipped and step.persistent_state_bytes > 0
    assert before.tensors[0].to_bytes() != after.tensors[0].to_bytes()
    assert set(step.to_dict()) >= {"loss", "gradient_norm_before_clip", "clipped"}
    with pytest.raises(harness.HarnessError, match="finite"):
        runner.forward(np.full((2, 4), np.nan, np.float32))
    with pytest.raises(harness.HarnessError, match="row count"):
        runner.train_step(np.ones((2, 4), np.float32), np.zeros((3, 3), np.float32))
    with pytest.raises(harness.HarnessError, match="positive"):
        runner.train_step(np.ones((2, 4), np.float32), np.zeros((2, 3), np.float32),
                          max_grad_norm=0.0)
    steps = runner.train(np.ones((2, 4), np.float32), np.zeros((2, 3), np.float32), steps=2)
    assert [s.optimizer_step for s in steps] == [2, 3]
    assert bank.read_expert_state(0, 0).revision == 4


def test_harness_refuses_bad_construction(tmp_path):
    bank = _small_bank(tmp_path)
    with pytest.raises(harness.HarnessError, match="ExpertBank"):
        harness.ExpertHarness(object(), backend=HostBackend())
    with pytest.raises(harness.HarnessError, match="not both"):
        harness.ExpertHarness(bank, backend=HostBackend(), device=object())


# ---- GPU parity of whole flows ----------------------------------------------------
def _twin_banks(tmp_path, shapes, group, seed, zero):
    banks = []
    for name in ("gpu", "cpu"):
        b = expert_bank.ExpertBank.create(tmp_path / name,
                                          expert_bank.BankConfig(1, 1, shapes, group))
        b.initialize_expert(0, 0, seed=seed, zero_optimizer_state=zero)
        banks.append(b)
    return banks


@pytest.mark.gpu
def test_harness_step_on_the_gpu_commits_the_oracle_images(tmp_path, vqdev):
    """Two steps of the harness on config-2-sized matrices (128 x 128, group
    16, seed 7, zero moments; x 32 x 128 ~ N(0,1), targets ~ N(0, 1e-2)):
    the GPU run and the CPU-oracle run commit byte-identical generations."""
    from gpu_util import say
    from oracle_backend import OracleBackend
    gpu_bank, cpu_bank = _twin_banks(tmp_path, ((128, 128),) * 3, 16, 7, True)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 128)).astype(np.float32)
    t = (rng.standard_normal((32, 128)) * 0.1).astype(np.float32)
    say("harness step parity")
    gpu = harness.ExpertHarness(gpu_bank, backend=vqdev)
    cpu = harness.ExpertHarness(cpu_bank, backend=OracleBackend())
    for _ in range(2):
        a = gpu.train_step(x, t, lr=1e-3, beta1=0.9, beta2=0.999, max_grad_norm=1.0)
        b = cpu.train_step(x, t, lr=1e-3, beta1=0.9, beta2=0.999, max_grad_norm=1.0)
        assert (a.loss, a.gradient_norm_before_clip, a.clipped) == \
               (b.loss, b.gradient_norm_before_clip, b.clipped)
        for ta, tb in zip(gpu_bank.read_expert(0, 0), cpu_bank.read_expert(0, 0)):
            assert ta.to_bytes() == tb.to_bytes()
    np.testing.assert_array_equal(gpu.forward(x), cpu.forward(x))


@pytest.mark.gpu
def test_config2_chain_and_clipped_step_match_the_oracle(vqdev):
    """benchmark config 2: three 128 x 128 matrices from initialize_expert(0, 0,
    seed=7) at group 16; x 32 x 128 ~ N(0,1) fitted and encoded and pushed
    through the three packed products in sequence (each output re-fitted and
    re-encoded); then one VQAdamW step (lr 1e-3, betas (0.9, 0.999)) per matrix
    on N(0, 1e-2) gradients clipped to global norm 1.0. Every image and output
    equals the CPU oracle's, bit for bit."""
    from gpu_util import say
    from oracle.vq4_numpy import clip_scale, expert_payload
    from oracle_backend import OracleBackend
    cpu = OracleBackend()
    weights = [vq.VQArray((128, 128), 16, *expert_payload((128, 128), 16, 7, 0, 0, i))
               for i in range(3)]
    rng = np.random.default_rng(7)
    x = rng.standard_normal((32, 128)).astype(np.float32)
    say("config2 chain")
    ha = hb = x
    for w in weights:
        ia = vqdev.encode(ha, vq.fit_codebook(ha, group=16), group=16)
        ib = cpu.encode(hb, vq.fit_codebook(hb, group=16), group=16)
        assert ia == ib
        ha, hb = vqdev.matmul(ia, w), cpu.matmul(ib, w)
        np.testing.assert_array_equal(ha.view(np.uint32), hb.view(np.uint32))
    grads = [(rng.standard_normal((128, 128)) * 0.1).astype(np.float32) for _ in range(3)]
    norm_scale = clip_scale(np.concatenate([g.reshape(-1) for g in grads]), 1.0)
    say("config2 step")
    for w, g in zip(weights, grads):
        g = g * np.float32(norm_scale)
        gi = vq.encode(g, vq.fit_codebook(g, group=16), group=16)
        opt_a = vq.VQAdamW(vqdev, w, lr=1e-3, betas=(0.9, 0.999))
        opt_b = vq.VQAdamW(cpu, w, lr=1e-3, betas=(0.9, 0.999))
        ra, rb = opt_a.step(gi), opt_b.step(gi)
        assert ra["changed_weight_values"] == rb["changed_weight_values"]
        for sa, sb in ((opt_a.weight, opt_b.weight), (opt_a.momentum, opt_b.momentum),
                       (opt_a.variance, opt_b.variance)):
            assert sa.to_bytes() == sb.to_bytes()


@pytest.mark.gpu
@pytest.mark.parametrize("shape,group,batch,certified", [((128, 128), 16, 32, True),
                                                         ((512, 384), 8, 64, True),
                                                         ((96, 256), 32, 3, True),
                                                         ((128, 128), 16, 32, False)])
def test_resident_harness_commits_the_default_images(tmp_path, vqdev, monkeypatch, shape, group,
                                                      batch, certified):
    """The resident harness (optimizer state kept on the device, codebooks
    fitted there, the clip from the device's sum of squares) commits
    byte-identical generations to the default GPU harness over three steps,
    the middle one clipped; a write by another harness in between is picked
    up. certified False: every clip falls back to numpy's norm of the
    downloaded gradient, the path taken when the device sum cannot certify
    numpy's float32 scale."""
    from gpu_util import say
    if not certified:
        monkeypatch.setattr(harness, "_certified_clip", lambda *args: None)
    a_bank, b_bank = _twin_banks(tmp_path, (shape,) * 3, group, 11, True)
    rng = np.random.default_rng(shape[0] + batch)
    x = rng.standard_normal((batch, shape[0])).astype(np.float32)
    t = (rng.standard_normal((batch, shape[1])) * 0.1).astype(np.float32)
    say("resident harness", shape, group, batch)
    res = harness.ExpertHarness(a_bank, backend=vqdev, resident=True)
    plain = harness.ExpertHarness(b_bank, backend=vqdev)
    try:
        for norm in (10.0, 1e-3, 10.0):
            a = res.train_step(x, t, lr=1e-3, beta1=0.9, beta2=0.999, max_grad_norm=norm)
            b = plain.train_step(x, t, lr=1e-3, beta1=0.9, beta2=0.999, max_grad_norm=norm)
            da, db = a.to_dict(), b.to_dict()
            da.pop("elapsed_seconds"), db.pop("elapsed_seconds")
            # the resident norm is the device's float64 sum of squares, within
            # the certified slack of numpy's dot product
            na, nb = da.pop("gradient_norm_before_clip"), db.pop("gradient_norm_before_clip")
            count = shape[0] * shape[1]
            assert abs(na - nb) <= nb * (count + 64) * 2.0 ** -53
            assert da == db
            for ta, tb in zip(a_bank.read_expert(0, 0), b_bank.read_expert(0, 0)):
                assert ta.to_bytes() == tb.to_bytes()
        np.testing.assert_array_equal(res.forward(x), plain.forward(x))
        # another writer commits to the resident expert: the next step reloads
        other = harness.ExpertHarness(a_bank, backend=vqdev)
        other.train_step(x, t, lr=1e-3)
        plain.train_step(x, t, lr=1e-3)
        a = res.train_step(x, t, lr=1e-3)
        b = plain.train_step(x, t, lr=1e-3)
        assert a.revision == b.revision == 6
        for ta, tb in zip(a_bank.read_expert(0, 0), b_bank.read_expert(0, 0)):
            assert ta.to_bytes() == tb.to_bytes()
    finally:
        res.close()


def test_certified_clip_brackets_numpys_norm():
    """The device's float64 sum of squares certifies numpy's clip only when
    every sum within the slack gives the same float32 scale and verdict; the
    certified scale then equals numpy's, and the norm agrees within it."""
    import math
    rng = np.random.default_rng(0)
    certified = 0
    for trial in range(300):
        g = (rng.standard_normal(1000) * 10.0 ** rng.uniform(-4, 1)).astype(np.float32)
        exact = math.fsum(np.square(g.astype(np.float64)))  # exact squares, exactly rounded sum
        clip = harness._certified_clip(exact, g.size, 1.0)
        norm, scale = harness._clip_factor(g, 1.0)
        if clip is None:
            continue
        certified += 1
        assert np.float32(clip[1]) == np.float32(scale) and (clip[1] < 1.0) == (scale < 1.0)
        assert abs(clip[0] - norm) <= norm * 1024 * 2.0 ** -53
    assert certified >= 290
    # a scale half a float32 ulp from a rounding boundary, and a norm at the
    # clip's threshold, are not certified
    f = np.float32(0.3)
    mid = float(f) + float(np.spacing(f)) / 2
    assert harness._certified_clip((1.0 / mid - 1e-6) ** 2, 10 ** 6, 1.0) is None
    assert harness._certified_clip((1.0 - 1e-6) ** 2, 10 ** 6, 1.0) is None
    assert harness._certified_clip(4.0, 10 ** 6, 1.0)[1] == 1.0 / (2.0 + 1e-6)
    with pytest.raises(harness.HarnessError, match="nonfinite"):
        harness._certified_clip(float("inf"), 10, 1.0)


@pytest.mark.gpu
@pytest.mark.parametrize("count", [1, 7, 4096, 1_000_003, 4_194_304])
def test_device_sum_of_squares_and_scale(vqdev, count):
    """ack_vq_sum_squares within its stated bound of the exactly rounded sum
    of the (exact) float64 squares; ack_vq_scale equal to numpy's float32
    multiply bit for bit; a nonfinite value makes the sum nonfinite."""
    import math
    from gpu_util import say
    rng = np.random.default_rng(count)
    x = (rng.standard_normal(count) * 3).astype(np.float32)
    device = vqdev.device
    buf, out = device.buffer(x.nbytes), device.buffer(8)
    try:
        say("sum of squares", count)
        buf.upload(x)
        vqdev.sum_squares_resident(buf, count, out)
        got = float(out.download(np.float64)[0])
        exact = math.fsum(np.square(x.astype(np.float64)))
        assert abs(got - exact) <= exact * (count / 65536 + 15) * 2.0 ** -53
        vqdev.scale_resident(buf, count, 0.7)
        y = buf.download(np.float32)
        np.testing.assert_array_equal(y.view(np.uint32), (x * np.float32(0.7)).view(np.uint32))
        x[count // 2] = np.inf
        buf.upload(x)
        vqdev.sum_squares_resident(buf, count, out)
        assert not math.isfinite(float(out.download(np.float64)[0]))
    finally:
        buf.free()
        out.free()


def test_resident_harness_needs_a_device_backend(tmp_path):
    bank = expert_bank.ExpertBank.create(
        tmp_path / "r", expert_bank.BankConfig(1, 1, ((4, 3), (4, 3), (4, 3)), 8))
    with pytest.raises(harness.HarnessError, match="VQDevice"):
        harness.ExpertHarness(bank, backend=HostBackend(), resident=True)
    with pytest.raises(harness.HarnessError, match="bool"):
        harness.ExpertHarness(bank, backend=HostBackend(), resident=1)


def test_forward_batch_equals_per_expert_forward_on_a_host_backend(tmp_path):
    bank = expert_bank.ExpertBank.create(
        tmp_path / "many", expert_bank.BankConfig(2, 3, ((16, 24), (16, 24), (16, 24)), 8))
    for layer in range(2):
        for e in range(3):
            bank.initialize_expert(layer, e, seed=layer * 10 + e)
    h = harness.ExpertHarness(bank, backend=HostBackend())
    rng = np.random.default_rng(1)
    xs = [rng.standard_normal((5, 16)).astype(np.float32) for _ in range(4)]
    experts = [(0, 2), (1, 0), (0, 2), (1, 1)]
    got = h.forward_batch(xs, experts)
    for x, (layer, e), y in zip(xs, experts, got):
        np.testing.assert_array_equal(y, h.forward(x, layer=layer, expert=e))
    with pytest.raises(harness.HarnessError, match="one input"):
        h.forward_batch(xs[:2], experts)
    with pytest.raises(harness.HarnessError, match="share one shape"):
        h.forward_batch([xs[0], xs[1][:3]], experts[:2])


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 4, 32])
def test_forward_batch_is_one_launch_over_many_experts(tmp_path, vqdev, m):
    """Eight experts of a 4096 x 4096 g16 bank in one batched launch: each
    output agrees with that expert's own forward and with the float64 product
    of the decoded operands within 1e-5."""
    from gpu_util import say
    from oracle import vq4_numpy as o
    bank = expert_bank.ExpertBank.create(
        tmp_path / "many", expert_bank.BankConfig(2, 4, ((4096, 4096),) * 3, 16))
    experts = [(layer, e) for layer in range(2) for e in range(4)]
    for layer, e in experts:
        bank.initialize_expert(layer, e, seed=3 + layer * 4 + e, zero_optimizer_state=True)
    h = harness.ExpertHarness(bank, backend=vqdev)
    rng = np.random.default_rng(m)
    xs = [rng.standard_normal((m, 4096)).astype(np.float32) for _ in experts]
    say("forward_batch", m, len(experts))
    got = h.forward_batch(xs, experts)
    for x, (layer, e), y in zip(xs, experts, got):
        one = h.forward(x, layer=layer, expert=e)
        assert o.max_rel(y, one) <= 1e-5
        x_img = h.encode_activations(x, 16)
        exact = o.matmul64(x_img.decode(), bank.read_expert(layer, e)[0].decode())
        assert o.max_rel(y, exact) <= 1e-5


def test_forward_batch_refuses_a_wrong_width(tmp_path):
    bank = expert_bank.ExpertBank.create(
        tmp_path / "mixed", expert_bank.BankConfig(2, 1, ((16, 24), (16, 24), (16, 24)), 8))
    bank.initialize_expert(0, 0, seed=1)
    bank.initialize_expert(1, 0, seed=2)
    h = harness.ExpertHarness(bank, backend=HostBackend())
    x = np.ones((2, 16), np.float32)
    with pytest.raises(harness.HarnessError, match="width"):
        h.forward_batch([x[:, :8]], [(0, 0)])
    assert h.forward_batch([x, x], [(0, 0), (1, 0)]).shape == (2, 2, 24)


# ---- command line and its files ------------------------------------------------------
def test_cli_file_helpers(tmp_path):
    """.npy inputs only (no archives, no symlinks, no pickles), checked as
    matrices; outputs never overwritten without --force, written whole."""
    good = tmp_path / "x.npy"
    np.save(good, np.ones((2, 3), np.float32))
    np.testing.assert_array_equal(harness._read_matrix(good, "input"), np.ones((2, 3)))
    archive = tmp_path / "x.npz"
    np.savez(archive, a=np.ones((2, 3), np.float32))
    with pytest.raises(harness.HarnessError, match="archive"):
        harness._read_matrix(archive, "input")
    link = tmp_path / "link.npy"
    link.symlink_to(good)
    with pytest.raises(harness.HarnessError, match="regular file"):
        harness._read_matrix(link, "input")
    junk = tmp_path / "junk.npy"
    junk.write_bytes(b"not an array")
    with pytest.raises(harness.HarnessError, match="readable NumPy"):
        harness._read_matrix(junk, "input")
    pickled = tmp_path / "obj.npy"
    np.save(pickled, np.array([{"a": 1}], dtype=object), allow_pickle=True)
    with pytest.raises(harness.HarnessError, match="readable NumPy"):
        harness._read_matrix(pickled, "input")
    wide = tmp_path / "f64.npy"
    np.save(wide, np.ones((2, 3)))
    with pytest.raises(harness.HarnessError, match="rank-2 float32"):
        harness._read_matrix(wide, "input")
    out = tmp_path / "sub" / "y.npy"
    harness._write_matrix(out, np.arange(6, dtype=np.float32).reshape(2, 3), force=False)
    with pytest.raises(harness.HarnessError, match="overwrite"):
        harness._write_matrix(out, np.zeros((2, 3), np.float32), force=False)
    harness._write_matrix(out, np.zeros((2, 3), np.float32), force=True)
    assert not np.load(out).any()
    assert sorted(p.name for p in out.parent.iterdir()) == ["y.npy"]   # no temporaries left


def test_cli_requires_the_device_flag(tmp_path, capsys):
    with pytest.raises(SystemExit):
        harness.main(["--bank", str(tmp_path), "--input", "x", "--output", "y"])
    assert "--device is required" in capsys.readouterr().err


@pytest.mark.gpu
def test_cli_forward_and_train_on_the_gpu(tmp_path, capsys):
    """The command line over a bank: a forward, then two training steps and
    the forward after them, each reported as JSON."""
    from gpu_util import say
    bank = _small_bank(tmp_path)
    x, t = tmp_path / "x.npy", tmp_path / "t.npy"
    np.save(x, np.ones((2, 4), np.float32))
    np.save(t, np.zeros((2, 3), np.float32))
    say("cli forward")
    assert harness.main(["--device", "--bank", str(bank.root), "--input", str(x),
                         "--output", str(tmp_path / "y.npy")]) == 0
    report = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert report["mode"] == "forward" and report["shape"] == [2, 3]
    assert np.load(tmp_path / "y.npy").shape == (2, 3)
    say("cli train")
    assert harness.main(["--device", "--bank", str(bank.root), "--input", str(x), "--target",
                         str(t), "--steps", "2", "--output", str(tmp_path / "y.npy"),
                         "--force"]) == 0
    report = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert report["mode"] == "train" and [s["optimizer_step"] for s in report["steps"]] == [1, 2]
    assert bank.read_expert_state(0, 0).revision == 3
    assert report["device"]["abi"]["vq_schema"] == 1


@pytest.mark.gpu
def test_cli_resident_commits_the_same_bytes(tmp_path, capsys):
    """--resident on the command line keeps the optimizer state on the GPU
    and commits the images the default run commits, byte for byte."""
    from gpu_util import say
    x, t = tmp_path / "x.npy", tmp_path / "t.npy"
    rng = np.random.default_rng(4)
    np.save(x, rng.standard_normal((2, 4)).astype(np.float32))
    np.save(t, rng.standard_normal((2, 3)).astype(np.float32))
    images = []
    for flag in ([], ["--resident"]):
        bank = _small_bank(tmp_path, "resident" if flag else "default")
        say("cli train", *flag)
        assert harness.main(["--device", "--bank", str(bank.root), "--input", str(x),
                             "--target", str(t), "--steps", "2", "--output",
                             str(tmp_path / "y.npy"), "--force", *flag]) == 0
        capsys.readouterr()
        state = bank.read_expert_state(0, 0)
        assert state.revision == 3
        images.append([img.to_bytes() for img in state.tensors])
    assert images[0] == images[1]
