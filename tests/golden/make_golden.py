"""Write the golden vectors in this directory from the reference's own Python.

Run in the build container only, where the reference is mounted:

    PYTHONPATH=/root/reference/src python tests/golden/make_golden.py

It imports the reference's CPU functions -- ``encode``, ``fit_codebook``,
``VQArray``, ``VQAdamW`` (src/alelyon_compute_kit/_kit/python/vq.py),
``ExpertBank`` (_kit/python/expert_bank.py:148-430: ``initialize_expert``
payloads and the files a short sequence of commits leaves on disk, at 10x13
and at 4096x4096) and the
harness's gradient clip (src/alelyon_compute_kit/harness.py:196-200, observed
through ``VulkanExpertHarness.train_step`` with a host backend) -- the
functions no closed form or known-answer test pins bit for bit, and records
their inputs and outputs as .npz fixtures (no pickles). Nothing under
/root/reference is needed, read or copied at test time.

With fixture names as arguments (``clip_scale``, ``bank_files``, ...) only
those files are written; the default writes all of them.
"""
from __future__ import annotations

import math
import sys
import tempfile
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent

try:
    from alelyon_compute_kit import harness as ref_harness
    from alelyon_compute_kit._kit.python import expert_bank as ref_bank
    from alelyon_compute_kit._kit.python import vq as ref_vq
except ImportError as exc:  # pragma: no cover - build container only
    sys.exit(f"the reference is not importable ({exc}); set PYTHONPATH=/root/reference/src")

if not str(Path(ref_vq.__file__)).startswith("/root/reference/"):
    sys.exit(f"refusing to record fixtures from {ref_vq.__file__}: not the reference")


def encode_cases() -> dict:
    rng = np.random.default_rng(20261201)
    out = {}
    n = 0
    for group in (8, 16, 32):
        for m in (1, group - 1, group, 8 * group + 3, 1000, 4096 + 5):
            x = rng.standard_normal(m).astype(np.float32)
            book = rng.standard_normal((16, group)).astype(np.float32)
            img = ref_vq.encode(x, book, group=group)
            out[f"c{n}_x"], out[f"c{n}_book"] = x, book
            out[f"c{n}_group"] = np.array(group)
            out[f"c{n}_codes"] = img.codes
            n += 1
        # exact ties: every value equals the midpoint of entries 3 and 9
        book = rng.standard_normal((16, group)).astype(np.float32)
        book[9] = book[3] + np.float32(2.0)
        x = np.tile(book[3] + np.float32(1.0), 40).astype(np.float32)
        img = ref_vq.encode(x, book, group=group)
        out[f"c{n}_x"], out[f"c{n}_book"] = x, book
        out[f"c{n}_group"] = np.array(group)
        out[f"c{n}_codes"] = img.codes
        n += 1
    out["count"] = np.array(n)
    return out


def review_shape(group, rare_at=-1):
    """The reference test's 65,536-value construction
    (tests/test_fit_codebook_keeps_every_entry.py:245-250)."""
    vectors = 65536 // group
    atoms = np.random.default_rng(1).standard_normal((16, group)).astype(np.float32)
    index = np.insert(np.arange(vectors - 1) % 15, rare_at % vectors, 15)
    return atoms, index


def fit_cases() -> dict:
    rng = np.random.default_rng(7)
    cases = []
    for group in (8, 16, 32):
        x = rng.standard_normal(1200 * group + 5).astype(np.float32)
        cases.append(dict(values=x, group=group, iterations=4, sample_vectors=4096, init=None))
        cases.append(dict(values=x, group=group, iterations=2, sample_vectors=64, init=None))
        init = rng.standard_normal((16, group)).astype(np.float32)
        cases.append(dict(values=x, group=group, iterations=4, sample_vectors=256, init=init))
    # occupancy patterns with exact duplicates (tests/test_fit_codebook_keeps_every_entry.py:43-48)
    atoms = np.random.default_rng(1).standard_normal((16, 16))
    for counts in ([64] * 16, [120] * 8 + [8] * 8,
                   [max(1, int(512 * 0.55 ** i)) for i in range(16)], [900] + [4] * 15):
        sample = np.repeat(atoms, counts, axis=0).astype(np.float32)
        cases.append(dict(values=sample.reshape(-1), group=16, iterations=4,
                          sample_vectors=4096, init=None))
    cases.append(dict(values=np.ones(512 * 16, dtype=np.float32), group=16, iterations=4,
                      sample_vectors=4096, init=None))
    # warm start whose whole-tensor pass keeps an entry the sample misses
    atoms8, index = review_shape(8, rare_at=1)
    cases.append(dict(values=atoms8[index].reshape(-1), group=8, iterations=4,
                      sample_vectors=4096, init=atoms8))
    # warm start from a zero book (a fresh optimizer's moments)
    cases.append(dict(values=(rng.standard_normal(5000 * 8) * 1e-3).astype(np.float32),
                      group=8, iterations=4, sample_vectors=4096,
                      init=np.zeros((16, 8), dtype=np.float32)))
    out = {}
    stored = []
    for i, c in enumerate(cases):
        book = ref_vq.fit_codebook(c["values"], group=c["group"], iterations=c["iterations"],
                                   sample_vectors=c["sample_vectors"], init=c["init"])
        # inputs shared between cases are stored once; c{i}_values_ref names the copy
        same = [j for j, v in stored if v is c["values"]]
        if same:
            out[f"c{i}_values_ref"] = np.array(same[0])
        else:
            out[f"c{i}_values"] = c["values"]
            stored.append((i, c["values"]))
        out[f"c{i}_group"] = np.array(c["group"])
        out[f"c{i}_iterations"] = np.array(c["iterations"])
        out[f"c{i}_sample_vectors"] = np.array(c["sample_vectors"])
        out[f"c{i}_init"] = (np.zeros((0,), np.float32) if c["init"] is None
                             else np.asarray(c["init"], np.float32))
        out[f"c{i}_book"] = book
    out["count"] = np.array(len(cases))
    return out


def config1() -> dict:
    """benchmark config 1: 256x256 N(0,1) seed 0, group 16, fit -> encode; x
    1x256 N(0,1) seed 1 fitted and encoded."""
    w = np.random.default_rng(0).standard_normal((256, 256)).astype(np.float32)
    book = ref_vq.fit_codebook(w, group=16)
    img = ref_vq.encode(w, book, group=16)
    x = np.random.default_rng(1).standard_normal((1, 256)).astype(np.float32)
    x_img = ref_vq.encode(x, ref_vq.fit_codebook(x, group=16), group=16)
    return {"w": w, "w_image": np.frombuffer(img.to_bytes(), dtype=np.uint8),
            "x": x, "x_image": np.frombuffer(x_img.to_bytes(), dtype=np.uint8),
            "w_decoded": img.decode(), "x_decoded": x_img.decode()}


def expert_payloads() -> dict:
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        bank = ref_bank.ExpertBank.create(
            Path(tmp) / "c2", ref_bank.BankConfig(1, 1, ((128, 128),) * 3, 16))
        bank.initialize_expert(0, 0, seed=7)
        for i, t in enumerate(bank.read_expert_state(0, 0).tensors):
            out[f"c2_{i}_codes"], out[f"c2_{i}_book"] = t.codes, t.codebook
        bank = ref_bank.ExpertBank.create(
            Path(tmp) / "h", ref_bank.BankConfig(1, 1, ((4, 3), (4, 3), (4, 3)), 8))
        bank.initialize_expert(0, 0, seed=4, zero_optimizer_state=True)
        for i, t in enumerate(bank.read_expert_state(0, 0).tensors):
            out[f"h_{i}_codes"], out[f"h_{i}_book"] = t.codes, t.codebook
    return out


class _Float32Backend:
    """A host backend whose AdamW is vq4.comp's arithmetic in numpy float32
    (every operation rounded, in the shader's order) and whose encode is the
    reference's CPU encode. Used to record VQAdamW.step end to end."""

    def encode(self, values, codebook, *, group):
        return ref_vq.encode(values, codebook, group=group)

    def decode(self, value):
        return value.decode()

    def adamw(self, weight, momentum, variance, gradient, *, lr, beta1, beta2, eps,
              weight_decay, step):
        f = np.float32
        c = np.array([lr, beta1, beta2, eps, weight_decay, 1 - beta1 ** step,
                      1 - beta2 ** step], dtype=np.float32)
        w, m, v, g = (s.decode() for s in (weight, momentum, variance, gradient))
        nm = c[1] * m + (f(1) - c[1]) * g
        nv = c[2] * v + (f(1) - c[2]) * (g * g)
        cm, cv = nm / c[5], nv / c[6]
        den = np.sqrt(cv) + c[3]
        nw = w * (f(1) - c[0] * c[4]) - c[0] * cm / den
        return nw.astype(np.float32), nm.astype(np.float32), nv.astype(np.float32)


def vqadamw_steps() -> dict:
    rng = np.random.default_rng(11)
    out = {}
    for i, (shape, group) in enumerate((((64, 48), 16), ((40, 40), 8), ((3000, 32), 32))):
        w = (rng.standard_normal(shape) * 0.05).astype(np.float32)
        weight = ref_vq.encode(w, ref_vq.fit_codebook(w, group=group), group=group)
        opt = ref_vq.VQAdamW(_Float32Backend(), weight, lr=1e-3, betas=(0.9, 0.999),
                             eps=1e-8, weight_decay=0.01)
        out[f"s{i}_group"] = np.array(group)
        out[f"s{i}_shape"] = np.array(shape)
        out[f"s{i}_w0_codes"], out[f"s{i}_w0_book"] = weight.codes, weight.codebook
        for step in range(2):
            g = (rng.standard_normal(shape) * 1e-2).astype(np.float32)
            g_img = ref_vq.encode(g, ref_vq.fit_codebook(g, group=group), group=group)
            out[f"s{i}_g{step}_codes"], out[f"s{i}_g{step}_book"] = g_img.codes, g_img.codebook
            report = opt.step(g_img)
            out[f"s{i}_changed{step}"] = np.array(report["changed_weight_values"])
            for name, state in (("w", opt.weight), ("m", opt.momentum), ("v", opt.variance)):
                out[f"s{i}_{name}{step + 1}_codes"] = state.codes
                out[f"s{i}_{name}{step + 1}_book"] = state.codebook
    return out


def bank_files() -> dict:
    """Every file of a small bank the reference writes: create, three seeded
    experts (one with zeroed optimizer state), then two committed updates of
    expert (0, 1) carrying other experts' payloads. Generation ids are random
    (uuid4), so the history of expert (0, 1)'s generations is recorded too."""
    with tempfile.TemporaryDirectory() as tmp:
        root = Path(tmp) / "bank"
        config = ref_bank.BankConfig(2, 2, ((10, 13), (13, 10), (10, 13)), 8)
        bank = ref_bank.ExpertBank.create(root, config)
        history = []

        def generation():
            text = (root / "expert-0-1.json").read_text()
            return text.split('"generation":"')[1].split('"')[0]

        bank.initialize_expert(0, 1, seed=3)
        history.append(generation())
        bank.initialize_expert(1, 0, seed=5, zero_optimizer_state=True)
        bank.initialize_expert(1, 1, seed=9)
        bank.write_expert(0, 1, bank.read_expert(1, 0), updated_count=100, optimizer_step=1)
        history.append(generation())
        bank.write_expert(0, 1, bank.read_expert(1, 1), updated_count=17, optimizer_step=4)
        history.append(generation())
        stats = ref_bank._json(bank.stats())
        names = sorted(p.name for p in root.iterdir())
        blobs = [(root / n).read_bytes() for n in names]
    offsets = np.cumsum([0] + [len(b) for b in blobs]).astype(np.int64)
    return {"names": np.array(names), "offsets": offsets,
            "blob": np.frombuffer(b"".join(blobs), dtype=np.uint8),
            "history_0_1": np.array(history),
            "stats": np.frombuffer(stats, dtype=np.uint8)}


def bank_scale() -> dict:
    """A bank of full-size experts (three 4096x4096 group-16 matrices): two
    seeded experts (one with zeroed optimizer state) and a committed update of
    expert (0, 0) carrying expert (0, 1)'s payload. There are nine 525 KB shards,
    so the fixture keeps each file's name, size and SHA-256, and the pointer
    and bank JSON texts in full (generation ids as recorded)."""
    import hashlib
    with tempfile.TemporaryDirectory() as tmp:
        root = Path(tmp) / "bank"
        config = ref_bank.BankConfig(1, 2, ((4096, 4096),) * 3, 16)
        bank = ref_bank.ExpertBank.create(root, config)
        history = []

        def generation():
            text = (root / "expert-0-0.json").read_text()
            return text.split('"generation":"')[1].split('"')[0]

        bank.initialize_expert(0, 0, seed=11)
        history.append(generation())
        bank.initialize_expert(0, 1, seed=12, zero_optimizer_state=True)
        bank.write_expert(0, 0, bank.read_expert(0, 1), updated_count=4096, optimizer_step=2)
        history.append(generation())
        stats = ref_bank._json(bank.stats())
        names = sorted(p.name for p in root.iterdir())
        sizes = [(root / n).stat().st_size for n in names]
        digests = [hashlib.sha256((root / n).read_bytes()).hexdigest() for n in names]
        texts = {n: (root / n).read_bytes() for n in names if n.endswith(".json")}
    text_names = sorted(texts)
    offsets = np.cumsum([0] + [len(texts[n]) for n in text_names]).astype(np.int64)
    return {"names": np.array(names), "sizes": np.array(sizes, np.int64),
            "sha256": np.array(digests), "json_names": np.array(text_names),
            "json_offsets": offsets,
            "json_blob": np.frombuffer(b"".join(texts[n] for n in text_names), dtype=np.uint8),
            "history_0_0": np.array(history),
            "stats": np.frombuffer(stats, dtype=np.uint8)}


class _ClipRecorder:
    """A host backend for the reference harness that keeps the dense gradient
    it returns from the transposed product. The harness scales that array in
    place by its clip factor (harness.py:196-200) before encoding it, so after
    ``train_step`` the kept array holds the clipped gradient exactly as the
    reference computed it; a copy taken before returning holds the unclipped
    one."""

    def __init__(self):
        self.before = None
        self.after = None

    def encode(self, values, codebook, *, group):
        return ref_vq.encode(values, codebook, group=group)

    def decode(self, value):
        return value.decode()

    def matmul(self, left, right, *, transpose_a=False, transpose_b=False):
        a, b = left.decode(), right.decode()
        out = ((a.T if transpose_a else a) @ (b.T if transpose_b else b)).astype(np.float32)
        if transpose_a:
            self.before, self.after = out.copy(), out
        return out

    def adamw(self, weight, momentum, variance, gradient, *, lr, beta1, beta2, eps,
              weight_decay, step):
        return _Float32Backend().adamw(weight, momentum, variance, gradient, lr=lr, beta1=beta1,
                                       beta2=beta2, eps=eps, weight_decay=weight_decay, step=step)


def clip_cases() -> dict:
    """The reference harness's clip on real steps: per case the unclipped
    gradient, the clipped one, the norm it reported and whether it clipped."""
    rng = np.random.default_rng(77)
    out = {}
    cases = [((4, 3), 8, 2, 0.01), ((4, 3), 8, 2, 1e6), ((64, 48), 16, 32, 1.0),
             ((64, 48), 16, 32, 0.05), ((40, 40), 8, 5, 3.0)]
    with tempfile.TemporaryDirectory() as tmp:
        for i, (shape, group, rows, max_norm) in enumerate(cases):
            bank = ref_bank.ExpertBank.create(Path(tmp) / f"b{i}",
                                              ref_bank.BankConfig(1, 1, (shape,) * 3, group))
            bank.initialize_expert(0, 0, seed=i, zero_optimizer_state=True)
            rec = _ClipRecorder()
            runner = ref_harness.VulkanExpertHarness(bank, backend=rec)
            x = rng.standard_normal((rows, shape[0])).astype(np.float32)
            y = rng.standard_normal((rows, shape[1])).astype(np.float32)
            step = runner.train_step(x, y, max_grad_norm=max_norm)
            out[f"c{i}_max_norm"] = np.array(max_norm, np.float64)
            out[f"c{i}_before"], out[f"c{i}_after"] = rec.before, rec.after
            out[f"c{i}_norm"] = np.array(step.gradient_norm_before_clip, np.float64)
            out[f"c{i}_clipped"] = np.array(step.clipped)
    out["count"] = np.array(len(cases))
    return out


FIXTURES = {
    "encode_cpu": encode_cases,
    "fit_codebook": fit_cases,
    "config1": config1,
    "expert_payloads": expert_payloads,
    "vqadamw_steps": vqadamw_steps,
    "bank_files": bank_files,
    "bank_scale": bank_scale,
    "clip_scale": clip_cases,
}


def main(argv=None) -> int:
    names = list(sys.argv[1:] if argv is None else argv) or list(FIXTURES)
    for name in names:
        np.savez_compressed(OUT / f"{name}.npz", **FIXTURES[name]())
        print(f"{name}.npz", (OUT / f"{name}.npz").stat().st_size)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
