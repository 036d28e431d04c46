"""Linear-expert driver of the vq4 path: forward and one clipped MSE update.

The caller hands one expert's activations (and, to train, targets) as finite
float32 rank-2 arrays; weight, momentum and variance live in an
``ExpertBank``. Activations are vq4-coded with a codebook fitted on the CPU,
the packed products and the optimizer step run on the GPU through
``VQDevice``, and a successful step is committed to the bank atomically.

Semantics follow src/alelyon_compute_kit/harness.py:89-248 of the reference:
the same encode-then-multiply forward (:140-160), the same MSE gradient
``x^T (2/N) (x W - t)`` through the packed product with A transposed
(:186-195), the same global L2 clip ``scale = min(1, max_norm / (||g|| +
1e-6))`` in float64 (:196-200), the same ``VQAdamW`` warm start from the
bank's moments and step (:203-213), and the same commit (:217-223). Only the
device differs; the reference's class name is kept as an alias so callers
that import ``VulkanExpertHarness`` keep working.

Diagnostic reductions (loss, gradient norm) are host float64 work here as
there. With ``resident=True`` the expert's weight, momentum and variance stay
on the device between steps (in the fused optimizer step's input layout),
codebooks are fitted on the device (the same books as the host fit), and only
activation-sized arrays and the reductions' inputs cross the bus; a step
commits the same images as the default path, byte for byte.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import tempfile
import time
from contextlib import ExitStack
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import ack, expert_bank, vq


class HarnessError(ValueError):
    """The supplied model state, arrays or job boundary is not admissible."""


@dataclass(frozen=True)
class ExpertStep:
    """What one committed expert update did."""

    layer: int
    expert: int
    optimizer_step: int
    revision: int
    loss: float
    gradient_norm_before_clip: float
    clipped: bool
    elapsed_seconds: float
    persistent_state_bytes: int
    input_layout: dict
    activation_layout: dict
    gradient_layout: dict

    def to_dict(self) -> dict:
        return {name: getattr(self, name) for name in (
            "layer", "expert", "optimizer_step", "revision", "loss",
            "gradient_norm_before_clip", "clipped", "elapsed_seconds",
            "persistent_state_bytes", "input_layout", "activation_layout", "gradient_layout")}


def _matrix(value, name: str) -> np.ndarray:
    array = np.asarray(value)
    if array.dtype != np.dtype("float32") or array.ndim != 2:
        raise HarnessError(f"{name} must be a rank-2 float32 array")
    if array.size == 0 or not np.isfinite(array).all():
        raise HarnessError(f"{name} must be nonempty and finite")
    return np.ascontiguousarray(array)


def _positive(value, name: str) -> float:
    if isinstance(value, (bool, np.bool_)):
        raise HarnessError(f"{name} must be finite and positive")
    try:
        number = float(value)
    except (TypeError, ValueError) as exc:
        raise HarnessError(f"{name} must be finite and positive") from exc
    if not (math.isfinite(number) and number > 0):
        raise HarnessError(f"{name} must be finite and positive")
    return number


class _ResidentExpert:
    """One expert's weight, momentum and variance on the device, laid out as
    the fused optimizer step reads them: the codes of W, M, V and a gradient
    slot back to back, then their four books. ``images`` are the host images
    the buffers hold."""

    def __init__(self, device: ack.Device, images):
        w = images[0]
        self.words = w.layout["code_bytes"] // 4
        self.book = vq.ENTRIES * w.group
        self.codes4 = device.buffer(4 * self.words * 4)
        try:
            self.books4 = device.buffer(4 * self.book * 4)
        except BaseException:
            self.codes4.free()
            raise
        self.load(images)

    def load(self, images) -> None:
        codes = np.zeros(4 * self.words, np.uint32)
        books = np.zeros(4 * self.book, np.float32)
        for i, t in enumerate(images[:3]):
            codes[i * self.words:(i + 1) * self.words] = t.codes
            books[i * self.book:(i + 1) * self.book] = t.codebook.reshape(-1)
        self.codes4.upload(codes)
        self.books4.upload(books)
        self.images = tuple(images[:3])

    def holds(self, images) -> bool:
        return len(images) >= 3 and all(a == b for a, b in zip(self.images, images[:3]))

    def free(self) -> None:
        self.codes4.free()
        self.books4.free()


class ExpertHarness:
    """One durable linear expert driven through the vq4 kernels.

    ``backend`` may be any object with the ``VQDevice`` methods (host-only
    tests inject fakes). Without one, the harness opens an ``ack.Device``
    itself -- importing this module opens nothing. ``resident=True`` (a
    ``VQDevice`` backend only) keeps each expert's optimizer state on the
    device between steps and fits codebooks there.
    """

    def __init__(self, bank: expert_bank.ExpertBank, *, backend=None, device=None,
                 resident: bool = False):
        if not isinstance(bank, expert_bank.ExpertBank):
            raise HarnessError("bank must be an ExpertBank")
        if backend is not None and device is not None:
            raise HarnessError("supply backend or device, not both")
        if not isinstance(resident, bool):
            raise HarnessError("resident must be a bool")
        self.bank = bank
        self._device = device
        self._owns_device = False
        if backend is None:
            if device is None:
                self._device = ack.Device()
                self._owns_device = True
            backend = vq.VQDevice(self._device)
        if resident and not isinstance(backend, vq.VQDevice):
            raise HarnessError("a resident harness needs a VQDevice backend")
        self.backend = backend
        self.resident = resident
        self._residents: dict[tuple[int, int], _ResidentExpert] = {}

    @classmethod
    def open(cls, root, *, device=None, backend=None, resident=False) -> "ExpertHarness":
        """Open an existing bank; creates and initializes nothing."""
        return cls(expert_bank.ExpertBank.open(root), backend=backend, device=device,
                   resident=resident)

    def __enter__(self) -> "ExpertHarness":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def close(self) -> None:
        for res in self._residents.values():
            res.free()
        self._residents.clear()
        if self._owns_device and self._device is not None:
            self._device.close()
            self._device = None

    # -- pieces ----------------------------------------------------------------
    def _state(self, layer: int, expert: int) -> expert_bank.ExpertState:
        try:
            state = self.bank.read_expert_state(layer, expert)
        except expert_bank.ExpertBankError as exc:
            raise HarnessError(str(exc)) from exc
        if len(state.tensors) < 3:
            raise HarnessError("expert state must contain weight, momentum and variance")
        w, m, v = state.tensors[:3]
        if not (w.shape == m.shape == v.shape and w.group == m.group == v.group):
            raise HarnessError("expert optimizer state geometry disagrees")
        return state

    def _encode(self, values: np.ndarray, group: int) -> vq.VQArray:
        # Calibration needs one whole vector: a batch smaller than a group is
        # zero-padded for the fit only; the image keeps the exact geometry.
        sample = values
        if values.size < group:
            sample = np.pad(values.reshape(-1), (0, group - values.size))
        return self.backend.encode(values, vq.fit_codebook(sample, group=group), group=group)

    # -- the resident path ---------------------------------------------------------
    def _resident_for(self, layer: int, expert: int, state) -> _ResidentExpert:
        res = self._residents.get((layer, expert))
        if res is not None and res.holds(state.tensors):
            return res
        if res is not None:            # the bank moved on under us: reload
            res.load(state.tensors)
            return res
        res = _ResidentExpert(self.backend.device, state.tensors)
        self._residents[(layer, expert)] = res
        return res

    def _device_image(self, values: np.ndarray, group: int, buf, status, on_device=None):
        """fit_codebook and encode on the device: the image ``_encode`` makes
        (the same tiny-batch padding for the fit), left in device buffers.
        ``on_device``, a buffer already holding ``values`` as float32, saves
        the upload (tensors of at least one vector need no padding)."""
        flat = values.reshape(-1)
        if on_device is not None and flat.size >= group:
            vals, size = on_device, flat.size
        else:
            sample = flat if flat.size >= group else np.pad(flat, (0, group - flat.size))
            sample = np.ascontiguousarray(sample, dtype=np.float32)
            vals, size = buf(sample.nbytes), sample.size
            vals.upload(sample)
        book = buf(vq.ENTRIES * group * 4)
        self.backend.fit_resident(vals, size, book, status, group=group)
        codes = buf(vq.storage_layout(values.shape, group)["code_bytes"])
        self.backend.run((0, flat.size, 1, 1, group, vq.ENTRIES, 0, 0), [vals, book], codes,
                         status)
        return codes, book

    @staticmethod
    def _checked(status) -> None:
        flags = int(status.download(np.uint32)[0])
        if flags:
            raise HarnessError(f"expert device arithmetic refused: status={flags}")

    def _forward_resident(self, x: np.ndarray, weight, res: _ResidentExpert) -> np.ndarray:
        device, group = self.backend.device, weight.group
        m, k = x.shape
        n = weight.shape[1]
        with ExitStack() as cleanup:
            def buf(nbytes):
                b = device.buffer(nbytes)
                cleanup.callback(b.free)
                return b
            status = buf(4)
            status.upload(np.zeros(1, np.uint32))
            xc, xb = self._device_image(x, group, buf, status)
            y = buf(m * n * 4)
            self.backend.run((2, m, n, k, group, vq.ENTRIES, 0, 0),
                             [xc, xb, res.codes4, res.books4], y, status)
            self._checked(status)
            return y.download(np.float32).reshape(m, n)

    def _step_resident(self, x, target, state, res: _ResidentExpert, lr, beta1, beta2, eps,
                       weight_decay, max_grad_norm):
        """The train_step flow below on resident state; returns (loss, norm,
        scale, new images, report bytes, input/activation/gradient layouts)."""
        device = self.backend.device
        weight = state.tensors[0]
        group = weight.group
        m, k = x.shape
        n = weight.shape[1]
        with ExitStack() as cleanup:
            def buf(nbytes):
                b = device.buffer(nbytes)
                cleanup.callback(b.free)
                return b
            status = buf(4)
            status.upload(np.zeros(1, np.uint32))
            xc, xb = self._device_image(x, group, buf, status)
            tc, tb = self._device_image(target, group, buf, status)
            y, t_dec = buf(m * n * 4), buf(m * n * 4)
            self.backend.run((2, m, n, k, group, vq.ENTRIES, 0, 0),
                             [xc, xb, res.codes4, res.books4], y, status)
            self.backend.run((1, m * n, 1, 1, group, vq.ENTRIES, 0, 0), [tc, tb], t_dec, status)
            self._checked(status)
            residual = y.download(np.float32).reshape(m, n) - \
                t_dec.download(np.float32).reshape(m, n)
            loss = float(np.mean(np.square(residual, dtype=np.float64)))
            if not math.isfinite(loss):
                raise HarnessError("expert loss is nonfinite")
            residual *= np.float32(2.0 / residual.size)
            rc, rb = self._device_image(residual, group, buf, status)
            grad = buf(k * n * 4)
            self.backend.run((2, k, n, m, group, vq.ENTRIES, 1, 0), [xc, xb, rc, rb], grad,
                             status)
            self._checked(status)
            gradient = grad.download(np.float32).reshape(k, n)
            norm = float(np.linalg.norm(gradient.astype(np.float64)))
            if not math.isfinite(norm):
                raise HarnessError("expert gradient norm is nonfinite")
            scale = min(1.0, max_grad_norm / (norm + 1e-6))
            gradient *= np.float32(scale)
            # unclipped, the device copy is already the gradient to encode
            gc, gb = self._device_image(gradient, group, buf, status,
                                        on_device=grad if scale == 1.0 else None)
            res.codes4.copy_from(gc, res.words * 4, offset=3 * res.words * 4)
            res.books4.copy_from(gb, res.book * 4, offset=3 * res.book * 4)
            try:
                coeff = vq.VQDevice.adamw_coefficients(lr, beta1, beta2, eps, weight_decay,
                                                       state.optimizer_step + 1)
            except ValueError as exc:
                raise HarnessError(f"expert optimizer refused the update: {exc}") from exc
            cb = buf(coeff.nbytes)
            cb.upload(coeff)
            out_codes, out_books = buf(3 * res.words * 4), buf(3 * res.book * 4)
            changed = buf(4)
            self.backend.adamw_step_resident(res.codes4, res.books4, cb, out_codes, out_books,
                                             changed, status,
                                             count=weight.layout["elements"], group=group)
            self._checked(status)
            codes = out_codes.download(np.uint32).reshape(3, res.words)
            books = out_books.download(np.float32).reshape(3, vq.ENTRIES, group)
            images = tuple(vq.VQArray(weight.shape, group, codes[i], books[i]) for i in range(3))
            res.codes4.copy_from(out_codes, 3 * res.words * 4)
            res.books4.copy_from(out_books, 3 * res.book * 4)
            res.images = images
        layouts = tuple(vq.storage_layout(a.shape, group) for a in (x, target, gradient))
        return loss, norm, scale, images, layouts

    # -- the driver surface ------------------------------------------------------
    def forward(self, inputs, *, layer: int = 0, expert: int = 0) -> np.ndarray:
        """``inputs @ weight`` through the packed product."""
        x = _matrix(inputs, "inputs")
        state = self._state(layer, expert)
        weight = state.tensors[0]
        if x.shape[1] != weight.shape[0]:
            raise HarnessError(f"inputs have width {x.shape[1]}, expert expects {weight.shape[0]}")
        if self.resident:
            return self._forward_resident(x, weight, self._resident_for(layer, expert, state))
        return self.backend.matmul(self._encode(x, weight.group), weight)

    def forward_batch(self, inputs, experts) -> np.ndarray:
        """``inputs[i] @ weight(experts[i])`` for several experts of the bank at
        once (``experts`` are (layer, expert) pairs; every input has the same
        shape). On a ``VQDevice`` backend the products run as one batched
        launch over the packed weights (``ack_vq_batch``); each result equals
        ``forward`` of that input within FP32 rounding (the kernel may split
        the sums differently for a batch than for one product)."""
        pairs = [tuple(int(v) for v in e) for e in experts]
        xs = [_matrix(v, "inputs") for v in inputs]
        if not pairs or len(xs) != len(pairs):
            raise HarnessError("one input matrix per expert is required")
        if any(x.shape != xs[0].shape for x in xs):
            raise HarnessError("batched inputs must share one shape")
        weights = [self._state(layer, expert).tensors[0] for layer, expert in pairs]
        if xs[0].shape[1] != weights[0].shape[0]:
            raise HarnessError(f"inputs have width {xs[0].shape[1]}, "
                               f"expert expects {weights[0].shape[0]}")
        group = weights[0].group
        if any(w.shape != weights[0].shape or w.group != group for w in weights):
            raise HarnessError("batched experts must share one weight shape and group")
        images = [self._encode(x, group) for x in xs]
        if isinstance(self.backend, vq.VQDevice):
            return self.backend.matmul_batch(images, weights)
        return np.stack([self.backend.matmul(a, w) for a, w in zip(images, weights)])

    def train_step(self, inputs, targets, *, layer: int = 0, expert: int = 0,
                   lr: float = 1e-3, beta1: float = 0.9, beta2: float = 0.95,
                   eps: float = 1e-8, weight_decay: float = 0.0,
                   max_grad_norm: float = 1.0) -> ExpertStep:
        """One MSE update of the expert, committed atomically to the bank."""
        x, target = _matrix(inputs, "inputs"), _matrix(targets, "targets")
        if x.shape[0] != target.shape[0]:
            raise HarnessError("inputs and targets must have the same row count")
        state = self._state(layer, expert)
        weight, momentum, variance = state.tensors[:3]
        if x.shape[1] != weight.shape[0] or target.shape[1] != weight.shape[1]:
            raise HarnessError("inputs/targets do not match expert matrix geometry")
        max_grad_norm = _positive(max_grad_norm, "max_grad_norm")
        group = weight.group
        t0 = time.perf_counter()
        if self.resident:
            res = self._resident_for(layer, expert, state)
            try:
                loss, norm, scale, images, layouts = self._step_resident(
                    x, target, state, res, lr, beta1, beta2, eps, weight_decay, max_grad_norm)
            except (ValueError, ack.AckError) as exc:
                # a failed step leaves the device copy unknown: reload next time
                self._residents.pop((layer, expert)).free()
                if isinstance(exc, HarnessError):
                    raise
                raise HarnessError(f"expert step failed on the device: {exc}") from exc
            return self._commit(layer, expert, weight, images, state.optimizer_step + 1, loss,
                                norm, scale, t0, layouts)
        x_img = self._encode(x, group)
        t_img = self._encode(target, group)
        residual = self.backend.matmul(x_img, weight) - self.backend.decode(t_img)
        loss = float(np.mean(np.square(residual, dtype=np.float64)))
        if not math.isfinite(loss):
            raise HarnessError("expert loss is nonfinite")
        residual *= np.float32(2.0 / residual.size)          # d(mean square)/d(prediction)
        r_img = self._encode(residual, group)
        gradient = self.backend.matmul(x_img, r_img, transpose_a=True)
        norm = float(np.linalg.norm(gradient.astype(np.float64)))
        if not math.isfinite(norm):
            raise HarnessError("expert gradient norm is nonfinite")
        scale = min(1.0, max_grad_norm / (norm + 1e-6))
        gradient *= np.float32(scale)
        g_img = self._encode(gradient, group)
        try:
            opt = vq.VQAdamW(self.backend, weight, lr=lr, betas=(beta1, beta2), eps=eps,
                             weight_decay=weight_decay)
            opt.momentum, opt.variance = momentum, variance
            opt.steps = state.optimizer_step
            update = opt.step(g_img)
        except (TypeError, ValueError, ack.AckError) as exc:
            raise HarnessError(f"expert optimizer refused the update: {exc}") from exc
        return self._commit(layer, expert, weight, (opt.weight, opt.momentum, opt.variance),
                            opt.steps, loss, norm, scale, t0,
                            (x_img.layout, t_img.layout, g_img.layout),
                            update["persistent_state_bytes"])

    def _commit(self, layer, expert, weight, images, optimizer_step, loss, norm, scale, t0,
                layouts, state_bytes=None) -> ExpertStep:
        try:
            receipt = self.bank.write_expert(layer, expert, images,
                                             updated_count=weight.layout["elements"],
                                             optimizer_step=optimizer_step)
        except expert_bank.ExpertBankError as exc:
            raise HarnessError(f"expert update was not committed: {exc}") from exc
        elapsed = time.perf_counter() - t0
        if not (math.isfinite(elapsed) and elapsed > 0):
            raise HarnessError("expert step elapsed time is invalid")
        if state_bytes is None:
            state_bytes = sum(a.layout["serialized_bytes"] for a in images)
        return ExpertStep(layer=layer, expert=expert, optimizer_step=optimizer_step,
                          revision=receipt["revision"], loss=loss,
                          gradient_norm_before_clip=norm, clipped=scale < 1.0,
                          elapsed_seconds=elapsed, persistent_state_bytes=state_bytes,
                          input_layout=layouts[0], activation_layout=layouts[1],
                          gradient_layout=layouts[2])

    def train(self, inputs, targets, *, steps: int = 1, **kwargs) -> tuple[ExpertStep, ...]:
        """Bounded sequential steps, each committed before the next."""
        if type(steps) is not int or not 1 <= steps <= 1_000_000:
            raise HarnessError("steps must be an integer in 1..1000000")
        return tuple(self.train_step(inputs, targets, **kwargs) for _ in range(steps))


# The reference's name for this class (harness.py:89); the device is HIP here.
VulkanExpertHarness = ExpertHarness


def _load_matrix(path: Path, name: str) -> np.ndarray:
    if path.is_symlink() or not path.is_file():
        raise HarnessError(f"{name} must be a regular file")
    try:
        value = np.load(path, allow_pickle=False)
    except (OSError, ValueError) as exc:
        raise HarnessError(f"{name} is not a readable NumPy array") from exc
    if not isinstance(value, np.ndarray):
        raise HarnessError(f"{name} must be a single .npy array, not an archive")
    return _matrix(value, name)


def _save_matrix(path: Path, value: np.ndarray, *, force: bool) -> None:
    if path.exists() and not force:
        raise HarnessError(f"refusing to overwrite existing output: {path}")
    path.parent.mkdir(parents=True, exist_ok=True)
    fd, name = tempfile.mkstemp(prefix=f".{path.name}.", suffix=".tmp", dir=path.parent)
    os.close(fd)
    scratch = Path(name)
    try:
        with scratch.open("wb") as stream:
            np.save(stream, value, allow_pickle=False)
            stream.flush()
            os.fsync(stream.fileno())
        os.replace(scratch, path)
    finally:
        scratch.unlink(missing_ok=True)


def main(argv=None) -> int:
    """``python -m alelyon_compute_kit.harness --device --bank B --input X --output Y
    [--target T --steps N]`` (the reference's CLI, harness.py:280-315)."""
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--bank", type=Path, required=True)
    parser.add_argument("--input", type=Path, required=True)
    parser.add_argument("--output", type=Path, required=True)
    parser.add_argument("--target", type=Path)
    parser.add_argument("--layer", type=int, default=0)
    parser.add_argument("--expert", type=int, default=0)
    parser.add_argument("--steps", type=int, default=1)
    parser.add_argument("--lr", type=float, default=1e-3)
    parser.add_argument("--max-grad-norm", type=float, default=1.0)
    parser.add_argument("--device", action="store_true", help="explicitly open the GPU")
    parser.add_argument("--resident", action="store_true",
                        help="keep the optimizer state on the device between steps")
    parser.add_argument("--force", action="store_true")
    args = parser.parse_args(argv)
    if not args.device:
        parser.error("--device is required; execution is never implicit")
    inputs = _load_matrix(args.input, "input")
    with ExpertHarness.open(args.bank, resident=args.resident) as harness:
        if args.target is None:
            result = harness.forward(inputs, layer=args.layer, expert=args.expert)
            report = {"mode": "forward", "shape": list(result.shape)}
        else:
            targets = _load_matrix(args.target, "target")
            steps = harness.train(inputs, targets, steps=args.steps, layer=args.layer,
                                  expert=args.expert, lr=args.lr,
                                  max_grad_norm=args.max_grad_norm)
            result = harness.forward(inputs, layer=args.layer, expert=args.expert)
            report = {"mode": "train", "steps": [s.to_dict() for s in steps]}
        _save_matrix(args.output, result, force=args.force)
        report["device"] = harness._device.capability_record()
        report["model_quality_validated"] = False
    print(json.dumps(report, sort_keys=True, allow_nan=False))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
