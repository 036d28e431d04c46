"""Linear-expert driver of the vq4 path: forward and one clipped MSE update.

A caller hands one expert's activations (and, to train, targets) as finite
float32 rank-2 arrays; the expert's weight, momentum and variance live in an
``ExpertBank``. Activations are vq4-coded with a freshly fitted codebook, the
packed products and the optimizer step run on the GPU through ``VQDevice``,
and a successful step is committed to the bank atomically.

The arithmetic of a step is the reference's
(src/alelyon_compute_kit/harness.py:140-223), since its committed bytes are
observable: encode-then-multiply forward; the MSE gradient
``x^T (2/N)(x W - t)`` through the packed product with A transposed; the
global L2 clip ``min(1, max_norm / (||g|| + 1e-6))`` with the norm in
float64; ``VQAdamW`` continuing from the bank's moments and step; one commit
declaring every weight value updated. The reference's class name is kept as
an alias, so callers importing ``VulkanExpertHarness`` keep working.

With ``resident=True`` the expert's weight, momentum and variance stay on
the device between steps (in the fused optimizer step's input layout),
codebooks are fitted there (the same books as the host fit), and only
activation-sized arrays and the inputs of the host float64 reductions cross
the bus; a resident step commits the default path's images byte for byte.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import tempfile
import time
from contextlib import ExitStack
from dataclasses import dataclass, fields
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
        return {f.name: getattr(self, f.name) for f in fields(self)}


def _as_matrix(value, name: str) -> np.ndarray:
    """A nonempty, finite, rank-2 float32 array (C-contiguous)."""
    array = np.asarray(value)
    if array.dtype != np.float32 or array.ndim != 2:
        raise HarnessError(f"{name} must be a rank-2 float32 array")
    if not array.size or not np.isfinite(array).all():
        raise HarnessError(f"{name} must be nonempty and finite")
    return np.ascontiguousarray(array)


def _finite_positive(value, name: str) -> float:
    number = math.nan
    if not isinstance(value, (bool, np.bool_)):
        try:
            number = float(value)
        except (TypeError, ValueError):
            pass
    if not (math.isfinite(number) and number > 0):
        raise HarnessError(f"{name} must be finite and positive")
    return number


def _calibration_sample(values: np.ndarray, group: int) -> np.ndarray:
    """The values a codebook is fitted on: the fit needs one whole vector, so
    fewer values than a group are zero-padded (for the fit only; the image
    keeps the exact geometry)."""
    flat = values.reshape(-1)
    if flat.size >= group:
        return values
    return np.concatenate([flat, np.zeros(group - flat.size, dtype=flat.dtype)])


@dataclass
class _StepResult:
    """A step's outcome before its commit."""

    loss: float
    norm: float
    scale: float
    images: tuple          # new (weight, momentum, variance)
    layouts: tuple         # input, activation and gradient image layouts
    state_bytes: int | None = None


# ---- resident optimizer state ------------------------------------------------------
class _DeviceState:
    """One expert's weight, momentum and variance on the device, laid out as
    the fused optimizer step reads them: the codes of W, M, V and a gradient
    slot back to back in one buffer, their four books in another."""

    def __init__(self, device: ack.Device, images):
        first = images[0]
        self.words = first.layout["code_bytes"] // 4
        self.book = vq.ENTRIES * first.group
        self.pool: dict[str, ack.Buffer] = {}  # a step's buffers, kept for the next step
        with ExitStack() as undo:
            self.codes4 = device.buffer(16 * self.words)
            undo.callback(self.codes4.free)
            self.books4 = device.buffer(16 * self.book)
            undo.callback(self.books4.free)
            self.load(images)
            undo.pop_all()

    def load(self, images) -> None:
        """Upload the first three images, the gradient slot zeroed."""
        trio = tuple(images[:3])
        self.codes4.upload(np.concatenate([t.codes for t in trio] + [np.zeros(self.words,
                                                                             np.uint32)]))
        self.books4.upload(np.concatenate([t.codebook.reshape(-1) for t in trio]
                                          + [np.zeros(self.book, np.float32)]))
        self.images = trio

    def holds(self, images) -> bool:
        return len(images) >= 3 and all(a == b for a, b in zip(self.images, images[:3]))

    def scratch(self, device: ack.Device):
        """A buffer source for one step that reuses this state's buffers from
        step to step: slot ``key`` keeps its buffer while its size stays."""
        def get(nbytes: int, key: str) -> ack.Buffer:
            buf = self.pool.get(key)
            if buf is None or buf.nbytes != nbytes:
                if buf is not None:
                    buf.free()
                    del self.pool[key]
                buf = self.pool[key] = device.buffer(nbytes)
            return buf
        return get

    def free(self) -> None:
        self.codes4.free()
        self.books4.free()
        while self.pool:
            self.pool.popitem()[1].free()


class ExpertHarness:
    """One durable linear expert driven through the vq4 kernels.

    ``backend`` may be any object with ``VQDevice``'s methods (host-only
    tests inject fakes); without one the harness opens an ``ack.Device``
    itself. Importing this module opens nothing. ``resident=True`` (a
    ``VQDevice`` backend only) keeps each expert's optimizer state on the
    device between steps.
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
        self._own_device = backend is None and device is None
        if backend is None:
            self._device = device if device is not None else ack.Device()
            backend = vq.VQDevice(self._device)
        if resident and not isinstance(backend, vq.VQDevice):
            raise HarnessError("a resident harness needs a VQDevice backend")
        self.backend = backend
        self.resident = resident
        self._on_device: dict[tuple[int, int], _DeviceState] = {}

    @classmethod
    def open(cls, root, *, device=None, backend=None, resident=False) -> "ExpertHarness":
        """A harness over an existing bank; creates and initializes nothing."""
        return cls(expert_bank.ExpertBank.open(root), backend=backend, device=device,
                   resident=resident)

    def __enter__(self) -> "ExpertHarness":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def close(self) -> None:
        while self._on_device:
            self._on_device.popitem()[1].free()
        if self._own_device and self._device is not None:
            self._device.close()
            self._device = None

    # -- shared pieces -------------------------------------------------------------------
    def _expert(self, layer: int, expert: int) -> expert_bank.ExpertState:
        """The expert's committed state, with weight, momentum and variance of
        one geometry."""
        try:
            state = self.bank.read_expert_state(layer, expert)
        except expert_bank.ExpertBankError as exc:
            raise HarnessError(str(exc)) from exc
        if len(state.tensors) < 3:
            raise HarnessError("expert state must contain weight, momentum and variance")
        trio = state.tensors[:3]
        if len({(t.shape, t.group) for t in trio}) != 1:
            raise HarnessError("expert optimizer state geometry disagrees")
        return state

    def encode_activations(self, values: np.ndarray, group: int) -> vq.VQArray:
        """``values`` as a vq4 image with a codebook fitted on them (host fit,
        backend encode)."""
        book = vq.fit_codebook(_calibration_sample(values, group), group=group)
        return self.backend.encode(values, book, group=group)

    @staticmethod
    def _width(x: np.ndarray, weight) -> None:
        if x.shape[1] != weight.shape[0]:
            raise HarnessError(f"inputs have width {x.shape[1]}, expert expects {weight.shape[0]}")

    # -- forward -----------------------------------------------------------------------------
    def forward(self, inputs, *, layer: int = 0, expert: int = 0) -> np.ndarray:
        """``inputs @ weight`` through the packed product."""
        x = _as_matrix(inputs, "inputs")
        state = self._expert(layer, expert)
        weight = state.tensors[0]
        self._width(x, weight)
        if self.resident:
            return self._forward_on_device(x, weight, self._device_state(layer, expert, state))
        return self.backend.matmul(self.encode_activations(x, weight.group), weight)

    def forward_batch(self, inputs, experts) -> np.ndarray:
        """``inputs[i] @ weight(experts[i])`` for several experts of the bank
        at once (``experts`` are (layer, expert) pairs, every input of one
        shape). On a ``VQDevice`` backend the products run as one batched
        launch over the packed weights (``ack_vq_batch``); each result equals
        that input's ``forward`` within FP32 rounding (a batch may split the
        sums differently from one product)."""
        ids = [tuple(int(v) for v in pair) for pair in experts]
        xs = [_as_matrix(v, "inputs") for v in inputs]
        if not ids or len(xs) != len(ids):
            raise HarnessError("one input matrix per expert is required")
        if len({x.shape for x in xs}) != 1:
            raise HarnessError("batched inputs must share one shape")
        weights = [self._expert(layer, expert).tensors[0] for layer, expert in ids]
        self._width(xs[0], weights[0])
        if len({(w.shape, w.group) for w in weights}) != 1:
            raise HarnessError("batched experts must share one weight shape and group")
        images = [self.encode_activations(x, weights[0].group) for x in xs]
        if isinstance(self.backend, vq.VQDevice):
            return self.backend.matmul_batch(images, weights)
        return np.stack([self.backend.matmul(a, w) for a, w in zip(images, weights)])

    # -- one training step ---------------------------------------------------------------
    def train_step(self, inputs, targets, *, layer: int = 0, expert: int = 0,
                   lr: float = 1e-3, beta1: float = 0.9, beta2: float = 0.95,
                   eps: float = 1e-8, weight_decay: float = 0.0,
                   max_grad_norm: float = 1.0) -> ExpertStep:
        """One MSE update of the expert, committed atomically to the bank."""
        x, target = _as_matrix(inputs, "inputs"), _as_matrix(targets, "targets")
        if x.shape[0] != target.shape[0]:
            raise HarnessError("inputs and targets must have the same row count")
        state = self._expert(layer, expert)
        weight = state.tensors[0]
        if (x.shape[1], target.shape[1]) != weight.shape:
            raise HarnessError("inputs/targets do not match expert matrix geometry")
        max_grad_norm = _finite_positive(max_grad_norm, "max_grad_norm")
        hyper = {"lr": lr, "beta1": beta1, "beta2": beta2, "eps": eps,
                 "weight_decay": weight_decay}
        started = time.perf_counter()
        if self.resident:
            result = self._step_on_device(layer, expert, state, x, target, hyper, max_grad_norm)
        else:
            result = self._step(state, x, target, hyper, max_grad_norm)
        return self._commit(layer, expert, weight, state.optimizer_step + 1, result, started)

    def _step(self, state, x, target, hyper, max_grad_norm) -> _StepResult:
        weight, momentum, variance = state.tensors[:3]
        group = weight.group
        x_img = self.encode_activations(x, group)
        t_img = self.encode_activations(target, group)
        residual = self.backend.matmul(x_img, weight) - self.backend.decode(t_img)
        loss = _mse(residual)
        residual *= np.float32(2.0 / residual.size)        # d(mean square)/d(prediction)
        r_img = self.encode_activations(residual, group)
        gradient = self.backend.matmul(x_img, r_img, transpose_a=True)
        norm, scale = _clip_factor(gradient, max_grad_norm)
        gradient *= np.float32(scale)
        g_img = self.encode_activations(gradient, group)
        try:
            optimizer = vq.VQAdamW(self.backend, weight, lr=hyper["lr"],
                                   betas=(hyper["beta1"], hyper["beta2"]), eps=hyper["eps"],
                                   weight_decay=hyper["weight_decay"])
            optimizer.momentum, optimizer.variance = momentum, variance
            optimizer.steps = state.optimizer_step
            report = optimizer.step(g_img)
        except (TypeError, ValueError, ack.AckError) as exc:
            raise HarnessError(f"expert optimizer refused the update: {exc}") from exc
        return _StepResult(loss, norm, scale,
                           (optimizer.weight, optimizer.momentum, optimizer.variance),
                           (x_img.layout, t_img.layout, g_img.layout),
                           report["persistent_state_bytes"])

    def _commit(self, layer, expert, weight, optimizer_step, result: _StepResult,
                started: float) -> ExpertStep:
        try:
            receipt = self.bank.write_expert(layer, expert, result.images,
                                             updated_count=weight.layout["elements"],
                                             optimizer_step=optimizer_step)
        except expert_bank.ExpertBankError as exc:
            raise HarnessError(f"expert update was not committed: {exc}") from exc
        elapsed = time.perf_counter() - started
        if not (math.isfinite(elapsed) and elapsed > 0):
            raise HarnessError("expert step elapsed time is invalid")
        state_bytes = result.state_bytes
        if state_bytes is None:
            state_bytes = sum(t.layout["serialized_bytes"] for t in result.images)
        input_layout, activation_layout, gradient_layout = result.layouts
        return ExpertStep(layer=layer, expert=expert, optimizer_step=optimizer_step,
                          revision=receipt["revision"], loss=result.loss,
                          gradient_norm_before_clip=result.norm, clipped=result.scale < 1.0,
                          elapsed_seconds=elapsed, persistent_state_bytes=state_bytes,
                          input_layout=input_layout, activation_layout=activation_layout,
                          gradient_layout=gradient_layout)

    def train(self, inputs, targets, *, steps: int = 1, **kwargs) -> tuple[ExpertStep, ...]:
        """Bounded sequential steps, each committed before the next."""
        if type(steps) is not int or not 1 <= steps <= 1_000_000:
            raise HarnessError("steps must be an integer in 1..1000000")
        return tuple(self.train_step(inputs, targets, **kwargs) for _ in range(steps))

    # -- the resident path ----------------------------------------------------------------
    def _device_state(self, layer: int, expert: int, state) -> _DeviceState:
        """The expert's state on the device, reloaded when the bank moved on
        (another writer committed since this harness's last step)."""
        held = self._on_device.get((layer, expert))
        if held is None:
            held = self._on_device[(layer, expert)] = _DeviceState(self.backend.device,
                                                                   state.tensors)
        elif not held.holds(state.tensors):
            held.load(state.tensors)
        return held

    def _device_image(self, shape, group: int, scratch, status, name: str, values=None,
                      resident=None):
        """``encode_activations`` on the device: the codebook fitted and the
        values encoded there, left in device buffers. The values come from the
        host array ``values`` or, when ``resident`` (a buffer holding them as
        float32) is given and holds at least one vector, from the device."""
        count = int(np.prod(shape))
        if resident is not None and count >= group:
            source, fitted = resident, count
        else:  # the values, zero-padded to one vector for the fit if fewer
            sample = np.ascontiguousarray(_calibration_sample(values.reshape(-1), group),
                                          dtype=np.float32)
            source, fitted = scratch(sample.nbytes, name + ".values"), sample.size
            source.upload(sample)
        book = scratch(4 * vq.ENTRIES * group, name + ".book")
        self.backend.fit_resident(source, fitted, book, status, group=group)
        codes = scratch(vq.storage_layout(shape, group)["code_bytes"], name + ".codes")
        self.backend.run((0, count, 1, 1, group, vq.ENTRIES, 0, 0), [source, book], codes,
                         status)
        return codes, book

    @staticmethod
    def _settled(status) -> None:
        flags = int(status.download(np.uint32)[0])
        if flags:
            raise HarnessError(f"expert device arithmetic refused: status={flags}")

    def _scratch_space(self, stack: ExitStack):
        device = self.backend.device

        def scratch(nbytes: int, key: str = "") -> ack.Buffer:
            buf = device.buffer(nbytes)
            stack.callback(buf.free)
            return buf
        return scratch

    def _forward_on_device(self, x: np.ndarray, weight, held: _DeviceState) -> np.ndarray:
        (m, k), n, group = x.shape, weight.shape[1], weight.group
        with ExitStack() as stack:
            scratch = self._scratch_space(stack)
            status = scratch(4)
            status.upload(np.zeros(1, np.uint32))
            xc, xb = self._device_image(x.shape, group, scratch, status, "x", values=x)
            y = scratch(4 * m * n)
            self.backend.run((2, m, n, k, group, vq.ENTRIES, 0, 0),
                             [xc, xb, held.codes4, held.books4], y, status)
            self._settled(status)
            return y.download(np.float32).reshape(m, n)

    def _step_on_device(self, layer, expert, state, x, target, hyper,
                        max_grad_norm) -> _StepResult:
        held = self._device_state(layer, expert, state)
        try:
            return self._device_step(held, state, x, target, hyper, max_grad_norm)
        except (ValueError, ack.AckError) as exc:
            # a failed step leaves the device copy unknown: reload it next time
            self._on_device.pop((layer, expert)).free()
            if isinstance(exc, HarnessError):
                raise
            raise HarnessError(f"expert step failed on the device: {exc}") from exc

    def _device_step(self, held: _DeviceState, state, x, target, hyper,
                     max_grad_norm) -> _StepResult:
        """``_step`` on resident state: the same arithmetic in the same order,
        with fits and encodes on the device, the loss on the host and the
        gradient's norm from the device's float64 sum of squares whenever that
        certifies the clip numpy's norm would give (else the gradient comes to
        the host for numpy's norm). The step's buffers persist in ``held``."""
        weight = state.tensors[0]
        (m, k), n, group = x.shape, weight.shape[1], weight.group
        run = self.backend.run
        scratch = held.scratch(self.backend.device)
        status = scratch(4, "status")
        status.upload(np.zeros(1, np.uint32))
        xc, xb = self._device_image(x.shape, group, scratch, status, "x", values=x)
        tc, tb = self._device_image(target.shape, group, scratch, status, "t", values=target)
        prediction, decoded = scratch(4 * m * n, "prediction"), scratch(4 * m * n, "decoded")
        run((2, m, n, k, group, vq.ENTRIES, 0, 0), [xc, xb, held.codes4, held.books4],
            prediction, status)
        run((1, m * n, 1, 1, group, vq.ENTRIES, 0, 0), [tc, tb], decoded, status)
        self._settled(status)
        residual = prediction.download(np.float32).reshape(m, n) - \
            decoded.download(np.float32).reshape(m, n)
        loss = _mse(residual)
        residual *= np.float32(2.0 / residual.size)
        rc, rb = self._device_image(residual.shape, group, scratch, status, "r", values=residual)
        dense = scratch(4 * k * n, "gradient")
        run((2, k, n, m, group, vq.ENTRIES, 1, 0), [xc, xb, rc, rb], dense, status)
        total = scratch(8, "sum_squares")
        self.backend.sum_squares_resident(dense, k * n, total)
        self._settled(status)
        clip = _certified_clip(float(total.download(np.float64)[0]), k * n, max_grad_norm)
        if clip is None or k * n < group:
            # numpy's norm could round the scale (or the verdict) differently
            gradient = dense.download(np.float32).reshape(k, n)
            norm, scale = _clip_factor(gradient, max_grad_norm)
            gradient *= np.float32(scale)
            # unclipped, the device copy already holds the gradient to encode
            gc, gb = self._device_image((k, n), group, scratch, status, "g", values=gradient,
                                        resident=dense if scale == 1.0 else None)
        else:
            norm, scale = clip
            if scale != 1.0:
                self.backend.scale_resident(dense, k * n, np.float32(scale))
            gc, gb = self._device_image((k, n), group, scratch, status, "g", resident=dense)
        held.codes4.copy_from(gc, 4 * held.words, offset=12 * held.words)
        held.books4.copy_from(gb, 4 * held.book, offset=12 * held.book)
        try:
            block = vq.adamw_coefficients(hyper["lr"], hyper["beta1"], hyper["beta2"],
                                          hyper["eps"], hyper["weight_decay"],
                                          state.optimizer_step + 1)
        except ValueError as exc:
            raise HarnessError(f"expert optimizer refused the update: {exc}") from exc
        coefficients = scratch(block.nbytes, "coefficients")
        coefficients.upload(block)
        new_codes = scratch(12 * held.words, "new_codes")
        new_books = scratch(12 * held.book, "new_books")
        changed = scratch(4, "changed")
        self.backend.adamw_step_resident(held.codes4, held.books4, coefficients, new_codes,
                                         new_books, changed, status,
                                         count=weight.layout["elements"], group=group)
        self._settled(status)
        codes = new_codes.download(np.uint32).reshape(3, held.words)
        books = new_books.download(np.float32).reshape(3, vq.ENTRIES, group)
        images = tuple(vq.VQArray(weight.shape, group, c, b) for c, b in zip(codes, books))
        held.codes4.copy_from(new_codes, 12 * held.words)
        held.books4.copy_from(new_books, 12 * held.book)
        held.images = images
        layouts = tuple(vq.storage_layout(shape, group) for shape in (x.shape, target.shape, (k, n)))
        return _StepResult(loss, norm, scale, images, layouts)


def _mse(residual: np.ndarray) -> float:
    loss = float(np.mean(np.square(residual, dtype=np.float64)))
    if not math.isfinite(loss):
        raise HarnessError("expert loss is nonfinite")
    return loss


def _certified_clip(total: float, count: int, max_grad_norm: float):
    """(norm, scale) from a float64 sum of squares of ``count`` float32 values
    taken within (count / 65536 + 15)·2^-53 of the exact sum (the device's),
    when numpy's ``np.linalg.norm`` of the same values (a float64 dot product,
    within (count − 1)·2^-53 in any order) would lead to the same float32
    scale and the same clip verdict; None when it might not. The norm reported
    is this sum's; numpy's own differs from it in the last bits, as it does
    between BLAS builds and thread counts."""
    if not math.isfinite(total):
        raise HarnessError("expert gradient norm is nonfinite")
    slack = (count + count / 65536 + 64) * 2.0 ** -53 * 1.01

    def scale_of(sum_of_squares: float) -> float:
        return min(1.0, max_grad_norm / (math.sqrt(sum_of_squares) + 1e-6))

    # the scale falls as the sum rises: the two ends bracket numpy's
    high, low = scale_of(total * (1 - slack)), scale_of(total * (1 + slack))
    if np.float32(high) != np.float32(low) or (high < 1.0) != (low < 1.0):
        return None
    return math.sqrt(total), scale_of(total)


def _clip_factor(gradient: np.ndarray, max_grad_norm: float) -> tuple[float, float]:
    """(||g||_2 in float64, min(1, max_norm / (||g|| + 1e-6)))."""
    norm = float(np.linalg.norm(gradient.astype(np.float64)))
    if not math.isfinite(norm):
        raise HarnessError("expert gradient norm is nonfinite")
    return norm, min(1.0, max_grad_norm / (norm + 1e-6))


# The reference's name for this class (harness.py:89); the device is HIP here.
VulkanExpertHarness = ExpertHarness


# ---- command line -------------------------------------------------------------------------
_ZIP_MAGIC = b"PK\x03\x04"


def _read_matrix(path: Path, name: str) -> np.ndarray:
    """A single .npy array from a regular file, as a checked matrix."""
    if path.is_symlink() or not path.is_file():
        raise HarnessError(f"{name} must be a regular file")
    try:
        with path.open("rb") as stream:
            if stream.read(len(_ZIP_MAGIC)) == _ZIP_MAGIC:
                raise HarnessError(f"{name} must be a single .npy array, not an archive")
            stream.seek(0)
            array = np.lib.format.read_array(stream, allow_pickle=False)
    except (OSError, ValueError) as exc:
        if isinstance(exc, HarnessError):
            raise
        raise HarnessError(f"{name} is not a readable NumPy array") from exc
    return _as_matrix(array, name)


def _write_matrix(path: Path, value: np.ndarray, *, force: bool) -> None:
    """Write ``value`` as .npy through a temporary file renamed into place."""
    if path.exists() and not force:
        raise HarnessError(f"refusing to overwrite existing output: {path}")
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = tempfile.NamedTemporaryFile(dir=path.parent, prefix=f".{path.name}.",
                                            suffix=".tmp", delete=False)
    try:
        with temporary as stream:
            np.lib.format.write_array(stream, np.asarray(value), allow_pickle=False)
            stream.flush()
            os.fsync(stream.fileno())
        os.replace(temporary.name, path)
    finally:
        Path(temporary.name).unlink(missing_ok=True)


def main(argv=None) -> int:
    """``python -m alelyon_compute_kit.harness --device --bank B --input X
    --output Y [--target T ...]``: a forward, or ``--steps`` training steps
    and then a forward; prints a JSON report."""
    parser = argparse.ArgumentParser(description=__doc__)
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
                        help="keep the expert's optimizer state on the GPU between steps "
                             "(the same commits as without it)")
    parser.add_argument("--force", action="store_true")
    args = parser.parse_args(argv)
    if not args.device:
        parser.error("--device is required; execution is never implicit")
    inputs = _read_matrix(args.input, "input")
    where = {"layer": args.layer, "expert": args.expert}
    with ExpertHarness.open(args.bank, resident=args.resident) as runner:
        report = {"device": runner._device.capability_record(), "model_quality_validated": False}
        if args.target is not None:
            targets = _read_matrix(args.target, "target")
            steps = runner.train(inputs, targets, steps=args.steps, lr=args.lr,
                                 max_grad_norm=args.max_grad_norm, **where)
            report.update(mode="train", steps=[s.to_dict() for s in steps])
        result = runner.forward(inputs, **where)
        _write_matrix(args.output, result, force=args.force)
        if args.target is None:
            report.update(mode="forward", shape=list(result.shape))
    print(json.dumps(report, sort_keys=True, allow_nan=False))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
