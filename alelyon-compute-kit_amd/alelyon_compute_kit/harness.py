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

Diagnostic reductions (loss, gradient norm) and codebook calibration are CPU
work here as there.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import tempfile
import time
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


class ExpertHarness:
    """One durable linear expert driven through the vq4 kernels.

    ``backend`` may be any object with the ``VQDevice`` methods (host-only
    tests inject fakes). Without one, the harness opens an ``ack.Device``
    itself -- importing this module opens nothing.
    """

    def __init__(self, bank: expert_bank.ExpertBank, *, backend=None, device=None):
        if not isinstance(bank, expert_bank.ExpertBank):
            raise HarnessError("bank must be an ExpertBank")
        if backend is not None and device is not None:
            raise HarnessError("supply backend or device, not both")
        self.bank = bank
        self._device = device
        self._owns_device = False
        if backend is None:
            if device is None:
                self._device = ack.Device()
                self._owns_device = True
            backend = vq.VQDevice(self._device)
        self.backend = backend

    @classmethod
    def open(cls, root, *, device=None, backend=None) -> "ExpertHarness":
        """Open an existing bank; creates and initializes nothing."""
        return cls(expert_bank.ExpertBank.open(root), backend=backend, device=device)

    def __enter__(self) -> "ExpertHarness":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def close(self) -> None:
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

    # -- the driver surface ------------------------------------------------------
    def forward(self, inputs, *, layer: int = 0, expert: int = 0) -> np.ndarray:
        """``inputs @ weight`` through the packed product."""
        x = _matrix(inputs, "inputs")
        weight = self._state(layer, expert).tensors[0]
        if x.shape[1] != weight.shape[0]:
            raise HarnessError(f"inputs have width {x.shape[1]}, expert expects {weight.shape[0]}")
        return self.backend.matmul(self._encode(x, weight.group), weight)

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
        try:
            receipt = self.bank.write_expert(
                layer, expert, (opt.weight, opt.momentum, opt.variance),
                updated_count=weight.layout["elements"], optimizer_step=opt.steps)
        except expert_bank.ExpertBankError as exc:
            raise HarnessError(f"expert update was not committed: {exc}") from exc
        elapsed = time.perf_counter() - t0
        if not (math.isfinite(elapsed) and elapsed > 0):
            raise HarnessError("expert step elapsed time is invalid")
        return ExpertStep(layer=layer, expert=expert, optimizer_step=opt.steps,
                          revision=receipt["revision"], loss=loss,
                          gradient_norm_before_clip=norm, clipped=scale < 1.0,
                          elapsed_seconds=elapsed,
                          persistent_state_bytes=update["persistent_state_bytes"],
                          input_layout=x_img.layout, activation_layout=t_img.layout,
                          gradient_layout=g_img.layout)

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
    parser.add_argument("--force", action="store_true")
    args = parser.parse_args(argv)
    if not args.device:
        parser.error("--device is required; execution is never implicit")
    inputs = _load_matrix(args.input, "input")
    with ExpertHarness.open(args.bank) as harness:
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
