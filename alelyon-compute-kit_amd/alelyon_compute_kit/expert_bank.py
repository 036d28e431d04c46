"""Durable storage of vq4 expert matrices: the bank the harness trains through.

A bank is a directory. ``bank.json`` fixes its shape (layers, experts per
layer, the matrices of one expert, the group). Each materialized expert has a
pointer ``expert-L-E.json`` naming its current generation; a generation is
one ``.vq`` shard per matrix, each the ``VQArray`` wire image, checked by
length and sha256. A write lays down the new shards and a pending pointer,
then publishes the pointer with one atomic rename, so readers see either the
old generation or the new one.

The on-disk format -- file names, the canonical JSON (sorted keys, compact
separators, no NaN), the pointer fields and the counters -- is the
reference's (src/alelyon_compute_kit/_kit/python/expert_bank.py:29-355), so
banks written here and there are interchangeable. The deterministic payload
generator of ``initialize_expert`` follows expert_bank.py:357-390: it defines
BASELINE config 2's inputs.

Single trusted writer, concurrent readers. Hashes detect changed bytes; they
authenticate nothing.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import re
import stat
import time
import uuid
from dataclasses import dataclass
from pathlib import Path
from typing import Sequence

import numpy as np

from .vq import ENTRIES, GROUPS, VQArray, storage_layout

MAX_SHARD_BYTES = 128 * 1024 * 1024
MAX_METADATA_BYTES = 128 * 1024
SCHEMA = "ack-expert-bank/v1"
# A rename over a pointer another process holds open can be refused
# transiently (the reference retries Windows' sharing violation,
# expert_bank.py:31-37); retry for about a second, then refuse the commit.
_RENAME_TRIES = 50
_RENAME_PAUSE_S = 0.02
_POINTER_NAME = re.compile(r"expert-([0-9]+)-([0-9]+)\.json\Z")
_SHA256_HEX = re.compile(r"[0-9a-f]{64}\Z")
_GENERATION_HEX = re.compile(r"[0-9a-f]{32}\Z")
_POINTER_FIELDS = frozenset({"schema", "config_sha256", "layer", "expert", "generation",
                             "revision", "shards", "parameter_update_applications",
                             "update_commits", "optimizer_step"})


class ExpertBankError(ValueError):
    """A bank, payload, declaration or boundary is not admissible."""


def _int(value, name: str, low: int = 0, high: int = (1 << 63) - 1) -> int:
    # bool is an int subclass; it is refused like any other non-int
    if type(value) is not int or value < low or value > high:
        raise ExpertBankError(f"{name} must be an integer in {low}..{high}")
    return value


def _require_fields(value, fields, what: str) -> None:
    if not isinstance(value, dict) or set(value) != set(fields):
        raise ExpertBankError(f"invalid {what} fields")


def canonical_json(value) -> bytes:
    """The bank's byte form of a JSON value: sorted keys, no spaces, UTF-8."""
    return json.dumps(value, sort_keys=True, separators=(",", ":"),
                      allow_nan=False).encode("utf-8")


def _no_duplicates(pairs):
    out = {}
    for key, item in pairs:
        if key in out:
            raise ExpertBankError("duplicate metadata key")
        out[key] = item
    return out


def _refuse_constant(name):
    raise ExpertBankError("nonfinite metadata")


def _load_canonical(data: bytes):
    """Parse metadata and insist it is already in canonical form."""
    try:
        value = json.loads(data, object_pairs_hook=_no_duplicates,
                           parse_constant=_refuse_constant)
        again = canonical_json(value)
    except ExpertBankError:
        raise
    except (UnicodeError, json.JSONDecodeError, RecursionError) as exc:
        raise ExpertBankError("invalid bank metadata") from exc
    except ValueError as exc:
        raise ExpertBankError(str(exc)) from exc
    if again != data:
        raise ExpertBankError("noncanonical bank metadata")
    return value


def _sha256(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


@dataclass(frozen=True)
class BankConfig:
    """Shape of a bank: ``layers`` x ``experts_per_layer`` experts, each made of
    the 2-D ``matrix_shapes`` (1..16 of them), all coded at ``group``."""

    layers: int
    experts_per_layer: int
    matrix_shapes: tuple[tuple[int, int], ...]
    group: int = 16

    def __post_init__(self):
        _int(self.layers, "layers", 1, 1_000_000)
        _int(self.experts_per_layer, "experts_per_layer", 1, 1_000_000)
        if type(self.group) is not int or self.group not in GROUPS:
            raise ExpertBankError("group must be 8, 16 or 32")
        shapes = self.matrix_shapes
        if not isinstance(shapes, (tuple, list)) or not 1 <= len(shapes) <= 16:
            raise ExpertBankError("matrix_shapes must contain 1..16 matrices")
        checked = []
        for shape in shapes:
            if not isinstance(shape, (tuple, list)) or len(shape) != 2:
                raise ExpertBankError("each matrix must have two dimensions")
            dims = tuple(_int(d, "matrix dimension", 1) for d in shape)
            try:
                layout = storage_layout(dims, self.group)
            except ValueError as exc:
                raise ExpertBankError(str(exc)) from exc
            if layout["serialized_bytes"] > MAX_SHARD_BYTES:
                raise ExpertBankError("matrix exceeds shard byte limit")
            checked.append(dims)
        object.__setattr__(self, "matrix_shapes", tuple(checked))
        _int(self.potential_parameters, "potential_parameters")

    @property
    def parameters_per_expert(self) -> int:
        return sum(rows * cols for rows, cols in self.matrix_shapes)

    @property
    def potential_parameters(self) -> int:
        return self.layers * self.experts_per_layer * self.parameters_per_expert

    def to_dict(self) -> dict:
        return {"layers": self.layers, "experts_per_layer": self.experts_per_layer,
                "matrix_shapes": [list(s) for s in self.matrix_shapes], "group": self.group}

    @classmethod
    def from_dict(cls, value) -> "BankConfig":
        _require_fields(value, ("layers", "experts_per_layer", "matrix_shapes", "group"),
                        "config")
        return cls(**value)


@dataclass(frozen=True)
class ExpertState:
    """One pointer snapshot: the tensors and the optimizer bookkeeping."""

    tensors: tuple[VQArray, ...]
    optimizer_step: int
    revision: int
    parameter_update_applications: int


def _read_regular(path: Path, limit: int) -> bytes:
    """Read a regular, non-symlinked file of at most ``limit`` bytes."""
    info = path.lstat()
    if not stat.S_ISREG(info.st_mode) or info.st_size > limit:
        raise ExpertBankError("file is not regular or exceeds byte limit")
    with path.open("rb") as stream:
        data = stream.read(limit + 1)
    if len(data) != info.st_size:
        raise ExpertBankError("file changed size or exceeds byte limit")
    return data


def _create_durable(path: Path, data: bytes) -> None:
    """Create ``path`` (never overwrite) and flush it to stable storage."""
    with path.open("xb") as stream:
        stream.write(data)
        stream.flush()
        os.fsync(stream.fileno())


class ExpertBank:
    """A fixed bank; ``create`` and ``open`` never materialize experts."""

    def __init__(self, root: Path, config: BankConfig, config_hash: str):
        self.root = root
        self.config = config
        self._config_hash = config_hash

    # -- bank lifecycle ------------------------------------------------------
    @classmethod
    def create(cls, root, config: BankConfig) -> "ExpertBank":
        if not isinstance(config, BankConfig):
            raise ExpertBankError("config must be BankConfig")
        path = Path(root)
        path.mkdir(parents=False, exist_ok=False)  # a fresh directory only
        if path.is_symlink():
            raise ExpertBankError("bank root must not be a symlink")
        path = path.resolve(strict=True)
        data = canonical_json({"schema": SCHEMA, "config": config.to_dict()})
        _create_durable(path / "bank.json", data)
        return cls(path, config, _sha256(data))

    @classmethod
    def open(cls, root) -> "ExpertBank":
        path = Path(root)
        if path.is_symlink() or not path.is_dir():
            raise ExpertBankError("bank root must be a regular directory")
        path = path.resolve(strict=True)
        data = _read_regular(path / "bank.json", MAX_METADATA_BYTES)
        value = _load_canonical(data)
        _require_fields(value, ("schema", "config"), "bank")
        if value["schema"] != SCHEMA:
            raise ExpertBankError("unsupported bank schema")
        return cls(path, BankConfig.from_dict(value["config"]), _sha256(data))

    def _verify_config(self) -> None:
        if (self.root.is_symlink() or not self.root.is_dir()
                or _sha256(_read_regular(self.root / "bank.json", MAX_METADATA_BYTES))
                != self._config_hash):
            raise ExpertBankError("bank configuration changed")

    # -- names -----------------------------------------------------------------
    def _base(self, layer: int, expert: int) -> str:
        _int(layer, "layer", 0, self.config.layers - 1)
        _int(expert, "expert", 0, self.config.experts_per_layer - 1)
        return f"expert-{layer}-{expert}"

    def _shard_path(self, base: str, generation: str, index: int) -> Path:
        return self.root / f"{base}-g{generation}-t{index}.vq"

    # -- pointers --------------------------------------------------------------
    def _load_pointer(self, layer: int, expert: int):
        """The committed pointer of an expert (validated), or None."""
        path = self.root / f"{self._base(layer, expert)}.json"
        try:
            data = _read_regular(path, MAX_METADATA_BYTES)
        except FileNotFoundError:
            return None
        p = _load_canonical(data)
        _require_fields(p, _POINTER_FIELDS, "expert")
        same_identity = (
            p["schema"] == SCHEMA and p["config_sha256"] == self._config_hash
            and type(p["layer"]) is int and p["layer"] == layer
            and type(p["expert"]) is int and p["expert"] == expert
            and isinstance(p["generation"], str) and _GENERATION_HEX.fullmatch(p["generation"]))
        if not same_identity:
            raise ExpertBankError("expert identity mismatch")
        _int(p["revision"], "revision", 1)
        _int(p["optimizer_step"], "optimizer_step", 0, 1 << 53)
        applications = _int(p["parameter_update_applications"], "parameter_update_applications")
        commits = _int(p["update_commits"], "update_commits", 0, p["revision"])
        # every update commit applies at least one and at most one expert's
        # worth of parameter updates
        if ((applications == 0) != (commits == 0) or applications < commits
                or applications > commits * self.config.parameters_per_expert):
            raise ExpertBankError("inconsistent update counters")
        shards = p["shards"]
        if not isinstance(shards, list) or len(shards) != len(self.config.matrix_shapes):
            raise ExpertBankError("expert shard count mismatch")
        for shard, shape in zip(shards, self.config.matrix_shapes):
            _require_fields(shard, ("bytes", "sha256"), "shard")
            _int(shard["bytes"], "shard bytes", 1, MAX_SHARD_BYTES)
            expected = storage_layout(shape, self.config.group)["serialized_bytes"]
            if (shard["bytes"] != expected or not isinstance(shard["sha256"], str)
                    or not _SHA256_HEX.fullmatch(shard["sha256"])):
                raise ExpertBankError("shard identity or layout mismatch")
        return p

    def _load_generation(self, pointer: dict, *, keep: bool = True) -> tuple[VQArray, ...]:
        base = self._base(pointer["layer"], pointer["expert"])
        arrays = []
        for index, (shard, shape) in enumerate(zip(pointer["shards"], self.config.matrix_shapes)):
            path = self._shard_path(base, pointer["generation"], index)
            try:
                data = _read_regular(path, MAX_SHARD_BYTES)
            except FileNotFoundError as exc:
                raise ExpertBankError(
                    f"missing shard {path.name} of a committed generation") from exc
            if len(data) != shard["bytes"] or _sha256(data) != shard["sha256"]:
                raise ExpertBankError("shard checksum mismatch")
            try:
                array = VQArray.from_bytes(data, max_bytes=MAX_SHARD_BYTES)
            except ValueError as exc:
                raise ExpertBankError(f"invalid VQ shard: {exc}") from exc
            if array.shape != shape or array.group != self.config.group:
                raise ExpertBankError("decoded shard geometry mismatch")
            if keep:
                arrays.append(array)
        return tuple(arrays)

    # -- reads -----------------------------------------------------------------
    def read_expert(self, layer: int, expert: int) -> tuple[VQArray, ...]:
        return self.read_expert_state(layer, expert).tensors

    def read_expert_state(self, layer: int, expert: int) -> ExpertState:
        """Tensors and optimizer bookkeeping of one pointer snapshot."""
        self._verify_config()
        pointer = self._load_pointer(layer, expert)
        if pointer is None:
            raise ExpertBankError("expert is not materialized")
        return ExpertState(self._load_generation(pointer), pointer["optimizer_step"],
                           pointer["revision"], pointer["parameter_update_applications"])

    # -- writes ----------------------------------------------------------------
    def write_expert(self, layer: int, expert: int, tensors: Sequence[VQArray], *,
                     updated_count: int = 0, optimizer_step: int | None = None) -> dict:
        """Commit a new generation of one expert; returns the receipt.

        A refused write removes every file it created and leaves the previous
        generation current.
        """
        self._verify_config()
        base = self._base(layer, expert)
        _int(updated_count, "updated_count", 0, self.config.parameters_per_expert)
        if optimizer_step is not None:
            _int(optimizer_step, "optimizer_step", 0, 1 << 53)
        shapes = self.config.matrix_shapes
        if not isinstance(tensors, (tuple, list)) or len(tensors) != len(shapes):
            raise ExpertBankError("one VQArray per configured matrix is required")
        for array, shape in zip(tensors, shapes):
            if (not isinstance(array, VQArray) or array.shape != shape
                    or array.group != self.config.group):
                raise ExpertBankError("VQArray geometry mismatch")
            if array.layout["serialized_bytes"] > MAX_SHARD_BYTES:
                raise ExpertBankError("shard byte limit exceeded")
        before = self._load_pointer(layer, expert)
        prior_step = 0 if before is None else before["optimizer_step"]
        step = prior_step if optimizer_step is None else optimizer_step
        if step < prior_step:
            raise ExpertBankError("optimizer_step must not regress")
        if before is not None:
            self._load_generation(before, keep=False)  # never build on corrupt state
        generation = uuid.uuid4().hex
        pointer = {
            "schema": SCHEMA, "config_sha256": self._config_hash,
            "layer": layer, "expert": expert, "generation": generation,
            "optimizer_step": step,
            "revision": 1 if before is None else before["revision"] + 1,
            "shards": [],
            "parameter_update_applications":
                updated_count + (0 if before is None else before["parameter_update_applications"]),
            "update_commits":
                (1 if updated_count > 0 else 0) + (0 if before is None else before["update_commits"]),
        }
        _int(pointer["parameter_update_applications"], "parameter_update_applications")
        pending = self.root / f"pending-{generation}.json"
        created: list[Path] = []
        try:
            for index, array in enumerate(tensors):
                image = array.to_bytes()
                # the exposed arrays are read-only, but a caller can still
                # have changed them: write only an image that parses back
                VQArray.from_bytes(image, max_bytes=MAX_SHARD_BYTES)
                shard = self._shard_path(base, generation, index)
                _create_durable(shard, image)
                created.append(shard)
                pointer["shards"].append({"bytes": len(image), "sha256": _sha256(image)})
            _create_durable(pending, canonical_json(pointer))
            created.append(pending)
            self._verify_config()
            if self._load_pointer(layer, expert) != before:
                raise ExpertBankError("another writer changed this expert")
            self._publish(pending, self.root / f"{base}.json")
        except BaseException:
            for path in created:
                try:
                    path.unlink()
                except FileNotFoundError:
                    pass
            raise
        return {"layer": layer, "expert": expert, "revision": pointer["revision"],
                "optimizer_step": step,
                "materialized_parameters": self.config.parameters_per_expert,
                "updated_count": updated_count,
                "parameter_update_applications": pointer["parameter_update_applications"],
                "generation_bytes": sum(s["bytes"] for s in pointer["shards"])}

    @staticmethod
    def _publish(pending: Path, target: Path) -> None:
        for attempt in range(_RENAME_TRIES):
            try:
                os.replace(pending, target)
                return
            except PermissionError as exc:
                if attempt + 1 == _RENAME_TRIES:
                    raise ExpertBankError(
                        "pointer replacement refused; a reader may hold the pointer open") from exc
                time.sleep(_RENAME_PAUSE_S)

    def initialize_expert(self, layer: int, expert: int, *, seed: int = 0,
                          zero_optimizer_state: bool = False) -> dict:
        """Materialize deterministic payloads (expert_bank.py:357-390).

        Matrix i draws from ``default_rng(SeedSequence([seed, layer, expert,
        i]))``: uniform u32 code words (nibbles past the last vector zeroed),
        then a standard-normal 16 x group book scaled by 1/sqrt(rows). With
        ``zero_optimizer_state`` matrices 1 and 2 (momentum and variance) are
        all-zero images instead.
        """
        self._verify_config()
        self._base(layer, expert)
        _int(seed, "seed", 0, (1 << 64) - 1)
        if not isinstance(zero_optimizer_state, bool):
            raise ExpertBankError("zero_optimizer_state must be bool")
        if zero_optimizer_state and len(self.config.matrix_shapes) < 3:
            raise ExpertBankError("zero optimizer state needs three matrix roles")
        if self._load_pointer(layer, expert) is not None:
            raise ExpertBankError("expert is already materialized")
        group = self.config.group
        arrays = []
        for index, shape in enumerate(self.config.matrix_shapes):
            layout = storage_layout(shape, group)
            words = layout["code_bytes"] // 4
            if zero_optimizer_state and index in (1, 2):
                codes = np.zeros(words, dtype=np.uint32)
                book = np.zeros((ENTRIES, group), dtype=np.float32)
            else:
                rng = np.random.default_rng(np.random.SeedSequence([seed, layer, expert, index]))
                codes = rng.integers(0, 1 << 32, words, dtype=np.uint32)
                live = layout["vectors"] % 8
                if live:
                    codes[-1] &= np.uint32((1 << (4 * live)) - 1)
                book = rng.standard_normal((ENTRIES, group), dtype=np.float32)
                book *= np.float32(1.0 / math.sqrt(shape[0]))
            arrays.append(VQArray(shape, group, codes, book))
        return self.write_expert(layer, expert, arrays)

    def stats(self) -> dict:
        """Validate every committed generation and census the directory.

        ``disk_bytes`` is the sum of file lengths (history and interrupted
        writes included), not allocated blocks; update applications are the
        writers' declared cumulative counts.
        """
        self._verify_config()
        materialized = applications = updated = committed = disk = 0
        for path in self.root.iterdir():
            info = path.lstat()
            if not stat.S_ISREG(info.st_mode):
                raise ExpertBankError("unexpected nonregular bank entry")
            disk += info.st_size
            match = _POINTER_NAME.fullmatch(path.name)
            if match is None:
                continue
            layer, expert = int(match.group(1)), int(match.group(2))
            if path.name != f"{self._base(layer, expert)}.json":
                raise ExpertBankError("noncanonical expert filename")
            pointer = self._load_pointer(layer, expert)
            if pointer is None:
                raise ExpertBankError("expert pointer disappeared")
            self._load_generation(pointer, keep=False)
            materialized += 1
            applications += pointer["parameter_update_applications"]
            updated += 1 if pointer["update_commits"] > 0 else 0
            committed += sum(s["bytes"] for s in pointer["shards"])
        return {"potential_experts": self.config.layers * self.config.experts_per_layer,
                "potential_parameters": self.config.potential_parameters,
                "materialized_experts": materialized,
                "materialized_parameters": materialized * self.config.parameters_per_expert,
                "updated_experts": updated,
                "parameter_update_applications": applications,
                "unique_updated_parameters": None,
                "committed_payload_bytes": committed, "disk_bytes": disk}
