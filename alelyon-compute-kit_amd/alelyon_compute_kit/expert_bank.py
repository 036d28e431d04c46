"""Durable storage of vq4 expert matrices: the bank the harness trains through.

A bank is one directory. ``bank.json`` fixes its shape: layers, experts per
layer, the matrices of one expert and their group. A materialized expert
has a pointer ``expert-L-E.json`` that names its current generation; a
generation is one ``.vq`` shard per matrix (the ``VQArray`` wire image),
each checked by length and sha256. A commit writes the new shards and a
pending pointer, then renames the pointer over the old one, so a reader sees
either the old generation or the new one, never a mixture.

The on-disk format -- file names, canonical JSON (sorted keys, compact
separators, no NaN), the pointer's fields and counters, the commit order --
is the reference's (src/alelyon_compute_kit/_kit/python/expert_bank.py:29-355),
so banks written here and there are interchangeable; so are the refusal
texts. ``initialize_expert``'s seeded payloads follow expert_bank.py:357-390
and define benchmark config 2's inputs.

One trusted writer, concurrent readers. Hashes detect changed bytes; they
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
from dataclasses import dataclass, replace
from pathlib import Path
from typing import Sequence

import numpy as np

from .vq import ENTRIES, GROUPS, VQArray, storage_layout

SCHEMA = "ack-expert-bank/v1"
MAX_SHARD_BYTES = 128 * 1024 * 1024
MAX_METADATA_BYTES = 128 * 1024
MAX_COUNT = (1 << 63) - 1
MAX_OPTIMIZER_STEP = 1 << 53
# A rename over a pointer that a reader holds open can be refused for a
# moment on some platforms (the reference retries Windows' sharing violation,
# expert_bank.py:31-37): about a second of retries, then the commit is refused.
PUBLISH_ATTEMPTS = 50
PUBLISH_PAUSE_S = 0.02

_POINTER_FILE = re.compile(r"expert-([0-9]+)-([0-9]+)\.json")
_HEX64 = re.compile(r"[0-9a-f]{64}")
_HEX32 = re.compile(r"[0-9a-f]{32}")
_POINTER_KEYS = frozenset(("schema", "config_sha256", "layer", "expert", "generation",
                           "revision", "shards", "parameter_update_applications",
                           "update_commits", "optimizer_step"))


class ExpertBankError(ValueError):
    """A bank, payload, declaration or boundary is not admissible."""


def _whole(value, name: str, low: int = 0, high: int = MAX_COUNT) -> int:
    """An exact int in low..high (bool, float and numpy ints are refused)."""
    if type(value) is int and low <= value <= high:
        return value
    raise ExpertBankError(f"{name} must be an integer in {low}..{high}")


def _fields(value, expected, what: str) -> dict:
    if isinstance(value, dict) and value.keys() == set(expected):
        return value
    raise ExpertBankError(f"invalid {what} fields")


def _sha256(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


# ---- canonical JSON --------------------------------------------------------------
def canonical_json(value) -> bytes:
    """The one byte form of a metadata value: UTF-8, keys sorted, no spaces,
    no NaN or infinity."""
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False)
    return text.encode("utf-8")


def _unique_object(pairs):
    keys = [key for key, _ in pairs]
    if len(set(keys)) != len(keys):
        raise ExpertBankError("duplicate metadata key")
    return dict(pairs)


def _no_constants(_name):
    raise ExpertBankError("nonfinite metadata")


_STRICT_DECODER = json.JSONDecoder(object_pairs_hook=_unique_object, parse_constant=_no_constants)


def _from_canonical(data: bytes):
    """Parse metadata that must already be in canonical form."""
    try:
        value = _STRICT_DECODER.decode(data.decode("utf-8"))
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


# ---- configuration -----------------------------------------------------------------
@dataclass(frozen=True)
class BankConfig:
    """The fixed shape of a bank: ``layers`` x ``experts_per_layer`` experts,
    each a sequence of 1..16 matrices of ``matrix_shapes`` at ``group``."""

    layers: int
    experts_per_layer: int
    matrix_shapes: tuple[tuple[int, int], ...]
    group: int = 16

    def __post_init__(self):
        _whole(self.layers, "layers", 1, 1_000_000)
        _whole(self.experts_per_layer, "experts_per_layer", 1, 1_000_000)
        if type(self.group) is not int or self.group not in GROUPS:
            raise ExpertBankError("group must be 8, 16 or 32")
        shapes = self.matrix_shapes
        if not isinstance(shapes, (tuple, list)) or not 1 <= len(shapes) <= 16:
            raise ExpertBankError("matrix_shapes must contain 1..16 matrices")
        checked = []
        for shape in shapes:
            if not isinstance(shape, (tuple, list)) or len(shape) != 2:
                raise ExpertBankError("each matrix must have two dimensions")
            dims = tuple(_whole(d, "matrix dimension", 1) for d in shape)
            try:
                image_bytes = storage_layout(dims, self.group)["serialized_bytes"]
            except ValueError as exc:
                raise ExpertBankError(str(exc)) from exc
            if image_bytes > MAX_SHARD_BYTES:
                raise ExpertBankError("matrix exceeds shard byte limit")
            checked.append(dims)
        object.__setattr__(self, "matrix_shapes", tuple(checked))
        _whole(self.potential_parameters, "potential_parameters")

    @property
    def parameters_per_expert(self) -> int:
        return sum(rows * cols for rows, cols in self.matrix_shapes)

    @property
    def potential_parameters(self) -> int:
        return self.layers * self.experts_per_layer * self.parameters_per_expert

    def shard_bytes(self) -> tuple[int, ...]:
        """The image size of each matrix: what every shard must measure."""
        return tuple(storage_layout(s, self.group)["serialized_bytes"] for s in self.matrix_shapes)

    def to_dict(self) -> dict:
        return {"layers": self.layers, "experts_per_layer": self.experts_per_layer,
                "matrix_shapes": [list(s) for s in self.matrix_shapes], "group": self.group}

    @classmethod
    def from_dict(cls, value) -> "BankConfig":
        fields = _fields(value, ("layers", "experts_per_layer", "matrix_shapes", "group"), "config")
        return cls(**fields)


@dataclass(frozen=True)
class ExpertState:
    """One pointer snapshot: the tensors and the optimizer bookkeeping."""

    tensors: tuple[VQArray, ...]
    optimizer_step: int
    revision: int
    parameter_update_applications: int


# ---- the directory -------------------------------------------------------------------
class _Directory:
    """Checked file operations under the bank's root."""

    def __init__(self, root: Path):
        self.root = root

    def read(self, name: str, limit: int) -> bytes:
        """A regular, non-symlinked file of at most ``limit`` bytes, read in
        full; FileNotFoundError when absent."""
        path = self.root / name
        info = path.lstat()
        if not stat.S_ISREG(info.st_mode) or info.st_size > limit:
            raise ExpertBankError("file is not regular or exceeds byte limit")
        with path.open("rb") as stream:
            data = stream.read(limit + 1)
        if len(data) != info.st_size:
            raise ExpertBankError("file changed size or exceeds byte limit")
        return data

    def create(self, name: str, data: bytes) -> None:
        """A new file (never an overwrite), flushed to stable storage."""
        with (self.root / name).open("xb") as stream:
            stream.write(data)
            stream.flush()
            os.fsync(stream.fileno())

    def publish(self, source: str, target: str) -> None:
        """Atomically rename ``source`` over ``target``, retrying a transient
        refusal."""
        for attempt in range(PUBLISH_ATTEMPTS):
            try:
                os.replace(self.root / source, self.root / target)
                return
            except PermissionError as exc:
                if attempt == PUBLISH_ATTEMPTS - 1:
                    raise ExpertBankError("pointer replacement refused; a reader may hold "
                                          "the pointer open") from exc
                time.sleep(PUBLISH_PAUSE_S)

    def discard(self, names) -> None:
        for name in names:
            (self.root / name).unlink(missing_ok=True)


# ---- the pointer ----------------------------------------------------------------------
@dataclass(frozen=True)
class _Pointer:
    """An expert's committed generation and its counters (the pointer file)."""

    layer: int
    expert: int
    generation: str
    revision: int
    optimizer_step: int
    applications: int          # parameter_update_applications
    commits: int               # update_commits
    shards: tuple[tuple[int, str], ...]   # (bytes, sha256) per matrix

    @property
    def base(self) -> str:
        return f"expert-{self.layer}-{self.expert}"

    def shard_file(self, index: int) -> str:
        return f"{self.base}-g{self.generation}-t{index}.vq"

    def to_json(self, config_sha256: str) -> bytes:
        return canonical_json({
            "schema": SCHEMA, "config_sha256": config_sha256, "layer": self.layer,
            "expert": self.expert, "generation": self.generation,
            "optimizer_step": self.optimizer_step, "revision": self.revision,
            "shards": [{"bytes": size, "sha256": digest} for size, digest in self.shards],
            "parameter_update_applications": self.applications,
            "update_commits": self.commits})

    @classmethod
    def parse(cls, data: bytes, layer: int, expert: int, config: BankConfig,
              config_sha256: str) -> "_Pointer":
        """Validate a pointer file against the bank and the expert it must name."""
        value = _fields(_from_canonical(data), _POINTER_KEYS, "expert")
        generation = value["generation"]
        identity = (value["schema"] == SCHEMA and value["config_sha256"] == config_sha256
                    and type(value["layer"]) is int and value["layer"] == layer
                    and type(value["expert"]) is int and value["expert"] == expert
                    and isinstance(generation, str) and _HEX32.fullmatch(generation))
        if not identity:
            raise ExpertBankError("expert identity mismatch")
        revision = _whole(value["revision"], "revision", 1)
        step = _whole(value["optimizer_step"], "optimizer_step", 0, MAX_OPTIMIZER_STEP)
        applications = _whole(value["parameter_update_applications"],
                              "parameter_update_applications")
        commits = _whole(value["update_commits"], "update_commits", 0, revision)
        # applications and commits are zero together; each commit declares at
        # least one and at most one expert's worth of updated values
        if (applications == 0) != (commits == 0) or not \
                commits <= applications <= commits * config.parameters_per_expert:
            raise ExpertBankError("inconsistent update counters")
        records = value["shards"]
        expected = config.shard_bytes()
        if not isinstance(records, list) or len(records) != len(expected):
            raise ExpertBankError("expert shard count mismatch")
        shards = []
        for record, size in zip(records, expected):
            record = _fields(record, ("bytes", "sha256"), "shard")
            length = _whole(record["bytes"], "shard bytes", 1, MAX_SHARD_BYTES)
            digest = record["sha256"]
            if length != size or not isinstance(digest, str) or not _HEX64.fullmatch(digest):
                raise ExpertBankError("shard identity or layout mismatch")
            shards.append((length, digest))
        return cls(layer, expert, generation, revision, step, applications, commits, tuple(shards))


# ---- the bank --------------------------------------------------------------------------
class ExpertBank:
    """A fixed logical bank of vq4 experts; ``create`` and ``open`` never
    materialize an expert's payloads."""

    def __init__(self, root: Path, config: BankConfig, config_hash: str):
        self.root = Path(root)
        self.config = config
        self._config_hash = config_hash
        self._dir = _Directory(self.root)

    # -- lifetime ------------------------------------------------------------------------
    @classmethod
    def create(cls, root, config: BankConfig) -> "ExpertBank":
        """A new bank in a directory that must not exist yet."""
        if not isinstance(config, BankConfig):
            raise ExpertBankError("config must be BankConfig")
        path = Path(root)
        path.mkdir(parents=False, exist_ok=False)
        if path.is_symlink():
            raise ExpertBankError("bank root must not be a symlink")
        path = path.resolve(strict=True)
        data = canonical_json({"schema": SCHEMA, "config": config.to_dict()})
        _Directory(path).create("bank.json", data)
        return cls(path, config, _sha256(data))

    @classmethod
    def open(cls, root) -> "ExpertBank":
        """An existing bank, its configuration validated."""
        path = Path(root)
        if path.is_symlink() or not path.is_dir():
            raise ExpertBankError("bank root must be a regular directory")
        path = path.resolve(strict=True)
        data = _Directory(path).read("bank.json", MAX_METADATA_BYTES)
        head = _fields(_from_canonical(data), ("schema", "config"), "bank")
        if head["schema"] != SCHEMA:
            raise ExpertBankError("unsupported bank schema")
        return cls(path, BankConfig.from_dict(head["config"]), _sha256(data))

    def _check(self) -> None:
        """Refuse to act on a bank whose configuration file changed."""
        if self.root.is_symlink() or not self.root.is_dir() or \
                _sha256(self._dir.read("bank.json", MAX_METADATA_BYTES)) != self._config_hash:
            raise ExpertBankError("bank configuration changed")

    def _validate_id(self, layer: int, expert: int) -> None:
        _whole(layer, "layer", 0, self.config.layers - 1)
        _whole(expert, "expert", 0, self.config.experts_per_layer - 1)

    def _pointer(self, layer: int, expert: int) -> _Pointer | None:
        self._validate_id(layer, expert)
        try:
            data = self._dir.read(f"expert-{layer}-{expert}.json", MAX_METADATA_BYTES)
        except FileNotFoundError:
            return None
        return _Pointer.parse(data, layer, expert, self.config, self._config_hash)

    def _tensors(self, pointer: _Pointer, *, keep: bool = True) -> tuple[VQArray, ...]:
        """The generation's shards, each checked by length, hash and geometry."""
        out = []
        for index, ((size, digest), shape) in enumerate(zip(pointer.shards,
                                                            self.config.matrix_shapes)):
            name = pointer.shard_file(index)
            try:
                data = self._dir.read(name, MAX_SHARD_BYTES)
            except FileNotFoundError as exc:
                raise ExpertBankError(f"missing shard {name} of a committed generation") from exc
            if len(data) != size or _sha256(data) != digest:
                raise ExpertBankError("shard checksum mismatch")
            try:
                image = VQArray.from_bytes(data, max_bytes=MAX_SHARD_BYTES)
            except ValueError as exc:
                raise ExpertBankError(f"invalid VQ shard: {exc}") from exc
            if (image.shape, image.group) != (shape, self.config.group):
                raise ExpertBankError("decoded shard geometry mismatch")
            if keep:
                out.append(image)
        return tuple(out)

    # -- reads ---------------------------------------------------------------------------
    def read_expert(self, layer: int, expert: int) -> tuple[VQArray, ...]:
        return self.read_expert_state(layer, expert).tensors

    def read_expert_state(self, layer: int, expert: int) -> ExpertState:
        """The tensors and optimizer bookkeeping of one pointer snapshot."""
        self._check()
        pointer = self._pointer(layer, expert)
        if pointer is None:
            raise ExpertBankError("expert is not materialized")
        return ExpertState(self._tensors(pointer), pointer.optimizer_step, pointer.revision,
                           pointer.applications)

    # -- the commit ----------------------------------------------------------------------
    def write_expert(self, layer: int, expert: int, tensors: Sequence[VQArray], *,
                     updated_count: int = 0, optimizer_step: int | None = None) -> dict:
        """Commit ``tensors`` (one image per configured matrix) as the expert's
        next generation. ``updated_count`` declares how many values the update
        changed; ``optimizer_step`` (default: unchanged) may not go back."""
        self._check()
        self._validate_id(layer, expert)
        _whole(updated_count, "updated_count", 0, self.config.parameters_per_expert)
        if optimizer_step is not None:
            _whole(optimizer_step, "optimizer_step", 0, MAX_OPTIMIZER_STEP)
        if not isinstance(tensors, (tuple, list)) or \
                len(tensors) != len(self.config.matrix_shapes):
            raise ExpertBankError("one VQArray per configured matrix is required")
        for image, shape in zip(tensors, self.config.matrix_shapes):
            if not isinstance(image, VQArray) or (image.shape, image.group) != \
                    (shape, self.config.group):
                raise ExpertBankError("VQArray geometry mismatch")
            if image.layout["serialized_bytes"] > MAX_SHARD_BYTES:
                raise ExpertBankError("shard byte limit exceeded")
        before = self._pointer(layer, expert)
        if before is None:
            before = _Pointer(layer, expert, "", 0, 0, 0, 0, ())
            fresh = True
        else:
            self._tensors(before, keep=False)  # never build on corrupt committed state
            fresh = False
        step = before.optimizer_step if optimizer_step is None else optimizer_step
        if step < before.optimizer_step:
            raise ExpertBankError("optimizer_step must not regress")
        after = replace(before, generation=uuid.uuid4().hex, revision=before.revision + 1,
                        optimizer_step=step, applications=before.applications + updated_count,
                        commits=before.commits + (updated_count > 0), shards=())
        _whole(after.applications, "parameter_update_applications")
        pending = f"pending-{after.generation}.json"
        written: list[str] = []
        try:
            shards = []
            for index, image in enumerate(tensors):
                data = image.to_bytes()
                # the arrays an image exposes could have been changed behind
                # its back: what goes to disk must still parse
                VQArray.from_bytes(data, max_bytes=MAX_SHARD_BYTES)
                name = after.shard_file(index)
                self._dir.create(name, data)
                written.append(name)
                shards.append((len(data), _sha256(data)))
            after = replace(after, shards=tuple(shards))
            self._dir.create(pending, after.to_json(self._config_hash))
            written.append(pending)
            self._check()
            now = self._pointer(layer, expert)
            if (now is None) != fresh or (now is not None and now != before):
                raise ExpertBankError("another writer changed this expert")
            self._dir.publish(pending, f"{after.base}.json")
        except BaseException:
            self._dir.discard(written)  # a refused commit leaves nothing of its own behind
            raise
        return {"layer": layer, "expert": expert, "revision": after.revision,
                "optimizer_step": step,
                "materialized_parameters": self.config.parameters_per_expert,
                "updated_count": updated_count,
                "parameter_update_applications": after.applications,
                "generation_bytes": sum(size for size, _ in after.shards)}

    def initialize_expert(self, layer: int, expert: int, *, seed: int = 0,
                          zero_optimizer_state: bool = False) -> dict:
        """Commit deterministic payloads for an expert that has none.

        Matrix i draws from ``default_rng(SeedSequence([seed, layer, expert,
        i]))``: uniform u32 code words (unused nibbles of the last word
        cleared), then a standard-normal float32 book scaled by 1/sqrt(rows).
        ``zero_optimizer_state`` makes matrices 1 and 2 all-zero (the
        momentum and variance the VQAdamW harness starts from).
        """
        self._check()
        self._validate_id(layer, expert)
        _whole(seed, "seed", 0, (1 << 64) - 1)
        if not isinstance(zero_optimizer_state, bool):
            raise ExpertBankError("zero_optimizer_state must be bool")
        shapes, group = self.config.matrix_shapes, self.config.group
        if zero_optimizer_state and len(shapes) < 3:
            raise ExpertBankError("zero optimizer state needs three matrix roles")
        if self._pointer(layer, expert) is not None:
            raise ExpertBankError("expert is already materialized")
        images = []
        for index, shape in enumerate(shapes):
            words = storage_layout(shape, group)["code_bytes"] // 4
            if zero_optimizer_state and index in (1, 2):
                codes = np.zeros(words, dtype=np.uint32)
                book = np.zeros((ENTRIES, group), dtype=np.float32)
            else:
                draw = np.random.default_rng(np.random.SeedSequence([seed, layer, expert, index]))
                codes = draw.integers(0, 1 << 32, words, dtype=np.uint32)
                live = -(-shape[0] * shape[1] // group) % 8  # nibbles used in the last word
                if live:
                    codes[-1] &= np.uint32((1 << (4 * live)) - 1)
                book = draw.standard_normal((ENTRIES, group), dtype=np.float32)
                book *= np.float32(1.0 / math.sqrt(shape[0]))
            images.append(VQArray(shape, group, codes, book))
        return self.write_expert(layer, expert, images)

    def stats(self) -> dict:
        """Validate every committed generation and total the bank: experts,
        parameters, declared update applications, committed and on-disk bytes
        (logical file lengths, history included). A coherent census needs a
        quiescent writer."""
        self._check()
        experts = applications = updated = committed = disk = 0
        for path in self.root.iterdir():
            info = path.lstat()
            if not stat.S_ISREG(info.st_mode):
                raise ExpertBankError("unexpected nonregular bank entry")
            disk += info.st_size
            match = _POINTER_FILE.fullmatch(path.name)
            if match is None:
                continue
            layer, expert = int(match[1]), int(match[2])
            self._validate_id(layer, expert)
            if path.name != f"expert-{layer}-{expert}.json":
                raise ExpertBankError("noncanonical expert filename")
            pointer = self._pointer(layer, expert)
            if pointer is None:
                raise ExpertBankError("expert pointer disappeared")
            self._tensors(pointer, keep=False)
            experts += 1
            applications += pointer.applications
            updated += pointer.commits > 0
            committed += sum(size for size, _ in pointer.shards)
        return {"potential_experts": self.config.layers * self.config.experts_per_layer,
                "potential_parameters": self.config.potential_parameters,
                "materialized_experts": experts,
                "materialized_parameters": experts * self.config.parameters_per_expert,
                "updated_experts": updated,
                "parameter_update_applications": applications,
                "unique_updated_parameters": None,
                "committed_payload_bytes": committed, "disk_bytes": disk}
