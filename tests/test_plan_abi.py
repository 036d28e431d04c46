"""Admission and C-ABI refusals, host only.

Restates the reference's known-answer tests for the plan
(src/alelyon_compute_kit/_kit/tests/vq4_plan.rs) and the ABI
(_kit/tests/vq4_abi.rs) against libackvq.so, plus this library's own
multiply-add bound. No call here reaches a device: forged handles must be
refused before any lookup dereferences them.
"""
from __future__ import annotations

import ctypes
import re
import struct

import pytest

from conftest import ROOT

MAX_VALUES = 1 << 28
MAX_DIM = 65536
FORGED = ctypes.c_void_p(2 ** 64 - 1)

ACK_ERR_NULL, ACK_ERR_SHAPE, ACK_ERR_SIZE, ACK_ERR_CLOSED = -1, -3, -4, -6


def block(words):
    return struct.pack("<8I", *words)


class Plan:
    def __init__(self, lib, words, bounds=0):
        self.req = (ctypes.c_uint64 * 6)()
        self.work = ctypes.c_uint32()
        self.grid = (ctypes.c_uint32 * 3)()
        p = block(words)
        self.rc = lib.cdll.ack_vq_plan_query(p, len(p), bounds, self.req,
                                             ctypes.byref(self.work), self.grid)
        self.error = lib.last_error() if self.rc else ""
        self.words = words

    @property
    def required(self):
        return list(self.req)

    @property
    def dispatch(self):
        return list(self.grid)


def refusal(lib, words, bounds=0):
    plan = Plan(lib, words, bounds)
    assert plan.rc != 0, f"{words} admitted"
    return plan.error.rsplit(": ", 1)[-1]


def check_buffers(lib, words, capacities, ids):
    p = block(words)
    caps = (ctypes.c_uint64 * 6)(*capacities)
    idv = (ctypes.c_uint64 * 6)(*ids)
    rc = lib.cdll.ack_vq_plan_check_buffers(p, len(p), caps, idv)
    return rc, (lib.last_error().rsplit(": ", 1)[-1] if rc else "ok")


# ---- vq4_plan.rs ------------------------------------------------------------
@pytest.mark.parametrize("group", [8, 16, 32])
def test_packed_cost_counts_padding_and_complete_codebooks(lib, group):
    for length, words in [(1, 1), (group, 1), (group * 8, 1), (group * 8 + 1, 2)]:
        enc = Plan(lib, [0, length, 1, 1, group, 16, 0, 0])
        dec = Plan(lib, [1, length, 1, 1, group, 16, 0, 0])
        assert enc.rc == dec.rc == 0
        assert enc.required == [4 * length, 64 * group, 0, 0, 4 * words, 4]
        assert dec.required == [4 * words, 64 * group, 0, 0, 4 * length, 4]
        assert enc.work.value == words
        assert dec.work.value == length


def test_adamw_is_four_packed_states_and_three_dense_scratch_arrays(lib):
    p = Plan(lib, [3, 129, 1, 1, 16, 16, 0, 0])
    assert p.required == [32, 4096, 28, 0, 1548, 4]
    assert p.work.value == 129
    assert p.dispatch == [3, 1, 1]
    assert Plan(lib, [3, MAX_VALUES // 3, 1, 1, 8, 16, 0, 0]).rc == 0
    assert refusal(lib, [3, MAX_VALUES // 3 + 1, 1, 1, 8, 16, 0, 0]) == "vq-address-limit-exceeded"


def test_matmul_transposes_preserve_storage_counts(lib):
    for flags in range(4):
        p = Plan(lib, [2, 3, 5, 7, 8, 16, flags, 0])
        assert p.required == [4, 512, 4, 512, 60, 4]
        assert p.work.value == 15
        assert p.dispatch == [1, 1, 1]


@pytest.mark.parametrize("slot,value,name", [
    (0, 4, "vq-operation-out-of-range"), (4, 0, "vq-unsupported-group"),
    (4, 4, "vq-unsupported-group"), (4, 64, "vq-unsupported-group"),
    (5, 0, "vq-codebook-entries-not-16"), (5, 15, "vq-codebook-entries-not-16"),
    (5, 17, "vq-codebook-entries-not-16"), (6, 1, "vq-unsupported-flags"),
    (7, 1, "vq-nonzero-reserved-word")])
def test_all_schema_words_are_closed(lib, slot, value, name):
    words = [0, 64, 1, 1, 8, 16, 0, 0]
    words[slot] = value
    assert refusal(lib, words) == name


def test_flags_are_closed_per_operation(lib):
    assert refusal(lib, [2, 1, 1, 1, 8, 16, 4, 0]) == "vq-unsupported-flags"
    for op in (1, 3):
        assert refusal(lib, [op, 1, 1, 1, 8, 16, 1, 0]) == "vq-unsupported-flags"


def test_zero_mismatched_or_overflowing_geometry_refuses(lib):
    for op in range(4):
        for axis in (1, 2, 3):
            words = [op, 1, 1, 1, 8, 16, 0, 0]
            words[axis] = 0
            assert refusal(lib, words) == "vq-invalid-geometry"
    for op in (0, 1, 3):
        for axis in (2, 3):
            words = [op, 1, 1, 1, 8, 16, 0, 0]
            words[axis] = 2
            assert refusal(lib, words) == "vq-invalid-geometry"
    assert refusal(lib, [0, 2 ** 32 - 1, 1, 1, 8, 16, 0, 0]) == "vq-address-limit-exceeded"
    assert refusal(lib, [1, MAX_VALUES + 1, 1, 1, 8, 16, 0, 0]) == "vq-address-limit-exceeded"
    assert refusal(lib, [2, MAX_DIM + 1, 1, 1, 8, 16, 0, 0]) == "vq-invalid-geometry"
    for words in ([2, MAX_DIM, MAX_DIM, 1, 8, 16, 0, 0], [2, MAX_DIM, 1, MAX_DIM, 8, 16, 0, 0],
                  [2, 1, MAX_DIM, MAX_DIM, 8, 16, 0, 0]):
        assert refusal(lib, words) == "vq-address-limit-exceeded"


def test_each_read_and_write_capacity_is_checked_in_bytes(lib):
    for op in range(4):
        words = [2, 11, 9, 7, 16, 16, 0, 0] if op == 2 else [op, 129, 1, 1, 16, 16, 0, 0]
        caps = Plan(lib, words).required
        ids = [1, 2, 3, 4, 5, 6]
        assert check_buffers(lib, words, caps, ids) == (0, "ok")
        for slot in range(6):
            if caps[slot] == 0:
                continue
            short = list(caps)
            short[slot] -= 1
            assert check_buffers(lib, words, short, ids) == (ACK_ERR_SIZE,
                                                             f"vq-binding-{slot}-too-small")


def test_every_output_alias_including_unread_inputs_refuses(lib):
    words = [0, 64, 1, 1, 8, 16, 0, 0]
    caps = [4096] * 6
    for slot in range(4):
        ids = [1, 2, 3, 4, 5, 6]
        ids[4] = ids[slot]
        assert check_buffers(lib, words, caps, ids) == (ACK_ERR_SHAPE, "vq-output-aliases-input")
    for slot in range(5):
        ids = [1, 2, 3, 4, 5, 6]
        ids[5] = ids[slot]
        assert check_buffers(lib, words, caps, ids) == (ACK_ERR_SHAPE, "vq-status-aliases-operand")
    assert check_buffers(lib, words, caps, [1, 1, 1, 1, 2, 3]) == (0, "ok")
    for slot in range(6):
        ids = [1, 2, 3, 4, 5, 6]
        ids[slot] = 0
        assert check_buffers(lib, words, caps, ids) == (ACK_ERR_SHAPE,
                                                        "vq-null-allocation-identity")


def test_maximum_tensor_uses_bounded_two_dimensional_grid(lib):
    p = Plan(lib, [1, MAX_VALUES, 1, 1, 32, 16, 0, 0])
    x, y, z = p.dispatch
    assert (x, y, z) == (65535, 65, 1)
    assert x * y * 64 >= MAX_VALUES
    assert x * y * 64 < 2 ** 32


def test_reference_matmul_work_bound(lib):
    """The reference's scalar-shader bound (vq4_ops.rs:23), kept as a mode."""
    assert Plan(lib, [2, 1024, 1024, 256, 8, 16, 0, 0], bounds=1).rc == 0
    assert refusal(lib, [2, 1024, 1024, 257, 8, 16, 0, 0], bounds=1) == "vq-matmul-work-limit"
    assert refusal(lib, [2, 4096, 4096, 4096, 8, 16, 0, 0], bounds=1) == "vq-matmul-work-limit"


def test_library_matmul_work_bound(lib):
    """This library admits 2^38 multiply-adds: the 2048 x 14336 x 4096
    prefill product is one call; 2^42 is refused with the same name."""
    assert Plan(lib, [2, 2048, 14336, 4096, 32, 16, 0, 0]).rc == 0
    assert Plan(lib, [2, 2048, 4096, 14336, 32, 16, 2, 0]).rc == 0
    assert refusal(lib, [2, 16384, 16384, 16384, 8, 16, 0, 0]) == "vq-matmul-work-limit"


# ---- vq4_abi.rs -------------------------------------------------------------
def call(lib, plan, length):
    b = FORGED
    return lib.cdll.ack_vq(FORGED, b, b, b, b, b, b, plan, length)


def test_schema_is_one(lib):
    assert lib.cdll.ack_vq_schema() == 1


def test_null_and_wrong_sized_blocks_refuse_before_any_handle_lookup(lib):
    assert call(lib, None, 32) == ACK_ERR_NULL
    assert "null plan" in lib.last_error()
    p = block([0, 1, 1, 1, 8, 16, 0, 0])
    for length in (0, 1, 31, 33, 2 ** 64 - 1):
        assert call(lib, p, length) == ACK_ERR_SIZE
        assert "plan has" in lib.last_error()


@pytest.mark.parametrize("words,code,name", [
    ([4, 1, 1, 1, 8, 16, 0, 0], ACK_ERR_SHAPE, "vq-operation-out-of-range"),
    ([0, 1, 1, 1, 4, 16, 0, 0], ACK_ERR_SHAPE, "vq-unsupported-group"),
    ([0, 1, 1, 1, 8, 15, 0, 0], ACK_ERR_SHAPE, "vq-codebook-entries-not-16"),
    ([2, 1, 1, 1, 8, 16, 4, 0], ACK_ERR_SHAPE, "vq-unsupported-flags"),
    ([0, 1, 1, 1, 8, 16, 0, 1], ACK_ERR_SHAPE, "vq-nonzero-reserved-word"),
    ([0, 0, 1, 1, 8, 16, 0, 0], ACK_ERR_SHAPE, "vq-invalid-geometry"),
    ([0, 2 ** 32 - 1, 1, 1, 8, 16, 0, 0], ACK_ERR_SIZE, "vq-address-limit-exceeded"),
    ([3, 1 << 28, 1, 1, 8, 16, 0, 0], ACK_ERR_SIZE, "vq-address-limit-exceeded")])
def test_malformed_schema_refuses_by_name_before_any_device_lookup(lib, words, code, name):
    p = block(words)
    assert call(lib, p, len(p)) == code
    assert lib.last_error().endswith(name), lib.last_error()


def test_all_valid_operations_reach_closed_device_refusal_without_dereference(lib):
    for op in range(4):
        p = block([op, 1, 1, 1, 8, 16, 0, 0])
        assert call(lib, p, len(p)) == ACK_ERR_CLOSED
        assert "is not open" in lib.last_error()


def test_excessive_matmul_work_refuses_before_device_lookup(lib):
    p = block([2, 16384, 16384, 16384, 8, 16, 0, 0])
    assert call(lib, p, len(p)) == ACK_ERR_SIZE
    assert lib.last_error().endswith("vq-matmul-work-limit")


def test_batch_count_zero_is_refused(lib):
    p = block([0, 1, 1, 1, 8, 16, 0, 0])
    b = FORGED
    assert lib.cdll.ack_vq_batch(FORGED, b, b, b, b, b, b, p, len(p), 0) == ACK_ERR_SHAPE


def test_transfers_refuse_forged_devices(lib):
    buf = ctypes.create_string_buffer(4)
    assert lib.cdll.ack_upload(FORGED, FORGED, buf, 4) == ACK_ERR_CLOSED
    assert lib.cdll.ack_download(FORGED, FORGED, buf, 4) == ACK_ERR_CLOSED
    assert lib.cdll.ack_buffer_free(FORGED, FORGED) == ACK_ERR_CLOSED
    assert lib.cdll.ack_close(FORGED) == ACK_ERR_CLOSED
    assert lib.cdll.ack_upload(FORGED, FORGED, None, 4) == ACK_ERR_NULL
    assert not lib.cdll.ack_buffer_alloc(FORGED, 0)
    assert "zero-byte" in lib.last_error()


def test_library_exports_every_declared_symbol(lib):
    header = (ROOT / "include" / "ack_vq.h").read_text()
    declared = set(re.findall(r"\b(ack_[a-z0-9_]+)\s*\(", header))
    assert {"ack_vq", "ack_vq_schema", "ack_open", "ack_download"} <= declared
    for name in sorted(declared):
        assert hasattr(lib.cdll, name), f"libackvq.so does not export {name}"


# ---- ack_abi_info / ack_device_info (ffi.rs:1005-1060, :1212-1250) -----------
def test_info_struct_layouts_are_the_references():
    """The C structs' layouts as ffi.rs declares them: AckAbiInfo 96 bytes,
    AckDeviceInfo 616 with `identity` at byte 160 (the end of the hashed
    numeric fields, 8..160)."""
    from alelyon_compute_kit import ack
    assert ctypes.sizeof(ack.AckAbiInfo) == 96
    assert ctypes.sizeof(ack.AckDeviceInfo) == 616
    assert ack.AckDeviceInfo.identity.offset == 160
    assert ack.AckDeviceInfo.device_name.offset == 168


def test_abi_info_reports_no_operator_family(lib):
    """This library serves vq4/v1 only: every operator bit, operator schema
    and capability reads 0 (absent); the layout's ABI version is 14; the
    shader and build identities are set. A null or short struct is refused
    as the reference refuses it."""
    from alelyon_compute_kit import ack
    info = ack.abi_info(lib)
    assert (info.size, info.version, info.operators) == (96, 14, 0)
    assert info.shaders != 0 and info.build != 0
    assert all(getattr(info, name) == 0 for name, _ in ack.AckAbiInfo._fields_[5:])
    assert lib.cdll.ack_abi_info(None, 96) == ACK_ERR_NULL
    small = ack.AckAbiInfo()
    assert lib.cdll.ack_abi_info(ctypes.byref(small), 95) == ack.ACK_ERR_ABI
    assert "smaller than this library's 96" in lib.last_error()


def test_device_info_refuses_before_any_device_lookup(lib):
    from alelyon_compute_kit import ack
    out = ack.AckDeviceInfo()
    assert lib.cdll.ack_device_info(FORGED, None, 616) == ACK_ERR_NULL
    assert lib.cdll.ack_device_info(FORGED, ctypes.byref(out), 615) == ack.ACK_ERR_ABI
    assert lib.cdll.ack_device_info(None, ctypes.byref(out), 616) == ACK_ERR_NULL
    assert lib.cdll.ack_device_info(FORGED, ctypes.byref(out), 616) == ACK_ERR_CLOSED


# ---- this library's extensions ------------------------------------------------
def _path(lib, entry, words):
    out = ctypes.create_string_buffer(32)
    p = block(words)
    rc = getattr(lib.cdll, entry)(p, len(p), out, len(out))
    return rc, out.value.decode()


@pytest.mark.parametrize("words,path", [
    ((2, 1, 4096, 4096, 16, 16, 0, 0), "gemv-direct"),        # one weight of 2^24 values
    ((2, 1, 8192, 8192, 16, 16, 0, 0), "gemv-pairs"),         # past 2^25 values: pair bins
    ((2, 1, 4096, 4096, 16, 16, 1, 0), "gemv-direct"),        # m = 1: A's layout is moot
    ((2, 8, 4096, 4096, 16, 16, 1, 0), "gemv-direct"),        # up to 8 rows, A either way
    ((2, 8, 8192, 8192, 16, 16, 1, 0), "gemv-rows"),
    ((2, 9, 4096, 4096, 16, 16, 0, 0), "onehot-mfma"),        # past 8 rows
    ((2, 8, 4096, 4096, 16, 16, 0, 0), "onehot-mfma"),        # 8 rows, B of 2^24 values
    ((2, 4, 4096, 4096, 16, 16, 0, 0), "gemv-direct"),        # below 8 rows
    ((2, 32, 4096, 4096, 16, 16, 0, 0), "onehot-mfma"),
    ((2, 32, 4096, 16384, 16, 16, 0, 0), "onehot-mfma"),       # long k: split over blocks
    ((2, 32, 4096, 16384, 8, 16, 0, 0), "gemv-rows"),          # packed g 8: chunks of 8 rows
    ((2, 32, 512, 512, 16, 16, 0, 0), "general"),              # small weight: bit-exact kernel
    ((2, 2048, 14336, 4096, 32, 16, 0, 0), "onehot-mfma"),    # config 4 forward
    ((2, 64, 14336, 4096, 32, 16, 0, 0), "onehot-mfma"),
    ((2, 12, 14336, 4096, 32, 16, 0, 0), "onehot-mfma"),
    ((2, 12, 14336, 4096, 32, 16, 1, 0), "gemv-rows"),         # A transposed: chunks of 8
    ((2, 2048, 14336, 4096, 8, 16, 0, 0), "general"),          # g 8: neither
    ((2, 2048, 4096, 14336, 32, 16, 2, 0), "gram-mfma"),
    ((2, 4, 4096, 4096, 16, 16, 2, 0), "gram-mfma"),           # both grouped along k
    ((2, 4, 4096, 4096, 16, 16, 3, 0), "general"),             # A along m, B along k
    ((2, 1, 4100, 4096, 16, 16, 0, 0), "general"),             # n not whole words of groups
    ((0, 100, 1, 1, 16, 16, 0, 0), "encode"), ((1, 100, 1, 1, 16, 16, 0, 0), "decode"),
    ((3, 100, 1, 1, 16, 16, 0, 0), "adamw")])
def test_kernel_path_choice(lib, words, path):
    assert _path(lib, "ack_vq_path_name", words) == (0, path)


@pytest.mark.parametrize("words,path", [
    ((2, 1, 4096, 4096, 16, 16, 0, 0), "gemv-direct"),
    ((2, 1, 8192, 8192, 16, 16, 0, 0), "gemv-pairs"),
    ((2, 19, 2048, 3072, 8, 16, 0, 0), "onehot-mfma"),        # dense A from 9 rows
    ((2, 8, 2048, 3072, 8, 16, 0, 0), "gemv-direct"),
    ((2, 19, 2048, 3072, 8, 16, 1, 0), "gemv-rows"),
    ((2, 5, 2048, 3000, 8, 16, 1, 0), "gemv-direct"),         # ragged k, x stored k x m
    ((2, 128, 768, 512, 8, 16, 0, 0), "onehot-mfma"),         # dense A: group 8 admitted
    ((2, 2048, 14336, 4096, 32, 16, 0, 0), "onehot-mfma"),     # config 4 forward, dense X
    ((2, 2048, 4096, 14336, 32, 16, 2, 0), "general"),         # no Gram path for dense A
    ((2, 9, 200, 64, 16, 16, 1, 0), "general")])
def test_dense_product_path_choice(lib, words, path):
    assert _path(lib, "ack_vq_dense_path_name", words) == (0, path)


def test_dense_product_refuses_before_any_device_lookup(lib):
    b = FORGED
    assert _path(lib, "ack_vq_dense_path_name", (0, 1, 1, 1, 8, 16, 0, 0))[0] == ACK_ERR_SHAPE
    p = block([0, 1, 1, 1, 8, 16, 0, 0])
    assert lib.cdll.ack_vq_matmul_dense(b, b, b, b, b, b, p, len(p)) == ACK_ERR_SHAPE
    assert "plan op must be 2" in lib.last_error()
    p = block([2, 1, 1, 1, 8, 16, 4, 0])
    assert lib.cdll.ack_vq_matmul_dense(b, b, b, b, b, b, p, len(p)) == ACK_ERR_SHAPE
    assert lib.cdll.ack_vq_matmul_dense(b, b, b, b, b, b, p, 31) == ACK_ERR_SIZE
    p = block([2, 4, 64, 64, 16, 16, 0, 0])
    assert lib.cdll.ack_vq_matmul_dense(FORGED, b, b, b, b, b, p, len(p)) == ACK_ERR_CLOSED


def test_device_fit_and_copy_refuse_before_any_device_lookup(lib):
    b = FORGED
    fit = lib.cdll.ack_vq_fit_codebook
    assert fit(b, b, None, b, b, 64, 12, 4, 4096) == ACK_ERR_SHAPE          # group
    assert fit(b, b, None, b, b, 7, 8, 4, 4096) == ACK_ERR_SIZE             # no whole vector
    assert "complete vector" in lib.last_error()
    assert fit(b, b, None, b, b, (1 << 28) + 8, 8, 4, 4096) == ACK_ERR_SIZE
    assert fit(b, b, None, b, b, 64, 8, 33, 4096) == ACK_ERR_SHAPE          # iterations
    assert fit(b, b, None, b, b, 64, 8, 4, 15) == ACK_ERR_SHAPE             # sample size
    assert fit(b, b, None, b, b, 64, 8, 4, 4096) == ACK_ERR_CLOSED
    assert lib.cdll.ack_buffer_copy(b, b, 0, b, 0, 4) == ACK_ERR_CLOSED
