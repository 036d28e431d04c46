"""ack_device_info and the capability record on a real device: the values
come from the HIP runtime, the identity is the reference's FNV-1a over the
numeric fields and the shader identity (ffi.rs:1212-1250, :1419-1428), and
the record has the reference's keys (src/alelyon_compute_kit/_kit/python/
ack.py:527-596) plus abi.vq_schema."""
from __future__ import annotations

import ctypes
import json

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

# the key tree of the reference's capability_record (its dict literal)
REFERENCE_KEYS = {
    "schema": None,
    "abi": {"version": None, "operators": None, "op_schema_matmul_bf16": None,
            "op_schema_cast": None, "op_schema_matmul_f32": None, "op_schema_matmul_f16": None,
            "op_schema_index": None, "op_schema_convert": None, "op_schema_intwise": None,
            "op_schema_pointwise": None,
            "reserved_op_schemas": {"reduce": None, "rowwise": None, "loss": None,
                                    "embedding": None},
            "shaders": None, "build": None,
            "capabilities": {"streams": None, "rng": None, "optimizer": None,
                             "serialization": None}},
    "device": {"name": None, "vendor_id": None, "device_id": None, "device_type": None,
               "device_uuid": None, "driver_uuid": None, "driver_id": None,
               "driver_version_raw": None, "driver_name": None, "driver_info": None,
               "api_version": None, "features": None, "subgroup_size": None,
               "timestamp_valid_bits": None, "timestamp_period_ns": None,
               "device_local_bytes": None,
               "limits": {"max_storage_buffer_bytes": None, "max_push_constant_bytes": None,
                          "max_workgroup_invocations": None, "max_workgroup_count": None,
                          "max_workgroup_size": None},
               "matmul": {"tile": None, "k_multiple": None, "layouts": None,
                          "operand_dtype": None, "result_dtype": None},
               "cast_modes": None, "identity": None},
}


def _keys(tree):
    return {k: (_keys(v) if isinstance(v, dict) else None) for k, v in tree.items()}


def _fnv1a(data: bytes, h: int = 0xCBF29CE484222325) -> int:
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_device_info_values_and_identity(device):
    from alelyon_compute_kit import ack
    say("device info")
    info = device.info()
    assert info.size == 616 and info.version == 1
    assert info.vendor_id == 0x1002 and info.device_type == 2
    assert info.subgroup_size == 64
    assert info.device_local_bytes > 200 * (1 << 30)          # MI355X: 288 GB of HBM3E
    assert info.max_workgroup_invocations == 1024
    assert info.timestamp_valid_bits == 64 and info.timestamp_period_ns > 0
    assert any(info.device_uuid) and not any(info.driver_uuid)
    assert info.features & 1 and not info.features & 16      # matrix cores; fixed wave size
    assert (info.matmul_tile, info.matmul_layouts, info.cast_modes) == (0, 0, 0)
    assert b"gfx950" in info.driver_info
    assert info.device_name.decode() == device.name
    # identity: FNV-1a over bytes 8..160, then the shader identity (LE u64)
    raw = bytes(ctypes.string_at(ctypes.addressof(info), 616))
    shaders = ack.abi_info().shaders
    want = _fnv1a(shaders.to_bytes(8, "little"), _fnv1a(raw[8:160]))
    assert info.identity == want
    assert device.info().identity == info.identity          # stable across calls


def test_capability_record_has_the_reference_keys(device):
    say("capability record")
    record = device.capability_record()
    json.dumps(record, allow_nan=False)
    got = _keys(record)
    assert got["abi"].pop("vq_schema") is None and record["abi"]["vq_schema"] == 1
    assert got == REFERENCE_KEYS
    assert record["abi"]["operators"] == 0 and record["abi"]["version"] == 14
    assert record["device"]["vendor_id"] == 0x1002
    assert "subgroup_size_control" not in record["device"]["features"]
    assert record["device"]["identity"] == f"{device.info().identity:016x}"
