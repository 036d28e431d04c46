"""The ACKVQ4 wire image and VQArray, host only (vq.py:70-151; README.md:60-61)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden


def test_readme_image_size_and_rate():
    from alelyon_compute_kit import vq
    layout = vq.storage_layout((256, 256), 16)
    assert layout["serialized_bytes"] == 3128
    assert layout["bits_per_value"] == 0.3818359375
    assert layout["sub_bit"] is True
    assert layout == {"elements": 65536, "vectors": 4096, "code_bytes": 2048,
                      "codebook_bytes": 1024, "metadata_bytes": 56, "serialized_bytes": 3128,
                      "payload_bytes": 3072, "bits_per_value": 0.3818359375, "sub_bit": True}


def test_benchmark_image_sizes():
    from alelyon_compute_kit import vq
    assert vq.storage_layout((4096, 4096), 16)["serialized_bytes"] == 525368
    assert vq.storage_layout((4096, 4096), 16)["payload_bytes"] == 525312
    assert vq.storage_layout((4096, 14336), 32)["serialized_bytes"] == 919608
    assert vq.storage_layout((8192, 8192), 8)["serialized_bytes"] == 4194872
    assert vq.storage_layout((128, 128), 16)["serialized_bytes"] == 1592


def test_config1_image_is_byte_identical_to_the_reference():
    """benchmark config 1 through this package's CPU encode and fit gives the
    reference's exact 3,128-byte image (recorded from the reference)."""
    from alelyon_compute_kit import vq
    g = golden("config1.npz")
    book = vq.fit_codebook(g["w"], group=16)
    img = vq.encode(g["w"], book, group=16)
    data = img.to_bytes()
    assert len(data) == 3128
    assert data == g["w_image"].tobytes()
    x_img = vq.encode(g["x"], vq.fit_codebook(g["x"], group=16), group=16)
    assert x_img.to_bytes() == g["x_image"].tobytes()
    back = vq.VQArray.from_bytes(data)
    assert back == img
    np.testing.assert_array_equal(back.decode(), g["w_decoded"])


def test_image_matches_the_oracle_packing():
    from alelyon_compute_kit import vq
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(3)
    for shape, group in (((5, 7), 8), ((3, 100), 16), ((1000,), 32), ((2, 3, 4, 5, 6, 7), 8)):
        m = int(np.prod(shape))
        vectors = -(-m // group)
        idx = rng.integers(0, 16, vectors)
        codes = o.pack_indices(idx)
        book = rng.standard_normal((16, group)).astype(np.float32)
        img = vq.VQArray(shape, group, codes, book)
        assert img.to_bytes() == o.image_bytes(shape, group, codes, book)
        np.testing.assert_array_equal(img.decode().reshape(-1), o.decode(codes, book, m, group))


def test_vqarray_refusals():
    from alelyon_compute_kit import vq
    book = np.zeros((16, 8), np.float32)
    with pytest.raises(ValueError, match="exact uint32"):
        vq.VQArray((9,), 8, np.zeros(2, np.uint32), book)
    with pytest.raises(ValueError, match="unused codeword bits"):
        vq.VQArray((9,), 8, np.array([0x100], np.uint32), book)
    with pytest.raises(ValueError, match="finite float32"):
        vq.VQArray((9,), 8, np.zeros(1, np.uint32), np.full((16, 8), np.nan, np.float32))
    with pytest.raises(ValueError, match="shape"):
        vq.VQArray((9,), 8, np.zeros(1, np.uint32), np.zeros((16, 16), np.float32))
    with pytest.raises(ValueError, match="group"):
        vq.VQArray((9,), 12, np.zeros(1, np.uint32), book)
    with pytest.raises(ValueError, match="rank"):
        vq.VQArray((1,) * 7, 8, np.zeros(1, np.uint32), book)
    img = vq.VQArray((9,), 8, np.array([0x21], np.uint32), book)
    with pytest.raises(AttributeError):
        img.group = 16
    assert not img.codes.flags.writeable


def test_from_bytes_refusals():
    from alelyon_compute_kit import vq
    img = vq.VQArray((9,), 8, np.array([0x21], np.uint32), np.ones((16, 8), np.float32))
    data = img.to_bytes()
    assert vq.VQArray.from_bytes(data) == img
    with pytest.raises(ValueError, match="truncated header"):
        vq.VQArray.from_bytes(data[:20])
    with pytest.raises(ValueError, match="length mismatch"):
        vq.VQArray.from_bytes(data + b"\0")
    bad = bytearray(data)
    bad[0:1] = b"X"
    with pytest.raises(ValueError, match="header"):
        vq.VQArray.from_bytes(bytes(bad))
    with pytest.raises(ValueError, match="byte limit"):
        vq.VQArray.from_bytes(data, max_bytes=40)
