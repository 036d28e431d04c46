"""Host-side pieces of bench.py that need no GPU: the one-GPU refusal and the
relabelled batch the config-3 launches stream."""
from __future__ import annotations

import numpy as np


def test_bench_refuses_more_than_one_gpu(capsys):
    import bench
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_relabelled_items_decode_to_the_same_tensor():
    """Item i maps code c to perm_i[c] and moves book row c to perm_i[c]:
    byte-distinct images (so a batch cannot be served from one cached image)
    whose decodes are bit-identical to the original's."""
    import bench
    from oracle import vq4_numpy as o
    rng = np.random.default_rng(0)
    group, count = 16, 6
    values = 4096
    idx = rng.integers(0, 16, values // group)
    codes = o.pack_indices(idx)
    book = rng.standard_normal((16, group)).astype(np.float32)
    out_codes, out_books = bench.relabelled_items(codes, book, count, 4)
    ref = o.decode(codes, book, values, group)
    assert np.array_equal(out_codes[0], codes) and np.array_equal(out_books[0], book)
    for i in range(count):
        got = o.decode(out_codes[i], out_books[i], values, group)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), i
    distinct = {out_codes[i].tobytes() for i in range(count)}
    assert len(distinct) == count
