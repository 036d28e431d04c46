"""Benchmark of the vq4 packed matmul on one MI355X.

Metric: packed-weight GB/s (and % of HBM peak) at M=1, and
TFLOP/s at M=2048.

Headline line (`value`): benchmark config 3, the decode-shaped GEMV -- a
4096x4096 weight ~N(0, 0.02^2) at group 16 times one activation row
~N(0,1), both vq4-encoded -- measured cache-cold: one step is one batched
launch (ack_vq_batch) over R distinct packed weights whose total exceeds
twice the 256 MiB Infinity Cache, so every packed byte comes from HBM.
`value` = R * 525,312 B / (kernel time per launch), timed with HIP events on
the library's stream, inputs resident in HBM. The R weights are one
genuinely encoded weight with a different relabelling of its 16 entries
each (codes permuted, book rows permuted back): every item decodes to the
same matrix, so all R outputs must agree, while no two items share bytes.

Secondary lines (`extra`):
* `prefill`: benchmark config 4, X 2048x4096 times W 4096x14336 at group 32 and
  dY 2048x14336 times W^T: algorithmic TFLOP/s = 2*M*N*K / time, plus each
  kernel's executed-work rate against its own peak;
* `gemv_m4`, `gemv_m8`: config 3 at M = 4 and 8, the same cache-cold batch;
* `config5`: benchmark config 5, an 8192x8192 row-normalised weight at group 8:
  GPU encode (read GB/s and FP32 VALU fraction), decode, op-3 AdamW, and one
  fused VQAdamW step end to end.

`cpu_baseline`: the oracle's numpy CPU path for config 3 (decode the weight
with a gather, then numpy matmul) on a bounded sample of matrices, timed on
this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--items R] [--no-extra]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "alelyon-compute-kit_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0     # dense (bf16 and fp16 alike)
W_BYTES = 524288 + 1024           # packed codes + codebook of one 4096x4096 g16 weight
SUSTAINED_LAUNCHES = 80              # back-to-back launches for the sustained (power-limited) rate


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def relabelled_items(codes: np.ndarray, book: np.ndarray, count: int, seed: int):
    """`count` byte-distinct images of one tensor: item i maps code c to
    perm_i[c] and stores book row c at perm_i[c]."""
    rng = np.random.default_rng(seed)
    raw = codes.view(np.uint8)
    out_codes = np.empty((count, codes.size), np.uint32)
    out_books = np.empty((count, 16, book.shape[1]), np.float32)
    for i in range(count):
        perm = np.arange(16) if i == 0 else rng.permutation(16)
        lut = (perm[np.arange(256) & 15] | (perm[np.arange(256) >> 4] << 4)).astype(np.uint8)
        out_codes[i] = lut[raw].view(np.uint32)
        out_books[i, perm] = book
    return out_codes, out_books


def timed(device, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    device.synchronize()
    device.timer_start()
    for _ in range(steps):
        fn()
    ms = device.timer_stop()
    return ms / steps


def bench_gemv(device, dev, items, steps, warmup, m=1, single=True, flags=0):
    """Config 3 at activation height m: one batched launch over `items`
    relabelled 4096x4096 g16 weights, HIP-event timed on the library stream.
    flags bit 0: the activations are stored 4096 x m (A transposed)."""
    from alelyon_compute_kit import vq
    from oracle.vq4_numpy import ShaderOracle, max_rel
    rng = np.random.default_rng(3)
    log(f"encoding the 4096x4096 weight (m={m})")
    w = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    w_img = dev.encode(w, vq.fit_codebook(w, group=16), group=16)
    x = rng.standard_normal((m, 4096)).astype(np.float32)
    xs = np.ascontiguousarray(x.T) if flags & 1 else x     # as A is stored
    x_img = dev.encode(xs, vq.fit_codebook(xs, group=16), group=16)
    log(f"building {items} relabelled weights")
    codes, books = relabelled_items(w_img.codes, w_img.codebook, items, 4)
    xa = np.tile(x_img.codes, items)
    xb = np.tile(x_img.codebook.reshape(-1), items)
    bufs = [device.buffer(a.nbytes) for a in (xa, xb, codes, books)]
    for b, a in zip(bufs, (xa, xb, codes, books)):
        b.upload(a)
    out = device.buffer(items * m * 4096 * 4)
    status = device.buffer(4)
    status.upload(np.zeros(1, np.uint32))
    words = (2, m, 4096, 4096, 16, 16, flags, 0)
    path = dev.path_name(words, count=items)
    single_ms = single_path = y_single = None
    dense = None
    try:
        def launch():
            dev.run(words, bufs, out, status, count=items)
        log(f"timing {steps} launches of {items} items, m={m}, path {path}")
        ms = timed(device, launch, steps, warmup)
        status_word = int(status.download(np.uint32)[0])
        y = out.download(np.float32).reshape(items, m, 4096)
        if single:
            # single-matrix latency (resident, cache-warm): one ack_vq of item 0
            arrays = (x_img.codes, x_img.codebook, w_img.codes, w_img.codebook)
            s_bufs = [device.buffer(a.nbytes) for a in arrays]
            for b, a in zip(s_bufs, arrays):
                b.upload(a)
            s_out = device.buffer(m * 4096 * 4)
            single_ms = timed(device, lambda: dev.run(words, s_bufs, s_out, status), 50, 5)
            single_path = dev.path_name(words)
            y_single = s_out.download(np.float32).reshape(m, 4096)
            # the dense-activation product on the same weight: x as float32
            d_x = device.buffer(xs.nbytes)
            d_x.upload(xs)
            dense_ms = timed(device, lambda: dev.run_dense(words, d_x, s_bufs[2], s_bufs[3],
                                                           s_out, status), 50, 5)
            dense = {"single_us": dense_ms * 1e3, "path": dev.dense_path_name(words),
                     "max_rel_vs_float64": None}
            y_dense = s_out.download(np.float32).reshape(m, 4096)
            status_word |= int(status.download(np.uint32)[0])   # the single products' bits
            for b in s_bufs + [s_out, d_x]:
                b.free()
    finally:
        for b in bufs + [out, status]:
            b.free()
    if status_word:
        raise SystemExit(f"status word {status_word} after the GEMV launches (m={m})")
    oracle = ShaderOracle()
    ref, _ = oracle.matmul(x_img.codes, x_img.codebook, w_img.codes, w_img.codebook,
                           m, 4096, 4096, 16, flags)
    err = max(max_rel(y[0], ref), float(np.max(np.abs(y - y[0]))) / float(np.max(np.abs(ref))))
    if dense is not None:
        exact = x.astype(np.float64) @ w_img.decode().astype(np.float64)
        dense["max_rel_vs_float64"] = max_rel(y_dense, exact)
    single_err = None if y_single is None else max_rel(y_single, ref)
    return {"ms": ms, "single_ms": single_ms, "single_path": single_path, "single_err": single_err,
            "path": path,
            "max_rel": err, "dense": dense,
            "gbs": items * W_BYTES / (ms * 1e-3) / 1e9, "x_img": x_img, "w_img": w_img}


def bench_sustained(device, dev, items, launches):
    """Config 3's batched launch held for `launches` in a row, after every
    other measurement: the GPU's power management lowers the shader clock
    after about 1.5 ms of this load (the LDS-atomic binning follows the
    clock; a plain HBM read does not), so this is the rate a long decode
    loop sees. The inputs are bench_gemv's (its outputs were checked there)."""
    from alelyon_compute_kit import vq
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    w_img = dev.encode(w, vq.fit_codebook(w, group=16), group=16)
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    x_img = dev.encode(x, vq.fit_codebook(x, group=16), group=16)
    codes, books = relabelled_items(w_img.codes, w_img.codebook, items, 4)
    arrays = (np.tile(x_img.codes, items), np.tile(x_img.codebook.reshape(-1), items), codes, books)
    bufs = [device.buffer(a.nbytes) for a in arrays]
    out = device.buffer(items * 4096 * 4)
    status = device.buffer(4)
    try:
        for b, a in zip(bufs, arrays):
            b.upload(a)
        status.upload(np.zeros(1, np.uint32))
        words = (2, 1, 4096, 4096, 16, 16, 0, 0)
        log(f"timing {launches} back-to-back launches (sustained rate)")
        ms = timed(device, lambda: dev.run(words, bufs, out, status, count=items), launches, 0)
        if int(status.download(np.uint32)[0]):
            raise SystemExit("status word set during the sustained launches")
    finally:
        for b in bufs + [out, status]:
            b.free()
    return ms


def bench_prefill(device, dev, steps, warmup, policy=0, dense=True):
    """Config 4 forward and backward (and the dense-X forward), every output
    checked against a float64 product. policy 1 forces the general kernel."""
    from alelyon_compute_kit import vq
    rng = np.random.default_rng(4)
    m, k, n = 2048, 4096, 14336
    log("encoding the config-4 operands")
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    w_img = dev.encode(w, vq.fit_codebook(w, group=32), group=32)
    del w
    x = rng.standard_normal((m, k)).astype(np.float32)
    x_img = dev.encode(x, vq.fit_codebook(x, group=32), group=32)
    dy = (rng.standard_normal((m, n)) * 0.1).astype(np.float32)
    dy_img = dev.encode(dy, vq.fit_codebook(dy, group=32), group=32)
    del dy
    results = {}
    for name, a, flags, nn in (("forward", x_img, 0, n), ("backward", dy_img, 2, k)):
        kk = k if flags == 0 else n
        arrays = (a.codes, a.codebook, w_img.codes, w_img.codebook)
        bufs = [device.buffer(arr.nbytes) for arr in arrays]
        for b, arr in zip(bufs, arrays):
            b.upload(arr)
        out = device.buffer(m * nn * 4)
        status = device.buffer(4)
        status.upload(np.zeros(1, np.uint32))
        words = (2, m, nn, kk, 32, 16, flags, 0)
        try:
            device.set_policy(policy)
            log(f"timing {name}: {m}x{nn}x{kk}, path {dev.path_name(words)}, policy {policy}")
            ms = timed(device, lambda: dev.run(words, bufs, out, status), steps, warmup)
            flags_out = int(status.download(np.uint32)[0])
            y = out.download(np.float32).reshape(m, nn)
        finally:
            device.set_policy(0)
            for b in bufs + [out, status]:
                b.free()
        if flags_out:
            raise SystemExit(f"status word {flags_out} after the {name} launches")
        log(f"checking every {name} output against a float64 product")
        wd = w_img.decode().astype(np.float64)
        err, row_err = _all_rows_error(y, a.decode().astype(np.float64) @ (wd if flags == 0
                                                                         else wd.T))
        del wd
        flop = 2.0 * m * nn * kk
        path = "general" if policy == 1 else dev.path_name(words)
        entry = {"ms": ms, "tflops": flop / (ms * 1e-3) / 1e12, "path": path,
                 "max_rel": err, "max_row_rel": row_err}
        # what the kernel actually executes, against that work's own peak
        executed = _executed(path, m, nn, kk, ms)
        if executed:
            entry["executed"] = executed
        results[name] = entry
    if not dense:
        return results
    # the forward product with X handed over dense (no activation encode)
    words = (2, m, n, k, 32, 16, 0, 0)
    bufs = [device.buffer(arr.nbytes) for arr in (x, w_img.codes, w_img.codebook)]
    for b, arr in zip(bufs, (x, w_img.codes, w_img.codebook)):
        b.upload(arr)
    out = device.buffer(m * n * 4)
    status = device.buffer(4)
    status.upload(np.zeros(1, np.uint32))
    try:
        path = dev.dense_path_name(words)
        log(f"timing the dense-activation forward: {m}x{n}x{k}, path {path}")
        ms = timed(device, lambda: dev.run_dense(words, *bufs, out, status), steps, warmup)
        flags_out = int(status.download(np.uint32)[0])
        y = out.download(np.float32).reshape(m, n)
    finally:
        for b in bufs + [out, status]:
            b.free()
    if flags_out:
        raise SystemExit(f"status word {flags_out} after the dense forward launches")
    err, row_err = _all_rows_error(y, x.astype(np.float64) @ w_img.decode().astype(np.float64))
    flop = 2.0 * m * n * k
    results["forward_dense_x"] = {"ms": ms, "tflops": flop / (ms * 1e-3) / 1e12, "path": path,
                                  "max_rel": err, "max_row_rel": row_err}
    executed = _executed(path, m, n, k, ms)
    if executed:
        results["forward_dense_x"]["executed"] = executed
    return results


def _executed(path, m, nn, kk, ms):
    """The work a factorised config-4 kernel executes, against that work's own
    peak (the codebook factorisation executes far fewer operations than the
    algorithmic 2 M N K), or None for the general kernel."""
    if path == "onehot-mfma":
        # A's values (book rows, or dense x) as three bf16 terms times the
        # one-hot of B's codes: inner dimension kk, 16 nn / 32 S columns
        ops = 2.0 * m * (16 * nn // 32) * kk * 3
        what = "bf16 MFMA flops (3-term A operand, FP32-exact)"
    elif path == "gram-mfma":
        # one-hot x Gram GEMM of inner dimension 16 k/g, each Gram entry as
        # three bf16 terms (hi + mid + lo: every FP32 entry exactly)
        ops = 2.0 * m * nn * (3 * 16 * kk // 32)
        what = "bf16 MFMA flops (3-term Gram operand, FP32-exact)"
    else:
        return None
    tflops = ops / (ms * 1e-3) / 1e12
    return {"what": what, "tflops": tflops, "peak": BF16_MFMA_PEAK_TFLOPS,
            "frac": tflops / BF16_MFMA_PEAK_TFLOPS}


def other_paths(items, steps, warmup):
    """The kernels no headline workload takes, on the headline shapes:
    k_gemv_rows (config 3 batch at M = 4 and 8 with A stored 4096 x M, where
    rows cannot run as pair-bin instances) and k_matmul_general (config 4
    forward and backward under policy 1)."""
    from alelyon_compute_kit import ack, vq
    out = {}
    with ack.Device() as device:
        dev = vq.VQDevice(device)
        for m in (4, 8):
            r = bench_gemv(device, dev, items, steps, warmup, m=m, single=False, flags=1)
            out[f"gemv_m{m}_a_transposed"] = {
                "workload": f"config 3 at M={m}, A stored 4096 x {m}, same cache-cold batch",
                "ms": r["ms"], "gbs": r["gbs"], "hbm_frac": r["gbs"] / HBM_PEAK_GBS,
                "path": r["path"], "max_rel_vs_oracle": r["max_rel"]}
        out["config4_general"] = bench_prefill(device, dev, max(2, steps // 4), 1, policy=1,
                                               dense=False)
    return out


def _all_rows_error(y: np.ndarray, ref: np.ndarray):
    """(max-rel over the whole output, largest max-rel of one row against
    that row's own largest magnitude), every output compared."""
    diff = np.abs(y - ref)
    scale = np.abs(ref)
    whole = float(diff.max() / scale.max())
    per_row = diff.max(axis=1) / np.maximum(scale.max(axis=1), np.finfo(np.float64).tiny)
    return whole, float(per_row.max())


def bench_chunk(device, dev, steps, warmup, m=128):
    """A smaller prefill chunk: X m x 4096 . W 4096 x 4096 g32, packed and dense
    X (the one-hot path's 64-row blocks), every output against float64."""
    from alelyon_compute_kit import vq
    rng = np.random.default_rng(6)
    k = n = 4096
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    w_img = dev.encode(w, vq.fit_codebook(w, group=32), group=32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x_img = dev.encode(x, vq.fit_codebook(x, group=32), group=32)
    words = (2, m, n, k, 32, 16, 0, 0)
    wd = w_img.decode().astype(np.float64)
    res = {"workload": f"X {m}x{k} . W {k}x{n} g32, one product"}
    for name, arrays, dense in (("packed", (x_img.codes, x_img.codebook, w_img.codes,
                                            w_img.codebook), False),
                                ("dense_x", (x, w_img.codes, w_img.codebook), True)):
        bufs = [device.buffer(a.nbytes) for a in arrays]
        for b_, a in zip(bufs, arrays):
            b_.upload(a)
        out, status = device.buffer(m * n * 4), device.buffer(4)
        status.upload(np.zeros(1, np.uint32))
        try:
            if dense:
                fn, path = (lambda: dev.run_dense(words, *bufs, out, status)), dev.dense_path_name(words)
            else:
                fn, path = (lambda: dev.run(words, bufs, out, status)), dev.path_name(words)
            log(f"timing the {m}-row chunk ({name}), path {path}")
            ms = timed(device, fn, steps, warmup)
            flags_out = int(status.download(np.uint32)[0])
            y = out.download(np.float32).reshape(m, n)
        finally:
            for b_ in bufs + [out, status]:
                b_.free()
        if flags_out:
            raise SystemExit(f"status word {flags_out} after the {m}-row chunk ({name})")
        a64 = x.astype(np.float64) if dense else x_img.decode().astype(np.float64)
        err, row_err = _all_rows_error(y, a64 @ wd)
        res[name] = {"us": ms * 1e3, "path": path, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12,
                     "max_rel": err, "max_row_rel": row_err}
    return res


def bench_config5(device, dev, steps, warmup):
    """Config 5: 8192x8192 row-normalised N(0,1) weight at group 8 -- GPU
    encode and decode throughput, op-3 AdamW, and the fused VQAdamW step
    (re-encoding weight and both moments) on N(0, 1e-3) gradients."""
    from alelyon_compute_kit import vq
    n, g = 8192, 8
    m = n * n
    rng = np.random.default_rng(5)
    log("config 5: building the 8192x8192 weight")
    w = rng.standard_normal((n, n), dtype=np.float32)
    w /= np.linalg.norm(w, axis=1, keepdims=True).astype(np.float32)
    book = vq.fit_codebook(w, group=g)
    words = vq.storage_layout((n, n), g)["code_bytes"] // 4
    out = {}
    wb = device.buffer(w.nbytes)
    bk = device.buffer(book.nbytes)
    codes = device.buffer(words * 4)
    dense = device.buffer(w.nbytes)
    status = device.buffer(4)
    try:
        wb.upload(w)
        bk.upload(book)
        status.upload(np.zeros(1, np.uint32))
        enc = (0, m, 1, 1, g, 16, 0, 0)
        ms = timed(device, lambda: dev.run(enc, [wb, bk], codes, status), steps, warmup)
        read = 4.0 * m
        out["encode"] = {"ms": ms, "read_gbs": read / (ms * 1e-3) / 1e9,
                         "hbm_frac": read / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "path": dev.path_name(enc)}
        valu = load_counter("encode_config5_counters.json", "valu_lane_ops_per_launch")
        if valu:
            # lane operations the screened argmin executes per launch (PMC
            # SQ_INSTS_VALU x 64 lanes, recorded under profiles/). A counter
            # from one run over another run's time is no roofline, so only
            # the count is reported here; its fraction of the VALU rate is
            # the profile's, from that profile's own kernel time.
            out["encode"]["valu_executed"] = {
                "what": "VALU lane operations per launch (SQ_INSTS_VALU x 64)",
                "lane_ops": valu, "source": "profiles/encode_config5_counters.json"}
        dec = (1, m, 1, 1, g, 16, 0, 0)
        ms = timed(device, lambda: dev.run(dec, [codes, bk], dense, status), steps, warmup)
        moved = 4.0 * m + 4.0 * words
        out["decode"] = {"ms": ms, "gbs": moved / (ms * 1e-3) / 1e9,
                         "hbm_frac": moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        flags = int(status.download(np.uint32)[0])
        if flags:
            raise SystemExit(f"status word {flags} after the config-5 codec launches")
        w_codes = codes.download(np.uint32)
        # fit_codebook of the weight on the device (cold start, 4096-vector
        # sample, 4 iterations) beside the native host fit of the same tensor
        ms = timed(device, lambda: dev.fit_resident(wb, m, dense, status, group=g), steps, warmup)
        if not np.array_equal(dense.download(np.float32)[:16 * g].reshape(16, g), book):
            raise SystemExit("device fit_codebook differs from the host fit")
        t0 = time.perf_counter()
        vq.fit_codebook(w, group=g)
        out["fit"] = {"ms": ms, "host_ms": (time.perf_counter() - t0) * 1e3,
                      "bit_identical_to_host": True}
    finally:
        for b in (wb, bk, codes, dense, status):
            b.free()
    del w
    w_img = vq.VQArray((n, n), g, w_codes, book)
    grad = (rng.standard_normal((n, n), dtype=np.float32) * np.float32(np.sqrt(1e-3)))
    g_img = dev.encode(grad, vq.fit_codebook(grad, group=g), group=g)
    del grad
    opt = vq.VQAdamW(dev, w_img, lr=1e-3, betas=(0.9, 0.999))
    # op-3 AdamW to dense scratch, resident
    count, c4, b4, coeff = vq.VQDevice.op3_inputs(
        opt.weight, opt.momentum, opt.variance, g_img, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1)
    bufs = [device.buffer(a.nbytes) for a in (c4, b4, coeff)]
    scratch = device.buffer(3 * count * 4)
    status = device.buffer(4)
    try:
        for b, a in zip(bufs, (c4, b4, coeff)):
            b.upload(a)
        status.upload(np.zeros(1, np.uint32))
        op3 = (3, count, 1, 1, g, 16, 0, 0)
        ms = timed(device, lambda: dev.run(op3, bufs, scratch, status), steps, warmup)
        moved = 12.0 * count + float(c4.nbytes + b4.nbytes)
        out["adamw_op3"] = {"ms": ms, "gbs": moved / (ms * 1e-3) / 1e9,
                            "hbm_frac": moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    finally:
        for b in bufs + [scratch, status]:
            b.free()
    # the fused step on resident buffers: AdamW at the sample, three device
    # fits, the encode pass
    words3 = 3 * words
    bufs = [device.buffer(a.nbytes) for a in (c4, b4, coeff)]
    extra = [device.buffer(words3 * 4), device.buffer(3 * 16 * g * 4), device.buffer(4),
             device.buffer(4)]
    try:
        for b, a in zip(bufs, (c4, b4, coeff)):
            b.upload(a)
        extra[3].upload(np.zeros(1, np.uint32))
        ms = timed(device, lambda: dev.adamw_step_resident(*bufs, *extra, count=count, group=g),
                   steps, warmup)
        if int(extra[3].download(np.uint32)[0]):
            raise SystemExit("status word set by the fused step")
        out["fused_step_resident"] = {"ms": ms, "changed_weight_values":
                                      int(extra[2].download(np.uint32)[0])}
    finally:
        for b in bufs + extra:
            b.free()
    # the fused step end to end (host images in, host images out: PCIe included)
    t0 = time.perf_counter()
    report = opt.step(g_img)
    out["fused_step"] = {"seconds_end_to_end": time.perf_counter() - t0,
                         "changed_weight_values": report["changed_weight_values"],
                         "note": "uploads of the four packed states, the resident step, "
                                 "downloads of three packed states"}
    return out


def bench_harness(device, dev, steps=3):
    """ExpertHarness.train_step on one expert, default (images uploaded per
    call, host codebook fits) against resident (optimizer state kept on the
    device, device fits): seconds per committed step, end to end."""
    import tempfile
    from alelyon_compute_kit import expert_bank, harness
    out = {}
    for name, shape, group, batch in (("config2", (128, 128), 16, 32),
                                      ("w4096", (4096, 4096), 16, 32)):
        rng = np.random.default_rng(21)
        x = rng.standard_normal((batch, shape[0])).astype(np.float32)
        t = (rng.standard_normal((batch, shape[1])) * 0.1).astype(np.float32)
        entry = {"expert": f"{shape[0]}x{shape[1]} g{group}, batch {batch}"}
        images = {}
        for mode in ("default", "resident"):
            with tempfile.TemporaryDirectory() as tmp:
                bank = expert_bank.ExpertBank.create(
                    Path(tmp) / "bank", expert_bank.BankConfig(1, 1, (shape,) * 3, group))
                bank.initialize_expert(0, 0, seed=7, zero_optimizer_state=True)
                h = harness.ExpertHarness(bank, backend=dev, resident=(mode == "resident"))
                try:
                    h.train_step(x, t)                       # warm-up (and first upload)
                    t0 = time.perf_counter()
                    for _ in range(steps):
                        h.train_step(x, t)
                    entry[f"{mode}_s_per_step"] = (time.perf_counter() - t0) / steps
                    images[mode] = [a.to_bytes() for a in bank.read_expert(0, 0)]
                finally:
                    h.close()
        entry["identical_commits"] = images["default"] == images["resident"]
        out[name] = entry
        log(f"harness {name}: {entry}")
    return out


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(x_img, w_img, budget_s=10.0):
    """The oracle's numpy CPU path for config 3: decode + matmul per matrix
    (the value), with the other CPU phases of the path -- the codebook fit
    and the float64 encode of the same weight -- timed beside it."""
    from oracle import vq4_numpy as o
    blas = {}
    try:
        from threadpoolctl import threadpool_info
        for info in threadpool_info():
            if info.get("user_api") == "blas":
                blas = {"vendor": info.get("internal_api"), "threads": info.get("num_threads")}
                break
    except Exception:  # pragma: no cover - threadpoolctl is optional
        pass
    threads = int(blas.get("threads") or os.cpu_count() or 1)
    x = o.decode(x_img.codes, x_img.codebook, 4096, 16).reshape(1, 4096)

    def median_of(fn, runs=5):
        fn()                                           # warm-up
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times))

    decode_s = median_of(lambda: o.decode(w_img.codes, w_img.codebook, 4096 * 4096, 16))
    wd = o.decode(w_img.codes, w_img.codebook, 4096 * 4096, 16).reshape(4096, 4096)
    matmul_s = median_of(lambda: x @ wd)
    fit_s = median_of(lambda: o.fit_codebook(wd, 16), runs=3)
    encode_s = median_of(lambda: o.encode64(wd.reshape(-1)[:1 << 20], w_img.codebook, 16),
                         runs=3) * 16               # 1/16 of the weight, scaled
    # the value: decode + matmul per matrix, repeated for about budget_s
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        w_dense = o.decode(w_img.codes, w_img.codebook, 4096 * 4096, 16).reshape(4096, 4096)
        _ = x @ w_dense
        times.append(time.perf_counter() - t0)
        if len(times) >= 1000:
            break
    per = float(np.median(times))
    return {"value": W_BYTES / per / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} matrices of config 3 (numpy gather decode of the 4096x4096 "
                      f"g16 weight + numpy matmul with a 1x4096 row), median {per * 1e3:.1f} ms "
                      f"per matrix; BLAS threads {threads}",
            "host": {"cpu": _cpu_model(), "os_cpu_count": os.cpu_count(),
                     "affinity_cores": len(os.sched_getaffinity(0)), "blas": blas},
            "phases_ms": {"decode": decode_s * 1e3, "matmul": matmul_s * 1e3,
                          "fit_codebook": fit_s * 1e3, "encode_float64": encode_s * 1e3},
            "phases_note": "one 4096x4096 g16 weight each; warm-up then median of 5 (fit and "
                           "encode: 3; encode timed on 1/16 of the weight and scaled)"}


def hbm_calibration() -> dict:
    """What plain memory kernels reach on this GPU: a 512 MiB copy (three
    launches; the byte count the traffic counters are scaled by) and the
    read probe (libackprobe.so, built beside the library) streaming 1.5 GiB
    with the GEMV's code loads (the read ceiling the GEMV is held to), median
    of ten event-timed launches after two."""
    import ctypes

    import torch
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    dst.copy_(src)
    stop.record()
    stop.synchronize()
    copy_ms = start.elapsed_time(stop)
    del src, dst
    read_bytes = 3 << 29
    probe = ctypes.CDLL(str(ROOT / "alelyon-compute-kit_amd" / "alelyon_compute_kit" / "_lib"
                            / "libackprobe.so"))
    probe.ack_probe_read_ms.argtypes = (ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32,
                                        ctypes.POINTER(ctypes.c_float))
    probe.ack_probe_read_ms.restype = ctypes.c_int32
    buf = torch.ones(read_bytes // 4, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    times = (ctypes.c_float * 12)()
    rc = probe.ack_probe_read_ms(ctypes.c_void_p(buf.data_ptr()), read_bytes, 12, times)
    del buf
    if rc != 0:
        raise SystemExit(f"read probe failed: {rc}")
    read_ms = float(np.median(list(times)[2:]))
    return {"copy_bytes": 512 << 20, "launches": 3,
            "copy_gbs": round(2 * (512 << 20) / (copy_ms * 1e-3) / 1e9, 1),
            "read_bytes": read_bytes, "read_ms": round(read_ms, 4),
            "read_gbs": round(read_bytes / (read_ms * 1e-3) / 1e9, 1),
            "read_frac": round(read_bytes / (read_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def load_counter(name: str, key: str):
    """A figure from a counter summary under profiles/ (None when absent)."""
    path = ROOT / "profiles" / name
    if path.is_file():
        try:
            return json.loads(path.read_text()).get(key)
        except ValueError:
            return None
    return None


def load_traffic():
    return load_counter("gemv_pairs_config3_traffic.json", "traffic_bytes_per_launch")


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--items", type=int, default=1024)
    parser.add_argument("--no-prefill", action="store_true")
    parser.add_argument("--no-extra", action="store_true",
                        help="skip the secondary lines (config 3 at m=4/8, config 5)")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--other-paths", action="store_true",
                        help="only time the kernels the headline workloads do not take and exit: "
                             "config 3 at M=4 and 8 with A stored 4096 x M (k_gemv_rows) and "
                             "config 4 on the general kernel (the shader's order), one JSON line")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run the HBM calibration and exit: a 512 MiB device-to-"
                             "device copy (the reference for scaling FETCH_SIZE/WRITE_SIZE "
                             "counters) and a read-only pass over 1.5 GiB (the streaming-read "
                             "ceiling), each timed with HIP events")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the vq4 path runs on one device; sharding would split a weight's output "
              "columns or the batched instances across GPUs, and the optimizer refit would "
              "all-gather its calibration sample)",
              file=sys.stderr)
        return 2
    if args.copy_calibration:
        print(json.dumps(hbm_calibration()))
        return 0
    if args.other_paths:
        print(json.dumps(other_paths(args.items, args.steps, args.warmup)))
        return 0
    from alelyon_compute_kit import ack, vq
    with ack.Device() as device:
        dev = vq.VQDevice(device)
        log("device", device.name)
        gemv = bench_gemv(device, dev, args.items, args.steps, args.warmup)
        prefill = None if args.no_prefill else bench_prefill(device, dev, max(3, args.steps // 4),
                                                              1)
        chunk = None if args.no_prefill else bench_chunk(device, dev, max(5, args.steps), 2)
        wide = {}
        c5 = None
        hstep = None
        if not args.no_extra:
            for m in (4, 8):
                r = bench_gemv(device, dev, args.items, max(3, args.steps // 2), 1, m=m)
                wide[m] = r
            c5 = bench_config5(device, dev, max(3, args.steps // 4), 1)
            hstep = bench_harness(device, dev)
        sustained_ms = bench_sustained(device, dev, args.items, SUSTAINED_LAUNCHES)
    gbs = args.items * W_BYTES / (gemv["ms"] * 1e-3) / 1e9
    line = {
        "metric": "vq4 packed matmul: packed-weight GB/s (% HBM peak) at M=1; TFLOP/s at M=2048",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gemv["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 (u4 codes)",
        "data": "synthetic: seeded N(0,0.02^2) weight and N(0,1) activation, vq4-encoded on the "
                "GPU; R byte-distinct relabellings of the weight",
        "config": {"workload": "config 3: decode-shaped GEMV, W 4096x4096 g16, M=1, cache-cold "
                               f"batch of {args.items} packed weights per launch",
                   "items": args.items, "m": 1, "n": 4096, "k": 4096, "group": 16,
                   "path": gemv["path"], "hbm_fraction": round(gbs / HBM_PEAK_GBS, 4),
                   "single_matrix_us": round(gemv["single_ms"] * 1e3, 3),
                   "single_matrix_path": gemv["single_path"],
                   "single_matrix_max_rel": gemv["single_err"],
                   "sustained_gbs": round(args.items * W_BYTES / (sustained_ms * 1e-3) / 1e9, 2),
                   "sustained_launches": SUSTAINED_LAUNCHES,
                   "max_rel_vs_oracle": gemv["max_rel"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic()},
    }
    def tidy(v):
        if isinstance(v, float):
            return float(f"{v:.4g}")
        if isinstance(v, dict):
            return {k: tidy(x) for k, x in v.items()}
        return v

    extra = {}
    if gemv["dense"]:
        extra["gemv_dense_x"] = {"workload": "config 3 weight, one 1x4096 float32 activation "
                                             "row handed over dense (ack_vq_matmul_dense)",
                                 **tidy(gemv["dense"])}
    if chunk:
        extra["prefill_chunk"] = tidy(chunk)
    if prefill:
        extra["prefill"] = {
            "workload": "config 4: X 2048x4096 . W 4096x14336 g32 (forward), dY 2048x14336 . W^T "
                        "(backward)",
            **{f"{k}_{f}": tidy(v[f]) for k, v in prefill.items() for f in v},
            # *_tflops are algorithmic (2 M N K per direction); the codebook
            # factorisation executes far fewer operations than that, so each
            # kernel is held to the roofline of the work it does execute
            # (*_executed), never to the FP32 matrix peak
            "note": "tflops = 2*M*N*K / time (algorithmic); roofline fractions are of "
                    "executed work: bf16 MFMA (onehot-mfma, gram-mfma)"}
    for m, r in wide.items():
        extra[f"gemv_m{m}"] = {"workload": f"config 3 at M={m}, same cache-cold batch",
                               "gbs": tidy(r["gbs"]), "hbm_frac": tidy(r["gbs"] / HBM_PEAK_GBS),
                               "path": r["path"], "max_rel_vs_oracle": tidy(r["max_rel"]),
                               "single_matrix_us": tidy(r["single_ms"] * 1e3),
                               "single_matrix_path": r["single_path"],
                               "single_matrix_max_rel": tidy(r["single_err"]),
                               "single_dense_x": tidy(r["dense"])}
    if c5:
        extra["config5"] = {"workload": "config 5: 8192x8192 row-normalised N(0,1) weight, "
                                        "group 8; N(0,1e-3) gradient",
                            **tidy(c5)}
    if hstep:
        extra["harness_step"] = {"workload": "ExpertHarness.train_step (MSE, clip 1.0, fused "
                                             "VQAdamW, bank commit), seconds per step",
                                 **tidy(hstep)}
    if extra:
        line["extra"] = extra
    if not args.no_cpu:
        log("timing the CPU baseline")
        line["cpu_baseline"] = cpu_baseline(gemv["x_img"], gemv["w_img"])
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
