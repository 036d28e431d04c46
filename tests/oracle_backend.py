"""A VQDevice stand-in for tests that computes every device operation with the
CPU oracle (the scalar restatement of vq4.comp ops 0-3), so a whole caller
flow -- harness step, config-2 chain -- can be run on the CPU and compared with
the same flow on the GPU. Test infrastructure only."""
from __future__ import annotations

import numpy as np

from alelyon_compute_kit import vq
from oracle.vq4_numpy import ShaderOracle


class OracleBackend:
    def __init__(self, oracle: ShaderOracle | None = None):
        self.oracle = oracle or ShaderOracle()

    @staticmethod
    def _ok(status: int, what: str) -> None:
        if status:
            raise ValueError(f"oracle {what} status {status}")

    def encode(self, values, codebook, *, group):
        x = np.ascontiguousarray(values, dtype=np.float32)
        book = np.ascontiguousarray(codebook, dtype=np.float32)
        codes, status = self.oracle.encode(x, book, group)
        self._ok(status, "encode")
        return vq.VQArray(x.shape, group, codes, book)

    def decode(self, value):
        out, status = self.oracle.decode(value.codes, value.codebook,
                                         value.layout["elements"], value.group)
        self._ok(status, "decode")
        return out.reshape(value.shape)

    def matmul(self, a, b, *, transpose_a=False, transpose_b=False):
        m, n, k, flags = vq.VQDevice.matmul_geometry(a, b, transpose_a, transpose_b)
        out, status = self.oracle.matmul(a.codes, a.codebook, b.codes, b.codebook,
                                         m, n, k, a.group, flags)
        self._ok(status, "matmul")
        return out

    def adamw(self, weight, momentum, variance, gradient, *, lr, beta1, beta2, eps,
              weight_decay, step):
        count, codes, books, coefficients = vq.VQDevice.op3_inputs(
            weight, momentum, variance, gradient, lr, beta1, beta2, eps, weight_decay, step)
        out, status = self.oracle.adamw(codes, books, coefficients, count, weight.group)
        self._ok(status, "adamw")
        return tuple(x.reshape(weight.shape) for x in np.split(out, 3))
