"""The reference's PyTorch CPU BitLinear, restated for the CPU baseline.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline
leg, never by the spbitnet_amd package.

SparseBitLinear (python/baseline_pytorch.py:56-107) holds the 2:4 ternary
weight as a dense float32 {-1, 0, +1} matrix (:81) and computes, for a 16-bit
input vector x,
    absmax = max |x| (a Python float, :96)
    scale = 127 / absmax, or 0 for absmax 0 (:97)
    x_q = round(x * scale).clamp(-128, 127) in float32 (:98-99)
    y = W @ x_q (float32 BLAS matmul; exact: |y| <= (cols/2) * 128 < 2^24) (:103)
    out = (y * (gamma * absmax / 127)).half() (:106-107)
The weight here is built from the packed format (the oracle's unpack) rather
than from latent weights: the dense {-1, 0, +1} matrix is the same one
(python/convert_model.py:257-316 builds both from the same mask and signs).
"""
from __future__ import annotations

import numpy as np
import torch

from . import oracle as O


class TorchSparseBitLinear:
    def __init__(self, meta, values, gamma: float, rows: int, cols: int):
        dense = O.unpack(meta, values, rows, cols)
        self.weight = torch.from_numpy(dense.astype(np.float32))
        self.gamma = float(gamma)
        self.rows, self.cols = rows, cols

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward(x)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x_f32 = x.float()
        absmax = x_f32.abs().max().item()
        scale = 127.0 / absmax if absmax > 0 else 0.0
        x_q = (x_f32 * scale).round().clamp(-128, 127)
        y = self.weight @ x_q
        return (y * (self.gamma * absmax / 127.0)).half()

    def accumulators(self, x: torch.Tensor) -> torch.Tensor:
        """The float32 matmul output before dequantisation (exact integers)."""
        x_f32 = x.float()
        absmax = x_f32.abs().max().item()
        scale = 127.0 / absmax if absmax > 0 else 0.0
        return self.weight @ (x_f32 * scale).round().clamp(-128, 127)
