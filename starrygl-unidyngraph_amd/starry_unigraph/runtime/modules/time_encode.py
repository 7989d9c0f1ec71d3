"""Learnable cosine time encoding (runtime/modules/time_encode.py:13-58 in the
reference): phi(t) = cos(w t + b), w initialised to 10^-linspace(0, 9, dim),
b = 0. The parameters live in ``self.w`` (an ``nn.Linear(1, dim)`` whose
initial draw is replaced, so construction consumes the same RNG as the
reference). On the training path the encoding is evaluated inside the fused
attention kernels; ``forward`` is the stand-alone form of the same formula.
"""
from __future__ import annotations

import torch
import torch.nn as nn


class TimeEncode(nn.Module):
    def __init__(self, dim: int) -> None:
        super().__init__()
        self.dim = dim
        self.w = nn.Linear(1, dim)
        self.w.bias = nn.Parameter(torch.zeros(dim))
        self.w.weight = nn.Parameter((1.0 / 10 ** torch.linspace(0, 9, dim)).reshape(dim, 1))

    def forward(self, t: torch.Tensor) -> torch.Tensor:
        # fl(fl(t * w) + b): the product rounded, then the bias added, as the
        # attention kernels evaluate it
        tt = t.float().reshape(-1, 1)
        return torch.cos(tt * self.w.weight.reshape(1, -1) + self.w.bias).reshape(*t.shape, self.dim)
