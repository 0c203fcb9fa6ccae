"""Value-bin helpers of the serve decode (packages/shrimp/python/shrimp/losses.py:40-60).

These operate on whatever device the logits live on; the evaluator's fused
decode kernel (``shrimp_decode``) computes the same quantities on the GPU.
Training losses are not part of this build.
"""

from __future__ import annotations

import torch

from .constants import MOVES_LEFT_CAP, VALUE_BINS


def value_bins(*, device=None, dtype=None) -> torch.Tensor:
    return torch.linspace(-1.0, 1.0, VALUE_BINS, device=device, dtype=dtype)


def decode_binned_value(logits: torch.Tensor) -> torch.Tensor:
    """Softmax expectation over linspace(-1, 1, 65), clamped to [-1, 1]."""

    bins = value_bins(device=logits.device, dtype=logits.dtype)
    return (torch.softmax(logits, dim=-1) * bins).sum(dim=-1).clamp(-1.0, 1.0)


def decode_moves_left(logits: torch.Tensor) -> torch.Tensor:
    """decode_binned_value mapped affinely to [0, MOVES_LEFT_CAP]."""

    return (decode_binned_value(logits) + 1.0) * 0.5 * MOVES_LEFT_CAP
