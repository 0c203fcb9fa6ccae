"""Model-batch assembly for variable-N rows (host side).

Restates the serve-relevant part of ``packages/shrimp/python/shrimp/batching.py``:
``quantized_npad`` (:34-47) and ``collate_rows`` (:50-80). Pad rows carry zero
features, ``nbr`` pointing at Npad (the absent-neighbour sentinel), mask False
and zero coords.
"""

from __future__ import annotations

import numpy as np
import torch

PAIR_BUDGET = 2.0e7
PAD_QUANTUM = 256


def quantized_npad(max_nodes: int, quantize: int = PAD_QUANTUM) -> int:
    if quantize <= 1:
        return int(max_nodes)
    return -(-int(max_nodes) // quantize) * quantize


def collate_rows(rows: list, pad_to: int | None = None) -> dict:
    """Pad (Support, features) rows into one batch dict of CPU tensors:
    feats (B, Npad, F) f32, nbr (B, Npad, 6) int64 (missing -> Npad),
    mask (B, Npad) bool, coords (B, Npad, 2) int64, legal_counts (B,) int64."""

    npad = max(sup.num_nodes for sup, _ in rows)
    if pad_to is not None:
        if pad_to < npad:
            raise ValueError(f"pad_to {pad_to} < largest row {npad}")
        npad = int(pad_to)
    b = len(rows)
    f = rows[0][1].shape[1]
    feats = np.zeros((b, npad, f), dtype=np.float32)
    nbr = np.full((b, npad, 6), npad, dtype=np.int64)
    mask = np.zeros((b, npad), dtype=np.bool_)
    coords = np.zeros((b, npad, 2), dtype=np.int64)
    legal = np.zeros((b,), dtype=np.int64)
    for g, (sup, row_feats) in enumerate(rows):
        n = sup.num_nodes
        feats[g, :n] = row_feats
        nb = sup.nbr.astype(np.int64)
        nbr[g, :n] = np.where(nb >= 0, nb, npad)
        mask[g, :n] = True
        coords[g, :n] = sup.coords
        legal[g] = sup.legal_count
    return {
        "feats": torch.from_numpy(feats),
        "nbr": torch.from_numpy(nbr),
        "mask": torch.from_numpy(mask),
        "coords": torch.from_numpy(coords),
        "legal_counts": torch.from_numpy(legal),
    }
