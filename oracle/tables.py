"""Integer tables of the hot path, restated in numpy (test infrastructure).

- ``rel_bias_row``  packages/shrimp/python/shrimp/geometry.py:97-131
- ``cell_lut``      model.py:625-641 (35 x 35, clamp +-17)
- ``gather_index``  model.py:861-863
- ``pair_rows``     model.py:677-716 / 762-792 (key - query offsets); numpy, the
                    pinned checker
- ``pair_rows_torch`` the same rows built in torch the way the reference's CPU
                    path builds them (the forward oracle and the CPU baseline)
- ``seq_lens``      model.py:884-892
- ``ray_index``     hexfield_eq/_triton_ray.py:131-152 (slot table), 221-281 (join)
"""

from __future__ import annotations

import numpy as np

NUM_TOKENS = 8
BIAS_ROWS = 237
ROW_CELL_TOKEN = 234  # query cell, key token
ROW_TOKEN_CELL = 235  # query token, key cell
ROW_TOKEN_TOKEN = 236
LUT_M = 17
LUT_W = 2 * LUT_M + 1
DIRECTIONS = ((1, 0), (0, 1), (-1, 1), (-1, 0), (0, -1), (1, -1))
RAY_SLOTS = 32
RAY_AXES = ((1, 0), (0, 1), (1, -1))  # Q, R, QR


def hex_distance(dq, dr):
    return np.maximum(np.maximum(np.abs(dq), np.abs(dr)), np.abs(np.asarray(dq) + np.asarray(dr)))


def exact_disk(radius: int = 8) -> list:
    """Offsets with distance <= radius in ascending (dq, dr) order — the exact
    bias rows 0..216."""

    cells = [
        (dq, dr)
        for dq in range(-radius, radius + 1)
        for dr in range(-radius, radius + 1)
        if max(abs(dq), abs(dr), abs(dq + dr)) <= radius
    ]
    return sorted(cells)


_DISK_ROW = {c: i for i, c in enumerate(exact_disk(8))}


def rel_bias_row(dq: int, dr: int) -> int:
    d = max(abs(dq), abs(dr), abs(dq + dr))
    if d <= 8:
        return _DISK_ROW[(dq, dr)]
    if d <= 16:
        on_axis = dq == 0 or dr == 0 or dq + dr == 0
        return (217 if on_axis else 225) + (d - 9)
    return 233


def cell_lut() -> np.ndarray:
    lut = np.zeros(LUT_W * LUT_W, dtype=np.uint8)
    for i in range(LUT_W):
        for j in range(LUT_W):
            lut[i * LUT_W + j] = rel_bias_row(i - LUT_M, j - LUT_M)
    return lut


def gather_index(nbr: np.ndarray) -> np.ndarray:
    """(B, N, 6) neighbour rows (sentinel N) -> (B, N, 7), tap 0 = self."""

    b, n, _ = nbr.shape
    self_idx = np.broadcast_to(np.arange(n).reshape(1, n, 1), (b, n, 1))
    return np.concatenate([self_idx, nbr], axis=2).astype(np.int64)


def pair_rows(coords: np.ndarray, mask: np.ndarray, pad_row: int | None = None) -> np.ndarray:
    """(B, S, S) bias-table row of every (query, key) pair, S = 8 + N.

    Cells use the LUT row of (key - query); token rows are 236 / 235 / 234.
    With ``pad_row`` set, padded cell keys are replaced by it (the uint8
    variant, model.py:790-792)."""

    b, n, _ = coords.shape
    lut = cell_lut()
    dq = coords[:, None, :, 0] - coords[:, :, None, 0]
    dr = coords[:, None, :, 1] - coords[:, :, None, 1]
    qi = np.clip(dq, -LUT_M, LUT_M) + LUT_M
    ri = np.clip(dr, -LUT_M, LUT_M) + LUT_M
    cell = lut[qi * LUT_W + ri].astype(np.int64)
    s = NUM_TOKENS + n
    pair = np.full((b, s, s), ROW_TOKEN_TOKEN, dtype=np.int64)
    pair[:, :NUM_TOKENS, NUM_TOKENS:] = ROW_TOKEN_CELL
    pair[:, NUM_TOKENS:, :NUM_TOKENS] = ROW_CELL_TOKEN
    pair[:, NUM_TOKENS:, NUM_TOKENS:] = cell
    if pad_row is not None:
        dead = np.concatenate([np.zeros((b, NUM_TOKENS), bool), ~mask.astype(bool)], axis=1)
        pair = np.where(dead[:, None, :], pad_row, pair)
    return pair


def pair_rows_torch(coords, mask, pad_row: int | None = None):
    """``pair_rows`` vectorised in torch, as the reference builds it on its CPU
    path (model.py:677-716 ``_build_pair``; the uint8 variant with the pad
    row at model.py:762-792): int16 offsets, clamp to +-17, one LUT gather.
    Returns a (B, S, S) uint8 tensor (every row index is below 256); equal
    to ``pair_rows`` element for element (tests/test_oracle_tables.py)."""

    import torch

    c = torch.as_tensor(coords).to(torch.int16)
    b, n, _ = c.shape
    lut = torch.from_numpy(cell_lut())
    dq = c[:, None, :, 0] - c[:, :, None, 0]
    dr = c[:, None, :, 1] - c[:, :, None, 1]
    qi = (dq.clamp(-LUT_M, LUT_M) + LUT_M).to(torch.int32)
    ri = (dr.clamp(-LUT_M, LUT_M) + LUT_M).to(torch.int32)
    cell = lut[(qi * LUT_W + ri).reshape(-1).to(torch.int64)].reshape(b, n, n)
    s = NUM_TOKENS + n
    pair = torch.full((b, s, s), ROW_TOKEN_TOKEN, dtype=torch.uint8)
    pair[:, :NUM_TOKENS, NUM_TOKENS:] = ROW_TOKEN_CELL
    pair[:, NUM_TOKENS:, :NUM_TOKENS] = ROW_CELL_TOKEN
    pair[:, NUM_TOKENS:, NUM_TOKENS:] = cell
    if pad_row is not None:
        m = torch.as_tensor(mask).to(torch.bool)
        dead = torch.cat([torch.zeros(b, NUM_TOKENS, dtype=torch.bool), ~m], dim=1)
        pair = pair.masked_fill(dead[:, None, :], pad_row)
    return pair


def seq_lens(mask: np.ndarray) -> np.ndarray:
    """8 + (index of the last live cell + 1) per row."""

    n = mask.shape[1]
    idx = np.arange(1, n + 1)[None, :] * mask.astype(np.int64)
    return NUM_TOKENS + idx.max(axis=1)


def ray_slot_offsets() -> np.ndarray:
    """(32, 2): slot 0 self; 1 + axis*10 + dir*5 + (k-1) = dir_sign*k*axis; 31 unused."""

    off = np.zeros((RAY_SLOTS, 2), dtype=np.int64)
    for a, (aq, ar) in enumerate(RAY_AXES):
        for d, sgn in enumerate((1, -1)):
            for k in range(1, 6):
                s = 1 + a * 10 + d * 5 + (k - 1)
                off[s] = (sgn * k * aq, sgn * k * ar)
    return off


def ray_index(coords: np.ndarray, mask: np.ndarray) -> np.ndarray:
    """(B, N, 32) int32: row of the live cell at coords + slot offset, else N;
    slot 0 = own row (pad rows included), slot 31 = N."""

    b, n, _ = coords.shape
    off = ray_slot_offsets()
    out = np.full((b, n, RAY_SLOTS), n, dtype=np.int32)
    for g in range(b):
        where = {}
        for i in range(n):
            if mask[g, i]:
                where[(int(coords[g, i, 0]), int(coords[g, i, 1]))] = i
        for i in range(n):
            q, r = int(coords[g, i, 0]), int(coords[g, i, 1])
            for s in range(1, RAY_SLOTS - 1):
                j = where.get((q + int(off[s, 0]), r + int(off[s, 1])))
                if j is not None:
                    out[g, i, s] = j
            out[g, i, 0] = i
    return out


def tap_ray_slots() -> list:
    """For hex tap t (1..6, DIRECTIONS order) the ray slot of its distance-1
    neighbour (hexfield_eq/_raytap.py:83-96 with k = 1)."""

    off = ray_slot_offsets()
    out = []
    for dq, dr in DIRECTIONS:
        hits = [s for s in range(1, 31) if tuple(off[s]) == (dq, dr)]
        assert len(hits) == 1
        out.append(hits[0])
    return out
