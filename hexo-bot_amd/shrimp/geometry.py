"""Hex-lattice geometry on axial coordinates (q, r), exact integer math.

Mirrors the public functions of ``packages/shrimp/python/shrimp/geometry.py``
(``hex_dist`` :24, ``pack_action_id`` :30, ``rot60``/``reflect``/``apply_d6``
:53-71, ``on_win_axis`` :85, ``disk_offsets`` :97, ``rel_bias_index`` :117)
and adds the dense offset LUT the HIP attention kernel reads
(``cell_bias_lut``, the table ``ShrimpNet._cell_bias_lut`` builds at
``model.py:625-641``).
"""

from __future__ import annotations

import numpy as np

from .constants import (
    BIAS_DISK_RADIUS,
    BIAS_EXACT_ROWS,
    BIAS_FAR_ROW,
    BIAS_OFF_AXIS_BASE,
    BIAS_ON_AXIS_BASE,
    BIAS_RING_MAX,
    BIAS_RING_MIN,
    COORD_OFFSET,
)

_I16_MIN = -(1 << 15)
_I16_MAX = (1 << 15) - 1


def hex_dist(dq: int, dr: int) -> int:
    """Hex distance of an axial offset (third cube axis s = -dq - dr)."""

    return max(abs(dq), abs(dr), abs(dq + dr))


def pack_action_id(q: int, r: int) -> int:
    """((q + 2^15) << 16) | (r + 2^15); ValueError outside the i16 range."""

    if q < _I16_MIN or q > _I16_MAX or r < _I16_MIN or r > _I16_MAX:
        raise ValueError(f"coordinate out of i16 range: ({q}, {r})")
    return ((q + COORD_OFFSET) << 16) | (r + COORD_OFFSET)


def unpack_action_id(action_id: int) -> tuple[int, int]:
    return ((action_id >> 16) & 0xFFFF) - COORD_OFFSET, (action_id & 0xFFFF) - COORD_OFFSET


def rot60(q: int, r: int) -> tuple[int, int]:
    return -r, q + r


def reflect(q: int, r: int) -> tuple[int, int]:
    return q, -q - r


def apply_d6(index: int, q: int, r: int) -> tuple[int, int]:
    """D6 element ``index``: 0-5 rotate by 60*index degrees; 6-11 reflect
    first, then rotate by 60*(index-6) degrees."""

    if index < 0 or index >= 12:
        raise ValueError(f"D6 index out of range: {index}")
    if index >= 6:
        q, r = reflect(q, r)
    for _ in range(index % 6):
        q, r = rot60(q, r)
    return q, r


def d6_inverse(index: int) -> int:
    if index < 0 or index >= 12:
        raise ValueError(f"D6 index out of range: {index}")
    return index if index >= 6 else (-index) % 6


def on_win_axis(dq: int, dr: int) -> bool:
    """Collinear with one of the win axes Q=(1,0), R=(0,1), QR=(1,-1)."""

    return dq == 0 or dr == 0 or dq + dr == 0


def disk_offsets(radius: int) -> list[tuple[int, int]]:
    """Offsets with hex_dist <= radius, ascending by (dq, dr)."""

    out = []
    for dq in range(-radius, radius + 1):
        lo = max(-radius, -radius - dq)
        hi = min(radius, radius - dq)
        out.extend((dq, dr) for dr in range(lo, hi + 1))
    return out


_EXACT_ROW = {off: i for i, off in enumerate(disk_offsets(BIAS_DISK_RADIUS))}
if len(_EXACT_ROW) != BIAS_EXACT_ROWS:  # pragma: no cover - structural
    raise AssertionError("bias disk size mismatch")


def rel_bias_index(dq: int, dr: int) -> int:
    """Bias-table row of a (key - query) cell offset: the exact disk row for
    distance <= 8, an on-/off-axis ring row for distance 9..16, else the far
    row."""

    d = hex_dist(dq, dr)
    if d <= BIAS_DISK_RADIUS:
        return _EXACT_ROW[(dq, dr)]
    if d <= BIAS_RING_MAX:
        base = BIAS_ON_AXIS_BASE if on_win_axis(dq, dr) else BIAS_OFF_AXIS_BASE
        return base + d - BIAS_RING_MIN
    return BIAS_FAR_ROW


# Clamp bound and width of the dense offset LUT. Clamping each component to
# +-M keeps every offset with distance >= 17 in the far class (a clamped
# component of magnitude M=17 alone has distance >= 17), so the LUT is exact
# for every offset.
CELL_LUT_M = BIAS_RING_MAX + 1
CELL_LUT_W = 2 * CELL_LUT_M + 1


def cell_bias_lut() -> np.ndarray:
    """(W*W,) uint8: lut[(clamp(dq)+M)*W + clamp(dr)+M] = rel_bias_index."""

    m, w = CELL_LUT_M, CELL_LUT_W
    lut = np.empty(w * w, dtype=np.uint8)
    for dq in range(-m, m + 1):
        for dr in range(-m, m + 1):
            lut[(dq + m) * w + (dr + m)] = rel_bias_index(dq, dr)
    return lut
