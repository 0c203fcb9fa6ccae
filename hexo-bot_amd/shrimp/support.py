"""Support set and neighbour table of one position (host side, numpy).

Restates ``packages/shrimp/python/shrimp/support.py``:

- ``stones`` are occupied cells; ``legal`` are empty cells within hex distance
  R of some stone (R = ``SHRIMP_SUPPORT_RADIUS``, default 8; support.py:35);
  ``halo`` is the distance-(R+1) shell. With no stones the support is the
  origin plus its 6 neighbours (support.py:145-162).
- Node order is ``[legal | stones | halo]``, each segment ascending by (q, r)
  (support.py:179-183); ``nbr[row, k]`` is the row of ``cell + DIRECTIONS[k]``
  or -1 (support.py:196-205).

This is the input side of the hot path: the HIP forward consumes the padded
``nbr`` table built from it, so node order and the -1 convention are exact.
"""

from __future__ import annotations

import os
from collections.abc import Iterable
from dataclasses import dataclass

import numpy as np

from .constants import DIRECTIONS, LEGAL_RADIUS

SUPPORT_RADIUS = int(os.environ.get("SHRIMP_SUPPORT_RADIUS", "").strip() or LEGAL_RADIUS)


class SupportContractError(ValueError):
    """The closed-form legal set disagrees with an expected (engine) legal set
    (support.py:39-47)."""


@dataclass(frozen=True)
class Support:
    coords: np.ndarray  # (N, 2) int32 axial (q, r) in node order
    legal_count: int
    stone_count: int
    halo_count: int
    dist: np.ndarray  # (N,) int32 hex distance to the nearest stone
    nbr: np.ndarray  # (N, 6) int32 row-local neighbour rows, -1 if absent
    index: dict

    @property
    def num_nodes(self) -> int:
        return int(self.coords.shape[0])

    def legal_coords(self) -> np.ndarray:
        return self.coords[: self.legal_count]

    def segments(self) -> tuple[range, range, range]:
        a = self.legal_count
        b = a + self.stone_count
        return range(0, a), range(a, b), range(b, self.num_nodes)


def _distances(stones: set, reach: int) -> dict:
    """Multi-source breadth-first hex distances from ``stones`` out to
    ``reach`` steps (every cell of the union of radius-``reach`` disks)."""

    dist = {cell: 0 for cell in stones}
    layer = list(stones)
    for d in range(1, reach + 1):
        nxt = []
        for q, r in layer:
            for dq, dr in DIRECTIONS:
                cell = (q + dq, r + dr)
                if cell not in dist:
                    dist[cell] = d
                    nxt.append(cell)
        layer = nxt
    return dist


def neighbor_table(ordered: list, index: dict) -> np.ndarray:
    nbr = np.full((len(ordered), 6), -1, dtype=np.int32)
    for row, (q, r) in enumerate(ordered):
        for k, (dq, dr) in enumerate(DIRECTIONS):
            j = index.get((q + dq, r + dr))
            if j is not None:
                nbr[row, k] = j
    return nbr


def build_support(
    stones: list,
    *,
    expected_legal: Iterable | None = None,
    radius: int | None = None,
) -> Support:
    """Support of a position from its stone list (support.py:84-105).

    ``radius`` overrides ``SHRIMP_SUPPORT_RADIUS`` for this call only.
    """

    rad = SUPPORT_RADIUS if radius is None else int(radius)
    stone_set = {(int(q), int(r)) for q, r in stones}
    if not stone_set:
        ordered = [(0, 0)] + sorted(DIRECTIONS)
        index = {c: i for i, c in enumerate(ordered)}
        sup = Support(
            coords=np.asarray(ordered, dtype=np.int32),
            legal_count=1,
            stone_count=0,
            halo_count=6,
            dist=np.zeros(len(ordered), dtype=np.int32),
            nbr=neighbor_table(ordered, index),
            index=index,
        )
    else:
        dist = _distances(stone_set, rad + 1)
        legal = sorted(c for c, d in dist.items() if d <= rad and c not in stone_set)
        halo = sorted(c for c, d in dist.items() if d == rad + 1)
        ordered = legal + sorted(stone_set) + halo
        index = {c: i for i, c in enumerate(ordered)}
        sup = Support(
            coords=np.asarray(ordered, dtype=np.int32).reshape(-1, 2),
            legal_count=len(legal),
            stone_count=len(stone_set),
            halo_count=len(halo),
            dist=np.asarray([dist[c] for c in ordered], dtype=np.int32),
            nbr=neighbor_table(ordered, index),
            index=index,
        )
    if expected_legal is not None:
        _validate_legal(sup, expected_legal)
    return sup


def assert_decision_support(stones: list, expected_legal: Iterable) -> Support:
    return build_support(stones, expected_legal=expected_legal)


def _validate_legal(sup: Support, expected_legal: Iterable) -> None:
    want = {(int(q), int(r)) for q, r in expected_legal}
    have = {(int(q), int(r)) for q, r in sup.legal_coords().tolist()}
    if want != have:
        raise SupportContractError(
            "build_support legal set diverges from the engine "
            f"(closed-form {len(have)} vs engine {len(want)}); "
            f"in_engine_not_closed_form={sorted(want - have)[:8]} "
            f"in_closed_form_not_engine={sorted(have - want)[:8]}"
        )
