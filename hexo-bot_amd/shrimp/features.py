"""The 15 node-feature planes of one position (host side, numpy).

Restates ``packages/shrimp/python/shrimp/features.py``: the
``PositionFacts`` record (:54-77), turn bookkeeping (:80-93), the
single-colour window scan for hot / standing-win cells (:99-159), the feature
build (:165-210) and the opponent's last full turn (:213-233). The HIP
forward consumes these planes unchanged, so the values must be exact.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .constants import (
    DIST_SCALE,
    F_DIST_TO_STONE,
    F_EMPTY,
    F_FIRST_STONE,
    F_LEGAL,
    F_OPP_HOT,
    F_OPP_LAST_TURN,
    F_OPP_RECENCY,
    F_OPP_STONE,
    F_OPP_WIN_NOW,
    F_OWN_HOT,
    F_OWN_RECENCY,
    F_OWN_STONE,
    F_OWN_WIN_NOW,
    F_PHASE_SECOND,
    F_PLAYER_COLOUR,
    HOT_MIN_COUNT,
    HOT_MIN_PLACEMENTS,
    NUM_FEATURES,
    WIN_NOW_COUNT,
    WINDOW_LEN,
)
from .support import Support, build_support

PHASE_OPENING = "Opening"
PHASE_FIRST = "FirstStone"
PHASE_SECOND = "SecondStone"

AXIS_DELTAS: dict = {"Q": (1, 0), "R": (0, 1), "QR": (1, -1)}


@dataclass(frozen=True)
class PositionFacts:
    """One decision state: placement history ``(q, r, owner, placement_index)``
    in chronological order, side to move, phase, first stone of the current
    turn, and side-relative hot / standing-win cells."""

    records: tuple
    current_player: int
    phase: str
    first_stone: tuple | None
    own_hot: tuple
    opp_hot: tuple
    own_win: tuple
    opp_win: tuple

    @property
    def placements_made(self) -> int:
        return len(self.records)

    def stones(self) -> list:
        return [(q, r) for q, r, _o, _i in self.records]


def record_phase(ordinal: int) -> str:
    """Turn structure is 1 stone, then 2 per turn: record 0 opens, odd
    ordinals are first stones, even ordinals (>0) second stones."""

    if ordinal == 0:
        return PHASE_OPENING
    return PHASE_FIRST if ordinal % 2 == 1 else PHASE_SECOND


def record_player(ordinal: int) -> int:
    """Player 0 opens; then players alternate every two records starting with
    player 1 (records 1-2 player 1, 3-4 player 0, ...)."""

    if ordinal == 0:
        return 0
    return 1 - ((ordinal - 1) // 2) % 2


def window_scan(records: tuple, current_player: int, placements_made: int):
    """(own_hot, opp_hot, own_win, opp_win) from every length-6 window along
    the three win axes that contains a stone and holds one colour only.

    A window with 5 stones marks its single empty cell as a standing win; a
    window with >= 4 stones (once >= 7 placements exist) marks all its empty
    cells hot. Own vs opp is the window colour relative to ``current_player``.
    """

    colour = {(q, r): owner for q, r, owner, _ in records}
    marks = {"own_hot": set(), "opp_hot": set(), "own_win": set(), "opp_win": set()}
    hot_enabled = placements_made >= HOT_MIN_PLACEMENTS
    visited = set()
    for sq, sr in colour:
        for axis, (dq, dr) in AXIS_DELTAS.items():
            for shift in range(WINDOW_LEN):
                q0, r0 = sq - shift * dq, sr - shift * dr
                if (q0, r0, axis) in visited:
                    continue
                visited.add((q0, r0, axis))
                counts = [0, 0]
                empty = []
                for i in range(WINDOW_LEN):
                    cell = (q0 + i * dq, r0 + i * dr)
                    who = colour.get(cell)
                    if who is None:
                        empty.append(cell)
                    else:
                        counts[who] += 1
                if counts[0] and counts[1]:
                    continue
                owner = 0 if counts[0] else 1
                side = "own" if owner == current_player else "opp"
                total = counts[0] + counts[1]
                if total == WIN_NOW_COUNT:
                    marks[side + "_win"].update(empty)
                if total >= HOT_MIN_COUNT and hot_enabled:
                    marks[side + "_hot"].update(empty)
    return (
        tuple(sorted(marks["own_hot"])),
        tuple(sorted(marks["opp_hot"])),
        tuple(sorted(marks["own_win"])),
        tuple(sorted(marks["opp_win"])),
    )


def opp_last_turn_cells(facts: PositionFacts) -> list:
    """Cells of the opponent's most recent full turn: its newest second stone
    together with the record before it, or its opening stone."""

    opponent = 1 - facts.current_player
    recs = facts.records
    for ordinal in range(len(recs) - 1, -1, -1):
        if record_player(ordinal) != opponent:
            continue
        phase = record_phase(ordinal)
        if phase == PHASE_SECOND:
            prev = recs[ordinal - 1]
            cur = recs[ordinal]
            return [(prev[0], prev[1]), (cur[0], cur[1])]
        if phase == PHASE_OPENING:
            return [(recs[ordinal][0], recs[ordinal][1])]
    return []


def build_features(facts: PositionFacts, sup: Support) -> np.ndarray:
    """(N, 15) float32 planes in support node order (features.py:165-210)."""

    n = sup.num_nodes
    feats = np.zeros((n, NUM_FEATURES), dtype=np.float32)
    made = facts.placements_made
    for q, r, owner, placed in facts.records:
        row = sup.index[(q, r)]
        own = owner == facts.current_player
        feats[row, F_OWN_STONE if own else F_OPP_STONE] = 1.0
        plane = F_OWN_RECENCY if own else F_OPP_RECENCY
        recency = 1.0 / (1.0 + float(made - placed))
        if recency > feats[row, plane]:
            feats[row, plane] = recency
    feats[:, F_EMPTY] = 1.0 - feats[:, F_OWN_STONE] - feats[:, F_OPP_STONE]
    feats[: sup.legal_count, F_LEGAL] = 1.0
    if facts.phase == PHASE_SECOND:
        feats[:, F_PHASE_SECOND] = 1.0
        if facts.first_stone is not None:
            feats[sup.index[tuple(facts.first_stone)], F_FIRST_STONE] = 1.0
    if facts.current_player == 0:
        feats[:, F_PLAYER_COLOUR] = 1.0
    for cells, plane in (
        (facts.opp_hot, F_OPP_HOT),
        (facts.own_hot, F_OWN_HOT),
        (facts.opp_win, F_OPP_WIN_NOW),
        (facts.own_win, F_OWN_WIN_NOW),
    ):
        for cell in cells:
            feats[sup.index[tuple(cell)], plane] = 1.0
    feats[:, F_DIST_TO_STONE] = sup.dist.astype(np.float32) / DIST_SCALE
    for cell in opp_last_turn_cells(facts):
        feats[sup.index[cell], F_OPP_LAST_TURN] = 1.0
    return feats


def build_position(facts: PositionFacts, *, radius: int | None = None):
    """(Support, (N, 15) features) of one decision state."""

    sup = build_support(facts.stones(), radius=radius)
    return sup, build_features(facts, sup)
