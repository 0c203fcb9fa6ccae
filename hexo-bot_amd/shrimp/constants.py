"""Shrimp constants: feature plane indices, hex geometry radii, bias-row layout.

Values are the interface shared with the caller side (Rust featurizer, wire
ABI, checkpoints), so they match the reference one for one:
``packages/shrimp/python/shrimp/constants.py:15-126``.

Architecture knobs are read once from the environment at import, under the
reference's names (``SHRIMP_CHANNELS``, ``SHRIMP_ATTENTION_HEADS``,
``SHRIMP_TRUNK``); ``ShrimpNet`` also takes them as explicit arguments.
"""

from __future__ import annotations

import os

# Engine geometry (constants.py:15-16): legality radius and the halo shell.
LEGAL_RADIUS = 8
HALO_DIST = LEGAL_RADIUS + 1

# Tap order for the 6 neighbour taps (constants.py:20-27): the rot60 orbit of
# (1, 0). Tap 0 of every hex conv is the cell itself; taps 1..6 follow this.
DIRECTIONS: tuple[tuple[int, int], ...] = (
    (1, 0),
    (0, 1),
    (-1, 1),
    (-1, 0),
    (0, -1),
    (1, -1),
)

# Packed action id offset (constants.py:32).
COORD_OFFSET = 1 << 15

# u16 wire sentinel for a missing neighbour (constants.py:36).
NBR_SENTINEL_U16 = 0xFFFF

# Feature planes (constants.py:41-56).
F_OWN_STONE = 0
F_OPP_STONE = 1
F_EMPTY = 2
F_LEGAL = 3
F_PHASE_SECOND = 4
F_FIRST_STONE = 5
F_PLAYER_COLOUR = 6
F_OWN_RECENCY = 7
F_OPP_RECENCY = 8
F_OPP_HOT = 9
F_OWN_HOT = 10
F_DIST_TO_STONE = 11
F_OPP_LAST_TURN = 12
F_OPP_WIN_NOW = 13
F_OWN_WIN_NOW = 14
NUM_FEATURES = 15

# Window-scan thresholds (constants.py:63-66).
HOT_MIN_COUNT = 4
WIN_NOW_COUNT = 5
HOT_MIN_PLACEMENTS = 7
WINDOW_LEN = 6

# dist_to_stone scaling (constants.py:70-71).
DIST_SCALE = float(LEGAL_RADIUS)
HALO_DIST_FEATURE = HALO_DIST / DIST_SCALE

# Heads (constants.py:74-75).
VALUE_BINS = 65
MOVES_LEFT_CAP = 209


def _env_text(name: str, default: str) -> str:
    raw = os.environ.get(name, "").strip()
    return raw or default


# Trunk shape (constants.py:81-108), read once at import.
CHANNELS = int(_env_text("SHRIMP_CHANNELS", "96"))
NUM_TOKENS = 8
ATTENTION_HEADS = int(_env_text("SHRIMP_ATTENTION_HEADS", "4"))
if CHANNELS % ATTENTION_HEADS:
    raise ValueError(
        f"SHRIMP_CHANNELS={CHANNELS} not divisible by "
        f"SHRIMP_ATTENTION_HEADS={ATTENTION_HEADS}"
    )
HEAD_DIM = CHANNELS // ATTENTION_HEADS
MLP_RATIO = 2
TRUNK_LAYOUT = _env_text("SHRIMP_TRUNK", "CCCACCCACCA")


def validate_layout(layout: str) -> str:
    """A trunk layout is a non-empty C/A string ending in 'A' (the final
    LayerNorm reads the joint sequence the last attention block produced)."""

    if not layout or set(layout) - {"C", "A"} or not layout.endswith("A"):
        raise ValueError(
            f"SHRIMP_TRUNK={layout!r} must be a non-empty string of "
            "'C'/'A' ending with 'A'"
        )
    return layout


validate_layout(TRUNK_LAYOUT)

# Relative-position bias rows (constants.py:116-126).
BIAS_DISK_RADIUS = LEGAL_RADIUS
BIAS_EXACT_ROWS = 217
BIAS_RING_MIN = 9
BIAS_RING_MAX = 16
BIAS_ON_AXIS_BASE = 217
BIAS_OFF_AXIS_BASE = 225
BIAS_FAR_ROW = 233
BIAS_CELL_TOKEN_ROW = 234
BIAS_TOKEN_CELL_ROW = 235
BIAS_TOKEN_TOKEN_ROW = 236
BIAS_ROWS = 237

# Additive fill for padded key columns (model.py:53); finite in fp16/bf16.
PAD_KEY_MASK_VALUE = -3.0e4
