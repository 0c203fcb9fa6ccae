"""Seeded synthetic positions and operator inputs for the benchmark configs.

There is no engine or dataset on the MI355X box, so positions are generated
from a numpy PCG64 stream (seed 20261201 + config index):

- stones are distinct cells of the 217-cell radius-8 disk drawn in random
  placement order with independent Bernoulli(1/2) owners; the side to move,
  phase and first stone follow the turn structure (features.record_player /
  record_phase) and hot / win cells come from ``features.window_scan``;
- support radius 4 (legal <= 4, halo 5), so N = |union of radius-5 disks|;
- "l256" variant: stones are inserted in their random order and any stone
  that would push N past 256 is skipped (stop after 64 consecutive skips);
  positions ending with fewer than ``kmin`` stones are redrawn; batches are
  padded to Npad = 256;
- "spec" variant: all k drawn stones, Npad = ceil64(max N).

Config shapes (k ranges per config): cfg0 10-40 stones, cfg4 10-80 stones.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .batching import collate_rows
from .constants import LEGAL_RADIUS
from .features import (
    PHASE_SECOND,
    PositionFacts,
    build_position,
    record_phase,
    record_player,
    window_scan,
)
from .geometry import disk_offsets

SEED_BASE = 20261201
SUPPORT_RADIUS_CFG = 4
DISK = disk_offsets(LEGAL_RADIUS)
_HALO_DISK = disk_offsets(SUPPORT_RADIUS_CFG + 1)


@dataclass(frozen=True)
class PositionSpec:
    kmin: int
    kmax: int
    variant: str = "l256"
    cap: int = 256
    radius: int = SUPPORT_RADIUS_CFG


CONFIGS = {
    "cfg0": PositionSpec(10, 40),
    "cfg1": PositionSpec(10, 40),
    "cfg2": PositionSpec(10, 40),
    "cfg3": PositionSpec(10, 40),
    "cfg4": PositionSpec(10, 80),
    "cfg4_spec": PositionSpec(10, 80, variant="spec"),
}


def config_seed(name: str) -> int:
    return SEED_BASE + int(name[3])


def facts_from_stones(stones: list, owners) -> PositionFacts:
    k = len(stones)
    records = tuple((int(q), int(r), int(o), i) for i, ((q, r), o) in enumerate(zip(stones, owners)))
    player = record_player(k)
    phase = record_phase(k)
    first = (records[-1][0], records[-1][1]) if (phase == PHASE_SECOND and k > 0) else None
    own_hot, opp_hot, own_win, opp_win = window_scan(records, player, k)
    return PositionFacts(
        records=records, current_player=player, phase=phase, first_stone=first,
        own_hot=own_hot, opp_hot=opp_hot, own_win=own_win, opp_win=opp_win,
    )


def _cover(cell) -> set:
    q, r = cell
    return {(q + dq, r + dr) for dq, dr in _HALO_DISK}


def draw_facts(rng: np.random.Generator, spec: PositionSpec) -> PositionFacts:
    while True:
        k = int(rng.integers(spec.kmin, spec.kmax + 1))
        order = rng.permutation(len(DISK))
        if spec.variant == "spec":
            stones = [DISK[i] for i in order[:k]]
        else:
            covered: set = set()
            stones = []
            skips = 0
            for i in order:
                if len(stones) == k:
                    break
                cell = DISK[int(i)]
                grown = covered | _cover(cell)
                if len(grown) > spec.cap:
                    skips += 1
                    if skips >= 64:
                        break
                    continue
                skips = 0
                covered = grown
                stones.append(cell)
        if len(stones) >= spec.kmin:
            owners = rng.integers(0, 2, size=len(stones))
            return facts_from_stones(stones, owners)


def positions(name: str, count: int, seed: int | None = None) -> list:
    """``count`` (facts, Support, features) triples of config ``name``."""

    spec = CONFIGS[name]
    rng = np.random.Generator(np.random.PCG64(config_seed(name) if seed is None else seed))
    out = []
    for _ in range(count):
        facts = draw_facts(rng, spec)
        sup, feats = build_position(facts, radius=spec.radius)
        out.append((facts, sup, feats))
    return out


def position_batch(name: str, count: int, seed: int | None = None) -> dict:
    """Collated CPU batch (feats/nbr/mask/coords/legal_counts) plus the raw
    rows under ``rows``."""

    spec = CONFIGS[name]
    rows = positions(name, count, seed)
    if spec.variant == "spec":
        npad = max(64, -(-max(s.num_nodes for _, s, _ in rows) // 64) * 64)
    else:
        npad = spec.cap
    batch = collate_rows([(s, f) for _, s, f in rows], pad_to=npad)
    batch["rows"] = rows
    return batch


def serve_payload(name: str, count: int, seed: int | None = None, *,
                  request_moves_left: bool = False, request_logits: bool = False) -> tuple:
    """ABI-1 evaluator payload of ``count`` positions of config ``name``, built
    as the Rust bridge builds it (``packages/shrimp/rust/src/payload.rs:108-160``):
    rows sorted by support size, descending (ties in request order), f16
    features, i16 coordinates, u16 row-local neighbour ids with 0xFFFF for
    absent. Returns (payload, order): order[k] is the request index of row k."""

    rows = positions(name, count, seed)
    order = sorted(range(count), key=lambda i: (-rows[i][1].num_nodes, i))
    feats, qr, nbr, offs, legal = [], [], [], [0], []
    for i in order:
        _, sup, f = rows[i]
        feats.append(np.asarray(f, dtype=np.float16))
        qr.append(np.asarray(sup.coords, dtype=np.int16))
        nb = np.asarray(sup.nbr, dtype=np.int64)
        nbr.append(np.where(nb < 0, 0xFFFF, nb).astype(np.uint16))
        offs.append(offs[-1] + sup.num_nodes)
        legal.append(sup.legal_count)
    payload = {
        "abi": 1,
        "shape": (count, offs[-1]),
        "node_feats": np.concatenate(feats).tobytes(),
        "node_qr": np.concatenate(qr).tobytes(),
        "node_row_offsets": offs,
        "nbr": np.concatenate(nbr).tobytes(),
        "legal_counts": np.asarray(legal, dtype=np.int32).tobytes(),
        "request_moves_left": request_moves_left,
        "request_logits": request_logits,
    }
    return payload, order


# ---- operator-level inputs (configs 1-3) -------------------------------------------


def conv_inputs(count: int, channels: int = 128, seed: int | None = None, taps: int = 7) -> dict:
    """Config 1: x ~ N(0,1), W ~ N(0, 1/(taps*C)), bias ~ N(0, 0.02), over the
    cell sets of l256 positions (Npad 256)."""

    batch = position_batch("cfg1", count, seed)
    rng = np.random.Generator(np.random.PCG64((config_seed("cfg1") if seed is None else seed) + 7))
    b, n = batch["mask"].shape
    x = rng.standard_normal((b, n, channels), dtype=np.float32)
    w = (rng.standard_normal((taps, channels, channels), dtype=np.float32)
         / np.float32(np.sqrt(taps * channels)))
    bias = (rng.standard_normal(channels, dtype=np.float32) * np.float32(0.02))
    return {"batch": batch, "x": x, "w": w, "bias": bias}


def attention_inputs(count: int, heads: int = 8, d: int = 16, seed: int | None = None) -> dict:
    """Config 2: valid lengths n_b ~ U{64..256}; coords = first n_b cells of an
    l256 position; q, k, v ~ N(0,1) (B, H, 256, d); per-head 33x33 bias table
    ~ N(0, 0.5) over (dq, dr) clamped to [-16, 16]; no summary tokens."""

    batch = position_batch("cfg2", count, seed)
    rng = np.random.Generator(np.random.PCG64((config_seed("cfg2") if seed is None else seed) + 7))
    b, n = batch["mask"].shape
    lens = np.minimum(rng.integers(64, 257, size=b), batch["mask"].sum(1).numpy())
    mask = np.arange(n)[None, :] < lens[:, None]
    coords = batch["coords"].numpy() * mask[..., None]
    q = rng.standard_normal((b, heads, n, d), dtype=np.float32)
    k = rng.standard_normal((b, heads, n, d), dtype=np.float32)
    v = rng.standard_normal((b, heads, n, d), dtype=np.float32)
    table = rng.standard_normal((33 * 33, heads), dtype=np.float32) * np.float32(np.sqrt(0.5))
    return {"q": q, "k": k, "v": v, "coords": coords.astype(np.int32), "mask": mask,
            "lens": lens.astype(np.int32), "table": table}


def raytap_inputs(count: int, channels: int = 128, seed: int | None = None) -> dict:
    """Config 3: l256 cell sets, x ~ N(0,1), 31 independent tap weights
    W_s ~ N(0, 1/(31*C)), bias ~ N(0, 0.02)."""

    batch = position_batch("cfg3", count, seed)
    rng = np.random.Generator(np.random.PCG64((config_seed("cfg3") if seed is None else seed) + 7))
    b, n = batch["mask"].shape
    x = rng.standard_normal((b, n, channels), dtype=np.float32)
    w = (rng.standard_normal((31, channels, channels), dtype=np.float32)
         / np.float32(np.sqrt(31 * channels)))
    bias = rng.standard_normal(channels, dtype=np.float32) * np.float32(0.02)
    return {"batch": batch, "x": x, "w": w, "bias": bias}
