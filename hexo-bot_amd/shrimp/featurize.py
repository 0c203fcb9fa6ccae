"""Featurizer on the device: decision states -> padded forward inputs.

The device counterpart of ``build_position`` + ``collate_rows``
(``support.py:84-205``, ``features.py:80-240``, ``batching.py:45-80``; the
reference's production featurizer is Rust, ``support.rs:52`` /
``features.rs:19``). One workgroup per position builds the support (BFS to
radius R + 1), the [legal | stones | halo] node order, the neighbour table and
the 15 planes, including the single-colour window scan for hot / win-now
cells, and writes the padded batch the forward consumes. Only the placement
records travel to the device (8 bytes per stone instead of 30 bytes per
support node).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .features import PHASE_FIRST, PHASE_OPENING, PHASE_SECOND
from .support import SUPPORT_RADIUS

_PHASES = {PHASE_OPENING: 0, PHASE_FIRST: 1, PHASE_SECOND: 2}

STATUS_OK, STATUS_TOO_WIDE, STATUS_NPAD = 0, 2, 3


def pack_records(facts: list) -> dict:
    """CSR arrays of a list of ``PositionFacts``: records (q, r, owner,
    placement index) in order, offsets, side to move and phase."""

    n = [len(f.records) for f in facts]
    offs = np.zeros(len(facts) + 1, dtype=np.int64)
    offs[1:] = np.cumsum(n)
    rec = np.zeros((int(offs[-1]), 4), dtype=np.int64)
    for i, f in enumerate(facts):
        if f.records:
            rec[offs[i]:offs[i + 1]] = np.asarray(f.records, dtype=np.int64)
    return {
        "qr": rec[:, :2].astype(np.int32),
        "owner": rec[:, 2].astype(np.uint8),
        "index": rec[:, 3].astype(np.int32),
        "offsets": offs,
        "player": np.asarray([f.current_player for f in facts], dtype=np.uint8),
        "phase": np.asarray([_PHASES[f.phase] for f in facts], dtype=np.uint8),
    }


def featurize(facts: list, *, radius: int | None = None, npad: int | None = None,
              device="cuda", check: bool = True) -> dict:
    """Padded batch of ``facts`` built on ``device``: feats (B, Npad, 15) f32,
    nbr (B, Npad, 6) int32 (absent = Npad), mask (B, Npad) bool, coords
    (B, Npad, 2) int32, legal_counts (B,), counts (B, 4) = nodes / legal /
    stones / halo, status (B,). ``npad`` None picks the smallest multiple of 64
    that holds every position (one counting pass first). With ``check`` a
    non-zero status raises ValueError."""

    rad = SUPPORT_RADIUS if radius is None else int(radius)
    b = len(facts)
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("featurize runs on a ROCm device")
    pk = pack_records(facts)
    t = {k: torch.from_numpy(v).to(dev) for k, v in pk.items()}
    counts = torch.zeros((b, 4), dtype=torch.int32, device=dev)
    status = torch.zeros((b,), dtype=torch.int32, device=dev)
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    p = lambda x: None if x is None else x.data_ptr()

    def run(n, outs):
        _lib.check(lib.shrimp_featurize(
            p(t["qr"]) if t["qr"].numel() else None, p(t["owner"]) if t["owner"].numel() else None,
            p(t["index"]) if t["index"].numel() else None, p(t["offsets"]), p(t["player"]),
            p(t["phase"]), b, rad, n, *[p(o) for o in outs], p(counts), p(status), st),
            "featurize")

    if npad is None:
        run(0, (None, None, None, None))
        most = int(counts[:, 0].max().item()) if b else 0
        npad = max(64, -(-most // 64) * 64)
    feats = torch.empty((b, npad, 15), dtype=torch.float32, device=dev)
    nbr = torch.empty((b, npad, 6), dtype=torch.int32, device=dev)
    mask = torch.empty((b, npad), dtype=torch.uint8, device=dev)
    coords = torch.empty((b, npad, 2), dtype=torch.int32, device=dev)
    run(npad, (feats, nbr, mask, coords))
    if check and b and int(status.max().item()) != STATUS_OK:
        bad = torch.nonzero(status).flatten().tolist()
        raise ValueError(f"featurize: positions {bad[:8]} returned status "
                         f"{status[bad[0]].item()} (2: support wider than the device window, "
                         f"3: more nodes than npad={npad})")
    return {
        "feats": feats, "nbr": nbr, "mask": mask.bool(), "coords": coords,
        "legal_counts": counts[:, 1].long(), "counts": counts, "status": status,
    }
