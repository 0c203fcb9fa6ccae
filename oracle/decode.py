"""Serve decode and ABI-1 evaluator restated on the CPU (test infrastructure).

- ``decode_value`` / ``decode_moves_left``: losses.py:40-60
- ``plan_groups``: inference.py:201-223
- ``build_payload``: the Rust payload builder payload.rs:53-160 (rows sorted by
  support size descending, stable; f16 features, i16 coords, u16 nbr with
  0xFFFF)
- ``evaluate``: ShrimpEvaluator on the CPU (inference.py:509-604, 865-892,
  998-1042, 806-863) around ``forward.forward_policy_value``.
"""

from __future__ import annotations

import numpy as np
import torch

from . import forward as fwd

VALUE_BINS = 65
MOVES_LEFT_CAP = 209
NUM_FEATURES = 15
NUM_TOKENS = 8
QUANT_NODES = 64


def value_bins(dtype=torch.float64) -> torch.Tensor:
    return torch.linspace(-1.0, 1.0, VALUE_BINS, dtype=dtype)


def decode_value(logits: torch.Tensor) -> torch.Tensor:
    p = torch.softmax(logits, dim=-1)
    return (p * value_bins(logits.dtype)).sum(-1).clamp(-1.0, 1.0)


def decode_moves_left(logits: torch.Tensor) -> torch.Tensor:
    return (decode_value(logits) + 1.0) * 0.5 * MOVES_LEFT_CAP


def plan_groups(sizes, pair_ceiling=3.8e7, waste_fraction=0.18) -> list:
    groups = []
    n = len(sizes)
    i = 0
    while i < n:
        pad = max(QUANT_NODES, -(-int(sizes[i]) // QUANT_NODES) * QUANT_NODES)
        floor = pad - max(QUANT_NODES, int(waste_fraction * pad))
        j = i + 1
        while j < n and (j - i + 1) * (pad + NUM_TOKENS) ** 2 <= pair_ceiling and int(sizes[j]) >= floor:
            j += 1
        groups.append((i, j, pad))
        i = j
    return groups


def build_payload(rows: list, request_moves_left=False, request_logits=False) -> tuple:
    """rows: list of (Support, feats f32 (N, 15)) in request order. Returns
    (payload, order) where order[k] is the request index of payload row k."""

    order = sorted(range(len(rows)), key=lambda i: (-rows[i][0].num_nodes, i))
    feats, qr, nbr, offs, legal = [], [], [], [0], []
    for i in order:
        sup, f = rows[i]
        feats.append(f.astype(np.float16))
        qr.append(sup.coords.astype(np.int16))
        nb = sup.nbr.astype(np.int64)
        nbr.append(np.where(nb < 0, 0xFFFF, nb).astype(np.uint16))
        offs.append(offs[-1] + sup.num_nodes)
        legal.append(sup.legal_count)
    payload = {
        "abi": 1,
        "shape": (len(rows), offs[-1]),
        "node_feats": np.concatenate(feats).tobytes(),
        "node_qr": np.concatenate(qr).tobytes(),
        "node_row_offsets": offs,
        "nbr": np.concatenate(nbr).tobytes(),
        "legal_counts": np.asarray(legal, dtype=np.int32).tobytes(),
        "request_moves_left": request_moves_left,
        "request_logits": request_logits,
    }
    return payload, order


def evaluate(payload: dict, sd: dict, layout: str, heads: int, dtype=torch.float64) -> dict:
    """Reply dict of the CPU evaluator (fp32 features, the reference CPU path)."""

    b, total = (int(x) for x in payload["shape"])
    offs = np.asarray(payload["node_row_offsets"], dtype=np.int64)
    legal = np.frombuffer(payload["legal_counts"], dtype=np.int32)
    feats = np.frombuffer(payload["node_feats"], dtype=np.float16).reshape(total, NUM_FEATURES)
    qr = np.frombuffer(payload["node_qr"], dtype=np.int16).reshape(total, 2)
    nbr = np.frombuffer(payload["nbr"], dtype=np.uint16).reshape(total, 6)
    ml_req = bool(payload.get("request_moves_left", False))
    lg_req = bool(payload.get("request_logits", False))
    sizes = offs[1:] - offs[:-1]
    values, mls, priors, logits = [], [], [], []
    for s, e, pad in plan_groups(sizes):
        g = e - s
        pf = np.zeros((g, pad, NUM_FEATURES), np.float32)
        pn = np.full((g, pad, 6), pad, np.int64)
        pm = np.zeros((g, pad), bool)
        pc = np.zeros((g, pad, 2), np.int64)
        for k in range(g):
            o, n = int(offs[s + k]), int(sizes[s + k])
            pf[k, :n] = feats[o:o + n].astype(np.float32)
            rn = nbr[o:o + n].astype(np.int64)
            pn[k, :n] = np.where(rn == 0xFFFF, pad, rn)
            pm[k, :n] = True
            pc[k, :n] = qr[o:o + n]
        out = fwd.forward_policy_value(sd, layout, heads, pf, pn, pm, pc,
                                       request_moves_left=ml_req, dtype=dtype)
        values.append(decode_value(out["value"]))
        if ml_req:
            mls.append(decode_moves_left(out["moves_left"]))
        for k in range(g):
            lc = int(legal[s + k])
            row = out["policy"][k, :lc]
            priors.append(torch.softmax(row, dim=0))
            logits.append(row)
    reply = {
        "values_bytes": torch.cat(values).to(torch.float32).numpy().tobytes(),
        "priors_bytes": torch.cat(priors).to(torch.float32).numpy().tobytes(),
    }
    if ml_req:
        reply["moves_left_bytes"] = torch.cat(mls).to(torch.float32).numpy().tobytes()
    if lg_req:
        reply["priors_logits_bytes"] = torch.cat(logits).to(torch.float32).numpy().tobytes()
    return reply
