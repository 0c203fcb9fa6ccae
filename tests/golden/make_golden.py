"""Write the golden fixtures of tests/golden/*.npz from the reference package.

Run in the build container only (the reference is not present on the GPU
box):  python tests/golden/make_golden.py

It imports the reference's own Python modules from
/root/reference/packages/{shrimp,hexfield_eq}/python, generates seeded
synthetic positions (its own generator below; facts via the reference's
window_scan), loads seeded weights from oracle.weights into the reference
ShrimpNet, and stores inputs and outputs of:

  support_features.npz  build_support / build_features        (support.py, features.py)
  forward_cfg0.npz      ShrimpNet(32, 4, "CCA").forward_policy_value, trunk   (model.py)
  forward_cfg4.npz      ShrimpNet(128, 8, "CCACCACCACCA").forward_policy_value
  pair.npz              _build_pair_u8 / _build_pair          (model.py:677-792)
  ray_index.npz         hexfield_eq _build_ray_gather_index_impl (_triton_ray.py:221-281)
  decode.npz            decode_binned_value / decode_moves_left, plan_groups
  evaluator_cfg0.npz    ShrimpEvaluator(net, "cpu") payload -> reply (inference.py)

Only data is stored (inputs and expected outputs); no reference source.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np

os.environ["SHRIMP_SUPPORT_RADIUS"] = "4"
REPO = Path(__file__).resolve().parents[2]
REF = Path("/root/reference/packages")
OUT = Path(__file__).resolve().parent
sys.path.insert(0, str(REF / "shrimp" / "python"))
sys.path.insert(0, str(REF / "hexfield_eq" / "python"))
sys.path.insert(0, str(REPO))

import torch  # noqa: E402

from oracle import weights as W  # noqa: E402
from shrimp import features as rfeat  # noqa: E402  (reference package)
from shrimp import support as rsup  # noqa: E402
from shrimp.batching import collate_rows  # noqa: E402
from shrimp.inference import ShrimpEvaluator, plan_groups  # noqa: E402
from shrimp.losses import decode_binned_value, decode_moves_left  # noqa: E402
from shrimp.model import ShrimpNet  # noqa: E402

DISK8 = sorted(
    (q, r) for q in range(-8, 9) for r in range(-8, 9) if max(abs(q), abs(r), abs(q + r)) <= 8
)
DISK5 = [(q, r) for q in range(-5, 6) for r in range(-5, 6) if max(abs(q), abs(r), abs(q + r)) <= 5]


def facts_of(stones, owners):
    k = len(stones)
    records = tuple((int(q), int(r), int(o), i) for i, ((q, r), o) in enumerate(zip(stones, owners)))
    player = rfeat.record_player(k)
    phase = rfeat.record_phase(k)
    first = (records[-1][0], records[-1][1]) if (phase == rfeat.PHASE_SECOND and k) else None
    oh, ph, ow, pw = rfeat.window_scan(records, player, k)
    return rfeat.PositionFacts(records, player, phase, first, oh, ph, ow, pw)


def draw_stones(rng, kmin, kmax, cap):
    while True:
        k = int(rng.integers(kmin, kmax + 1))
        covered, stones, skips = set(), [], 0
        for i in rng.permutation(len(DISK8)):
            if len(stones) == k:
                break
            q, r = DISK8[int(i)]
            grown = covered | {(q + a, r + b) for a, b in DISK5}
            if cap is not None and len(grown) > cap:
                skips += 1
                if skips >= 64:
                    break
                continue
            skips = 0
            covered = grown
            stones.append((q, r))
        if len(stones) >= kmin:
            return stones, rng.integers(0, 2, size=len(stones))


def gen_rows(seed, count, kmin, kmax, cap=256, radius=4):
    rng = np.random.Generator(np.random.PCG64(seed))
    rsup._SUPPORT_RADIUS = radius
    rsup._SUPPORT_HALO = radius + 1
    rows, facts = [], []
    for _ in range(count):
        stones, owners = draw_stones(rng, kmin, kmax, cap)
        f = facts_of(stones, owners)
        rows.append(rfeat.build_position(f))
        facts.append((stones, owners))
    rsup._SUPPORT_RADIUS = 4
    rsup._SUPPORT_HALO = 5
    return rows, facts


def ragged(arrs, dtype):
    lens = np.asarray([len(a) for a in arrs], dtype=np.int64)
    width = max(int(np.asarray(a).size // max(len(a), 1)) for a in arrs)
    flat = np.concatenate([np.asarray(a, dtype=dtype).reshape(len(a), width) for a in arrs])
    return flat, lens


def save_support(path):
    rows4, facts4 = gen_rows(101, 10, 10, 40)
    rows8, facts8 = gen_rows(102, 3, 3, 12, cap=None, radius=8)
    rows0, facts0 = gen_rows(103, 1, 0, 0, cap=None)  # no stones: origin support
    rows = rows4 + rows8 + rows0
    facts = facts4 + facts8 + facts0
    radius = np.asarray([4] * len(rows4) + [8] * len(rows8) + [4] * len(rows0))
    stones, n_st = ragged([np.asarray(s, np.int64).reshape(-1, 2) for s, _ in facts], np.int64)
    owners, _ = ragged([np.asarray(o, np.int64).reshape(-1, 1) for _, o in facts], np.int64)
    coords, n_nodes = ragged([s.coords for s, _ in rows], np.int64)
    nbr, _ = ragged([s.nbr for s, _ in rows], np.int64)
    dist, _ = ragged([s.dist.reshape(-1, 1) for s, _ in rows], np.int64)
    feats, _ = ragged([f for _, f in rows], np.float32)
    counts = np.asarray([[s.legal_count, s.stone_count, s.halo_count] for s, _ in rows])
    np.savez_compressed(
        path, radius=radius, stones=stones, n_stones=n_st, owners=owners.reshape(-1),
        coords=coords, n_nodes=n_nodes, nbr=nbr, dist=dist.reshape(-1), feats=feats,
        counts=counts,
    )


def net_with(sd, c, h, layout):
    net = ShrimpNet(channels=c, attention_heads=h, trunk_layout=layout).eval()
    net.load_state_dict(sd)
    return net


def save_forward(path, c, h, layout, seed_pos, count, kmax, wseed, with_fresh):
    rows, facts = gen_rows(seed_pos, count, 10, kmax)
    batch = collate_rows(rows, pad_to=256)
    args = (batch["feats"], batch["nbr"], batch["mask"], batch["coords"])
    out = {}
    for mode, ws in (("parity", wseed), ("fresh", wseed + 1), ("heads", wseed + 2)):
        if mode == "fresh" and not with_fresh:
            continue
        net = net_with(W.make_state_dict(c, h, layout, seed=ws, mode=mode), c, h, layout)
        with torch.no_grad():
            r = net.forward_policy_value(*args, request_moves_left=True)
            cells, tokens, _ = net.trunk(*args)
        for k, v in r.items():
            out[f"{mode}_{k}"] = v.numpy()
        out[f"{mode}_cells"] = cells.numpy()
        out[f"{mode}_tokens"] = tokens.numpy()
        out[f"{mode}_seed"] = np.asarray(ws)
    np.savez_compressed(
        path, feats=batch["feats"].numpy(), nbr=batch["nbr"].numpy(), mask=batch["mask"].numpy(),
        coords=batch["coords"].numpy(), legal=batch["legal_counts"].numpy(),
        arch=np.asarray([c, h]), layout=np.asarray(layout), **out,
    )
    return batch


def save_pair(path, batch):
    net = ShrimpNet(channels=32, attention_heads=4, trunk_layout="CCA")
    with torch.no_grad():
        pu8 = net._build_pair_u8(batch["coords"], batch["mask"])
        pl, key_pad = net._build_pair(batch["coords"][:2], batch["mask"][:2])
    np.savez_compressed(
        path, coords=batch["coords"].numpy(), mask=batch["mask"].numpy(), pair_u8=pu8.numpy(),
        pair_long=pl.numpy(), key_pad=key_pad.numpy(),
    )


def save_ray(path, batch):
    from hexfield_eq._triton_ray import _build_ray_gather_index_impl

    coords = batch["coords"].clone()
    mask = batch["mask"].clone()
    idx = _build_ray_gather_index_impl(coords, mask)
    np.savez_compressed(path, coords=coords.numpy(), mask=mask.numpy(), idx=idx.numpy())


def save_decode(path):
    rng = np.random.Generator(np.random.PCG64(7))
    logits = torch.from_numpy(rng.normal(0, 2.0, size=(16, 65)).astype(np.float32))
    logits[0] = 0.0
    logits[1] = -50.0
    logits[1, 64] = 50.0
    sizes = np.asarray(sorted(rng.integers(20, 600, size=60).tolist(), reverse=True))
    groups = np.asarray(plan_groups(sizes), dtype=np.int64)
    np.savez_compressed(
        path, logits=logits.numpy(), value=decode_binned_value(logits).numpy(),
        moves_left=decode_moves_left(logits).numpy(), sizes=sizes, groups=groups,
    )


def save_evaluator(path):
    from oracle.decode import build_payload

    rows_a, _ = gen_rows(201, 6, 10, 40)
    rows_b, _ = gen_rows(202, 6, 1, 6, cap=None)
    rows = rows_a + rows_b
    payload, order = build_payload(rows, request_moves_left=True, request_logits=True)
    sd = W.make_state_dict(32, 4, "CCA", seed=11, mode="parity")
    ev = ShrimpEvaluator(net_with(sd, 32, 4, "CCA"), "cpu")
    reply = ev.evaluate_payload(payload)
    np.savez_compressed(
        path,
        shape=np.asarray(payload["shape"]),
        node_feats=np.frombuffer(payload["node_feats"], np.uint8),
        node_qr=np.frombuffer(payload["node_qr"], np.uint8),
        node_row_offsets=np.asarray(payload["node_row_offsets"], np.int64),
        nbr=np.frombuffer(payload["nbr"], np.uint8),
        legal_counts=np.frombuffer(payload["legal_counts"], np.uint8),
        values=np.frombuffer(reply["values_bytes"], np.float32),
        priors=np.frombuffer(reply["priors_bytes"], np.float32),
        moves_left=np.frombuffer(reply["moves_left_bytes"], np.float32),
        priors_logits=np.frombuffer(reply["priors_logits_bytes"], np.float32),
        wseed=np.asarray(11),
    )


def main():
    torch.manual_seed(0)
    save_support(OUT / "support_features.npz")
    b0 = save_forward(OUT / "forward_cfg0.npz", 32, 4, "CCA", 301, 8, 40, 1, True)
    save_forward(OUT / "forward_cfg4.npz", 128, 8, "CCACCACCACCA", 302, 2, 80, 3, False)
    save_pair(OUT / "pair.npz", b0)
    save_ray(OUT / "ray_index.npz", b0)
    save_decode(OUT / "decode.npz")
    save_evaluator(OUT / "evaluator_cfg0.npz")
    for p in sorted(OUT.glob("*.npz")):
        print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()
