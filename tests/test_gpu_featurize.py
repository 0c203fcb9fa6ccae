"""Device featurizer (shrimp_featurize) against the reference's featurizer
goldens and the host builder (support.py / features.py restated in
shrimp.support / shrimp.features, collated by shrimp.batching). Everything is
integer or exactly rounded, so every comparison is bit-exact."""

import numpy as np
import pytest
import torch

from shrimp import features
from shrimp.batching import collate_rows
from shrimp.featurize import STATUS_NPAD, STATUS_OK, STATUS_TOO_WIDE, featurize
from shrimp.synthetic import facts_from_stones, positions

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _host(facts, radius, npad=None):
    rows = [features.build_position(f, radius=radius) for f in facts]
    if npad is None:
        npad = max(64, -(-max(s.num_nodes for s, _ in rows) // 64) * 64)
    return collate_rows(rows, pad_to=npad), rows


def _same(dev, host, what):
    npad = host["feats"].shape[1]
    assert torch.equal(dev["mask"].cpu(), host["mask"]), what
    assert torch.equal(dev["coords"].cpu().long(), host["coords"]), what
    assert torch.equal(dev["nbr"].cpu().long(), host["nbr"]), what
    assert torch.equal(dev["legal_counts"].cpu(), host["legal_counts"]), what
    assert torch.equal(dev["feats"].cpu(), host["feats"]), what
    assert (dev["status"].cpu() == STATUS_OK).all(), what
    assert npad == dev["feats"].shape[1]


def test_featurize_matches_reference_golden(golden):
    """The 14 positions the reference featurizer wrote (radius 4 and 8)."""

    g = golden("support_features")
    so = np.concatenate([[0], np.cumsum(g["n_stones"])])
    no = np.concatenate([[0], np.cumsum(g["n_nodes"])])
    for radius in sorted(set(g["radius"].tolist())):
        idx = [p for p in range(len(g["radius"])) if g["radius"][p] == radius]
        facts = [facts_from_stones([tuple(s) for s in g["stones"][so[p]:so[p + 1]].tolist()],
                                   g["owners"][so[p]:so[p + 1]]) for p in idx]
        out = featurize(facts, radius=int(radius), device=DEV)
        for k, p in enumerate(idx):
            n = int(g["n_nodes"][p])
            sl = slice(no[p], no[p + 1])
            assert out["counts"][k, 0].item() == n
            assert out["counts"][k, 1:].cpu().tolist() == g["counts"][p].tolist()
            np.testing.assert_array_equal(out["coords"][k, :n].cpu().numpy(), g["coords"][sl])
            nbr = out["nbr"][k, :n].cpu().numpy().astype(np.int64)
            npad = out["nbr"].shape[1]
            np.testing.assert_array_equal(np.where(nbr == npad, -1, nbr), g["nbr"][sl])
            np.testing.assert_array_equal(out["feats"][k, :n].cpu().numpy(), g["feats"][sl])
            np.testing.assert_array_equal(out["feats"][k, :n, 11].cpu().numpy() * 8.0,
                                          g["dist"][sl].astype(np.float32))


@pytest.mark.parametrize("name,count", [("cfg4", 96), ("cfg0", 64)])
def test_featurize_matches_host_builder(name, count):
    """Generated decision states (10-80 stones, both phases and colours to
    move) against build_position + collate_rows, at the generator's Npad."""

    rows = positions(name, count, seed=31)
    facts = [f for f, _, _ in rows]
    npad = max(64, -(-max(s.num_nodes for _, s, _ in rows) // 64) * 64)
    host, _ = _host(facts, None, npad)
    dev = featurize(facts, npad=npad, device=DEV)
    _same(dev, host, name)


def test_featurize_small_and_edge_positions():
    """No stones (origin + 6 neighbours), one stone, a straight five (win-now
    cells), hot windows past 7 placements, both radius settings."""

    cases = [
        [],
        [(0, 0)],
        [(0, 0), (3, -1)],
        [(i, 0) for i in range(5)] + [(0, 3), (1, 3), (2, 3)],
        [(i, 0) for i in range(4)] + [(0, 2), (1, 2), (2, 2), (5, -3), (6, -3)],
        [(q, r) for q in range(-2, 3) for r in range(-2, 3) if abs(q + r) <= 2],
    ]
    facts = []
    for stones in cases:
        owners = [features.record_player(i) for i in range(len(stones))]
        facts.append(facts_from_stones(stones, owners))
    for radius in (8, 4, 2):
        host, _ = _host(facts, radius)
        dev = featurize(facts, radius=radius, npad=host["feats"].shape[1], device=DEV)
        _same(dev, host, f"edge cases radius {radius}")


def test_featurize_status_codes():
    """A support wider than the device window and an Npad smaller than the
    support are reported per position, with the other positions intact."""

    near = facts_from_stones([(0, 0), (1, 0), (0, 1)], [0, 1, 1])
    wide = facts_from_stones([(0, 0), (70, 0), (0, 1)], [0, 1, 1])
    host, _ = _host([near], None)
    npad = host["feats"].shape[1]
    out = featurize([near, wide, near], npad=npad, device=DEV, check=False)
    assert out["status"].cpu().tolist() == [STATUS_OK, STATUS_TOO_WIDE, STATUS_OK]
    assert not out["mask"][1].any()
    assert torch.equal(out["feats"][0].cpu(), host["feats"][0])
    assert torch.equal(out["nbr"][2].cpu().long(), host["nbr"][0])
    small = featurize([near], npad=64, device=DEV, check=False)
    assert small["status"].item() == STATUS_NPAD
    with pytest.raises(ValueError):
        featurize([near, wide], npad=npad, device=DEV)


def test_forward_from_device_features():
    """The forward on device-built inputs equals the forward on host-built
    ones (same values, int32 neighbour rows)."""

    from oracle import weights
    from shrimp.model import ShrimpNet

    layout = "CCACCACCACCA"
    net = ShrimpNet(channels=128, attention_heads=8, trunk_layout=layout)
    net.load_state_dict(weights.make_state_dict(128, 8, layout, seed=5))
    net = net.to(DEV).eval()
    rows = positions("cfg4", 24, seed=5)
    facts = [f for f, _, _ in rows]
    host, _ = _host(facts, None, 256)
    dev = featurize(facts, npad=256, device=DEV)
    assert torch.equal(dev["feats"].cpu(), host["feats"])
    a = net.forward_policy_value(host["feats"].to(DEV), host["nbr"].to(DEV),
                                 host["mask"].to(DEV), host["coords"].to(DEV))
    b = net.forward_policy_value(dev["feats"], dev["nbr"], dev["mask"], dev["coords"])
    for key in ("policy", "value"):
        assert torch.equal(a[key], b[key]), key
