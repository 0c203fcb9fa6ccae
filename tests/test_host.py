"""Host-side shrimp modules against the reference's golden outputs and the
reference tests' invariants (tests/test_shrimp_geometry.py,
tests/test_shrimp_support.py)."""

import random

import numpy as np
import pytest
import torch

from shrimp import constants as C
from shrimp import features, geometry, support
from shrimp.batching import collate_rows
from shrimp.inference import plan_groups

from oracle import tables


def _facts(stones, owners):
    from shrimp.synthetic import facts_from_stones

    return facts_from_stones([tuple(s) for s in stones], owners)


def test_support_and_features_match_reference(golden):
    g = golden("support_features")
    so = np.concatenate([[0], np.cumsum(g["n_stones"])])
    no = np.concatenate([[0], np.cumsum(g["n_nodes"])])
    for p in range(len(g["n_stones"])):
        stones = g["stones"][so[p]:so[p + 1]].tolist()
        owners = g["owners"][so[p]:so[p + 1]]
        facts = _facts(stones, owners)
        sup, feats = features.build_position(facts, radius=int(g["radius"][p]))
        sl = slice(no[p], no[p + 1])
        np.testing.assert_array_equal(sup.coords, g["coords"][sl])
        np.testing.assert_array_equal(sup.nbr, g["nbr"][sl])
        np.testing.assert_array_equal(sup.dist, g["dist"][sl])
        assert [sup.legal_count, sup.stone_count, sup.halo_count] == g["counts"][p].tolist()
        np.testing.assert_array_equal(feats, g["feats"][sl])


def test_geometry_invariants():
    rng = random.Random(13)
    for _ in range(500):
        dq, dr = rng.randint(-30, 30), rng.randint(-30, 30)
        assert geometry.hex_dist(dq, dr) == (abs(dq) + abs(dr) + abs(dq + dr)) // 2
        assert geometry.rel_bias_index(dq, dr) == tables.rel_bias_row(dq, dr)
        for sym in range(12):
            tq, tr = geometry.apply_d6(sym, dq, dr)
            assert geometry.apply_d6(geometry.d6_inverse(sym), tq, tr) == (dq, dr)
            assert geometry.hex_dist(tq, tr) == geometry.hex_dist(dq, dr)
    d = C.DIRECTIONS
    for i in range(6):
        assert geometry.rot60(*d[i]) == d[(i + 1) % 6]
        assert geometry.reflect(*d[i]) == d[5 - i]
    for _ in range(200):
        q, r = rng.randint(-2000, 2000), rng.randint(-2000, 2000)
        assert geometry.unpack_action_id(geometry.pack_action_id(q, r)) == (q, r)
    np.testing.assert_array_equal(geometry.cell_bias_lut(), tables.cell_lut())


def test_support_invariants():
    sup = support.build_support([])
    assert sup.num_nodes == 7 and sup.legal_count == 1
    rng = random.Random(3)
    stones = list({(rng.randint(-6, 6), rng.randint(-6, 6)) for _ in range(15)})
    sup = support.build_support(stones, radius=4)
    n = sup.num_nodes
    for i in range(n):
        for k in range(6):
            j = sup.nbr[i, k]
            if j >= 0:
                assert sup.nbr[j, (k + 3) % 6] == i
    lg, st, ha = sup.segments()
    for seg in (lg, st, ha):
        rows = [tuple(sup.coords[i]) for i in seg]
        assert rows == sorted(rows)
    assert all(sup.dist[i] == 5 for i in ha)
    with pytest.raises(support.SupportContractError):
        support.build_support(stones, radius=4, expected_legal=[(100, 100)])


def test_collate_pad_conventions():
    rows = [features.build_position(_facts([(0, 0), (1, 0)], [0, 1]), radius=4)]
    batch = collate_rows(rows, pad_to=128)
    n = rows[0][0].num_nodes
    assert batch["feats"].shape == (1, 128, 15)
    assert (batch["nbr"][0, n:] == 128).all()
    assert (batch["nbr"][0, :n] <= 128).all()
    assert batch["mask"][0, :n].all() and not batch["mask"][0, n:].any()
    with pytest.raises(ValueError):
        collate_rows(rows, pad_to=n - 1)


def test_plan_groups_matches_reference(golden):
    g = golden("decode")
    assert plan_groups(g["sizes"]) == [tuple(x) for x in g["groups"].tolist()]


def test_group_stream_assignment():
    """Groups go in order to the stream with the least work so far."""

    from shrimp.inference import assign_group_streams

    assert assign_group_streams([5, 5, 4, 3, 1], 2) == [0, 1, 0, 1, 1]
    assert assign_group_streams([9, 1, 1, 1], 2) == [0, 1, 1, 1]
    assert assign_group_streams([3, 2, 1], 1) == [0, 0, 0]
    assert assign_group_streams([], 2) == []


def test_synthetic_l256_generator():
    from shrimp import synthetic

    batch = synthetic.position_batch("cfg4", 24)
    assert batch["feats"].shape == (24, 256, 15)
    for facts, sup, _ in batch["rows"]:
        assert sup.num_nodes <= 256
        assert len(facts.records) >= 10
    again = synthetic.position_batch("cfg4", 24)
    assert np.array_equal(batch["feats"].numpy(), again["feats"].numpy())
    spec = synthetic.position_batch("cfg4_spec", 4)
    assert spec["feats"].shape[1] % 64 == 0 and spec["feats"].shape[1] > 256


def test_row_launches_refuse_mismatched_strides():
    """Row kernels address rows by the strides they are given; the launch
    wrappers refuse a tensor whose layout disagrees (a compact clone of a
    strided view, a short buffer) before anything reaches the device."""

    from shrimp import ops

    seq = torch.empty(4, 264, 128, dtype=torch.bfloat16)
    cells = seq[:, 8:]
    ops._check_rows("ok", cells, 264 * 128, 128, 4, 256, 128)
    with pytest.raises(ValueError, match="strides"):
        ops._check_rows("clone", cells.clone(), 264 * 128, 128, 4, 256, 128)
    with pytest.raises(ValueError, match="strides"):
        ops._check_rows("short", torch.empty(3, 256, 128), 256 * 128, 128, 4, 256, 128)
    with pytest.raises(ValueError, match="strides"):
        ops._check_rows("narrow", torch.empty(4, 256, 64), 256 * 64, 64, 4, 256, 128)


def test_serve_payload_matches_the_oracle_builder():
    """The package's ABI-1 payload builder (the Rust bridge's layout) gives the
    same bytes and row order as the oracle's builder on the same rows."""

    from oracle import decode as odec
    from shrimp import synthetic

    payload, order = synthetic.serve_payload("cfg0", 6)
    rows = synthetic.positions("cfg0", 6)
    want, worder = odec.build_payload([(s, f) for _, s, f in rows])
    assert order == worder
    for key in ("abi", "shape", "node_feats", "node_qr", "node_row_offsets", "nbr", "legal_counts"):
        assert payload[key] == want[key], key


def test_batch_limit_keeps_buffers_under_32_bit_offsets():
    """One forward launch sequence takes at most as many positions as keep every
    buffer extent that a kernel checks below the 32-bit buffer-offset limit,
    whichever attention path runs (staged: q plane + K/V fragments; unstaged:
    the three q/k/v planes the fused q/k/v kernel writes as one extent);
    max_batch lowers it further. The extents are recomputed here the way the
    kernels' argument checks compute them (qkv.hip, attn.hip, mlp.hip)."""

    from shrimp.model import ShrimpNet
    from shrimp.runtime import HipForward

    limit = HipForward.BUFFER_LIMIT
    C, H, dpad = 128, 8, 16
    rt = HipForward(ShrimpNet(channels=C, attention_heads=H, trunk_layout="CCACCACCACCA"))
    for precision, elem in (("bf16", 2), ("fp32", 4)):
        rt.precision = precision
        for npad in (256, 464, 512, 576):
            for staged in (True, False):
                rt.use_staged_attn = staged
                B = rt.batch_limit(npad)
                S = npad + 8
                SP = (S + 15) // 16 * 16
                extents = {
                    "attn_qkv qe (3 planes)": 3 * B * H * S * dpad * elem,
                    "attn q/k/v plane": ((B - 1) * H * S * dpad + (H - 1) * S * dpad + S * dpad) * elem,
                    "attn_staged kvf": B * H * SP * 64,
                    "attn out": ((B - 1) * S * C + (H - 1) * 16 + (S - 1) * C + 16) * elem,
                    "mlp hidden rows": ((B * S - 1) * 2 * C + 2 * C) * elem,
                    "seq rows": ((B * S - 1) * C + C) * elem,
                }
                for name, e in extents.items():
                    assert e < limit, (precision, npad, staged, B, name, e)
                # and the bound is tight: one more position would overflow a buffer
                per = max(3 * H * S * dpad * elem, S * 2 * C * elem, H * SP * 64)
                assert (B + 1) * per >= limit, (precision, npad, B)
    rt.precision = "bf16"
    assert rt.batch_limit(256) == (limit - 1) // (3 * H * 264 * dpad * 2)
    rt.max_batch = 7
    assert rt.batch_limit(256) == 7
    assert rt.batch_limit(10 ** 7) == 1


def _payload(sizes, legal):
    total = int(sum(sizes))
    return {
        "abi": 1, "shape": (len(sizes), total),
        "node_feats": np.zeros((total, C.NUM_FEATURES), np.float16).tobytes(),
        "node_qr": np.zeros((total, 2), np.int16).tobytes(),
        "node_row_offsets": np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64),
        "nbr": np.full((total, 6), 0xFFFF, np.uint16).tobytes(),
        "legal_counts": np.asarray(legal, np.int32).tobytes(),
    }


def test_evaluator_payload_validation():
    """The serve side refuses payloads whose rows break the wire contract
    before anything is uploaded (inference.py:509-531 checks shape and byte
    counts; rows sorted by size and legal counts within the row are what
    plan_groups and the decode rely on)."""

    from shrimp.inference import ShrimpEvaluator

    parse = ShrimpEvaluator._parse
    b, total, *_ = parse(_payload([70, 64, 10], [5, 64, 0]))
    assert (b, total) == (3, 144)
    assert parse(_payload([], []))[0] == 0
    with pytest.raises(ValueError, match="sorted by support size"):
        parse(_payload([10, 70], [1, 1]))
    with pytest.raises(ValueError, match="legal_counts must lie"):
        parse(_payload([70, 64], [71, 1]))
    with pytest.raises(ValueError, match="legal_counts must lie"):
        parse(_payload([70, 64], [1, -1]))
    bad = _payload([70, 64], [1, 1])
    bad["abi"] = 2
    with pytest.raises(ValueError, match="ABI"):
        parse(bad)
    bad = _payload([70, 64], [1, 1])
    bad["node_row_offsets"] = np.array([0, 50, 134], np.int64)
    with pytest.raises(ValueError, match="sorted"):
        parse(bad)
    bad = _payload([70, 64], [1, 1])
    bad["node_row_offsets"] = np.array([0, 140, 134], np.int64)
    with pytest.raises(ValueError, match="non-decreasing"):
        parse(bad)
    bad = _payload([70, 64], [1, 1])
    bad["legal_counts"] = bad["legal_counts"][:4]
    with pytest.raises(ValueError, match="legal_counts byte count"):
        parse(bad)
    bad = _payload([70, 64], [1, 1])
    bad["nbr"] = bad["nbr"][:-12]
    with pytest.raises(ValueError, match="nbr byte count"):
        parse(bad)


def test_busy_trace_report_arithmetic():
    """GpuBusyTrace's report (the keys of the reference's PerfTrace report,
    inference.py:171-199) from known per-payload device times."""

    from shrimp.inference import GpuBusyTrace

    class _Ev:
        def __init__(self, ms):
            self.ms = ms

        def elapsed_time(self, other):
            return other.ms - self.ms

    tr = GpuBusyTrace()
    assert tr.report()["gpu_idle_fraction"] is None
    tr._t_first = 100.0
    for n, (a, b) in ((10, (0.0, 2.0)), (30, (5.0, 9.0)), (20, (9.0, 15.0))):
        tr.finish((_Ev(a), _Ev(b)), n)
    tr._t_last = 100.024
    rep = tr.report()
    assert rep["device_busy_ms"] == 12.0 and rep["wall_window_ms"] == 24.0
    assert rep["gpu_busy_fraction"] == 0.5 and rep["gpu_idle_fraction"] == 0.5
    assert rep["measured_flushes"] == 3 and rep["measured_states"] == 60
    assert rep["mean_batch"] == 20.0 and rep["median_batch"] == 20.0
    assert rep["mean_forward_ms"] == 4.0 and rep["median_forward_ms"] == 4.0
    assert rep["mean_ms_per_state"] == 0.2
