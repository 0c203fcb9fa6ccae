"""Pins the oracle's floating-point functions: golden outputs of the reference
ShrimpNet / evaluator, a dense-grid convolution (tests/test_shrimp_model.py:81-136),
torch's scaled_dot_product_attention, and closed forms."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decode, forward, tables, weights


def _fwd(g, mode, **kw):
    c, h = (int(x) for x in g["arch"])
    layout = str(g["layout"])
    sd = weights.make_state_dict(c, h, layout, seed=int(g[f"{mode}_seed"]), mode=mode)
    return forward.forward_policy_value(
        sd, layout, h, g["feats"], g["nbr"], g["mask"], g["coords"],
        request_moves_left=True, return_trunk=True, **kw,
    )


@pytest.mark.parametrize("name,mode", [("forward_cfg0", "parity"), ("forward_cfg0", "fresh"),
                                       ("forward_cfg4", "parity")])
def test_forward_matches_reference_golden(golden, name, mode):
    g = golden(name)
    out = _fwd(g, mode)
    for key in ("policy", "value", "moves_left", "cells", "tokens"):
        want = torch.from_numpy(g[f"{mode}_{key}"]).double()
        got = out[key]
        scale = 1.0 + want.abs().max().item()
        err = (got - want).abs().max().item()
        assert err <= 2e-5 * scale, f"{name}/{mode}/{key}: {err}"
    # pad logits are exactly zero
    mask = torch.from_numpy(g["mask"])
    assert (out["policy"][~mask] == 0).all()


def test_forward_fp32_close_to_fp64(golden):
    g = golden("forward_cfg0")
    a = _fwd(g, "parity", dtype=torch.float32)
    b = _fwd(g, "parity", dtype=torch.float64)
    for k in ("policy", "value"):
        assert (a[k].double() - b[k]).abs().max().item() < 1e-4


def test_hex_conv_equals_dense_grid_conv():
    """Tap 0 = centre (1,1) of a 3x3 kernel, axial (dq, dr) at (dr+1, dq+1)."""

    torch.manual_seed(1)
    rng = np.random.default_rng(3)
    cells = sorted({(int(q), int(r)) for q, r in rng.integers(-6, 7, size=(40, 2))})
    n = len(cells)
    index = {c: i for i, c in enumerate(cells)}
    nbr = np.full((1, n, 6), n, dtype=np.int64)
    for i, (q, r) in enumerate(cells):
        for k, (dq, dr) in enumerate(tables.DIRECTIONS):
            nbr[0, i, k] = index.get((q + dq, r + dr), n)
    cin, cout = 5, 4
    w = torch.randn(7, cin, cout, dtype=torch.float64)
    b = torch.randn(cout, dtype=torch.float64)
    x = torch.randn(1, n, cin, dtype=torch.float64)
    gidx = torch.from_numpy(tables.gather_index(nbr))
    mask = torch.ones(1, n, dtype=torch.bool)
    out = forward.hex_conv(x, gidx, mask, w, b)
    kern = torch.zeros(cout, cin, 3, 3, dtype=torch.float64)
    kern[:, :, 1, 1] = w[0].T
    for k, (dq, dr) in enumerate(tables.DIRECTIONS):
        kern[:, :, dr + 1, dq + 1] = w[k + 1].T
    grid = torch.zeros(1, cin, 41, 41, dtype=torch.float64)
    for i, (q, r) in enumerate(cells):
        grid[0, :, r + 20, q + 20] = x[0, i]
    dense = F.conv2d(grid, kern, bias=b, padding=1)
    for i, (q, r) in enumerate(cells):
        assert torch.allclose(out[0, i], dense[0, :, r + 20, q + 20], atol=1e-12)


def test_raytap_conv_reduces_to_hex_conv():
    """With weight only on slot 0 and the distance-1 slots the 31-tap conv is
    the 7-tap conv; extra slots add exactly their own gathered term."""

    rng = np.random.default_rng(5)
    coords = np.stack(np.meshgrid(np.arange(-4, 5), np.arange(-4, 5)), -1).reshape(1, -1, 2)
    n = coords.shape[1]
    mask = np.ones((1, n), bool)
    mask[0, -7:] = False
    ridx = torch.from_numpy(tables.ray_index(coords, mask))
    idx7 = torch.cat([ridx[:, :, :1], ridx[:, :, tables.tap_ray_slots()]], dim=2)
    x = torch.from_numpy(rng.standard_normal((1, n, 6)))
    w7 = torch.from_numpy(rng.standard_normal((7, 6, 3)))
    b = torch.from_numpy(rng.standard_normal(3))
    w31 = torch.zeros(31, 6, 3, dtype=torch.float64)
    w31[0] = w7[0]
    for t, s in enumerate(tables.tap_ray_slots()):
        w31[s] = w7[t + 1]
    m = torch.from_numpy(mask)
    a = forward.raytap_conv(x, ridx, m, w31, b)
    c = forward.hex_conv(x, idx7, m, w7, b)
    assert torch.allclose(a, c, atol=1e-12)
    # brute force, every slot weighted
    w31 = torch.from_numpy(rng.standard_normal((31, 6, 3)))
    a = forward.raytap_conv(x, ridx, m, w31, b)
    for i in range(n):
        want = b.clone()
        for s in range(31):
            j = int(ridx[0, i, s])
            if j < n:
                want = want + x[0, j] @ w31[s]
        want = want * float(mask[0, i])
        assert torch.allclose(a[0, i], want, atol=1e-12)


def test_attention_equals_sdpa():
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 3, 20, 8, dtype=torch.float64) for _ in range(3))
    bias = torch.randn(2, 3, 20, 20, dtype=torch.float64)
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=bias)
    assert torch.allclose(forward.attention(q, k, v, bias), want, atol=1e-12)


def test_attn_pair_masks_keys_and_rows():
    torch.manual_seed(1)
    b, h, s, d = 2, 2, 12, 4
    q, k, v = (torch.randn(b, h, s, d, dtype=torch.float64) for _ in range(3))
    pair = torch.randint(0, 5, (b, s, s))
    table2 = torch.randn(5, h, dtype=torch.float64)
    lens = torch.tensor([7, 12])
    out = forward.attn_pair(q, k, v, pair, table2, lens)
    assert (out[0, :, 7:] == 0).all()
    # row 0 of batch 0 by hand
    sc = (q[0, 1, 3] @ k[0, 1, :7].T) / math.sqrt(d) + table2[pair[0, 3, :7], 1]
    want = torch.softmax(sc, 0) @ v[0, 1, :7]
    assert torch.allclose(out[0, 1, 3], want, atol=1e-12)


def test_decode_matches_reference(golden):
    g = golden("decode")
    logits = torch.from_numpy(g["logits"]).double()
    assert np.allclose(decode.decode_value(logits).numpy(), g["value"], atol=1e-6)
    assert np.allclose(decode.decode_moves_left(logits).numpy(), g["moves_left"], atol=1e-4)
    assert decode.plan_groups(g["sizes"]) == [tuple(x) for x in g["groups"].tolist()]


def test_decode_closed_forms():
    z = torch.zeros(1, 65, dtype=torch.float64)
    assert abs(decode.decode_value(z).item()) < 1e-15  # symmetric bins
    one_hot = torch.full((1, 65), -1e4, dtype=torch.float64)
    one_hot[0, 48] = 0.0
    assert decode.decode_value(one_hot).item() == pytest.approx(-1 + 2 * 48 / 64)
    assert decode.decode_moves_left(one_hot).item() == pytest.approx((2 * 48 / 64) * 0.5 * 209)


def test_evaluator_matches_reference_reply(golden):
    g = golden("evaluator_cfg0")
    payload = {
        "abi": 1, "shape": tuple(int(x) for x in g["shape"]),
        "node_feats": g["node_feats"].tobytes(), "node_qr": g["node_qr"].tobytes(),
        "node_row_offsets": g["node_row_offsets"].tolist(), "nbr": g["nbr"].tobytes(),
        "legal_counts": g["legal_counts"].tobytes(),
        "request_moves_left": True, "request_logits": True,
    }
    sd = weights.make_state_dict(32, 4, "CCA", seed=int(g["wseed"]), mode="parity")
    reply = decode.evaluate(payload, sd, "CCA", 4)
    for key, gk in (("values_bytes", "values"), ("priors_bytes", "priors"),
                    ("moves_left_bytes", "moves_left"), ("priors_logits_bytes", "priors_logits")):
        got = np.frombuffer(reply[key], np.float32)
        assert got.shape == g[gk].shape, key
        scale = 1.0 + np.abs(g[gk]).max()
        assert np.abs(got - g[gk]).max() <= 2e-5 * scale, key
