"""Pins the oracle's floating-point functions: golden outputs of the reference
ShrimpNet / evaluator, a dense-grid convolution (tests/test_shrimp_model.py:81-136),
torch's scaled_dot_product_attention, and closed forms."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decode, forward, tables, weights

from gates import LOGIT_TOL, TRUNK_MEAN


def _fwd(g, mode, **kw):
    c, h = (int(x) for x in g["arch"])
    layout = str(g["layout"])
    sd = weights.make_state_dict(c, h, layout, seed=int(g[f"{mode}_seed"]), mode=mode)
    return forward.forward_policy_value(
        sd, layout, h, g["feats"], g["nbr"], g["mask"], g["coords"],
        request_moves_left=True, return_trunk=True, **kw,
    )


@pytest.mark.parametrize("name,mode", [("forward_cfg0", "parity"), ("forward_cfg0", "fresh"),
                                       ("forward_cfg0", "heads"), ("forward_cfg4", "parity"),
                                       ("forward_cfg4", "heads")])
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


def _mutations(sd):
    """Composition mistakes a forward could make with correct kernels: a block
    reading a zeroed, another block's or a head-permuted bias table, and a
    skipped attention sub-block."""

    out = {}
    s = dict(sd)
    s["bias_tables.0"] = torch.zeros_like(s["bias_tables.0"])
    out["zeroed table 0"] = s
    s = dict(sd)
    s["bias_tables.0"] = s["bias_tables.0"].flip(1)
    out["heads of table 0 reversed"] = s
    s = dict(sd)
    s["bias_tables.3"] = s["bias_tables.3"].roll(1, 1)
    out["heads of table 3 rotated"] = s
    s = dict(sd)
    s["bias_tables.0"], s["bias_tables.1"] = s["bias_tables.1"], s["bias_tables.0"]
    out["tables 0 and 1 swapped"] = s
    s = dict(sd)
    s["attn_blocks.0.ls_attn.gamma"] = torch.zeros_like(s["attn_blocks.0.ls_attn.gamma"])
    out["attention sub-block 0 skipped"] = s
    return out


@pytest.mark.parametrize("mode", ["parity", "heads"])
def test_trunk_gates_see_composition_mistakes(golden, mode):
    """The GPU forward tests gate the trunk output's tokens at TRUNK_MEAN (mean
    absolute error) and, with O(1) heads, the value logits at LOGIT_TOL. Each
    composition mistake moves the fp32 reference by at least twice a gate, so
    a forward that made it fails the GPU test even with exact kernels."""

    g = golden("forward_cfg4")
    c, h = (int(x) for x in g["arch"])
    layout = str(g["layout"])
    sd = weights.make_state_dict(c, h, layout, seed=int(g[f"{mode}_seed"]), mode=mode)
    args = (g["feats"], g["nbr"], g["mask"], g["coords"])

    def run(d):
        return forward.forward_policy_value(d, layout, h, *args, request_moves_left=True,
                                            return_trunk=True, dtype=torch.float32)

    base = run(sd)
    for name, bad in _mutations(sd).items():
        o = run(bad)
        tok = (o["tokens"] - base["tokens"]).abs().mean().item()
        val = (o["value"] - base["value"]).abs().max().item()
        print(f"{mode} {name}: tokens mean {tok:.4f}, value max {val:.4f}")
        assert tok >= 2 * TRUNK_MEAN, name
        if mode == "heads":
            assert val >= 2 * LOGIT_TOL, name


def test_forward_fp32_close_to_fp64(golden):
    g = golden("forward_cfg0")
    a = _fwd(g, "parity", dtype=torch.float32)
    b = _fwd(g, "parity", dtype=torch.float64)
    for k in ("policy", "value"):
        assert (a[k].double() - b[k]).abs().max().item() < 1e-4


def _dense_grid_case(seed, cin, cout):
    """A random cell set (axial coordinates within +-6), its neighbour table,
    inputs, weights, and the same convolution as a dense F.conv2d over a
    41 x 41 grid: tap 0 = centre (1, 1) of a 3x3 kernel, axial (dq, dr) at
    (dr + 1, dq + 1). Returns (cells, gidx, x, w, b, dense)."""

    rng = np.random.default_rng(seed)
    cells = sorted({(int(q), int(r)) for q, r in rng.integers(-6, 7, size=(40, 2))})
    n = len(cells)
    index = {c: i for i, c in enumerate(cells)}
    nbr = np.full((1, n, 6), n, dtype=np.int64)
    for i, (q, r) in enumerate(cells):
        for k, (dq, dr) in enumerate(tables.DIRECTIONS):
            nbr[0, i, k] = index.get((q + dq, r + dr), n)
    w = torch.from_numpy(rng.standard_normal((7, cin, cout)))
    b = torch.from_numpy(rng.standard_normal(cout))
    x = torch.from_numpy(rng.standard_normal((1, n, cin)))
    gidx = torch.from_numpy(tables.gather_index(nbr))
    kern = torch.zeros(cout, cin, 3, 3, dtype=torch.float64)
    kern[:, :, 1, 1] = w[0].T
    for k, (dq, dr) in enumerate(tables.DIRECTIONS):
        kern[:, :, dr + 1, dq + 1] = w[k + 1].T
    grid = torch.zeros(1, cin, 41, 41, dtype=torch.float64)
    for i, (q, r) in enumerate(cells):
        grid[0, :, r + 20, q + 20] = x[0, i]
    dense = F.conv2d(grid, kern, bias=b, padding=1)
    rows = torch.stack([dense[0, :, r + 20, q + 20] for q, r in cells])  # (n, cout)
    return cells, gidx, x, w, b, rows


def test_hex_conv_equals_dense_grid_conv():
    cells, gidx, x, w, b, dense = _dense_grid_case(3, 5, 4)
    mask = torch.ones(1, len(cells), dtype=torch.bool)
    out = forward.hex_conv(x, gidx, mask, w, b)
    assert torch.allclose(out[0], dense, atol=1e-12)


@pytest.mark.parametrize("relu", [False, True])
def test_hex_conv_ln_equals_dense_grid_conv_then_layer_norm(relu):
    """hex_conv_ln (shrimp::hex_conv_ln, _triton_conv.py:139-196) against the
    dense-grid convolution followed by torch's F.layer_norm over the output
    channels, the optional ReLU and the row mask; a LayerNorm over the wrong
    axis, a dropped affine or an unmasked row each fail."""

    cells, gidx, x, w, b, dense = _dense_grid_case(7, 6, 8)
    n = len(cells)
    rng = np.random.default_rng(8)
    ln_w = torch.from_numpy(rng.uniform(0.5, 1.5, 8))
    ln_b = torch.from_numpy(rng.normal(0, 0.3, 8))
    mask = torch.from_numpy(rng.random(n) > 0.25)[None]
    out = forward.hex_conv_ln(x, gidx, mask, w, b, ln_w, ln_b, 1e-5, relu)
    want = F.layer_norm(dense, (8,), ln_w, ln_b, 1e-5)
    if relu:
        want = F.relu(want)
    want = want * mask[0, :, None].double()
    assert torch.allclose(out[0], want, atol=1e-12)
    assert (out[0][~mask[0]] == 0).all()
    plain = forward.hex_conv(x, gidx, mask, w, b)[0]
    assert (plain - want).abs().max().item() > 1e-1  # the LayerNorm is not a no-op here


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


def _pair_case(golden, b, compact):
    """Live cells of golden position b (all of them, or those with |q|, |r| <= 8
    so every offset lies within +-16), their coordinates, and the reference's
    pair rows between them (pair.npz, written by _build_pair_u8)."""

    g = golden("pair")
    coords, mask, pair = g["coords"][b], g["mask"][b], g["pair_u8"][b]
    sel = np.flatnonzero(mask)
    if compact:
        sel = sel[(np.abs(coords[sel]) <= 8).all(1)]
    return coords[sel], pair[np.ix_(8 + sel, 8 + sel)]


@pytest.mark.parametrize("m", [17, 16])
@pytest.mark.parametrize("b", [0, 3])
def test_attn_offset_table_matches_reference_pair_rows(golden, m, b):
    """attn_offset_table (config 2's attention) against the reference's own
    pair rows: with the per-offset table T[(dq + m)(2m + 1) + dr + m] =
    table[lut(dq, dr)] it must equal attn_pair with table[pair[i, j]], where
    pair comes from the reference's _build_pair_u8 (key - query offsets, the
    35x35 LUT clamped at 17). m = 17 covers whole boards (offsets up to 26:
    the clamp); m = 16, config 2's table, covers compact cell sets. A swap of
    dq and dr, or query - key instead of key - query, fails (checked below by
    transposing or negating the coordinates)."""

    coords, pair = _pair_case(golden, b, compact=(m == 16))
    n = coords.shape[0]
    hd, d = 3, 4
    rng = np.random.default_rng(10 * b + m)
    table = torch.from_numpy(rng.normal(0, 0.8, size=(tables.BIAS_ROWS, hd)))
    lut35 = tables.cell_lut()  # (35 * 35,) rows, offsets clamped to +-17
    w = 2 * m + 1
    off = np.arange(-m, m + 1)
    dq, dr = np.meshgrid(off, off, indexing="ij")
    t = table[torch.from_numpy(lut35[(dq.ravel() + 17) * 35 + dr.ravel() + 17].astype(np.int64))]
    assert t.shape == (w * w, hd)
    q, k, v = (torch.from_numpy(rng.standard_normal((1, hd, n, d))) for _ in range(3))
    live = torch.ones(1, n, dtype=torch.bool)
    got = forward.attn_offset_table(q, k, v, torch.from_numpy(coords)[None], live, t, m)
    tab2 = torch.cat([table, torch.full((1, hd), -3.0e4, dtype=table.dtype)])
    want = forward.attn_pair(q, k, v, torch.from_numpy(pair.astype(np.int64))[None], tab2,
                             torch.tensor([n]))
    assert torch.allclose(got, want, atol=1e-12)
    for wrong in (coords[:, ::-1].copy(), -coords):
        bad = forward.attn_offset_table(q, k, v, torch.from_numpy(wrong)[None], live, t, m)
        assert (bad - want).abs().max().item() > 1e-2


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
