"""hexfield_eq::ray_attn and hexfield_eq::hex_conv_ln_raytap (K1) on the GPU
against the float64 oracle (oracle/hexfield.py), at the reference's gates:
3e-3 absolute for ray attention (tests/test_hexfield_eq_triton_ray.py:55) and
5e-3 absolute for K1 (tests/test_hexfield_eq_raytap.py:869). Boards follow the
reference's fixtures (a lone cell, hex disks, padded rows) plus an elongated
chain and a 512-row board. At the bench shape (B = 1024, N = 256) sampled
positions are checked against the oracle and the two ray-attention kernels
(LDS-staged, global) must agree bit for bit."""

import math

import numpy as np
import pytest
import torch

from oracle import hexfield as ohf
from oracle import tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _disk(radius):
    return [(q, r) for q in range(-radius, radius + 1) for r in range(-radius, radius + 1)
            if abs(q + r) <= radius]


def _board(kind, n_pad, rng):
    """coords (N, 2), mask (N,): live cells in random order, holes and tail
    padding with far-away coordinates."""

    if kind == "lone":
        cells = [(0, 0)]
    elif kind == "chain":
        cells = [(q, r) for q in range(-30, 31) for r in (-1, 0, 1)]
    elif kind.startswith("disk"):
        cells = _disk(int(kind[4:]))
    else:
        raise ValueError(kind)
    cells = [cells[i] for i in rng.permutation(len(cells))]
    keep = [c for c in cells if rng.random() > 0.1] or cells[:1]
    assert len(keep) <= n_pad
    coords = np.zeros((n_pad, 2), dtype=np.int64)
    mask = np.zeros(n_pad, dtype=bool)
    # live rows with a few pad holes in between
    slots = np.sort(rng.choice(min(n_pad, len(keep) + 8), size=len(keep), replace=False))
    coords[:, 0] = 500 + np.arange(n_pad) * 20
    coords[slots] = keep
    mask[slots] = True
    return coords, mask


def _batch(kinds, n_pad, seed):
    rng = np.random.default_rng(seed)
    cs, ms = zip(*[_board(k, n_pad, rng) for k in kinds])
    return np.stack(cs), np.stack(ms)


def _seq_lens(mask):
    n = mask.shape[1]
    return torch.from_numpy((np.arange(1, n + 1)[None] * mask).max(1).astype(np.int32))


def _ray_index(coords, mask):
    from hexfield_eq import build_ray_gather_index

    idx = build_ray_gather_index(torch.from_numpy(coords).to(DEV), torch.from_numpy(mask).to(DEV))
    np.testing.assert_array_equal(idx.cpu().numpy(), tables.ray_index(coords, mask))
    return idx


def _nbr(coords, mask):
    b, n, _ = coords.shape
    out = np.full((b, n, 6), n, dtype=np.int64)
    for g in range(b):
        where = {tuple(coords[g, i]): i for i in range(n) if mask[g, i]}
        for i in range(n):
            for t, (dq, dr) in enumerate(tables.DIRECTIONS):
                j = where.get((coords[g, i, 0] + dq, coords[g, i, 1] + dr))
                if j is not None:
                    out[g, i, t] = j
    return out


def _ray_inputs(b, h, n, d, seed):
    gen = torch.Generator().manual_seed(seed)
    # (B, N, H, D) projections viewed as (B, H, N, D), as RayAttention passes them
    qkv = [torch.randn(b, n, h, d, generator=gen).half().to(DEV).transpose(1, 2) for _ in range(3)]
    slot_bias = (0.5 * torch.randn(32, h, generator=gen)).half()
    raylen = torch.randint(0, 6, (b, n, 12), generator=gen, dtype=torch.uint8)
    return qkv, slot_bias, raylen


def _ray_check(coords, mask, h, d, blockers, seed, variant=0):
    from hexfield_eq import ray_attn
    from hexfield_eq.ops import ray_attn_variant

    b, n = mask.shape
    idx = _ray_index(coords, mask)
    (q, k, v), sb, rl = _ray_inputs(b, h, n, d, seed)
    sl = _seq_lens(mask)
    prev = ray_attn_variant(variant)
    try:
        got = ray_attn(q, k, v, idx, sb.to(DEV), rl.to(DEV), sl.to(DEV), blockers)
    finally:
        ray_attn_variant(prev)
    want = ohf.ray_attn(q.cpu(), k.cpu(), v.cpu(), idx.cpu(), sb, rl, sl, blockers)
    assert got.dtype == torch.float16 and got.shape == (b, h, n, d)
    assert float(want.abs().max()) > 0.5  # the comparison is not between zeros
    torch.testing.assert_close(got.double().cpu(), want, atol=3e-3, rtol=0)
    return got


@pytest.mark.parametrize("variant", [0, 1], ids=["auto", "global"])
@pytest.mark.parametrize("blockers", [True, False], ids=["blockers", "geometric"])
@pytest.mark.parametrize("d", [16, 32, 64, 128])
def test_ray_attn_matches_oracle(d, blockers, variant):
    coords, mask = _batch(["lone", "disk3", "disk8", "chain"], 256, seed=d)
    _ray_check(coords, mask, 6, d, blockers, seed=d + 1, variant=variant)


@pytest.mark.parametrize("h", [8, 5, 1])
def test_ray_attn_other_head_counts(h):
    """Heads past the three win axes see only themselves; an odd head count
    leaves the last workgroup one head."""

    coords, mask = _batch(["disk4", "disk2", "chain"], 192, seed=h)
    _ray_check(coords, mask, h, 16, True, seed=h + 7)


def test_ray_attn_absent_self_and_short_rows():
    """A row whose every slot is absent is zero; rows >= seq_lens are zero
    (seq_lens 0 included); an index past N counts as absent."""

    from hexfield_eq import ray_attn

    coords, mask = _batch(["disk3", "disk3", "lone"], 64, seed=3)
    b, n = mask.shape
    idx = _ray_index(coords, mask)
    idx[0, 5, :] = n
    idx[1, 2, 3:9] = n + 100
    (q, k, v), sb, rl = _ray_inputs(b, 6, n, 16, 4)
    sl = _seq_lens(mask)
    sl[2] = 0
    got = ray_attn(q, k, v, idx, sb.to(DEV), rl.to(DEV), sl.to(DEV), True)
    want = ohf.ray_attn(q.cpu(), k.cpu(), v.cpu(), idx.cpu(), sb, rl, sl, True)
    torch.testing.assert_close(got.double().cpu(), want, atol=3e-3, rtol=0)
    assert (got[0, :, 5] == 0).all() and (got[2] == 0).all()


def test_ray_attn_bench_shape_samples_and_variants_agree():
    """B = 1024, N = 256, H = 6, D = 16 (the bench workload): positions 0, 517
    and 1023 against the oracle; the staged and global kernels bit-identical."""

    from hexfield_eq import ray_attn
    from hexfield_eq.ops import ray_attn_variant

    rng = np.random.default_rng(11)
    b, n, h, d = 1024, 256, 6, 16
    kinds = [["disk8", "disk6", "chain", "disk4"][i % 4] for i in range(b)]
    cs, ms = zip(*[_board(k, n, rng) for k in kinds])
    coords, mask = np.stack(cs), np.stack(ms)
    from hexfield_eq import build_ray_gather_index

    idx = build_ray_gather_index(torch.from_numpy(coords).to(DEV), torch.from_numpy(mask).to(DEV))
    (q, k, v), sb, rl = _ray_inputs(b, h, n, d, 12)
    sl = _seq_lens(mask)
    args = (q, k, v, idx, sb.to(DEV), rl.to(DEV), sl.to(DEV), True)
    staged = ray_attn(*args)
    prev = ray_attn_variant(1)
    try:
        glob = ray_attn(*args)
    finally:
        ray_attn_variant(prev)
    assert torch.equal(staged, glob)
    for p in (0, 517, 1023):
        sel = slice(p, p + 1)
        np.testing.assert_array_equal(idx[sel].cpu().numpy(), tables.ray_index(coords[sel], mask[sel]))
        want = ohf.ray_attn(q[sel].cpu(), k[sel].cpu(), v[sel].cpu(), idx[sel].cpu(), sb,
                            rl[sel], sl[sel], True)
        torch.testing.assert_close(staged[sel].double().cpu(), want, atol=3e-3, rtol=0)


# ---- K1 ---------------------------------------------------------------------------------


def _k1_inputs(coords, mask, c, cout, seed):
    b, n = mask.shape
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, n, c, generator=gen).half()
    weight = (torch.randn(7, c, cout, generator=gen) * 0.05).half()
    bias = torch.randn(cout, generator=gen) * 0.02
    lnw = torch.rand(cout, generator=gen) + 0.5
    lnb = torch.randn(cout, generator=gen) * 0.1
    alpha = torch.stack([0.8 ** k * (1.0 + 0.1 * torch.randn(c, generator=gen)) for k in range(5)])
    raylen = torch.randint(0, 6, (b, n, 12), generator=gen, dtype=torch.uint8)
    gidx = torch.from_numpy(tables.gather_index(_nbr(coords, mask)))
    return x, weight, bias, lnw, lnb, alpha.half(), raylen, gidx


def _k1_check(coords, mask, c, cout, corb, seed, relus=(True, False)):
    from hexfield_eq import build_tap_reach, hex_conv_ln_raytap

    x, w, bias, lnw, lnb, alpha, raylen, gidx = _k1_inputs(coords, mask, c, cout, seed)
    ray_idx = _ray_index(coords, mask)
    reach = build_tap_reach(raylen.to(DEV))
    m = torch.from_numpy(mask)
    assert torch.equal(reach.cpu(), ohf.build_tap_reach(raylen))
    for relu in relus:
        got = hex_conv_ln_raytap(x.to(DEV), gidx.to(DEV), m.to(DEV), w.to(DEV), bias.to(DEV),
                                 lnw.to(DEV), lnb.to(DEV), ray_idx, reach, alpha.to(DEV),
                                 1e-5, relu, corb)
        want = ohf.conv_ln_raytap(x, gidx, m, w, bias, lnw, lnb, ray_idx.cpu(), reach.cpu(), alpha,
                                  1e-5, relu, corb)
        assert got.dtype == torch.float16
        assert float(want.abs().max()) > 0.5
        torch.testing.assert_close(got.double().cpu(), want, atol=5e-3, rtol=0)


@pytest.mark.parametrize("c,cout,corb", [(128, 128, 128), (96, 96, 8), (128, 64, 16),
                                         (64, 96, 64), (96, 128, 32)])
def test_conv_ln_raytap_matches_oracle(c, cout, corb):
    coords, mask = _batch(["disk4", "disk8", "lone", "chain"], 256, seed=c + cout)
    _k1_check(coords, mask, c, cout, corb, seed=corb)


@pytest.mark.parametrize("n_pad,kinds", [(64, ["disk3", "disk4"]), (200, ["disk7", "chain"]),
                                         (512, ["disk12", "disk9"])])
def test_conv_ln_raytap_row_counts(n_pad, kinds):
    """Npad not a multiple of 64 (partial wave), and 512 rows (eight waves)."""

    coords, mask = _batch(kinds, n_pad, seed=n_pad)
    _k1_check(coords, mask, 96, 96, 8, seed=n_pad + 1, relus=(True,))


def test_conv_ln_raytap_bench_shape_samples():
    """B = 1024, N = 256, C = Cout = 128 (the bench workload): three positions
    against the oracle."""

    from hexfield_eq import build_tap_reach, hex_conv_ln_raytap

    rng = np.random.default_rng(21)
    b, n, c = 1024, 256, 128
    kinds = [["disk8", "disk6", "chain", "disk4"][i % 4] for i in range(b)]
    cs, ms = zip(*[_board(k, n, rng) for k in kinds])
    coords, mask = np.stack(cs), np.stack(ms)
    picks = (0, 517, 1023)
    x, w, bias, lnw, lnb, alpha, raylen, _ = _k1_inputs(coords[:1], mask[:1], c, c, 22)
    gen = torch.Generator().manual_seed(23)
    x = torch.randn(b, n, c, generator=gen).half()
    raylen = torch.randint(0, 6, (b, n, 12), generator=gen, dtype=torch.uint8)
    from hexfield_eq import build_ray_gather_index

    ray_idx = build_ray_gather_index(torch.from_numpy(coords).to(DEV), torch.from_numpy(mask).to(DEV))
    gsel = {p: torch.from_numpy(tables.gather_index(_nbr(coords[p:p + 1], mask[p:p + 1]))) for p in picks}
    gidx = torch.full((b, n, 7), n, dtype=torch.int64)
    gidx[:, :, 0] = torch.arange(n)
    for p in picks:
        gidx[p] = gsel[p][0]
    reach = build_tap_reach(raylen.to(DEV))
    m = torch.from_numpy(mask)
    got = hex_conv_ln_raytap(x.to(DEV), gidx.to(DEV), m.to(DEV), w.to(DEV), bias.to(DEV),
                             lnw.to(DEV), lnb.to(DEV), ray_idx, reach, alpha.to(DEV), 1e-5, True, 8)
    for p in picks:
        sel = slice(p, p + 1)
        want = ohf.conv_ln_raytap(x[sel], gidx[sel], m[sel], w, bias, lnw, lnb, ray_idx[sel].cpu(),
                                  reach[sel].cpu(), alpha, 1e-5, True, 8)
        torch.testing.assert_close(got[sel].double().cpu(), want, atol=5e-3, rtol=0)
    assert not torch.isnan(got).any()
    assert math.isfinite(float(got.float().abs().max()))
