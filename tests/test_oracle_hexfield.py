"""Pins the hexfield oracle (oracle/hexfield.py): ray attention against a dense
brute force written from coordinates alone (the flex score_mod semantics of
hexfield_eq/model.py:365-420), closed forms, and the ray-tap conv against the
plain hex conv (init equivalence, tests/test_hexfield_eq_raytap.py:253-266)
and the 31-tap conv (factored identity). The reference's own hexfield tests
compare its CUDA kernels with its torch twins on random inputs and hold no
fixtures for these two ops."""

import math

import numpy as np
import pytest
import torch

from oracle import forward, hexfield, tables

AXIS_OF_COSET = ((1, 0), (0, 1), (1, -1))


def _board(seed, n_pad=48, radius=3, drop=0.15):
    """Hex disk of the given radius (cells in random order, some dropped),
    live rows first, then pad rows with far-away coordinates."""

    rng = np.random.default_rng(seed)
    cells = [(q, r) for q in range(-radius, radius + 1) for r in range(-radius, radius + 1)
             if abs(q + r) <= radius]
    rng.shuffle(cells)
    cells = [c for c in cells if rng.random() > drop]
    n = len(cells)
    assert n <= n_pad
    coords = np.zeros((1, n_pad, 2), dtype=np.int64)
    coords[0, :n] = cells
    coords[0, n:, 0] = 100 + np.arange(n_pad - n) * 20
    mask = np.zeros((1, n_pad), dtype=bool)
    mask[0, :n] = True
    return coords, mask


def _boards(seeds, n_pad=48):
    cs, ms = zip(*[_board(s, n_pad) for s in seeds])
    return np.concatenate(cs), np.concatenate(ms)


def _seq_lens(mask):
    n = mask.shape[1]
    return torch.from_numpy((np.arange(1, n + 1)[None] * mask).max(1)).to(torch.int32)


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


def _dense_ray_attn(q, k, v, coords, mask, slot_bias, raylen, blockers):
    """Every (query, key) pair tested from coordinates: live iff key == query,
    or the key is a live cell on the head's win axis at signed step kk with
    1 <= |kk| <= 5 (and |kk| <= the query's raylen for that side, axis and
    direction). Bias of a live pair = slot_bias at the slot of its offset."""

    b, h, n, d = q.shape
    off = tables.ray_slot_offsets()
    slot_of = {(int(off[s, 0]), int(off[s, 1])): s for s in range(1, 31)}
    out = torch.zeros(b, h, n, d, dtype=torch.float64)
    for g in range(b):
        for hh in range(h):
            coset, side = hh // 2, hh % 2
            for i in range(n):
                if not mask[g, i]:
                    continue
                keys = [(i, 0)]
                for j in range(n):
                    if j == i or not mask[g, j]:
                        continue
                    dq = int(coords[g, j, 0] - coords[g, i, 0])
                    dr = int(coords[g, j, 1] - coords[g, i, 1])
                    if coset >= 3:
                        continue
                    aq, ar = AXIS_OF_COSET[coset]
                    kk = dq if aq != 0 else dr
                    if (kk * aq, kk * ar) != (dq, dr) or not 1 <= abs(kk) <= 5:
                        continue
                    if blockers:
                        slot = side * 6 + coset * 2 + (0 if kk > 0 else 1)
                        if abs(kk) > int(raylen[g, i, slot]):
                            continue
                    keys.append((j, slot_of[(dq, dr)]))
                sc = [float(q[g, hh, i] @ k[g, hh, j]) / math.sqrt(d) + float(slot_bias[s, hh])
                      for j, s in keys]
                m = max(sc)
                p = [math.exp(x - m) for x in sc]
                l = sum(p)
                for (j, _), w in zip(keys, p):
                    out[g, hh, i] += (w / l) * v[g, hh, j]
    return out


def _qkv(b, h, n, d, seed):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(b, h, n, d, generator=gen, dtype=torch.float64) for _ in range(3)]


@pytest.mark.parametrize("blockers", [True, False])
def test_ray_attn_matches_dense_brute_force(blockers):
    coords, mask = _boards([1, 2])
    b, n = mask.shape
    h, d = 6, 8
    q, k, v = _qkv(b, h, n, d, 3)
    rng = np.random.default_rng(4)
    raylen = torch.from_numpy(rng.integers(0, 6, size=(b, n, 12)).astype(np.uint8))
    slot_bias = torch.from_numpy(rng.normal(size=(32, h)))
    idx = torch.from_numpy(tables.ray_index(coords, mask))
    got = hexfield.ray_attn(q, k, v, idx, slot_bias, raylen, _seq_lens(mask), blockers)
    want = _dense_ray_attn(q, k, v, coords, mask, slot_bias, raylen, blockers)
    live = torch.from_numpy(mask).view(b, 1, n, 1)
    torch.testing.assert_close(got * live, want, rtol=1e-12, atol=1e-12)


def test_ray_attn_closed_forms():
    coords, mask = _boards([5, 6])
    b, n = mask.shape
    h, d = 8, 4  # heads 6 and 7 ride no win axis: self only
    q, k, v = _qkv(b, h, n, d, 7)
    idx = torch.from_numpy(tables.ray_index(coords, mask))
    sl = _seq_lens(mask)
    rows = (torch.arange(n).view(1, n) < sl.long().view(b, 1)).view(b, 1, n, 1).double()
    sb = torch.from_numpy(np.random.default_rng(8).normal(size=(32, h)))
    # Every ray blocked at the query: only the row itself is live.
    zero = torch.zeros(b, n, 12, dtype=torch.uint8)
    got = hexfield.ray_attn(q, k, v, idx, sb, zero, sl, True)
    torch.testing.assert_close(got, v * rows, rtol=0, atol=0)
    # Heads past the three axes: self only, whatever the rays.
    five = torch.full((b, n, 12), 5, dtype=torch.uint8)
    got = hexfield.ray_attn(q, k, v, idx, sb, five, sl, True)
    torch.testing.assert_close(got[:, 6:], (v * rows)[:, 6:], rtol=0, atol=0)
    # Blockers off == every reach 5.
    torch.testing.assert_close(hexfield.ray_attn(q, k, v, idx, sb, zero, sl, False), got,
                               rtol=0, atol=0)
    # Zero queries and bias: the mean of the live rows (self + on-axis cells
    # within five steps).
    zq = torch.zeros_like(q)
    got = hexfield.ray_attn(zq, k, v, idx, torch.zeros(32, h, dtype=torch.float64), five, sl, True)
    for g in range(b):
        for hh in range(6):
            a = AXIS_OF_COSET[hh // 2]
            where = {tuple(coords[g, j]): j for j in range(n) if mask[g, j]}
            for i in range(n):
                if not mask[g, i]:
                    continue
                js = [i] + [where[c] for c in
                            [(coords[g, i, 0] + s * kk * a[0], coords[g, i, 1] + s * kk * a[1])
                             for s in (1, -1) for kk in range(1, 6)] if c in where]
                torch.testing.assert_close(got[g, hh, i], v[g, hh, js].mean(0), rtol=1e-12,
                                           atol=1e-12)


def test_ray_attn_absent_slots_and_pad_rows():
    """An all-absent row (self slot sentinel too) and rows >= seq_lens are zero;
    indices outside [0, N) are absent."""

    coords, mask = _boards([9])
    b, n = mask.shape
    h, d = 6, 4
    q, k, v = _qkv(b, h, n, d, 10)
    idx = torch.from_numpy(tables.ray_index(coords, mask))
    idx[0, 3, :] = n
    idx[0, 4, 1:] = -5
    sl = _seq_lens(mask)
    got = hexfield.ray_attn(q, k, v, idx, torch.zeros(32, h, dtype=torch.float64),
                            torch.full((b, n, 12), 5, dtype=torch.uint8), sl, True)
    assert (got[0, :, 3] == 0).all()
    torch.testing.assert_close(got[0, :, 4], v[0, :, 4], rtol=0, atol=0)
    assert (got[0, :, int(sl[0]):] == 0).all()


def test_slot_luts_match_geometry():
    """T7 (tests/test_hexfield_eq_raytap.py:190-219): the tap/step slot of
    every (tap, k) holds the offset k * DIRECTIONS[t]; the raylen slot of
    (side, tap) is side*6 + axis*2 + dir with the tap on +-axis."""

    off = tables.ray_slot_offsets()
    lut = hexfield.tap_ray_slot_lut()
    seen = set()
    for t, (dq, dr) in enumerate(tables.DIRECTIONS):
        for k in range(1, 6):
            s = int(lut[t, k - 1])
            assert tuple(off[s]) == (k * dq, k * dr)
            seen.add(s)
    assert seen == set(range(1, 31))
    assert [int(x) for x in lut[:, 0]] == tables.tap_ray_slots()
    rl = hexfield.tap_raylen_slots()
    for t, (dq, dr) in enumerate(tables.DIRECTIONS):
        for side in range(2):
            a, direc = divmod(int(rl[side, t]) - side * 6, 2)
            aq, ar = AXIS_OF_COSET[a]
            sgn = 1 if direc == 0 else -1
            assert (sgn * aq, sgn * ar) == (dq, dr)


def _conv_case(seed, c=16, cout=24, corb=8):
    coords, mask = _boards([seed, seed + 1])
    b, n = mask.shape
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, n, c, generator=gen).to(torch.float16).double()
    w = (torch.randn(7, c, cout, generator=gen) / math.sqrt(7 * c)).double()
    bias = torch.randn(cout, generator=gen).double() * 0.1
    lnw = 1 + 0.1 * torch.randn(cout, generator=gen).double()
    lnb = 0.1 * torch.randn(cout, generator=gen).double()
    ray_idx = torch.from_numpy(tables.ray_index(coords, mask))
    gidx = torch.from_numpy(tables.gather_index(_nbr(coords, mask)))
    m = torch.from_numpy(mask)
    return coords, mask, x, w, bias, lnw, lnb, ray_idx, gidx, m, corb


def test_conv_ln_raytap_init_alpha_is_the_hex_conv():
    """alpha = (1, 0, 0, 0, 0) and every reach >= 1: each direction tap is its
    distance-1 neighbour, so K1 is the plain 7-tap conv + LN."""

    _, mask, x, w, bias, lnw, lnb, ray_idx, gidx, m, corb = _conv_case(11)
    b, n = mask.shape
    c = x.shape[2]
    alpha = torch.zeros(5, c, dtype=torch.float64)
    alpha[0] = 1
    reach = torch.from_numpy(np.random.default_rng(12).integers(1, 6, (b, n, 2, 6)).astype(np.uint8))
    for relu in (False, True):
        got = hexfield.conv_ln_raytap(x, gidx, m, w, bias, lnw, lnb, ray_idx, reach, alpha,
                                      1e-5, relu, corb)
        want = forward.hex_conv_ln(x, gidx, m, w, bias, lnw, lnb, 1e-5, relu)
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_conv_ln_raytap_is_the_factored_31_tap_conv():
    """Reach 5 everywhere: K1 == the 31-tap conv with W(t, k) = diag(alpha_k)
    W_t and W_self = W_0 (the factored identity of the ray-tap spec)."""

    _, mask, x, w, bias, lnw, lnb, ray_idx, gidx, m, corb = _conv_case(13)
    b, n = mask.shape
    c, cout = w.shape[1], w.shape[2]
    alpha = torch.randn(5, c, generator=torch.Generator().manual_seed(14)).double()
    reach = torch.full((b, n, 2, 6), 5, dtype=torch.uint8)
    w31 = torch.zeros(31, c, cout, dtype=torch.float64)
    w31[0] = w[0]
    lut = hexfield.tap_ray_slot_lut()
    for t in range(6):
        for k in range(5):
            w31[int(lut[t, k])] = alpha[k].view(c, 1) * w[1 + t]
    got = hexfield.conv_ln_raytap(x, gidx, m, w, bias, lnw, lnb, ray_idx, reach, alpha,
                                  1e-5, True, corb, round_fp16=False)
    want = forward.hex_conv_ln(x, ray_idx[:, :, :31], m, w31, bias, lnw, lnb, 1e-5, True)
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


def test_conv_ln_raytap_visibility_is_a_column_or_step_mask():
    """A side's reach 0 == that side's alpha columns zeroed (side(c) =
    (c mod corb) >= corb/2); a uniform reach r == alpha rows k > r zeroed."""

    _, mask, x, w, bias, lnw, lnb, ray_idx, gidx, m, corb = _conv_case(15)
    b, n = mask.shape
    c = x.shape[2]
    alpha = torch.randn(5, c, generator=torch.Generator().manual_seed(16)).double()
    five = torch.full((b, n, 2, 6), 5, dtype=torch.uint8)
    opp = (torch.arange(c) % corb) >= corb // 2

    def run(reach, a):
        return hexfield.conv_ln_raytap(x, gidx, m, w, bias, lnw, lnb, ray_idx, reach, a,
                                       1e-5, False, corb, round_fp16=False)

    own_blind = five.clone()
    own_blind[:, :, 0] = 0
    torch.testing.assert_close(run(own_blind, alpha * opp.double()), run(five, alpha * opp.double()))
    torch.testing.assert_close(run(own_blind, alpha), run(five, alpha * opp.double()),
                               rtol=1e-12, atol=1e-12)
    for r in range(6):
        cut = alpha.clone()
        cut[r:] = 0
        torch.testing.assert_close(run(torch.full_like(five, r), alpha), run(five, cut),
                                   rtol=1e-12, atol=1e-12)
