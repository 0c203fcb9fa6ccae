"""Pins the oracle's integer tables: golden tensors from the reference, the
reference's own geometry invariants (tests/test_shrimp_geometry.py:70-89) and
brute force."""

import numpy as np

from oracle import tables


def test_exact_rows_are_a_bijection_over_the_disk():
    disk = tables.exact_disk(8)
    assert len(disk) == 217
    rows = sorted(tables.rel_bias_row(dq, dr) for dq, dr in disk)
    assert rows == list(range(217))


def test_ring_and_far_rows():
    for d in range(9, 17):
        assert tables.rel_bias_row(d, 0) == 217 + d - 9
        assert tables.rel_bias_row(0, d) == 217 + d - 9
        assert tables.rel_bias_row(d, -d) == 217 + d - 9
        assert tables.rel_bias_row(d, -1) == 225 + d - 9
    assert tables.rel_bias_row(17, 0) == 233
    assert tables.rel_bias_row(40, -11) == 233


def test_lut_matches_unclamped_rows_everywhere():
    lut = tables.cell_lut()
    for dq in range(-40, 41):
        for dr in range(-40, 41):
            i = (min(max(dq, -17), 17) + 17) * 35 + min(max(dr, -17), 17) + 17
            assert lut[i] == tables.rel_bias_row(dq, dr), (dq, dr)


def test_pair_rows_match_reference_pair_tensors(golden):
    g = golden("pair")
    pu8 = tables.pair_rows(g["coords"], g["mask"], pad_row=237)
    np.testing.assert_array_equal(pu8, g["pair_u8"].astype(np.int64))
    pl = tables.pair_rows(g["coords"][:2], g["mask"][:2])
    np.testing.assert_array_equal(pl, g["pair_long"])


def test_pair_rows_torch_equals_numpy(golden):
    """The torch pair builder (the forward oracle's and the CPU baseline's)
    equals the pinned numpy rows bit for bit: golden positions with and
    without the pad row, and wide random boards whose offsets pass the
    +-17 clamp."""

    import torch

    g = golden("pair")
    for pad in (None, 237):
        got = tables.pair_rows_torch(g["coords"], g["mask"], pad_row=pad)
        assert got.dtype == torch.uint8
        np.testing.assert_array_equal(got.numpy().astype(np.int64),
                                      tables.pair_rows(g["coords"], g["mask"], pad_row=pad))
    rng = np.random.default_rng(11)
    coords = rng.integers(-30, 31, size=(3, 50, 2))
    mask = rng.random((3, 50)) > 0.3
    for pad in (None, 237):
        np.testing.assert_array_equal(
            tables.pair_rows_torch(coords, mask, pad_row=pad).numpy().astype(np.int64),
            tables.pair_rows(coords, mask, pad_row=pad))


def test_pair_rows_brute_force_on_small_board():
    rng = np.random.default_rng(0)
    coords = rng.integers(-20, 21, size=(2, 9, 2))
    mask = rng.random((2, 9)) > 0.2
    pair = tables.pair_rows(coords, mask, pad_row=237)
    for b in range(2):
        for i in range(17):
            for j in range(17):
                if j >= 8 and not mask[b, j - 8]:
                    want = 237
                elif i < 8 and j < 8:
                    want = 236
                elif i < 8:
                    want = 235
                elif j < 8:
                    want = 234
                else:
                    ci, cj = coords[b, i - 8], coords[b, j - 8]
                    want = tables.rel_bias_row(int(cj[0] - ci[0]), int(cj[1] - ci[1]))
                assert pair[b, i, j] == want


def test_seq_lens():
    mask = np.array([[1, 1, 0, 1, 0, 0], [0, 0, 0, 0, 0, 0], [1] * 6], dtype=bool)
    assert tables.seq_lens(mask).tolist() == [8 + 4, 8, 8 + 6]


def test_ray_index_matches_reference_join(golden):
    g = golden("ray_index")
    got = tables.ray_index(g["coords"], g["mask"])
    np.testing.assert_array_equal(got, g["idx"])


def test_ray_slot_geometry():
    off = tables.ray_slot_offsets()
    seen = set()
    for s in range(1, 31):
        q, r = int(off[s, 0]), int(off[s, 1])
        d = max(abs(q), abs(r), abs(q + r))
        assert 1 <= d <= 5
        assert q == 0 or r == 0 or q + r == 0  # on a win axis
        seen.add((q, r))
    assert len(seen) == 30
    # tap t's distance-1 neighbour slot lies along DIRECTIONS[t]
    for t, s in enumerate(tables.tap_ray_slots()):
        assert tuple(off[s]) == tables.DIRECTIONS[t]
