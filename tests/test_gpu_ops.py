"""Operator-level parity of the gfx950 kernels against the CPU oracle.

Inputs are rounded to bf16 before the oracle sees them, so the comparison
measures the kernels' own arithmetic (fp32 accumulation, bf16 output):
tolerance |got - want| <= 2e-2 + 1e-2 * |want| for bf16 outputs; integer
tables are bit-exact."""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import decode as odec
from oracle import forward as ofwd
from oracle import tables
from shrimp import ops as _ops  # noqa: F401  (registers torch.ops.shrimp.*)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(x):
    return torch.as_tensor(x).to(torch.bfloat16).to(torch.float64)


def close(got, want, atol=2e-2, rtol=1e-2, what=""):
    got = got.detach().to("cpu", torch.float64)
    want = want.detach().to("cpu", torch.float64)
    err = (got - want).abs() - rtol * want.abs()
    worst = err.max().item()
    assert worst <= atol, f"{what}: max excess error {worst}"


@pytest.fixture(params=[0, 1, 2, 3], ids=["auto", "global", "staged", "big"])
def conv_variant(request):
    """Runs a conv test with the automatic kernel choice (at these small
    batches: one 64-row tile per workgroup), with the global-gather kernel
    forced, with the small-tile LDS-staged kernel forced, and with the
    automatic choice minus the small-batch split (big-tile staged kernel for
    128 -> 128 channels, 7 taps)."""

    from shrimp import _lib

    lib = _lib.load()
    prev = lib.shrimp_conv_variant(request.param)
    try:
        yield request.param
    finally:
        lib.shrimp_conv_variant(prev)


@pytest.fixture(params=[0, 1, 2, 3], ids=["auto", "one_head", "four_waves", "chunked"])
def attn_variant(request):
    """Runs an attention test with the automatic kernel choice (two heads per
    workgroup; eight waves at head dim 16), with one head per workgroup, with
    two heads on four waves, and with the chunked kernel (keys streamed
    through LDS, the path of sequences too long for one workgroup's LDS)."""

    from shrimp import _lib

    lib = _lib.load()
    prev = lib.shrimp_attn_variant(request.param)
    try:
        yield request.param
    finally:
        lib.shrimp_attn_variant(prev)


@pytest.fixture(scope="module")
def conv_case():
    from shrimp import synthetic

    return synthetic.conv_inputs(6, channels=128)


def _gidx(batch):
    return torch.from_numpy(tables.gather_index(batch["nbr"].numpy()))


@pytest.mark.parametrize("epi", ["plain", "ln_relu", "ln"])
def test_hex_conv_ops(conv_case, epi, conv_variant):
    torch.manual_seed(0)
    b = conv_case["batch"]
    x = torch.from_numpy(conv_case["x"])
    w = torch.from_numpy(conv_case["w"])
    bias = torch.from_numpy(conv_case["bias"])
    gidx = _gidx(b)
    mask = b["mask"]
    lnw = torch.rand(128) + 0.5
    lnb = torch.randn(128) * 0.1
    if epi == "plain":
        got = torch.ops.shrimp.hex_conv(x.to(DEV), gidx.to(DEV), mask.to(DEV), w.to(DEV), bias.to(DEV))
        want = ofwd.hex_conv(bf(x), gidx, mask, bf(w), bias.double())
    else:
        relu = epi == "ln_relu"
        got = torch.ops.shrimp.hex_conv_ln(
            x.to(DEV), gidx.to(DEV), mask.to(DEV), w.to(DEV), bias.to(DEV), lnw.to(DEV),
            lnb.to(DEV), 1e-5, relu,
        )
        want = ofwd.hex_conv_ln(bf(x), gidx, mask, bf(w), bias.double(), lnw.double(),
                                lnb.double(), 1e-5, relu)
    assert got.dtype == torch.bfloat16 and got.shape == want.shape
    close(got, want, what=epi)
    assert (got.cpu()[~mask] == 0).all()


@pytest.mark.parametrize("c", [32, 64, 96, 192, 256])
def test_hex_conv_widths(c, conv_variant):
    from shrimp import synthetic

    case = synthetic.conv_inputs(2, channels=c)
    b = case["batch"]
    x, w, bias = (torch.from_numpy(case[k]) for k in ("x", "w", "bias"))
    gidx = _gidx(b)
    got = torch.ops.shrimp.hex_conv(x.to(DEV), gidx.to(DEV), b["mask"].to(DEV), w.to(DEV), bias.to(DEV))
    want = ofwd.hex_conv(bf(x), gidx, b["mask"], bf(w), bias.double())
    close(got, want, what=f"C={c}")


def test_conv_residual_and_head_epilogues(conv_case, conv_variant):
    from shrimp import ops

    b = conv_case["batch"]
    B, N = b["mask"].shape
    x = torch.from_numpy(conv_case["x"])
    w = torch.from_numpy(conv_case["w"])
    bias = torch.from_numpy(conv_case["bias"])
    gidx = _gidx(b)
    mask = b["mask"]
    g = torch.rand(128) * 0.5 + 0.5
    lnw = torch.rand(128) + 0.5
    lnb = torch.randn(128) * 0.1
    resid = torch.randn(B, N, 128) * mask[..., None]
    xd = x.to(DEV, torch.bfloat16).contiguous()
    idx = gidx.to(DEV, torch.int32).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    wp = ops.pack_conv_weight(w.to(DEV))
    out = resid.to(DEV, torch.bfloat16).contiguous()
    resid_bf = bf(resid)
    ops.launch_conv(
        x=xd, x_sb=N * 128, x_sn=128, idx=idx, taps=7, idx_stride=7, mask8=m8, wpack=wp,
        bias=bias.to(DEV), B=B, N=N, cin_pad=128, cout=128, ln_w=lnw.to(DEV), ln_b=lnb.to(DEV),
        resid=out, r_sb=N * 128, r_sn=128, gamma=g.to(DEV), out=out, o_sb=N * 128, o_sn=128,
    )
    y = ofwd.hex_conv_ln(bf(x), gidx, mask, bf(w), bias.double(), lnw.double(), lnb.double(), 1e-5, False)
    want = torch.relu(resid_bf + g.double() * y)
    close(out, want, what="residual")

    hw = torch.randn(128) * 0.1
    hb = torch.randn(1)
    head = torch.empty(B, N, device=DEV)
    ops.launch_conv(
        x=xd, x_sb=N * 128, x_sn=128, idx=idx, taps=7, idx_stride=7, mask8=m8, wpack=wp,
        bias=bias.to(DEV), B=B, N=N, cin_pad=128, cout=128, relu=True, head_w=hw.to(DEV),
        head_b=hb.to(DEV), head_out=head,
    )
    yc = torch.relu(ofwd.hex_conv(bf(x), gidx, mask, bf(w), bias.double()))
    want = (yc @ hw.double() + hb.double()) * mask.double()
    close(head, want, atol=1e-2, rtol=1e-3, what="head")
    assert (head.cpu()[~mask] == 0).all()


@pytest.fixture(scope="module")
def spec576_case():
    """36 spec-sized positions (supports past 512 cells among them) padded to
    576 cells, with N(0, 1) rows and a 7-tap 128 -> 128 weight."""

    from shrimp import synthetic
    from shrimp.batching import collate_rows

    rows = [r for r in synthetic.positions("cfg4_spec", 80, seed=57) if r[1].num_nodes <= 576]
    big = [r for r in rows if r[1].num_nodes > 512]
    rows = (big[:6] + [r for r in rows if r[1].num_nodes <= 512])[:36]
    b = collate_rows([(s, f) for _, s, f in rows], pad_to=576)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(36, 576, 128, generator=g) * b["mask"][..., None]
    w = torch.randn(7, 128, 128, generator=g) / math.sqrt(7 * 128)
    bias = torch.randn(128, generator=g) * 0.02
    return b, x, w, bias


def test_conv_past_512_rows_split_over_two_workgroups(spec576_case):
    """Npad 576 at a batch of 36 positions runs the big-tile conv with each
    position's rows split over two workgroups of three waves (each staging the
    whole position): conv + LN + ReLU, the LayerScale residual and the policy
    head against the fp64 oracle; the same rows through two batches of 18
    (the row-split kernel) agree to the bf16 tolerance."""

    from shrimp import ops

    b, x, w, bias = spec576_case
    mask = b["mask"]
    B, N = mask.shape
    assert B >= 32 and N == 576 and int(mask.sum(1).max()) > 512
    gidx = _gidx(b)
    g = torch.rand(128) * 0.5 + 0.5
    lnw = torch.rand(128) + 0.5
    lnb = torch.randn(128) * 0.1
    xd = x.to(DEV, torch.bfloat16).contiguous()
    idx = gidx.to(DEV, torch.int32).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    wp = ops.pack_conv_weight(w.to(DEV))
    common = dict(x_sb=N * 128, x_sn=128, taps=7, idx_stride=7, wpack=wp, bias=bias.to(DEV),
                  cin_pad=128, cout=128)
    print("spec576 conv ln_relu", flush=True)
    y1 = torch.empty(B, N, 128, dtype=torch.bfloat16, device=DEV)
    ops.launch_conv(x=xd, idx=idx, mask8=m8, B=B, N=N, ln_w=lnw.to(DEV), ln_b=lnb.to(DEV),
                    relu=True, out=y1, o_sb=N * 128, o_sn=128, **common)
    want = ofwd.hex_conv_ln(bf(x), gidx, mask, bf(w), bias.double(), lnw.double(), lnb.double(),
                            1e-5, True)
    close(y1, want, what="ln_relu N=576")
    assert (y1.cpu()[~mask] == 0).all()
    # the same positions in two batches of 18 (row-split kernel)
    halves = torch.empty_like(y1)
    for h0 in (0, 18):
        ops.launch_conv(x=xd[h0:h0 + 18], idx=idx[h0:h0 + 18], mask8=m8[h0:h0 + 18], B=18, N=N,
                        ln_w=lnw.to(DEV), ln_b=lnb.to(DEV), relu=True, out=halves[h0:h0 + 18],
                        o_sb=N * 128, o_sn=128, **common)
    close(halves, y1.double().cpu(), what="split vs row-split N=576")
    print("spec576 conv residual", flush=True)
    resid = torch.randn(B, N, 128) * mask[..., None]
    out = resid.to(DEV, torch.bfloat16).contiguous()
    ops.launch_conv(x=xd, idx=idx, mask8=m8, B=B, N=N, ln_w=lnw.to(DEV), ln_b=lnb.to(DEV),
                    resid=out, r_sb=N * 128, r_sn=128, gamma=g.to(DEV), out=out, o_sb=N * 128,
                    o_sn=128, **common)
    y = ofwd.hex_conv_ln(bf(x), gidx, mask, bf(w), bias.double(), lnw.double(), lnb.double(),
                         1e-5, False)
    close(out, torch.relu(bf(resid) + g.double() * y), what="residual N=576")
    print("spec576 conv head", flush=True)
    hw = torch.randn(128) * 0.1
    hb = torch.randn(1)
    head = torch.empty(B, N, device=DEV)
    ops.launch_conv(x=xd, idx=idx, mask8=m8, B=B, N=N, relu=True, head_w=hw.to(DEV),
                    head_b=hb.to(DEV), head_out=head, **common)
    yc = torch.relu(ofwd.hex_conv(bf(x), gidx, mask, bf(w), bias.double()))
    close(head, (yc @ hw.double() + hb.double()) * mask.double(), atol=1e-2, rtol=1e-3,
          what="head N=576")
    assert (head.cpu()[~mask] == 0).all()


def _block_case(conv_case, n):
    """conv_case cut (n < 256) or zero-padded (n > 256) to n cells per position;
    neighbours outside [0, n) become the sentinel n."""

    b = conv_case["batch"]
    x = torch.from_numpy(conv_case["x"])
    gidx = _gidx(b)
    mask = b["mask"]
    B, N0 = mask.shape
    if n <= N0:
        x, gidx, mask = x[:, :n], gidx[:, :n].clone(), mask[:, :n]
        gidx[(gidx < 0) | (gidx >= n)] = n
    else:
        x = torch.cat([x, torch.zeros(B, n - N0, 128)], 1)
        gidx = torch.where(gidx >= N0, torch.full_like(gidx, n), gidx)
        pad = torch.full((B, n - N0, 7), n, dtype=gidx.dtype)
        pad[..., 0] = torch.arange(N0, n)
        gidx = torch.cat([gidx, pad], 1)
        mask = torch.cat([mask, torch.zeros(B, n - N0, dtype=mask.dtype)], 1)
    return x * mask[..., None], gidx.contiguous(), mask.contiguous()


@pytest.mark.parametrize("n", [256, 64, 200, 300, 512])
def test_conv_block_fused(conv_case, n):
    """ConvBlock in one launch (y1 kept in LDS) against the two-launch path
    (bit-identical: same MFMA order, same epilogue arithmetic, y1 rounded to
    bf16 either way) and against the oracle's ConvBlock (model.py:419-421)."""

    from shrimp import ops

    torch.manual_seed(n)
    x, gidx, mask = _block_case(conv_case, n)
    B, N = mask.shape
    w1 = torch.from_numpy(conv_case["w"])
    w2 = torch.randn(7, 128, 128) / math.sqrt(7 * 128)
    b1 = torch.from_numpy(conv_case["bias"])
    b2 = torch.randn(128) * 0.02
    l1w, l2w = torch.rand(128) + 0.5, torch.rand(128) + 0.5
    l1b, l2b = torch.randn(128) * 0.1, torch.randn(128) * 0.1
    g = torch.rand(128) * 0.5 + 0.5
    assert ops.conv_block_supported(7, N, 128, 128)
    d = {k: v.to(DEV) for k, v in dict(b1=b1, b2=b2, l1w=l1w, l2w=l2w, l1b=l1b, l2b=l2b, g=g).items()}
    idx = gidx.to(DEV, torch.int32).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    wp1, wp2 = ops.pack_conv_weight(w1.to(DEV)), ops.pack_conv_weight(w2.to(DEV))
    xd = x.to(DEV, torch.bfloat16).contiguous()
    print(f"conv_block n={N} B={B}", flush=True)

    fused = xd.clone()  # in place, as the forward runs it
    ops.launch_conv_block(
        x=fused, x_sb=N * 128, x_sn=128, idx=idx, idx_stride=7, mask8=m8, B=B, N=N, C=128,
        w1=wp1, b1=d["b1"], ln1_w=d["l1w"], ln1_b=d["l1b"], eps1=1e-5, w2=wp2, b2=d["b2"],
        ln2_w=d["l2w"], ln2_b=d["l2b"], eps2=1e-5, gamma=d["g"], out=fused, o_sb=N * 128, o_sn=128,
    )
    y1 = torch.empty_like(xd)
    common = dict(idx=idx, taps=7, idx_stride=7, mask8=m8, B=B, N=N, cin_pad=128, cout=128)
    # the big-tile convs (this small batch would otherwise take the row split,
    # whose products run in another order)
    from shrimp import _lib

    prev = _lib.load().shrimp_conv_variant(3)
    try:
        ops.launch_conv(x=xd, x_sb=N * 128, x_sn=128, wpack=wp1, bias=d["b1"], ln_w=d["l1w"],
                        ln_b=d["l1b"], relu=True, out=y1, o_sb=N * 128, o_sn=128, **common)
        two = xd.clone()
        ops.launch_conv(x=y1, x_sb=N * 128, x_sn=128, wpack=wp2, bias=d["b2"], ln_w=d["l2w"],
                        ln_b=d["l2b"], resid=two, r_sb=N * 128, r_sn=128, gamma=d["g"], out=two,
                        o_sb=N * 128, o_sn=128, **common)
        torch.cuda.synchronize()
    finally:
        _lib.load().shrimp_conv_variant(prev)
    diff = (fused.float() - two.float()).abs().max().item()
    print(f"fused vs two launches: max diff {diff:.3e}", flush=True)
    assert torch.equal(fused, two)

    if N <= 256:
        bx = bf(x)
        y = ofwd.hex_conv_ln(bx, gidx, mask, bf(w1), b1.double(), l1w.double(), l1b.double(), 1e-5, True)
        y = ofwd.hex_conv_ln(bf(y), gidx, mask, bf(w2), b2.double(), l2w.double(), l2b.double(), 1e-5, False)
        want = torch.relu(bx + g.double() * y)
        close(fused, want, what=f"conv block n={N}")
    assert (fused.cpu()[~mask] == 0).all()


@pytest.mark.parametrize("n", [256, 64, 200, 300])
def test_conv_block_pair_matches_two_blocks(conv_case, n):
    """Two ConvBlocks in one launch (the first block's output rows handed to
    the second in LDS) against two shrimp_conv_block launches: bit-identical,
    including the masked rows and the rows past N (the zero row)."""

    from shrimp import ops

    torch.manual_seed(100 + n)
    x, gidx, mask = _block_case(conv_case, n)
    B, N = mask.shape
    assert ops.conv_block_pair_supported(7, N, 128, 128)
    blocks = []
    for _ in range(2):
        blocks.append(dict(
            w1=ops.pack_conv_weight((torch.randn(7, 128, 128) / math.sqrt(7 * 128)).to(DEV)),
            b1=(torch.randn(128) * 0.02).to(DEV), ln1_w=(torch.rand(128) + 0.5).to(DEV),
            ln1_b=(torch.randn(128) * 0.1).to(DEV), eps1=1e-5,
            w2=ops.pack_conv_weight((torch.randn(7, 128, 128) / math.sqrt(7 * 128)).to(DEV)),
            b2=(torch.randn(128) * 0.02).to(DEV), ln2_w=(torch.rand(128) + 0.5).to(DEV),
            ln2_b=(torch.randn(128) * 0.1).to(DEV), eps2=1e-5,
            gamma=(torch.rand(128) * 0.5 + 0.5).to(DEV)))
    idx = gidx.to(DEV, torch.int32).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    xd = x.to(DEV, torch.bfloat16).contiguous()
    print(f"conv_block_pair n={N} B={B}", flush=True)
    common = dict(idx=idx, idx_stride=7, mask8=m8, B=B, N=N, C=128)
    two = xd.clone()
    for blk in blocks:
        ops.launch_conv_block(x=two, x_sb=N * 128, x_sn=128, out=two, o_sb=N * 128, o_sn=128,
                              **common, **blk)
    pair = xd.clone()
    ops.launch_conv_block_pair(x=pair, x_sb=N * 128, x_sn=128, blocks=blocks, out=pair,
                               o_sb=N * 128, o_sn=128, **common)
    # out of place: the first block reads x and writes out
    oop = torch.zeros_like(xd)
    ops.launch_conv_block_pair(x=xd, x_sb=N * 128, x_sn=128, blocks=blocks, out=oop,
                               o_sb=N * 128, o_sn=128, **common)
    torch.cuda.synchronize()
    diff = (pair.float() - two.float()).abs().max().item()
    print(f"pair vs two launches: max diff {diff:.3e}", flush=True)
    assert torch.equal(pair, two)
    assert torch.equal(oop, two)
    assert (pair.cpu()[~mask] == 0).all()


def test_conv_block_pair_rejects_mismatched_blocks(conv_case):
    """The second block must read the first block's output with the same index,
    mask and shape."""

    from shrimp import _lib, ops

    x, gidx, mask = _block_case(conv_case, 64)
    B, N = mask.shape
    idx = gidx.to(DEV, torch.int32).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    xd = x.to(DEV, torch.bfloat16).contiguous()
    other = torch.zeros_like(xd)
    blk = dict(w1=ops.pack_conv_weight(torch.zeros(7, 128, 128, device=DEV)),
               b1=torch.zeros(128, device=DEV), ln1_w=torch.ones(128, device=DEV),
               ln1_b=torch.zeros(128, device=DEV), eps1=1e-5,
               w2=ops.pack_conv_weight(torch.zeros(7, 128, 128, device=DEV)),
               b2=torch.zeros(128, device=DEV), ln2_w=torch.ones(128, device=DEV),
               ln2_b=torch.zeros(128, device=DEV), eps2=1e-5, gamma=torch.ones(128, device=DEV))
    c1, c2 = ops._block_args(xd, N * 128, 128, idx, 7, m8, B, N, 128, out=xd, o_sb=N * 128,
                             o_sn=128, **blk)
    c3, c4 = ops._block_args(other, N * 128, 128, idx, 7, m8, B, N, 128, out=other,
                             o_sb=N * 128, o_sn=128, **blk)
    lib = _lib.load()
    rc = lib.shrimp_conv_block_pair(ops.ctypes_ref(c1), ops.ctypes_ref(c2), ops.ctypes_ref(c3),
                                    ops.ctypes_ref(c4), None)
    assert rc != 0
    assert b"first block's output" in lib.shrimp_last_error()


def test_conv_block_rejects_other_shapes(conv_case):
    from shrimp import _lib, ops

    lib = _lib.load()
    assert not ops.conv_block_supported(7, 576, 128, 128)
    assert not ops.conv_block_supported(7, 256, 64, 64)
    assert not ops.conv_block_supported(31, 256, 128, 128)
    prev = lib.shrimp_conv_variant(1)
    try:
        assert not ops.conv_block_supported(7, 256, 128, 128)
    finally:
        lib.shrimp_conv_variant(prev)
    x = torch.zeros(1, 576, 128, dtype=torch.bfloat16, device=DEV)
    z = torch.zeros(128, device=DEV)
    wp = torch.zeros(7 * 128 * 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="conv_block"):
        ops.launch_conv_block(
            x=x, x_sb=576 * 128, x_sn=128, idx=torch.zeros(1, 576, 7, dtype=torch.int32, device=DEV),
            idx_stride=7, mask8=torch.zeros(1, 576, dtype=torch.uint8, device=DEV), B=1, N=576,
            C=128, w1=wp, b1=z, ln1_w=z, ln1_b=z, eps1=1e-5, w2=wp, b2=z, ln2_w=z, ln2_b=z,
            eps2=1e-5, gamma=z, out=x, o_sb=576 * 128, o_sn=128,
        )


@pytest.mark.parametrize("c", [32, 128])
def test_hex_conv_multi_tile_positions(c, conv_variant):
    """Spec-variant positions (Npad = ceil64(max N) > 256: several row tiles
    per position in the staged kernel, N not a multiple of the tile)."""

    from shrimp import synthetic

    b = synthetic.position_batch("cfg4_spec", 3, seed=11)
    B, N = b["mask"].shape
    assert N > 256
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((B, N, c), dtype=np.float32))
    w = torch.from_numpy(rng.standard_normal((7, c, 128), dtype=np.float32) / np.sqrt(7 * c))
    bias = torch.from_numpy(rng.standard_normal(128, dtype=np.float32) * 0.02)
    gidx = _gidx(b)
    got = torch.ops.shrimp.hex_conv(x.to(DEV), gidx.to(DEV), b["mask"].to(DEV), w.to(DEV), bias.to(DEV))
    want = ofwd.hex_conv(bf(x), gidx, b["mask"], bf(w), bias.double())
    close(got, want, what=f"N={N} C={c}")


def test_conv_variants_agree_at_full_shape():
    """At config 1's row shape (Npad=256, C=128) with B=512 positions (config
    1 itself, B=1024, is test_cfg1_conv_bias_relu): the global-gather and the
    staged kernels issue the same MFMA sequence on the same operands
    (bit-identical outputs); the big-tile kernel sums the same products in
    another order (channel chunk before tap), so it agrees to fp32 rounding:
    at most one bf16 ulp on a few elements."""

    from shrimp import _lib, synthetic

    case = synthetic.conv_inputs(512, channels=128)
    b = case["batch"]
    x, w, bias = (torch.from_numpy(case[k]).to(DEV) for k in ("x", "w", "bias"))
    gidx, mask = _gidx(b).to(DEV), b["mask"].to(DEV)
    lnw = torch.rand(128, device=DEV) + 0.5
    lnb = torch.randn(128, device=DEV) * 0.1
    lib = _lib.load()
    outs = []
    for v in (3, 1, 2):
        prev = lib.shrimp_conv_variant(v)
        try:
            outs.append(torch.ops.shrimp.hex_conv_ln(x, gidx, mask, w, bias, lnw, lnb, 1e-5, True))
        finally:
            lib.shrimp_conv_variant(prev)
    assert torch.equal(outs[1], outs[2])
    a, c = outs[0].float(), outs[1].float()
    diff = (a - c).abs()
    # one bf16 ulp of the larger value, plus 1e-5 absolute for outputs at the
    # ReLU edge (fp32 reordering moves the LayerNorm output by ~1e-6 there)
    ulp = torch.maximum(a.abs(), c.abs()) * 2.0 ** -7 + 1e-5
    frac = (diff > 0).float().mean().item()
    print(f"big-tile vs global: max diff {diff.max().item():.3e}, {frac:.4f} of outputs differ, "
          f"worst / allowed {(diff / ulp).max().item():.3f}", flush=True)
    assert (diff <= ulp).all()
    assert frac < 0.05
    print(f"max LDS per block: {lib.shrimp_max_lds_per_block()} bytes", flush=True)


def test_prep_pair_and_ray_index_exact(golden):
    from shrimp import _lib

    g = golden("pair")
    coords = torch.from_numpy(g["coords"])
    mask = torch.from_numpy(g["mask"])
    B, N = mask.shape
    nbr = torch.from_numpy(golden("forward_cfg0")["nbr"])
    lib = _lib.load()
    idx = torch.empty(B, N, 7, dtype=torch.int32, device=DEV)
    m8 = torch.empty(B, N, dtype=torch.uint8, device=DEV)
    c32 = torch.empty(B, N, 2, dtype=torch.int32, device=DEV)
    sl = torch.empty(B, dtype=torch.int32, device=DEV)
    sm = torch.empty(B, N + 8, dtype=torch.uint8, device=DEV)
    nb = nbr.to(DEV)
    md = mask.to(DEV)
    cd = coords.to(DEV)
    _lib.check(lib.shrimp_prep_inputs(nb.data_ptr(), _lib.DT_I64, md.data_ptr(), cd.data_ptr(),
                                      _lib.DT_I64, None, 0, 0, B, N, 8, idx.data_ptr(), m8.data_ptr(),
                                      c32.data_ptr(), sl.data_ptr(), sm.data_ptr(), None,
                                      _lib.stream_handle()), "prep")
    np.testing.assert_array_equal(idx.cpu().numpy(), tables.gather_index(nbr.numpy()))
    np.testing.assert_array_equal(sl.cpu().numpy(), tables.seq_lens(mask.numpy()))
    np.testing.assert_array_equal(c32.cpu().numpy(), coords.numpy())
    np.testing.assert_array_equal(sm.cpu().numpy()[:, 8:], mask.numpy())
    assert (sm.cpu().numpy()[:, :8] == 1).all()

    lut = torch.from_numpy(tables.cell_lut()).to(DEV)
    pair = torch.empty(B, N + 8, N + 8, dtype=torch.uint8, device=DEV)
    _lib.check(lib.shrimp_build_pair_u8(c32.data_ptr(), m8.data_ptr(), lut.data_ptr(), 17, B, N, 8,
                                        234, 235, 236, 237, pair.data_ptr(), _lib.stream_handle()),
               "pair")
    np.testing.assert_array_equal(pair.cpu().numpy(), g["pair_u8"])

    ridx = torch.empty(B, N, 32, dtype=torch.int32, device=DEV)
    _lib.check(lib.shrimp_build_ray_index(c32.data_ptr(), m8.data_ptr(), B, N, ridx.data_ptr(),
                                          _lib.stream_handle()), "ray")
    np.testing.assert_array_equal(ridx.cpu().numpy(), golden("ray_index")["idx"])


def test_raytap_conv_31_taps(conv_variant):
    from shrimp import _lib, ops, synthetic

    case = synthetic.raytap_inputs(4, channels=128)
    b = case["batch"]
    B, N = b["mask"].shape
    coords = b["coords"].to(torch.int32)
    mask = b["mask"]
    ridx = torch.from_numpy(tables.ray_index(coords.numpy(), mask.numpy()))
    x, w, bias = (torch.from_numpy(case[k]) for k in ("x", "w", "bias"))
    lib = _lib.load()
    c32 = coords.to(DEV).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    idx = torch.empty(B, N, 32, dtype=torch.int32, device=DEV)
    _lib.check(lib.shrimp_build_ray_index(c32.data_ptr(), m8.data_ptr(), B, N, idx.data_ptr(),
                                          _lib.stream_handle()), "ray")
    assert torch.equal(idx.cpu(), ridx)
    out = torch.empty(B, N, 128, dtype=torch.bfloat16, device=DEV)
    ops.launch_conv(
        x=x.to(DEV, torch.bfloat16).contiguous(), x_sb=N * 128, x_sn=128, idx=idx, taps=31,
        idx_stride=32, mask8=m8, wpack=ops.pack_conv_weight(w.to(DEV)), bias=bias.to(DEV),
        B=B, N=N, cin_pad=128, cout=128, out=out, o_sb=N * 128, o_sn=128,
    )
    want = ofwd.raytap_conv(bf(x), ridx, mask, bf(w), bias.double())
    close(out, want, what="raytap")


@pytest.mark.parametrize("mode", ["qkv", "gelu", "resid", "plain"])
@pytest.mark.parametrize("c", [32, 128])
def test_linear_modes(mode, c):
    from shrimp import _lib, ops

    torch.manual_seed(1)
    B, S, H = 3, 40, 4 if c == 32 else 8
    d = c // H
    dpad = max(16, -(-d // 16) * 16)
    rows = B * S
    n_in = 2 * c if mode == "resid" else c
    n_out = {"qkv": 3 * c, "gelu": 2 * c, "resid": c, "plain": c}[mode]
    x = torch.randn(rows, n_in)
    w = torch.randn(n_out, n_in) * 0.1
    bias = torch.randn(n_out) * 0.1
    lnw = torch.rand(n_in) + 0.5
    lnb = torch.randn(n_in) * 0.1
    use_ln = mode in ("qkv", "gelu")
    xd = x.to(DEV, torch.bfloat16).contiguous()
    wp = ops.pack_linear_weight(w.to(DEV))
    xin = bf(x)
    if use_ln:
        xin = torch.nn.functional.layer_norm(xin, (n_in,), lnw.double(), lnb.double(), 1e-5)
        xin = bf(xin)  # the kernel feeds normalised rows to MFMA in bf16
    y = xin @ bf(w).T + bias.double()
    kw = dict(x=xd, x_sr=n_in, wpack=wp, bias=bias.to(DEV), rows=rows, n_in=n_in, n_out=n_out)
    if use_ln:
        kw.update(ln_w=lnw.to(DEV), ln_b=lnb.to(DEV), eps=1e-5)
    if mode == "qkv":
        out = torch.zeros(3, B, H, S, dpad, dtype=torch.bfloat16, device=DEV)
        ops.launch_linear(mode=_lib.LIN_QKV, out=out, B=B, S=S, H=H, dpad=dpad, **kw)
        want = y.reshape(B, S, 3, H, d).permute(2, 0, 3, 1, 4)
        close(out[..., :d], want, what="qkv")
        assert (out[..., d:] == 0).all()
    elif mode == "gelu":
        out = torch.empty(rows, n_out, dtype=torch.bfloat16, device=DEV)
        ops.launch_linear(mode=_lib.LIN_GELU, out=out, o_sr=n_out, **kw)
        close(out, torch.nn.functional.gelu(y), what="gelu")
    elif mode == "resid":
        res = torch.randn(rows, n_out)
        g = torch.rand(n_out)
        m = (torch.rand(rows) > 0.3)
        out = res.to(DEV, torch.bfloat16).contiguous()
        ops.launch_linear(mode=_lib.LIN_RESID, out=out, o_sr=n_out, resid=out, r_sr=n_out,
                          gamma=g.to(DEV), mask=m.to(DEV, torch.uint8), **kw)
        close(out, bf(res) + g.double() * y * m.double()[:, None], what="resid")
    else:
        out = torch.empty(rows, n_out, dtype=torch.bfloat16, device=DEV)
        ops.launch_linear(mode=_lib.LIN_PLAIN, out=out, o_sr=n_out, **kw)
        close(out, y, what="plain")


def _mlp_case(rows, seed=2):
    torch.manual_seed(seed)
    c, hdim = 128, 256
    x = torch.randn(rows, c)
    seq = torch.randn(rows, c)
    m = torch.rand(rows) > 0.25
    wo, bo = torch.randn(c, c) * 0.08, torch.randn(c) * 0.1
    w1, b1 = torch.randn(hdim, c) * 0.08, torch.randn(hdim) * 0.1
    w2, b2 = torch.randn(c, hdim) * 0.06, torch.randn(c) * 0.1
    ga, gm = torch.rand(c) * 0.5 + 0.25, torch.rand(c) * 0.5 + 0.25
    lnw, lnb = torch.rand(c) + 0.5, torch.randn(c) * 0.1
    return x, seq, m, (wo, bo, ga, lnw, lnb, w1, b1, w2, b2, gm)


def _mlp_restated(x, s_in, m, p):
    """AttnBlock's tail in float64 with the kernel's bf16 points (MFMA inputs:
    x, the LayerNorm output, the GELU output and the folded weights); s1 and
    the result stay unrounded (the kernel rounds only its stores)."""

    wo, bo, ga, lnw, lnb, w1, b1, w2, b2, gm = p
    c = x.shape[1]
    d = lambda t: t.double()
    s1 = d(s_in) + (bf(x) @ bf(ga[:, None] * wo).T + d(ga * bo)) * d(m)[:, None]
    n = bf(torch.nn.functional.layer_norm(s1, (c,), None, None, 1e-5))
    hid = bf(torch.nn.functional.gelu(n @ bf(w1 * lnw[None, :]).T + d(b1) + d(w1) @ d(lnb)))
    return s1 + (hid @ bf(gm[:, None] * w2).T + d(gm * b2)) * d(m)[:, None]


@pytest.mark.parametrize("rows", [1, 37, 4096 + 5])
def test_attn_mlp_fused(rows):
    """Fused out_proj + LayerScale residual + LN2 + fc1 + GELU(erf) + fc2 +
    residual (C=128) against a float64 restatement of AttnBlock's tail with
    the kernel's bf16 points (MFMA inputs; s1 stays fp32 inside the kernel as
    the fc2 accumulators' start, and only the stored result is rounded). The
    kernel folds the LayerScales and LN2's affine into the weights before
    rounding them to bf16, so the reference rounds the folded weights the
    same way. Row counts cover a single row, a ragged block and several
    blocks per wave; masked rows must keep their residual exactly."""

    from shrimp import ops

    x, seq, m, p = _mlp_case(rows)
    wo, bo, ga, lnw, lnb, w1, b1, w2, b2, gm = p
    c, hdim = 128, 256
    d = lambda t: t.double()
    want = _mlp_restated(x, bf(seq), m, p)
    # the same block in the model's own terms (unfolded fp64): within bf16 noise
    s1u = d(seq) + d(ga) * ((d(x) @ d(wo).T + d(bo)) * d(m)[:, None])
    hu = torch.nn.functional.gelu(
        torch.nn.functional.layer_norm(s1u, (c,), d(lnw), d(lnb), 1e-5) @ d(w1).T + d(b1))
    model = s1u + d(gm) * ((hu @ d(w2).T + d(b2)) * d(m)[:, None])

    seq_d = seq.to(DEV, torch.bfloat16).contiguous()
    g = lambda t: t.to(DEV)
    packed = ops.pack_attn_mlp(g(wo), g(bo), g(ga), g(lnw), g(lnb), g(w1), g(b1), g(w2), g(b2), g(gm))
    ops.launch_attn_mlp(x=x.to(DEV, torch.bfloat16).contiguous(), x_sr=c, seq=seq_d, s_sr=c,
                        mask=m.to(DEV, torch.uint8), packed=packed, eps=1e-5, rows=rows, C=c,
                        hidden=hdim)
    close(seq_d, want, what=f"attn_mlp rows={rows}")
    close(seq_d, model, atol=5e-2, rtol=2e-2, what=f"attn_mlp vs model rows={rows}")
    assert torch.equal(seq_d.cpu()[~m].double(), bf(seq)[~m])


def test_attn_mlp_token_low_parts():
    """The token rows (the first n_tokens of every S rows) carry a second
    bf16, their rounding remainder: the kernel reads seq + tok_lo as the
    residual and writes the new remainder, so hi + lo follows the fp64
    restatement to about 2^-16 relative (a bf16 stream alone: 2^-9), while
    cell rows are exactly the same as without tok_lo and tok_lo bytes of
    cells are never touched. Masked token rows keep hi and lo."""

    from shrimp import ops

    B, S, nt, c = 5, 24, 8, 128
    rows = B * S
    x, seq, m, p = _mlp_case(rows, seed=3)
    m[S + 2] = False  # a masked token row
    hi = seq.to(torch.bfloat16)
    lo = (seq - hi.float()).to(torch.bfloat16)
    tok = (torch.arange(rows) % S) < nt
    d_in = hi.double() + torch.where(tok[:, None], lo.double(), torch.zeros(1).double())
    want = _mlp_restated(x, d_in, m, p)
    wo, bo, ga, lnw, lnb, w1, b1, w2, b2, gm = p
    g = lambda t: t.to(DEV)
    packed = ops.pack_attn_mlp(g(wo), g(bo), g(ga), g(lnw), g(lnb), g(w1), g(b1), g(w2), g(b2), g(gm))
    xd = x.to(DEV, torch.bfloat16).contiguous()
    md = m.to(DEV, torch.uint8)

    seq_a = hi.to(DEV).contiguous()
    lo_d = lo.reshape(B, S, c)[:, :nt].to(DEV).contiguous()
    ops.launch_attn_mlp(x=xd, x_sr=c, seq=seq_a, s_sr=c, mask=md, packed=packed, eps=1e-5,
                        rows=rows, C=c, hidden=256, tok_lo=lo_d, S=S, n_tokens=nt)
    seq_b = hi.to(DEV).contiguous()
    ops.launch_attn_mlp(x=xd, x_sr=c, seq=seq_b, s_sr=c, mask=md, packed=packed, eps=1e-5,
                        rows=rows, C=c, hidden=256)
    got_hi = seq_a.cpu().double()
    got_lo = torch.zeros(rows, c, dtype=torch.float64)
    got_lo.view(B, S, c)[:, :nt] = lo_d.cpu().double()
    got = got_hi + got_lo
    tw = want[tok]
    e_both = (got[tok] - tw).abs() / tw.abs().clamp(min=1.0)
    e_hi = (got_hi[tok] - tw).abs() / tw.abs().clamp(min=1.0)
    print(f"token rows: hi + lo rel err mean {e_both.mean().item():.3e} max "
          f"{e_both.max().item():.3e}; hi alone mean {e_hi.mean().item():.3e} max "
          f"{e_hi.max().item():.3e}", flush=True)
    # hi + lo: fp32 accumulation, plus the odd element where the kernel and the
    # restatement round a LayerNorm or GELU value to different bf16 neighbours;
    # hi alone: a quarter of a bf16 ulp on average (~1e-3 relative)
    assert e_both.max().item() <= 2e-3
    assert e_both.mean().item() * 8 <= e_hi.mean().item()
    # cell rows: identical to the call without low parts
    assert torch.equal(seq_a.cpu()[~tok], seq_b.cpu()[~tok])
    close(seq_a[~tok.to(DEV)], want[~tok], what="attn_mlp cells with tok_lo")
    # the masked token row keeps its hi and lo
    assert torch.equal(seq_a.cpu()[S + 2], hi[S + 2])
    assert torch.equal(lo_d.cpu()[1, 2], lo.reshape(B, S, c)[1, 2])


@pytest.mark.parametrize("h,dpad", [(8, 16), (4, 32), (2, 64)])
def test_attn_qkv_fused(h, dpad):
    """LN1 + q/k/v projection (C=128) into the head-major layout against a
    float64 restatement; LN1's affine is folded into the bf16 weights the same
    way the packer folds it. Padding lanes past d are never written."""

    from shrimp import ops

    torch.manual_seed(3)
    c, B, S = 128, 3, 45
    rows, d = B * S, c // h
    x = torch.randn(rows, c) * 2 + 0.5
    w, b = torch.randn(3 * c, c) * 0.08, torch.randn(3 * c) * 0.1
    lnw, lnb = torch.rand(c) + 0.5, torch.randn(c) * 0.1
    n = bf(torch.nn.functional.layer_norm(bf(x), (c,), None, None, 1e-5))
    y = n @ bf(w * lnw[None, :]).T + (b.double() + w.double() @ lnb.double())
    want = y.reshape(B, S, 3, h, d).permute(2, 0, 3, 1, 4)
    model = (torch.nn.functional.layer_norm(bf(x), (c,), lnw.double(), lnb.double(), 1e-5)
             @ w.double().T + b.double()).reshape(B, S, 3, h, d).permute(2, 0, 3, 1, 4)
    out = torch.full((3, B, h, S, dpad), 7.0, dtype=torch.bfloat16, device=DEV)
    packed = ops.pack_attn_qkv(w.to(DEV), b.to(DEV), lnw.to(DEV), lnb.to(DEV))
    ops.launch_attn_qkv(x=x.to(DEV, torch.bfloat16).contiguous(), x_sr=c, qkv=out,
                        packed=packed, eps=1e-5, rows=rows, B=B, S=S, H=h, C=c, dpad=dpad)
    close(out[..., :d], want, what=f"qkv H={h}")
    close(out[..., :d], model, atol=4e-2, rtol=2e-2, what=f"qkv vs model H={h}")
    assert (out[..., d:].float() == 7.0).all()


def test_attn_mlp_pack_rejects_other_shapes():
    from shrimp import ops

    z = lambda *s: torch.zeros(*s, device=DEV)
    assert ops.pack_attn_mlp(z(64, 64), z(64), z(64), z(64), z(64), z(128, 64), z(128),
                             z(64, 128), z(64), z(64)) is None


# query-block counts 5, 4, 2 and 9, 9, 3: a leftover block split over four
# waves (5), over four and over eight waves (9), and none
@pytest.mark.parametrize("S,lens", [(70, [70, 61, 23]), (140, [140, 129, 33])])
@pytest.mark.parametrize("d", [16, 32, 64])
def test_attn_pair_op(d, S, lens, attn_variant):
    torch.manual_seed(2)
    B, H = 3, 4
    q, k, v = (torch.randn(B, H, S, d) for _ in range(3))
    rows = 238
    table2 = torch.randn(rows, H) * 0.5
    table2[rows - 1] = -3.0e4
    pair = torch.randint(0, rows - 1, (B, S, S), dtype=torch.uint8)
    pair[1, :, 50:60] = rows - 1  # pad keys inside the bound
    lens = torch.tensor(lens, dtype=torch.int32)
    got = torch.ops.shrimp.attn_pair(q.to(DEV), k.to(DEV), v.to(DEV), pair.to(DEV),
                                     table2.to(DEV), lens.to(DEV))
    want = ofwd.attn_pair(bf(q), bf(k), bf(v), pair, table2.double(), lens)
    close(got, want, atol=1e-2, what=f"attn d={d}")


@pytest.mark.parametrize("qk_gain", [1.0, 12.0])
def test_attn_offset_table_cfg2(attn_variant, qk_gain):
    """Config 2's attention at B=4 against the oracle; qk_gain 12 gives
    softmax rows dominated by one key (scores spread over ~100 in log2
    units)."""

    from shrimp import ops, synthetic

    case = synthetic.attention_inputs(4, heads=8, d=16)
    q, k, v = (torch.from_numpy(case[n]) for n in ("q", "k", "v"))
    q, k = q * qk_gain, k * qk_gain
    B, H, S, d = q.shape
    table = torch.from_numpy(case["table"])  # (33*33, H)
    btab = torch.cat([table, torch.zeros(3, H)]) * (1.0 / math.log(2.0))
    coords = torch.from_numpy(case["coords"])
    mask = torch.from_numpy(case["mask"])
    lens = torch.from_numpy(case["lens"])
    out = torch.empty(B, H, S, d, dtype=torch.bfloat16, device=DEV)
    qd, kd, vd = (t.to(DEV, torch.bfloat16).contiguous() for t in (q, k, v))
    ops.launch_attn(
        q=qd, k=kd, v=vd, qkv_sb=H * S * d, qkv_sh=S * d, seq_lens=lens.to(DEV), o=out,
        o_sb=H * S * d, o_sh=S * d, o_sr=d, B=B, S=S, H=H, d=d, dpad=16,
        coords=coords.to(DEV, torch.int32).contiguous(), mask8=mask.to(DEV, torch.uint8),
        btab=btab.to(DEV).contiguous(), lut_m=16, n_tokens=0,
    )
    want = ofwd.attn_offset_table(bf(q), bf(k), bf(v), coords, mask, table.double(), 16)
    close(out, want, atol=1e-2, what="cfg2 attention")


def _attn_block_ref(x, w, b, lnw, lnb, coords, mask, lens, table, H, eps=1e-5):
    """float64 LN1 -> q/k/v -> biased, key-masked attention with the packer's
    folded weights (bf16 W diag(ln_w), fp32 b + W ln_b) and the reference's
    pair rows (tables.pair_rows): (B, H, S, d); rows past the bound are 0."""

    B, S, c = x.shape
    d = c // H
    n = torch.nn.functional.layer_norm(x.double(), (c,), None, None, eps)
    y = n @ bf(w * lnw[None, :]).T + (b.double() + w.double() @ lnb.double())
    q, k, v = y.reshape(B, S, 3, H, d).permute(2, 0, 3, 1, 4)
    pair = torch.from_numpy(tables.pair_rows(coords.numpy(), mask.numpy()))
    bias = table.double()[pair].permute(0, 3, 1, 2)  # (B, H, S, S)
    keys = torch.arange(S)
    live = torch.cat([torch.ones(B, 8, dtype=torch.bool), mask.bool()], dim=1)
    live &= keys[None, :] < lens[:, None].long()
    bias = torch.where(live[:, None, None, :], bias, torch.full_like(bias, float("-inf")))
    s = (q @ k.transpose(-2, -1)) / math.sqrt(d) + bias
    out = torch.softmax(s, dim=-1) @ v
    rows = keys[None, :] < lens[:, None].long()
    return torch.where(rows[:, None, :, None], out, torch.zeros_like(out))


@pytest.mark.parametrize("S,lens,wide", [
    # 17 query blocks (the last one split over the waves), ragged bounds (one
    # inside the split block), a bound inside the tokens, tokens only, an
    # empty position
    (264, [264, 251, 8 + 16 * 15 + 3, 40, 5, 8, 0], False),
    # coordinates wider than the unclamped table: clamped-LUT path
    (264, [264, 200, 137], True),
    (40, [40, 33, 17], False),
    # the longest sequence the kernel covers (20 blocks, 5 per wave)
    (320, [320, 300, 8 + 16 * 16 + 1], False),
])
def test_attn_fused_matches_reference(S, lens, wide, attn_variant):
    """LN1 -> q/k/v -> attention in one launch against a float64 restatement
    (tolerance 2e-2 + 2e-2 |want|: q/k/v, P and V are bf16, the offset table
    fp16), and against the q/k/v kernel followed by the attention kernel (which
    rounds the normalised rows to bf16 before the projection: within 3e-2).
    Rows past each position's bound are exactly zero."""

    from shrimp import ops
    from shrimp.constants import BIAS_ROWS
    from shrimp.geometry import CELL_LUT_M, cell_bias_lut

    torch.manual_seed(11)
    c, H, d, nt = 128, 8, 16, 8
    B, N = len(lens), S - 8
    x = (torch.randn(B, S, c) * 1.5 + 0.3).to(torch.bfloat16)
    w, b = torch.randn(3 * c, c) * 0.08, torch.randn(3 * c) * 0.1
    lnw, lnb = torch.rand(c) + 0.5, torch.randn(c) * 0.1
    packed = ops.pack_attn_qkv(w.to(DEV), b.to(DEV), lnw.to(DEV), lnb.to(DEV))
    span = 40 if wide else 6
    coords = torch.randint(-span, span + 1, (B, N, 2), dtype=torch.int32)
    mask = torch.rand(B, N) > 0.2
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    table = torch.randn(BIAS_ROWS, H) * 0.5
    lut = torch.from_numpy(cell_bias_lut()).to(DEV)
    btab, xtab = ops.attn_bias_table(table.to(DEV), lut, CELL_LUT_M)
    assert ops.attn_fused_supported(c, H, S, 16)
    xd = x.to(DEV)
    outs = []
    for fused in (True, False):
        o = torch.full((B, S, c), 7.0, dtype=torch.bfloat16, device=DEV)
        kw = dict(seq_lens=seq_lens.to(DEV), o=o, o_sb=S * c, o_sh=d, o_sr=c, B=B, S=S, H=H,
                  d=d, dpad=16, coords=coords.to(DEV), mask8=mask.to(DEV, torch.uint8),
                  btab=btab, xtab=xtab, lut_m=CELL_LUT_M, n_tokens=nt)
        if fused:
            ops.launch_attn_fused(x=xd, x_sb=S * c, x_sr=c, packed=packed, eps=1e-5, **kw)
        else:
            qkv = torch.empty((3, B, H, S, 16), dtype=torch.bfloat16, device=DEV)
            ops.launch_attn_qkv(x=xd, x_sr=c, qkv=qkv, packed=packed, eps=1e-5, rows=B * S, B=B,
                                S=S, H=H, C=c, dpad=16)
            ops.launch_attn(q=qkv[0], k=qkv[1], v=qkv[2], qkv_sb=H * S * 16, qkv_sh=S * 16, **kw)
        outs.append(o.cpu())
    got, two = outs
    for i, L in enumerate(lens):
        assert (got[i, L:] == 0).all(), f"position {i}: rows past the bound"
    want = _attn_block_ref(x, w, b, lnw, lnb, coords, mask, seq_lens, table, H)
    g4 = got.double().reshape(B, S, H, d).permute(0, 2, 1, 3)
    print(f"attn fused S={S} wide={wide}: max |got - f64| = {(g4 - want).abs().max().item():.3e}",
          flush=True)
    close(g4, want, atol=2e-2, rtol=2e-2, what=f"attn fused S={S} wide={wide}")
    diff = (got.double() - two.double()).abs().max().item()
    print(f"attn fused S={S} wide={wide}: max |fused - two launches| = {diff:.3e}", flush=True)
    assert diff <= 3e-2


def test_decode_kernel(golden):
    from shrimp import _lib

    g = golden("decode")
    logits = torch.from_numpy(g["logits"])
    B = logits.shape[0]
    pol = torch.randn(B, 50)
    legal = torch.randint(1, 50, (B,), dtype=torch.int32)
    off = torch.zeros(B, dtype=torch.int64)
    off[1:] = torch.cumsum(legal.to(torch.int64), 0)[:-1]
    total = int(legal.sum())
    vals = torch.empty(B, device=DEV)
    ml = torch.empty(B, device=DEV)
    pri = torch.empty(total, device=DEV)
    lg = torch.empty(total, device=DEV)
    # keep every device tensor referenced until the kernel has run
    ld, pd, legd, offd = logits.to(DEV), pol.to(DEV), legal.to(DEV), off.to(DEV)
    _lib.check(_lib.load().shrimp_decode(
        ld.data_ptr(), ld.data_ptr(), pd.data_ptr(), 50, legd.data_ptr(), offd.data_ptr(), B,
        65, 209.0, vals.data_ptr(), ml.data_ptr(), pri.data_ptr(), lg.data_ptr(),
        _lib.stream_handle()), "decode")
    torch.cuda.synchronize()
    assert np.allclose(vals.cpu().numpy(), g["value"], atol=1e-6)
    assert np.allclose(ml.cpu().numpy(), g["moves_left"], atol=1e-3)
    want = torch.cat([torch.softmax(pol[i, : legal[i]].double(), 0) for i in range(B)])
    assert torch.allclose(pri.cpu().double(), want, atol=1e-6)
    assert torch.equal(lg.cpu(), torch.cat([pol[i, : legal[i]] for i in range(B)]))


# ---- configs 1-3 at their own shapes ---------------------------------------------------


def _sample_rows(B):
    return [0, 1, B // 2, B - 1]


@pytest.fixture(scope="module")
def cfg1_full():
    from shrimp import synthetic

    return synthetic.conv_inputs(1024, channels=128)


@pytest.mark.parametrize("B", [4, 1024])
def test_cfg1_conv_bias_relu(cfg1_full, B, conv_variant):
    """Config 1's op: 7-tap gather-GEMM with the fused bias + ReLU + mask
    epilogue (no LayerNorm), at B=4 and at config 1's own B=1024: finite, pad
    rows exactly zero, sampled positions against the oracle, and (B=1024) the
    sampled positions equal to a sub-batch run of the same kernel choice."""

    from shrimp import ops

    b = cfg1_full["batch"]
    x = torch.from_numpy(cfg1_full["x"][:B])
    w = torch.from_numpy(cfg1_full["w"])
    bias = torch.from_numpy(cfg1_full["bias"])
    gidx = _gidx(b)[:B].contiguous()
    mask = b["mask"][:B].contiguous()
    N = mask.shape[1]
    wp = ops.pack_conv_weight(w.to(DEV))
    bd = bias.to(DEV)

    def run(rows):
        xd = x[rows].to(DEV, torch.bfloat16).contiguous()
        out = torch.full((len(rows), N, 128), 3.0, dtype=torch.bfloat16, device=DEV)
        ops.launch_conv(x=xd, x_sb=N * 128, x_sn=128, idx=gidx[rows].to(DEV, torch.int32).contiguous(),
                        taps=7, idx_stride=7, mask8=mask[rows].to(DEV, torch.uint8).contiguous(),
                        wpack=wp, bias=bd, B=len(rows), N=N, cin_pad=128, cout=128, relu=True,
                        out=out, o_sb=N * 128, o_sn=128)
        return out.cpu()

    print(f"cfg1 conv bias+relu B={B}", flush=True)
    full = run(list(range(B)))
    assert torch.isfinite(full.float()).all()
    assert (full[~mask] == 0).all()
    assert (full.float() >= 0).all()
    rows = _sample_rows(B)
    want = torch.relu(ofwd.hex_conv(bf(x[rows]), gidx[rows], mask[rows], bf(w), bias.double()))
    close(full[rows], want, what=f"cfg1 B={B}")
    if B > 4:
        assert torch.equal(full[rows], run(rows))


@pytest.fixture(scope="module")
def cfg2_full():
    from shrimp import synthetic

    return synthetic.attention_inputs(1024, heads=8, d=16)


@pytest.mark.parametrize("linear", [False, True], ids=["clamped", "linear"])
def test_cfg2_attention_full_shape(cfg2_full, attn_variant, linear):
    """Config 2's op at its own shape (B=1024, H=8, L=256, d=16, lengths
    U[64, 256], 33x33 per-head offset table): finite, rows past each length
    exactly zero, sampled positions against the oracle (attn_offset_table,
    pinned against the reference's pair rows), and equal to a sub-batch run.
    Clamped: the clamped-LUT path; linear: with the unclamped fp16 offset
    table (bench.cfg2_xtab) the compact positions take the linear path."""

    from bench import cfg2_xtab
    from shrimp import ops

    c = cfg2_full
    q, k, v = (torch.from_numpy(c[n]) for n in ("q", "k", "v"))
    B, H, S, d = q.shape
    table = torch.from_numpy(c["table"])
    btab = (torch.cat([table, torch.zeros(3, H)]) * (1.0 / math.log(2.0))).to(DEV).contiguous()
    xtab = cfg2_xtab(btab, 16) if linear else None
    coords, mask, lens = (torch.from_numpy(c[n]) for n in ("coords", "mask", "lens"))

    def run(rows):
        n = len(rows)
        qd, kd, vd = (t[rows].to(DEV, torch.bfloat16).contiguous() for t in (q, k, v))
        out = torch.full((n, H, S, d), 5.0, dtype=torch.bfloat16, device=DEV)
        ops.launch_attn(
            q=qd, k=kd, v=vd, qkv_sb=H * S * d, qkv_sh=S * d, seq_lens=lens[rows].to(DEV), o=out,
            o_sb=H * S * d, o_sh=S * d, o_sr=d, B=n, S=S, H=H, d=d, dpad=16,
            coords=coords[rows].to(DEV, torch.int32).contiguous(),
            mask8=mask[rows].to(DEV, torch.uint8).contiguous(), btab=btab, xtab=xtab, lut_m=16,
            n_tokens=0,
        )
        return out.cpu()

    print(f"cfg2 attention B={B} linear={linear}", flush=True)
    full = run(list(range(B)))
    assert torch.isfinite(full.float()).all()
    for i in range(B):
        assert (full[i, :, int(lens[i]):] == 0).all(), i
    rows = _sample_rows(B)
    want = ofwd.attn_offset_table(bf(q[rows]), bf(k[rows]), bf(v[rows]), coords[rows], mask[rows],
                                  table.double(), 16)
    close(full[rows], want, atol=1e-2, what="cfg2 B=1024")
    assert torch.equal(full[rows], run(rows))


def test_cfg2_staged_rows_path(cfg2_full):
    """Config 2's op as bench.py times it: the key table (shrimp_attn_keys) and
    the staged kernel over the K / V rows (shrimp_attn_staged with kvf NULL).
    Bit-identical to the row-layout kernel at the same wave count (four waves,
    two heads per workgroup), against the oracle on sampled positions, and
    unchanged when the K and V rows of dead keys (masked cells, rows past each
    length) hold NaN."""

    from bench import cfg2_xtab
    from shrimp import _lib, ops

    c = cfg2_full
    q, k, v = (torch.from_numpy(c[n]) for n in ("q", "k", "v"))
    B, H, S, d = q.shape
    table = torch.from_numpy(c["table"])
    btab = (torch.cat([table, torch.zeros(3, H)]) * (1.0 / math.log(2.0))).to(DEV).contiguous()
    xtab = cfg2_xtab(btab, 16)
    coords, mask, lens = (torch.from_numpy(c[n]) for n in ("coords", "mask", "lens"))
    assert ops.attn_staged_supported(H, S, 16)
    dead = ~mask.bool() | (torch.arange(S)[None, :] >= lens[:, None].long())  # (B, S)
    assert dead.any() and (~mask.bool()).any()
    cd = coords.to(DEV, torch.int32).contiguous()
    md = mask.to(DEV, torch.uint8).contiguous()
    ld = lens.to(DEV)
    qd = q.to(DEV, torch.bfloat16).contiguous()
    meta = torch.empty(B * ops.attn_keys_ints(S), dtype=torch.int32, device=DEV)
    kw = dict(qkv_sb=H * S * d, qkv_sh=S * d, seq_lens=ld, o_sb=H * S * d, o_sh=S * d, o_sr=d, B=B,
              S=S, H=H, d=d, dpad=16, btab=btab, xtab=xtab, lut_m=16, n_tokens=0)

    def staged(kt, vt):
        out = torch.full((B, H, S, d), 5.0, dtype=torch.bfloat16, device=DEV)
        ops.launch_attn_keys(coords=cd, mask8=md, seq_lens=ld, B=B, S=S, n_tokens=0, meta=meta)
        ops.launch_attn_staged(q=qd, k=kt.to(DEV, torch.bfloat16).contiguous(),
                               v=vt.to(DEV, torch.bfloat16).contiguous(), meta=meta, o=out, **kw)
        return out.cpu()

    print(f"cfg2 staged rows B={B}", flush=True)
    got = staged(k, v)
    lib = _lib.load()
    prev = lib.shrimp_attn_variant(2)
    try:
        print("cfg2 row-layout kernel, four waves", flush=True)
        ref = torch.empty((B, H, S, d), dtype=torch.bfloat16, device=DEV)
        ops.launch_attn(q=qd, k=k.to(DEV, torch.bfloat16).contiguous(),
                        v=v.to(DEV, torch.bfloat16).contiguous(), o=ref, coords=cd, mask8=md, **kw)
        ref = ref.cpu()
    finally:
        lib.shrimp_attn_variant(prev)
    assert torch.isfinite(got.float()).all()
    for i in range(B):
        assert (got[i, :, int(lens[i]):] == 0).all(), i
    assert torch.equal(got, ref)
    rows = _sample_rows(B)
    want = ofwd.attn_offset_table(bf(q[rows]), bf(k[rows]), bf(v[rows]), coords[rows], mask[rows],
                                  table.double(), 16)
    close(got[rows], want, atol=1e-2, what="cfg2 staged rows")
    kn, vn = k.clone(), v.clone()
    dm = dead[:, None, :, None].expand_as(kn)
    kn[dm] = float("nan")
    vn[dm] = float("nan")
    print("cfg2 staged rows, NaN in dead keys' rows", flush=True)
    assert torch.equal(staged(kn, vn), got)


def test_staged_rows_eight_waves():
    """shrimp_attn_staged over K / V rows past the 64 KiB LDS budget (S = 384:
    eight waves with a compute unit's LDS), masked cells scattered inside each
    length, a length of 17 and an empty position: live query rows against the
    oracle, rows past each length zero, and the same output with NaN in the
    K / V rows of dead keys (masked cells, rows past the length)."""

    from bench import cfg2_xtab
    from shrimp import ops

    g = torch.Generator().manual_seed(23)
    B, H, S, d = 12, 8, 384, 16
    assert ops.attn_staged_supported(H, S, 16)
    grid = torch.stack(torch.meshgrid(torch.arange(20), torch.arange(20), indexing="ij"), -1)
    grid = grid.reshape(-1, 2)
    coords = torch.stack([grid[torch.randperm(400, generator=g)[:S]] for _ in range(B)])
    lens = torch.randint(200, S + 1, (B,), generator=g, dtype=torch.int32)
    lens[0], lens[1], lens[2] = S, 17, 0
    inside = torch.arange(S)[None, :] < lens[:, None].long()
    mask = inside & (torch.rand(B, S, generator=g) > 0.1)
    q, k, v = (torch.randn(B, H, S, d, generator=g) for _ in range(3))
    table = torch.randn(33 * 33, H, generator=g) * 0.7
    btab = (torch.cat([table, torch.zeros(3, H)]) * (1.0 / math.log(2.0))).to(DEV).contiguous()
    xtab = cfg2_xtab(btab, 16)
    cd = coords.to(DEV, torch.int32).contiguous()
    md = mask.to(DEV, torch.uint8).contiguous()
    ld = lens.to(DEV)
    meta = torch.empty(B * ops.attn_keys_ints(S), dtype=torch.int32, device=DEV)

    def staged(kt, vt):
        out = torch.full((B, H, S, d), 5.0, dtype=torch.bfloat16, device=DEV)
        ops.launch_attn_keys(coords=cd, mask8=md, seq_lens=ld, B=B, S=S, n_tokens=0, meta=meta)
        ops.launch_attn_staged(
            q=q.to(DEV, torch.bfloat16).contiguous(), k=kt.to(DEV, torch.bfloat16).contiguous(),
            v=vt.to(DEV, torch.bfloat16).contiguous(), qkv_sb=H * S * d, qkv_sh=S * d, meta=meta,
            seq_lens=ld, o=out, o_sb=H * S * d, o_sh=S * d, o_sr=d, B=B, S=S, H=H, d=d, dpad=16,
            btab=btab, xtab=xtab, lut_m=16, n_tokens=0)
        return out.cpu()

    print(f"staged rows, eight waves, B={B} S={S}", flush=True)
    got = staged(k, v)
    assert torch.isfinite(got.float()).all()
    for i in range(B):
        assert (got[i, :, int(lens[i]):] == 0).all(), i
    want = ofwd.attn_offset_table(bf(q), bf(k), bf(v), coords, mask, table.double(), 16)
    sel = mask[:, None, :, None].expand_as(want)
    close(got[sel], want[sel], atol=1e-2, what="staged rows S=384")
    dead = ~mask[:, None, :, None].expand_as(k)
    kn, vn = k.clone(), v.clone()
    kn[dead] = float("nan")
    vn[dead] = float("nan")
    print("staged rows, eight waves, NaN in dead keys' rows", flush=True)
    assert torch.equal(staged(kn, vn), got)


@pytest.fixture(scope="module")
def cfg3_full():
    from shrimp import synthetic

    return synthetic.raytap_inputs(1024, channels=128)


def test_cfg3_raytap_full_shape(cfg3_full):
    """Config 3's op at its own shape (B=1024, L=256, C=128, 31 independent
    taps over the 32-slot ray index built on the device): finite, pad rows
    exactly zero, sampled positions against the oracle's 31-tap conv, and
    equal to a sub-batch run."""

    from shrimp import _lib, ops

    c = cfg3_full
    b = c["batch"]
    B, N = b["mask"].shape
    x, w, bias = (torch.from_numpy(c[k]) for k in ("x", "w", "bias"))
    coords = b["coords"].to(torch.int32)
    mask = b["mask"]
    lib = _lib.load()
    wp = ops.pack_conv_weight(w.to(DEV))
    bd = bias.to(DEV)

    def run(rows):
        n = len(rows)
        c32 = coords[rows].to(DEV).contiguous()
        m8 = mask[rows].to(DEV, torch.uint8).contiguous()
        idx = torch.empty(n, N, 32, dtype=torch.int32, device=DEV)
        _lib.check(lib.shrimp_build_ray_index(c32.data_ptr(), m8.data_ptr(), n, N, idx.data_ptr(),
                                              _lib.stream_handle()), "ray")
        out = torch.full((n, N, 128), 3.0, dtype=torch.bfloat16, device=DEV)
        ops.launch_conv(x=x[rows].to(DEV, torch.bfloat16).contiguous(), x_sb=N * 128, x_sn=128,
                        idx=idx, taps=31, idx_stride=32, mask8=m8, wpack=wp, bias=bd, B=n, N=N,
                        cin_pad=128, cout=128, out=out, o_sb=N * 128, o_sn=128)
        return out.cpu(), idx.cpu()

    print(f"cfg3 raytap B={B}", flush=True)
    full, idx = run(list(range(B)))
    assert torch.isfinite(full.float()).all()
    assert (full[~mask] == 0).all()
    rows = _sample_rows(B)
    ridx = torch.from_numpy(tables.ray_index(coords[rows].numpy(), mask[rows].numpy()))
    assert torch.equal(idx[rows], ridx)
    want = ofwd.raytap_conv(bf(x[rows]), ridx, mask[rows], bf(w), bias.double())
    close(full[rows], want, what="cfg3 B=1024")
    assert torch.equal(full[rows], run(rows)[0])


def test_attn_keys_tokens_equals_separate_launches():
    """shrimp_attn_keys_tokens writes the same key table as shrimp_attn_keys
    and the same token rows as shrimp_fill_tokens (both vec4 and scalar token
    paths), and leaves the cell rows alone; bad token arguments are refused
    before anything runs."""

    from shrimp import _lib, ops

    lib = _lib.load()
    g = torch.Generator().manual_seed(11)
    for B, N, C, off in ((37, 61, 128, 0), (5, 20, 24, 1)):
        nt = 4
        S = N + nt
        mask = (torch.rand(B, N, generator=g) < 0.7).to(torch.uint8)
        mask[1] = 0  # a position with no live cell
        coords = torch.randint(-9, 9, (B, N, 2), generator=g, dtype=torch.int32)
        last = torch.where(mask.bool(), torch.arange(1, N + 1), torch.zeros(N, dtype=torch.int64))
        lens = (nt + last.max(1).values).to(torch.int32)
        cd, md, ld = coords.to(DEV), mask.to(DEV), lens.to(DEV)
        # off = 1: tokens one float into an allocation (not 16-byte aligned: scalar path)
        tok = torch.randn(nt * C + off, generator=g).to(DEV)[off:].view(nt, C)
        out = {}
        for fused in (False, True):
            print(f"attn_keys_tokens B={B} N={N} C={C} off={off} fused={fused}", flush=True)
            meta = torch.full((B, ops.attn_keys_ints(S)), -7, dtype=torch.int32, device=DEV)
            seq = torch.full((B, S, C), 3.0, dtype=torch.bfloat16, device=DEV)
            lo = torch.full((B, nt, C), 3.0, dtype=torch.bfloat16, device=DEV)
            if fused:
                ops.launch_attn_keys(coords=cd, mask8=md, seq_lens=ld, B=B, S=S, n_tokens=nt,
                                     meta=meta, tokens=tok, seq=seq, seq_sb=S * C, tok_lo=lo)
            else:
                ops.launch_attn_keys(coords=cd, mask8=md, seq_lens=ld, B=B, S=S, n_tokens=nt,
                                     meta=meta)
                _lib.check(lib.shrimp_fill_tokens(tok.data_ptr(), nt, C, seq.data_ptr(), S * C,
                                                  lo.data_ptr(), B, _lib.stream_handle()),
                           "fill_tokens")
            torch.cuda.synchronize()
            out[fused] = (meta.cpu(), seq.cpu(), lo.cpu())
        for a, b in zip(out[False], out[True]):
            assert torch.equal(a, b)
        seq = out[True][1].float()
        assert torch.equal(seq[:, :nt], tok.cpu().to(torch.bfloat16).float().expand(B, nt, C))
        assert (seq[:, nt:] == 3.0).all()
        lo = out[True][2].float()
        assert torch.equal(lo, (tok.cpu() - seq[0, :nt]).to(torch.bfloat16).float().expand(B, nt, C))
    meta = torch.empty((2, ops.attn_keys_ints(8)), dtype=torch.int32, device=DEV)
    seq = torch.empty((2, 8, 16), dtype=torch.bfloat16, device=DEV)
    ln = torch.full((2,), 4, dtype=torch.int32, device=DEV)
    tok = torch.zeros((4, 16), device=DEV)
    # a position stride shorter than the token rows is refused
    assert lib.shrimp_attn_keys_tokens(None, None, ln.data_ptr(), 2, 4, 4, meta.data_ptr(),
                                       tok.data_ptr(), 16, seq.data_ptr(), 16, None,
                                       _lib.stream_handle()) == -1
    assert "position stride" in lib.shrimp_last_error().decode()
