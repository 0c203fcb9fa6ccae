"""The fp32 serve mode (the reference's serve with autocast off,
inference.py:50-68) against the fp32 reference: goldens of the reference
ShrimpNet (written in fp32 on the CPU) and the CPU oracle.

Tolerance (F32_RTOL, 1e-4 relative): for each compared output,
max |got - want| <= F32_RTOL * max |want|. The trunk output after ln_final
is compared the same way over tokens and live cells. Op-level tests compare
with float64 restatements at the same relative gate.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import decode as odec
from oracle import forward as ofwd
from oracle import tables, weights

from gates import F32_RTOL

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rel_close(got, want, what, rtol=F32_RTOL):
    got = torch.as_tensor(got).detach().to("cpu", torch.float64)
    want = torch.as_tensor(want).detach().to("cpu", torch.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    scale = want.abs().max().item()
    err = (got - want).abs().max().item()
    print(f"{what}: max abs err {err:.3e}, |ref| max {scale:.3f}, rel {err / max(scale, 1e-30):.2e}",
          flush=True)
    assert err <= rtol * max(scale, 1e-6), what


def _net(c, h, layout, seed, mode="parity"):
    from shrimp.model import ShrimpNet

    net = ShrimpNet(channels=c, attention_heads=h, trunk_layout=layout)
    net.load_state_dict(weights.make_state_dict(c, h, layout, seed=seed, mode=mode))
    net = net.to(DEV).eval()
    net.hip_runtime().precision = "fp32"
    return net


def _run(net, feats, nbr, mask, coords, trunk=True):
    t = lambda a: torch.as_tensor(a).to(DEV)
    rt = net.hip_runtime()
    rt.keep_buffers = trunk
    try:
        out = net.forward_policy_value(t(feats), t(nbr), t(mask), t(coords), request_moves_left=True)
        res = {k: v.cpu().double() for k, v in out.items()}
        if trunk:
            seqf = rt.last["seqf"]
            assert seqf.dtype == torch.float32
            seqf = seqf.cpu().double()
            res["tokens"], res["cells"] = seqf[:, :8], seqf[:, 8:]
    finally:
        rt.keep_buffers = False
        rt.last = None
    for k in ("policy", "value", "moves_left"):
        assert out[k].dtype == torch.float32
    return res


def _check(out, want, mask, what):
    m = torch.as_tensor(mask)
    for key in ("policy", "value", "moves_left"):
        rel_close(out[key], want[key], f"{what} {key}")
    rel_close(odec.decode_value(out["value"]), odec.decode_value(torch.as_tensor(want["value"]).double()),
              f"{what} decoded value")
    assert (out["policy"][~m] == 0).all()
    if "cells" in want:
        rel_close(out["tokens"], want["tokens"], f"{what} tokens")
        rel_close(out["cells"][m], torch.as_tensor(want["cells"])[m], f"{what} cells")
        assert (out["cells"][~m] == 0).all()


@pytest.mark.parametrize("name,mode", [("forward_cfg0", "parity"), ("forward_cfg0", "fresh"),
                                       ("forward_cfg0", "heads"), ("forward_cfg4", "parity"),
                                       ("forward_cfg4", "heads")])
def test_f32_forward_matches_reference_golden(golden, name, mode):
    """Config 0 (C=32, H=4, CCA, the fp32 config) and the config 4
    architecture against the reference ShrimpNet's fp32 outputs."""

    g = golden(name)
    c, h = (int(x) for x in g["arch"])
    net = _net(c, h, str(g["layout"]), int(g[f"{mode}_seed"]), mode)
    out = _run(net, g["feats"], g["nbr"], g["mask"], g["coords"])
    want = {k: g[f"{mode}_{k}"] for k in ("policy", "value", "moves_left", "cells", "tokens")}
    _check(out, want, g["mask"], f"fp32 {name}/{mode}")


def test_f32_cfg0_batch_matches_oracle():
    """Config 0's own workload: B=64 positions of 10-40 stones (L256), C=32,
    H=4, CCA, against the fp32 oracle."""

    from shrimp import synthetic

    b = synthetic.position_batch("cfg0", 64)
    sd = weights.make_state_dict(32, 4, "CCA", seed=21, mode="heads")
    net = _net(32, 4, "CCA", seed=21, mode="heads")
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    want = ofwd.forward_policy_value(sd, "CCA", 4, b["feats"], b["nbr"], b["mask"], b["coords"],
                                     request_moves_left=True, dtype=torch.float64,
                                     return_trunk=True)
    _check(out, want, b["mask"], "fp32 cfg0 B=64")


@pytest.mark.parametrize("c,h,npad", [(96, 4, 256), (96, 4, 512), (192, 3, 256), (192, 3, 512)])
def test_f32_other_widths(c, h, npad):
    """Reference default width (C=96, H=4: d=24) and the main config's
    (C=192, H=3: d=64), at Npad 256 and 512."""

    b = _wide_batch(npad)
    layout = "CCA"
    sd = weights.make_state_dict(c, h, layout, seed=c + h, mode="heads")
    net = _net(c, h, layout, seed=c + h, mode="heads")
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    want = ofwd.forward_policy_value(sd, layout, h, b["feats"], b["nbr"], b["mask"], b["coords"],
                                     request_moves_left=True, dtype=torch.float64,
                                     return_trunk=True)
    _check(out, want, b["mask"], f"fp32 C={c} H={h} Npad={npad}")


def _wide_batch(npad):
    """Three positions padded to npad: L256 positions for 256, spec-variant
    positions (supports of 280-512 cells) for 512."""

    from shrimp import synthetic
    from shrimp.batching import collate_rows

    if npad == 256:
        return synthetic.position_batch("cfg4", 3, seed=31)
    rows = [r for r in synthetic.positions("cfg4_spec", 12, seed=32) if r[1].num_nodes <= npad][:3]
    assert len(rows) == 3 and max(r[1].num_nodes for r in rows) > 256
    return collate_rows([(s, f) for _, s, f in rows], pad_to=npad)


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "graphs"])
def test_f32_evaluator_matches_reference_reply(golden, graphs):
    """The reference evaluator's reply (fp32 on the CPU) from the fp32 serve
    mode: ABI-1 payload in, reply bytes out."""

    from shrimp.inference import ShrimpEvaluator

    g = golden("evaluator_cfg0")
    payload = {
        "abi": 1, "shape": tuple(int(x) for x in g["shape"]),
        "node_feats": g["node_feats"].tobytes(), "node_qr": g["node_qr"].tobytes(),
        "node_row_offsets": g["node_row_offsets"].tolist(), "nbr": g["nbr"].tobytes(),
        "legal_counts": g["legal_counts"].tobytes(),
        "request_moves_left": True, "request_logits": True,
    }
    ev = ShrimpEvaluator(_net(32, 4, "CCA", int(g["wseed"])), DEV, graphs=graphs)
    reply = ev.evaluate_payload(payload)
    for key, gk in (("values_bytes", "values"), ("priors_bytes", "priors"),
                    ("moves_left_bytes", "moves_left"), ("priors_logits_bytes", "priors_logits")):
        got = np.frombuffer(reply[key], np.float32)
        rel_close(torch.from_numpy(got.copy()), torch.from_numpy(g[gk]), f"fp32 evaluator {key}")


def test_f32_and_bf16_modes_switch():
    """One module serves in both precisions: switching repacks the weights,
    and the bf16 result stays within the bf16 gate of the fp32 one."""

    from gates import LOGIT_TOL
    from shrimp import synthetic

    b = synthetic.position_batch("cfg0", 6, seed=4)
    net = _net(32, 4, "CCA", seed=1)
    f32a = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=False)
    net.hip_runtime().precision = "bf16"
    bf = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=False)
    net.hip_runtime().precision = "fp32"
    f32b = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=False)
    for k in ("policy", "value", "moves_left"):
        assert torch.equal(f32a[k], f32b[k]), k
        assert (f32a[k] - bf[k]).abs().max().item() <= LOGIT_TOL, k
    net.hip_runtime().precision = "fp16"
    with pytest.raises(ValueError, match="precision"):
        _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=False)
    net.hip_runtime().precision = "fp32"


# ---- op level -----------------------------------------------------------------------------


def _gidx(batch):
    return torch.from_numpy(tables.gather_index(batch["nbr"].numpy()))


def _pack_conv32(w, cin_pad):
    from shrimp import _lib

    t, cin, cout = w.shape
    out = torch.empty(t * cin_pad * cout, dtype=torch.float32, device=DEV)
    wd = w.to(DEV, torch.float32).contiguous()
    _lib.check(_lib.load().shrimp_pack_conv_weight_f32(wd.data_ptr(), out.data_ptr(), t, cin,
                                                       cin_pad, cout, _lib.stream_handle()), "pack")
    torch.cuda.synchronize()
    return out


def _pack_lin32(w):
    from shrimp import _lib

    n_out, n_in = w.shape
    out = torch.empty(n_in * n_out, dtype=torch.float32, device=DEV)
    wd = w.to(DEV, torch.float32).contiguous()
    _lib.check(_lib.load().shrimp_pack_linear_weight_f32(wd.data_ptr(), out.data_ptr(), n_in,
                                                         n_out, _lib.stream_handle()), "pack")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("epi", ["plain", "relu", "ln", "ln_relu", "resid", "head"])
@pytest.mark.parametrize("cin,cout", [(15, 32), (32, 32), (128, 128), (96, 96), (192, 192)])
def test_f32_hex_conv(epi, cin, cout):
    from shrimp import _lib, synthetic

    if epi in ("resid",) and cin != cout:
        pytest.skip("residual needs cin == cout")
    b = synthetic.position_batch("cfg1", 3, seed=cin + cout)
    B, N = b["mask"].shape
    rng = np.random.default_rng(cin * 7 + cout)
    cp = -(-cin // 16) * 16
    x = torch.from_numpy(rng.standard_normal((B, N, cin)))
    w = torch.from_numpy(rng.standard_normal((7, cin, cout)) / np.sqrt(7 * cin))
    bias = torch.from_numpy(rng.standard_normal(cout) * 0.1)
    lnw = torch.from_numpy(rng.uniform(0.5, 1.5, cout))
    lnb = torch.from_numpy(rng.normal(0, 0.1, cout))
    g = torch.from_numpy(rng.uniform(0.5, 1.0, cout))
    hw = torch.from_numpy(rng.normal(0, cout ** -0.5, cout))
    hb = torch.from_numpy(rng.normal(0, 0.1, 1))
    resid = torch.from_numpy(rng.standard_normal((B, N, cout))) * b["mask"][..., None]
    gidx = _gidx(b)
    mask = b["mask"]
    xd = torch.zeros(B, N, cp, dtype=torch.float32, device=DEV)
    xd[..., :cin] = x.to(DEV, torch.float32)
    f = lambda t: t.to(DEV, torch.float32).contiguous()
    wp = _pack_conv32(w, cp)
    out = resid.to(DEV, torch.float32).contiguous() if epi == "resid" else \
        torch.full((B, N, cout), 7.0, device=DEV)
    head = torch.full((B, N), 7.0, device=DEV)
    keep = [f(t) for t in (bias, lnw, lnb, g, hw, hb)]
    a = _lib.ConvArgs(
        x=xd.data_ptr(), x_sb=N * cp, x_sn=cp, idx=gidx.to(DEV, torch.int32).contiguous().data_ptr(),
        taps=7, idx_stride=7, mask=mask.to(DEV, torch.uint8).data_ptr(), w=wp.data_ptr(),
        bias=keep[0].data_ptr(), eps=1e-5, B=B, N=N, cin_pad=cp, cout=cout,
        out=out.data_ptr(), o_sb=N * cout, o_sn=cout,
    )
    idx_d = gidx.to(DEV, torch.int32).contiguous()
    m8 = mask.to(DEV, torch.uint8)
    a.idx, a.mask = idx_d.data_ptr(), m8.data_ptr()
    if epi in ("ln", "ln_relu", "resid"):
        a.ln_w, a.ln_b = keep[1].data_ptr(), keep[2].data_ptr()
    if epi in ("relu", "ln_relu", "head"):
        a.relu = 1
    if epi == "resid":
        a.resid, a.r_sb, a.r_sn, a.gamma = out.data_ptr(), N * cout, cout, keep[3].data_ptr()
    if epi == "head":
        a.head_w, a.head_b, a.head_out = keep[4].data_ptr(), keep[5].data_ptr(), head.data_ptr()
        a.out = None
    _lib.check(_lib.load().shrimp_hex_conv_f32(ctypes.byref(a), _lib.stream_handle()), "conv")
    torch.cuda.synchronize()
    acc = ofwd.hex_conv(x, gidx, torch.ones_like(mask), w, bias)
    md = mask.double()[..., None]
    if epi == "plain":
        want = acc * md
    elif epi == "relu":
        want = torch.relu(acc) * md
    elif epi == "head":
        want = ((torch.relu(acc) @ hw) + hb) * mask.double()
        rel_close(head.cpu(), want, f"fp32 conv head {cin}->{cout}")
        return
    else:
        y = torch.nn.functional.layer_norm(acc, (cout,), lnw, lnb, 1e-5)
        if epi == "ln_relu":
            y = torch.relu(y)
        y = y * md
        want = torch.relu(resid + g * y) if epi == "resid" else y
    rel_close(out.cpu(), want, f"fp32 conv {epi} {cin}->{cout}")


@pytest.mark.parametrize("mode", ["qkv", "gelu", "resid", "plain"])
@pytest.mark.parametrize("c,h", [(32, 4), (128, 8), (96, 4), (192, 3)])
@pytest.mark.parametrize("B,S", [(3, 37), (1, 9)])
def test_f32_linear_modes(mode, c, h, B, S):
    """Every linear mode against float64. 9 rows leave three of a workgroup's
    four waves without rows (they still take part in the weight staging)."""
    from shrimp import _lib

    rng = np.random.default_rng(c + len(mode) + S)
    d = c // h
    rows = B * S
    n_in = 2 * c if mode == "resid" else c
    n_out = {"qkv": 3 * c, "gelu": 2 * c, "resid": c, "plain": c}[mode]
    x = torch.from_numpy(rng.standard_normal((rows, n_in)) * 1.5 + 0.3)
    w = torch.from_numpy(rng.standard_normal((n_out, n_in)) / np.sqrt(n_in))
    bias = torch.from_numpy(rng.normal(0, 0.1, n_out))
    lnw = torch.from_numpy(rng.uniform(0.5, 1.5, n_in))
    lnb = torch.from_numpy(rng.normal(0, 0.1, n_in))
    use_ln = mode in ("qkv", "gelu")
    xin = torch.nn.functional.layer_norm(x, (n_in,), lnw, lnb, 1e-5) if use_ln else x
    y = xin @ w.T + bias
    f = lambda t: t.to(DEV, torch.float32).contiguous()
    xd, bd, lwd, lbd = f(x), f(bias), f(lnw), f(lnb)
    wp = _pack_lin32(w)
    a = _lib.LinearArgs(x=xd.data_ptr(), x_sr=n_in, w=wp.data_ptr(), bias=bd.data_ptr(), eps=1e-5,
                        rows=rows, in_features=n_in, out_features=n_out)
    if use_ln:
        a.ln_w, a.ln_b = lwd.data_ptr(), lbd.data_ptr()
    res = torch.from_numpy(rng.standard_normal((rows, n_out)))
    g = torch.from_numpy(rng.uniform(0, 1, n_out))
    m = torch.from_numpy(rng.uniform(size=rows) > 0.3)
    gd, md = f(g), m.to(DEV, torch.uint8)
    if mode == "qkv":
        out = torch.full((3, B, h, S, d), 7.0, device=DEV)
        a.mode, a.B, a.S, a.H, a.dpad = _lib.LIN_QKV, B, S, h, d
        want = y.reshape(B, S, 3, h, d).permute(2, 0, 3, 1, 4)
    elif mode == "resid":
        out = f(res)
        a.mode, a.resid, a.r_sr, a.gamma, a.mask = _lib.LIN_RESID, out.data_ptr(), n_out, \
            gd.data_ptr(), md.data_ptr()
        want = res + g * y * m.double()[:, None]
    else:
        out = torch.full((rows, n_out), 7.0, device=DEV)
        a.mode = _lib.LIN_GELU if mode == "gelu" else _lib.LIN_PLAIN
        want = torch.nn.functional.gelu(y) if mode == "gelu" else y
    a.out, a.o_sr = out.data_ptr(), n_out
    _lib.check(_lib.load().shrimp_linear_f32(ctypes.byref(a), _lib.stream_handle()), "linear")
    torch.cuda.synchronize()
    rel_close(out.cpu(), want, f"fp32 linear {mode} C={c}")


@pytest.mark.parametrize("d", [8, 16, 24, 64])
@pytest.mark.parametrize("S,lens", [(40, [40, 33, 9]), (270, [270, 200, 0])])
@pytest.mark.parametrize("radius", [20, 12])
def test_f32_attention_coords(d, S, lens, radius):
    """Coords-mode attention with 8 summary tokens, dead cells and key bounds
    (including an empty position), against the float64 restatement with the
    reference's pair rows. Coordinates within +-12 keep every position's live
    span at most 26 (the head-dim-16 kernel's unclamped table), +-20 do not
    (its clamped table)."""

    from shrimp import _lib, ops
    from shrimp.constants import BIAS_ROWS
    from shrimp.geometry import CELL_LUT_M, cell_bias_lut

    torch.manual_seed(d + S + radius)
    B, H, nt = len(lens), 3, 8
    N = S - nt
    q, k, v = (torch.randn(B, H, S, d, dtype=torch.float64) for _ in range(3))
    coords = torch.randint(-radius, radius + 1, (B, N, 2), dtype=torch.int32)
    mask = torch.rand(B, N) > 0.2
    table = torch.randn(BIAS_ROWS, H) * 0.5
    lut = torch.from_numpy(cell_bias_lut()).to(DEV)
    btab, _ = ops.attn_bias_table(table.to(DEV), lut, CELL_LUT_M)
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    f = lambda t: t.to(DEV, torch.float32).contiguous()
    qd, kd, vd = f(q), f(k), f(v)
    out = torch.full((B, H, S, d), 7.0, device=DEV)
    cd, md, sd = coords.to(DEV).contiguous(), mask.to(DEV, torch.uint8), seq_lens.to(DEV)
    a = _lib.AttnArgs(q=qd.data_ptr(), k=kd.data_ptr(), v=vd.data_ptr(), qkv_sb=H * S * d,
                      qkv_sh=S * d, seq_lens=sd.data_ptr(), coords=cd.data_ptr(), mask=md.data_ptr(),
                      btab=btab.data_ptr(), lut_m=CELL_LUT_M, n_tokens=nt, o=out.data_ptr(),
                      o_sb=H * S * d, o_sh=S * d, o_sr=d, B=B, S=S, H=H, d=d, dpad=d)
    _lib.check(_lib.load().shrimp_attn_f32(ctypes.byref(a), _lib.stream_handle()), "attn_f32")
    torch.cuda.synchronize()
    pair = torch.from_numpy(tables.pair_rows(coords.numpy(), mask.numpy()))
    bias = table.double()[pair].permute(0, 3, 1, 2)
    live = torch.cat([torch.ones(B, nt, dtype=torch.bool), mask], 1)
    live &= torch.arange(S)[None, :] < seq_lens[:, None].long()
    bias = torch.where(live[:, None, None, :], bias, torch.full_like(bias, float("-inf")))
    s = (q @ k.transpose(-2, -1)) / math.sqrt(d) + bias
    want = torch.nan_to_num(torch.softmax(s, -1)) @ v
    rows = torch.arange(S)[None, :] < seq_lens[:, None].long()
    want = torch.where(rows[:, None, :, None], want, torch.zeros_like(want))
    rel_close(out.cpu(), want, f"fp32 attention d={d} S={S}")


@pytest.mark.parametrize("radius", [20, 12])
def test_f32_attention_mfma_matches_chunked(radius):
    """At head dim 16 (coords mode) shrimp_attn_f32 runs the MFMA kernel; the
    chunked kernel (attention variant 3) on the same inputs agrees to the fp32
    tolerance, at the forward's shape (S = 264, 8 heads)."""

    from shrimp import _lib, ops
    from shrimp.constants import BIAS_ROWS
    from shrimp.geometry import CELL_LUT_M, cell_bias_lut

    torch.manual_seed(radius)
    B, H, S, d, nt = 6, 8, 264, 16, 8
    N = S - nt
    f = lambda t: t.to(DEV, torch.float32).contiguous()
    q, k, v = (f(torch.randn(B, H, S, d)) for _ in range(3))
    coords = torch.randint(-radius, radius + 1, (B, N, 2), dtype=torch.int32).to(DEV).contiguous()
    mask = (torch.rand(B, N) > 0.1).to(DEV, torch.uint8)
    table = torch.randn(BIAS_ROWS, H) * 0.5
    lut = torch.from_numpy(cell_bias_lut()).to(DEV)
    btab, _ = ops.attn_bias_table(table.to(DEV), lut, CELL_LUT_M)
    sd = torch.tensor([264, 200, 137, 16, 9, 0], dtype=torch.int32, device=DEV)
    lib = _lib.load()
    outs = []
    for variant in (0, 3):
        out = torch.full((B, S, H * d), 7.0, device=DEV)
        a = _lib.AttnArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), qkv_sb=H * S * d,
                          qkv_sh=S * d, seq_lens=sd.data_ptr(), coords=coords.data_ptr(),
                          mask=mask.data_ptr(), btab=btab.data_ptr(), lut_m=CELL_LUT_M,
                          n_tokens=nt, o=out.data_ptr(), o_sb=S * H * d, o_sh=d, o_sr=H * d,
                          B=B, S=S, H=H, d=d, dpad=d)
        prev = lib.shrimp_attn_variant(variant)
        try:
            _lib.check(lib.shrimp_attn_f32(ctypes.byref(a), _lib.stream_handle()), "attn_f32")
            torch.cuda.synchronize()
        finally:
            lib.shrimp_attn_variant(prev)
        outs.append(out.cpu())
    rel_close(outs[0], outs[1], f"fp32 attention MFMA vs chunked, coords +-{radius}")


def test_f32_attention_pair_mode():
    from shrimp import _lib

    torch.manual_seed(3)
    B, H, S, d = 3, 4, 70, 16
    q, k, v = (torch.randn(B, H, S, d, dtype=torch.float64) for _ in range(3))
    rows = 238
    table2 = torch.randn(rows, H) * 0.5
    table2[rows - 1] = -3.0e4
    pair = torch.randint(0, rows - 1, (B, S, S), dtype=torch.uint8)
    pair[1, :, 50:60] = rows - 1
    lens = torch.tensor([70, 61, 23], dtype=torch.int32)
    f = lambda t: t.to(DEV, torch.float32).contiguous()
    qd, kd, vd, td = f(q), f(k), f(v), f(table2)
    pd, ld = pair.to(DEV).contiguous(), lens.to(DEV)
    out = torch.full((B, H, S, d), 7.0, device=DEV)
    a = _lib.AttnArgs(q=qd.data_ptr(), k=kd.data_ptr(), v=vd.data_ptr(), qkv_sb=H * S * d,
                      qkv_sh=S * d, seq_lens=ld.data_ptr(), pair=pd.data_ptr(), p_sb=S * S, p_sq=S,
                      table2=td.data_ptr(), table_rows=rows, n_tokens=0, o=out.data_ptr(),
                      o_sb=H * S * d, o_sh=S * d, o_sr=d, B=B, S=S, H=H, d=d, dpad=d)
    _lib.check(_lib.load().shrimp_attn_f32(ctypes.byref(a), _lib.stream_handle()), "attn_f32")
    torch.cuda.synchronize()
    want = ofwd.attn_pair(q, k, v, pair, table2.double(), lens)
    rel_close(out.cpu(), want, "fp32 attention pair mode")
