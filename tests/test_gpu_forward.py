"""Full serve forward on the GPU against the reference goldens and the CPU
oracle. Tolerances (tests/gates.py): policy logits, value logits and decoded
value within 2e-2 absolute (bf16 path vs the fp32 reference); the trunk
output (after ln_final, std ~1) within TRUNK_MEAN in mean absolute error over
tokens and over live cells, and within TRUNK_ROW_REL per row (relative L2).

The "heads" weight mode gives the serve heads O(1) weights, so the logits
are O(1) and the 2e-2 gate sees trunk errors; the trunk gates see the
summary tokens, which attend to every cell in every attention block (a
zeroed, swapped or head-permuted bias table moves the tokens' mean absolute
value by 0.02-0.09 and a skipped attention sub-block by 0.5;
tests/test_oracle_forward.py::test_trunk_gates_see_composition_mistakes
checks those margins on the CPU)."""

import numpy as np
import pytest
import torch

from oracle import decode as odec
from oracle import forward as ofwd
from oracle import weights

from gates import LOGIT_TOL as TOL
from gates import TRUNK_MEAN, TRUNK_ROW_REL

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _net(c, h, layout, seed, mode="parity"):
    from shrimp.model import ShrimpNet

    net = ShrimpNet(channels=c, attention_heads=h, trunk_layout=layout)
    net.load_state_dict(weights.make_state_dict(c, h, layout, seed=seed, mode=mode))
    return net.to(DEV).eval()


def _run(net, feats, nbr, mask, coords, ml=True, trunk=False):
    t = lambda a: torch.as_tensor(a).to(DEV)
    rt = net.hip_runtime()
    rt.keep_buffers = trunk
    try:
        out = net.forward_policy_value(t(feats), t(nbr), t(mask), t(coords), request_moves_left=ml)
        res = {k: v.cpu().double() for k, v in out.items()}
        if trunk:
            seqf = rt.last["seqf"].cpu().double()
            res["tokens"], res["cells"] = seqf[:, :8], seqf[:, 8:]
    finally:
        rt.keep_buffers = False
        rt.last = None
    return res


def _check(out, want, mask, what):
    for key in ("policy", "value", "moves_left"):
        if key not in want:
            continue
        w = torch.as_tensor(want[key]).double()
        err = (out[key] - w).abs().max().item()
        print(f"{what} {key}: max abs err {err:.3e} (|ref| max {w.abs().max().item():.3f})", flush=True)
        assert err <= TOL, f"{what}/{key}: {err}"
    v_got = odec.decode_value(out["value"])
    v_want = odec.decode_value(torch.as_tensor(want["value"]).double())
    assert (v_got - v_want).abs().max().item() <= TOL
    assert (out["policy"][~torch.as_tensor(mask)] == 0).all()


def _check_trunk(out, want, mask, what):
    """Tokens and live cells of the trunk output (after ln_final) against the
    reference's; pad cells are exactly zero."""

    m = torch.as_tensor(mask)
    for key in ("tokens", "cells"):
        got, w = out[key], torch.as_tensor(want[key]).double()
        if key == "cells":
            assert (got[~m] == 0).all(), f"{what}: pad cells not zero"
            got, w = got[m], w[m]
        got, w = got.reshape(-1, got.shape[-1]), w.reshape(-1, w.shape[-1])
        err = (got - w).abs()
        row = ((got - w).norm(dim=1) / w.norm(dim=1).clamp(min=1e-6)).max().item()
        print(f"{what} {key}: mean abs err {err.mean().item():.3e}, max {err.max().item():.3e}, "
              f"worst row rel {row:.3e} (ref std {w.std().item():.3f})", flush=True)
        assert err.mean().item() <= TRUNK_MEAN, f"{what}/{key} mean"
        assert row <= TRUNK_ROW_REL, f"{what}/{key} row"


@pytest.mark.parametrize("name,mode", [("forward_cfg0", "parity"), ("forward_cfg0", "fresh"),
                                       ("forward_cfg0", "heads"), ("forward_cfg4", "parity"),
                                       ("forward_cfg4", "heads")])
def test_forward_matches_reference_golden(golden, name, mode):
    g = golden(name)
    c, h = (int(x) for x in g["arch"])
    net = _net(c, h, str(g["layout"]), int(g[f"{mode}_seed"]), mode)
    out = _run(net, g["feats"], g["nbr"], g["mask"], g["coords"], trunk=True)
    want = {k: g[f"{mode}_{k}"] for k in ("policy", "value", "moves_left", "cells", "tokens")}
    _check(out, want, g["mask"], f"{name}/{mode}")
    _check_trunk(out, want, g["mask"], f"{name}/{mode}")


@pytest.fixture(scope="module")
def cfg4_batch():
    from shrimp import synthetic

    return synthetic.position_batch("cfg4", 32, seed=77)


def test_forward_cfg4_matches_oracle(cfg4_batch):
    b = cfg4_batch
    layout = "CCACCACCACCA"
    net = _net(128, 8, layout, seed=5, mode="heads")
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    want = ofwd.forward_policy_value(
        weights.make_state_dict(128, 8, layout, seed=5, mode="heads"), layout, 8, b["feats"],
        b["nbr"], b["mask"], b["coords"], request_moves_left=True, dtype=torch.float32,
        return_trunk=True,
    )
    _check(out, want, b["mask"], "cfg4 B=32")
    _check_trunk(out, want, b["mask"], "cfg4 B=32")


def test_forward_cfg4_b512_matches_oracle():
    """Config 4 at the batch the benchmark is quoted on: the bench's own 512
    positions (seeded L256 generator, Npad 256), C=128, H=8, 12 blocks, the
    "heads" weights (O(1) logits), through forward_policy_value against the
    fp32 oracle (the reference's CPU path restated). Prints each output's
    largest error and the share of its gate it uses."""

    from shrimp import synthetic

    b = synthetic.position_batch("cfg4", 512)
    assert b["mask"].shape == (512, 256)
    layout = "CCACCACCACCA"
    sd = weights.make_state_dict(128, 8, layout, seed=5, mode="heads")
    net = _net(128, 8, layout, seed=5, mode="heads")
    print("cfg4 B=512 forward", flush=True)
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    print("cfg4 B=512 oracle", flush=True)
    want = ofwd.forward_policy_value(sd, layout, 8, b["feats"], b["nbr"], b["mask"], b["coords"],
                                     request_moves_left=True, dtype=torch.float32,
                                     return_trunk=True)
    for key in ("policy", "value", "moves_left"):
        err = (out[key] - want[key].double()).abs().max().item()
        print(f"cfg4 B=512 {key}: max abs err {err:.3e} = {100 * err / TOL:.0f}% of the "
              f"{TOL:g} gate", flush=True)
    v_err = (odec.decode_value(out["value"]) - odec.decode_value(want["value"].double())).abs()
    print(f"cfg4 B=512 decoded value: max abs err {v_err.max().item():.3e}", flush=True)
    _check(out, want, b["mask"], "cfg4 B=512")
    _check_trunk(out, want, b["mask"], "cfg4 B=512")


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


def test_forward_c128_ragged_pad_matches_oracle():
    """C=128, H=8 at Npad 464 (7 x 64 + 16): a small batch runs the row-split
    convs, whose last 64-row tile holds 16 rows, so three of its four waves
    have no rows (they still take part in the shared weight staging)."""

    from shrimp import synthetic
    from shrimp.batching import collate_rows

    rows = [r for r in synthetic.positions("cfg4_spec", 24, seed=34) if r[1].num_nodes <= 464][:3]
    assert len(rows) == 3
    b = collate_rows([(s, f) for _, s, f in rows], pad_to=464)
    c, h, layout = 128, 8, "CCA"
    net = _net(c, h, layout, seed=11, mode="heads")
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    want = ofwd.forward_policy_value(
        weights.make_state_dict(c, h, layout, seed=11, mode="heads"), layout, h, b["feats"],
        b["nbr"], b["mask"], b["coords"], request_moves_left=True, dtype=torch.float32,
        return_trunk=True,
    )
    _check(out, want, b["mask"], "C=128 H=8 Npad=464")
    _check_trunk(out, want, b["mask"], "C=128 H=8 Npad=464")


@pytest.mark.parametrize("c,h,npad", [(96, 4, 256), (96, 4, 512), (192, 3, 256), (192, 3, 512),
                                      (192, 3, 576)])
def test_forward_other_widths_match_oracle(c, h, npad):
    """The reference's default width (C=96, H=4: head dim 24, padded to 32)
    and its main config's (C=192, H=3: head dim 64) at Npad 256, 512 and 576
    (S = 584 at head dim 64 exceeds one workgroup's LDS: the chunked
    attention kernel) against the oracle; these widths take the generic
    linear kernels and two-launch ConvBlocks."""

    b = _wide_batch(min(npad, 512))
    if npad == 576:
        from shrimp.batching import collate_rows
        from shrimp import synthetic

        rows = [r for r in synthetic.positions("cfg4_spec", 12, seed=32) if r[1].num_nodes <= 512][:3]
        b = collate_rows([(s, f) for _, s, f in rows], pad_to=576)
    layout = "CCA"
    net = _net(c, h, layout, seed=c + h, mode="heads")
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    want = ofwd.forward_policy_value(
        weights.make_state_dict(c, h, layout, seed=c + h, mode="heads"), layout, h, b["feats"],
        b["nbr"], b["mask"], b["coords"], request_moves_left=True, dtype=torch.float32,
        return_trunk=True,
    )
    _check(out, want, b["mask"], f"C={c} H={h} Npad={npad}")
    _check_trunk(out, want, b["mask"], f"C={c} H={h} Npad={npad}")


@pytest.mark.parametrize("npad,count", [(512, 136), (576, 136), (576, 24)])
def test_forward_c128_spec_sizes_match_oracle(npad, count):
    """C=128, H=8, the full 12-block trunk on spec-faithful positions (supports
    of 280-544 cells, as the evaluator groups them) padded to Npad 512 and
    576, against the oracle. 136 positions run the large-batch kernels (the
    fused ConvBlock pair at 512; at 576, past one workgroup's fused-block
    LDS, the two-launch convs); 24 positions run the small-batch row split."""

    from shrimp import synthetic
    from shrimp.batching import collate_rows

    rows = [r for r in synthetic.positions("cfg4_spec", 3 * count, seed=41 + npad)
            if r[1].num_nodes <= npad]
    if npad == 576:
        big = [r for r in rows if r[1].num_nodes > 512]
        rows = big[: count // 4] + [r for r in rows if r[1].num_nodes <= 512]
    rows = rows[:count]
    assert len(rows) == count and max(r[1].num_nodes for r in rows) > npad - 64
    b = collate_rows([(s, f) for _, s, f in rows], pad_to=npad)
    layout = "CCACCACCACCA"
    net = _net(128, 8, layout, seed=13, mode="heads")
    what = f"C=128 H=8 Npad={npad} B={count}"
    print(what, flush=True)
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    want = ofwd.forward_policy_value(
        weights.make_state_dict(128, 8, layout, seed=13, mode="heads"), layout, 8, b["feats"],
        b["nbr"], b["mask"], b["coords"], request_moves_left=True, dtype=torch.float32,
        return_trunk=True,
    )
    _check(out, want, b["mask"], what)
    _check_trunk(out, want, b["mask"], what)


def test_forward_feature_and_index_dtypes(cfg4_batch):
    """f16 features + int32 nbr/coords (the evaluator wire types) give the
    same result as f32 + int64 up to the f16 rounding of the features."""

    b = cfg4_batch
    net = _net(128, 8, "CCACCACCACCA", seed=5)
    a = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    c = _run(net, b["feats"].half(), b["nbr"].int(), b["mask"], b["coords"].int())
    assert (a["policy"] - c["policy"]).abs().max().item() <= TOL


def test_linear_and_clamped_bias_paths_agree(cfg4_batch):
    """The attention kernel's unclamped-table path (compact positions) and its
    clamped-LUT path give the same forward up to fp16-vs-fp32 table rounding."""

    b = cfg4_batch
    net = _net(128, 8, "CCACCACCACCA", seed=5)
    lin = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    net.hip_runtime().use_linear_bias = False
    try:
        clamp = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    finally:
        net.hip_runtime().use_linear_bias = True
    for key in ("policy", "value"):
        assert (lin[key] - clamp[key]).abs().max().item() <= 1e-2, key


def test_fused_and_unfused_mlp_paths_agree(cfg4_batch):
    """The fused LN1 + q/k/v and attention-block MLP kernels (per-channel
    factors folded into bf16 weights) and the separate linear kernels give the
    same forward up to bf16 rounding points, fp32 summation order and the
    GELU evaluation (|error| <= 3.8e-6)."""

    b = cfg4_batch
    net = _net(128, 8, "CCACCACCACCA", seed=5)
    fused = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    rt = net.hip_runtime()
    rt.use_fused_mlp = rt.use_fused_qkv = rt.use_fused_block = False
    try:
        plain = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    finally:
        rt.use_fused_mlp = rt.use_fused_qkv = rt.use_fused_block = True
    for key in ("policy", "value", "moves_left"):
        err = (fused[key] - plain[key]).abs().max().item()
        print(f"fused vs unfused {key}: {err:.3e}", flush=True)
        assert err <= 1e-2, key


def test_large_batch_launch_fusions_are_bit_identical():
    """At batches that give every position its own workgroup (2 B > compute
    units) the forward runs consecutive ConvBlocks as one pair launch and the
    final LayerNorm, pooling and policy conv as one launch; both hand rows over
    inside the workgroup instead of through HBM and must give the same bits as
    the separate launches (one ConvBlock launch per block, shrimp_trunk_tail
    and the policy conv), and as ConvBlocks run as two conv launches each
    (conv1 + LN + ReLU to HBM, conv2 + LN + residual). The launch names each
    forward recorded show which kernels ran."""

    from shrimp import synthetic

    b = synthetic.position_batch("cfg4", 160, seed=78)
    net = _net(128, 8, "CCACCACCACCA", seed=6)
    rt = net.hip_runtime()
    print("large batch fusions B=160", flush=True)

    def run(**flags):
        old = {k: getattr(rt, k) for k in flags}
        for k, v in flags.items():
            setattr(rt, k, v)
        rt.timeline = []
        try:
            out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
            names = [n for n, _ in rt.timeline]
        finally:
            rt.timeline = None
            for k, v in old.items():
                setattr(rt, k, v)
        return out, names

    fused, n_fused = run()
    assert n_fused.count("conv_block_pair") == 4 and "policy_tail" in n_fused, n_fused
    plain, n_plain = run(use_block_pair=False, use_fused_tail=False)
    assert n_plain.count("conv_block") == 8 and "conv_block_pair" not in n_plain, n_plain
    assert "tail" in n_plain and "policy" in n_plain, n_plain
    # one ConvBlock as two conv launches: the same arithmetic as the fused block
    two, n_two = run(use_fused_block=False, use_fused_tail=False)
    assert n_two.count("conv1") == 8 and n_two.count("conv2") == 8, n_two
    for other, what in ((plain, "block launches"), (two, "two-conv blocks")):
        for key in ("policy", "value", "moves_left"):
            err = (fused[key] - other[key]).abs().max().item()
            print(f"fused launches vs {what} {key}: {err:.3e}", flush=True)
            assert torch.equal(fused[key], other[key]), (what, key)
    assert fused["value"].abs().max() > 0 and fused["policy"].abs().max() > 0


def test_fused_attention_option_matches_oracle(cfg4_batch):
    """The one-launch LN1 + q/k/v + attention option (no q/k/v tensor): the
    forward stays within tolerance of the oracle and of the default two-launch
    path (LayerNorm is folded into the projection there, so the bits differ)."""

    b = cfg4_batch
    layout = "CCACCACCACCA"
    net = _net(128, 8, layout, seed=5, mode="heads")
    base = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    rt = net.hip_runtime()
    rt.use_fused_attn = True
    try:
        fused = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    finally:
        rt.use_fused_attn = False
    want = ofwd.forward_policy_value(
        weights.make_state_dict(128, 8, layout, seed=5, mode="heads"), layout, 8, b["feats"],
        b["nbr"], b["mask"], b["coords"], request_moves_left=True, dtype=torch.float32,
        return_trunk=True,
    )
    _check(fused, want, b["mask"], "cfg4 B=32 fused attention")
    _check_trunk(fused, want, b["mask"], "cfg4 B=32 fused attention")
    for key in ("policy", "value", "moves_left"):
        err = (fused[key] - base[key]).abs().max().item()
        print(f"fused vs two-launch attention {key}: {err:.3e}", flush=True)
        assert err <= 2e-2, key


def test_rows_are_independent_of_batch(cfg4_batch):
    """padded == single-row (tests/test_shrimp_model.py:139-164): a row's
    outputs do not depend on the rest of the batch (bit-exact here)."""

    b = cfg4_batch
    net = _net(128, 8, "CCACCACCACCA", seed=5)
    full = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    sub = [3, 17, 30]
    part = _run(net, b["feats"][sub], b["nbr"][sub], b["mask"][sub], b["coords"][sub])
    for key in ("policy", "value", "moves_left"):
        assert torch.equal(full[key][sub], part[key]), key


def test_batches_above_the_limit_split_bit_exact(cfg4_batch):
    """A batch above the runtime's per-launch limit runs as slices: the
    outputs equal the unsplit forward's bit for bit (rows are independent)."""

    b = cfg4_batch
    net = _net(128, 8, "CCACCACCACCA", seed=5)
    rt = net.hip_runtime()
    args = [torch.as_tensor(b[k][:12]).to(DEV) for k in ("feats", "nbr", "mask", "coords")]
    full = rt.forward(*args, request_moves_left=True)
    full = {k: v.clone() for k, v in full.items()}
    rt.max_batch = 5
    try:
        assert rt.batch_limit(args[0].shape[1]) == 5
        split = rt.forward(*args, request_moves_left=True)
    finally:
        rt.max_batch = None
    for key in ("policy", "value", "moves_left"):
        assert split[key].shape == full[key].shape, key
        assert torch.equal(split[key], full[key]), key


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "graphs"])
def test_evaluator_matches_reference_reply(golden, graphs):
    """The reference evaluator's reply (ShrimpEvaluator(net, "cpu"), written
    by tests/golden/make_golden.py) from the eager forward and from the
    captured-graph forward (SHRIMP_CUDA_GRAPHS=1 in the reference)."""

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
    if graphs:
        assert len(ev.model.hip_runtime()._graphs) >= 1
    for key, gk, tol in (("values_bytes", "values", TOL), ("priors_bytes", "priors", 5e-3),
                         ("moves_left_bytes", "moves_left", 209 * TOL),
                         ("priors_logits_bytes", "priors_logits", TOL)):
        got = np.frombuffer(reply[key], np.float32)
        assert got.shape == g[gk].shape, key
        err = np.abs(got - g[gk]).max()
        print(f"evaluator {key}: max abs err {err:.3e}", flush=True)
        assert err <= tol, key


def test_full_size_cfg4_properties():
    """Config 4 at its real shape (B=512, Npad=256): finite outputs, pad
    logits exactly zero, and rows equal to a sub-batch run."""

    from shrimp import synthetic

    b = synthetic.position_batch("cfg4", 512)
    net = _net(128, 8, "CCACCACCACCA", seed=9)
    out = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"])
    assert torch.isfinite(out["policy"]).all() and torch.isfinite(out["value"]).all()
    assert (out["policy"][~b["mask"]] == 0).all()
    sub = [0, 255, 511]
    part = _run(net, b["feats"][sub], b["nbr"][sub], b["mask"][sub], b["coords"][sub])
    assert torch.equal(out["policy"][sub], part["policy"])
    assert torch.equal(out["value"][sub], part["value"])


def _host_pack(payload, start, end, pad):
    """Host pack of payload rows start..end-1 (inference.py:865-892 restated)."""

    from shrimp.constants import NUM_FEATURES

    b, total = (int(x) for x in payload["shape"])
    offs = np.asarray(payload["node_row_offsets"], dtype=np.int64)
    feats = np.frombuffer(payload["node_feats"], np.float16).reshape(total, NUM_FEATURES)
    qr = np.frombuffer(payload["node_qr"], np.int16).reshape(total, 2)
    nbr = np.frombuffer(payload["nbr"], np.uint16).reshape(total, 6)
    g = end - start
    pf = np.zeros((g, pad, NUM_FEATURES), np.float16)
    pn = np.full((g, pad, 6), 0xFFFF, np.uint16)
    pm = np.zeros((g, pad), bool)
    pc = np.zeros((g, pad, 2), np.int32)
    for k in range(g):
        o, n = int(offs[start + k]), int(offs[start + k + 1] - offs[start + k])
        pf[k, :n], pn[k, :n], pm[k, :n], pc[k, :n] = feats[o:o + n], nbr[o:o + n], True, qr[o:o + n]
    return pf, pn, pm, pc


def test_prep_csr_matches_host_pack():
    """The device pack from the CSR payload (one kernel) writes exactly what
    the host pack followed by the padded-batch preparation writes."""

    from shrimp import _lib, synthetic
    from shrimp.inference import plan_groups

    payload, _ = synthetic.serve_payload("cfg4_spec", 12)
    b, total = (int(x) for x in payload["shape"])
    offs = np.asarray(payload["node_row_offsets"], dtype=np.int64)
    feats = torch.from_numpy(np.frombuffer(payload["node_feats"], np.float16).copy()).view(total, 15)
    qr = torch.from_numpy(np.frombuffer(payload["node_qr"], np.int16).copy()).view(total, 2)
    nbr = torch.from_numpy(np.frombuffer(payload["nbr"], np.int16).copy()).view(total, 6)
    d = [t.to(DEV) for t in (feats, qr, nbr, torch.from_numpy(offs))]
    lib = _lib.load()
    st = _lib.stream_handle()
    groups = plan_groups(offs[1:] - offs[:-1])
    assert len(groups) >= 2
    for start, end, pad in groups:
        g = end - start
        print(f"prep_csr group rows {start}..{end} pad {pad}", flush=True)
        outs = []
        for mode in ("csr", "host"):
            o = [torch.full((g, pad, 7), -5, dtype=torch.int32, device=DEV),
                 torch.full((g, pad), 7, dtype=torch.uint8, device=DEV),
                 torch.full((g, pad, 2), -5, dtype=torch.int32, device=DEV),
                 torch.full((g,), -5, dtype=torch.int32, device=DEV),
                 torch.full((g, pad + 8), 7, dtype=torch.uint8, device=DEV),
                 torch.full((g, pad, 32), 3.0, dtype=torch.bfloat16, device=DEV)]
            ptrs = [t.data_ptr() for t in o]
            if mode == "csr":
                rc = lib.shrimp_prep_csr(d[0].data_ptr(), 15, d[1].data_ptr(), d[2].data_ptr(),
                                         d[3].data_ptr(), start, g, pad, 8, *ptrs, st)
            else:
                pf, pn, pm, pc = (torch.from_numpy(x).to(DEV) for x in _host_pack(payload, start, end, pad))
                rc = lib.shrimp_prep_inputs(pn.view(torch.int16).data_ptr(), _lib.DT_U16, pm.data_ptr(),
                                            pc.data_ptr(), _lib.DT_I32, pf.data_ptr(), _lib.DT_F16, 15,
                                            g, pad, 8, *ptrs, st)
            _lib.check(rc, mode)
            torch.cuda.synchronize()
            outs.append(o)
        for a, c in zip(*outs):
            assert torch.equal(a, c)


@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "graphs"])
def test_evaluator_multi_group_matches_oracle(graphs):
    """Spec-variant payload (supports of 280-544 nodes): several groups with
    different pad widths, packed on the device, against the CPU oracle's
    evaluator on the same payload; eager and captured-graph forwards. O(1)
    head weights ("heads" mode), so the value / logit gates see trunk
    errors."""

    from oracle import decode as odec
    from shrimp import synthetic
    from shrimp.inference import ShrimpEvaluator, plan_groups

    payload, _ = synthetic.serve_payload("cfg4_spec", 10, request_moves_left=True, request_logits=True)
    offs = np.asarray(payload["node_row_offsets"], dtype=np.int64)
    assert len(plan_groups(offs[1:] - offs[:-1])) >= 2
    sd = weights.make_state_dict(32, 4, "CCA", seed=3, mode="heads")
    net = _net(32, 4, "CCA", seed=3, mode="heads")
    ev = ShrimpEvaluator(net, DEV, graphs=graphs)
    got = ev.evaluate_payload(payload)
    if graphs:
        assert len(net.hip_runtime()._graphs) >= 1
    want = odec.evaluate(payload, sd, "CCA", 4)
    for key, tol in (("values_bytes", TOL), ("priors_bytes", 5e-3), ("moves_left_bytes", 209 * TOL),
                     ("priors_logits_bytes", TOL)):
        a = np.frombuffer(got[key], np.float32)
        b = np.frombuffer(want[key], np.float32)
        assert a.shape == b.shape, key
        err = np.abs(a - b).max()
        print(f"evaluator multi-group {key}: max abs err {err:.3e}", flush=True)
        assert err <= tol, key


def test_evaluator_group_streams_are_bit_identical():
    """A spec-variant payload of 300 positions (groups of 111, 140, 45 and 4
    rows at Npad 576, 512, 448 and 384; C = 128, H = 8): its groups' forwards
    spread over two or three side streams give the same reply bytes as one
    stream, twice in a row (the second payload reuses the streams and the
    memory the first one freed on them)."""

    from shrimp import synthetic
    from shrimp.inference import ShrimpEvaluator, plan_groups

    payload, _ = synthetic.serve_payload("cfg4_spec", 300, seed=5, request_moves_left=True,
                                         request_logits=True)
    offs = np.asarray(payload["node_row_offsets"], dtype=np.int64)
    groups = plan_groups(offs[1:] - offs[:-1])
    print(f"group streams: groups {[(e - s, p) for s, e, p in groups]}", flush=True)
    assert len(groups) >= 3
    net = _net(128, 8, "CCACCACCACCA", seed=6, mode="heads")
    ev = ShrimpEvaluator(net, DEV, graphs=False)
    ev.group_streams = 1
    want = ev.evaluate_payload(payload)
    for n in (2, 3, 3):
        ev.group_streams = n
        got = ev.evaluate_payload(payload)
        assert len(ev._group_streams) >= n
        for key in want:
            assert got[key] == want[key], (n, key)


def test_graph_replays_match_eager():
    """Captured forwards (graphs=True) against the eager evaluator, payload by
    payload, with eager work and synchronizations between the replays: a
    second payload reuses a bucket with fewer rows (pad rows reset), the
    first payload is then replayed again. Same kernels on the same inputs:
    byte-identical replies."""

    from shrimp import synthetic
    from shrimp.inference import ShrimpEvaluator

    net = _net(128, 8, "CCACCACCACCA", seed=7)
    eager = ShrimpEvaluator(net, DEV, graphs=False)
    graphed = ShrimpEvaluator(net, DEV, graphs=True)
    pa, _ = synthetic.serve_payload("cfg4", 11, seed=5, request_moves_left=True)
    pb, _ = synthetic.serve_payload("cfg4", 6, seed=6, request_moves_left=True)
    want = {k: eager.evaluate_payload(p) for k, p in (("a", pa), ("b", pb))}
    for step, (k, p) in enumerate((("a", pa), ("b", pb), ("a", pa), ("b", pb))):
        print(f"graph replay step {step} payload {k}", flush=True)
        got = graphed.evaluate_payload(p)
        torch.cuda.synchronize()
        for key in want[k]:
            assert got[key] == want[k][key], (step, key)
        # eager work between replays
        _run(net, *(torch.as_tensor(x) for x in _host_pack(pb, 0, 2, 256)))
        torch.cuda.synchronize()
    rt = net.hip_runtime()
    assert len(rt._graphs) >= 1



@pytest.mark.parametrize("graphs", [False, True], ids=["eager", "graphs"])
def test_evaluator_pipelined_submissions_match(graphs):
    """Three payloads submitted before any is collected (uploads on the copy
    stream overlap the forwards), collected out of order: each reply is
    byte-identical to evaluating that payload alone."""

    from shrimp import synthetic
    from shrimp.inference import ShrimpEvaluator

    net = _net(128, 8, "CCACCACCACCA", seed=9)
    ev = ShrimpEvaluator(net, DEV, graphs=graphs)
    pays = [synthetic.serve_payload("cfg4", n, seed=s, request_moves_left=(s % 2 == 0))[0]
            for n, s in ((40, 11), (7, 12), (64, 13))]
    want = [ev.evaluate_payload(p) for p in pays]
    handles = [ev.submit_payload(p) for p in pays]
    for i in (1, 0, 2):
        print(f"pipelined result {i} graphs={graphs}", flush=True)
        got = ev.result(handles[i])
        assert set(got) == set(want[i])
        for key in want[i]:
            assert got[key] == want[i][key], (i, key)


def test_evaluator_busy_trace_counts_every_payload():
    """With the busy trace on (SHRIMP_PERF_TRACE=1 sets it), every collected
    payload adds its device time and rows to the report; tracing leaves the
    reply bytes unchanged."""

    from shrimp import synthetic
    from shrimp.inference import GpuBusyTrace, ShrimpEvaluator

    net = _net(128, 8, "CCACCACCACCA", seed=9)
    ev = ShrimpEvaluator(net, DEV)
    assert ev.perf_trace_report() is None
    pays = [synthetic.serve_payload("cfg4", n, seed=s)[0] for n, s in ((40, 21), (9, 22), (64, 23))]
    want = [ev.evaluate_payload(p) for p in pays]
    ev._perf = GpuBusyTrace()
    got = [ev.evaluate_payload(pays[0])]
    handles = [ev.submit_payload(p) for p in pays[1:]]
    got += [ev.result(h) for h in handles]
    assert got == want
    rep = ev.perf_trace_report()
    print("busy trace:", rep, flush=True)
    assert rep["measured_flushes"] == 3 and rep["measured_states"] == 113
    assert rep["device_busy_ms"] > 0 and rep["wall_window_ms"] > 0
    assert 0 < rep["gpu_busy_fraction"] <= 1.5
    assert rep["mean_batch"] == round(113 / 3, 1) and rep["median_batch"] == 40.0


def test_staged_attention_matches_the_row_layout_path(cfg4_batch):
    """The staged attention (K and V in fragment order from the q/k/v kernel,
    the key table once per forward, DMA staging) against the (3, B, H, S,
    dpad) layout with the in-kernel key setup at the same wave count: both
    compute the same products in the same order and drop dead keys the same
    way, so the forward is bit-identical."""

    from shrimp import _lib

    b = cfg4_batch
    net = _net(128, 8, "CCACCACCACCA", seed=5, mode="heads")
    rt = net.hip_runtime()
    rt.use_staged_attn = False
    # the staged kernel runs four waves per workgroup: the row-layout kernel's
    # four-wave variant splits the last query block the same way
    lib = _lib.load()
    prev = lib.shrimp_attn_variant(2)
    try:
        base = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    finally:
        lib.shrimp_attn_variant(prev)
        rt.use_staged_attn = True
    rt.keep_buffers = True
    try:
        net.forward_policy_value(*[torch.as_tensor(b[k]).to(DEV) for k in ("feats", "nbr", "mask", "coords")])
        assert rt.last["staged"], "the staged path did not run"
    finally:
        rt.keep_buffers = False
        rt.last = None
    staged = _run(net, b["feats"], b["nbr"], b["mask"], b["coords"], trunk=True)
    for key in ("policy", "value", "moves_left", "tokens", "cells"):
        err = (staged[key] - base[key]).abs().max().item()
        print(f"staged vs row-layout attention {key}: {err:.3e}", flush=True)
        assert err == 0.0, key


def _keys_table(coords, mask, seq_lens, S, nt, xw=53, xd=26):
    """numpy restatement of shrimp_attn_keys' table (layout in attn.hip)."""

    B = coords.shape[0]
    sp = (S + 15) // 16 * 16
    nkb = sp // 16
    ints = (4 * sp + 3 * nkb + 8 + 3) & ~3
    out = np.zeros((B, ints), np.int64)
    for p in range(B):
        L = int(min(max(seq_lens[p], 0), S))
        cls = np.full(sp, 2)
        q = np.zeros(sp, np.int64)
        r = np.zeros(sp, np.int64)
        for key in range(sp):
            if key < nt and key < L:
                cls[key] = 1
            elif nt <= key < L:
                q[key], r[key] = coords[p, key - nt]
                cls[key] = 0 if mask[p, key - nt] else 2
        live = cls == 0
        span_ok = nt <= 16 and live.any()
        q0 = r0 = 0
        if live.any():
            q0, r0 = q[live].min(), r[live].min()
            span_ok = span_ok and q[live].max() - q0 <= xd and r[live].max() - r0 <= xd
        else:
            q0 = r0 = 1 << 30
        m = out[p]
        m[0:2 * sp:2], m[1:2 * sp:2] = q, r
        if span_ok:
            m[2 * sp:3 * sp] = (np.where(live, q, q0) * xw + np.where(live, r, r0)) * 4
        m[3 * sp:4 * sp] = cls
        for blk in range(nkb):
            keys = np.arange(blk * 16, blk * 16 + 16)
            past = keys >= L
            special = (~past) & ((cls[keys] != 0) | (keys < nt))
            m[4 * sp + blk] = int(past.any() or special.any())
            m[4 * sp + nkb + blk] = int(special.any())
            m[4 * sp + 2 * nkb + blk] = int(past.any() or ((~past) & (cls[keys] == 2)).any())
        h = 4 * sp + 3 * nkb
        m[h], m[h + 1], m[h + 2] = int(span_ok), q0, r0
    return out.astype(np.int32)


def test_attn_keys_table_matches_restatement():
    """shrimp_attn_keys against a numpy restatement on positions with tokens,
    masked cells inside the bound, a short bound, a wide (non-LINEAR) span and
    an empty position."""

    from shrimp import ops

    rng = np.random.default_rng(4)
    B, N, nt = 5, 40, 8
    S = N + nt
    coords = rng.integers(-6, 7, size=(B, N, 2)).astype(np.int32)
    mask = np.ones((B, N), np.uint8)
    mask[1, 5] = 0
    mask[1, 17] = 0
    coords[3, 2] = (40, -3)  # span > 26
    mask[4] = 0
    seq_lens = np.array([S, S, 30, S, 0], np.int32)
    meta = torch.empty((B, ops.attn_keys_ints(S)), dtype=torch.int32, device=DEV)
    ops.launch_attn_keys(coords=torch.as_tensor(coords).to(DEV), mask8=torch.as_tensor(mask).to(DEV),
                         seq_lens=torch.as_tensor(seq_lens).to(DEV), B=B, S=S, n_tokens=nt, meta=meta)
    got = meta.cpu().numpy()
    want = _keys_table(coords, mask, seq_lens, S, nt)
    assert got.shape == want.shape
    for p in range(B):
        bad = np.nonzero(got[p] != want[p])[0]
        assert bad.size == 0, (p, bad[:8], got[p][bad[:8]], want[p][bad[:8]])
