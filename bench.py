"""Shrimp forward benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds T]

Workload: ShrimpNet(channels=128, heads=8, trunk "CCACCACCACCA") serve forward
(forward_policy_value: policy logits + value logits) at B=512 positions,
Npad=256 (S=264), bf16 kernels, seeded random-init weights, seeded synthetic
positions (shrimp.synthetic "cfg4": 10-80 stones, support radius 4, L256
capped). Inputs are device-resident before timing. One step = one forward.

Prints one JSON line with the metric, the per-kernel roofline of the
dominant kernel (the fused ConvBlock, timed live with HIP events on the
launch stream, re-launched alone and inside the forward), the attention
kernel's figures, per-kernel times inside real forwards, configs 1-3 as
standalone ops at B=1024 with their rooflines, the fp32 serve mode's
forward, and the CPU baseline (the reference CPU forward restated in the
oracle, fp32 eager with sdpa, on the same 512 positions: the median of five
forwards, rank 0 only).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "hexo-bot_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "Shrimp fwd positions/sec @B=512 bf16 on 1 MI355X; attn/conv % MFMA peak"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
B, NPAD, C, H, LAYOUT = 512, 256, 128, 8, "CCACCACCACCA"


def _events_time(fn, reps, stream):
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


def kernel_timings(net, inputs, reps=50):
    """Re-launch single kernels of the forward on its own buffers (ConvBlocks 0
    and 1 as the forward's one pair launch, ConvBlock 0 alone, its conv1 alone,
    the attention kernel and the row kernels of attention block 0); average
    duration per launch from HIP events on the launch stream. Re-launches write
    into copies, never into the forward's residual stream."""

    import torch

    from shrimp import ops
    from shrimp.geometry import CELL_LUT_M

    rt = net.hip_runtime()
    rt.keep_buffers = True
    net.forward_policy_value(*inputs)
    L = rt.last
    rt.keep_buffers = False
    P = L["P"]
    b, n, s = L["B"], L["N"], L["S"]
    cells = L["seq"][:, 8:]
    k = P.convs[0]
    stream = torch.cuda.current_stream()

    def conv():
        ops.launch_conv(
            x=cells, x_sb=s * C, x_sn=C, idx=L["idx"], taps=7, idx_stride=7, mask8=L["mask8"],
            wpack=k.w1, bias=k.b1, B=b, N=n, cin_pad=C, cout=C, ln_w=k.ln1w, ln_b=k.ln1b,
            eps=k.eps1, relu=True, out=L["y1"], o_sb=n * C, o_sn=C, stream=L["stream"],
        )

    # same (position, row) strides as `cells` (a clone of the view would be compact)
    cells_out = L["seq"].clone()[:, 8:]

    def block():
        ops.launch_conv_block(
            x=cells, x_sb=s * C, x_sn=C, idx=L["idx"], idx_stride=7, mask8=L["mask8"], B=b, N=n,
            C=C, w1=k.w1, b1=k.b1, ln1_w=k.ln1w, ln1_b=k.ln1b, eps1=k.eps1, w2=k.w2, b2=k.b2,
            ln2_w=k.ln2w, ln2_b=k.ln2b, eps2=k.eps2, gamma=k.gamma, out=cells_out,
            o_sb=s * C, o_sn=C, stream=L["stream"],
        )

    k2 = P.convs[1]
    pair_blocks = [dict(w1=q.w1, b1=q.b1, ln1_w=q.ln1w, ln1_b=q.ln1b, eps1=q.eps1, w2=q.w2, b2=q.b2,
                        ln2_w=q.ln2w, ln2_b=q.ln2b, eps2=q.eps2, gamma=q.gamma) for q in (k, k2)]

    def pair():
        ops.launch_conv_block_pair(
            x=cells, x_sb=s * C, x_sn=C, idx=L["idx"], idx_stride=7, mask8=L["mask8"], B=b, N=n,
            C=C, blocks=pair_blocks, out=cells_out, o_sb=s * C, o_sn=C, stream=L["stream"],
        )

    a = P.attn[0]
    seq = L["seq"]
    # the forward keeps no q/k/v tensor when attention projects its own
    qkv = L["qkv"]
    if qkv is None:
        qkv = torch.empty((3, b, H, s, P.dpad), dtype=torch.bfloat16, device=seq.device)
    bias_kw = dict(
        seq_lens=L["seq_lens"], o=L["att"], o_sb=s * C, o_sh=P.d, o_sr=C, B=b, S=s, H=H,
        d=P.d, dpad=P.dpad, coords=L["coords32"], mask8=L["mask8"], btab=a.btab_xtab[0],
        xtab=a.btab_xtab[1], lut_m=CELL_LUT_M, n_tokens=8, stream=L["stream"],
    )

    staged = bool(L.get("staged"))

    def attn():
        if staged:
            kw = {k: v for k, v in bias_kw.items() if k not in ("coords", "mask8")}
            ops.launch_attn_staged(q=qkv[0], qkv_sb=H * s * P.dpad, qkv_sh=s * P.dpad,
                                   kvf=L["kvf"], meta=L["meta"], **kw)
            return
        ops.launch_attn(q=qkv[0], k=qkv[1], v=qkv[2], qkv_sb=H * s * P.dpad,
                        qkv_sh=s * P.dpad, **bias_kw)

    def attn_fused():
        ops.launch_attn_fused(x=seq, x_sb=s * C, x_sr=C, packed=a.qkv, eps=a.eps1, **bias_kw)

    from shrimp import _lib

    rows = b * s

    def lin(mode, x, x_sr, w, bias, n_in, n_out, out, o_sr, **kw):
        return lambda: ops.launch_linear(
            x=x, x_sr=x_sr, wpack=w, bias=bias, rows=rows, n_in=n_in, n_out=n_out, mode=mode,
            out=out, o_sr=o_sr, stream=L["stream"], **kw)

    # Timing re-launches write into the forward's scratch buffers only (never
    # back into seq): residual modes target a copy.
    seq_copy = seq.clone()
    qkv_fn = (lambda: ops.launch_attn_qkv_kvf(
        x=seq, x_sr=C, q=qkv, kvf=L["kvf"], packed=a.qkv, eps=a.eps1, rows=rows, B=b, S=s, H=H,
        C=C, dpad=P.dpad, stream=L["stream"])) if staged else (lambda: ops.launch_attn_qkv(
        x=seq, x_sr=C, qkv=qkv[0], packed=a.qkv, eps=a.eps1, rows=rows, B=b, S=s, H=H, C=C,
        dpad=P.dpad, stream=L["stream"])) if P.fused_qkv else lin(
            _lib.LIN_QKV, seq, C, a.qkv_w, a.qkv_b, C, 3 * C, qkv[0], 0, ln_w=a.ln1w,
            ln_b=a.ln1b, B=b, S=s, H=H, dpad=P.dpad)
    linears = {"qkv": (qkv_fn, rows * C * 3 * C * 2.0, rows * (C + 3 * C) * 2.0)}
    if P.fused_mlp:
        linears["attn_mlp"] = (
            lambda: ops.launch_attn_mlp(
                x=L["att"], x_sr=C, seq=seq_copy, s_sr=C, mask=L["seq_mask"], packed=a.mlp,
                eps=a.eps2, rows=rows, C=C, hidden=2 * C, stream=L["stream"]),
            rows * (C * C + 4 * C * C) * 2.0, rows * 3 * C * 2.0)
    else:
        hid = L["hid"]
        linears.update({
            "out_proj": (lin(_lib.LIN_RESID, L["att"], C, a.out_w, a.out_b, C, C, seq_copy, C,
                             resid=seq_copy, r_sr=C, gamma=a.g_attn, mask=L["seq_mask"]),
                         rows * C * C * 2.0, rows * 3 * C * 2.0),
            "fc1": (lin(_lib.LIN_GELU, seq, C, a.fc1_w, a.fc1_b, C, 2 * C, hid, 2 * C,
                        ln_w=a.ln2w, ln_b=a.ln2b), rows * C * 2 * C * 2.0, rows * 3 * C * 2.0),
            "fc2": (lin(_lib.LIN_RESID, hid, 2 * C, a.fc2_w, a.fc2_b, 2 * C, C, seq_copy, C,
                        resid=seq_copy, r_sr=C, gamma=a.g_mlp, mask=L["seq_mask"]),
                    rows * 2 * C * C * 2.0, rows * 4 * C * 2.0),
        })
    conv()
    block()
    pair()
    qkv_fn()
    attn()
    conv_ms = _events_time(conv, reps, stream)
    block_ms = _events_time(block, reps, stream)
    pair_ms = _events_time(pair, reps, stream)
    attn_ms = _events_time(attn, reps, stream)
    # the one-launch LN1 + q/k/v + attention kernel, timed whichever path the
    # forward takes
    fused_ms = None
    if P.fused_qkv and ops.attn_fused_supported(C, H, s, P.dpad):
        attn_fused()
        fused_ms = _events_time(attn_fused, reps, stream)
    extra = {}
    for name, (fn, flops, nbytes) in linears.items():
        fn()
        ms = _events_time(fn, reps, stream)
        extra[name] = {"ms": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                       "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    seq_lens = L["seq_lens"].cpu().to(torch.float64)
    valid_rows = int(L["mask8"].sum().item())
    return {
        "pair_ms": pair_ms,
        "pair_flops": 4 * 2.0 * 7 * C * C * b * n,
        # x in, the first block's rows out (the second block's residual) and back
        # in, the second block's rows out; index, mask, four weight sets
        "pair_bytes": b * n * C * 2 * 4 + b * n * 7 * 4 + b * n + 4 * 7 * C * C * 2,
        "block_ms": block_ms,
        "block_flops": 2 * 2.0 * 7 * C * C * b * n,
        "block_bytes": b * n * C * 2 * 2 + b * n * 7 * 4 + b * n + 2 * 7 * C * C * 2,
        "conv_ms": conv_ms,
        "conv_flops": 2.0 * 7 * C * C * b * n,
        "conv_flops_valid": 2.0 * 7 * C * C * valid_rows,
        "conv_bytes": b * n * C * 2 * 2 + b * n * 7 * 4 + 7 * C * C * 2,
        "attn_ms": attn_ms,
        "attn_staged": staged,
        "attn_fused_ms": fused_ms,
        "forward_attn_fused": bool(L["attn_fused"]),
        "attn_flops": float(4 * P.d * H * (seq_lens ** 2).sum().item()),
        "attn_bytes": float(4 * 2 * P.d * H * seq_lens.sum().item()),
        "proj_flops": rows * C * 3 * C * 2.0,
        "proj_bytes": rows * C * 2 * 2.0,
        "linears": extra,
    }


def evaluator_timing(net, count: int = B, graphs: bool = False, reps: int = 5) -> dict:
    """Secondary figure: the ABI-1 evaluator end to end on the same 512 cfg4
    positions as a wire payload (parse, upload of the CSR arrays, device pack,
    forward, decode, reply bytes back on the host). Wall clock per payload;
    host-device copies included, so it is reported beside `value`, not as it."""

    import numpy as np
    import torch

    from shrimp import synthetic
    from shrimp.inference import ShrimpEvaluator, plan_groups

    payload, _ = synthetic.serve_payload("cfg4", count)
    ev = ShrimpEvaluator(net, "cuda", graphs=graphs)
    ev.evaluate_payload(payload)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        ev.evaluate_payload(payload)
    el = (time.perf_counter() - t0) / reps
    # A caller that keeps one payload in flight (submit the next, then collect
    # the previous) overlaps uploads and host work with the forward.
    warm = [ev.submit_payload(payload), ev.submit_payload(payload)]
    for h in warm:
        ev.result(h)
    handles = [ev.submit_payload(payload)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        handles.append(ev.submit_payload(payload))
        ev.result(handles.pop(0))
    ev.result(handles.pop(0))
    el_pipe = (time.perf_counter() - t0) / (reps + 1)
    offs = np.asarray(payload["node_row_offsets"], dtype=np.int64)
    nbytes = sum(len(payload[k]) for k in ("node_feats", "node_qr", "nbr", "legal_counts"))
    return {
        "path": "ShrimpEvaluator.evaluate_payload (payload bytes -> reply bytes)",
        "graphs": graphs,
        "positions": count,
        "positions_per_s": round(count / el, 1),
        "ms_per_payload": round(el * 1e3, 4),
        "pipelined_positions_per_s": round(count / el_pipe, 1),
        "pipelined_ms_per_payload": round(el_pipe * 1e3, 4),
        "groups": len(plan_groups(offs[1:] - offs[:-1])),
        "payload_bytes": nbytes,
        "reps": reps,
    }


def featurize_timing(rows, reps: int = 20) -> dict:
    """The featurizer row: the 512 cfg4 decision states (placement records)
    -> padded forward inputs on the device (``shrimp_featurize``), timed with
    HIP events around the launch (records already resident); the host builder
    (``build_position`` + ``collate_rows``, one thread) on the same states for
    comparison. The device output is checked against the host batch."""

    import ctypes

    import torch

    from shrimp import _lib
    from shrimp.batching import collate_rows
    from shrimp.featurize import featurize, pack_records
    from shrimp.features import build_position
    from shrimp.synthetic import CONFIGS

    facts = [f for f, _, _ in rows]
    rad = CONFIGS["cfg4"].radius  # the support radius the positions were drawn for
    dev = torch.device("cuda")
    out = featurize(facts, radius=rad, npad=NPAD, device=dev)
    t0 = time.perf_counter()
    host = collate_rows([build_position(f, radius=rad) for f in facts], pad_to=NPAD)
    host_s = time.perf_counter() - t0
    exact = bool(torch.equal(out["feats"].cpu(), host["feats"]) and
                 torch.equal(out["nbr"].cpu().long(), host["nbr"]))
    pk = {k: torch.from_numpy(v).to(dev) for k, v in pack_records(facts).items()}
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    b = len(facts)
    args = [pk["qr"].data_ptr(), pk["owner"].data_ptr(), pk["index"].data_ptr(),
            pk["offsets"].data_ptr(), pk["player"].data_ptr(), pk["phase"].data_ptr(), b, rad, NPAD,
            out["feats"].data_ptr(), out["nbr"].data_ptr(),
            torch.empty((b, NPAD), dtype=torch.uint8, device=dev).data_ptr(),
            out["coords"].data_ptr(), out["counts"].data_ptr(), out["status"].data_ptr(), st]
    run = lambda: _lib.check(lib.shrimp_featurize(*args), "featurize")
    run()
    ms = _events_time(run, reps, torch.cuda.current_stream(dev))
    stones = int(pk["offsets"][-1].item())
    return {
        "kernel": "featurize_kernel (records -> support, node order, nbr, 15 planes, padded)",
        "positions": b,
        "launch_ms": round(ms, 5),
        "positions_per_s": round(b / (ms * 1e-3), 1),
        "input_bytes": stones * 12 + (b + 1) * 8 + 2 * b,
        "output_bytes": b * NPAD * (15 * 4 + 6 * 4 + 1 + 2 * 4),
        "host_builder_positions_per_s": round(b / host_s, 1),
        "host_builder_threads": 1,
        "matches_host_builder": exact,
    }


def hexfield_timing(reps: int = 50, cpu_sample: int = 16) -> dict:
    """The hexfield ray kernels at the config-3 shape (B = 1024 cfg3 cell sets,
    Npad = 256, 32-slot ray index from shrimp_build_ray_index, random raylen
    0..5): ray attention with 6 heads of 16 (C = 96) and K1 (ray-tap conv +
    LayerNorm + ReLU) at C = Cout = 128 (orbit width 128) and C = Cout = 96
    (orbit width 8). HIP events on the launch stream around back-to-back
    launches; algorithmic bytes count each row of q/k/v/x/idx once (live rows
    only where the kernel skips the rest) and every output row. The CPU
    column is the fp32 oracle on ``cpu_sample`` positions, one thread."""

    import numpy as np
    import torch

    from hexfield_eq import build_ray_gather_index, build_tap_reach, ops as hops
    from oracle import hexfield as ohf
    from shrimp import synthetic

    dev = torch.device("cuda")
    stream = torch.cuda.current_stream(dev)
    bt = synthetic.position_batch("cfg3", 1024)
    mask = bt["mask"].to(dev)
    coords = bt["coords"].to(dev)
    b, n = mask.shape
    gen = torch.Generator().manual_seed(5)
    idx = build_ray_gather_index(coords, mask)
    raylen = torch.randint(0, 6, (b, n, 12), generator=gen, dtype=torch.uint8).to(dev)
    cell = torch.arange(1, n + 1, device=dev, dtype=torch.int32)
    seq = (cell * mask.to(torch.int32)).amax(dim=1).to(torch.int32)
    live_rows = int(seq.sum().item())
    out = {}

    # ray attention
    h, d = 6, 16
    q, k, v = [torch.randn(b, n, h, d, generator=gen).half().to(dev).transpose(1, 2)
               for _ in range(3)]
    sb = (0.5 * torch.randn(32, h, generator=gen)).half().to(dev)
    o = torch.empty((b, h, n, d), dtype=torch.float16, device=dev)
    run = lambda: hops.launch_ray_attn(q, k, v, idx, sb, raylen, seq, True, o)
    run()
    ms = _events_time(run, reps, stream)
    prev = hops.ray_attn_variant(1)
    run()
    ms_glob = _events_time(run, reps, stream)
    hops.ray_attn_variant(prev)
    # live (row, head, slot) triples, for the flop count
    ii = idx.long()
    present = (ii >= 0) & (ii < n)
    rows_live = torch.arange(n, device=dev)[None, :] < seq[:, None].long()
    slots = torch.arange(32, device=dev)
    kk = (slots - 1) % 5 + 1
    live_pairs = 0
    for hh in range(h):
        ax, side = hh // 2, hh % 2
        geo = (slots >= 1 + 10 * ax) & (slots <= 10 + 10 * ax)
        dirn = ((slots - 1) % 10) // 5
        rl = raylen.long()[:, :, side * 6 + ax * 2 + dirn.clamp(0, 1)]
        ok = present & ((slots == 0) | (geo & (kk <= rl)))
        live_pairs += int((ok & rows_live[:, :, None]).sum().item())
    flops = live_pairs * 4 * d
    nbytes = 3 * live_rows * h * d * 2 + b * n * h * d * 2 + live_rows * (32 * 4 + 12) + b * 4
    sel = slice(0, cpu_sample)
    qc, kc, vc = q[sel].cpu().float(), k[sel].cpu().float(), v[sel].cpu().float()
    t0 = time.perf_counter()
    ohf.ray_attn(qc, kc, vc, idx[sel].cpu(), sb.cpu(), raylen[sel].cpu(), seq[sel].cpu(), True,
                 dtype=torch.float32)
    cpu_s = time.perf_counter() - t0
    out["ray_attn"] = {
        "kernel": "ray_attn_kernel<16, staged> (K/V of a head pair in LDS)",
        "workload": f"B={b} Npad={n} H={h} D={d} blockers, cfg3 cell sets",
        "launch_ms": round(ms, 5),
        "launch_ms_global_gather": round(ms_glob, 5),
        "algorithmic_bytes": nbytes,
        "bound": "hbm",
        "achieved_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "peak_gbs": PEAK_HBM_GBS,
        "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "live_slot_pairs": live_pairs,
        "flops": flops,
        "positions_per_s": round(b / (ms * 1e-3), 1),
        "cpu_oracle_positions_per_s": round(cpu_sample / cpu_s, 1),
        "cpu_sample": f"{cpu_sample} positions, fp32 gathered oracle, 1 process",
    }

    # K1 ray-tap conv + LN
    reach = build_tap_reach(raylen)
    nbr = bt["nbr"].to(dev).to(torch.int32)
    gidx = torch.cat([torch.arange(n, device=dev, dtype=torch.int32).view(1, n, 1).expand(b, n, 1),
                      nbr], dim=2).contiguous()
    m8 = mask.to(torch.uint8).contiguous()
    re12 = reach.reshape(b, n, 12).contiguous()
    for c, corb in ((128, 128), (96, 8)):
        x = torch.randn(b, n, c, generator=gen).half().to(dev)
        w = (torch.randn(7, c, c, generator=gen) / np.sqrt(7 * c)).half().to(dev)
        bias = (0.02 * torch.randn(c, generator=gen)).to(dev)
        lnw = (torch.rand(c, generator=gen) + 0.5).to(dev)
        lnb = (0.1 * torch.randn(c, generator=gen)).to(dev)
        alpha = torch.stack([0.8 ** kk_ * (1 + 0.1 * torch.randn(c, generator=gen))
                             for kk_ in range(5)]).half().to(dev)
        packed = hops.pack_raytap_weight(w)
        y = torch.empty((b, n, c), dtype=torch.float16, device=dev)
        run = lambda: hops.launch_conv_ln_raytap(x, gidx, m8, packed, bias, lnw, lnb, idx, re12,
                                                 alpha, 1e-5, True, corb, y)
        run()
        ms = _events_time(run, reps, stream)
        kflops = b * n * 7 * c * c * 2
        kbytes = b * n * (c * 2 + 32 * 4 + 12 + 7 * 4 + 1 + c * 2) + 7 * c * c * 2
        tfl = kflops / (ms * 1e-3) / 1e12
        xs, ws = x[sel].cpu().float(), w.cpu().float()
        t0 = time.perf_counter()
        ohf.conv_ln_raytap(xs, gidx[sel].cpu(), mask[sel].cpu(), ws, bias.cpu(), lnw.cpu(),
                           lnb.cpu(), idx[sel].cpu(), reach[sel].cpu(), alpha.cpu().float(), 1e-5,
                           True, corb, dtype=torch.float32)
        cpu_s = time.perf_counter() - t0
        out[f"conv_ln_raytap_c{c}"] = {
            "kernel": f"conv_ln_raytap_kernel<{c}, {c}> (orbit width {corb})",
            "workload": f"B={b} Npad={n} C=Cout={c}, 7 taps from 31 ray rows, LN + ReLU",
            "launch_ms": round(ms, 5),
            "bound": "mfma",
            "achieved_tflops": round(tfl, 2),
            "peak_tflops": PEAK_BF16_TFLOPS,
            "frac": round(tfl / PEAK_BF16_TFLOPS, 4),
            "flops": kflops,
            "algorithmic_bytes": kbytes,
            "hbm_gbs_algorithmic": round(kbytes / (ms * 1e-3) / 1e9, 1),
            "positions_per_s": round(b / (ms * 1e-3), 1),
            "cpu_oracle_positions_per_s": round(cpu_sample / cpu_s, 1),
            "cpu_sample": f"{cpu_sample} positions, fp32 oracle, 1 process",
        }
    return out


def _host_cpu() -> dict:
    """CPU model (every model string lscpu and /proc/cpuinfo report, the
    longest kept), sockets and cores from lscpu, and the cores this process
    may use (sched affinity)."""

    names, info = [], {}
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            key, _, val = ln.partition(":")
            info.setdefault(key.strip(), val.strip())
            if key.strip() in ("Model name", "BIOS Model name"):
                names.append(val.strip())
    except Exception:  # lscpu missing: the model comes from /proc/cpuinfo or stays unknown
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.lower().startswith("model name"):
                    names.append(ln.split(":", 1)[1].strip())
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"model": max(names, key=len) if names else None,
            "sockets": info.get("Socket(s)"), "cores_per_socket": info.get("Core(s) per socket"),
            "threads_per_core": info.get("Thread(s) per core"),
            "vendor": info.get("Vendor ID"), "family": info.get("CPU family"),
            "model_id": info.get("Model"), "flags_avx512f": "avx512f" in info.get("Flags", ""),
            "cores_visible": os.cpu_count(), "cores_usable": usable}


def cpu_baseline(batch, seconds: float, sample: int = 512, runs: int = 5, warmup: int = 2):
    """The reference CPU forward restated (oracle.forward: the pair rows built
    in torch as model.py:677-716 does, the fp16 bias per block, sdpa with that
    mask, fp32 eager) on the same cfg4 workload: the first `sample` of the 512
    positions as one batch, `warmup` untimed forwards, then the median of
    `runs` timed forwards (more while the timed total stays under `seconds`);
    positions/s on the host cores this process may use, capped by
    OMP_NUM_THREADS where the host sets it (the GPU box allots 16 threads per
    GPU)."""

    import statistics

    import torch

    from oracle import forward as ofwd
    from oracle import weights

    host = _host_cpu()
    threads = host["cores_usable"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    threads = int(os.environ.get("SHRIMP_CPU_THREADS", "0")) or max(1, threads)
    torch.set_num_threads(threads)
    sd = weights.make_state_dict(C, H, LAYOUT, seed=0, mode="fresh")
    args = [batch[k][:sample] for k in ("feats", "nbr", "mask", "coords")]
    n = int(args[0].shape[0])
    for _ in range(warmup):
        ofwd.forward_policy_value(sd, LAYOUT, H, *args, dtype=torch.float32)
    times = []
    while len(times) < runs or sum(times) < seconds:
        t0 = time.perf_counter()
        ofwd.forward_policy_value(sd, LAYOUT, H, *args, dtype=torch.float32)
        times.append(time.perf_counter() - t0)
        if len(times) >= 4 * runs:
            break
    med = statistics.median(times)
    return {
        "value": round(n / med, 3),
        "unit": "positions/s",
        "cores": threads,
        "kind": "port",
        "sample": f"median of {len(times)} forwards of {n} cfg4 positions after {warmup} warm-ups "
                  f"(fp32 eager oracle: torch pair rows, fp16 bias, sdpa; "
                  f"{min(times):.2f}-{max(times):.2f} s per forward, torch threads {threads})",
        "cpu_model": host["model"],
        "cpu_vendor_family_model": f"{host['vendor']} family {host['family']} model {host['model_id']}",
        "cpu_avx512f": host["flags_avx512f"],
        "sockets": host["sockets"],
        "cores_per_socket": host["cores_per_socket"],
        "threads_per_core": host["threads_per_core"],
        "cores_visible": host["cores_visible"],
        "cores_usable": host["cores_usable"],
    }


def forward_flops(N: int, c: int = C, layout: str = LAYOUT, features: int = 15) -> float:
    """Padded-dense FLOPs of one position's forward at Npad = N (S = N + 8):
    per ConvBlock two 7-tap convs (2 * 2 * 7 * C^2 * N); per attention block
    q/k/v (6 C^2 S), QK^T and PV over all heads (4 S^2 C), out_proj
    (2 C^2 S) and the MLP (8 C^2 S); the stem (2 * 7 * features * C * N) and
    the policy conv (2 * 7 * C^2 * N). 1.425 GFLOP at N = 256, C = 128."""

    s = N + 8
    f = layout.count("C") * 28.0 * c * c * N
    f += layout.count("A") * (16.0 * c * c * s + 4.0 * s * s * c)
    return f + 14.0 * c * c * N + 14.0 * features * c * N


def spec_timing(net, reps: int = 10) -> dict:
    """The spec-faithful positions (all 10-80 stones, supports of 280-544
    cells: shrimp.synthetic "cfg4_spec", 512 positions) on the same network,
    inputs device-resident: (a) the whole batch padded to one Npad
    (ceil64 of its largest support: 576) in one forward; (b) the batch as
    the evaluator serves it: rows sorted by size and cut by plan_groups
    (padding to the 64-quantized anchor, the reference's pair ceiling and
    waste fraction), one forward per group, the groups spread over three
    streams as ShrimpEvaluator does (assign_group_streams); (c) the same
    groups one after another on one stream. positions/s over the 512, HIP
    events on the launch stream (which waits for the side streams), and the
    padded-dense TFLOP/s."""

    import torch

    from shrimp import synthetic
    from shrimp.batching import collate_rows
    from shrimp.inference import assign_group_streams, plan_groups

    dev = torch.device("cuda")
    stream = torch.cuda.current_stream(dev)
    batch = synthetic.position_batch("cfg4_spec", B)
    rows = batch["rows"]
    npad = int(batch["mask"].shape[1])
    sizes = sorted((s.num_nodes for _, s, _ in rows), reverse=True)

    def dev_inputs(b):
        return (b["feats"].to(dev, torch.float16), b["nbr"].to(dev, torch.int32),
                b["mask"].to(dev), b["coords"].to(dev, torch.int32))

    one = dev_inputs(batch)
    order = sorted(range(len(rows)), key=lambda i: -rows[i][1].num_nodes)
    groups = []
    for g0, g1, pad in plan_groups(sizes):
        sel = [rows[order[i]] for i in range(g0, g1)]
        groups.append((pad, g1 - g0, dev_inputs(collate_rows([(s, f) for _, s, f in sel], pad_to=pad))))
    run_one = lambda: net.forward_policy_value(*one)
    run_seq = lambda: [net.forward_policy_value(*g[2]) for g in groups]
    side = [torch.cuda.Stream(dev) for _ in range(3)]
    slots = assign_group_streams([n * (pad + 8) ** 2 for pad, n, _ in groups], len(side))

    def run_groups():
        for s in side:
            s.wait_stream(stream)
        outs = []
        for (pad, n, inp), k in zip(groups, slots):
            with torch.cuda.stream(side[k]):
                outs.append(net.forward_policy_value(*inp))
        for s in side:
            stream.wait_stream(s)
        return outs

    res = {"workload": f"B={B} cfg4_spec positions, supports {min(sizes)}-{max(sizes)} cells",
           "generator": "spec seed 20261205"}
    gflops = sum(n * forward_flops(pad) for pad, n, _ in groups)
    for name, fn, flops in (
        ("one_batch", run_one, B * forward_flops(npad)),
        ("grouped", run_groups, gflops),
        ("grouped_one_stream", run_seq, gflops),
    ):
        for _ in range(3):
            fn()
        torch.cuda.synchronize(dev)
        ms = _events_time(fn, reps, stream)
        res[name] = {"ms_per_512": round(ms, 4), "positions_per_s": round(B / (ms * 1e-3), 1),
                     "tflops_padded": round(flops / (ms * 1e-3) / 1e12, 2),
                     "bf16_mfma_frac_padded": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    res["one_batch"]["npad"] = npad
    res["grouped"]["groups"] = [{"npad": pad, "positions": n, "stream": k}
                                for (pad, n, _), k in zip(groups, slots)]
    return res


def forward_timeline(net, inputs, reps: int = 10) -> dict:
    """Per-kernel times inside real forwards: HIP events recorded on the
    launch stream after every launch of `reps` eager forwards; average per
    launch and total per forward for each kernel kind."""

    import torch

    rt = net.hip_runtime()
    rt.timeline = []
    try:
        for _ in range(reps):
            net.forward_policy_value(*inputs)
        torch.cuda.synchronize()
        marks = rt.timeline
    finally:
        rt.timeline = None
    per: dict = {}
    for (_, e0), (name, e1) in zip(marks, marks[1:]):
        if name == "start":
            continue
        per.setdefault(name, []).append(e0.elapsed_time(e1))
    return {name: {"launches_per_forward": len(v) // reps,
                   "avg_ms": round(sum(v) / len(v), 5),
                   "ms_per_forward": round(sum(v) / reps, 5)} for name, v in per.items()}


def _device_gather_index(batch, dev):
    """(B, N, 7) gather index and (B, N) mask bytes of a position batch, built by
    the product's input-preparation kernel (shrimp_prep_inputs) from the batch's
    neighbour rows, as the forward builds them."""

    import torch

    from shrimp import _lib
    from shrimp.constants import NUM_TOKENS

    lib = _lib.load()
    feats = batch["feats"].to(dev, torch.float16).contiguous()
    nbr = batch["nbr"].to(dev, torch.int32).contiguous()
    mask = batch["mask"].to(dev, torch.bool).contiguous()
    coords = batch["coords"].to(dev, torch.int32).contiguous()
    b, n, f = feats.shape
    i32, u8 = torch.int32, torch.uint8
    idx = torch.empty((b, n, 7), dtype=i32, device=dev)
    m8 = torch.empty((b, n), dtype=u8, device=dev)
    coords32 = torch.empty((b, n, 2), dtype=i32, device=dev)
    seq_lens = torch.empty((b,), dtype=i32, device=dev)
    seq_mask = torch.empty((b, n + NUM_TOKENS), dtype=u8, device=dev)
    xin = torch.empty((b, n, 32), dtype=torch.bfloat16, device=dev)
    _lib.check(
        lib.shrimp_prep_inputs(
            nbr.data_ptr(), _lib.DT_I32, mask.data_ptr(), coords.data_ptr(), _lib.DT_I32,
            feats.data_ptr(), _lib.DT_F16, f, b, n, NUM_TOKENS, idx.data_ptr(), m8.data_ptr(),
            coords32.data_ptr(), seq_lens.data_ptr(), seq_mask.data_ptr(), _lib.ptr(xin),
            _lib.stream_handle(dev),
        ),
        "prep_inputs",
    )
    return idx, m8


def ops_timing(reps: int = 30) -> dict:
    """Configs 1-3 as standalone ops at their own shapes (B = 1024, Npad = 256),
    HIP events around back-to-back launches on the launch stream:

    cfg1  7-tap gather-GEMM 128 -> 128 with the fused bias + ReLU + mask
          epilogue; work 2*7*C*C per row over all B*N rows (60.13 GFLOP),
          bytes (Cin + Cout)*2 + 7*4 per row + weights (141.8 MB);
    cfg2  rel-biased masked attention, H = 8, d = 16, lengths U[64, 256], the
          33x33 per-head offset table, no tokens; work 4*d*H*sum n_b^2, bytes
          8*d*H*sum n_b (Q, K, V in, O out) + coordinates + table; timed as
          the key table plus the staged kernel over the K / V rows, with the
          row-layout kernel (shrimp_attn) beside it;
    cfg3  31 independent tap weights over the 32-slot ray index (built on
          the device), 128 -> 128; work 2*31*C*C per row (266.3 GFLOP), bytes
          2*C*2 + 32*4 per row + weights."""

    import math

    import torch

    from shrimp import _lib, ops, synthetic

    dev = torch.device("cuda")
    stream = torch.cuda.current_stream(dev)
    lib = _lib.load()
    res = {}

    # cfg1
    case = synthetic.conv_inputs(1024, channels=128)
    b = case["batch"]
    bb, n = b["mask"].shape
    x = torch.from_numpy(case["x"]).to(dev, torch.bfloat16).contiguous()
    wp = ops.pack_conv_weight(torch.from_numpy(case["w"]).to(dev))
    bias = torch.from_numpy(case["bias"]).to(dev)
    idx, m8 = _device_gather_index(b, dev)
    out = torch.empty((bb, n, 128), dtype=torch.bfloat16, device=dev)
    run = lambda: ops.launch_conv(x=x, x_sb=n * 128, x_sn=128, idx=idx, taps=7, idx_stride=7,
                                  mask8=m8, wpack=wp, bias=bias, B=bb, N=n, cin_pad=128, cout=128,
                                  relu=True, out=out, o_sb=n * 128, o_sn=128)
    run()
    ms = _events_time(run, reps, stream)
    rows = bb * n
    valid = int(b["mask"].sum().item())
    flops = 2.0 * 7 * 128 * 128 * rows
    nbytes = rows * (256 * 2 + 7 * 4) + 7 * 128 * 128 * 2 + 4 * 128
    tfl = flops / (ms * 1e-3) / 1e12
    res["cfg1"] = {
        "op": "hex_conv bias+ReLU (7 taps, 128 -> 128)", "workload": f"B={bb} Npad={n}",
        "launch_ms": round(ms, 5), "flops": flops, "flops_valid_rows": 2.0 * 7 * 128 * 128 * valid,
        "algorithmic_bytes": nbytes, "bound": "mfma", "achieved_tflops": round(tfl, 2),
        "peak_tflops": PEAK_BF16_TFLOPS, "frac": round(tfl / PEAK_BF16_TFLOPS, 4),
        "hbm_gbs_algorithmic": round(nbytes / (ms * 1e-3) / 1e9, 1),
    }
    del x, out

    # cfg2
    c2 = synthetic.attention_inputs(1024, heads=8, d=16)
    q, k, v = (torch.from_numpy(c2[nm]).to(dev, torch.bfloat16).contiguous() for nm in "qkv")
    B2, H2, S2, d2 = q.shape
    table = torch.from_numpy(c2["table"])
    btab = (torch.cat([table, torch.zeros(3, H2)]) * (1.0 / math.log(2.0))).to(dev).contiguous()
    xtab = cfg2_xtab(btab, 16)
    coords = torch.from_numpy(c2["coords"]).to(dev, torch.int32).contiguous()
    mask2 = torch.from_numpy(c2["mask"]).to(dev, torch.uint8).contiguous()
    lens = torch.from_numpy(c2["lens"]).to(dev)
    o = torch.empty((B2, H2, S2, d2), dtype=torch.bfloat16, device=dev)
    rows = lambda: ops.launch_attn(q=q, k=k, v=v, qkv_sb=H2 * S2 * d2, qkv_sh=S2 * d2, seq_lens=lens,
                                   o=o, o_sb=H2 * S2 * d2, o_sh=S2 * d2, o_sr=d2, B=B2, S=S2, H=H2,
                                   d=d2, dpad=16, coords=coords, mask8=mask2, btab=btab, xtab=xtab,
                                   lut_m=16, n_tokens=0)
    rows()
    ms_rows = _events_time(rows, reps, stream)
    # the op as served: the key table (attn_keys) and the staged kernel over the
    # K / V rows, both launches timed
    meta = torch.empty(B2 * ops.attn_keys_ints(S2), dtype=torch.int32, device=dev)

    def run():
        ops.launch_attn_keys(coords=coords, mask8=mask2, seq_lens=lens, B=B2, S=S2, n_tokens=0,
                             meta=meta)
        ops.launch_attn_staged(q=q, k=k, v=v, qkv_sb=H2 * S2 * d2, qkv_sh=S2 * d2, meta=meta,
                               seq_lens=lens, o=o, o_sb=H2 * S2 * d2, o_sh=S2 * d2, o_sr=d2, B=B2,
                               S=S2, H=H2, d=d2, dpad=16, btab=btab, xtab=xtab, lut_m=16, n_tokens=0)

    run()
    ms = _events_time(run, reps, stream)
    nb = c2["lens"].astype("float64")
    flops = float(4 * d2 * H2 * (nb ** 2).sum())
    nbytes = float(8 * d2 * H2 * nb.sum() + nb.sum() * (2 * 4 + 1) + btab.numel() * 4)
    tfl = flops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    res["cfg2"] = {
        "op": "attention, coords bias (33x33 table), key mask", "workload":
            f"B={B2} H={H2} L={S2} d={d2} lengths U[64,256] (sum {int(nb.sum())})",
        "launch_ms": round(ms, 5), "flops": flops, "algorithmic_bytes": nbytes, "bound": "hbm",
        "achieved_gbs": round(gbs, 1), "peak_gbs": PEAK_HBM_GBS, "frac": round(gbs / PEAK_HBM_GBS, 4),
        "tflops": round(tfl, 2), "mfma_frac": round(tfl / PEAK_BF16_TFLOPS, 4),
        "path": "attn_keys + attn_staged over the K / V rows",
        "row_layout_launch_ms": round(ms_rows, 5),
    }
    del q, k, v, o

    # cfg3
    c3 = synthetic.raytap_inputs(1024, channels=128)
    b3 = c3["batch"]
    B3, n3 = b3["mask"].shape
    x3 = torch.from_numpy(c3["x"]).to(dev, torch.bfloat16).contiguous()
    wp3 = ops.pack_conv_weight(torch.from_numpy(c3["w"]).to(dev))
    bias3 = torch.from_numpy(c3["bias"]).to(dev)
    c32 = b3["coords"].to(dev, torch.int32).contiguous()
    m83 = b3["mask"].to(dev, torch.uint8).contiguous()
    ridx = torch.empty((B3, n3, 32), dtype=torch.int32, device=dev)
    _lib.check(lib.shrimp_build_ray_index(c32.data_ptr(), m83.data_ptr(), B3, n3, ridx.data_ptr(),
                                          _lib.stream_handle(dev)), "ray index")
    out3 = torch.empty((B3, n3, 128), dtype=torch.bfloat16, device=dev)
    run = lambda: ops.launch_conv(x=x3, x_sb=n3 * 128, x_sn=128, idx=ridx, taps=31, idx_stride=32,
                                  mask8=m83, wpack=wp3, bias=bias3, B=B3, N=n3, cin_pad=128,
                                  cout=128, out=out3, o_sb=n3 * 128, o_sn=128)
    run()
    ms = _events_time(run, reps, stream)
    rows = B3 * n3
    flops = 2.0 * 31 * 128 * 128 * rows
    nbytes = rows * (2 * 128 * 2 + 32 * 4) + 31 * 128 * 128 * 2
    tfl = flops / (ms * 1e-3) / 1e12
    res["cfg3"] = {
        "op": "31-tap ray conv (independent tap weights, 128 -> 128)", "workload": f"B={B3} Npad={n3}",
        "launch_ms": round(ms, 5), "flops": flops, "algorithmic_bytes": nbytes, "bound": "mfma",
        "achieved_tflops": round(tfl, 2), "peak_tflops": PEAK_BF16_TFLOPS,
        "frac": round(tfl / PEAK_BF16_TFLOPS, 4),
        "hbm_gbs_algorithmic": round(nbytes / (ms * 1e-3) / 1e9, 1),
    }
    return res


def cfg2_xtab(btab, m: int):
    """The attention kernel's unclamped offset table for a (2m+1)^2 per-offset
    table: fp16(btab[clamped (dq, dr), h]) at offset x = (dq + XD)(2 XD + 1) +
    dr + XD over |dq|, |dr| <= XD, in the head pair major layout (what
    shrimp_attn_bias_table writes for the model's LUT), so compact cell sets
    take the kernel's linear-offset path."""

    import torch

    from shrimp.ops import ATTN_XD, xtab_pairs

    r = torch.arange(-ATTN_XD, ATTN_XD + 1, device=btab.device)
    dq, dr = torch.meshgrid(r, r, indexing="ij")
    pos = (dq.clamp(-m, m) + m) * (2 * m + 1) + dr.clamp(-m, m) + m
    return xtab_pairs(btab[pos.reshape(-1)].half())


def fp32_timing(net, inputs, steps: int = 10) -> dict:
    """Secondary figure: the config 4 forward in the fp32 serve mode (fp32
    activations; the GEMMs and attention as three bf16 MFMA products of hi / lo
    split operands, the 16-channel stem on fp32 MFMA), same inputs and
    weights. tflops_padded counts each product once (the fp32 forward's
    padded FLOPs); the bf16 MFMA work is three times that."""

    import torch

    rt = net.hip_runtime()
    prev = rt.precision
    rt.precision = "fp32"
    try:
        net.forward_policy_value(*inputs)
        torch.cuda.synchronize()
        ms = _events_time(lambda: net.forward_policy_value(*inputs), steps,
                          torch.cuda.current_stream())
        tl = forward_timeline(net, inputs, reps=3)
    finally:
        rt.precision = prev
    return {
        "workload": "shrimp_forward_policy_value_cfg4 (fp32 serve mode)",
        "dtype": "fp32",
        "positions_per_s": round(B / (ms * 1e-3), 1),
        "ms_per_step": round(ms, 4),
        "tflops_padded": round(1.425e9 * B / (ms * 1e-3) / 1e12, 2),
        "mfma": "bf16, three products per fp32 product (hi·lo + lo·hi + hi·hi)",
        "bf16_mfma_frac": round(3 * 1.425e9 * B / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "in_forward": tl,
    }


def _phase_stats(starts, ends, nbytes, resident):
    """One phase over all workgroups: start and end stamps (10 ns ticks) and the
    phase's algorithmic HBM bytes per workgroup. gbs_over_span: every
    workgroup's bytes over the span (first start to last end), a lower bound on
    what the chip moved while the phase ran; gbs_resident: `resident`
    workgroups (as many as the chip holds at once) each moving its bytes in the
    mean per-workgroup duration, the rate while all resident workgroups are in
    the phase together."""

    import numpy as np

    d = (ends - starts).astype(np.float64) * 1e-2  # us
    span = float(ends.max() - starts.min()) * 1e-2
    total = float(nbytes) * len(starts)
    r = {
        "workgroups": int(len(starts)),
        "mean_us": round(float(d.mean()), 2),
        "median_us": round(float(np.median(d)), 2),
        "max_us": round(float(d.max()), 2),
        "span_us": round(span, 2),
        "bytes_per_workgroup": int(nbytes),
    }
    if nbytes:
        r["gbs_over_span"] = round(total / (span * 1e-6) / 1e9, 1)
        r["resident_workgroups"] = int(min(resident, len(starts)))
        r["gbs_resident"] = round(min(resident, len(starts)) * float(nbytes) / (float(d.mean()) * 1e-6) / 1e9, 1)
    return r


def _clock_stats(stamps, s, e, mfma_cycles=0):
    """Core clock of a phase between workgroup stamps s and e, from a run that
    stored the core clock counter at slot + 8 beside each: cycles over 10 ns
    ticks summed over the workgroups, and, for a phase with mfma_cycles of MFMA
    issue per wave, the MFMA pipe's busy share at that clock."""

    import numpy as np

    ticks = (stamps[:, e] - stamps[:, s]).astype(np.float64)
    cyc = (stamps[:, e + 8] - stamps[:, s + 8]).astype(np.float64)
    r = {"core_clock_ghz": round(float(cyc.sum() / (ticks.sum() * 10.0)), 3)}
    if mfma_cycles:
        r["mfma_busy_at_clock"] = round(float(mfma_cycles / cyc.mean()), 3)
    return r


def phase_report(net, inputs, dev) -> dict:
    """Phase timings and per-phase HBM rates of three kernels, from the phase
    build (libshrimp_hip_phase.so, SHRIMP_PHASE_CLOCK=1: the kernels store the
    100 MHz constant clock at their phase boundaries; the release build has no
    such code):

    - hex_block_pair_kernel, the fourth pair launch of one cfg4 forward (B=512,
      Npad 256, 2 waves per workgroup): gather (rows and indices staged into
      LDS: 256 rows x 256 B + 7 indices x 4 B per row), the four convs (no HBM
      beyond L2-resident weights), the LDS-only epilogue 1 of each block, and
      the two residual epilogues (256 rows x 256 B read + 256 B stored each);
    - hex_conv_big_kernel<bias+ReLU>, the cfg1 op (B=1024, Npad 256): gather,
      conv, epilogue (256 B stored per row);
    - the staged attention kernel, the fourth attention launch of the same
      forward (2048 workgroups of one position and two heads): staging (the
      pair's K/V fragments, 2 x 2 x SP x 32 B, and a quarter of the position's
      key table, which its four workgroups share), then the query blocks (q
      fragments in, outputs stored: 2 x 2 x S x 16 x 2 B). The staging rate is
      given for the first generation of resident workgroups (those starting
      within 2 us of the first), which stage together.
    Rates: over each phase's span, and for the workgroups the chip holds at
    once (two per CU for the conv kernels, three for the attention) each moving
    its bytes in the mean per-workgroup duration. The stamps (a clock read and
    a wait for it) slow the kernels by 5-15 %; compare the launch spans with
    the release kernels' launch times. Timings and rates come from a run with
    the constant clock only; the core clock columns (core_clock_ghz, and the
    MFMA pipe's busy share in the conv phases) from a second run that also
    reads the core clock counter at each workgroup stamp."""

    import numpy as np
    import torch

    from shrimp import _lib, ops, synthetic

    release = _lib.load()
    phase = _lib.load(_lib.PHASE_LIB_PATH)
    nb, npad = inputs[2].shape
    case = synthetic.conv_inputs(1024, channels=128)
    b1 = case["batch"]
    bb, n = b1["mask"].shape
    x = torch.from_numpy(case["x"]).to(dev, torch.bfloat16).contiguous()
    wp = ops.pack_conv_weight(torch.from_numpy(case["w"]).to(dev))
    bias = torch.from_numpy(case["bias"]).to(dev)
    gi, m8 = _device_gather_index(b1, dev)
    out = torch.empty((bb, n, 128), dtype=torch.bfloat16, device=dev)
    conv_st = torch.zeros(1 << 20, dtype=torch.int64, device=dev)
    attn_st = torch.zeros(1 << 20, dtype=torch.int64, device=dev)

    def collect(clock):
        """Stamps of the fourth pair launch, the fourth attention launch and the
        cfg1 op; clock adds the core clock counter to the workgroup stamps."""
        conv_st.zero_()
        attn_st.zero_()
        _lib.check(phase.shrimp_phase_clock(conv_st.data_ptr(), 0 | (4 if clock else 0)), "phase_clock")
        _lib.check(phase.shrimp_phase_clock(attn_st.data_ptr(), 1 | (4 if clock else 0)), "phase_clock")
        for _ in range(5):
            net.forward_policy_value(*inputs)
        torch.cuda.synchronize(dev)
        c = conv_st[: nb * 32].view(nb, 32).cpu().numpy()
        hb = attn_st[: nb * 4 * 32].view(nb * 4, 32).cpu().numpy()
        conv_st.zero_()
        for _ in range(3):
            ops.launch_conv(x=x, x_sb=n * 128, x_sn=128, idx=gi, taps=7, idx_stride=7, mask8=m8,
                            wpack=wp, bias=bias, B=bb, N=n, cin_pad=128, cout=128, relu=True,
                            out=out, o_sb=n * 128, o_sn=128)
        torch.cuda.synchronize(dev)
        c1 = conv_st[: bb * 32].view(bb, 32).cpu().numpy()
        _lib.check(phase.shrimp_phase_clock(None, 0), "phase_clock")
        _lib.check(phase.shrimp_phase_clock(None, 1), "phase_clock")
        return c, hb, c1

    _lib._LIB = phase
    rt = net.hip_runtime()
    rt.invalidate()
    try:
        c, hb, c1 = collect(False)
        kc, khb, kc1 = collect(True)
    finally:
        _lib._LIB = release
        rt.invalidate()

    res = {}
    S = npad + 8
    SP = (S + 15) // 16 * 16
    row, idx = 256, 7 * 4
    waves = (npad + 127) // 128
    w_epi4 = c[:, 16:16 + waves].min(1)
    w_end = c[:, 24:24 + waves].max(1)
    bounds = [("gather", 0, 1, npad * (row + idx)), ("conv1", 1, 2, 0), ("epilogue1", 2, 3, 0),
              ("conv2", 3, 4, 0), ("epilogue2", 4, 5, 2 * npad * row), ("conv3", 5, 6, 0),
              ("epilogue3", 6, 7, 0)]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    conv_mfma = 7 * 4 * 64 * 16  # MFMA issue cycles of one 7-tap conv per wave
    pair = {}
    for name, s, e, by in bounds:
        pair[name] = _phase_stats(c[:, s], c[:, e], by, 2 * cus)
        pair[name].update(_clock_stats(kc, s, e, conv_mfma if name.startswith("conv") else 0))
    pair["conv4"] = _phase_stats(c[:, 7], w_epi4, 0, 2 * cus)
    pair["epilogue4"] = _phase_stats(w_epi4, w_end, 2 * npad * row, 2 * cus)
    pair["launch_span_us"] = round(float(w_end.max() - c[:, 0].min()) * 1e-2, 2)
    res["hex_block_pair_kernel"] = pair

    nw = 8 if hb[:, 16 + 4:24].max() > 0 else 4
    a_end = hb[:, 16:16 + nw].max(1)
    mbytes = int(release.shrimp_attn_keys_bytes(S))
    stage_b = 2 * 2 * SP * 32 + mbytes // 4
    first = hb[:, 0] < hb[:, 0].min() + 200
    kfirst = khb[:, 0] < khb[:, 0].min() + 200
    att = {
        "staging_first_generation": _phase_stats(hb[first, 0], hb[first, 1], stage_b, 3 * cus),
        "staging_all": _phase_stats(hb[:, 0], hb[:, 1], stage_b, 3 * cus),
        "query_blocks": _phase_stats(hb[:, 1], a_end, 2 * 2 * S * 16 * 2, 3 * cus),
        "launch_span_us": round(float(a_end.max() - hb[:, 0].min()) * 1e-2, 2),
        "waves_per_workgroup": nw,
    }
    att["staging_first_generation"].update(_clock_stats(khb[kfirst], 0, 1))
    att["staging_all"].update(_clock_stats(khb, 0, 1))
    res["attn_kernel_staged"] = att

    wv = (n + 127) // 128
    e0, e1 = c1[:, 16:16 + wv].min(1), c1[:, 24:24 + wv].max(1)
    res["hex_conv_big_kernel_cfg1"] = {
        "gather": {**_phase_stats(c1[:, 0], c1[:, 1], n * (row + idx), 2 * cus), **_clock_stats(kc1, 0, 1)},
        "conv": _phase_stats(c1[:, 1], e0, 0, 2 * cus),
        "epilogue": _phase_stats(e0, e1, n * row, 2 * cus),
        "launch_span_us": round(float(e1.max() - c1[:, 0].min()) * 1e-2, 2),
    }
    return res


def _block_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    FETCH_SIZE / WRITE_SIZE passes (profiles/block_traffic.json), used only when
    they were taken on this build's kernel source: the file records the sha256
    of hex_conv.hip it was measured on, and a different source gives
    (None, reason) instead of a stale figure."""

    import hashlib

    tfile = ROOT / "profiles" / "block_traffic.json"
    src = ROOT / "hexo-bot_amd" / "csrc" / "hex_conv.hip"
    if not tfile.exists():
        return None, "no counter passes recorded"
    rec = json.loads(tfile.read_text())
    sha = hashlib.sha256(src.read_bytes()).hexdigest()
    if rec.get("kernel_source_sha256") != sha:
        return None, "counter passes were taken on another hex_conv.hip; not measured for this build"
    return rec.get("bytes_per_launch"), f"{rec.get('source')} (hex_conv.hip sha256 {sha[:12]})"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # defaults: 30 untimed forwards (the clock settles over the first ~15 of a
    # run), then 100 timed ones (about 0.13 s)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--spec-only", action="store_true",
                    help="only time the spec-faithful positions (spec_timing) and print that")
    ap.add_argument("--phases", action="store_true",
                    help="only print the phase build's per-phase timings and HBM rates "
                         "(phase_report) and exit")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run 5 plain device copies of this many MiB (the "
                         "calibration kernel for HBM traffic counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one MI355X: the Shrimp forward shards by position with no "
            "collective, and this build runs single-GPU only (--gpus 1).",
            file=sys.stderr,
        )
        return 2

    import torch

    from shrimp import _lib, synthetic
    from shrimp.model import ShrimpNet

    dev = torch.device("cuda:0")
    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        print(json.dumps({"copy_probe_bytes": n, "reps": 5}), flush=True)
        return 0
    _lib.load()
    torch.manual_seed(0)
    net = ShrimpNet(channels=C, attention_heads=H, trunk_layout=LAYOUT).to(dev).eval()
    if args.spec_only:
        print(json.dumps({"spec": spec_timing(net, reps=args.steps)}), flush=True)
        return 0
    batch = synthetic.position_batch("cfg4", B)
    inputs = (
        batch["feats"].to(dev, torch.float16),
        batch["nbr"].to(dev, torch.int32),
        batch["mask"].to(dev),
        batch["coords"].to(dev, torch.int32),
    )
    if args.phases:
        print(json.dumps({"phases": phase_report(net, inputs, dev)}), flush=True)
        return 0
    for _ in range(args.warmup):
        net.forward_policy_value(*inputs)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    t0 = time.perf_counter()
    ms = _events_time(lambda: net.forward_policy_value(*inputs), args.steps, stream)
    torch.cuda.synchronize(dev)
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kt = kernel_timings(net, inputs)
    timeline = forward_timeline(net, inputs)

    block_tflops = kt["block_flops"] / (kt["block_ms"] * 1e-3) / 1e12
    pair_tflops = kt["pair_flops"] / (kt["pair_ms"] * 1e-3) / 1e12
    tl_pair = timeline.get("conv_block_pair", {}).get("avg_ms")
    conv_tflops = kt["conv_flops"] / (kt["conv_ms"] * 1e-3) / 1e12
    fused = kt["forward_attn_fused"]
    a_ms = kt["attn_fused_ms"] if fused else kt["attn_ms"]
    a_flops = kt["attn_flops"] + (kt["proj_flops"] if fused else 0.0)
    a_bytes = kt["proj_bytes"] if fused else kt["attn_bytes"]
    attn_tflops = a_flops / (a_ms * 1e-3) / 1e12
    traffic, traffic_source = _block_traffic()
    line = {
        "metric": METRIC,
        "value": round(B / (ms * 1e-3), 1),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "wall_ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "shrimp_forward_policy_value_cfg4",
            "positions": B, "npad": NPAD, "seq_len": NPAD + 8, "channels": C, "heads": H,
            "trunk": LAYOUT, "support_radius": 4, "generator": "l256 seed 20261205",
        },
        "roofline": {
            "kernel": "hex_block_pair_kernel (ConvBlocks 0 and 1 in one launch, each conv1 + LN + "
                      "ReLU, conv2 + LN + LayerScale residual + ReLU; B=512 x 256 rows)",
            "bound": "mfma",
            "achieved": round(pair_tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(pair_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes": kt["pair_bytes"],
            "launch_ms": round(kt["pair_ms"], 5),
            "flops_per_launch": kt["pair_flops"],
            "in_forward_launch_ms": tl_pair,
            "in_forward_frac": (round(kt["pair_flops"] / (tl_pair * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
                                if tl_pair else None),
        },
        "single_block": {
            "kernel": "hex_block_kernel (ConvBlock 0 alone, the launch a lone 'C' takes)",
            "launch_ms": round(kt["block_ms"], 5),
            "tflops": round(block_tflops, 2),
            "mfma_frac": round(block_tflops / PEAK_BF16_TFLOPS, 4),
            "algorithmic_bytes": kt["block_bytes"],
        },
        "single_conv": {
            "kernel": "hex_conv_big_kernel<LN|RELU> (ConvBlock 0 conv1 alone)",
            "launch_ms": round(kt["conv_ms"], 5),
            "tflops": round(conv_tflops, 2),
            "mfma_frac": round(conv_tflops / PEAK_BF16_TFLOPS, 4),
        },
        "attention": {
            "kernel": ("attn_kernel<16,2,coords,proj> (block 0: LN1 + q/k/v projection + "
                       "attention)") if fused else (
                           "attn_kernel<16,2,coords,staged> (block 0: K/V fragments and the key "
                           "table by DMA)" if kt["attn_staged"] else "attn_kernel<16,2,coords> (block 0)"),
            "bound": "valu (d=16: one exp + ~4 VALU per score vs 64 MFMA flops)",
            "launch_ms": round(a_ms, 5),
            "tflops": round(attn_tflops, 2),
            "mfma_frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
            "hbm_gbs_algorithmic": round(a_bytes / (a_ms * 1e-3) / 1e9, 1),
            "two_launch_ms": {"qkv": kt["linears"]["qkv"]["ms"],
                              "attn": round(kt["attn_ms"], 5)},
            "one_launch_ms": None if kt["attn_fused_ms"] is None else round(kt["attn_fused_ms"], 5),
        },
        "block0_row_kernels": kt["linears"],
        "in_forward": timeline,
        "ops": ops_timing(),
        "fp32": fp32_timing(net, inputs),
        "forward_tflops_padded": round(forward_flops(NPAD) * B / (ms * 1e-3) / 1e12, 2),
        "spec": spec_timing(net),
        "featurize": featurize_timing(batch["rows"]),
        "hexfield": hexfield_timing(),
        "evaluator": evaluator_timing(net),
        "evaluator_graphs": evaluator_timing(net, graphs=True),
        "evaluator_small": [evaluator_timing(net, 32, g, reps=20) for g in (False, True)],
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(batch, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
