"""Launch helpers over the C ABI and the reference's operator names.

``shrimp::hex_conv``, ``shrimp::hex_conv_ln`` and ``shrimp::attn_pair`` are
registered with the signatures of the reference's serve ops
(``packages/shrimp/python/shrimp/_triton_conv.py:93-128,198-239``,
``_triton_attn.py:132-171``), each with a fake kernel, so code written against
the reference can call ``torch.ops.shrimp.*`` unchanged. They run the gfx950
kernels of ``libshrimp_hip.so`` and return bfloat16 (the reference returns
float16; MI355X computes these paths in bf16). Inputs must live on a ROCm
device; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .constants import (
    BIAS_CELL_TOKEN_ROW,
    BIAS_TOKEN_CELL_ROW,
    BIAS_TOKEN_TOKEN_ROW,
    NUM_TOKENS,
)
from .geometry import CELL_LUT_M


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{what}: the shrimp MI355X build runs on a ROCm device only "
            f"(got a {t.device} tensor)"
        )


def cin_pad_of(c: int) -> int:
    return -(-int(c) // 32) * 32


# ---- weight packing ------------------------------------------------------------------


def pack_conv_weight(weight: torch.Tensor, cin_pad: int | None = None) -> torch.Tensor:
    """(T, cin, cout) conv weight -> packed bf16 MFMA fragments (uint8 bytes)."""

    require_device(weight, "pack_conv_weight")
    t, cin, cout = weight.shape
    cp = cin_pad_of(cin) if cin_pad is None else int(cin_pad)
    lib = _lib.load()
    w32 = weight.detach().to(torch.float32).contiguous()
    out = torch.empty(lib.shrimp_conv_wpack_bytes(t, cp, cout), dtype=torch.uint8, device=weight.device)
    _lib.check(
        lib.shrimp_pack_conv_weight(w32.data_ptr(), out.data_ptr(), t, cin, cp, cout,
                                    _lib.stream_handle(weight.device)),
        "pack_conv_weight",
    )
    return out


def pack_linear_weight(weight: torch.Tensor) -> torch.Tensor:
    """nn.Linear weight (out, in) -> packed bf16 MFMA fragments (uint8 bytes)."""

    require_device(weight, "pack_linear_weight")
    n_out, n_in = weight.shape
    lib = _lib.load()
    w32 = weight.detach().to(torch.float32).contiguous()
    out = torch.empty(lib.shrimp_linear_wpack_bytes(n_in, n_out), dtype=torch.uint8, device=weight.device)
    _lib.check(
        lib.shrimp_pack_linear_weight(w32.data_ptr(), out.data_ptr(), n_in, n_out,
                                      _lib.stream_handle(weight.device)),
        "pack_linear_weight",
    )
    return out


def pack_attn_qkv(qkv_w, qkv_b, ln_w, ln_b):
    """(3C, C) q/k/v weights + biases and LN1's affine -> the fused QKV
    kernel's packed weights, or None when C has no fused kernel."""

    require_device(qkv_w, "pack_attn_qkv")
    c = int(qkv_w.shape[1])
    lib = _lib.load()
    nbytes = lib.shrimp_attn_qkv_pack_bytes(c)
    if nbytes == 0:
        return None
    dev = qkv_w.device
    ts = [t.detach().to(device=dev, dtype=torch.float32).contiguous()
          for t in (qkv_w, qkv_b, ln_w, ln_b)]
    packed = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    scratch = torch.empty(3 * c * c, dtype=torch.float32, device=dev)
    _lib.check(lib.shrimp_pack_attn_qkv(*[t.data_ptr() for t in ts], packed.data_ptr(),
                                        scratch.data_ptr(), c, _lib.stream_handle(dev)),
               "pack_attn_qkv")
    torch.cuda.current_stream(dev).synchronize()
    return packed


def pack_attn_mlp(out_w, out_b, g_attn, ln_w, ln_b, fc1_w, fc1_b, fc2_w, fc2_b, g_mlp):
    """AttnBlock out_proj / LN2 / fc1 / fc2 / LayerScale parameters -> the
    fused MLP kernel's packed weights (per-channel factors folded in), or
    None when the shape has no fused kernel (C != 128 or hidden != 2C)."""

    require_device(out_w, "pack_attn_mlp")
    c = int(out_w.shape[0])
    hidden = int(fc1_w.shape[0])
    lib = _lib.load()
    nbytes = lib.shrimp_attn_mlp_pack_bytes(c, hidden)
    if nbytes == 0:
        return None
    dev = out_w.device
    ts = [t.detach().to(device=dev, dtype=torch.float32).contiguous()
          for t in (out_w, out_b, g_attn, ln_w, ln_b, fc1_w, fc1_b, fc2_w, fc2_b, g_mlp)]
    w = _lib.MlpWeights(*[t.data_ptr() for t in ts], C=c, hidden=hidden)
    packed = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    scratch = torch.empty(c * hidden, dtype=torch.float32, device=dev)
    _lib.check(lib.shrimp_pack_attn_mlp(ctypes_ref(w), packed.data_ptr(), scratch.data_ptr(),
                                        _lib.stream_handle(dev)), "pack_attn_mlp")
    torch.cuda.current_stream(dev).synchronize()  # ts / scratch die with this frame
    return packed


ATTN_XD = 26  # SHRIMP_ATTN_XD of the C ABI
ATTN_XP = 2816  # SHRIMP_ATTN_XP: (2 XD + 1)^2 offsets per head pair, padded


def attn_bias_table(table: torch.Tensor, lut_u8: torch.Tensor, lut_m: int = CELL_LUT_M):
    """Per-block (BIAS_ROWS, H) table -> (btab, xtab): btab ((2M+1)^2 + 3, H)
    fp32, the LUT-indexed table with log2(e) folded in; xtab ((H + 1) // 2,
    ATTN_XP, 2) fp16, the same values indexed by unclamped offsets (|dq|, |dr|
    <= XD), head pair major (see xtab_pairs)."""

    require_device(table, "attn_bias_table")
    rows, h = table.shape
    w = 2 * lut_m + 1
    t32 = table.detach().to(torch.float32).contiguous()
    btab = torch.empty((w * w + 3, h), dtype=torch.float32, device=table.device)
    xtab = torch.empty(((h + 1) // 2, ATTN_XP, 2), dtype=torch.float16, device=table.device)
    _lib.check(
        _lib.load().shrimp_attn_bias_table(
            t32.data_ptr(), rows, h, lut_u8.data_ptr(), lut_m, BIAS_CELL_TOKEN_ROW,
            BIAS_TOKEN_CELL_ROW, BIAS_TOKEN_TOKEN_ROW, btab.data_ptr(), xtab.data_ptr(),
            _lib.stream_handle(table.device),
        ),
        "attn_bias_table",
    )
    return btab, xtab


def xtab_pairs(xh: torch.Tensor) -> torch.Tensor:
    """((2 XD + 1)^2, H) fp16 offset table -> the head pair major layout the
    kernels read, ((H + 1) // 2, ATTN_XP, 2): entry [p, x, j] is xh[x, 2 p + j],
    zeros for the padding offsets and the missing second head of an odd H."""

    n, h = xh.shape
    xw = 2 * ATTN_XD + 1
    if n != xw * xw:
        raise ValueError(f"xtab_pairs: {n} offsets, expected {xw * xw}")
    hp = (h + 1) // 2
    out = xh.new_zeros((ATTN_XP, 2 * hp))
    out[:n, :h] = xh
    return out.view(ATTN_XP, hp, 2).permute(1, 0, 2).contiguous()


# ---- raw launches ----------------------------------------------------------------------


def _check_rows(name, t, sb, sn, B, N, width):
    """Refuses a launch whose (position, row) strides or extent disagree with the
    tensor the pointer comes from: the kernels address rows by these strides."""

    if (t.dim() != 3 or t.stride(2) != 1 or t.stride(0) != sb or t.stride(1) != sn
            or t.shape[0] < B or t.shape[1] < N or t.shape[2] < width):
        raise ValueError(
            f"{name}: tensor {tuple(t.shape)} with strides {t.stride()} does not hold "
            f"(B={B}, N={N}, width={width}) rows at strides ({sb}, {sn})")


def launch_conv(
    *, x, x_sb, x_sn, idx, taps, idx_stride, mask8, wpack, bias, B, N, cin_pad, cout,
    ln_w=None, ln_b=None, eps=1e-5, relu=False, resid=None, r_sb=0, r_sn=0, gamma=None,
    head_w=None, head_b=None, head_out=None, out=None, o_sb=0, o_sn=0, stream=None,
):
    _check_rows("hex_conv x", x, x_sb, x_sn, B, N, cin_pad)
    if out is not None:
        _check_rows("hex_conv out", out, o_sb, o_sn, B, N, cout)
    if resid is not None:
        _check_rows("hex_conv resid", resid, r_sb, r_sn, B, N, cout)
    if head_out is not None and (not head_out.is_contiguous() or head_out.numel() < B * N):
        raise ValueError(f"hex_conv head_out: needs a contiguous (B={B}, N={N}) tensor")
    a = _lib.ConvArgs(
        x=x.data_ptr(), x_sb=x_sb, x_sn=x_sn, idx=idx.data_ptr(), taps=taps,
        idx_stride=idx_stride, mask=mask8.data_ptr(), w=wpack.data_ptr(), bias=bias.data_ptr(),
        ln_w=_lib.ptr(ln_w), ln_b=_lib.ptr(ln_b), eps=float(eps), relu=int(bool(relu)),
        resid=_lib.ptr(resid), r_sb=r_sb, r_sn=r_sn, gamma=_lib.ptr(gamma),
        head_w=_lib.ptr(head_w), head_b=_lib.ptr(head_b), head_out=_lib.ptr(head_out),
        out=_lib.ptr(out), o_sb=o_sb, o_sn=o_sn, B=B, N=N, cin_pad=cin_pad, cout=cout,
    )
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_hex_conv(ctypes_ref(a), s), "hex_conv")


def conv_block_supported(taps, N, cin_pad, cout):
    """True when shrimp_conv_block has a fused kernel for this ConvBlock shape."""
    return bool(_lib.load().shrimp_conv_block_supported(taps, N, cin_pad, cout))


def _block_args(x, x_sb, x_sn, idx, idx_stride, mask8, B, N, C, w1, b1, ln1_w, ln1_b, eps1,
                w2, b2, ln2_w, ln2_b, eps2, gamma, out, o_sb, o_sn):
    """shrimp_conv_args of one ConvBlock's two convs (shrimp_conv_block's contract)."""
    _check_rows("conv_block x", x, x_sb, x_sn, B, N, C)
    _check_rows("conv_block out", out, o_sb, o_sn, B, N, C)
    c1 = _lib.ConvArgs(
        x=x.data_ptr(), x_sb=x_sb, x_sn=x_sn, idx=idx.data_ptr(), taps=7, idx_stride=idx_stride,
        mask=mask8.data_ptr(), w=w1.data_ptr(), bias=b1.data_ptr(), ln_w=ln1_w.data_ptr(),
        ln_b=ln1_b.data_ptr(), eps=float(eps1), relu=1, B=B, N=N, cin_pad=C, cout=C,
    )
    c2 = _lib.ConvArgs(
        w=w2.data_ptr(), bias=b2.data_ptr(), ln_w=ln2_w.data_ptr(), ln_b=ln2_b.data_ptr(),
        eps=float(eps2), relu=0, resid=x.data_ptr(), r_sb=x_sb, r_sn=x_sn,
        gamma=gamma.data_ptr(), out=out.data_ptr(), o_sb=o_sb, o_sn=o_sn, B=B, N=N,
        cin_pad=C, cout=C,
    )
    return c1, c2


def launch_conv_block(
    *, x, x_sb, x_sn, idx, idx_stride, mask8, B, N, C, w1, b1, ln1_w, ln1_b, eps1,
    w2, b2, ln2_w, ln2_b, eps2, gamma, out, o_sb, o_sn, stream=None,
):
    """ConvBlock.forward (reference model.py:395-422) as one launch; y1 stays on chip.

    `out` may alias `x`. Raises when conv_block_supported() is false for the shape.
    """
    c1, c2 = _block_args(x, x_sb, x_sn, idx, idx_stride, mask8, B, N, C, w1, b1, ln1_w, ln1_b,
                         eps1, w2, b2, ln2_w, ln2_b, eps2, gamma, out, o_sb, o_sn)
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_conv_block(ctypes_ref(c1), ctypes_ref(c2), s), "conv_block")


def conv_block_pair_supported(taps, N, cin_pad, cout):
    """True when shrimp_conv_block_pair can run two ConvBlocks of this shape in one launch."""
    return bool(_lib.load().shrimp_conv_block_pair_supported(taps, N, cin_pad, cout))


def launch_conv_block_pair(*, x, x_sb, x_sn, idx, idx_stride, mask8, B, N, C, blocks, out, o_sb,
                           o_sn, stream=None):
    """Two consecutive ConvBlocks (model.py:395-422) in one launch, in place on `out`
    after the first: `blocks` holds two dicts of w1, b1, ln1_w, ln1_b, eps1, w2, b2,
    ln2_w, ln2_b, eps2, gamma. The first block reads `x` and writes `out`; the second
    reads and writes `out` (its rows handed over inside the workgroup)."""
    if len(blocks) != 2:
        raise ValueError("launch_conv_block_pair takes two blocks")
    c1, c2 = _block_args(x, x_sb, x_sn, idx, idx_stride, mask8, B, N, C, out=out, o_sb=o_sb,
                         o_sn=o_sn, **blocks[0])
    c3, c4 = _block_args(out, o_sb, o_sn, idx, idx_stride, mask8, B, N, C, out=out, o_sb=o_sb,
                         o_sn=o_sn, **blocks[1])
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_conv_block_pair(ctypes_ref(c1), ctypes_ref(c2), ctypes_ref(c3),
                                                  ctypes_ref(c4), s), "conv_block_pair")


def launch_linear(
    *, x, x_sr, wpack, bias, rows, n_in, n_out, mode, out, o_sr=0, ln_w=None, ln_b=None,
    eps=1e-5, resid=None, r_sr=0, gamma=None, mask=None, B=0, S=0, H=0, dpad=0,
    tok_lo=None, n_tokens=0, stream=None,
):
    """shrimp_linear; in the RESID mode ``tok_lo`` (B, n_tokens, n_out) bf16
    carries the low parts of the token rows (rows r with r % S < n_tokens)."""

    a = _lib.LinearArgs(
        x=x.data_ptr(), x_sr=x_sr, w=wpack.data_ptr(), bias=bias.data_ptr(),
        ln_w=_lib.ptr(ln_w), ln_b=_lib.ptr(ln_b), eps=float(eps), mode=mode,
        resid=_lib.ptr(resid), r_sr=r_sr, gamma=_lib.ptr(gamma), mask=_lib.ptr(mask),
        out=out.data_ptr(), o_sr=o_sr, rows=rows, in_features=n_in, out_features=n_out,
        B=B, S=S, H=H, dpad=dpad, tok_lo=_lib.ptr(tok_lo), n_tokens=n_tokens,
    )
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_linear(ctypes_ref(a), s), "linear")


def launch_attn_qkv(*, x, x_sr, qkv, packed, eps, rows, B, S, H, C, dpad, stream=None):
    """LN1 + q/k/v projection into the head-major (3, B, H, S, dpad) layout."""

    a = _lib.QkvArgs(x=x.data_ptr(), x_sr=x_sr, qkv=qkv.data_ptr(), packed=packed.data_ptr(),
                     eps=float(eps), rows=rows, B=B, S=S, H=H, C=C, dpad=dpad)
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_attn_qkv(ctypes_ref(a), s), "attn_qkv")


def launch_attn_mlp(*, x, x_sr, seq, s_sr, mask, packed, eps, rows, C, hidden, tok_lo=None,
                    S=None, n_tokens=0, stream=None):
    """Fused out_proj + residual + LN2 + fc1 + GELU + fc2 + residual, seq in
    place; ``tok_lo`` (B, n_tokens, C) bf16 carries the low parts of the token
    rows (the first n_tokens of every S rows). Without S the rows are one
    position."""

    a = _lib.MlpArgs(
        x=x.data_ptr(), x_sr=x_sr, seq=seq.data_ptr(), s_sr=s_sr, mask=mask.data_ptr(),
        packed=packed.data_ptr(), eps=float(eps), rows=rows, C=C, hidden=hidden,
        tok_lo=_lib.ptr(tok_lo), S=rows if S is None else S, n_tokens=n_tokens,
    )
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_attn_mlp(ctypes_ref(a), s), "attn_mlp")


def launch_attn(
    *, q, k, v, qkv_sb, qkv_sh, seq_lens, o, o_sb, o_sh, o_sr, B, S, H, d, dpad,
    pair=None, p_sb=0, p_sq=0, table2=None, coords=None, mask8=None, btab=None, xtab=None,
    lut_m=CELL_LUT_M, n_tokens=NUM_TOKENS, stream=None,
):
    a = _lib.AttnArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), qkv_sb=qkv_sb, qkv_sh=qkv_sh,
        seq_lens=seq_lens.data_ptr(), pair=_lib.ptr(pair), p_sb=p_sb, p_sq=p_sq,
        table2=_lib.ptr(table2), table_rows=0 if table2 is None else int(table2.shape[0]),
        coords=_lib.ptr(coords), mask=_lib.ptr(mask8), btab=_lib.ptr(btab),
        xtab=_lib.ptr(xtab), lut_m=lut_m,
        n_tokens=n_tokens, o=o.data_ptr(), o_sb=o_sb, o_sh=o_sh, o_sr=o_sr,
        B=B, S=S, H=H, d=d, dpad=dpad,
    )
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_attn(ctypes_ref(a), s), "attn")


def launch_attn_qkv_kvf(*, x, x_sr, q, kvf, packed, eps, rows, B, S, H, C, dpad, stream=None):
    """LN1 + q/k/v projection: q into the (B, H, S, dpad) layout of ``q``, k and v
    into the staged attention's fragment layout ``kvf`` (B, H, 2, SP, 16)."""

    a = _lib.QkvArgs(x=x.data_ptr(), x_sr=x_sr, qkv=q.data_ptr(), packed=packed.data_ptr(),
                     eps=float(eps), rows=rows, B=B, S=S, H=H, C=C, dpad=dpad)
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_attn_qkv_kvf(ctypes_ref(a), kvf.data_ptr(), s), "attn_qkv_kvf")


def attn_keys_ints(S: int) -> int:
    """int32 words of one position's key table (shrimp_attn_keys)."""

    return int(_lib.load().shrimp_attn_keys_bytes(S)) // 4


def launch_attn_keys(*, coords, mask8, seq_lens, B, S, n_tokens, meta, tokens=None, seq=None,
                     seq_sb=0, tok_lo=None, stream=None):
    """Key table of every position for the staged attention (once per forward).
    With ``tokens`` ((n_tokens, C) fp32) the same launch also writes the token
    rows of ``seq`` (positions ``seq_sb`` elements apart) and ``tok_lo``, as
    shrimp_fill_tokens does."""

    s = _lib.stream_handle() if stream is None else stream
    lib = _lib.load()
    if tokens is None:
        _lib.check(lib.shrimp_attn_keys(
            _lib.ptr(coords), _lib.ptr(mask8), seq_lens.data_ptr(), B, S, n_tokens,
            meta.data_ptr(), s), "attn_keys")
        return
    _lib.check(lib.shrimp_attn_keys_tokens(
        _lib.ptr(coords), _lib.ptr(mask8), seq_lens.data_ptr(), B, S, n_tokens, meta.data_ptr(),
        tokens.data_ptr(), tokens.shape[-1], seq.data_ptr(), seq_sb, _lib.ptr(tok_lo), s),
        "attn_keys_tokens")


def attn_staged_supported(H: int, S: int, dpad: int) -> bool:
    return bool(_lib.load().shrimp_attn_staged_supported(H, S, dpad))


def launch_attn_staged(
    *, q, qkv_sb, qkv_sh, meta, seq_lens, o, o_sb, o_sh, o_sr, B, S, H, d, dpad, btab, xtab,
    kvf=None, k=None, v=None, lut_m=CELL_LUT_M, n_tokens=NUM_TOKENS, stream=None,
):
    """Attention over K / V fragments from launch_attn_qkv_kvf (``kvf``), or over
    K / V rows ``k``, ``v`` in the layout of ``q`` (``kvf`` None), with the key
    table from launch_attn_keys (coords mode, LINEAR table required)."""

    if kvf is None and (k is None or v is None):
        raise ValueError("launch_attn_staged: kvf, or k and v rows, required")
    a = _lib.AttnArgs(
        q=q.data_ptr(), k=_lib.ptr(k), v=_lib.ptr(v), qkv_sb=qkv_sb, qkv_sh=qkv_sh,
        seq_lens=seq_lens.data_ptr(), pair=None, p_sb=0, p_sq=0, table2=None, table_rows=0,
        coords=None, mask=None, btab=btab.data_ptr(), xtab=xtab.data_ptr(), lut_m=lut_m,
        n_tokens=n_tokens, o=o.data_ptr(), o_sb=o_sb, o_sh=o_sh, o_sr=o_sr,
        B=B, S=S, H=H, d=d, dpad=dpad,
    )
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_attn_staged(ctypes_ref(a), _lib.ptr(kvf), meta.data_ptr(), s),
               "attn_staged")


def attn_fused_supported(C: int, H: int, S: int, dpad: int) -> bool:
    """Shapes the one-launch LN1 -> q/k/v -> attention kernel covers."""

    return bool(_lib.load().shrimp_attn_fused_supported(C, H, S, dpad))


def launch_attn_fused(
    *, x, x_sb, x_sr, packed, eps, seq_lens, o, o_sb, o_sh, o_sr, B, S, H, d, dpad,
    coords=None, mask8=None, btab=None, xtab=None, lut_m=CELL_LUT_M, n_tokens=NUM_TOKENS,
    stream=None,
):
    """AttnBlock LN1 -> q/k/v -> RelPosAttention in one launch (model.py:497-503, 448-492);
    ``packed`` is the output of ``pack_attn_qkv``, ``x`` the block input rows."""

    _check_rows("attn_fused x", x, x_sb, x_sr, B, S, H * d)
    a = _lib.AttnArgs(
        q=None, k=None, v=None, qkv_sb=0, qkv_sh=0, seq_lens=seq_lens.data_ptr(), pair=None,
        p_sb=0, p_sq=0, table2=None, table_rows=0, coords=_lib.ptr(coords),
        mask=_lib.ptr(mask8), btab=_lib.ptr(btab), xtab=_lib.ptr(xtab), lut_m=lut_m,
        n_tokens=n_tokens, o=o.data_ptr(), o_sb=o_sb, o_sh=o_sh, o_sr=o_sr,
        B=B, S=S, H=H, d=d, dpad=dpad,
    )
    pj = _lib.AttnProjArgs(x=x.data_ptr(), x_sb=x_sb, x_sr=x_sr, packed=packed.data_ptr(),
                           eps=float(eps))
    s = _lib.stream_handle() if stream is None else stream
    _lib.check(_lib.load().shrimp_attn_fused(ctypes_ref(a), ctypes_ref(pj), s), "attn_fused")


def ctypes_ref(struct):
    import ctypes

    return ctypes.byref(struct)


# ---- the reference operator ABI -----------------------------------------------------------


def _bf16_rows(x: torch.Tensor, cin_pad: int) -> torch.Tensor:
    """x (B, N, C) -> contiguous bf16 (B, N, cin_pad) (zero channel padding)."""

    b, n, c = x.shape
    xb = x.to(torch.bfloat16)
    if c == cin_pad:
        return xb.contiguous()
    out = torch.zeros((b, n, cin_pad), dtype=torch.bfloat16, device=x.device)
    out[..., :c] = xb
    return out


def _conv_common(x, gather_idx, mask, weight, bias, ln_weight, ln_bias, eps, relu):
    require_device(x, "shrimp::hex_conv")
    b, n, c = x.shape
    t = weight.shape[0]
    cout = weight.shape[-1]
    cp = cin_pad_of(c)
    xb = _bf16_rows(x, cp)
    idx = gather_idx.to(torch.int32).contiguous()
    m8 = mask.to(torch.uint8).contiguous()
    wp = pack_conv_weight(weight, cp)
    out = torch.empty((b, n, cout), dtype=torch.bfloat16, device=x.device)
    launch_conv(
        x=xb, x_sb=n * cp, x_sn=cp, idx=idx, taps=t, idx_stride=idx.shape[-1], mask8=m8,
        wpack=wp, bias=bias.to(torch.float32).contiguous(), B=b, N=n, cin_pad=cp, cout=cout,
        ln_w=None if ln_weight is None else ln_weight.to(torch.float32).contiguous(),
        ln_b=None if ln_bias is None else ln_bias.to(torch.float32).contiguous(),
        eps=eps, relu=relu, out=out, o_sb=n * cout, o_sn=cout,
    )
    return out


@torch.library.custom_op("shrimp::hex_conv", mutates_args=())
def hex_conv(
    x: torch.Tensor,
    gather_idx: torch.Tensor,
    mask: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
) -> torch.Tensor:
    """out[b, i] = mask * (sum_t x[b, gather_idx[b, i, t]] @ weight[t] + bias);
    gather_idx entries outside [0, N) (the reference's Npad sentinel) read as
    zero rows."""

    return _conv_common(x, gather_idx, mask, weight, bias, None, None, 1e-5, False)


@hex_conv.register_fake
def _hex_conv_fake(x, gather_idx, mask, weight, bias):
    return x.new_empty((x.shape[0], x.shape[1], weight.shape[-1]), dtype=torch.bfloat16)


@torch.library.custom_op("shrimp::hex_conv_ln", mutates_args=())
def hex_conv_ln(
    x: torch.Tensor,
    gather_idx: torch.Tensor,
    mask: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    eps: float,
    relu: bool,
) -> torch.Tensor:
    """hex_conv followed by LayerNorm over the output channels (fp32 stats on
    the accumulator), optional ReLU and the row mask."""

    return _conv_common(x, gather_idx, mask, weight, bias, ln_weight, ln_bias, eps, relu)


@hex_conv_ln.register_fake
def _hex_conv_ln_fake(x, gather_idx, mask, weight, bias, ln_weight, ln_bias, eps, relu):
    return x.new_empty((x.shape[0], x.shape[1], weight.shape[-1]), dtype=torch.bfloat16)


@torch.library.custom_op("shrimp::attn_pair", mutates_args=())
def attn_pair(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    pair: torch.Tensor,
    table2: torch.Tensor,
    seq_lens: torch.Tensor,
) -> torch.Tensor:
    """softmax(q k^T / sqrt(D) + table2[pair[b, i, j], h]) v over keys
    j < seq_lens[b]; q/k/v (B, H, S, D). Query rows >= seq_lens[b] are 0."""

    require_device(q, "shrimp::attn_pair")
    b, h, s, d = q.shape
    dpad = max(16, -(-d // 16) * 16)

    def prep(t):
        t = t.to(torch.bfloat16)
        if dpad != d:
            t = torch.nn.functional.pad(t, (0, dpad - d))
        return t.contiguous()

    qb, kb, vb = prep(q), prep(k), prep(v)
    pr = pair.to(torch.uint8).contiguous()
    tab = table2.to(torch.float32).contiguous()
    sl = seq_lens.to(torch.int32).contiguous()
    out = torch.empty((b, h, s, d), dtype=torch.bfloat16, device=q.device)
    launch_attn(
        q=qb, k=kb, v=vb, qkv_sb=h * s * dpad, qkv_sh=s * dpad, seq_lens=sl,
        o=out, o_sb=h * s * d, o_sh=s * d, o_sr=d, B=b, S=s, H=h, d=d, dpad=dpad,
        pair=pr, p_sb=s * s, p_sq=s, table2=tab, n_tokens=0,
    )
    return out


@attn_pair.register_fake
def _attn_pair_fake(q, k, v, pair, table2, seq_lens):
    return q.new_empty(q.shape, dtype=torch.bfloat16)
