"""hexfield_eq serve ops over the C ABI (``include/shrimp_hip.h``).

Op names and argument meaning follow the reference's custom ops:
``hexfield_eq::ray_gather_index`` (``_triton_ray.py:284-295``),
``hexfield_eq::ray_attn`` (``_triton_ray.py:681-715``) and
``hexfield_eq::hex_conv_ln_raytap`` (``_triton_conv.py:501-555``), and the
slot tables of ``_raytap.py:47-107``. They run the gfx950 kernels of
``libshrimp_hip.so`` in fp16 (the reference's serve dtype) and raise for
shapes the kernels do not cover; there is no CPU path.
"""

from __future__ import annotations

import functools

import torch

from shrimp import _lib
from shrimp.ops import require_device

RAY_GATHER_SLOTS = 32
RAY_REACH = 5
RAYLEN_SLOTS = 12
DIRECTIONS = ((1, 0), (0, 1), (-1, 1), (-1, 0), (0, -1), (1, -1))
AXES = ((1, 0), (0, 1), (1, -1))  # Q, R, QR

RayAttnArgs = _lib.RayAttnArgs
RaytapArgs = _lib.RaytapArgs


def _load():
    return _lib.load()


# ---- slot geometry (_triton_ray.py:131-152, _raytap.py:47-107) ----------------------------


@functools.lru_cache(maxsize=1)
def slot_offset_table() -> torch.Tensor:
    """(32, 2) long: slot 0 self (0, 0); slot 1 + axis*10 + dir*5 + (k-1) the
    offset dir_sign * k * axis (dir 0 = +, 1 = -); slot 31 (0, 0), never live."""

    off = torch.zeros(RAY_GATHER_SLOTS, 2, dtype=torch.long)
    for a, (aq, ar) in enumerate(AXES):
        for d, sgn in enumerate((1, -1)):
            for k in range(1, RAY_REACH + 1):
                off[1 + a * 10 + d * 5 + k - 1] = torch.tensor([sgn * k * aq, sgn * k * ar])
    return off


@functools.lru_cache(maxsize=1)
def tap_axis_dir() -> tuple:
    """(axis, dir) of direction taps 1..6: +axis -> dir 0, -axis -> dir 1."""

    out = []
    for dq, dr in DIRECTIONS:
        for a, (aq, ar) in enumerate(AXES):
            if (dq, dr) == (aq, ar):
                out.append((a, 0))
            elif (dq, dr) == (-aq, -ar):
                out.append((a, 1))
    return tuple(out)


@functools.lru_cache(maxsize=1)
def tap_raylen_slots() -> torch.Tensor:
    """(2, 6) long: raylen slot side*6 + axis*2 + dir of (side, tap - 1)."""

    out = torch.empty(2, 6, dtype=torch.long)
    for side in range(2):
        for t, (a, d) in enumerate(tap_axis_dir()):
            out[side, t] = side * 6 + a * 2 + d
    return out


@functools.lru_cache(maxsize=1)
def tap_ray_slot_lut() -> torch.Tensor:
    """(6, 5) long: slot of the cell k steps along direction tap t."""

    out = torch.empty(6, RAY_REACH, dtype=torch.long)
    for t, (a, d) in enumerate(tap_axis_dir()):
        for k in range(1, RAY_REACH + 1):
            out[t, k - 1] = 1 + a * 10 + d * 5 + (k - 1)
    return out


def build_tap_reach(raylen: torch.Tensor) -> torch.Tensor:
    """(B, N, 12) u8 raylen wire buffer -> (B, N, 2, 6) u8 per-(side, tap) reach."""

    return raylen[:, :, tap_raylen_slots().to(raylen.device)]


# ---- launches -------------------------------------------------------------------------------


def _strides_ok(t: torch.Tensor) -> bool:
    return (t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1])
            and t.data_ptr() % 16 == 0)


def _fp16_view(t: torch.Tensor) -> torch.Tensor:
    t = t.to(torch.float16)
    return t if _strides_ok(t) else t.contiguous()


def launch_ray_attn(q, k, v, idx, slot_bias16, raylen, seq_lens32, blockers, out) -> None:
    """Raw launch: q/k/v/out fp16 (B, H, N, D) views with 8-element-aligned
    strides, idx int32 (B, N, 32), slot_bias16 (32, H) fp16 contiguous, raylen
    u8 (B, N, 12) (ignored without blockers), seq_lens32 int32 (B,)."""

    b, h, n, d = q.shape
    a = RayAttnArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
        q_sb=q.stride(0), q_sh=q.stride(1), q_sn=q.stride(2),
        k_sb=k.stride(0), k_sh=k.stride(1), k_sn=k.stride(2),
        v_sb=v.stride(0), v_sh=v.stride(1), v_sn=v.stride(2),
        idx=idx.data_ptr(), idx_sb=idx.stride(0), idx_sn=idx.stride(1),
        slot_bias=slot_bias16.data_ptr(),
        raylen=raylen.data_ptr() if blockers else None,
        rl_sb=raylen.stride(0) if blockers else 0, rl_sn=raylen.stride(1) if blockers else 0,
        seq_lens=seq_lens32.data_ptr(), out=out.data_ptr(),
        o_sb=out.stride(0), o_sh=out.stride(1), o_sn=out.stride(2),
        B=b, H=h, N=n, D=d, blockers=1 if blockers else 0,
    )
    _lib.check(_load().shrimp_ray_attn(_lib.ctypes.byref(a), _lib.stream_handle(q.device)),
               "hexfield_eq::ray_attn")


def ray_attn_variant(v: int) -> int:
    """0 = automatic (K/V staged in LDS when they fit), 1 = global gathers;
    other values only query. Returns the previous setting."""

    return int(_load().shrimp_ray_attn_variant(int(v)))


def pack_raytap_weight(weight: torch.Tensor) -> torch.Tensor:
    """(7, C, Cout) conv weight -> packed fp16 MFMA fragments (uint8 bytes)."""

    require_device(weight, "pack_raytap_weight")
    t, c, cout = weight.shape
    if t != 7:
        raise ValueError(f"hex_conv_ln_raytap: weight has {t} taps, expected 7")
    lib = _load()
    nbytes = lib.shrimp_raytap_wpack_bytes(c, cout)
    if nbytes == 0:
        raise ValueError(f"hex_conv_ln_raytap: C={c}, Cout={cout} not in {{64, 96, 128}}")
    w16 = weight.detach().to(torch.float16).contiguous()
    out = torch.empty(nbytes, dtype=torch.uint8, device=weight.device)
    _lib.check(lib.shrimp_pack_raytap_weight(w16.data_ptr(), c, cout, out.data_ptr(),
                                             _lib.stream_handle(weight.device)),
               "pack_raytap_weight")
    return out


def launch_conv_ln_raytap(x, gidx32, mask8, packed, bias32, lnw32, lnb32, ray_idx32, reach8,
                          alpha16, eps, relu, corb, out) -> None:
    """Raw launch of K1 on prepared buffers (see the header for layouts)."""

    b, n, c = x.shape
    a = RaytapArgs(
        x=x.data_ptr(), x_sb=x.stride(0), x_sn=x.stride(1),
        gather_idx=gidx32.data_ptr(), g_sb=gidx32.stride(0), g_sn=gidx32.stride(1),
        mask=mask8.data_ptr(), packed_w=packed.data_ptr(), bias=bias32.data_ptr(),
        ln_w=lnw32.data_ptr(), ln_b=lnb32.data_ptr(),
        ray_idx=ray_idx32.data_ptr(), r_sb=ray_idx32.stride(0), r_sn=ray_idx32.stride(1),
        reach=reach8.data_ptr(), re_sb=reach8.stride(0), re_sn=reach8.stride(1),
        alpha=alpha16.data_ptr(), eps=float(eps), relu=1 if relu else 0, corb=int(corb),
        out=out.data_ptr(), o_sb=out.stride(0), o_sn=out.stride(1),
        B=b, N=n, C=c, Cout=out.shape[-1],
    )
    _lib.check(_load().shrimp_conv_ln_raytap(_lib.ctypes.byref(a), _lib.stream_handle(x.device)),
               "hexfield_eq::hex_conv_ln_raytap")


# ---- the reference operator names ------------------------------------------------------------


@torch.library.custom_op("hexfield_eq::ray_gather_index", mutates_args=())
def build_ray_gather_index(coords: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """(B, N, 32) int32: slot 0 = the row itself, slot 1 + axis*10 + dir*5 +
    (k-1) = the live cell at coords + dir_sign * k * axis (else N), slot 31 = N."""

    require_device(coords, "hexfield_eq::ray_gather_index")
    b, n, _ = coords.shape
    c32 = coords.to(torch.int32).contiguous()
    m8 = mask.to(torch.uint8).contiguous()
    out = torch.empty((b, n, RAY_GATHER_SLOTS), dtype=torch.int32, device=coords.device)
    lib = _load()
    _lib.check(lib.shrimp_build_ray_index(c32.data_ptr(), m8.data_ptr(), b, n, out.data_ptr(),
                                          _lib.stream_handle(coords.device)),
               "hexfield_eq::ray_gather_index")
    return out


@build_ray_gather_index.register_fake
def _ray_gather_index_fake(coords, mask):
    b, n, _ = coords.shape
    return coords.new_empty((b, n, RAY_GATHER_SLOTS), dtype=torch.int32)


@torch.library.custom_op("hexfield_eq::ray_attn", mutates_args=())
def ray_attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    idx: torch.Tensor,
    slot_bias: torch.Tensor,
    raylen: torch.Tensor,
    seq_lens: torch.Tensor,
    blockers: bool,
) -> torch.Tensor:
    """Gathered ray attention, q/k/v (B, H, N, D) with D in {16, 32, 64, 128}:
    per row and head, softmax over the self slot and the live slots of the
    head's win axis (step k within raylen with blockers), fp32 math, fp16
    out, rows >= seq_lens zero. slot_bias (32, H) is rounded to fp16 as the
    reference's kernel path does."""

    require_device(q, "hexfield_eq::ray_attn")
    b, h, n, d = q.shape
    if d not in (16, 32, 64, 128):
        raise ValueError(f"hexfield_eq::ray_attn: head_dim {d} not in (16, 32, 64, 128)")
    qh, kh, vh = _fp16_view(q), _fp16_view(k), _fp16_view(v)
    ix = idx.to(torch.int32)
    if ix.stride(-1) != 1:
        ix = ix.contiguous()
    sb = slot_bias.to(torch.float16).contiguous()
    sl = seq_lens.to(torch.int32).contiguous()
    rl = raylen.to(torch.uint8) if blockers else raylen
    if blockers and rl.stride(-1) != 1:
        rl = rl.contiguous()
    out = torch.empty((b, h, n, d), dtype=torch.float16, device=q.device)
    launch_ray_attn(qh, kh, vh, ix, sb, rl, sl, blockers, out)
    return out


@ray_attn.register_fake
def _ray_attn_fake(q, k, v, idx, slot_bias, raylen, seq_lens, blockers):
    return q.new_empty(q.shape, dtype=torch.float16)


@torch.library.custom_op("hexfield_eq::hex_conv_ln_raytap", mutates_args=())
def hex_conv_ln_raytap(
    x: torch.Tensor,
    gather_idx: torch.Tensor,
    mask: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    ray_idx: torch.Tensor,
    reach: torch.Tensor,
    alpha: torch.Tensor,
    eps: float,
    relu: bool,
    corb: int,
) -> torch.Tensor:
    """K1: [x[centre] | 6 reach-masked alpha-weighted ray taps] @ weight.reshape(7C,
    Cout) + bias, LayerNorm (+ReLU), row mask; fp16 out. ``reach`` (B, N, 2, 6)
    u8, ``alpha`` (5, C), ``corb`` the orbit width whose halves carry the
    own / opp visibility split."""

    require_device(x, "hexfield_eq::hex_conv_ln_raytap")
    b, n, c = x.shape
    cout = weight.shape[-1]
    xh = _fp16_view(x)
    gi = gather_idx.to(torch.int32)
    if gi.stride(-1) != 1:
        gi = gi.contiguous()
    m8 = mask.to(torch.uint8).contiguous()
    ri = ray_idx.to(torch.int32)
    if ri.stride(-1) != 1:
        ri = ri.contiguous()
    re = reach.to(torch.uint8).reshape(b, n, 12)
    if re.stride(-1) != 1:
        re = re.contiguous()
    packed = pack_raytap_weight(weight.reshape(7, c, cout))
    out = torch.empty((b, n, cout), dtype=torch.float16, device=x.device)
    launch_conv_ln_raytap(
        xh, gi, m8, packed, bias.to(torch.float32).contiguous(),
        ln_weight.to(torch.float32).contiguous(), ln_bias.to(torch.float32).contiguous(),
        ri, re, alpha.to(torch.float16).contiguous(), eps, relu, corb, out,
    )
    return out


@hex_conv_ln_raytap.register_fake
def _hex_conv_ln_raytap_fake(x, gather_idx, mask, weight, bias, ln_weight, ln_bias, ray_idx,
                             reach, alpha, eps, relu, corb):
    return x.new_empty((x.shape[0], x.shape[1], weight.shape[-1]), dtype=torch.float16)
