"""ctypes binding of ``libshrimp_hip.so`` (the C ABI in ``include/shrimp_hip.h``).

The library is built in-tree (``hexo-bot_amd/shrimp/_lib/``) by
``__graft_entry__.build()`` / ``make -C hexo-bot_amd/csrc``. There is no
fallback: if the library is missing every GPU entry point raises, naming the
build step.

``SHRIMP_HIP_LIB`` (a path) loads another build of the same ABI in its place,
e.g. the checked build ``libshrimp_hip_check.so`` (``make -C hexo-bot_amd/csrc
check``: the kernels' input checks, and a device synchronisation after every
launch that reports a failed check as status -3).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIB_PATH = LIB_DIR / "libshrimp_hip.so"
CHECK_LIB_PATH = LIB_DIR / "libshrimp_hip_check.so"
PHASE_LIB_PATH = LIB_DIR / "libshrimp_hip_phase.so"

DT_BF16, DT_F32, DT_F16, DT_I64, DT_I32, DT_U16, DT_U8 = range(7)
LIN_PLAIN, LIN_GELU, LIN_RESID, LIN_QKV = range(4)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class ConvArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_sb", _i64), ("x_sn", _i64),
        ("idx", _vp), ("taps", _i32), ("idx_stride", _i32),
        ("mask", _vp), ("w", _vp), ("bias", _vp),
        ("ln_w", _vp), ("ln_b", _vp), ("eps", _f32), ("relu", _i32),
        ("resid", _vp), ("r_sb", _i64), ("r_sn", _i64), ("gamma", _vp),
        ("head_w", _vp), ("head_b", _vp), ("head_out", _vp),
        ("out", _vp), ("o_sb", _i64), ("o_sn", _i64),
        ("B", _i32), ("N", _i32), ("cin_pad", _i32), ("cout", _i32),
    ]


class LinearArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_sr", _i64), ("w", _vp), ("bias", _vp),
        ("ln_w", _vp), ("ln_b", _vp), ("eps", _f32), ("mode", _i32),
        ("resid", _vp), ("r_sr", _i64), ("gamma", _vp), ("mask", _vp),
        ("out", _vp), ("o_sr", _i64),
        ("rows", _i32), ("in_features", _i32), ("out_features", _i32),
        ("B", _i32), ("S", _i32), ("H", _i32), ("dpad", _i32),
        ("tok_lo", _vp), ("n_tokens", _i32),
    ]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("qkv_sb", _i64), ("qkv_sh", _i64),
        ("seq_lens", _vp),
        ("pair", _vp), ("p_sb", _i64), ("p_sq", _i64), ("table2", _vp), ("table_rows", _i32),
        ("coords", _vp), ("mask", _vp), ("btab", _vp), ("xtab", _vp), ("lut_m", _i32),
        ("n_tokens", _i32),
        ("o", _vp), ("o_sb", _i64), ("o_sh", _i64), ("o_sr", _i64),
        ("B", _i32), ("S", _i32), ("H", _i32), ("d", _i32), ("dpad", _i32),
    ]


class AttnProjArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_sb", _i64), ("x_sr", _i64), ("packed", _vp), ("eps", _f32),
    ]


class TailArgs(ctypes.Structure):
    _fields_ = [
        ("seq", _vp), ("s_sb", _i64), ("mask", _vp), ("ln_w", _vp), ("ln_b", _vp),
        ("eps", _f32), ("out_seq", _vp),
        ("vr_w", _vp), ("vr_b", _vp), ("vh_w", _vp), ("vh_b", _vp), ("value", _vp),
        ("mr_w", _vp), ("mr_b", _vp), ("mh_w", _vp), ("mh_b", _vp), ("moves_left", _vp),
        ("workspace", _vp),
        ("B", _i32), ("S", _i32), ("n_tokens", _i32), ("C", _i32), ("bins", _i32),
        ("tok_lo", _vp),
    ]


class QkvArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_sr", _i64), ("qkv", _vp), ("packed", _vp), ("eps", _f32),
        ("rows", _i32), ("B", _i32), ("S", _i32), ("H", _i32), ("C", _i32), ("dpad", _i32),
    ]


class MlpWeights(ctypes.Structure):
    _fields_ = [
        ("out_w", _vp), ("out_b", _vp), ("g_attn", _vp), ("ln_w", _vp), ("ln_b", _vp),
        ("fc1_w", _vp), ("fc1_b", _vp), ("fc2_w", _vp), ("fc2_b", _vp), ("g_mlp", _vp),
        ("C", _i32), ("hidden", _i32),
    ]


class MlpArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_sr", _i64), ("seq", _vp), ("s_sr", _i64), ("mask", _vp),
        ("packed", _vp), ("eps", _f32), ("rows", _i32), ("C", _i32), ("hidden", _i32),
        ("tok_lo", _vp), ("S", _i32), ("n_tokens", _i32),
    ]


class RayAttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp),
        ("q_sb", _i64), ("q_sh", _i64), ("q_sn", _i64),
        ("k_sb", _i64), ("k_sh", _i64), ("k_sn", _i64),
        ("v_sb", _i64), ("v_sh", _i64), ("v_sn", _i64),
        ("idx", _vp), ("idx_sb", _i64), ("idx_sn", _i64),
        ("slot_bias", _vp), ("raylen", _vp), ("rl_sb", _i64), ("rl_sn", _i64),
        ("seq_lens", _vp), ("out", _vp), ("o_sb", _i64), ("o_sh", _i64), ("o_sn", _i64),
        ("B", _i32), ("H", _i32), ("N", _i32), ("D", _i32), ("blockers", _i32),
    ]


class RaytapArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("x_sb", _i64), ("x_sn", _i64),
        ("gather_idx", _vp), ("g_sb", _i64), ("g_sn", _i64),
        ("mask", _vp), ("packed_w", _vp), ("bias", _vp), ("ln_w", _vp), ("ln_b", _vp),
        ("ray_idx", _vp), ("r_sb", _i64), ("r_sn", _i64),
        ("reach", _vp), ("re_sb", _i64), ("re_sn", _i64),
        ("alpha", _vp), ("eps", _f32), ("relu", _i32), ("corb", _i32),
        ("out", _vp), ("o_sb", _i64), ("o_sn", _i64),
        ("B", _i32), ("N", _i32), ("C", _i32), ("Cout", _i32),
    ]


# Exported symbols and their ctypes signatures; tests check every one of them
# against the header and the built library.
SIGNATURES: dict = {
    "shrimp_last_error": (ctypes.c_char_p, []),
    "shrimp_abi_version": (ctypes.c_int, []),
    "shrimp_conv_variant": (ctypes.c_int, [ctypes.c_int]),
    "shrimp_attn_variant": (ctypes.c_int, [ctypes.c_int]),
    "shrimp_max_lds_per_block": (ctypes.c_int, []),
    "shrimp_conv_wpack_bytes": (ctypes.c_size_t, [ctypes.c_int] * 3),
    "shrimp_pack_conv_weight": (ctypes.c_int, [_vp, _vp] + [ctypes.c_int] * 4 + [_vp]),
    "shrimp_linear_wpack_bytes": (ctypes.c_size_t, [ctypes.c_int] * 2),
    "shrimp_pack_linear_weight": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp]),
    "shrimp_hex_conv": (ctypes.c_int, [ctypes.POINTER(ConvArgs), _vp]),
    "shrimp_conv_block_supported": (ctypes.c_int, [ctypes.c_int] * 4),
    "shrimp_conv_block": (ctypes.c_int, [ctypes.POINTER(ConvArgs), ctypes.POINTER(ConvArgs), _vp]),
    "shrimp_conv_block_pair_supported": (ctypes.c_int, [ctypes.c_int] * 4),
    "shrimp_conv_block_pair": (ctypes.c_int, [ctypes.POINTER(ConvArgs)] * 4 + [_vp]),
    "shrimp_linear": (ctypes.c_int, [ctypes.POINTER(LinearArgs), _vp]),
    "shrimp_attn_qkv": (ctypes.c_int, [ctypes.POINTER(QkvArgs), _vp]),
    "shrimp_attn_qkv_kvf": (ctypes.c_int, [ctypes.POINTER(QkvArgs), _vp, _vp]),
    "shrimp_attn_keys_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "shrimp_attn_keys": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "shrimp_attn_keys_tokens": (
        ctypes.c_int,
        [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp, ctypes.c_int, _vp, _i64,
         _vp, _vp],
    ),
    "shrimp_attn_staged_supported": (ctypes.c_int, [ctypes.c_int] * 3),
    "shrimp_attn_staged": (ctypes.c_int, [ctypes.POINTER(AttnArgs), _vp, _vp, _vp]),
    "shrimp_attn_qkv_pack_bytes": (ctypes.c_size_t, [ctypes.c_int]),
    "shrimp_pack_attn_qkv": (ctypes.c_int, [_vp] * 6 + [ctypes.c_int, _vp]),
    "shrimp_attn_mlp": (ctypes.c_int, [ctypes.POINTER(MlpArgs), _vp]),
    "shrimp_attn_mlp_pack_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "shrimp_pack_attn_mlp": (ctypes.c_int, [ctypes.POINTER(MlpWeights), _vp, _vp, _vp]),
    "shrimp_attn": (ctypes.c_int, [ctypes.POINTER(AttnArgs), _vp]),
    "shrimp_featurize": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "shrimp_attn_fused": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.POINTER(AttnProjArgs), _vp]),
    "shrimp_attn_fused_supported": (ctypes.c_int, [ctypes.c_int] * 4),
    "shrimp_attn_bias_table": (
        ctypes.c_int,
        [_vp, ctypes.c_int, ctypes.c_int, _vp] + [ctypes.c_int] * 4 + [_vp, _vp, _vp],
    ),
    "shrimp_prep_inputs": (
        ctypes.c_int,
        [_vp, ctypes.c_int, _vp, _vp, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int,
         ctypes.c_int, ctypes.c_int, ctypes.c_int] + [_vp] * 7,
    ),
    "shrimp_prep_csr": (
        ctypes.c_int,
        [_vp, ctypes.c_int, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        + [_vp] * 7,
    ),
    "shrimp_fill_tokens": (
        ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, _i64, _vp, ctypes.c_int, _vp]
    ),
    "shrimp_trunk_tail": (ctypes.c_int, [ctypes.POINTER(TailArgs), _vp]),
    "shrimp_policy_tail_supported": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "shrimp_policy_tail": (ctypes.c_int, [ctypes.POINTER(ConvArgs), ctypes.POINTER(TailArgs), _vp]),
    "shrimp_trunk_tail_noalloc": (ctypes.c_int, [ctypes.POINTER(TailArgs), _vp]),
    "shrimp_decode": (
        ctypes.c_int,
        [_vp, _vp, _vp, _i64, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        + [_vp] * 5,
    ),
    "shrimp_build_pair_u8": (
        ctypes.c_int, [_vp, _vp, _vp] + [ctypes.c_int] * 8 + [_vp, _vp]
    ),
    "shrimp_build_ray_index": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "shrimp_ray_attn": (ctypes.c_int, [ctypes.POINTER(RayAttnArgs), _vp]),
    "shrimp_ray_attn_variant": (ctypes.c_int, [ctypes.c_int]),
    "shrimp_raytap_wpack_bytes": (ctypes.c_size_t, [ctypes.c_int] * 2),
    "shrimp_pack_raytap_weight": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, _vp]),
    "shrimp_conv_ln_raytap": (ctypes.c_int, [ctypes.POINTER(RaytapArgs), _vp]),
    "shrimp_conv_wpack_bytes_f32": (ctypes.c_size_t, [ctypes.c_int] * 3),
    "shrimp_pack_conv_weight_f32": (ctypes.c_int, [_vp, _vp] + [ctypes.c_int] * 4 + [_vp]),
    "shrimp_pack_linear_weight_f32": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp]),
    "shrimp_hex_conv_f32": (ctypes.c_int, [ctypes.POINTER(ConvArgs), _vp]),
    "shrimp_linear_f32": (ctypes.c_int, [ctypes.POINTER(LinearArgs), _vp]),
    "shrimp_attn_f32": (ctypes.c_int, [ctypes.POINTER(AttnArgs), _vp]),
    "shrimp_trunk_tail_f32": (ctypes.c_int, [ctypes.POINTER(TailArgs), _vp]),
    "shrimp_prep_feats_f32": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, _vp, _vp]),
    "shrimp_prep_csr_feats_f32": (ctypes.c_int, [_vp, ctypes.c_int, _vp] + [ctypes.c_int] * 3
                                  + [_vp, _vp]),
    "shrimp_phase_clock": (ctypes.c_int, [_vp, ctypes.c_int]),
    "shrimp_fill_tokens_f32": (
        ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, _i64, ctypes.c_int, _vp]
    ),
}

_LIB = None


class HipLibraryMissing(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library, with every signature bound."""

    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else Path(os.environ.get("SHRIMP_HIP_LIB") or LIB_PATH)
    if not p.exists():
        raise HipLibraryMissing(
            f"{p} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(or `make -C hexo-bot_amd/csrc`) before using the shrimp HIP forward"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().shrimp_last_error()
        raise RuntimeError(f"{what} failed ({status}): {msg.decode() if msg else ''}")


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""

    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
