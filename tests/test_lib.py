"""The C-ABI library: it loads, exports every symbol include/shrimp_hip.h
declares, its struct layouts match the ctypes mirrors, and argument checks
fail with a message before any device work (no GPU needed)."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from shrimp import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "shrimp_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(shrimp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built; run __graft_entry__.build()")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name


def test_version(lib):
    assert lib.shrimp_abi_version() == 1


def test_struct_layouts_match_c(tmp_path):
    exe = tmp_path / "abi_layout"
    subprocess.run(
        ["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(ROOT / "tests" / "abi_layout.c"), "-o", str(exe)],
        check=True,
    )
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    mirrors = {
        "shrimp_conv_args": _lib.ConvArgs,
        "shrimp_linear_args": _lib.LinearArgs,
        "shrimp_attn_args": _lib.AttnArgs,
        "shrimp_attn_proj_args": _lib.AttnProjArgs,
        "shrimp_tail_args": _lib.TailArgs,
        "shrimp_qkv_args": _lib.QkvArgs,
        "shrimp_mlp_weights": _lib.MlpWeights,
        "shrimp_mlp_args": _lib.MlpArgs,
        "shrimp_ray_attn_args": _lib.RayAttnArgs,
        "shrimp_raytap_args": _lib.RaytapArgs,
    }
    seen = 0
    for line in filter(None, lines):
        key, val = line.split()
        sname, field = key.split(".")
        cls = mirrors[sname]
        if field == "__size__":
            assert ctypes.sizeof(cls) == int(val), sname
        else:
            assert getattr(cls, field).offset == int(val), key
        seen += 1
    names = {f for cls in mirrors.values() for f, _ in cls._fields_}
    assert seen == len(mirrors) + sum(len(c._fields_) for c in mirrors.values())
    assert names


def test_bad_arguments_fail_with_message(lib):
    a = _lib.ConvArgs(B=1, N=4, cin_pad=33, cout=128, taps=7, idx_stride=7,
                      x=1, idx=1, mask=1, w=1, bias=1, out=1, x_sn=64)
    rc = lib.shrimp_hex_conv(ctypes.byref(a), None)
    assert rc == -1
    assert b"cin_pad" in lib.shrimp_last_error()
    la = _lib.LinearArgs(rows=4, in_features=100, out_features=128, x=1, w=1, bias=1, out=1,
                         x_sr=100, o_sr=128, mode=0)
    assert lib.shrimp_linear(ctypes.byref(la), None) == -1
    aa = _lib.AttnArgs(B=1, S=8, H=2, d=6, dpad=16, q=1, k=1, v=1, o=1, seq_lens=1)
    assert lib.shrimp_attn(ctypes.byref(aa), None) == -1
    assert b"head dim" in lib.shrimp_last_error()
    assert lib.shrimp_build_ray_index(1, 1, 1, 5000, 1, None) == -1
    # featurizer: radius range and required outputs are checked before any launch
    one = (ctypes.c_int64 * 2)(0, 0)
    cnt = (ctypes.c_int32 * 4)()
    stt = (ctypes.c_int32 * 1)()
    assert lib.shrimp_featurize(None, None, None, one, None, None, 1, 0, 64, None, None, None,
                                None, cnt, stt, None) == -1
    assert b"radius" in lib.shrimp_last_error()
    assert lib.shrimp_featurize(None, None, None, one, None, None, 1, 8, 64, cnt, None, None,
                                None, cnt, stt, None) == -1
    assert b"outputs" in lib.shrimp_last_error()
    # one-launch LN1 + q/k/v + attention: C = 128, H = 8, dpad = 16, S <= 320 only
    assert lib.shrimp_attn_fused_supported(128, 8, 264, 16) == 1
    assert lib.shrimp_attn_fused_supported(128, 8, 320, 16) == 1
    assert lib.shrimp_attn_fused_supported(128, 8, 321, 16) == 0
    assert lib.shrimp_attn_fused_supported(128, 4, 264, 32) == 0
    assert lib.shrimp_attn_fused_supported(64, 8, 264, 16) == 0
    pj = _lib.AttnProjArgs(x=1, x_sb=264 * 128, x_sr=128, packed=1, eps=1e-5)
    fa = _lib.AttnArgs(B=1, S=400, H=8, d=16, dpad=16, o=1, seq_lens=1, btab=1, coords=1,
                       mask=1, o_sb=400 * 128, o_sh=16, o_sr=128, n_tokens=8)
    assert lib.shrimp_attn_fused(ctypes.byref(fa), ctypes.byref(pj), None) == -1
    assert b"S <= 320" in lib.shrimp_last_error()
    fa.S = 264
    pj.x_sr = 100
    assert lib.shrimp_attn_fused(ctypes.byref(fa), ctypes.byref(pj), None) == -1
    assert b"x strides" in lib.shrimp_last_error()
    # hexfield ray attention: head dim, strides, blockers without raylen
    ra = _lib.RayAttnArgs(B=1, H=6, N=64, D=24, q=16, k=16, v=16, out=16, idx=16, slot_bias=16,
                          seq_lens=16, idx_sb=64 * 32, idx_sn=32, blockers=0)
    assert lib.shrimp_ray_attn(ctypes.byref(ra), None) == -1
    assert b"head dim" in lib.shrimp_last_error()
    ra.D = 16
    ra.q_sn = 12
    assert lib.shrimp_ray_attn(ctypes.byref(ra), None) == -1
    assert b"multiples of 8" in lib.shrimp_last_error()
    ra.q_sn = -96  # the kernel's 32-bit row offsets take no negative strides
    assert lib.shrimp_ray_attn(ctypes.byref(ra), None) == -1
    assert b"[0, 2^31)" in lib.shrimp_last_error()
    ra.q_sn = 96
    ra.blockers = 1
    assert lib.shrimp_ray_attn(ctypes.byref(ra), None) == -1
    assert b"raylen" in lib.shrimp_last_error()
    ra.B = 0
    assert lib.shrimp_ray_attn(ctypes.byref(ra), None) == 0  # nothing to do
    prev = lib.shrimp_ray_attn_variant(1)
    assert lib.shrimp_ray_attn_variant(-1) == 1
    lib.shrimp_ray_attn_variant(prev)
    # hexfield K1: channel sets, N bound, orbit width
    assert lib.shrimp_raytap_wpack_bytes(96, 96) == 7 * 96 * 96 * 2
    assert lib.shrimp_raytap_wpack_bytes(100, 128) == 0
    assert lib.shrimp_pack_raytap_weight(16, 80, 128, 16, None) == -1
    rt = _lib.RaytapArgs(B=1, N=600, C=128, Cout=128, corb=8)
    assert lib.shrimp_conv_ln_raytap(ctypes.byref(rt), None) == -1
    assert b"N=600" in lib.shrimp_last_error()
    rt = _lib.RaytapArgs(B=1, N=64, C=128, Cout=128, corb=12, x=16, gather_idx=16, mask=16,
                         packed_w=16, bias=16, ln_w=16, ln_b=16, ray_idx=16, reach=16, alpha=16,
                         out=16, x_sb=64 * 128, x_sn=128, o_sb=64 * 128, o_sn=128, r_sn=32,
                         re_sn=12, g_sn=7)
    assert lib.shrimp_conv_ln_raytap(ctypes.byref(rt), None) == -1
    assert b"corb=12" in lib.shrimp_last_error()
    # token rows: nothing to write takes no pointers; a position stride shorter
    # than the token rows is refused, by the key-table launch that writes them too
    assert lib.shrimp_fill_tokens(None, 4, 128, None, 0, None, 0, None) == 0
    assert lib.shrimp_fill_tokens(None, 0, 128, None, 0, None, 3, None) == 0
    assert lib.shrimp_fill_tokens(None, 4, 128, None, 0, None, 3, None) == -1
    assert b"null pointer" in lib.shrimp_last_error()
    assert lib.shrimp_fill_tokens(16, 4, 128, 16, 256, None, 3, None) == -1
    assert b"position stride" in lib.shrimp_last_error()
    assert lib.shrimp_attn_keys_tokens(16, 16, 16, 3, 68, 4, 16, 16, 128, 16, 256, None,
                                       None) == -1
    assert b"position stride" in lib.shrimp_last_error()


def test_variant_switches(lib):
    """Process-wide kernel switches: valid values are set and return the
    previous one, others only query (attention: 0 auto, 1 one head, 2 two heads
    on four waves, 3 the chunked kernel)."""
    prev = lib.shrimp_attn_variant(2)
    try:
        assert lib.shrimp_attn_variant(4) == 2  # out of range: query only
        assert lib.shrimp_attn_variant(-1) == 2
        assert lib.shrimp_attn_variant(3) == 2
        assert lib.shrimp_attn_variant(-1) == 3
        assert lib.shrimp_attn_variant(2) == 3
        assert lib.shrimp_attn_variant(1) == 2
        assert lib.shrimp_attn_variant(-1) == 1
    finally:
        lib.shrimp_attn_variant(prev)
    prev = lib.shrimp_conv_variant(3)
    try:
        assert lib.shrimp_conv_variant(4) == 3
        assert lib.shrimp_conv_variant(-1) == 3
    finally:
        lib.shrimp_conv_variant(prev)


def test_host_side_under_address_and_ub_sanitizers():
    """The host side of every entry point (argument checks, extent arithmetic,
    launch wrappers, error text) built with -fsanitize=address,undefined and
    driven by tests/abi_asan.cpp: known rejections with their messages, null
    argument structs, and 2 x 20000 rounds of boundary-value argument sets
    (every call OK, EINVAL with a message or ELAUNCH; no sanitizer report)."""
    import os

    csrc = ROOT / "hexo-bot_amd" / "csrc"
    exe = ROOT / "_build" / "asan" / "abi_asan"
    subprocess.run(["make", "-C", str(csrc), "-j8", "asan"], check=True, capture_output=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    for seed in (20261202, 7):
        r = subprocess.run([str(exe), "20000", str(seed)], capture_output=True, text=True, env=env)
        if r.returncode == 2 and "GPU(s) visible" in r.stderr:
            pytest.skip("the sanitizer driver runs only where no GPU is visible")
        assert r.returncode == 0, r.stdout + r.stderr
        assert "0 failures" in r.stdout and "runtime error" not in r.stderr, r.stdout + r.stderr


def test_missing_library_raises(tmp_path):
    with pytest.raises(_lib.HipLibraryMissing):
        _lib.load(tmp_path / "nope.so")
