"""The checked build (libshrimp_hip_check.so, SHRIMP_DEBUG=1): the kernels'
input checks compiled in, a device synchronisation and a read of the fault
word after every launch.

On valid inputs it gives the release build's forward bit for bit (the checks
only read). Inputs outside a kernel's contract that the release kernels clamp
(a neighbour index below -1 reads the zero row, a sequence length past S is
cut to S) come back from the checked build as status -3 naming the failed
check, and the checked build still returns the release build's output for them.
The release library is loaded by its own path, so these tests also hold when
SHRIMP_HIP_LIB points the package at the checked build.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def libs():
    from shrimp import _lib

    if not _lib.CHECK_LIB_PATH.exists():
        pytest.fail(f"{_lib.CHECK_LIB_PATH} not built; run __graft_entry__.build()")
    _lib.load()
    return _lib, _lib.load(_lib.LIB_PATH), _lib.load(_lib.CHECK_LIB_PATH)


@pytest.fixture(autouse=True)
def _restore_library():
    """Each test switches the package's library; the next one starts from the
    default again."""
    from shrimp import _lib

    default = _lib.load()
    yield
    _lib._LIB = default


def _use(_lib, lib):
    _lib._LIB = lib


def test_checked_forward_is_bit_identical(libs):
    from shrimp import synthetic
    from shrimp.model import ShrimpNet

    _lib, release, checked = libs
    c, h, layout = 128, 8, "CCACCACCACCA"
    net = ShrimpNet(channels=c, attention_heads=h, trunk_layout=layout)
    net.load_state_dict(weights.make_state_dict(c, h, layout, seed=3, mode="heads"))
    net = net.to(DEV).eval()
    b = synthetic.position_batch("cfg4", 40, seed=11)
    args = [b[k].to(DEV) for k in ("feats", "nbr", "mask", "coords")]
    outs = []
    for lib in (release, checked):
        _use(_lib, lib)
        net.hip_runtime().invalidate()
        out = net.forward_policy_value(*args, request_moves_left=True)
        torch.cuda.synchronize()
        outs.append({k: v.clone() for k, v in out.items()})
    net.hip_runtime().invalidate()
    for key in outs[0]:
        assert torch.equal(outs[0][key], outs[1][key]), key
    assert checked.shrimp_abi_version() == 1


def _conv_args(_lib, x, idx, mask8, w, bias, out, B, N):
    return _lib.ConvArgs(
        x=x.data_ptr(), x_sb=N * 128, x_sn=128, idx=idx.data_ptr(), taps=7, idx_stride=7,
        mask=mask8.data_ptr(), w=w.data_ptr(), bias=bias.data_ptr(), relu=1,
        out=out.data_ptr(), o_sb=N * 128, o_sn=128, B=B, N=N, cin_pad=128, cout=128,
    )


def test_checked_build_reports_a_negative_neighbour_index(libs):
    """One gathered neighbour index is -7 (the reference's kernels would gather
    before the rows; absent is -1 or any index at or past N): the release conv
    reads the zero row for it, the checked build returns the same output and
    status -3 naming the conv index check."""
    from shrimp import ops

    _lib, release, checked = libs
    B, N = 4, 256
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, N, 128, generator=g).to(torch.bfloat16).to(DEV)
    idx = torch.randint(-1, N + 1, (B, N, 7), generator=g, dtype=torch.int32)
    idx[..., 0] = torch.arange(N, dtype=torch.int32)
    clean = idx.clone()
    clean[1, 17, 3] = N  # the zero row
    bad = idx.clone()
    bad[1, 17, 3] = -7
    mask8 = torch.ones(B, N, dtype=torch.uint8, device=DEV)
    w = ops.pack_conv_weight((torch.randn(7, 128, 128, generator=g) / 30).to(DEV))
    bias = (torch.randn(128, generator=g) * 0.02).to(DEV)
    outs = {}
    for name, lib, table in (("release_bad", release, bad), ("checked_clean", checked, clean),
                             ("checked_bad", checked, bad)):
        out = torch.empty(B, N, 128, dtype=torch.bfloat16, device=DEV)
        dev_idx = table.to(DEV)
        a = _conv_args(_lib, x, dev_idx, mask8, w, bias, out, B, N)
        print(f"checked build: {name}", flush=True)
        rc = lib.shrimp_hex_conv(ctypes.byref(a), ctypes.c_void_p(_lib.stream_handle()))
        torch.cuda.synchronize()
        outs[name] = (rc, lib.shrimp_last_error().decode(), out.cpu())
    assert outs["release_bad"][0] == 0
    assert outs["checked_clean"][0] == 0, outs["checked_clean"][1]
    rc, msg, got = outs["checked_bad"]
    assert rc == -3 and "conv index" in msg, (rc, msg)
    assert torch.equal(got, outs["release_bad"][2])
    assert torch.equal(got, outs["checked_clean"][2])
    # the fault word was cleared by the report: the next clean launch is OK
    a = _conv_args(_lib, x, clean.to(DEV), mask8, w, bias,
                   torch.empty(B, N, 128, dtype=torch.bfloat16, device=DEV), B, N)
    assert checked.shrimp_hex_conv(ctypes.byref(a), ctypes.c_void_p(_lib.stream_handle())) == 0


def test_checked_build_reports_a_length_past_the_sequence(libs):
    """seq_lens[b] = S + 9 through the operator attention (pair mode): the
    release kernel cuts it to S, the checked build reports it."""
    _lib, release, checked = libs
    B, H, S, d = 2, 2, 64, 16
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(B, H, S, d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    pair = torch.randint(0, 10, (B, S, S), generator=g, dtype=torch.uint8).to(DEV)
    table2 = torch.randn(10, H, generator=g).to(DEV)
    good = torch.tensor([S, 40], dtype=torch.int32, device=DEV)
    bad = torch.tensor([S + 9, 40], dtype=torch.int32, device=DEV)
    res = {}
    for name, lib, lens in (("release_bad", release, bad), ("checked_good", checked, good),
                            ("checked_bad", checked, bad)):
        _use(_lib, lib)
        print(f"checked build: attention {name}", flush=True)
        try:
            out = torch.ops.shrimp.attn_pair(q, k, v, pair, table2, lens)
            torch.cuda.synchronize()
            res[name] = (None, out.cpu())
        except RuntimeError as e:
            torch.cuda.synchronize()
            res[name] = (str(e), None)
    assert res["release_bad"][0] is None and res["checked_good"][0] is None, res
    assert torch.equal(res["release_bad"][1], res["checked_good"][1])
    err = res["checked_bad"][0]
    assert err is not None and "(-3)" in err and "sequence length" in err, err
