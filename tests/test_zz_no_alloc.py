"""shrimp_trunk_tail_noalloc (the trunk tail with its head inputs in the
library's fixed device array instead of a caller workspace) against
shrimp_trunk_tail with a workspace: bit-identical outputs on two calls in a
row, the second with fewer positions, and a refused oversize call."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, N, C, seed):
    g = torch.Generator().manual_seed(seed)
    S = N + 8
    bins = 65
    f = lambda *s, scale=1.0: (torch.randn(*s, generator=g) * scale).to(DEV)
    seq = f(B, S, C).to(torch.bfloat16).contiguous()
    mask = (torch.rand(B, N, generator=g) > 0.3).to(torch.uint8).to(DEV)
    mask[:, 0] = 1
    return dict(
        B=B, N=N, S=S, C=C, bins=bins, seq=seq, mask=mask,
        ln_w=f(C, scale=0.2) + 1.0, ln_b=f(C, scale=0.1),
        vr_w=f(3 * C, C, scale=C ** -0.5), vr_b=f(C, scale=0.02),
        vh_w=f(C, bins, scale=C ** -0.5), vh_b=f(bins, scale=0.02),
        mr_w=f(3 * C, C, scale=C ** -0.5), mr_b=f(C, scale=0.02),
        mh_w=f(C, bins, scale=C ** -0.5), mh_b=f(bins, scale=0.02),
    )


def _run(c, noalloc):
    from shrimp import _lib

    B, S, C, bins = c["B"], c["S"], c["C"], c["bins"]
    out_seq = torch.full((B, S, C), 7.0, dtype=torch.bfloat16, device=DEV)
    value = torch.full((B, bins), 7.0, device=DEV)
    ml = torch.full((B, bins), 7.0, device=DEV)
    ws = None if noalloc else torch.empty((B, 6 * C), device=DEV)
    a = _lib.TailArgs(
        seq=c["seq"].data_ptr(), s_sb=S * C, mask=c["mask"].data_ptr(),
        ln_w=c["ln_w"].data_ptr(), ln_b=c["ln_b"].data_ptr(), eps=1e-5,
        out_seq=out_seq.data_ptr(), vr_w=c["vr_w"].data_ptr(), vr_b=c["vr_b"].data_ptr(),
        vh_w=c["vh_w"].data_ptr(), vh_b=c["vh_b"].data_ptr(), value=value.data_ptr(),
        mr_w=c["mr_w"].data_ptr(), mr_b=c["mr_b"].data_ptr(), mh_w=c["mh_w"].data_ptr(),
        mh_b=c["mh_b"].data_ptr(), moves_left=ml.data_ptr(),
        workspace=None if ws is None else ws.data_ptr(), B=B, S=S, n_tokens=8, C=C, bins=bins,
    )
    lib = _lib.load()
    fn = lib.shrimp_trunk_tail_noalloc if noalloc else lib.shrimp_trunk_tail
    _lib.check(fn(ctypes.byref(a), _lib.stream_handle()), "trunk_tail")
    torch.cuda.synchronize()
    return out_seq.cpu(), value.cpu(), ml.cpu()


def test_noalloc_tail_matches_workspace_tail():
    for B, N, C, seed in ((96, 256, 128, 1), (5, 64, 32, 2)):
        print(f"noalloc tail B={B} N={N} C={C}", flush=True)
        c = _case(B, N, C, seed)
        want = _run(c, noalloc=False)
        got = _run(c, noalloc=True)
        for w, g in zip(want, got):
            assert torch.equal(w, g)
        assert torch.isfinite(got[1]).all() and torch.isfinite(got[2]).all()


def test_noalloc_tail_refuses_oversize():
    from shrimp import _lib

    C = 128
    B = 2 * 1024 * 1024 // (6 * C) + 1  # one position past the fixed array
    dummy = torch.zeros(16, device=DEV)
    p = dummy.data_ptr()
    a = _lib.TailArgs(seq=p, s_sb=0, mask=p, ln_w=p, ln_b=p, eps=1e-5, out_seq=p, vr_w=p,
                      vr_b=p, vh_w=p, vh_b=p, value=p, mr_w=p, mr_b=p, mh_w=p, mh_b=p,
                      moves_left=p, workspace=None, B=B, S=264, n_tokens=8, C=C, bins=65)
    lib = _lib.load()
    rc = lib.shrimp_trunk_tail_noalloc(ctypes.byref(a), _lib.stream_handle())
    assert rc == -1
    assert b"exceeds the fixed scratch" in lib.shrimp_last_error()
