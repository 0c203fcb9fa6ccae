"""The phase build (libshrimp_hip_phase.so, SHRIMP_PHASE_CLOCK=1): the conv
kernels store the 100 MHz constant clock at their phase boundaries into the
buffer shrimp_phase_clock sets (unit 0), and with unit 4 also the core clock
counter beside each workgroup stamp (slot + 8). The stamps only write: the
outputs equal the release build's bit for bit. The release build refuses the
call, and so does the phase build for a unit outside 0, 1, 4, 5.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _restore_library():
    from shrimp import _lib

    default = _lib.load()
    yield
    _lib._LIB = default


def test_phase_build_stamps_and_results():
    from bench import _device_gather_index
    from shrimp import _lib, ops, synthetic

    if not _lib.PHASE_LIB_PATH.exists():
        pytest.fail(f"{_lib.PHASE_LIB_PATH} not built; run __graft_entry__.build()")
    release = _lib.load(_lib.LIB_PATH)
    phase = _lib.load(_lib.PHASE_LIB_PATH)
    # 256 positions: one big-tile workgroup per position (the stamped kernel)
    case = synthetic.conv_inputs(256, channels=128, seed=5)
    b1 = case["batch"]
    B, N = b1["mask"].shape
    x = torch.from_numpy(case["x"]).to(DEV, torch.bfloat16).contiguous()
    wp = ops.pack_conv_weight(torch.from_numpy(case["w"]).to(DEV))
    bias = torch.from_numpy(case["bias"]).to(DEV)
    gi, m8 = _device_gather_index(b1, DEV)
    stamps = torch.zeros(B * 32, dtype=torch.int64, device=DEV)

    assert release.shrimp_phase_clock(stamps.data_ptr(), 0) == -1  # no stamps in release
    assert phase.shrimp_phase_clock(stamps.data_ptr(), 2) == -1
    assert phase.shrimp_phase_clock(stamps.data_ptr(), 6) == -1

    outs, st = {}, {}
    for name, lib, unit in (("release", release, None), ("phase", phase, 0),
                            ("phase_clock", phase, 4)):
        _lib._LIB = lib
        stamps.zero_()
        if unit is not None:
            _lib.check(lib.shrimp_phase_clock(stamps.data_ptr(), unit), "phase_clock")
        out = torch.empty((B, N, 128), dtype=torch.bfloat16, device=DEV)
        print(f"phase build: conv B={B} {name}", flush=True)
        ops.launch_conv(x=x, x_sb=N * 128, x_sn=128, idx=gi, taps=7, idx_stride=7, mask8=m8,
                        wpack=wp, bias=bias, B=B, N=N, cin_pad=128, cout=128, relu=True,
                        out=out, o_sb=N * 128, o_sn=128)
        torch.cuda.synchronize()
        if unit is not None:
            _lib.check(lib.shrimp_phase_clock(None, 0), "phase_clock")
        outs[name] = out.cpu()
        st[name] = stamps.view(B, 32).cpu().clone()

    assert torch.equal(outs["phase"], outs["release"])
    assert torch.equal(outs["phase_clock"], outs["release"])
    assert (st["release"] == 0).all()
    for name in ("phase", "phase_clock"):
        s = st[name]
        # gather start, gather end (slots 0, 1), per-wave epilogue start / end
        assert (s[:, 0] > 0).all() and (s[:, 1] >= s[:, 0]).all(), name
        assert (s[:, 16] >= s[:, 1]).all() and (s[:, 24] >= s[:, 16]).all(), name
    assert (st["phase"][:, 8:10] == 0).all()  # no core clock without unit + 4
    c = st["phase_clock"]
    assert (c[:, 8] > 0).all() and (c[:, 9] > c[:, 8]).all()
    # cycles over 10 ns ticks: a core clock between 0.5 and 5 GHz
    ghz = (c[:, 9] - c[:, 8]).double().sum() / ((c[:, 1] - c[:, 0]).double().sum() * 10.0)
    assert 0.5 < float(ghz) < 5.0, float(ghz)
