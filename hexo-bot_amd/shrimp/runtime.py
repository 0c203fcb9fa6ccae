"""HipForward: the serve forward of ShrimpNet as a fixed sequence of gfx950
kernel launches on the current HIP stream.

Device layout of one batch (B positions, N = Npad cells, S = N + 8 rows):

    seq   (B, S, C)  bf16  residual stream; rows 0..7 are the summary tokens,
                           rows 8.. the cells (the reference's cat([tokens, x]),
                           model.py:921-926, kept in place instead of re-built)
    y1    (B, N, C)  bf16  first conv of a ConvBlock
    qkv   (3, B, H, S, dpad) bf16 head-major projections
    att   (B, S, C)  bf16  attention output, heads concatenated
    hid   (B, S, 2C) bf16  MLP hidden (unfused MLP path only)
    seqf  (B, S, C)  bf16  after the final LayerNorm (cells masked)

Kernel sequence (reference lines in model.py):
    prep_inputs          gather_idx / mask / coords / seq_lens / padded feats  :861-892
    hex_conv  (stem)     conv + LN + ReLU + mask                               :865
    per 'C': hex_conv x2 conv1+LN+ReLU+mask -> y1; conv2+LN+mask, ReLU(x+g*y)  :395-422
             (one conv_block launch per 'C', one conv_block_pair per 'CC')
    per 'A': attn_qkv (LN1, q/k/v) -> attn -> attn_mlp (out_proj, residual, LN2,
             fc1, GELU, fc2, residual; three linear launches when C != 128)   :448-514
    trunk_tail           final LN, pooled mean, value / moves-left heads       :927-935, 990-1002
    hex_conv  (policy)   conv + ReLU + Linear(C,1) + mask                      :1011-1020
Weights are packed once into MFMA fragment order (bf16) and re-packed when
any parameter changes (tracked through tensor version counters).

precision "fp32" (the reference's serve with autocast off,
inference.py:50-68) runs the same sequence on the fp32 kernels: fp32
activations end to end (seq, y1, qkv, att, hid, seqf all fp32); the GEMMs
whose input width is a multiple of 32 on bf16 MFMA over hi / lo split
operands (three products per tile, about 2^-16 relative error per product),
only the 16-channel stem on fp32 MFMA; the head-dim-16 coords attention on
the split-operand MFMA kernel, other head dims and pair mode on the chunked
fp32 kernel; the bias tables rounded to fp16 as the reference's no-grad bias
is (model.py:737-760).
"""

from __future__ import annotations

import ctypes
import os
from types import SimpleNamespace

import torch

from . import _lib
from .constants import NUM_TOKENS, VALUE_BINS
from .geometry import CELL_LUT_M
from .ops import (
    attn_bias_table,
    attn_keys_ints,
    attn_staged_supported,
    conv_block_pair_supported,
    conv_block_supported,
    attn_fused_supported,
    launch_attn,
    launch_attn_fused,
    launch_attn_keys,
    launch_attn_mlp,
    launch_attn_qkv,
    launch_attn_qkv_kvf,
    launch_attn_staged,
    launch_conv,
    launch_conv_block,
    launch_conv_block_pair,
    launch_linear,
    pack_attn_mlp,
    pack_attn_qkv,
    pack_conv_weight,
    pack_linear_weight,
    require_device,
)

_NBR_DT = {
    torch.int64: _lib.DT_I64,
    torch.int32: _lib.DT_I32,
    torch.uint16: _lib.DT_U16,
}
_FEAT_DT = {
    torch.float32: _lib.DT_F32,
    torch.float16: _lib.DT_F16,
    torch.bfloat16: _lib.DT_BF16,
}
_COORD_DT = {torch.int64: _lib.DT_I64, torch.int32: _lib.DT_I32}


def head_dim_pad(d: int) -> int:
    return max(16, -(-d // 16) * 16)


def default_precision() -> str:
    """"bf16" unless SHRIMP_SERVE_AUTOCAST=0 (the reference's switch for an
    fp32 serve on CUDA devices, inference.py:50-68), then "fp32"."""

    return "fp32" if os.environ.get("SHRIMP_SERVE_AUTOCAST", "1") == "0" else "bf16"


PRECISIONS = ("bf16", "fp32")


class HipForward:
    def __init__(self, net) -> None:
        self.net = net
        self._packed = None
        self._key = None
        # When set, the device buffers of the last forward stay referenced in
        # ``self.last`` (used to re-launch single kernels for timing).
        self.keep_buffers = False
        self.last = None
        # The unclamped offset table lets the attention kernel index biases
        # linearly for compact positions; off forces the clamped LUT path.
        self.use_linear_bias = True
        # Fused out_proj + MLP kernel where it applies; off runs the three
        # linear kernels (used to check one against the other).
        self.use_fused_mlp = True
        # Two consecutive ConvBlocks in one launch (the first one's output
        # rows handed to the second inside the workgroup) where it applies;
        # off runs one launch per block (bit-identical).
        self.use_block_pair = True
        # Final LayerNorm, pooled head inputs and policy conv in one launch
        # (the normalised cells never leave the workgroup) where it applies;
        # off, and whenever keep_buffers asks for seqf, runs shrimp_trunk_tail
        # and the policy conv (bit-identical outputs).
        self.use_fused_tail = True
        # LN1 + q/k/v kernel with LN1 folded into its weights where it
        # applies; off runs the linear kernel's QKV mode.
        self.use_fused_qkv = True
        # LN1 + q/k/v projection inside the attention kernel (no q/k/v
        # tensor, 3 x B x S x C bf16 less memory) where it applies; off (the
        # default: about 1% faster at B=512) runs the q/k/v kernel, then
        # attention.
        self.use_fused_attn = False
        # Staged attention where it applies (C = 128, H = 8, the LINEAR
        # table): the q/k/v kernel writes K and V in the attention kernel's
        # fragment order and a once-per-forward key table replaces the
        # per-workgroup key setup, so the attention kernel stages by DMA;
        # off runs the (3, B, H, S, dpad) layout and the in-kernel setup.
        self.use_staged_attn = True
        # ConvBlock as one launch (conv1's output kept in LDS) where a fused
        # kernel exists; off runs the two convolutions.
        self.use_fused_block = True
        # Batch size from which the one-workgroup-per-position kernels run
        # (None: above half the compute units).
        self.fused_min_batch = None
        self._cu_cache: dict = {}
        # Captured forwards (graph_forward_csr), keyed by (batch bucket, Npad,
        # moves-left, device); dropped when a parameter changes.
        self._graphs: dict = {}
        self._graph_params = None
        self._graph_pool = None
        self._empty_rows: dict = {}
        # "bf16" (bf16 activations, fp32 accumulation) or "fp32"
        self.precision = default_precision()
        # Largest batch of one forward launch sequence (None: the buffer limit
        # below); forward() splits larger batches into independent slices.
        self.max_batch = None
        # When a list, eager forwards append (name, event) after each launch
        # (HIP events on the launch stream) so a caller can read per-kernel
        # times inside a real forward; None (the default) records nothing.
        self.timeline = None

    def _mark(self, name: str) -> None:
        if self.timeline is not None:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self.timeline.append((name, ev))

    def _cus(self, dev) -> int:
        """Compute units of the device. Batches of at most half that many
        positions run ConvBlocks as two row-split convolutions (same bits as the
        fused block): the fused block gives each position one workgroup and
        would leave most units idle."""

        if dev.index not in self._cu_cache:
            self._cu_cache[dev.index] = torch.cuda.get_device_properties(dev).multi_processor_count
        return self._cu_cache[dev.index]

    def _fused_batch(self, B: int, N: int, dev) -> bool:
        """Whether a batch of B positions at Npad = N takes the
        one-workgroup-per-position kernels (fused ConvBlock, block pair, policy
        tail), or ``fused_min_batch`` positions when that is set. Up to 256
        cells a fused workgroup is two waves and two fit a compute unit, so the
        row-split convolutions win until the batch passes half the compute
        units. Past 256 cells a fused workgroup is three or four waves with the
        unit's LDS to itself, while the row split stages the whole position
        once per 64-row tile and runs ceil(B N / 64 / CUs) rounds of those:
        measured at Npad 512 (whole forward), 40 positions 0.91 ms either way,
        98 positions 1.15 ms fused against 1.67 ms split, 128 positions 1.25
        against 1.71 ms; 16 positions 0.73 against 0.54 ms."""

        if self.fused_min_batch is not None:
            return B >= self.fused_min_batch
        if N > 256:
            return B >= 40
        return 2 * B > self._cus(dev)

    def invalidate(self) -> None:
        self._packed = None
        self._key = None

    def _param_key(self, device) -> tuple:
        return (str(device), self.precision) + tuple(
            (p.data_ptr(), p._version) for p in self.net.parameters()
        )

    @property
    def fp32(self) -> bool:
        if self.precision not in PRECISIONS:
            raise ValueError(f"HipForward.precision must be one of {PRECISIONS}, "
                             f"not {self.precision!r}")
        return self.precision == "fp32"

    def weights(self, device: torch.device) -> SimpleNamespace:
        key = self._param_key(device)
        if self._packed is not None and key == self._key:
            return self._packed
        self._packed = self._pack32(device) if self.fp32 else self._pack(device)
        self._key = key
        return self._packed

    @torch.no_grad()
    def _pack(self, device: torch.device) -> SimpleNamespace:
        net = self.net

        def f32(t):
            return t.detach().to(device=device, dtype=torch.float32).contiguous()

        def conv_w(conv, cin_pad=None):
            return pack_conv_weight(conv.weight.detach().to(device), cin_pad)

        def lin_w(lin):
            return pack_linear_weight(lin.weight.detach().to(device))

        c = net.channels
        P = SimpleNamespace()
        P.C, P.H = c, net.heads
        P.d = c // P.H
        P.dpad = head_dim_pad(P.d)
        P.layout = net.trunk_layout
        P.stem = SimpleNamespace(
            w=conv_w(net.stem, 32), b=f32(net.stem.bias), lnw=f32(net.stem_ln.weight),
            lnb=f32(net.stem_ln.bias), eps=net.stem_ln.eps,
        )
        P.convs = []
        for blk in net.conv_blocks:
            P.convs.append(
                SimpleNamespace(
                    w1=conv_w(blk.conv1), b1=f32(blk.conv1.bias), ln1w=f32(blk.ln1.weight),
                    ln1b=f32(blk.ln1.bias), eps1=blk.ln1.eps,
                    w2=conv_w(blk.conv2), b2=f32(blk.conv2.bias), ln2w=f32(blk.ln2.weight),
                    ln2b=f32(blk.ln2.bias), eps2=blk.ln2.eps, gamma=f32(blk.ls.gamma),
                )
            )
        lut = net._cell_bias_lut_u8.to(device)
        P.lut = lut
        P.attn = []
        for i, blk in enumerate(net.attn_blocks):
            at = blk.attn
            qkv_w = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight], 0)
            qkv_b = torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias], 0)
            P.attn.append(
                SimpleNamespace(
                    ln1w=f32(blk.ln1.weight), ln1b=f32(blk.ln1.bias), eps1=blk.ln1.eps,
                    qkv_w=pack_linear_weight(qkv_w.detach().to(device)), qkv_b=f32(qkv_b),
                    # LN1 + q/k/v as one kernel with LN1 folded into the
                    # weights where it applies (C = 128); else None
                    qkv=pack_attn_qkv(qkv_w.to(device), qkv_b.to(device), blk.ln1.weight,
                                      blk.ln1.bias),
                    out_w=lin_w(at.out_proj), out_b=f32(at.out_proj.bias),
                    ln2w=f32(blk.ln2.weight), ln2b=f32(blk.ln2.bias), eps2=blk.ln2.eps,
                    fc1_w=lin_w(blk.fc1), fc1_b=f32(blk.fc1.bias),
                    fc2_w=lin_w(blk.fc2), fc2_b=f32(blk.fc2.bias),
                    # out_proj + MLP as one fused kernel where its weights fit
                    # one workgroup's LDS (C = 128, hidden = 2C); else None
                    mlp=pack_attn_mlp(at.out_proj.weight, at.out_proj.bias, blk.ls_attn.gamma,
                                      blk.ln2.weight, blk.ln2.bias, blk.fc1.weight, blk.fc1.bias,
                                      blk.fc2.weight, blk.fc2.bias, blk.ls_mlp.gamma),
                    g_attn=f32(blk.ls_attn.gamma), g_mlp=f32(blk.ls_mlp.gamma),
                    btab_xtab=attn_bias_table(net.bias_tables[i].detach().to(device), lut,
                                              CELL_LUT_M),
                )
            )
        P.fused_mlp = all(a.mlp is not None for a in P.attn)
        P.fused_qkv = all(a.qkv is not None for a in P.attn)
        P.tokens = f32(net.tokens)
        P.lnf = SimpleNamespace(w=f32(net.ln_final.weight), b=f32(net.ln_final.bias),
                                eps=net.ln_final.eps)
        # head weights transposed (k-major) for the tail kernel
        P.value = SimpleNamespace(
            rw=f32(net.value_reduction.weight.t()), rb=f32(net.value_reduction.bias),
            hw=f32(net.value_head.weight.t()), hb=f32(net.value_head.bias),
        )
        P.ml = SimpleNamespace(
            rw=f32(net.ml_reduction.weight.t()), rb=f32(net.ml_reduction.bias),
            hw=f32(net.moves_left_head.weight.t()), hb=f32(net.moves_left_head.bias),
        )
        P.policy = SimpleNamespace(
            w=conv_w(net.policy_conv), b=f32(net.policy_conv.bias),
            hw=f32(net.policy_head.weight.reshape(-1)), hb=f32(net.policy_head.bias.reshape(-1)),
        )
        return P

    @torch.no_grad()
    def _pack32(self, device: torch.device) -> SimpleNamespace:
        """fp32 weights in the fp32 kernels' fragment order."""

        net = self.net
        lib = _lib.load()
        st = _lib.stream_handle(device)

        def f32(t):
            return t.detach().to(device=device, dtype=torch.float32).contiguous()

        def conv_w(conv, cin_pad=None):
            w = f32(conv.weight)
            t, cin, cout = w.shape
            cp = -(-cin // 16) * 16 if cin_pad is None else cin_pad
            out = torch.empty(t * cp * cout, dtype=torch.float32, device=device)
            _lib.check(lib.shrimp_pack_conv_weight_f32(w.data_ptr(), out.data_ptr(), t, cin, cp,
                                                       cout, st), "pack_conv_weight_f32")
            torch.cuda.current_stream(device).synchronize()  # w dies with this frame
            return out

        def lin_w(weight):
            w = f32(weight)
            n_out, n_in = w.shape
            out = torch.empty(n_in * n_out, dtype=torch.float32, device=device)
            _lib.check(lib.shrimp_pack_linear_weight_f32(w.data_ptr(), out.data_ptr(), n_in, n_out,
                                                         st), "pack_linear_weight_f32")
            torch.cuda.current_stream(device).synchronize()
            return out

        c = net.channels
        P = SimpleNamespace()
        P.C, P.H = c, net.heads
        P.d = c // P.H
        if P.d % 4:
            raise ValueError(f"fp32 serve: head dim {P.d} must be a multiple of 4")
        P.layout = net.trunk_layout
        P.stem = SimpleNamespace(
            w=conv_w(net.stem, 16), b=f32(net.stem.bias), lnw=f32(net.stem_ln.weight),
            lnb=f32(net.stem_ln.bias), eps=net.stem_ln.eps,
        )
        P.convs = [
            SimpleNamespace(
                w1=conv_w(blk.conv1), b1=f32(blk.conv1.bias), ln1w=f32(blk.ln1.weight),
                ln1b=f32(blk.ln1.bias), eps1=blk.ln1.eps,
                w2=conv_w(blk.conv2), b2=f32(blk.conv2.bias), ln2w=f32(blk.ln2.weight),
                ln2b=f32(blk.ln2.bias), eps2=blk.ln2.eps, gamma=f32(blk.ls.gamma),
            )
            for blk in net.conv_blocks
        ]
        lut = net._cell_bias_lut_u8.to(device)
        P.attn = []
        for i, blk in enumerate(net.attn_blocks):
            at = blk.attn
            qkv_w = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight], 0)
            qkv_b = torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias], 0)
            # the reference's no-grad bias rounds the block's table to fp16
            table = net.bias_tables[i].detach().to(device).half().float()
            P.attn.append(
                SimpleNamespace(
                    ln1w=f32(blk.ln1.weight), ln1b=f32(blk.ln1.bias), eps1=blk.ln1.eps,
                    qkv_w=lin_w(qkv_w), qkv_b=f32(qkv_b),
                    out_w=lin_w(at.out_proj.weight), out_b=f32(at.out_proj.bias),
                    ln2w=f32(blk.ln2.weight), ln2b=f32(blk.ln2.bias), eps2=blk.ln2.eps,
                    fc1_w=lin_w(blk.fc1.weight), fc1_b=f32(blk.fc1.bias),
                    fc2_w=lin_w(blk.fc2.weight), fc2_b=f32(blk.fc2.bias),
                    g_attn=f32(blk.ls_attn.gamma), g_mlp=f32(blk.ls_mlp.gamma),
                    btab=attn_bias_table(table, lut, CELL_LUT_M)[0],
                )
            )
        P.tokens = f32(net.tokens)
        P.lnf = SimpleNamespace(w=f32(net.ln_final.weight), b=f32(net.ln_final.bias),
                                eps=net.ln_final.eps)
        P.value = SimpleNamespace(
            rw=f32(net.value_reduction.weight.t()), rb=f32(net.value_reduction.bias),
            hw=f32(net.value_head.weight.t()), hb=f32(net.value_head.bias),
        )
        P.ml = SimpleNamespace(
            rw=f32(net.ml_reduction.weight.t()), rb=f32(net.ml_reduction.bias),
            hw=f32(net.moves_left_head.weight.t()), hb=f32(net.moves_left_head.bias),
        )
        P.policy = SimpleNamespace(
            w=conv_w(net.policy_conv), b=f32(net.policy_conv.bias),
            hw=f32(net.policy_head.weight.reshape(-1)), hb=f32(net.policy_head.bias.reshape(-1)),
        )
        return P

    def _prep_buffers(self, B: int, N: int, dev) -> SimpleNamespace:
        i32, u8 = torch.int32, torch.uint8
        S = N + NUM_TOKENS
        f32 = self.fp32
        return SimpleNamespace(
            idx=torch.empty((B, N, 7), dtype=i32, device=dev),
            mask8=torch.empty((B, N), dtype=u8, device=dev),
            coords32=torch.empty((B, N, 2), dtype=i32, device=dev),
            seq_lens=torch.empty((B,), dtype=i32, device=dev),
            seq_mask=torch.empty((B, S), dtype=u8, device=dev),
            # stem input: bf16 (B, N, 32), or fp32 (B, N, 16) in the fp32 mode
            xin=None if f32 else torch.empty((B, N, 32), dtype=torch.bfloat16, device=dev),
            xin32=torch.empty((B, N, 16), dtype=torch.float32, device=dev) if f32 else None,
        )

    @torch.no_grad()
    def forward_csr(self, node_feats, node_qr, nbr, row_offsets, row0: int, B: int, N: int, *,
                    request_moves_left: bool = False) -> dict:
        """Forward over rows row0 .. row0 + B - 1 of ABI-1 payload arrays already on
        the device (node_feats (T, 15) f16, node_qr (T, 2) i16, nbr (T, 6) u16,
        row_offsets (rows + 1) int64), padded to N cells on the device
        (inference.py:865-892 / serve_pack.rs:155-216 in one kernel)."""

        require_device(node_feats, "HipForward.forward_csr")
        dev = node_feats.device
        for t, dt in ((node_feats, torch.float16), (node_qr, torch.int16), (nbr, torch.int16),
                      (row_offsets, torch.int64)):
            if t.dtype not in (dt, torch.uint16) or not t.is_contiguous() or t.device != dev:
                raise TypeError(f"forward_csr: {t.dtype} {tuple(t.shape)} is not a contiguous {dt} "
                                f"tensor on {dev}")
        if node_feats.dim() != 2 or node_feats.shape[1] > 32:
            raise ValueError("forward_csr: node_feats must be (T, F) with F <= 32")
        if row0 < 0 or row0 + B + 1 > row_offsets.shape[0]:
            raise ValueError("forward_csr: rows outside row_offsets")
        lim = self.batch_limit(N)
        if B > lim:
            parts = [self.forward_csr(node_feats, node_qr, nbr, row_offsets, row0 + i,
                                      min(lim, B - i), N, request_moves_left=request_moves_left)
                     for i in range(0, B, lim)]
            return {k: torch.cat([p[k] for p in parts]) for k in parts[0]}
        lib = _lib.load()
        st = _lib.stream_handle(dev)
        pb = self._prep_buffers(B, N, dev)
        self._prep_csr_rows(pb, 0, B, N, (node_feats, node_qr, nbr, row_offsets), row0, st)
        return self._trunk(pb, B, N, dev, request_moves_left)

    # ---- graph-captured serve forward (the reference's _GraphCache,
    # inference.py:226-352): one captured trunk per (batch bucket, Npad,
    # moves-left); the device pack runs eagerly into the capture's static
    # input buffers, pad rows of the bucket carry the pad convention.
    GRAPH_MAX_B = 260

    @staticmethod
    def graph_bucket(b: int):
        """Batch size of the captured forward serving b rows (multiples of 4)."""

        bb = max(4, -(-b // 4) * 4)
        return bb if bb <= HipForward.GRAPH_MAX_B else None

    def _prep_csr_rows(self, pb, lo: int, hi: int, N: int, csr, row0: int, st) -> None:
        """shrimp_prep_csr of rows row0.. into batch rows [lo, hi) of pb."""

        node_feats, node_qr, nbr, row_offsets = csr
        lib = _lib.load()
        _lib.check(
            lib.shrimp_prep_csr(
                node_feats.data_ptr(), node_feats.shape[1], node_qr.data_ptr(), nbr.data_ptr(),
                row_offsets.data_ptr(), row0, hi - lo, N, NUM_TOKENS, pb.idx[lo:].data_ptr(),
                pb.mask8[lo:].data_ptr(), pb.coords32[lo:].data_ptr(), pb.seq_lens[lo:].data_ptr(),
                pb.seq_mask[lo:].data_ptr(), None if pb.xin is None else pb.xin[lo:].data_ptr(),
                st,
            ),
            "prep_csr",
        )
        if pb.xin32 is not None:
            _lib.check(
                lib.shrimp_prep_csr_feats_f32(
                    node_feats.data_ptr(), node_feats.shape[1], row_offsets.data_ptr(), row0,
                    hi - lo, N, pb.xin32[lo:].data_ptr(), st,
                ),
                "prep_csr_feats_f32",
            )

    def _empty_csr(self, dev):
        """CSR arrays of rows with no cells: packing them writes pad rows."""

        e = self._empty_rows.get(dev)
        if e is None:
            e = (torch.zeros((1, 15), dtype=torch.float16, device=dev),
                 torch.zeros((1, 2), dtype=torch.int16, device=dev),
                 torch.zeros((1, 6), dtype=torch.int16, device=dev),
                 torch.zeros((self.GRAPH_MAX_B + 1,), dtype=torch.int64, device=dev))
            self._empty_rows[dev] = e
        return e

    @torch.no_grad()
    def graph_forward_csr(self, node_feats, node_qr, nbr, row_offsets, row0: int, B: int, N: int,
                          *, request_moves_left: bool = False):
        """forward_csr through a captured HIP graph; None when B is above the
        largest bucket (the caller runs forward_csr). The returned tensors are
        views of the capture's static outputs, and all captures share one
        memory pool: they are valid until the next graph replay of any bucket,
        so a caller consumes them (or clones) before that."""

        bb = self.graph_bucket(B)
        if bb is None:
            return None
        dev = node_feats.device
        key_p = self._param_key(dev)
        if key_p != self._graph_params:
            self._graphs.clear()
            self._graph_params = key_p
        key = (bb, N, bool(request_moves_left), dev)
        ent = self._graphs.get(key)
        st = _lib.stream_handle(dev)
        if ent is None:
            self.weights(dev)  # pack outside the capture
            pb = self._prep_buffers(bb, N, dev)
            self._prep_csr_rows(pb, 0, bb, N, self._empty_csr(dev), 0, st)
            keep, self.keep_buffers = self.keep_buffers, False
            tl, self.timeline = self.timeline, None
            try:
                cur = torch.cuda.current_stream(dev)
                side = torch.cuda.Stream(dev)
                side.wait_stream(cur)
                with torch.cuda.stream(side):
                    for _ in range(2):
                        self._trunk(pb, bb, N, dev, request_moves_left)
                cur.wait_stream(side)
                if self._graph_pool is None:
                    self._graph_pool = torch.cuda.graph_pool_handle()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self._graph_pool):
                    out = self._trunk(pb, bb, N, dev, request_moves_left)
            finally:
                self.keep_buffers = keep
                self.timeline = tl
            ent = SimpleNamespace(graph=graph, pb=pb, out=out, filled=0)
            self._graphs[key] = ent
            st = _lib.stream_handle(dev)
        self._prep_csr_rows(ent.pb, 0, B, N, (node_feats, node_qr, nbr, row_offsets), row0, st)
        if ent.filled > B:  # rows a larger group left behind go back to pad rows
            self._prep_csr_rows(ent.pb, B, ent.filled, N, self._empty_csr(dev), 0, st)
        ent.filled = B
        ent.graph.replay()
        return {k: v[:B] for k, v in ent.out.items()}

    # Kernels address activation rows through buffer resources with 32-bit
    # byte offsets: every activation buffer of one launch stays below this.
    BUFFER_LIMIT = 0x7FFF0000

    def batch_limit(self, N: int) -> int:
        """Positions one forward can take at Npad = N: every per-batch buffer
        whose byte extent a kernel checks against BUFFER_LIMIT stays under it at
        that batch. The widest per position are the MLP hidden rows (S, 2C), the
        three q / k / v planes (3, H, S, dpad) of the unstaged attention (the
        fused q/k/v kernel checks all three planes as one extent; the fp32 mode
        keeps the same planes in fp32) and the staged attention's K / V
        fragments (H, 2, SP, 16); the bound takes the largest of them whichever
        attention path the forward takes. max_batch caps it further."""

        net = self.net
        c, h = net.channels, net.heads
        dpad = head_dim_pad(c // h)
        elem = 4 if self.fp32 else 2
        s = N + NUM_TOKENS
        sp = (s + 15) // 16 * 16
        per = max(s * 2 * c * elem, 3 * h * s * dpad * elem, h * sp * 64)
        lim = max(1, (self.BUFFER_LIMIT - 1) // per)
        return lim if self.max_batch is None else max(1, min(lim, int(self.max_batch)))

    @torch.no_grad()
    def forward(self, feats, nbr, mask, coords, *, request_moves_left: bool = False) -> dict:
        require_device(feats, "ShrimpNet.forward_policy_value")
        dev = feats.device
        B, N, F = feats.shape
        lim = self.batch_limit(N)
        if B > lim:
            # rows are independent (per-position LayerNorm, masks, attention):
            # slices of at most `lim` positions give the same rows
            parts = [self.forward(feats[i:i + lim], nbr[i:i + lim], mask[i:i + lim],
                                  coords[i:i + lim], request_moves_left=request_moves_left)
                     for i in range(0, B, lim)]
            return {k: torch.cat([p[k] for p in parts]) for k in parts[0]}
        if nbr.dtype not in _NBR_DT or feats.dtype not in _FEAT_DT or coords.dtype not in _COORD_DT:
            raise TypeError(
                f"unsupported dtypes feats={feats.dtype} nbr={nbr.dtype} coords={coords.dtype}"
            )
        if tuple(nbr.shape) != (B, N, 6) or tuple(mask.shape) != (B, N) or tuple(coords.shape) != (B, N, 2):
            raise ValueError("feats/nbr/mask/coords shapes disagree")
        lib = _lib.load()
        st = _lib.stream_handle(dev)
        feats_c = feats.contiguous()
        nbr_c = nbr.contiguous()
        mask_c = mask.contiguous()
        if mask_c.dtype not in (torch.bool, torch.uint8):
            mask_c = mask_c.to(torch.bool)
        coords_c = coords.contiguous()

        pb = self._prep_buffers(B, N, dev)
        _lib.check(
            lib.shrimp_prep_inputs(
                nbr_c.data_ptr(), _NBR_DT[nbr_c.dtype], mask_c.data_ptr(), coords_c.data_ptr(),
                _COORD_DT[coords_c.dtype], feats_c.data_ptr(), _FEAT_DT[feats_c.dtype], F, B, N,
                NUM_TOKENS, pb.idx.data_ptr(), pb.mask8.data_ptr(), pb.coords32.data_ptr(),
                pb.seq_lens.data_ptr(), pb.seq_mask.data_ptr(), _lib.ptr(pb.xin), st,
            ),
            "prep_inputs",
        )
        if pb.xin32 is not None:
            _lib.check(
                lib.shrimp_prep_feats_f32(feats_c.data_ptr(), _FEAT_DT[feats_c.dtype], F, B, N,
                                          pb.xin32.data_ptr(), st),
                "prep_feats_f32",
            )
        return self._trunk(pb, B, N, dev, request_moves_left)

    def _trunk(self, pb: SimpleNamespace, B: int, N: int, dev, request_moves_left: bool) -> dict:
        """Everything after the input preparation: stem, blocks, tail, heads."""

        if self.fp32:
            return self._trunk32(pb, B, N, dev, request_moves_left)
        P = self.weights(dev)
        C, H, d, dpad = P.C, P.H, P.d, P.dpad
        S = N + NUM_TOKENS
        lib = _lib.load()
        st = _lib.stream_handle(dev)
        bf = torch.bfloat16
        idx, mask8, coords32 = pb.idx, pb.mask8, pb.coords32
        seq_lens, seq_mask, xin = pb.seq_lens, pb.seq_mask, pb.xin
        seq = torch.empty((B, S, C), dtype=bf, device=dev)
        # the token rows' residual stream is seq (bf16) + tok_lo (bf16): the
        # rounding remainder of every update, kept by the residual kernels
        tok_lo = torch.empty((B, NUM_TOKENS, C), dtype=bf, device=dev)
        cells = seq[:, NUM_TOKENS:]
        y1 = torch.empty((B, N, C), dtype=bf, device=dev)
        attn_fused = (P.fused_qkv and self.use_fused_qkv and self.use_fused_attn
                      and attn_fused_supported(C, H, S, dpad))
        staged = (not attn_fused and P.fused_qkv and self.use_fused_qkv and self.use_staged_attn
                  and self.use_linear_bias and d == dpad and attn_staged_supported(H, S, dpad))
        qkv = kvf = meta = None
        if staged:
            sp = (S + 15) // 16 * 16
            qkv = torch.empty((1, B, H, S, dpad), dtype=bf, device=dev)
            kvf = torch.empty((B, H, 2, sp, 16), dtype=bf, device=dev)
            meta = torch.empty((B, attn_keys_ints(S)), dtype=torch.int32, device=dev)
        elif not attn_fused:
            qkv = (torch.zeros if d != dpad else torch.empty)((3, B, H, S, dpad), dtype=bf, device=dev)
        att = torch.empty((B, S, C), dtype=bf, device=dev)
        fused = P.fused_mlp and self.use_fused_mlp
        hid = None if fused else torch.empty((B, S, 2 * C), dtype=bf, device=dev)

        conv_common = dict(idx=idx, taps=7, idx_stride=7, mask8=mask8, B=B, N=N, stream=st)
        self._mark("start")
        if staged:
            # the key table and the token rows in one launch
            launch_attn_keys(coords=coords32, mask8=mask8, seq_lens=seq_lens, B=B, S=S,
                             n_tokens=NUM_TOKENS, meta=meta, tokens=P.tokens, seq=seq,
                             seq_sb=S * C, tok_lo=tok_lo, stream=st)
            self._mark("attn_keys")
        else:
            _lib.check(
                lib.shrimp_fill_tokens(P.tokens.data_ptr(), NUM_TOKENS, C, seq.data_ptr(), S * C,
                                       tok_lo.data_ptr(), B, st),
                "fill_tokens",
            )
            self._mark("fill_tokens")
        launch_conv(
            x=xin, x_sb=N * 32, x_sn=32, wpack=P.stem.w, bias=P.stem.b, cin_pad=32, cout=C,
            ln_w=P.stem.lnw, ln_b=P.stem.lnb, eps=P.stem.eps, relu=True,
            out=cells, o_sb=S * C, o_sn=C, **conv_common,
        )
        self._mark("stem")
        ci = ai = 0
        rows = B * S
        fused_block = self.use_fused_block and self._fused_batch(B, N, dev) and conv_block_supported(7, N, C, C)
        pair_ok = fused_block and self.use_block_pair and conv_block_pair_supported(7, N, C, C)
        skip = False
        for li, kind in enumerate(P.layout):
            if skip:
                skip = False
                continue
            if kind == "C":
                k = P.convs[ci]
                ci += 1
                if pair_ok and P.layout[li + 1:li + 2] == "C":
                    k2 = P.convs[ci]
                    ci += 1
                    skip = True
                    blocks = [dict(w1=q.w1, b1=q.b1, ln1_w=q.ln1w, ln1_b=q.ln1b, eps1=q.eps1, w2=q.w2,
                                   b2=q.b2, ln2_w=q.ln2w, ln2_b=q.ln2b, eps2=q.eps2, gamma=q.gamma)
                              for q in (k, k2)]
                    launch_conv_block_pair(
                        x=cells, x_sb=S * C, x_sn=C, idx=idx, idx_stride=7, mask8=mask8, B=B, N=N,
                        C=C, blocks=blocks, out=cells, o_sb=S * C, o_sn=C, stream=st,
                    )
                    self._mark("conv_block_pair")
                    continue
                if fused_block:
                    launch_conv_block(
                        x=cells, x_sb=S * C, x_sn=C, idx=idx, idx_stride=7, mask8=mask8, B=B,
                        N=N, C=C, w1=k.w1, b1=k.b1, ln1_w=k.ln1w, ln1_b=k.ln1b, eps1=k.eps1,
                        w2=k.w2, b2=k.b2, ln2_w=k.ln2w, ln2_b=k.ln2b, eps2=k.eps2,
                        gamma=k.gamma, out=cells, o_sb=S * C, o_sn=C, stream=st,
                    )
                    self._mark("conv_block")
                    continue
                launch_conv(
                    x=cells, x_sb=S * C, x_sn=C, wpack=k.w1, bias=k.b1, cin_pad=C, cout=C,
                    ln_w=k.ln1w, ln_b=k.ln1b, eps=k.eps1, relu=True,
                    out=y1, o_sb=N * C, o_sn=C, **conv_common,
                )
                self._mark("conv1")
                launch_conv(
                    x=y1, x_sb=N * C, x_sn=C, wpack=k.w2, bias=k.b2, cin_pad=C, cout=C,
                    ln_w=k.ln2w, ln_b=k.ln2b, eps=k.eps2, relu=False,
                    resid=cells, r_sb=S * C, r_sn=C, gamma=k.gamma,
                    out=cells, o_sb=S * C, o_sn=C, **conv_common,
                )
                self._mark("conv2")
            else:
                a = P.attn[ai]
                ai += 1
                bias_args = dict(
                    seq_lens=seq_lens, o=att, o_sb=S * C, o_sh=d, o_sr=C, B=B, S=S, H=H, d=d,
                    dpad=dpad, coords=coords32, mask8=mask8, btab=a.btab_xtab[0],
                    xtab=a.btab_xtab[1] if self.use_linear_bias else None, lut_m=CELL_LUT_M,
                    n_tokens=NUM_TOKENS, stream=st,
                )
                if attn_fused:
                    launch_attn_fused(x=seq, x_sb=S * C, x_sr=C, packed=a.qkv, eps=a.eps1,
                                      **bias_args)
                    self._mark("attn_fused")
                elif staged:
                    launch_attn_qkv_kvf(x=seq, x_sr=C, q=qkv, kvf=kvf, packed=a.qkv, eps=a.eps1,
                                        rows=rows, B=B, S=S, H=H, C=C, dpad=dpad, stream=st)
                    self._mark("qkv")
                    launch_attn_staged(
                        q=qkv, qkv_sb=H * S * dpad, qkv_sh=S * dpad, kvf=kvf, meta=meta,
                        seq_lens=seq_lens, o=att, o_sb=S * C, o_sh=d, o_sr=C, B=B, S=S, H=H, d=d,
                        dpad=dpad, btab=a.btab_xtab[0], xtab=a.btab_xtab[1], lut_m=CELL_LUT_M,
                        n_tokens=NUM_TOKENS, stream=st,
                    )
                    self._mark("attn")
                elif P.fused_qkv and self.use_fused_qkv:
                    launch_attn_qkv(x=seq, x_sr=C, qkv=qkv, packed=a.qkv, eps=a.eps1, rows=rows,
                                    B=B, S=S, H=H, C=C, dpad=dpad, stream=st)
                    self._mark("qkv")
                else:
                    launch_linear(
                        x=seq, x_sr=C, wpack=a.qkv_w, bias=a.qkv_b, rows=rows, n_in=C,
                        n_out=3 * C, mode=_lib.LIN_QKV, out=qkv, ln_w=a.ln1w, ln_b=a.ln1b,
                        eps=a.eps1, B=B, S=S, H=H, dpad=dpad, stream=st,
                    )
                    self._mark("qkv")
                if not attn_fused and not staged:
                    launch_attn(q=qkv[0], k=qkv[1], v=qkv[2], qkv_sb=H * S * dpad,
                                qkv_sh=S * dpad, **bias_args)
                    self._mark("attn")
                if fused:
                    launch_attn_mlp(
                        x=att, x_sr=C, seq=seq, s_sr=C, mask=seq_mask, packed=a.mlp,
                        eps=a.eps2, rows=rows, C=C, hidden=2 * C, tok_lo=tok_lo, S=S,
                        n_tokens=NUM_TOKENS, stream=st,
                    )
                    self._mark("mlp")
                    continue
                launch_linear(
                    x=att, x_sr=C, wpack=a.out_w, bias=a.out_b, rows=rows, n_in=C, n_out=C,
                    mode=_lib.LIN_RESID, out=seq, o_sr=C, resid=seq, r_sr=C, gamma=a.g_attn,
                    mask=seq_mask, S=S, tok_lo=tok_lo, n_tokens=NUM_TOKENS, stream=st,
                )
                launch_linear(
                    x=seq, x_sr=C, wpack=a.fc1_w, bias=a.fc1_b, rows=rows, n_in=C, n_out=2 * C,
                    mode=_lib.LIN_GELU, out=hid, o_sr=2 * C, ln_w=a.ln2w, ln_b=a.ln2b,
                    eps=a.eps2, stream=st,
                )
                launch_linear(
                    x=hid, x_sr=2 * C, wpack=a.fc2_w, bias=a.fc2_b, rows=rows, n_in=2 * C,
                    n_out=C, mode=_lib.LIN_RESID, out=seq, o_sr=C, resid=seq, r_sr=C,
                    gamma=a.g_mlp, mask=seq_mask, S=S, tok_lo=tok_lo, n_tokens=NUM_TOKENS,
                    stream=st,
                )
                self._mark("mlp")

        seqf = torch.empty((B, S, C), dtype=bf, device=dev)
        value = torch.empty((B, VALUE_BINS), dtype=torch.float32, device=dev)
        ml = torch.empty((B, VALUE_BINS), dtype=torch.float32, device=dev) if request_moves_left else None
        tail_ws = torch.empty((B, 6 * C), dtype=torch.float32, device=dev)
        tail = _lib.TailArgs(
            seq=seq.data_ptr(), s_sb=S * C, mask=mask8.data_ptr(), ln_w=P.lnf.w.data_ptr(),
            ln_b=P.lnf.b.data_ptr(), eps=float(P.lnf.eps), out_seq=seqf.data_ptr(),
            vr_w=P.value.rw.data_ptr(), vr_b=P.value.rb.data_ptr(), vh_w=P.value.hw.data_ptr(),
            vh_b=P.value.hb.data_ptr(), value=value.data_ptr(),
            mr_w=P.ml.rw.data_ptr(), mr_b=P.ml.rb.data_ptr(), mh_w=P.ml.hw.data_ptr(),
            mh_b=P.ml.hb.data_ptr(), moves_left=_lib.ptr(ml), workspace=tail_ws.data_ptr(),
            B=B, S=S, n_tokens=NUM_TOKENS, C=C, bins=VALUE_BINS, tok_lo=tok_lo.data_ptr(),
        )
        policy = torch.empty((B, N), dtype=torch.float32, device=dev)
        if (self.use_fused_tail and not self.keep_buffers and self._fused_batch(B, N, dev)
                and lib.shrimp_policy_tail_supported(N, C)):
            pa = _lib.ConvArgs(
                x=seq.data_ptr() + NUM_TOKENS * C * seq.element_size(), x_sb=S * C, x_sn=C,
                idx=idx.data_ptr(), taps=7, idx_stride=7, mask=mask8.data_ptr(),
                w=P.policy.w.data_ptr(), bias=P.policy.b.data_ptr(), relu=1,
                head_w=P.policy.hw.data_ptr(), head_b=P.policy.hb.data_ptr(),
                head_out=policy.data_ptr(), B=B, N=N, cin_pad=C, cout=C,
            )
            _lib.check(lib.shrimp_policy_tail(ctypes.byref(pa), ctypes.byref(tail), st), "policy_tail")
            self._mark("policy_tail")
        else:
            _lib.check(lib.shrimp_trunk_tail(ctypes.byref(tail), st), "trunk_tail")
            self._mark("tail")
            launch_conv(
                x=seqf[:, NUM_TOKENS:], x_sb=S * C, x_sn=C, wpack=P.policy.w, bias=P.policy.b,
                cin_pad=C, cout=C, relu=True, head_w=P.policy.hw, head_b=P.policy.hb,
                head_out=policy, **conv_common,
            )
            self._mark("policy")
        out = {"policy": policy, "value": value}
        if request_moves_left:
            out["moves_left"] = ml
        if self.keep_buffers:
            self.last = dict(
                P=P, B=B, N=N, S=S, idx=idx, mask8=mask8, coords32=coords32, seq_lens=seq_lens,
                seq_mask=seq_mask, seq=seq, y1=y1, qkv=qkv, att=att, hid=hid, seqf=seqf,
                stream=st, attn_fused=attn_fused, staged=staged, kvf=kvf, meta=meta,
                tok_lo=tok_lo,
            )
        return out

    def _trunk32(self, pb: SimpleNamespace, B: int, N: int, dev, request_moves_left: bool) -> dict:
        """The fp32 serve mode's trunk: the launch sequence of _trunk on the fp32
        kernels (model.py:395-514, 905-1020), fp32 activations throughout."""

        P = self.weights(dev)
        C, H, d = P.C, P.H, P.d
        S = N + NUM_TOKENS
        lib = _lib.load()
        st = _lib.stream_handle(dev)
        f = torch.float32
        idx, mask8, coords32 = pb.idx, pb.mask8, pb.coords32
        seq_lens, seq_mask = pb.seq_lens, pb.seq_mask
        seq = torch.empty((B, S, C), dtype=f, device=dev)
        _lib.check(lib.shrimp_fill_tokens_f32(P.tokens.data_ptr(), NUM_TOKENS, C, seq.data_ptr(),
                                              S * C, B, st), "fill_tokens_f32")
        cells = seq[:, NUM_TOKENS:]
        y1 = torch.empty((B, N, C), dtype=f, device=dev)
        qkv = torch.empty((3, B, H, S, d), dtype=f, device=dev)
        att = torch.empty((B, S, C), dtype=f, device=dev)
        hid = torch.empty((B, S, 2 * C), dtype=f, device=dev)
        rows = B * S

        def conv(x, x_sb, x_sn, w, b, cin_pad, **kw):
            a = _lib.ConvArgs(
                x=x.data_ptr(), x_sb=x_sb, x_sn=x_sn, idx=idx.data_ptr(), taps=7, idx_stride=7,
                mask=mask8.data_ptr(), w=w.data_ptr(), bias=b.data_ptr(),
                ln_w=_lib.ptr(kw.get("ln_w")), ln_b=_lib.ptr(kw.get("ln_b")),
                eps=float(kw.get("eps", 1e-5)), relu=int(bool(kw.get("relu", False))),
                resid=_lib.ptr(kw.get("resid")), r_sb=S * C, r_sn=C,
                gamma=_lib.ptr(kw.get("gamma")), head_w=_lib.ptr(kw.get("head_w")),
                head_b=_lib.ptr(kw.get("head_b")), head_out=_lib.ptr(kw.get("head_out")),
                out=_lib.ptr(kw.get("out")), o_sb=kw.get("o_sb", 0), o_sn=kw.get("o_sn", 0),
                B=B, N=N, cin_pad=cin_pad, cout=C,
            )
            _lib.check(lib.shrimp_hex_conv_f32(ctypes.byref(a), st), "hex_conv_f32")

        def linear(x, x_sr, w, b, n_in, n_out, mode, out, o_sr=0, **kw):
            a = _lib.LinearArgs(
                x=x.data_ptr(), x_sr=x_sr, w=w.data_ptr(), bias=b.data_ptr(),
                ln_w=_lib.ptr(kw.get("ln_w")), ln_b=_lib.ptr(kw.get("ln_b")),
                eps=float(kw.get("eps", 1e-5)), mode=mode, resid=_lib.ptr(kw.get("resid")),
                r_sr=kw.get("r_sr", 0), gamma=_lib.ptr(kw.get("gamma")),
                mask=_lib.ptr(kw.get("mask")), out=out.data_ptr(), o_sr=o_sr, rows=rows,
                in_features=n_in, out_features=n_out, B=B, S=S, H=H, dpad=d,
            )
            _lib.check(lib.shrimp_linear_f32(ctypes.byref(a), st), "linear_f32")

        self._mark("start")
        conv(pb.xin32, N * 16, 16, P.stem.w, P.stem.b, 16, ln_w=P.stem.lnw, ln_b=P.stem.lnb,
             eps=P.stem.eps, relu=True, out=cells, o_sb=S * C, o_sn=C)
        self._mark("stem")
        ci = ai = 0
        for kind in P.layout:
            if kind == "C":
                k = P.convs[ci]
                ci += 1
                conv(cells, S * C, C, k.w1, k.b1, C, ln_w=k.ln1w, ln_b=k.ln1b, eps=k.eps1,
                     relu=True, out=y1, o_sb=N * C, o_sn=C)
                self._mark("conv1")
                conv(y1, N * C, C, k.w2, k.b2, C, ln_w=k.ln2w, ln_b=k.ln2b, eps=k.eps2,
                     resid=cells, gamma=k.gamma, out=cells, o_sb=S * C, o_sn=C)
                self._mark("conv2")
                continue
            a = P.attn[ai]
            ai += 1
            linear(seq, C, a.qkv_w, a.qkv_b, C, 3 * C, _lib.LIN_QKV, qkv, ln_w=a.ln1w,
                   ln_b=a.ln1b, eps=a.eps1)
            self._mark("qkv")
            at = _lib.AttnArgs(
                q=qkv[0].data_ptr(), k=qkv[1].data_ptr(), v=qkv[2].data_ptr(), qkv_sb=H * S * d,
                qkv_sh=S * d, seq_lens=seq_lens.data_ptr(), pair=None, p_sb=0, p_sq=0,
                table2=None, table_rows=0, coords=coords32.data_ptr(), mask=mask8.data_ptr(),
                btab=a.btab.data_ptr(), xtab=None, lut_m=CELL_LUT_M, n_tokens=NUM_TOKENS,
                o=att.data_ptr(), o_sb=S * C, o_sh=d, o_sr=C, B=B, S=S, H=H, d=d, dpad=d,
            )
            _lib.check(lib.shrimp_attn_f32(ctypes.byref(at), st), "attn_f32")
            self._mark("attn")
            linear(att, C, a.out_w, a.out_b, C, C, _lib.LIN_RESID, seq, o_sr=C, resid=seq, r_sr=C,
                   gamma=a.g_attn, mask=seq_mask)
            linear(seq, C, a.fc1_w, a.fc1_b, C, 2 * C, _lib.LIN_GELU, hid, o_sr=2 * C,
                   ln_w=a.ln2w, ln_b=a.ln2b, eps=a.eps2)
            linear(hid, 2 * C, a.fc2_w, a.fc2_b, 2 * C, C, _lib.LIN_RESID, seq, o_sr=C, resid=seq,
                   r_sr=C, gamma=a.g_mlp, mask=seq_mask)
            self._mark("mlp")

        seqf = torch.empty((B, S, C), dtype=f, device=dev)
        value = torch.empty((B, VALUE_BINS), dtype=f, device=dev)
        ml = torch.empty((B, VALUE_BINS), dtype=f, device=dev) if request_moves_left else None
        tail_ws = torch.empty((B, 6 * C), dtype=f, device=dev)
        tail = _lib.TailArgs(
            seq=seq.data_ptr(), s_sb=S * C, mask=mask8.data_ptr(), ln_w=P.lnf.w.data_ptr(),
            ln_b=P.lnf.b.data_ptr(), eps=float(P.lnf.eps), out_seq=seqf.data_ptr(),
            vr_w=P.value.rw.data_ptr(), vr_b=P.value.rb.data_ptr(), vh_w=P.value.hw.data_ptr(),
            vh_b=P.value.hb.data_ptr(), value=value.data_ptr(),
            mr_w=P.ml.rw.data_ptr(), mr_b=P.ml.rb.data_ptr(), mh_w=P.ml.hw.data_ptr(),
            mh_b=P.ml.hb.data_ptr(), moves_left=_lib.ptr(ml), workspace=tail_ws.data_ptr(),
            B=B, S=S, n_tokens=NUM_TOKENS, C=C, bins=VALUE_BINS,
        )
        _lib.check(lib.shrimp_trunk_tail_f32(ctypes.byref(tail), st), "trunk_tail_f32")
        self._mark("tail")
        policy = torch.empty((B, N), dtype=f, device=dev)
        conv(seqf[:, NUM_TOKENS:], S * C, C, P.policy.w, P.policy.b, C, relu=True,
             head_w=P.policy.hw, head_b=P.policy.hb, head_out=policy)
        self._mark("policy")
        out = {"policy": policy, "value": value}
        if request_moves_left:
            out["moves_left"] = ml
        if self.keep_buffers:
            self.last = dict(
                P=P, B=B, N=N, S=S, idx=idx, mask8=mask8, coords32=coords32, seq_lens=seq_lens,
                seq_mask=seq_mask, seq=seq, y1=y1, qkv=qkv, att=att, hid=hid, seqf=seqf,
                stream=st, attn_fused=False,
            )
        return out
