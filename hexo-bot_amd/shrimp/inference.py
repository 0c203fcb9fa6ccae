"""ShrimpEvaluator — the serve side of the ABI-1 wire protocol on MI355X.

Restates ``packages/shrimp/python/shrimp/inference.py``: payload validation
(:509-531), padding-aware grouping ``plan_groups`` (:201-223), per-group pack
(:865-892), the forward, and the decode (:998-1042) into the reply bytes
(:806-863). The Rust caller (``payload.rs:108-160`` builds the payload,
``:164-289`` parses the reply) is unchanged.

Payload: ``abi`` == 1, ``shape`` (B, T), ``node_feats`` f16 T x 15,
``node_qr`` i16 T x 2, ``node_row_offsets`` (B+1), ``nbr`` u16 T x 6 with
0xFFFF = absent, ``legal_counts`` i32 B, ``request_moves_left``,
``request_logits``. Rows arrive sorted by support size, descending.

Reply: ``values_bytes`` f32 x B in [-1, 1]; ``priors_bytes`` f32 x sum(L),
the softmax over each row's legal prefix, rows in order; optional
``moves_left_bytes`` f32 x B and ``priors_logits_bytes`` f32 x sum(L).

The payload's CSR arrays go to the device once (pinned host copies, one
non-blocking upload each, on the evaluator's copy stream); per group the pack
into the padded forward inputs (``shrimp_prep_csr``, one kernel: sentinel
remap, masks, coordinates, sequence lengths, stem features), the forward and
the decode (``shrimp_decode``: binned value, moves-left, legal-prefix softmax
and the flat gather in one kernel) run on the current stream once the upload
is done. ``result`` waits for that payload's work only and copies its outputs
back on the copy stream, so a caller that submits the next payload before
collecting this one (as the reference's ``submit_payload`` / ``result``
pair allows) overlaps the next upload and host parse with this forward.
"""

from __future__ import annotations

import ctypes
import os
import time

import numpy as np
import torch

from . import _lib
from .constants import MOVES_LEFT_CAP, NUM_FEATURES, NUM_TOKENS, VALUE_BINS
from .model import ShrimpNet

NBR_SENTINEL = 0xFFFF
PAIR_CEILING = float(os.environ.get("SHRIMP_PAIR_CEILING", 0) or 3.8e7)
QUANT_NODES = 64
WASTE_FRACTION = float(os.environ.get("SHRIMP_WASTE_FRACTION", 0) or 0.18)


def _upload(arr: np.ndarray, dtype: torch.dtype, dev: torch.device) -> torch.Tensor:
    """Host array -> device tensor through a pinned staging copy (non-blocking)."""

    host = torch.empty(arr.shape, dtype=dtype, pin_memory=True)
    host.numpy()[...] = arr
    return host.to(dev, non_blocking=True)


def _ceil_quant(n: int) -> int:
    return max(QUANT_NODES, -(-int(n) // QUANT_NODES) * QUANT_NODES)


def assign_group_streams(costs, n_streams: int) -> list:
    """Stream slot of each group when independent group forwards are spread
    over n_streams streams: groups in order, each to the slot with the least
    work so far (cost: positions x (Npad + tokens)^2, the attention's share),
    so the large first groups land on different streams."""

    load = [0.0] * max(1, int(n_streams))
    out = []
    for c in costs:
        k = min(range(len(load)), key=lambda i: load[i])
        out.append(k)
        load[k] += float(c)
    return out


def plan_groups(sizes) -> list:
    """(start, end, pad_to) groups over size-descending rows: a group is
    anchored at its first (largest) row, padded to the 64-quantized anchor, and
    stops growing when B * (pad_to + 8)^2 would pass PAIR_CEILING or the next
    row is smaller than the anchor by more than max(64, WASTE_FRACTION * pad_to)
    (inference.py:201-223)."""

    n = len(sizes)
    groups = []
    start = 0
    while start < n:
        pad_to = _ceil_quant(int(sizes[start]))
        floor = pad_to - max(QUANT_NODES, int(WASTE_FRACTION * pad_to))
        end = start + 1
        while end < n:
            if (end - start + 1) * (pad_to + NUM_TOKENS) ** 2 > PAIR_CEILING:
                break
            if int(sizes[end]) < floor:
                break
            end += 1
        groups.append((start, end, pad_to))
        start = end
    return groups


class GpuBusyTrace:
    """Device-busy instrument of the serve loop (SHRIMP_PERF_TRACE=1), with the
    report of the reference's PerfTrace (inference.py:113-199).

    submit_payload records a timing event on the compute stream before its
    first pack and one after its last decode; result reads the pair once the
    payload's work has finished (it waits for that anyway), so tracing adds two
    event records per payload and no synchronisation. Busy fraction = summed
    device time of the payloads / wall time from the first submit to the last
    result."""

    def __init__(self) -> None:
        self.flush_ms: list = []
        self.flush_states: list = []
        self._t_first = None
        self._t_last = None

    def begin(self, stream) -> tuple:
        if self._t_first is None:
            self._t_first = time.perf_counter()
        start = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        return start, torch.cuda.Event(enable_timing=True)

    def finish(self, events, n_states: int) -> None:
        """After the payload's outputs are on the host (both events done)."""

        self._t_last = time.perf_counter()
        start, end = events
        self.flush_ms.append(float(start.elapsed_time(end)))
        self.flush_states.append(int(n_states))

    def report(self) -> dict:
        ms, st = self.flush_ms, self.flush_states
        wall = 0.0
        if self._t_first is not None and self._t_last is not None:
            wall = max(0.0, (self._t_last - self._t_first) * 1e3)
        busy_ms = float(sum(ms))
        busy = busy_ms / wall if wall > 0 else 0.0
        n, states = len(ms), int(sum(st))
        rep = {
            "gpu_busy_fraction": round(busy, 4),
            "gpu_idle_fraction": round(1.0 - busy, 4) if wall > 0 else None,
            "device_busy_ms": round(busy_ms, 2),
            "wall_window_ms": round(wall, 2),
            "measured_flushes": n,
            "measured_states": states,
            "mean_batch": round(states / n, 1) if n else 0.0,
            "mean_forward_ms": round(busy_ms / n, 3) if n else 0.0,
            "mean_ms_per_state": round(busy_ms / states, 4) if states else 0.0,
        }
        if n >= 2:
            rep["median_forward_ms"] = round(float(np.median(ms)), 3)
            rep["median_batch"] = round(float(np.median(st)), 1)
        return rep


class ShrimpEvaluator:
    """graphs: replay each group's forward from a captured HIP graph keyed by
    (batch bucket, Npad, moves-left) instead of launching its kernels one by
    one; None follows SHRIMP_CUDA_GRAPHS=1 as the reference does
    (inference.py:463-467). Groups above the largest bucket run eagerly.

    group_streams (SHRIMP_GROUP_STREAMS, default 3): the eager forwards of a
    payload's groups are independent, so when a payload has several they are
    spread over this many side streams (default priority; assign_group_streams)
    and run concurrently; small groups at large Npad leave most compute units
    idle on their own. Results are bit-identical to one stream. Three side
    streams plus the compute stream use the four hardware queues a process
    gets by default (spec-size groups of 512 positions: 80 k positions/s on one
    stream, 97 k on two, 119 k on three, 95 k on four). 1 keeps every group on
    the compute stream; captured graphs always replay in order (their buffers
    share one memory pool)."""

    def __init__(self, model: ShrimpNet, device="cuda", graphs: bool | None = None):
        self.graphs = os.environ.get("SHRIMP_CUDA_GRAPHS") == "1" if graphs is None else bool(graphs)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError(
                "ShrimpEvaluator of the MI355X build serves on a ROCm device only "
                f"(got {self.device})"
            )
        self.model = model.to(self.device).eval()
        # Uploads and reply copies of payloads submitted while another is in
        # flight run here, beside the compute (default priority, like every
        # stream of this build); a lone payload stays on the caller's stream,
        # which saves the cross-stream waits.
        self._copy_stream = None
        self._inflight = 0
        self._perf = GpuBusyTrace() if os.environ.get("SHRIMP_PERF_TRACE") == "1" else None
        self.group_streams = max(1, int(os.environ.get("SHRIMP_GROUP_STREAMS", 0) or 3))
        self._group_streams: list = []

    def _copies(self) -> torch.cuda.Stream:
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(self.device)
        return self._copy_stream

    def __call__(self, payload: dict) -> dict:
        return self.evaluate_payload(payload)

    @torch.no_grad()
    def evaluate_payload(self, payload: dict) -> dict:
        return self.result(self.submit_payload(payload))

    def perf_trace_report(self) -> dict | None:
        """GpuBusyTrace report; None unless SHRIMP_PERF_TRACE=1 (inference.py:505-507)."""

        return self._perf.report() if self._perf is not None else None

    @staticmethod
    def _parse(payload: dict):
        if int(payload["abi"]) != 1:
            raise ValueError(f"unsupported shrimp ABI {payload['abi']}")
        b, total = (int(x) for x in payload["shape"])
        offsets = np.asarray(payload["node_row_offsets"], dtype=np.int64)
        if offsets.shape[0] != b + 1 or int(offsets[-1]) != total:
            raise ValueError("node_row_offsets inconsistent with shape")
        legal = np.frombuffer(payload["legal_counts"], dtype=np.int32)
        if legal.shape[0] != b:
            raise ValueError("legal_counts byte count mismatch")
        sizes = offsets[1:] - offsets[:-1]
        if b and (sizes < 0).any():
            raise ValueError("node_row_offsets must be non-decreasing")
        if b > 1 and (sizes[1:] > sizes[:-1]).any():
            # plan_groups pads each group to its first (largest) row
            raise ValueError("rows must arrive sorted by support size, descending")
        if b and ((legal < 0) | (legal > sizes)).any():
            raise ValueError("legal_counts must lie in [0, row size]")
        feats = np.frombuffer(payload["node_feats"], dtype=np.float16)
        if feats.shape[0] != total * NUM_FEATURES:
            raise ValueError("node_feats byte count mismatch")
        qr = np.frombuffer(payload["node_qr"], dtype=np.int16)
        nbr = np.frombuffer(payload["nbr"], dtype=np.uint16)
        if qr.shape[0] != total * 2 or nbr.shape[0] != total * 6:
            raise ValueError("node_qr / nbr byte count mismatch")
        return (b, total, offsets, legal, feats.reshape(total, NUM_FEATURES),
                qr.reshape(total, 2), nbr.reshape(total, 6))

    @torch.no_grad()
    def submit_payload(self, payload: dict) -> dict:
        b, total, offsets, legal, feats, qr, nbr = self._parse(payload)
        request_ml = bool(payload.get("request_moves_left", False))
        request_logits = bool(payload.get("request_logits", False))
        dev = self.device
        sizes = offsets[1:] - offsets[:-1]
        legal64 = legal.astype(np.int64)
        flat_off = np.zeros(b + 1, dtype=np.int64)
        np.cumsum(legal64, out=flat_off[1:])
        values = torch.empty(b, dtype=torch.float32, device=dev)
        ml = torch.empty(b, dtype=torch.float32, device=dev) if request_ml else None
        priors = torch.empty(int(flat_off[-1]), dtype=torch.float32, device=dev)
        logits = torch.empty_like(priors) if request_logits else None
        compute = torch.cuda.current_stream(dev)
        copies = self._copies() if self._inflight > 0 else compute
        with torch.cuda.stream(copies):
            d_legal = _upload(legal, torch.int32, dev)
            d_off = _upload(flat_off[:-1], torch.int64, dev)
            # the CSR payload itself; u16 neighbour ids travel as their int16 bits
            d_feats = _upload(feats, torch.float16, dev)
            d_qr = _upload(qr, torch.int16, dev)
            d_nbr = _upload(nbr.view(np.int16), torch.int16, dev)
            d_rows = _upload(offsets, torch.int64, dev)
        if copies is not compute:
            compute.wait_stream(copies)
            for t in (d_legal, d_off, d_feats, d_qr, d_nbr, d_rows):
                t.record_stream(compute)
        lib = _lib.load()
        rt = self.model.hip_runtime()
        perf = self._perf.begin(compute) if self._perf is not None else None
        groups = plan_groups(sizes)
        side = []
        if not self.graphs and self.group_streams > 1 and len(groups) > 1:
            while len(self._group_streams) < self.group_streams:
                self._group_streams.append(torch.cuda.Stream(dev))
            side = self._group_streams[: self.group_streams]
            rt.weights(dev)  # packed on the compute stream, before the side streams fork
            slots = assign_group_streams(
                [(e - s) * (p + NUM_TOKENS) ** 2 for s, e, p in groups], len(side))
            for s in side:
                s.wait_stream(compute)
                # this payload's inputs and outputs stay allocated until the
                # side streams are done with them
                for t in (d_legal, d_off, d_feats, d_qr, d_nbr, d_rows, values, ml, priors, logits):
                    if t is not None:
                        t.record_stream(s)
        for i, (start, end, pad_to) in enumerate(groups):
            g = end - start
            csr = (d_feats, d_qr, d_nbr, d_rows)
            launch = side[slots[i]] if side else compute
            with torch.cuda.stream(launch):
                stream = _lib.stream_handle(dev)
                out = rt.graph_forward_csr(*csr, start, g, pad_to, request_moves_left=request_ml) \
                    if self.graphs else None
                if out is None:
                    out = rt.forward_csr(*csr, start, g, pad_to, request_moves_left=request_ml)
                pol = out["policy"]
                _lib.check(
                    lib.shrimp_decode(
                        out["value"].data_ptr(),
                        out["moves_left"].data_ptr() if request_ml else None,
                        pol.data_ptr(), pol.stride(0),
                        d_legal[start:].data_ptr(), d_off[start:].data_ptr(), g, VALUE_BINS,
                        float(MOVES_LEFT_CAP), values[start:].data_ptr(),
                        ml[start:].data_ptr() if request_ml else None,
                        priors.data_ptr(), logits.data_ptr() if request_logits else None, stream,
                    ),
                    "decode",
                )
        for s in side:
            compute.wait_stream(s)
        if perf is not None:
            perf[1].record(compute)
        done = torch.cuda.Event()
        done.record(compute)
        self._inflight += 1
        return {
            "b": b, "request_ml": request_ml, "request_logits": request_logits,
            "values_gpu": values, "ml_gpu": ml, "priors_gpu": priors, "logits_gpu": logits,
            "done": done, "perf": perf,
        }

    @torch.no_grad()
    def result(self, handle: dict) -> dict:
        """Waits for this payload's work (not for payloads submitted after it)
        and returns its reply bytes."""

        names = [("values_bytes", "values_gpu")]
        names.append(("priors_bytes", "priors_gpu"))
        if handle["request_ml"]:
            names.append(("moves_left_bytes", "ml_gpu"))
        if handle["request_logits"]:
            names.append(("priors_logits_bytes", "logits_gpu"))
        self._inflight = max(0, self._inflight - 1)
        if self._inflight == 0:
            # nothing was submitted after this payload: copy on its own stream
            reply = {key: handle[src].cpu().numpy().astype(np.float32, copy=False).tobytes()
                     for key, src in names}
            self._trace(handle)
            return reply
        copies = self._copies()
        host = {}
        with torch.cuda.stream(copies):
            copies.wait_event(handle["done"])
            for key, src in names:
                t = handle[src]
                h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
                h.copy_(t, non_blocking=True)
                t.record_stream(copies)
                host[key] = h
            fetched = torch.cuda.Event()
            fetched.record(copies)
        fetched.synchronize()
        self._trace(handle)
        return {key: host[key].numpy().astype(np.float32, copy=False).tobytes() for key, _ in names}

    def _trace(self, handle: dict) -> None:
        if self._perf is not None and handle.get("perf") is not None:
            handle["perf"][1].synchronize()
            self._perf.finish(handle["perf"], handle["b"])
