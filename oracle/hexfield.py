"""CPU restatement of the two hexfield_eq serve kernels built on the 32-slot
ray gather index — TEST INFRASTRUCTURE ONLY (imported by ``tests/`` and the
``cpu_baseline`` leg of ``bench.py``; the shipped package never imports it).

  ray_attn        hexfield_eq::ray_attn: per query row and head, softmax over
                  the live ray slots of the head's win axis
                  (hexfield_eq/_triton_ray.py:377-528 kernel, :298-351 gathered
                  twin)
  conv_ln_raytap  hexfield_eq::hex_conv_ln_raytap (K1): a 7-tap conv whose six
                  direction taps are reach-masked, alpha-weighted sums over five
                  ray cells, then LayerNorm (+ReLU) and the row mask
                  (hexfield_eq/_triton_conv.py:390-499, reference :367-388,
                  _raytap.py:47-256)

Both compute in float64 (or the dtype given) from the caller's fp16 values;
the only intermediate rounding restated is the one the kernel does on purpose
(the direction-tap sums are stored as fp16 before the GEMM). How each function
is pinned (tests/test_oracle_hexfield.py):
  ray_attn        dense brute force from coordinates (the flex score_mod of
                  hexfield_eq/model.py:365-420: pair live iff self or
                  axis-aligned within reach), closed forms (raylen 0 -> v of the
                  row itself; q = 0 and zero bias -> mean of the live rows),
                  blockers off == raylen 5 everywhere
  conv_ln_raytap  alpha = (1, 0, 0, 0, 0) == the plain 7-tap hex conv + LN
                  (tests/test_hexfield_eq_raytap.py:253-266, T4); reach 5
                  everywhere == the 31-tap conv with W(d,k) = diag(alpha_k) W_d
                  (factored identity); a side's reach 0 == that side's alpha
                  columns zeroed
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .forward import gather_rows
from .tables import DIRECTIONS, RAY_AXES, RAY_SLOTS

RAY_REACH = 5
RAYLEN_SLOTS = 12


# ---- slot geometry (hexfield_eq/_raytap.py:47-107) -----------------------------------


def tap_axis_dir() -> list:
    """(axis, dir) of direction tap t = 1..6 (DIRECTIONS order): the tap's
    vector equals +axis -> dir 0, -axis -> dir 1 (_raytap.py:47-67)."""

    out = []
    for dq, dr in DIRECTIONS:
        hit = [(a, 0) for a, (aq, ar) in enumerate(RAY_AXES) if (dq, dr) == (aq, ar)]
        hit += [(a, 1) for a, (aq, ar) in enumerate(RAY_AXES) if (dq, dr) == (-aq, -ar)]
        assert len(hit) == 1
        out.append(hit[0])
    return out


def tap_raylen_slots() -> torch.Tensor:
    """(2, 6): raylen wire slot side*6 + axis*2 + dir read by (side, tap-1)
    (_raytap.py:70-80)."""

    out = torch.empty(2, 6, dtype=torch.long)
    for side in range(2):
        for t, (a, d) in enumerate(tap_axis_dir()):
            out[side, t] = side * 6 + a * 2 + d
    return out


def tap_ray_slot_lut() -> torch.Tensor:
    """(6, 5): ray slot 1 + axis*10 + dir*5 + (k-1) of the cell k steps along
    tap t (_raytap.py:83-96)."""

    out = torch.empty(6, RAY_REACH, dtype=torch.long)
    for t, (a, d) in enumerate(tap_axis_dir()):
        for k in range(1, RAY_REACH + 1):
            out[t, k - 1] = 1 + a * 10 + d * 5 + (k - 1)
    return out


def build_tap_reach(raylen: torch.Tensor) -> torch.Tensor:
    """(B, N, 12) u8 raylen -> (B, N, 2, 6) per-(side, tap) reach
    (_raytap.py:99-107)."""

    return raylen[:, :, tap_raylen_slots()]


def _slot_tables(h: int):
    """Per (head, slot): on-axis flag, step k and raylen slot, from
    _triton_ray.py:413-448 (slot 0 self, 1..30 axis*10 + dir*5 + k-1, 31 pad;
    head h rides win axis h // 2, side h % 2)."""

    on_axis = torch.zeros(h, RAY_SLOTS, dtype=torch.bool)
    kk = torch.zeros(RAY_SLOTS, dtype=torch.long)
    rl_slot = torch.zeros(h, RAY_SLOTS, dtype=torch.long)
    for s in range(1, RAY_SLOTS - 1):
        t = s - 1
        ax, dr, k = t // 10, (t % 10) // 5, t % 5 + 1
        kk[s] = k
        for hh in range(h):
            if ax == hh // 2:
                on_axis[hh, s] = True
                rl_slot[hh, s] = (hh % 2) * 6 + ax * 2 + dr
    return on_axis, kk, rl_slot


# ---- ray attention (hexfield_eq/_triton_ray.py:298-351, kernel :377-528) -------------


def ray_attn(q, k, v, idx, slot_bias, raylen, seq_lens, blockers, dtype=torch.float64):
    """q, k, v (B, H, N, D); idx (B, N, 32) (sentinel N; anything outside
    [0, N) is absent); slot_bias (32, H); raylen (B, N, 12) (read only with
    blockers); seq_lens (B,). Returns (B, H, N, D) in ``dtype``.

    Slot s of row i is live for head h when its index is present and s == 0,
    or s lies on axis h // 2 with step k <= raylen[i, side*6 + axis*2 + dir]
    (k <= 5 without blockers). score = q . k_s / sqrt(D) + slot_bias[s, h];
    out = sum_s softmax(score)_s v_s over the live slots; a row with no live
    slot, and every row >= seq_lens, is zero (the kernel's masked loads give
    zero values there)."""

    b, h, n, d = q.shape
    s = RAY_SLOTS
    ii = idx.to(torch.long)
    present = (ii >= 0) & (ii < n)
    ic = torch.where(present, ii, torch.zeros_like(ii))
    gi = ic.reshape(b, 1, n * s, 1).expand(b, h, n * s, d)
    kg = k.to(dtype).gather(2, gi).reshape(b, h, n, s, d)
    vg = v.to(dtype).gather(2, gi).reshape(b, h, n, s, d)
    scores = (q.to(dtype).unsqueeze(3) * kg).sum(-1) / math.sqrt(d)

    on_axis, kk, rl_slot = _slot_tables(h)
    if blockers:
        rl = raylen.to(torch.long)[:, :, rl_slot.reshape(-1)].reshape(b, n, h, s)
        reach_ok = kk.view(1, 1, 1, s) <= rl.permute(0, 2, 1, 3)
    else:
        reach_ok = (kk <= RAY_REACH).view(1, 1, 1, s)
    self_slot = (torch.arange(s) == 0).view(1, 1, 1, s)
    live = present[:, None] & (self_slot | (on_axis.view(1, h, 1, s) & reach_ok))
    scores = scores + slot_bias.to(dtype).t().reshape(1, h, 1, s)
    scores = torch.where(live, scores, torch.full_like(scores, -math.inf))
    m = scores.amax(-1, keepdim=True)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    p = torch.where(live, torch.exp(scores - m), torch.zeros_like(scores))
    l = p.sum(-1, keepdim=True)
    out = (p.unsqueeze(-1) * vg).sum(3) / torch.where(l > 0, l, torch.ones_like(l))
    rows = torch.arange(n).view(1, n) < seq_lens.to(torch.long).view(b, 1)
    return out * rows.view(b, 1, n, 1).to(dtype)


# ---- ray-tap conv + LN (hexfield_eq/_triton_conv.py:367-499) -------------------------


def raytap_taps(x, ray_idx, reach, alpha, corb, dtype=torch.float64, round_fp16=True):
    """(B, N, 6, C) direction-tap inputs (_raytap.py:236-256, kernel
    _triton_conv.py:441-475): tap t, channel c = sum_{k=1..5} alpha[k-1, c] *
    [k <= reach[i, side(c), t]] * x[ray_idx[i, slot(t, k)], c], side(c) =
    (c mod corb) >= corb / 2. The kernel accumulates in fp32 and stores the
    sum as fp16; ``round_fp16`` restates that store."""

    b, n, c = x.shape
    lut = tap_ray_slot_lut()
    xg = gather_rows(x.to(dtype), ray_idx.to(torch.long)[:, :, lut.reshape(-1)])
    xg = xg.reshape(b, n, 6, RAY_REACH, c)
    side = ((torch.arange(c) % corb) >= corb // 2).long()  # (C,)
    r = reach.to(torch.long)[:, :, side, :]  # (B, N, C, 6)
    ks = torch.arange(1, RAY_REACH + 1).view(1, 1, 1, RAY_REACH, 1)
    vis = (ks <= r.permute(0, 1, 3, 2).unsqueeze(3)).to(dtype)  # (B, N, 6, 5, C)
    taps = (xg * vis * alpha.to(dtype).view(1, 1, 1, RAY_REACH, c)).sum(3)
    if round_fp16:
        taps = taps.to(torch.float16).to(dtype)
    return taps


def conv_ln_raytap(x, gather_idx, mask, weight, bias, ln_w, ln_b, ray_idx, reach, alpha,
                   eps, relu, corb, dtype=torch.float64, round_fp16=True):
    """K1 (_triton_conv.py:390-499): tap 0 = x[gather_idx[., ., 0]], taps 1..6
    from :func:`raytap_taps`; conv = [tap0 | taps] @ weight.reshape(7C, Cout)
    + bias; LayerNorm over Cout (fp32 statistics in the kernel), optional
    ReLU, rows with mask 0 -> 0. Returns (B, N, Cout) in ``dtype``."""

    b, n, c = x.shape
    cout = weight.shape[-1]
    center = gather_rows(x.to(dtype), gather_idx[:, :, :1].to(torch.long))  # (B, N, 1, C)
    taps = raytap_taps(x, ray_idx, reach, alpha, corb, dtype, round_fp16)
    g = torch.cat([center, taps], dim=2).reshape(b, n, 7 * c)
    acc = g @ weight.to(dtype).reshape(7 * c, cout) + bias.to(dtype)
    y = F.layer_norm(acc, (cout,), ln_w.to(dtype), ln_b.to(dtype), eps)
    if relu:
        y = F.relu(y)
    return y * (mask.view(b, n, 1) != 0).to(dtype)
