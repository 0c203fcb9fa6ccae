"""Eager-torch CPU restatement of the Shrimp serve forward (test infrastructure).

Follows the reference's CPU path (no Triton, no flex): the materialised
gather + GEMM conv, the pair rows built in torch (model.py:677-716), the fp16
bias gathered per block (model.py:737-760) and ``scaled_dot_product_attention``
with that bias as its mask (model.py:481-485) of
``packages/shrimp/python/shrimp/model.py``. All functions take a ``dtype``
(float64 for pinning, float32 for the CPU baseline) and plain tensors;
weights come as a state dict with the reference's keys.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import tables

NUM_TOKENS = tables.NUM_TOKENS
PAD_KEY_MASK_VALUE = -3.0e4


def _t(x, dtype):
    if isinstance(x, np.ndarray):
        x = torch.from_numpy(x)
    return x.to(dtype)


# ---- convolutions -------------------------------------------------------------------


def gather_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """x (B, N, C), idx (B, N, T) -> (B, N, T, C); indices outside [0, N) read
    the appended zero row (model.py:366-368)."""

    b, n, c = x.shape
    t = idx.shape[2]
    x_ext = torch.cat([x, x.new_zeros(b, 1, c)], dim=1)
    ii = idx.to(torch.int64)
    ii = torch.where((ii >= 0) & (ii < n), ii, torch.full_like(ii, n))
    flat = ii.reshape(b, n * t, 1).expand(-1, -1, c)
    return x_ext.gather(1, flat).reshape(b, n, t, c)


def hex_conv(x, idx, mask, weight, bias):
    """HexNodeConv.forward (model.py:346-370) for any tap count T:
    mask * (sum_t x[idx[., ., t]] @ weight[t] + bias)."""

    b, n, _ = x.shape
    t, cin, cout = weight.shape
    g = gather_rows(x, idx[:, :, :t]).reshape(b, n, t * cin)
    out = g @ weight.reshape(t * cin, cout) + bias
    return out * mask.unsqueeze(-1).to(out.dtype)


def hex_conv_ln(x, idx, mask, weight, bias, ln_w, ln_b, eps, relu):
    """shrimp::hex_conv_ln semantics (_triton_conv.py:139-196): LN over Cout
    of the conv accumulator, optional ReLU, row mask."""

    b, n, _ = x.shape
    t, cin, cout = weight.shape
    g = gather_rows(x, idx[:, :, :t]).reshape(b, n, t * cin)
    acc = g @ weight.reshape(t * cin, cout) + bias
    y = F.layer_norm(acc, (cout,), ln_w, ln_b, eps)
    if relu:
        y = F.relu(y)
    return y * mask.unsqueeze(-1).to(y.dtype)


def raytap_conv(x, ray_idx, mask, weight, bias):
    """31-tap ray conv: y = mask * (sum_{s<31} x[ray_idx[., ., s]] @ W_s + b)
    with the 32-slot index of tables.ray_index (slot 31 unused)."""

    return hex_conv(x, ray_idx[:, :, :31], mask, weight, bias)


# ---- attention -----------------------------------------------------------------------


def attention(q, k, v, bias):
    """softmax(q k^T / sqrt(d) + bias) v, q/k/v (B, H, S, d), bias (B, H, S, S)."""

    d = q.shape[-1]
    scores = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(d)) + bias
    return torch.softmax(scores, dim=-1) @ v


def attn_pair(q, k, v, pair, table2, seq_lens):
    """shrimp::attn_pair semantics (_triton_attn.py:59-130): bias =
    table2[pair, h]; keys >= seq_lens[b] excluded; query rows >= seq_lens[b]
    return 0."""

    b, h, s, d = q.shape
    bias = table2[pair.to(torch.int64)]  # (B, S, S, H)
    bias = bias.permute(0, 3, 1, 2)
    key_ok = torch.arange(s)[None, :] < seq_lens.to(torch.int64)[:, None]  # (B, S)
    bias = torch.where(key_ok[:, None, None, :], bias, torch.full_like(bias, float("-inf")))
    out = attention(q, k, v, bias)
    row_ok = key_ok[:, None, :, None]
    return torch.where(row_ok, out, torch.zeros_like(out))


def attn_offset_table(q, k, v, coords, mask, table, m):
    """Config-2 attention: bias[b, h, i, j] = table[(clamp(dq,+-m)+m)*(2m+1) +
    clamp(dr,+-m)+m, h] with (dq, dr) = coords[j] - coords[i]; keys with mask 0
    excluded; query rows with mask 0 return 0. No summary tokens."""

    w = 2 * m + 1
    c = coords.to(torch.int64)
    dq = (c[:, None, :, 0] - c[:, :, None, 0]).clamp(-m, m) + m
    dr = (c[:, None, :, 1] - c[:, :, None, 1]).clamp(-m, m) + m
    bias = table[dq * w + dr].permute(0, 3, 1, 2)  # (B, H, S, S)
    live = mask.to(torch.bool)
    bias = torch.where(live[:, None, None, :], bias, torch.full_like(bias, float("-inf")))
    out = attention(q, k, v, bias)
    return torch.where(live[:, None, :, None], out, torch.zeros_like(out))


def block_bias(table, pair, key_live, dtype):
    """Reference no-grad bias (model.py:737-760): the table is rounded to
    float16, gathered per pair from its transposed (heads, rows) copy, and
    dead keys get +(-3e4) (also in fp16). pair: (B, S, S) row indices of
    any integer dtype."""

    bias_t = table.to(torch.float16).t().contiguous()  # (H, rows)
    bias = bias_t[:, pair.to(torch.int64)].permute(1, 0, 2, 3)  # (B, H, S, S) view
    fill = torch.where(key_live, 0.0, PAD_KEY_MASK_VALUE).to(torch.float16)
    return (bias + fill[:, None, None, :]).to(dtype)


# ---- the network ---------------------------------------------------------------------------


def _lin(sd, name, x):
    return x @ sd[name + ".weight"].t() + sd[name + ".bias"]


def _ln(sd, name, x, eps=1e-5):
    c = x.shape[-1]
    return F.layer_norm(x, (c,), sd[name + ".weight"], sd[name + ".bias"], eps)


def _conv(sd, name, x, gidx, mask):
    return hex_conv(x, gidx, mask, sd[name + ".weight"], sd[name + ".bias"])


def forward_policy_value(sd, layout, heads, feats, nbr, mask, coords, *,
                         request_moves_left=False, dtype=torch.float64, return_trunk=False):
    """ShrimpNet.forward_policy_value (model.py:851-1003) on the CPU.

    sd: state dict (reference keys); feats (B, N, 15); nbr (B, N, 6) with
    sentinel N; mask (B, N) bool; coords (B, N, 2)."""

    sd = {k: _t(v, dtype) for k, v in sd.items()}
    feats = _t(feats, dtype)
    nbr = torch.as_tensor(nbr).to(torch.int64)
    mask = torch.as_tensor(mask).to(torch.bool)
    coords_np = np.asarray(coords)
    b, n, _ = feats.shape
    c = sd["tokens"].shape[1]
    h = heads
    d = c // h
    m = mask.unsqueeze(-1).to(dtype)
    gidx = torch.from_numpy(tables.gather_index(nbr.numpy()))

    x = F.relu(_ln(sd, "stem_ln", _conv(sd, "stem", feats, gidx, mask))) * m
    pair = tables.pair_rows_torch(coords_np, mask)
    key_live = torch.cat([torch.ones(b, NUM_TOKENS, dtype=torch.bool), mask], dim=1)
    seq_mask = key_live.unsqueeze(-1).to(dtype)
    tokens = sd["tokens"].unsqueeze(0).expand(b, -1, -1)
    ci = ai = 0
    seq = None
    for pos, kind in enumerate(layout):
        if kind == "C":
            p = f"conv_blocks.{ci}"
            ci += 1
            y = F.relu(_ln(sd, p + ".ln1", _conv(sd, p + ".conv1", x, gidx, mask))) * m
            y = _ln(sd, p + ".ln2", _conv(sd, p + ".conv2", y, gidx, mask)) * m
            x = F.relu(x + sd[p + ".ls.gamma"] * y)
        else:
            p = f"attn_blocks.{ai}"
            bias = block_bias(sd[f"bias_tables.{ai}"], pair, key_live, dtype)
            ai += 1
            seq = torch.cat([tokens, x], dim=1)
            s = seq.shape[1]
            z = _ln(sd, p + ".ln1", seq)
            q = _lin(sd, p + ".attn.q_proj", z).reshape(b, s, h, d).transpose(1, 2)
            k = _lin(sd, p + ".attn.k_proj", z).reshape(b, s, h, d).transpose(1, 2)
            v = _lin(sd, p + ".attn.v_proj", z).reshape(b, s, h, d).transpose(1, 2)
            # the reference's default attention impl "sdpa" (model.py:481-485)
            a = F.scaled_dot_product_attention(q, k, v, attn_mask=bias)
            a = a.transpose(1, 2).reshape(b, s, c)
            a = _lin(sd, p + ".attn.out_proj", a)
            seq = seq + sd[p + ".ls_attn.gamma"] * (a * seq_mask)
            z = _ln(sd, p + ".ln2", seq)
            mlp = _lin(sd, p + ".fc2", F.gelu(_lin(sd, p + ".fc1", z)))
            seq = seq + sd[p + ".ls_mlp.gamma"] * (mlp * seq_mask)
            if pos != len(layout) - 1:
                tokens, x = seq[:, :NUM_TOKENS], seq[:, NUM_TOKENS:]
    seq = _ln(sd, "ln_final", seq)
    tokens, cells = seq[:, :NUM_TOKENS], seq[:, NUM_TOKENS:] * m
    counts = mask.sum(dim=1, keepdim=True).clamp(min=1).to(dtype)
    pooled = (cells * m).sum(dim=1) / counts
    vin = torch.cat([tokens[:, 0], tokens[:, 1], pooled], dim=1)
    value = _lin(sd, "value_head", F.relu(_lin(sd, "value_reduction", vin)))
    y = F.relu(_conv(sd, "policy_conv", cells, gidx, mask))
    policy = _lin(sd, "policy_head", y).squeeze(-1) * mask.to(dtype)
    out = {"policy": policy, "value": value}
    if request_moves_left:
        mlin = torch.cat([tokens[:, 4], tokens[:, 5], pooled], dim=1)
        out["moves_left"] = _lin(sd, "moves_left_head", F.relu(_lin(sd, "ml_reduction", mlin)))
    if return_trunk:
        out["cells"] = cells
        out["tokens"] = tokens
    return out
