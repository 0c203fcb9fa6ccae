"""Seeded ShrimpNet state dicts with the reference's keys (test infrastructure).

Every tensor comes from its own numpy PCG64 stream (seed mixed with the CRC32
of the key), so the same weights are rebuilt bit-identically by the golden
generator, the CPU oracle, the GPU tests and the benchmark's baseline leg —
no torch RNG involved.

``mode="fresh"``: the reference init laws (model.py:334-344, 373-381,
593-600, 655-669): conv U(+-1/sqrt(7 cin)); Linear N(0, 0.02) weights (the
+-2 truncation of trunc_normal_ never binds at std 0.02), zero biases;
LayerNorm 1 / 0; tokens N(0, 0.02); bias tables 0; LayerScale 1e-4.
``mode="parity"``: every branch made non-inert for numerical tests, in the
spirit of tests/test_shrimp_model.py:45-57: LayerNorm weights U(0.5, 1.5) and
biases N(0, 0.1), Linear biases N(0, 0.02), out_proj / fc2 N(0, 0.05),
bias tables N(0, 0.5), LayerScale U(0.5, 1.0).
``mode="heads"``: as "parity", with the serve heads' Linear weights N(0,
1 / fan_in) for the value / moves-left reduction and head and N(0, 1 / (4
fan_in)) for the policy head, so value logits are O(1) and policy logits
O(0.5): an absolute logit gate then sees an error in the trunk (with std
0.02 heads the logits are O(0.05) and a 2e-2 gate cannot).
"""

from __future__ import annotations

import zlib

import numpy as np
import torch

NUM_FEATURES = 15
NUM_TOKENS = 8
VALUE_BINS = 65
BIAS_ROWS = 237
STV_HORIZONS = (2, 6, 16)
# Linear layers of the serve heads (model.py:990-1020): O(1) weights in "heads" mode.
SERVE_HEADS = ("policy_head", "value_reduction", "value_head", "ml_reduction", "moves_left_head")


def param_shapes(channels: int, heads: int, layout: str) -> dict:
    """Ordered {key: (shape, kind)} of the reference ShrimpNet
    (model.py:584-623); kind in conv_w, conv_b, lin_w, lin_b, ln_w, ln_b,
    gamma, tokens, table."""

    c = channels
    s: dict = {}

    def conv(name, cin, cout):
        s[name + ".weight"] = ((7, cin, cout), "conv_w")
        s[name + ".bias"] = ((cout,), "conv_b")

    def lin(name, fin, fout):
        s[name + ".weight"] = ((fout, fin), "lin_w")
        s[name + ".bias"] = ((fout,), "lin_b")

    def ln(name):
        s[name + ".weight"] = ((c,), "ln_w")
        s[name + ".bias"] = ((c,), "ln_b")

    conv("stem", NUM_FEATURES, c)
    ln("stem_ln")
    for i in range(layout.count("C")):
        p = f"conv_blocks.{i}"
        conv(p + ".conv1", c, c)
        ln(p + ".ln1")
        conv(p + ".conv2", c, c)
        ln(p + ".ln2")
        s[p + ".ls.gamma"] = ((c,), "gamma")
    for i in range(layout.count("A")):
        p = f"attn_blocks.{i}"
        ln(p + ".ln1")
        for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
            lin(f"{p}.attn.{proj}", c, c)
        ln(p + ".ln2")
        lin(p + ".fc1", c, 2 * c)
        lin(p + ".fc2", 2 * c, c)
        s[p + ".ls_attn.gamma"] = ((c,), "gamma")
        s[p + ".ls_mlp.gamma"] = ((c,), "gamma")
    s["tokens"] = ((NUM_TOKENS, c), "tokens")
    for i in range(layout.count("A")):
        s[f"bias_tables.{i}"] = ((BIAS_ROWS, heads), "table")
    ln("ln_final")
    conv("policy_conv", c, c)
    lin("policy_head", c, 1)
    conv("opp_policy_conv", c, c)
    lin("opp_policy_head", c, 1)
    conv("soft_policy_conv", c, c)
    lin("soft_policy_head", c, 1)
    conv("cell_q_conv", c, c)
    lin("cell_q_head", c, VALUE_BINS)
    lin("value_reduction", 3 * c, c)
    lin("value_head", c, VALUE_BINS)
    lin("aux_reduction", 3 * c, c)
    for hz in STV_HORIZONS:
        lin(f"stv_heads.{hz}", c, VALUE_BINS)
    lin("ml_reduction", 3 * c, c)
    lin("moves_left_head", c, VALUE_BINS)
    return s


def make_state_dict(channels: int, heads: int, layout: str, seed: int = 0,
                    mode: str = "parity") -> dict:
    if mode not in ("parity", "fresh", "heads"):
        raise ValueError(mode)
    out = {}
    for key, (shape, kind) in param_shapes(channels, heads, layout).items():
        rng = np.random.Generator(np.random.PCG64((seed * 1000003) ^ zlib.crc32(key.encode())))
        if kind in ("conv_w", "conv_b"):
            cin = shape[1] if kind == "conv_w" else None
            if cin is None:
                cin = NUM_FEATURES if key.startswith("stem.") else channels
            bound = 1.0 / np.sqrt(7 * cin)
            v = rng.uniform(-bound, bound, size=shape)
        elif kind == "lin_w":
            std = 0.05 if (mode != "fresh" and (".out_proj." in key or ".fc2." in key)) else 0.02
            if mode == "heads" and key.split(".")[0] in SERVE_HEADS:
                std = (0.5 if key.startswith("policy_head.") else 1.0) / np.sqrt(shape[1])
            v = rng.normal(0.0, std, size=shape)
        elif kind == "lin_b":
            v = rng.normal(0.0, 0.02, size=shape) if mode != "fresh" else np.zeros(shape)
        elif kind == "ln_w":
            v = rng.uniform(0.5, 1.5, size=shape) if mode != "fresh" else np.ones(shape)
        elif kind == "ln_b":
            v = rng.normal(0.0, 0.1, size=shape) if mode != "fresh" else np.zeros(shape)
        elif kind == "gamma":
            v = rng.uniform(0.5, 1.0, size=shape) if mode != "fresh" else np.full(shape, 1e-4)
        elif kind == "tokens":
            v = rng.normal(0.0, 0.02, size=shape)
        elif kind == "table":
            v = rng.normal(0.0, np.sqrt(0.5), size=shape) if mode != "fresh" else np.zeros(shape)
        else:  # pragma: no cover
            raise AssertionError(kind)
        out[key] = torch.from_numpy(np.asarray(v, dtype=np.float32))
    return out
