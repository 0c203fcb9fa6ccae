"""ShrimpNet with the reference's module tree, parameter names and init laws,
whose serve forward runs on the gfx950 kernels of ``libshrimp_hip.so``.

Module layout and state-dict keys follow
``packages/shrimp/python/shrimp/model.py:327-1031`` so checkpoints of the
reference load unchanged (``infer_net_kwargs_from_state_dict`` :529-555).
``forward_policy_value`` (:972-1003) is the hot path: it hands the batch to
``shrimp.runtime.HipForward``, which runs

    prep -> stem conv+LN+ReLU -> [ConvBlock | AttnBlock]* -> final LN + value
    head -> policy conv + policy head

as a fixed sequence of HIP launches on the current stream (see runtime.py).
The modules carry parameters only; there is no CPU forward in this package.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from .constants import (
    ATTENTION_HEADS,
    BIAS_ROWS,
    CHANNELS,
    MLP_RATIO,
    NUM_FEATURES,
    NUM_TOKENS,
    PAD_KEY_MASK_VALUE,
    TRUNK_LAYOUT,
    VALUE_BINS,
    validate_layout,
)
from .geometry import CELL_LUT_M, CELL_LUT_W, cell_bias_lut

STV_HORIZONS = (2, 6, 16)

__all__ = [
    "PAD_KEY_MASK_VALUE",
    "STV_HORIZONS",
    "HexNodeConv",
    "LayerScale",
    "ConvBlock",
    "RelPosAttention",
    "AttnBlock",
    "ShrimpNet",
    "KNOWN_TRUNK_LAYOUTS",
    "infer_net_kwargs_from_state_dict",
]


class HexNodeConv(nn.Module):
    """7-tap hex conv: tap 0 = the cell, taps 1-6 = DIRECTIONS (model.py:327-370).

    ``forward`` is the ``shrimp::hex_conv`` operator (bf16 output)."""

    def __init__(self, in_channels: int, out_channels: int) -> None:
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.weight = nn.Parameter(torch.empty(7, in_channels, out_channels))
        self.bias = nn.Parameter(torch.empty(out_channels))
        bound = 1.0 / math.sqrt(7 * in_channels)
        nn.init.uniform_(self.weight, -bound, bound)
        nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x, gather_idx, mask):
        return torch.ops.shrimp.hex_conv(x, gather_idx, mask, self.weight, self.bias)


class LayerScale(nn.Module):
    def __init__(self, channels: int, init: float = 1e-4) -> None:
        super().__init__()
        self.gamma = nn.Parameter(torch.full((channels,), init))

    def forward(self, x):
        return x * self.gamma


class ConvBlock(nn.Module):
    """conv1 -> LN -> ReLU -> mask -> conv2 -> LN -> mask, out = ReLU(x + gamma*y)
    (model.py:384-422)."""

    def __init__(self, channels: int) -> None:
        super().__init__()
        self.conv1 = HexNodeConv(channels, channels)
        self.ln1 = nn.LayerNorm(channels)
        self.conv2 = HexNodeConv(channels, channels)
        self.ln2 = nn.LayerNorm(channels)
        self.ls = LayerScale(channels)


class RelPosAttention(nn.Module):
    """q/k/v/out projections of the rel-pos-biased MHSA (model.py:425-492)."""

    def __init__(self, channels: int, heads: int | None = None) -> None:
        super().__init__()
        self.heads = ATTENTION_HEADS if heads is None else int(heads)
        self.head_dim = channels // self.heads
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self.q_proj = nn.Linear(channels, channels)
        self.k_proj = nn.Linear(channels, channels)
        self.v_proj = nn.Linear(channels, channels)
        self.out_proj = nn.Linear(channels, channels)
        self.impl = "hip"


class AttnBlock(nn.Module):
    """Pre-norm transformer block, MLP width MLP_RATIO * C, GELU (model.py:495-514)."""

    def __init__(self, channels: int, heads: int | None = None) -> None:
        super().__init__()
        self.ln1 = nn.LayerNorm(channels)
        self.attn = RelPosAttention(channels, heads)
        self.ln2 = nn.LayerNorm(channels)
        self.fc1 = nn.Linear(channels, MLP_RATIO * channels)
        self.fc2 = nn.Linear(MLP_RATIO * channels, channels)
        self.ls_attn = LayerScale(channels)
        self.ls_mlp = LayerScale(channels)


KNOWN_TRUNK_LAYOUTS: dict = {
    (8, 3): "CCCACCCACCA",
    (10, 5): "CCACCACCACCACCA",
}


def infer_net_kwargs_from_state_dict(sd: dict) -> dict:
    """Constructor kwargs read off a checkpoint (model.py:529-555): channels
    from stem.bias / stem_ln.weight / tokens, heads from bias_tables.0, layout
    from the conv/attn block counts of the known layouts."""

    kwargs: dict = {}
    for key, axis in (("stem.bias", 0), ("stem_ln.weight", 0), ("tokens", 1)):
        shape = getattr(sd.get(key), "shape", None)
        if shape is not None and len(shape) > axis:
            kwargs["channels"] = int(shape[axis])
            break
    bt = sd.get("bias_tables.0")
    if bt is not None and len(getattr(bt, "shape", ())) == 2:
        kwargs["attention_heads"] = int(bt.shape[1])
    conv_ids = {int(k.split(".")[1]) for k in sd if k.startswith("conv_blocks.")}
    attn_ids = {int(k.split(".")[1]) for k in sd if k.startswith("attn_blocks.")}
    if conv_ids and attn_ids:
        layout = KNOWN_TRUNK_LAYOUTS.get((max(conv_ids) + 1, max(attn_ids) + 1))
        if layout is not None:
            kwargs["trunk_layout"] = layout
    return kwargs


class ShrimpNet(nn.Module):
    """Stem, trunk layout of ConvBlocks ('C') and AttnBlocks ('A'), final LN,
    heads (model.py:558-669)."""

    def __init__(
        self,
        channels: int = CHANNELS,
        attention_heads: int | None = None,
        trunk_layout: str | None = None,
    ) -> None:
        super().__init__()
        c = int(channels)
        heads = ATTENTION_HEADS if attention_heads is None else int(attention_heads)
        layout = validate_layout(TRUNK_LAYOUT if trunk_layout is None else str(trunk_layout))
        if c % heads:
            raise ValueError(f"channels {c} not divisible by heads {heads}")
        self._trunk_layout = layout
        self.stem = HexNodeConv(NUM_FEATURES, c)
        self.stem_ln = nn.LayerNorm(c)
        self.conv_blocks = nn.ModuleList([ConvBlock(c) for _ in range(layout.count("C"))])
        self.attn_blocks = nn.ModuleList([AttnBlock(c, heads) for _ in range(layout.count("A"))])
        self.tokens = nn.Parameter(torch.empty(NUM_TOKENS, c))
        self.bias_tables = nn.ParameterList(
            [nn.Parameter(torch.zeros(BIAS_ROWS, heads)) for _ in range(len(self.attn_blocks))]
        )
        self.ln_final = nn.LayerNorm(c)
        self.policy_conv = HexNodeConv(c, c)
        self.policy_head = nn.Linear(c, 1)
        self.opp_policy_conv = HexNodeConv(c, c)
        self.opp_policy_head = nn.Linear(c, 1)
        self.soft_policy_conv = HexNodeConv(c, c)
        self.soft_policy_head = nn.Linear(c, 1)
        self.cell_q_conv = HexNodeConv(c, c)
        self.cell_q_head = nn.Linear(c, VALUE_BINS)
        self.value_reduction = nn.Linear(3 * c, c)
        self.value_head = nn.Linear(c, VALUE_BINS)
        self.aux_reduction = nn.Linear(3 * c, c)
        self.stv_heads = nn.ModuleDict({str(h): nn.Linear(c, VALUE_BINS) for h in STV_HORIZONS})
        self.ml_reduction = nn.Linear(3 * c, c)
        self.moves_left_head = nn.Linear(c, VALUE_BINS)

        self._cell_bias_M = CELL_LUT_M
        lut = torch.from_numpy(cell_bias_lut())
        self.register_buffer("_cell_bias_lut", lut.to(torch.long), persistent=False)
        self.register_buffer("_cell_bias_lut_u8", lut.clone(), persistent=False)
        self._init_weights()
        self._hip = None

    @property
    def channels(self) -> int:
        return int(self.tokens.shape[1])

    @property
    def heads(self) -> int:
        return int(self.bias_tables[0].shape[1]) if len(self.bias_tables) else ATTENTION_HEADS

    @property
    def trunk_layout(self) -> str:
        return self._trunk_layout

    def _init_weights(self) -> None:
        """Linear: trunc_normal(0.02) weight, zero bias; LayerNorm: 1 / 0;
        tokens trunc_normal(0.02); convs keep their own uniform init; bias
        tables stay zero; LayerScale stays at 1e-4 (model.py:655-669)."""

        for module in self.modules():
            if isinstance(module, nn.Linear):
                nn.init.trunc_normal_(module.weight, std=0.02)
                nn.init.zeros_(module.bias)
            elif isinstance(module, nn.LayerNorm):
                nn.init.ones_(module.weight)
                nn.init.zeros_(module.bias)
        nn.init.trunc_normal_(self.tokens, std=0.02)

    def set_attention_impl(self, impl: str) -> None:
        """Kept for API compatibility; the HIP kernel is the only implementation."""

        for block in self.attn_blocks:
            block.attn.impl = impl

    # ---- HIP forward -------------------------------------------------------------

    def hip_runtime(self):
        """The per-module runtime holding packed weights and scratch shapes."""

        if self._hip is None:
            from .runtime import HipForward

            self._hip = HipForward(self)
        return self._hip

    def refresh_weights(self) -> None:
        """Re-pack kernel weights after an in-place parameter update."""

        self.hip_runtime().invalidate()

    @torch.no_grad()
    def forward_policy_value(
        self,
        feats: torch.Tensor,
        nbr: torch.Tensor,
        mask: torch.Tensor,
        coords: torch.Tensor,
        *,
        request_moves_left: bool = False,
    ) -> dict:
        """Serve forward (model.py:972-1003): ``policy`` (B, Npad) fp32 logits,
        pad cells 0; ``value`` (B, 65) fp32 logits; ``moves_left`` (B, 65) when
        requested.

        feats (B, Npad, 15) fp32/fp16/bf16; nbr (B, Npad, 6) int64/int32 with
        sentinel Npad (or uint16 with 0xFFFF); mask (B, Npad) bool; coords
        (B, Npad, 2) int64/int32 axial."""

        return self.hip_runtime().forward(
            feats, nbr, mask, coords, request_moves_left=request_moves_left
        )

    def forward(self, feats, nbr, mask, coords):
        raise NotImplementedError(
            "ShrimpNet.forward (all training heads, with autograd) is not part of the "
            "MI355X serve build; use forward_policy_value"
        )
