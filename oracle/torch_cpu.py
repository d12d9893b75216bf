"""Torch fp32 CPU restatement of the UNet and the VQ decoder -- the CPU BASELINE of
``bench.py`` (test infrastructure only; see ``oracle/__init__.py``).

The reference's own CPU path is MLX on ``mx.cpu`` (macOS arm64 only), which cannot run
here. This module is the stand-in the benchmark plan names: the same layer graph as
``oracle.unet`` (mlx_model.py:420-654, 720-819), each op a torch CPU kernel in float32 on
channels-last-3d tensors, so that a configuration's CPU time is that of an optimised CPU
framework rather than of the float64 checker. ``tests/test_oracle.py`` pins it against
``oracle.unet`` on small networks.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from .unet import UPSAMPLE_CONV, UnetConfig


class TorchLayers:
    """Source-keyed float32 layers on the CPU."""

    def __init__(self, weights: dict[str, np.ndarray]):
        self.w = {k: torch.from_numpy(np.asarray(v, np.float32)) for k, v in weights.items()}

    def conv(self, x: torch.Tensor, key: str, *, stride: int = 1, shift: torch.Tensor | None = None,
             residual: torch.Tensor | None = None) -> torch.Tensor:
        w = self.w[key + ".weight"]
        b = self.w.get(key + ".bias")
        k = w.shape[2]
        y = F.conv3d(x, w, b, stride=stride, padding=k // 2)
        if shift is not None:
            y = y + shift[:, :, None, None, None]
        if residual is not None:
            y = y + residual
        return y.contiguous(memory_format=torch.channels_last_3d)

    def upsample_conv(self, x: torch.Tensor, key: str) -> torch.Tensor:
        return self.conv(F.interpolate(x, scale_factor=2, mode="nearest"), key)

    def dense(self, x: torch.Tensor, key: str) -> torch.Tensor:
        return F.linear(x, self.w[key + ".weight"], self.w.get(key + ".bias"))

    def norm(self, x: torch.Tensor, key: str, *, groups: int, eps: float) -> torch.Tensor:
        return F.group_norm(x, groups, self.w[key + ".weight"], self.w[key + ".bias"], eps)

    def norm_silu_conv(self, x, norm_key, conv_key, *, groups, eps, shift=None, residual=None):
        return self.conv(F.silu(self.norm(x, norm_key, groups=groups, eps=eps)), conv_key, shift=shift,
                         residual=residual)

    def layer_norm(self, x: torch.Tensor, key: str, eps: float = 1e-5) -> torch.Tensor:
        w = self.w[key + ".weight"]
        return F.layer_norm(x, (w.shape[0],), w, self.w[key + ".bias"], eps)


def _groups(c: int) -> int:
    return 32 if c % 32 == 0 else c


class TorchUnet(TorchLayers):
    """``oracle.unet.Unet`` in torch fp32 on the CPU (mlx_model.py:420-654)."""

    def __init__(self, weights: dict[str, np.ndarray], cfg: UnetConfig):
        super().__init__(weights)
        self.cfg = cfg

    def residual(self, x, emb, key):
        shift = self.dense(F.silu(emb), key + ".emb_layers.1")
        h = self.norm_silu_conv(x, key + ".in_layers.0", key + ".in_layers.2", groups=_groups(x.shape[1]),
                                eps=1e-5, shift=shift)
        if key + ".skip_connection.weight" in self.w:
            x = self.conv(x, key + ".skip_connection")
        return self.norm_silu_conv(h, key + ".out_layers.0", key + ".out_layers.3", groups=_groups(h.shape[1]),
                                   eps=1e-5, residual=x)

    def attention(self, x, context, key, heads):
        ctx = x if context is None else context
        q, k, v = self.dense(x, key + ".to_q"), self.dense(ctx, key + ".to_k"), self.dense(ctx, key + ".to_v")
        b, lq, c = q.shape
        d = c // heads
        split = lambda t: t.reshape(b, t.shape[1], heads, d).transpose(1, 2)
        o = F.scaled_dot_product_attention(split(q), split(k), split(v), scale=d ** -0.5)
        return self.dense(o.transpose(1, 2).reshape(b, lq, c), key + ".to_out.0")

    def transformer(self, x, context, key):
        residual = x
        h = self.conv(self.norm(x, key + ".norm", groups=32, eps=1e-6), key + ".proj_in")
        b, c = h.shape[:2]
        sp = h.shape[2:]
        t = h.permute(0, 2, 3, 4, 1).reshape(b, -1, c)
        heads = c // self.cfg.num_head_channels
        blk = key + ".transformer_blocks.0"
        t = t + self.attention(self.layer_norm(t, blk + ".norm1"), None, blk + ".attn1", heads)
        t = t + self.attention(self.layer_norm(t, blk + ".norm2"), context, blk + ".attn2", heads)
        t = t + self.dense(F.gelu(self.dense(self.layer_norm(t, blk + ".norm3"), blk + ".ff.net.0.0")),
                           blk + ".ff.net.2")
        h = t.reshape(b, *sp, c).permute(0, 4, 1, 2, 3).contiguous(memory_format=torch.channels_last_3d)
        return self.conv(h, key + ".proj_out", residual=residual)

    def time_embed(self, timesteps):
        half = self.cfg.model_channels // 2
        freq = torch.exp(-math.log(10000) * torch.arange(half, dtype=torch.float32) / half)
        phase = torch.as_tensor(timesteps, dtype=torch.float32)[:, None] * freq[None]
        emb = torch.cat([torch.cos(phase), torch.sin(phase)], 1)
        return self.dense(F.silu(self.dense(emb, "time_embed.0")), "time_embed.2")

    def _input(self, x):
        return torch.as_tensor(np.asarray(x, np.float32)).contiguous(memory_format=torch.channels_last_3d)

    @torch.no_grad()
    def forward(self, x, timesteps, context):
        cfg = self.cfg
        emb = self.time_embed(timesteps)
        ctx = None
        if context is not None and not cfg.skip_context:
            ctx = self.dense(torch.as_tensor(np.asarray(context, np.float32)), "context_linear_projection")
        x = self.conv(self._input(x), "input_blocks.0.0")
        skips = [x]
        block, resolution = 1, 1
        for level in range(len(cfg.channel_mult)):
            for _ in range(cfg.num_res_blocks):
                key = f"input_blocks.{block}"
                x = self.residual(x, emb, key + ".0")
                if resolution in cfg.attention_resolutions:
                    x = self.transformer(x, ctx, key + ".1")
                skips.append(x)
                block += 1
            if level < len(cfg.channel_mult) - 1:
                x = self.conv(x, f"input_blocks.{block}.0.op", stride=2)
                skips.append(x)
                block += 1
                resolution *= 2
        x = self.residual(x, emb, "middle_block.0")
        x = self.transformer(x, ctx, "middle_block.1")
        x = self.residual(x, emb, "middle_block.2")
        block = 0
        for level in reversed(range(len(cfg.channel_mult))):
            for i in range(cfg.num_res_blocks + 1):
                key = f"output_blocks.{block}"
                x = self.residual(torch.cat([x, skips.pop()], 1), emb, key + ".0")
                has_attn = resolution in cfg.attention_resolutions
                if has_attn:
                    x = self.transformer(x, ctx, key + ".1")
                if level and i == cfg.num_res_blocks:
                    up = key + f".{2 if has_attn else 1}.conv"
                    assert UPSAMPLE_CONV.search(up)
                    x = self.upsample_conv(x, up)
                    resolution //= 2
                block += 1
        return self.norm_silu_conv(x, "out.0", "out.2", groups=_groups(x.shape[1]), eps=1e-5)

    @torch.no_grad()
    def encoder_stack(self, x, timesteps):
        cfg = self.cfg
        emb = self.time_embed(timesteps)
        x = self.conv(self._input(x), "input_blocks.0.0")
        block = 1
        for level in range(len(cfg.channel_mult)):
            for _ in range(cfg.num_res_blocks):
                x = self.residual(x, emb, f"input_blocks.{block}.0")
                block += 1
            if level < len(cfg.channel_mult) - 1:
                x = self.conv(x, f"input_blocks.{block}.0.op", stride=2)
                block += 1
        return x


class TorchVqDecoder(TorchLayers):
    """``oracle.unet.VqDecoder`` in torch fp32 on the CPU (mlx_model.py:720-727, 805-819)."""

    def __init__(self, weights, *, groups=16, eps=1e-6, levels=(2, 1, 0), upsample_levels=(1,), blocks=2):
        super().__init__(weights)
        self.groups, self.eps = groups, eps
        self.levels, self.upsample_levels, self.blocks = levels, upsample_levels, blocks

    def residual(self, x, key):
        h = self.norm_silu_conv(x, key + ".norm1", key + ".conv1", groups=self.groups, eps=self.eps)
        if key + ".nin_shortcut.weight" in self.w:
            x = self.conv(x, key + ".nin_shortcut")
        return self.norm_silu_conv(h, key + ".norm2", key + ".conv2", groups=self.groups, eps=self.eps, residual=x)

    def attn_block(self, x, key):
        h = self.norm(x, key + ".norm", groups=self.groups, eps=self.eps)
        b, c = x.shape[:2]
        sp = x.shape[2:]
        tok = lambda t: t.reshape(b, c, -1).transpose(1, 2)[:, None]
        q, k, v = (tok(self.conv(h, f"{key}.{n}")) for n in ("q", "k", "v"))
        o = F.scaled_dot_product_attention(q, k, v, scale=c ** -0.5)[:, 0]
        o = o.transpose(1, 2).reshape(b, c, *sp).contiguous(memory_format=torch.channels_last_3d)
        return self.conv(o, key + ".proj_out", residual=x)

    @torch.no_grad()
    def decode(self, z):
        x = torch.as_tensor(np.asarray(z, np.float32)).contiguous(memory_format=torch.channels_last_3d)
        x = self.conv(self.conv(x, "post_quant_conv"), "decoder.conv_in")
        x = self.residual(x, "decoder.mid.block_1")
        if "decoder.mid.attn_1.q.weight" in self.w:
            x = self.attn_block(x, "decoder.mid.attn_1")
        x = self.residual(x, "decoder.mid.block_2")
        for level in self.levels:
            for blk in range(self.blocks):
                x = self.residual(x, f"decoder.up.{level}.block.{blk}")
            if level in self.upsample_levels:
                x = self.upsample_conv(x, f"decoder.up.{level}.upsample.conv")
        return self.norm_silu_conv(x, "decoder.norm_out", "decoder.conv_out", groups=self.groups, eps=self.eps)
