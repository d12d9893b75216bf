"""Float64 restatement of the LDM 3-D UNet and the VQ decoder (test infrastructure only).

``half=True`` rounds to float16 at the points where the reference's conditioned FP16
path stores a half tensor (mlx_model.py:159-381: one rounding per fused conv /
dense / normalization / activation / residual sum); ``half=False`` keeps float64
throughout (the reference's FP32 networks, to FP32 accuracy).
"""

from __future__ import annotations

import math
import re
from dataclasses import dataclass

import numpy as np

from . import attention as att
from . import conv as cv
from . import norm as nm

# Convolutions applied only to a nearest-2x upsampling (mlx_model.py:79-81).
UPSAMPLE_CONV = re.compile(r"(?:^output_blocks\.\d+\.\d+|\.upsample)\.conv$")


@dataclass(frozen=True)
class UnetConfig:
    """Architecture of one 3-D UNet (mlx_model.py:45-72), plus the feed-forward inner
    multiplier that the reference reads off its weights."""

    model_channels: int
    num_res_blocks: int
    attention_resolutions: tuple[int, ...]
    channel_mult: tuple[int, ...] = (1, 2, 4)
    num_head_channels: int = 32
    skip_context: bool = False


class Layers:
    """Source-keyed float64 layers with an optional float16 storage rounding."""

    def __init__(self, weights: dict[str, np.ndarray], *, half: bool):
        self.w = {k: np.asarray(v, np.float64) for k, v in weights.items()}
        self.half = half

    def r(self, x: np.ndarray) -> np.ndarray:
        return cv.f16(x) if self.half else x

    def conv(self, x: np.ndarray, key: str, *, padding: int = 1, stride: int = 1,
             bias_extra: np.ndarray | None = None, residual: np.ndarray | None = None,
             output_scale: float = 1.0) -> np.ndarray:
        """3x3x3: one rounding of ``(conv + bias (+shift)) * scale + residual``
        (_nax_conv.py:239-274). Pointwise: the product is rounded, then the bias sum
        (mlx_model.py:183-194)."""
        w = self.w[key + ".weight"]
        b = self.w.get(key + ".bias")
        if w.shape[2] == 1:
            y = self.r(cv.conv3d(x, w, None, padding=0))
            if b is not None:
                y = self.r(y + b[None, :, None, None, None])
            assert bias_extra is None and residual is None
            return y
        bias = np.zeros(w.shape[0]) if b is None else b
        if bias_extra is not None:
            bias = bias[None] + bias_extra
        y = cv.conv3d(x, w, bias, stride=stride, padding=padding) * output_scale
        if residual is not None:
            y = y + residual
        return self.r(y)

    def upsample_conv(self, x: np.ndarray, key: str, output_scale: float = 1.0) -> np.ndarray:
        """Folded parity conv of the nearest 2x upsampling; FP16 folded weights are
        rounded once (mlx_model.py:272-288, _nax_conv.py:367-405)."""
        w = self.w[key + ".weight"]
        folded = cv.fold_upsample_weight(w).astype(np.float64)
        if self.half:
            folded = cv.f16(folded)
        y = cv.upsample_conv_folded(x, folded, self.w.get(key + ".bias")) * output_scale
        return self.r(y)

    def dense(self, x: np.ndarray, key: str) -> np.ndarray:
        w = self.w[key + ".weight"]
        b = self.w.get(key + ".bias")
        y = x @ w.T
        if b is not None:
            y = y + b
        return self.r(y)

    def norm(self, x: np.ndarray, key: str, *, groups: int, eps: float) -> np.ndarray:
        return self.r(nm.group_norm(x, self.w[key + ".weight"], self.w[key + ".bias"],
                                    groups=groups, eps=eps))

    def norm_silu_conv(self, x: np.ndarray, norm_key: str, conv_key: str, *, groups: int,
                       eps: float, shift: np.ndarray | None = None,
                       residual: np.ndarray | None = None, output_scale: float = 1.0) -> np.ndarray:
        """``residual + conv(silu(GN(x))) + shift`` with the prepared input rounded once
        and one output rounding (mlx_model.py:290-342)."""
        aff = nm.group_norm_affine(x, self.w[norm_key + ".weight"], self.w[norm_key + ".bias"],
                                   groups=groups, eps=eps)
        prepared = self.r(nm.silu(nm.apply_affine(x, aff)))
        return self.conv(prepared, conv_key, bias_extra=shift, residual=residual,
                         output_scale=output_scale)

    def silu(self, x: np.ndarray) -> np.ndarray:
        return self.r(nm.silu(x))

    def layer_norm(self, x: np.ndarray, key: str, eps: float = 1e-5) -> np.ndarray:
        return self.r(nm.layer_norm(x, self.w[key + ".weight"], self.w[key + ".bias"], eps))

    def gelu(self, x: np.ndarray) -> np.ndarray:
        return self.r(nm.gelu(x))


def timestep_embedding(timesteps: np.ndarray, channels: int) -> np.ndarray:
    """``[cos(t f), sin(t f)]`` with ``f_i = exp(-ln(1e4) i / half)`` (mlx_model.py:609-612)."""
    half = channels // 2
    freq = np.exp(-math.log(10000) * np.arange(half, dtype=np.float32) / half).astype(np.float32)
    phase = np.asarray(timesteps, np.float32)[:, None] * freq[None]
    return np.concatenate([np.cos(phase), np.sin(phase)], axis=1).astype(np.float64)


class Unet(Layers):
    """The LDM 3-D UNet forward pass (mlx_model.py:420-654)."""

    def __init__(self, weights: dict[str, np.ndarray], cfg: UnetConfig, *, half: bool):
        super().__init__(weights, half=half)
        self.cfg = cfg

    def residual(self, x: np.ndarray, emb: np.ndarray, key: str) -> np.ndarray:
        groups = 32 if x.shape[1] % 32 == 0 else x.shape[1]
        shift = self.dense(self.silu(emb), key + ".emb_layers.1")
        h = self.norm_silu_conv(x, key + ".in_layers.0", key + ".in_layers.2", groups=groups,
                                eps=1e-5, shift=shift)
        groups = 32 if h.shape[1] % 32 == 0 else h.shape[1]
        if key + ".skip_connection.weight" in self.w:
            x = self.conv(x, key + ".skip_connection", padding=0)
        return self.norm_silu_conv(h, key + ".out_layers.0", key + ".out_layers.3", groups=groups,
                                   eps=1e-5, residual=x)

    def attention(self, x: np.ndarray, context: np.ndarray | None, key: str, heads: int,
                  projected_kv: tuple[np.ndarray, np.ndarray] | None = None) -> np.ndarray:
        ctx = x if context is None else context
        q = self.dense(x, key + ".to_q")
        if projected_kv is None:
            k, v = self.dense(ctx, key + ".to_k"), self.dense(ctx, key + ".to_v")
        else:
            k, v = projected_kv
        depth = q.shape[-1] // heads
        out = self.r(att.attention_projected(q, k, v, heads, depth ** -0.5))
        return self.dense(out, key + ".to_out.0")

    def transformer(self, x: np.ndarray, context: np.ndarray | None, key: str,
                    projected_kv: dict | None = None) -> np.ndarray:
        residual = x
        x = self.conv(self.norm(x, key + ".norm", groups=32, eps=1e-6), key + ".proj_in", padding=0)
        b, c = x.shape[:2]
        sp = x.shape[2:]
        x = x.transpose(0, 2, 3, 4, 1).reshape(b, -1, c)
        heads = c // self.cfg.num_head_channels
        blk = key + ".transformer_blocks.0"
        x = self.r(x + self.attention(self.layer_norm(x, blk + ".norm1"), None, blk + ".attn1", heads))
        pkv = None if projected_kv is None else projected_kv.get(blk + ".attn2")
        x = self.r(x + self.attention(self.layer_norm(x, blk + ".norm2"), context, blk + ".attn2",
                                      heads, pkv))
        ff = self.gelu(self.dense(self.layer_norm(x, blk + ".norm3"), blk + ".ff.net.0.0"))
        x = self.r(x + self.dense(ff, blk + ".ff.net.2"))
        x = x.reshape(b, *sp, c).transpose(0, 4, 1, 2, 3)
        return self.r(residual + self.conv(x, key + ".proj_out", padding=0))

    def time_embed(self, timesteps: np.ndarray) -> np.ndarray:
        emb = self.r(timestep_embedding(timesteps, self.cfg.model_channels))
        return self.dense(self.silu(self.dense(emb, "time_embed.0")), "time_embed.2")

    def project_context(self, context: np.ndarray | None) -> np.ndarray | None:
        if context is None or self.cfg.skip_context:
            return None
        return self.dense(self.r(np.asarray(context, np.float64)), "context_linear_projection")

    def forward(self, x: np.ndarray, timesteps: np.ndarray, context: np.ndarray | None) -> np.ndarray:
        """``LdmUnet._forward`` (mlx_model.py:599-654)."""
        cfg = self.cfg
        emb = self.time_embed(timesteps)
        context = self.project_context(context)
        x = self.conv(self.r(np.asarray(x, np.float64)), "input_blocks.0.0")
        skips = [x]
        block, resolution = 1, 1
        for level in range(len(cfg.channel_mult)):
            for _ in range(cfg.num_res_blocks):
                key = f"input_blocks.{block}"
                x = self.residual(x, emb, key + ".0")
                if resolution in cfg.attention_resolutions:
                    x = self.transformer(x, context, key + ".1")
                skips.append(x)
                block += 1
            if level < len(cfg.channel_mult) - 1:
                x = self.conv(x, f"input_blocks.{block}.0.op", stride=2)
                skips.append(x)
                block += 1
                resolution *= 2
        x = self.residual(x, emb, "middle_block.0")
        x = self.transformer(x, context, "middle_block.1")
        x = self.residual(x, emb, "middle_block.2")
        block = 0
        for level in reversed(range(len(cfg.channel_mult))):
            for i in range(cfg.num_res_blocks + 1):
                key = f"output_blocks.{block}"
                x = self.residual(np.concatenate([x, skips.pop()], axis=1), emb, key + ".0")
                has_attn = resolution in cfg.attention_resolutions
                if has_attn:
                    x = self.transformer(x, context, key + ".1")
                if level and i == cfg.num_res_blocks:
                    x = self.upsample_conv(x, key + f".{2 if has_attn else 1}.conv")
                    resolution //= 2
                block += 1
        groups = 32 if x.shape[1] % 32 == 0 else x.shape[1]
        return self.norm_silu_conv(x, "out.0", "out.2", groups=groups, eps=1e-5)

    def encoder_stack(self, x: np.ndarray, timesteps: np.ndarray) -> np.ndarray:
        """Input convolution and the residual/downsampling encoder levels only, the
        block stack of config 3 (no attention)."""
        cfg = self.cfg
        emb = self.time_embed(timesteps)
        x = self.conv(self.r(np.asarray(x, np.float64)), "input_blocks.0.0")
        block = 1
        for level in range(len(cfg.channel_mult)):
            for _ in range(cfg.num_res_blocks):
                x = self.residual(x, emb, f"input_blocks.{block}.0")
                block += 1
            if level < len(cfg.channel_mult) - 1:
                x = self.conv(x, f"input_blocks.{block}.0.op", stride=2)
                block += 1
        return x


class VqDecoder(Layers):
    """VQ decoder (mlx_model.py:720-727, 805-819), generalised to a level list so the
    full-resolution config can be expressed; ``output_scale`` reproduces the scaled
    FP16 variant's post-upsampling scaling (_scaled_vq.py:24, 51-118) when given."""

    def __init__(self, weights: dict[str, np.ndarray], *, half: bool, groups: int = 16,
                 eps: float = 1e-6, levels: tuple[int, ...] = (2, 1, 0), upsample_levels=(1,),
                 blocks: int = 2):
        super().__init__(weights, half=half)
        self.groups, self.eps = groups, eps
        self.levels, self.upsample_levels, self.blocks = levels, upsample_levels, blocks

    def residual(self, x: np.ndarray, key: str) -> np.ndarray:
        h = self.norm_silu_conv(x, key + ".norm1", key + ".conv1", groups=self.groups, eps=self.eps)
        if key + ".nin_shortcut.weight" in self.w:
            x = self.conv(x, key + ".nin_shortcut", padding=0)
        return self.norm_silu_conv(h, key + ".norm2", key + ".conv2", groups=self.groups,
                                   eps=self.eps, residual=x)

    def attn_block(self, x: np.ndarray, key: str) -> np.ndarray:
        """Single-head spatial self-attention block: GN -> 1x1 q/k/v -> softmax(q k^T /
        sqrt(C)) v -> 1x1 proj_out -> residual (the VQ-GAN mid attention)."""
        h = self.norm(x, key + ".norm", groups=self.groups, eps=self.eps)
        q = self.conv(h, key + ".q", padding=0)
        k = self.conv(h, key + ".k", padding=0)
        v = self.conv(h, key + ".v", padding=0)
        b, c = x.shape[:2]
        sp = x.shape[2:]

        def tok(t: np.ndarray) -> np.ndarray:
            return t.reshape(b, c, -1).transpose(0, 2, 1)[:, None]

        o = self.r(att.attention(tok(q), tok(k), tok(v), c ** -0.5))[:, 0]
        o = o.transpose(0, 2, 1).reshape(b, c, *sp)
        return self.r(x + self.conv(o, key + ".proj_out", padding=0))

    def decode(self, z: np.ndarray) -> np.ndarray:
        x = self.conv(self.r(np.asarray(z, np.float64)), "post_quant_conv", padding=0)
        x = self.conv(x, "decoder.conv_in")
        x = self.residual(x, "decoder.mid.block_1")
        if "decoder.mid.attn_1.q.weight" in self.w:
            x = self.attn_block(x, "decoder.mid.attn_1")
        x = self.residual(x, "decoder.mid.block_2")
        for level in self.levels:
            for blk in range(self.blocks):
                x = self.residual(x, f"decoder.up.{level}.block.{blk}")
            if level in self.upsample_levels:
                x = self.upsample_conv(x, f"decoder.up.{level}.upsample.conv")
        return self.norm_silu_conv(x, "decoder.norm_out", "decoder.conv_out", groups=self.groups,
                                   eps=self.eps)
