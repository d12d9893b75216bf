"""The LDM 3-D UNet (LMNet / LINet architecture) on the HIP ops, channels-last.

Follows the reference's ``LdmUnet`` (src/lesiondiffusion_mlx/mlx_model.py:384-654):
time embedding -> input blocks (ResBlocks, spatial transformers at the configured
resolutions, stride-2 downsampling) -> middle block -> output blocks (skip concat,
upsampling) -> GroupNorm + SiLU + conv. Differences are in fusion only:

* every GroupNorm + SiLU feeds its conv as a prologue (never stored), the ResBlock time
  shift and residual join the conv epilogue;
* the decoder's ``concat([x, skip])`` is read from the two tensors (no copy);
* the transformer's token layout is the NDHWC activation itself (no transposes);
  self-attention q/k/v come from one GEMM, attention output projections and the
  feed-forward add their residual in the GEMM epilogue;
* all ResBlock time projections are one GEMM per forward.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Mapping
from dataclasses import dataclass

import numpy as np
import torch

from . import ops
from .layers import SourceLayers, groups_for, ncdhw_to_ndhwc, ndhwc_to_ncdhw


@dataclass(frozen=True)
class UnetConfig:
    """Architecture of one 3-D UNet (mlx_model.py:45-72)."""

    model_channels: int
    num_res_blocks: int
    attention_resolutions: tuple[int, ...]
    channel_mult: tuple[int, ...] = (1, 2, 4)
    num_head_channels: int = 32
    skip_context: bool = False


LMNET_CONFIG = UnetConfig(16, 1, (4,))                        # mlx_model.py:69
LINET_CONFIG = UnetConfig(128, 2, (4, 8), skip_context=True)  # mlx_model.py:72


class LdmUnet(SourceLayers):
    """Noise-prediction UNet. ``__call__`` takes and returns channels-first tensors like
    the reference (mlx_model.py:554-568); ``forward`` works on NDHWC."""

    def __init__(self, weights: Mapping[str, object], config: UnetConfig, *, device="cuda",
                 dtype: torch.dtype = torch.float16):
        super().__init__(weights, device=device, dtype=dtype)
        self.config = config
        # All ResBlock time projections read silu(emb): one GEMM.
        emb_keys = sorted(k[: -len(".weight")] for k in self.weights if k.endswith(".emb_layers.1.weight"))
        self.emb_slices: dict[str, tuple[int, int]] = {}
        if emb_keys:
            for k, r in zip(emb_keys, self.fuse_dense(emb_keys, "_emb_layers")):
                self.emb_slices[k[: -len(".emb_layers.1")]] = r
        # Self-attention (and context-free cross-attention) q/k/v: one GEMM each.
        self.qkv: dict[str, tuple[int, int]] = {}
        for k in self.weights:
            if k.endswith(".to_q.weight"):
                att = k[: -len(".to_q.weight")]
                is_self = att.endswith(".attn1") or config.skip_context
                if is_self:
                    self.fuse_dense([att + ".to_q", att + ".to_k", att + ".to_v"], att + ".qkv")
                else:
                    self.fuse_dense([att + ".to_k", att + ".to_v"], att + ".kv")

    # ------------------------------------------------------------- blocks
    def time_shifts(self, timesteps: torch.Tensor) -> torch.Tensor | None:
        """``emb_layers.1(silu(time_embed(t)))`` of every ResBlock, ``(B, sum O)``
        (mlx_model.py:609-614, 434)."""
        mc = self.config.model_channels
        t = ops.timestep_embedding(timesteps.to(torch.int32), mc, self.dtype)
        h = self.dense(t, "time_embed.0", act="silu")
        semb = self.dense(h, "time_embed.2", act="silu")
        return self.dense(semb, "_emb_layers") if self.emb_slices else None

    def residual(self, x: torch.Tensor, shifts: torch.Tensor | None, key: str,
                 x1: torch.Tensor | None = None) -> torch.Tensor:
        """Time-conditioned ResBlock (mlx_model.py:420-441); ``x1`` is the decoder skip."""
        c = x.shape[-1] + (0 if x1 is None else x1.shape[-1])
        shift = None
        if shifts is not None and key in self.emb_slices:
            lo, hi = self.emb_slices[key]
            shift = shifts[:, lo:hi]
        h = self.norm_silu_conv(x, key + ".in_layers.0", key + ".in_layers.2", groups=groups_for(c),
                                eps=1e-5, shift=shift, x1=x1, moments=True)
        if key + ".skip_connection" in self.packed:
            skip = self.conv(x, key + ".skip_connection", x1=x1)
        elif x1 is None:
            skip = x
        else:
            raise ValueError(f"{key}: concatenated input without a skip projection")
        return self.norm_silu_conv(h, key + ".out_layers.0", key + ".out_layers.3",
                                   groups=groups_for(h.shape[-1]), eps=1e-5, residual=skip, moments=True)

    def _attend(self, tok: torch.Tensor, att: str, heads: int, kv: tuple[torch.Tensor, torch.Tensor] | None,
                residual: torch.Tensor, ln: str) -> torch.Tensor:
        """``residual + attention(layer_norm(tok, ln))``; the LayerNorm runs inside the
        q/k/v (or to_q) dense layer's launch."""
        c = tok.shape[-1]
        if kv is None:
            qkv = self.dense(tok, att + ".qkv", ln=ln)
            q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
        else:
            q = self.dense(tok, att + ".to_q", ln=ln)
            k, v = kv
        o = ops.flash_attention(q, k, v, heads=heads, scale=(c // heads) ** -0.5)
        return self.dense(o, att + ".to_out.0", residual=residual)

    def transformer(self, x: torch.Tensor, context_kv: Mapping[str, tuple[torch.Tensor, torch.Tensor]] | None,
                    key: str) -> torch.Tensor:
        """Spatial transformer (mlx_model.py:522-552) on NDHWC ``x``."""
        b, d, h, w, c = x.shape
        aff = self.norm_affine(x, key + ".norm", groups=32, eps=1e-6)
        blk = key + ".transformer_blocks.0"
        kv = None if context_kv is None else context_kv.get(blk + ".attn2")
        if kv is None and not self.config.skip_context and context_kv is not None:
            raise ValueError(f"missing projected context for {blk}.attn2")
        tok = self.conv(x, key + ".proj_in", affine=aff).view(b, d * h * w, c)
        heads = c // self.config.num_head_channels
        tok = self._attend(tok, blk + ".attn1", heads, None, tok, blk + ".norm1")
        tok = self._attend(tok, blk + ".attn2", heads, kv, tok, blk + ".norm2")
        ff = self.dense(tok, blk + ".ff.net.0.0", act="gelu", ln=blk + ".norm3")
        tok = self.dense(ff, blk + ".ff.net.2", residual=tok)
        return self.conv(tok.view(b, d, h, w, c), key + ".proj_out", residual=x)

    def project_context(self, context: torch.Tensor | None) -> dict[str, tuple[torch.Tensor, torch.Tensor]] | None:
        """Context projection and every cross-attention's K/V, computed once per binding
        (prepare_denoiser, mlx_model.py:570-591)."""
        if context is None or self.config.skip_context:
            return None
        ctx = context.to(device=self.device, dtype=self.dtype).contiguous()
        proj = self.dense(ctx, "context_linear_projection")
        out: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}
        for k in self.packed:
            if k.endswith(".attn2.kv"):
                att = k[: -len(".kv")]
                kv = self.dense(proj, k)
                c = kv.shape[-1] // 2
                out[att] = (kv[..., :c], kv[..., c:])
        return out

    # ------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor, timesteps: torch.Tensor,
                context_kv: Mapping[str, tuple[torch.Tensor, torch.Tensor]] | None) -> torch.Tensor:
        """``LdmUnet._forward`` (mlx_model.py:599-654) on NDHWC fp16 ``x``."""
        cfg = self.config
        shifts = self.time_shifts(timesteps)
        x = self.conv(x, "input_blocks.0.0", moments=True)
        skips = [x]
        block, resolution = 1, 1
        for level in range(len(cfg.channel_mult)):
            for _ in range(cfg.num_res_blocks):
                key = f"input_blocks.{block}"
                x = self.residual(x, shifts, key + ".0")
                if resolution in cfg.attention_resolutions:
                    x = self.transformer(x, context_kv, key + ".1")
                skips.append(x)
                block += 1
            if level < len(cfg.channel_mult) - 1:
                x = self.conv(x, f"input_blocks.{block}.0.op", stride=2, moments=True)
                skips.append(x)
                block += 1
                resolution *= 2
        x = self.residual(x, shifts, "middle_block.0")
        x = self.transformer(x, context_kv, "middle_block.1")
        x = self.residual(x, shifts, "middle_block.2")
        block = 0
        for level in reversed(range(len(cfg.channel_mult))):
            for i in range(cfg.num_res_blocks + 1):
                key = f"output_blocks.{block}"
                x = self.residual(x, shifts, key + ".0", x1=skips.pop())
                has_attn = resolution in cfg.attention_resolutions
                if has_attn:
                    x = self.transformer(x, context_kv, key + ".1")
                if level and i == cfg.num_res_blocks:
                    x = self.upsample_conv(x, key + f".{2 if has_attn else 1}.conv", moments=True)
                    resolution //= 2
                block += 1
        return self.norm_silu_conv(x, "out.0", "out.2", groups=groups_for(x.shape[-1]), eps=1e-5)

    def encoder_stack(self, x: torch.Tensor, timesteps: torch.Tensor) -> torch.Tensor:
        """Input conv, ResBlocks and stride-2 downsampling of every level, without
        attention (the residual-block stack of the encoder)."""
        cfg = self.config
        shifts = self.time_shifts(timesteps)
        x = self.conv(x, "input_blocks.0.0", moments=True)
        block = 1
        for level in range(len(cfg.channel_mult)):
            for _ in range(cfg.num_res_blocks):
                x = self.residual(x, shifts, f"input_blocks.{block}.0")
                block += 1
            if level < len(cfg.channel_mult) - 1:
                x = self.conv(x, f"input_blocks.{block}.0.op", stride=2, moments=True)
                block += 1
        return x

    def __call__(self, x: torch.Tensor, timesteps: torch.Tensor, context: torch.Tensor | None) -> torch.Tensor:
        """Channels-first in and out, as the reference's ``LdmUnet.__call__``."""
        xs = ncdhw_to_ndhwc(x.to(device=self.device, dtype=self.dtype))
        t = timesteps.to(device=self.device, dtype=torch.int32)
        return ndhwc_to_ncdhw(self.forward(xs, t, self.project_context(context)))

    def prepare_denoiser(self, context: torch.Tensor | None) -> Callable[[torch.Tensor, torch.Tensor], torch.Tensor]:
        """Bind a context: its projections are computed once; the returned callable runs
        the NDHWC forward (mlx_model.py:570-597)."""
        kv = self.project_context(context)

        def denoise(x: torch.Tensor, timesteps: torch.Tensor) -> torch.Tensor:
            return self.forward(x, timesteps, kv)

        return denoise


# ------------------------------------------------------------ random init

def unet_state_dict(cfg: UnetConfig, *, in_channels: int, out_channels: int, context_dim: int | None,
                    ff_mult: int = 4, seed: int = 0, std_scale: float = 1.0) -> dict[str, np.ndarray]:
    """Random-init weights with upstream key names for ``cfg`` (an architecture stand-in
    when no checkpoint is available): convs/denses ~ N(0, 1/fan_in), norms gamma = 1 +
    N(0, 0.02^2), beta ~ N(0, 0.02^2), biases ~ N(0, 0.01^2). ``context_dim`` None means
    cross-attention attends to the block input (``skip_context``)."""
    rng = np.random.default_rng(seed)
    out: dict[str, np.ndarray] = {}
    mc = cfg.model_channels
    temb = 4 * mc

    def lin(key, fi, fo, bias=True):
        out[key + ".weight"] = (rng.standard_normal((fo, fi)) * std_scale / math.sqrt(fi)).astype(np.float32)
        if bias:
            out[key + ".bias"] = (rng.standard_normal(fo) * 0.01).astype(np.float32)

    def conv(key, fi, fo, k=3):
        out[key + ".weight"] = (rng.standard_normal((fo, fi, k, k, k)) * std_scale / math.sqrt(fi * k ** 3)).astype(np.float32)
        out[key + ".bias"] = (rng.standard_normal(fo) * 0.01).astype(np.float32)

    def norm(key, c):
        out[key + ".weight"] = (1 + rng.standard_normal(c) * 0.02).astype(np.float32)
        out[key + ".bias"] = (rng.standard_normal(c) * 0.02).astype(np.float32)

    def res(key, ci, co):
        norm(key + ".in_layers.0", ci)
        conv(key + ".in_layers.2", ci, co)
        lin(key + ".emb_layers.1", temb, co)
        norm(key + ".out_layers.0", co)
        conv(key + ".out_layers.3", co, co)
        if ci != co:
            conv(key + ".skip_connection", ci, co, 1)

    def xf(key, c):
        norm(key + ".norm", c)
        conv(key + ".proj_in", c, c, 1)
        conv(key + ".proj_out", c, c, 1)
        blk = key + ".transformer_blocks.0"
        for n in ("norm1", "norm2", "norm3"):
            norm(blk + "." + n, c)
        for a in ("attn1", "attn2"):
            kd = c if (a == "attn1" or context_dim is None) else context_dim
            lin(blk + f".{a}.to_q", c, c, bias=False)
            lin(blk + f".{a}.to_k", kd, c, bias=False)
            lin(blk + f".{a}.to_v", kd, c, bias=False)
            lin(blk + f".{a}.to_out.0", c, c)
        lin(blk + ".ff.net.0.0", c, ff_mult * c)
        lin(blk + ".ff.net.2", ff_mult * c, c)

    lin("time_embed.0", mc, temb)
    lin("time_embed.2", temb, temb)
    if context_dim is not None:
        lin("context_linear_projection", context_dim, context_dim, bias=False)
    conv("input_blocks.0.0", in_channels, mc)
    chans = [mc]
    ch, block, resolution = mc, 1, 1
    for level, mult in enumerate(cfg.channel_mult):
        for _ in range(cfg.num_res_blocks):
            res(f"input_blocks.{block}.0", ch, mult * mc)
            ch = mult * mc
            if resolution in cfg.attention_resolutions:
                xf(f"input_blocks.{block}.1", ch)
            chans.append(ch)
            block += 1
        if level < len(cfg.channel_mult) - 1:
            conv(f"input_blocks.{block}.0.op", ch, ch)
            chans.append(ch)
            block += 1
            resolution *= 2
    res("middle_block.0", ch, ch)
    xf("middle_block.1", ch)
    res("middle_block.2", ch, ch)
    block = 0
    for level in reversed(range(len(cfg.channel_mult))):
        for i in range(cfg.num_res_blocks + 1):
            skip = chans.pop()
            res(f"output_blocks.{block}.0", ch + skip, cfg.channel_mult[level] * mc)
            ch = cfg.channel_mult[level] * mc
            has_attn = resolution in cfg.attention_resolutions
            if has_attn:
                xf(f"output_blocks.{block}.1", ch)
            if level and i == cfg.num_res_blocks:
                conv(f"output_blocks.{block}.{2 if has_attn else 1}.conv", ch, ch)
                resolution //= 2
            block += 1
    norm("out.0", ch)
    conv("out.2", ch, out_channels)
    return out
