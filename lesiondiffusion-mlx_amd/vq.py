"""3-D VQ-GAN decoder on the HIP ops, channels-last (src/lesiondiffusion_mlx/mlx_model.py:
657-819) and its scaled-fp16 variant (_scaled_vq.py:27-118).

``VqDecoder.decode(z)`` quantizes the latent to its nearest codebook entries first (the
four-channel native search, ``ops.nearest_codebook4``) unless ``quantize=False``, as the
reference's ``decode(z, quantize=True)`` does. Its level list generalises the reference's
three-level layout so the full-resolution configuration -- two upsamplings and a
single-head mid-block attention -- uses the same code.
"""

from __future__ import annotations

import math
from collections.abc import Mapping

import numpy as np
import torch

from . import ops
from .layers import SourceLayers, ncdhw_to_ndhwc, ndhwc_to_ncdhw


class VqDecoder(SourceLayers):
    """``post_quant_conv -> conv_in -> mid (block_1, [attn_1], block_2) -> up levels ->
    GroupNorm + SiLU + conv_out`` (mlx_model.py:805-819), GroupNorm groups 16, eps 1e-6
    (mlx_model.py:722)."""

    def __init__(self, weights: Mapping[str, object], *, levels: tuple[int, ...] = (2, 1, 0),
                 upsample_levels: tuple[int, ...] = (1,), blocks: int = 2, groups: int = 16,
                 eps: float = 1e-6, device="cuda", dtype: torch.dtype = torch.float16):
        codebook = weights.get(self.CODEBOOK)
        super().__init__({k: v for k, v in weights.items() if k != self.CODEBOOK}, device=device, dtype=dtype)
        if dtype == torch.float32:
            self.QUANTIZE_DTYPE = torch.float32   # the FP32 decode quantizes in fp32 too
        self.levels, self.upsample_levels, self.blocks = levels, upsample_levels, blocks
        self.groups, self.eps = groups, eps
        self.set_codebook(codebook)
        for k in list(self.weights):
            if k.endswith(".attn_1.q.weight"):
                att = k[: -len(".q.weight")]
                ws = [self.weights[f"{att}.{n}.weight"] for n in ("q", "k", "v")]
                c = ws[0].shape[0]
                self.packed[att + ".qkv"] = ops.pack_weight(torch.cat([w.reshape(c, -1) for w in ws]).contiguous())
                self.bias32[att + ".qkv"] = torch.cat([self.weights[f"{att}.{n}.bias"].float()
                                                       for n in ("q", "k", "v")]).contiguous()

    CODEBOOK = "quantize.embedding.weight"
    QUANTIZE_DTYPE = torch.float16

    def set_codebook(self, codebook) -> None:
        """Use ``codebook`` ``(entries, 4)`` (host or device, any float dtype; None: none) from
        now on; its squared norms are recomputed on first use (the reference keeps them until
        the codebook is replaced, mlx_model.py:771-778)."""
        self._codebook = None
        if codebook is not None:
            t = codebook if isinstance(codebook, torch.Tensor) else torch.as_tensor(np.asarray(codebook))
            self._codebook = t.detach().to(device=self.device, dtype=torch.float32).contiguous()
        self._codebook_cache: dict[torch.dtype, tuple[torch.Tensor, torch.Tensor]] = {}

    def codebook(self, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        """(codebook, its squared norms) in ``dtype``."""
        if self._codebook is None:
            raise ValueError(f"no codebook: the weights have no {self.CODEBOOK}")
        if dtype not in self._codebook_cache:
            cb = self._codebook.to(dtype).contiguous()
            self._codebook_cache[dtype] = (cb, ops.squared_norms4(cb))
        return self._codebook_cache[dtype]

    def quantize(self, z: torch.Tensor, dtype: torch.dtype | None = None) -> torch.Tensor:
        """Nearest-codebook straight-through quantization of an NDHWC four-channel latent, in
        ``dtype`` (default: the decoder's quantization type), returned in that dtype
        (VqAutoencoder.quantize, mlx_model.py:742-803)."""
        dtype = dtype or self.QUANTIZE_DTYPE
        if z.shape[-1] != 4:
            raise ValueError(f"the native search takes four-channel latents, got {z.shape[-1]} channels")
        flat = z.to(dtype).reshape(-1, 4).contiguous()
        cb, norms = self.codebook(dtype)
        out = torch.empty_like(flat)
        ops.nearest_codebook4(flat, cb, norms, quantized=out)
        return out.view(z.shape)

    def norm_silu_conv_vq(self, x, norm_key, conv_key, *, eps_scale=1.0, output_scale=1.0, residual=None,
                          moments=False):
        return self.norm_silu_conv(x, norm_key, conv_key, groups=self.groups, eps=self.eps * eps_scale,
                                   residual=residual, output_scale=output_scale, moments=moments)

    def residual(self, x: torch.Tensor, key: str) -> torch.Tensor:
        """VQ ResBlock (mlx_model.py:720-727)."""
        h = self.norm_silu_conv_vq(x, key + ".norm1", key + ".conv1", eps_scale=self._eps_scale(key + ".norm1"),
                                   moments=True)
        if key + ".nin_shortcut" in self.packed:
            x = self.conv(x, key + ".nin_shortcut")
        return self.norm_silu_conv_vq(h, key + ".norm2", key + ".conv2",
                                      output_scale=self._branch_scale(key + ".conv2"), residual=x, moments=True)

    def attn_block(self, x: torch.Tensor, key: str) -> torch.Tensor:
        """Single-head spatial self-attention: GN -> 1x1 q/k/v (one GEMM, GN applied in
        its prologue) -> softmax(q k^T / sqrt(C)) v over all voxels -> 1x1 proj_out +
        residual."""
        b, d, h, w, c = x.shape
        aff = self.norm_affine(x, key + ".norm", groups=self.groups, eps=self.eps)
        qkv = self.conv(x, key + ".qkv", affine=aff).view(b, d * h * w, 3 * c)
        o = ops.flash_attention(qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:], heads=1, scale=c ** -0.5)
        return self.conv(o.view(b, d, h, w, c), key + ".proj_out", residual=x)

    def _eps_scale(self, norm_key: str) -> float:
        return 1.0

    def _branch_scale(self, conv_key: str) -> float:
        return 1.0

    def _upsample_scale(self, key: str) -> float:
        return 1.0

    def decode(self, z: torch.Tensor, *, quantize: bool = True) -> torch.Tensor:
        """NDHWC latent -> NDHWC fp16 volume at 2^(upsamplings) resolution; the latent is
        quantized first unless ``quantize`` is False (VqAutoencoder.decode,
        mlx_model.py:805-819)."""
        if quantize:
            z = self.quantize(z)
        x = self.conv(z.to(self.dtype), "post_quant_conv")
        x = self.conv(x, "decoder.conv_in", moments=True)
        x = self.residual(x, "decoder.mid.block_1")
        if "decoder.mid.attn_1.qkv" in self.packed:
            x = self.attn_block(x, "decoder.mid.attn_1")
        x = self.residual(x, "decoder.mid.block_2")
        for level in self.levels:
            for blk in range(self.blocks):
                x = self.residual(x, f"decoder.up.{level}.block.{blk}")
            if level in self.upsample_levels:
                key = f"decoder.up.{level}.upsample.conv"
                x = self.upsample_conv(x, key, output_scale=self._upsample_scale(key), moments=True)
        return self.norm_silu_conv_vq(x, "decoder.norm_out", "decoder.conv_out",
                                      eps_scale=self._eps_scale("decoder.norm_out"))

    def __call__(self, z: torch.Tensor, *, quantize: bool = True) -> torch.Tensor:
        """Channels-first latent in, channels-first volume out."""
        zz = ncdhw_to_ndhwc(z.to(device=self.device))
        if not quantize:
            zz = zz.to(self.dtype)
        return ndhwc_to_ncdhw(self.decode(zz, quantize=quantize))


class ScaledVqDecoder(VqDecoder):
    """The scaled-fp16 decoder of the reference's three-level layout (_scaled_vq.py):
    the upsampling conv and the residual branches after it store 0.25 x their value
    (the fp16 overflow fix, medmlx.py:1362-1366); GroupNorm over scaled inputs uses
    eps * 0.25^2, which leaves the normalised value unchanged."""

    SCALE = 0.25
    # The latent is quantized in fp32 before the half decode (_scaled_vq.py:45-49).
    QUANTIZE_DTYPE = torch.float32

    def _eps_scale(self, norm_key: str) -> float:
        scaled = norm_key == "decoder.norm_out" or (
            norm_key.startswith("decoder.up.0.block.") and norm_key.endswith(".norm1"))
        return self.SCALE ** 2 if scaled else 1.0

    def _branch_scale(self, conv_key: str) -> float:
        return self.SCALE if conv_key.startswith("decoder.up.0.block.") and conv_key.endswith(".conv2") else 1.0

    def _upsample_scale(self, key: str) -> float:
        if key != "decoder.up.1.upsample.conv":
            raise ValueError(f"{key}: the 0.25 output scale is defined only for decoder.up.1's "
                             "upsampling conv of the three-level decoder")
        return self.SCALE


def vq_decoder_state_dict(*, latent_channels: int, levels: list[tuple[int, int, bool]], mid_channels: int,
                          mid_attention: bool, out_channels: int = 1, seed: int = 0) -> tuple[dict[str, np.ndarray], dict]:
    """Random-init decoder weights with upstream key names. ``levels`` lists, in decode
    order, ``(level index, channels, upsample after)``; returns weights and the
    ``VqDecoder`` keyword arguments."""
    rng = np.random.default_rng(seed)
    out: dict[str, np.ndarray] = {}

    def conv(key, fi, fo, k=3):
        out[key + ".weight"] = (rng.standard_normal((fo, fi, k, k, k)) / math.sqrt(fi * k ** 3)).astype(np.float32)
        out[key + ".bias"] = (rng.standard_normal(fo) * 0.01).astype(np.float32)

    def norm(key, c):
        out[key + ".weight"] = (1 + rng.standard_normal(c) * 0.02).astype(np.float32)
        out[key + ".bias"] = (rng.standard_normal(c) * 0.02).astype(np.float32)

    def res(key, ci, co):
        norm(key + ".norm1", ci)
        conv(key + ".conv1", ci, co)
        norm(key + ".norm2", co)
        conv(key + ".conv2", co, co)
        if ci != co:
            conv(key + ".nin_shortcut", ci, co, 1)

    conv("post_quant_conv", latent_channels, latent_channels, 1)
    conv("decoder.conv_in", latent_channels, mid_channels)
    res("decoder.mid.block_1", mid_channels, mid_channels)
    if mid_attention:
        norm("decoder.mid.attn_1.norm", mid_channels)
        for n in ("q", "k", "v", "proj_out"):
            conv(f"decoder.mid.attn_1.{n}", mid_channels, mid_channels, 1)
    res("decoder.mid.block_2", mid_channels, mid_channels)
    ch = mid_channels
    for level, co, up in levels:
        res(f"decoder.up.{level}.block.0", ch, co)
        res(f"decoder.up.{level}.block.1", co, co)
        ch = co
        if up:
            conv(f"decoder.up.{level}.upsample.conv", ch, ch)
    norm("decoder.norm_out", ch)
    conv("decoder.conv_out", ch, out_channels)
    kw = {"levels": tuple(l for l, _, _ in levels), "upsample_levels": tuple(l for l, _, u in levels if u)}
    return out, kw
