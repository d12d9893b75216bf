"""State-dict-keyed layers over the HIP ops -- the MI355X counterpart of the reference's
``SourceLayers`` dispatch seam (src/lesiondiffusion_mlx/mlx_model.py:84-381).

Weights keep upstream names and Torch layouts (``input_blocks.1.0.in_layers.2.weight``
...). At construction every conv / dense weight is packed once for the kernels (the
reference prepacks its NAX weights the same way, mlx_model.py:118-137), biases and
normalisation affines are kept in fp32, and the weights of layers that read the same
input are concatenated so one GEMM serves them (self-attention q/k/v; all ResBlock time
projections). Activations are channels-last NDHWC fp16 device tensors; every op is a
hand-written kernel from ``libldx.so``.
"""

from __future__ import annotations

import re
from collections.abc import Mapping

import numpy as np
import torch

from . import ops

# Convolutions applied only to a nearest 2x upsampling (mlx_model.py:79-81).
UPSAMPLE_CONV = re.compile(r"(?:^output_blocks\.\d+\.\d+|\.upsample)\.conv$")


def to_device_weights(weights: Mapping[str, object], device: torch.device,
                      dtype: torch.dtype = torch.float16) -> dict[str, torch.Tensor]:
    """Host arrays / tensors -> device tensors of ``dtype`` (the network's type)."""
    out: dict[str, torch.Tensor] = {}
    for k, v in weights.items():
        t = torch.as_tensor(np.asarray(v) if not isinstance(v, torch.Tensor) else v)
        out[k] = t.to(device=device, dtype=dtype if t.is_floating_point() else t.dtype)
    return out


def groups_for(channels: int) -> int:
    """``32 if C % 32 == 0 else C`` (mlx_model.py:427, 436, 653)."""
    return 32 if channels % 32 == 0 else channels


class SourceLayers:
    """Packed, source-keyed conv / dense / norm layers on one device. ``dtype`` is the
    network's activation and weight type: fp16 (the conditioned networks) or fp32 (the
    FP32 networks -- LMNet, the FP32 VQ decode -- on the exact split-fp16 mode), the two
    the reference's networks run in. bf16 is an op-level type (conv3d, dense, attention)
    only: the network's GroupNorm, LayerNorm and timestep kernels take fp16 or fp32, so a
    bf16 network is rejected here rather than on its first forward."""

    def __init__(self, weights: Mapping[str, torch.Tensor], *, device: torch.device | str = "cuda",
                 dtype: torch.dtype = torch.float16):
        if dtype not in (torch.float16, torch.float32):
            raise ValueError(f"network dtype {dtype} not supported: fp16 or fp32 (bf16 is supported by the "
                             "conv3d / dense / attention ops, not by the network's normalisation layers)")
        self.device = torch.device(device)
        self.dtype = dtype
        self.weights = to_device_weights(weights, self.device, dtype)
        self.packed: dict[str, ops.PackedWeight] = {}
        self.bias32: dict[str, torch.Tensor] = {}
        self.vec32: dict[str, torch.Tensor] = {}
        for name, w in self.weights.items():
            if not name.endswith(".weight"):
                continue
            key = name[: -len(".weight")]
            if w.dim() == 5 and tuple(w.shape[2:]) == (3, 3, 3):
                pack = ops.pack_upsample_weight if UPSAMPLE_CONV.search(key) else ops.pack_weight
                self.packed[key] = pack(w)
            elif w.dim() == 5 and tuple(w.shape[2:]) == (1, 1, 1) or w.dim() == 2:
                self.packed[key] = ops.pack_weight(w)
            elif w.dim() == 1:
                self.vec32[name] = w.float().contiguous()
            b = self.weights.get(key + ".bias")
            if b is not None:
                self.bias32[key] = b.float().contiguous()
        for name, w in self.weights.items():
            if name.endswith(".bias") and w.dim() == 1:
                self.vec32[name] = w.float().contiguous()

    # ------------------------------------------------------------------ ops
    def conv(self, x: torch.Tensor, key: str, *, stride: int = 1, residual: torch.Tensor | None = None,
             x1: torch.Tensor | None = None, affine: torch.Tensor | None = None, silu: bool = False,
             shift: torch.Tensor | None = None, output_scale: float = 1.0,
             out: torch.Tensor | None = None, moments: bool = False) -> torch.Tensor:
        """3x3x3 (padding 1, stride 1 or 2) or pointwise conv keyed ``key`` with the fused
        prologue/epilogue of ``ops.nax_conv3d`` (mlx_model.py:159-202, 290-342);
        ``moments``: keep the output's GroupNorm moments for the norm that reads it next."""
        return ops.nax_conv3d(x, self.packed[key], self.bias32.get(key), stride=stride, residual=residual,
                              x1=x1, affine=affine, silu=silu, shift=shift, output_scale=output_scale,
                              out=out, moments=moments)

    def upsample_conv(self, x: torch.Tensor, key: str, *, output_scale: float = 1.0,
                      moments: bool = False) -> torch.Tensor:
        """Conv of the nearest 2x upsampling of ``x`` from folded weights
        (mlx_model.py:272-288)."""
        return ops.nax_conv3d(x, self.packed[key], self.bias32.get(key), upsample=True,
                              output_scale=output_scale, moments=moments)

    def dense(self, x: torch.Tensor, key: str, *, residual: torch.Tensor | None = None,
              act: str | None = None, affine: torch.Tensor | None = None,
              ln: str | None = None, ln_eps: float = 1e-5) -> torch.Tensor:
        """Linear layer on the last axis, one rounding (mlx_model.py:204-217); ``ln`` names
        a LayerNorm applied to ``x`` first -- fused into the same launch when the width
        allows (a multiple of 16, at most 512 channels), else as its own kernel."""
        if ln is not None:
            c = int(x.shape[-1])
            if affine is None and c % 16 == 0 and c <= 512 and x.dtype != torch.float32:
                return ops.dense(x, self.packed[key], self.bias32.get(key), residual=residual, act=act,
                                 ln=(self.vec32[ln + ".weight"], self.vec32[ln + ".bias"], ln_eps))
            x = self.layer_norm(x, ln, ln_eps)
        return ops.dense(x, self.packed[key], self.bias32.get(key), residual=residual, act=act, affine=affine)

    def norm_affine(self, x: torch.Tensor, key: str, *, groups: int, eps: float,
                    x1: torch.Tensor | None = None) -> torch.Tensor:
        """GroupNorm statistics folded with ``key``'s affine (group_norm_affine)."""
        return ops.group_norm_affine(x, self.vec32[key + ".weight"], self.vec32[key + ".bias"],
                                     groups=groups, eps=eps, x1=x1)

    def norm_silu_conv(self, x: torch.Tensor, norm_key: str, conv_key: str, *, groups: int, eps: float,
                       shift: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                       x1: torch.Tensor | None = None, output_scale: float = 1.0,
                       moments: bool = False) -> torch.Tensor:
        """``residual + conv(silu(GN(x))) + shift`` with the normalised input never stored
        (mlx_model.py:290-342). GN's statistics come from the moments the conv that wrote
        ``x`` (and ``x1``) kept, when it kept them; ``moments`` keeps this conv's."""
        aff = self.norm_affine(x, norm_key, groups=groups, eps=eps, x1=x1)
        return self.conv(x, conv_key, x1=x1, affine=aff, silu=True, shift=shift, residual=residual,
                         output_scale=output_scale, moments=moments)

    def layer_norm(self, x: torch.Tensor, key: str, eps: float = 1e-5) -> torch.Tensor:
        return ops.layer_norm(x, self.vec32[key + ".weight"], self.vec32[key + ".bias"], eps)

    # ------------------------------------------------------ fused weight sets
    def fuse_dense(self, keys: list[str], name: str) -> list[tuple[int, int]]:
        """Concatenate dense weights that read the same input into one packed weight
        ``name`` (outputs in the order of ``keys``); returns each key's column range."""
        ws = [self.weights[k + ".weight"] for k in keys]
        if any(w.dim() != 2 for w in ws) or len({w.shape[1] for w in ws}) != 1:
            raise ValueError(f"cannot fuse {keys}")
        self.packed[name] = ops.pack_weight(torch.cat(ws, 0).contiguous())
        bs = [self.weights.get(k + ".bias") for k in keys]
        if any(b is not None for b in bs):
            full = [b.float() if b is not None else torch.zeros(w.shape[0], device=self.device)
                    for b, w in zip(bs, ws)]
            self.bias32[name] = torch.cat(full).contiguous()
        ranges, at = [], 0
        for w in ws:
            ranges.append((at, at + w.shape[0]))
            at += w.shape[0]
        return ranges


def ncdhw_to_ndhwc(x: torch.Tensor) -> torch.Tensor:
    """Boundary layout change (the network keeps NDHWC internally)."""
    return x.permute(0, 2, 3, 4, 1).contiguous()


def ndhwc_to_ncdhw(x: torch.Tensor) -> torch.Tensor:
    return x.permute(0, 4, 1, 2, 3).contiguous()


__all__ = ["SourceLayers", "UPSAMPLE_CONV", "to_device_weights", "groups_for", "ncdhw_to_ndhwc",
           "ndhwc_to_ncdhw"]
