"""lesiondiffusion-mlx_amd: the MI355X (gfx950) dense hot path of lesiondiffusion-mlx's
3-D latent diffusion -- implicit-GEMM conv3d, flash attention, GroupNorm/SiLU fusion --
behind the reference's op-level API, plus the UNet / VQ-decoder / DDIM callers.

Importing this package loads ``libldx.so`` (built by ``__graft_entry__.build()``) and
fails if it is missing: every op runs a hand-written HIP kernel, there is no CPU path.
"""

from . import _lib, layers, ops, sampling, unet, vq, weights  # noqa: F401  (loads libldx.so)

__all__ = ["ops", "layers", "unet", "vq", "sampling", "weights"]
