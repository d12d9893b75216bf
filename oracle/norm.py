"""Float64 normalization / activation oracle (test infrastructure only).

Tensors are NCDHW for GroupNorm (channel axis 1) and ``(..., features)`` for
LayerNorm, as in the reference (src/lesiondiffusion_mlx/mlx_model.py:234-381).
"""

from __future__ import annotations

import math

import numpy as np


def group_norm_stats(x: np.ndarray, groups: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-(batch, group) mean and biased variance over ``(C / G) * D * H * W`` values,
    Torch ``group_norm`` statistics (the form of _source_half.py:266-306)."""
    x = np.asarray(x, dtype=np.float64)
    b, c = x.shape[:2]
    if c % groups:
        raise ValueError(f"groups {groups} must divide channels {c}")
    v = x.reshape(b, groups, -1)
    return v.mean(axis=2), v.var(axis=2)


def group_norm_affine(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, *, groups: int,
                      eps: float) -> np.ndarray:
    """Group statistics folded with the learned affine into per-(b, c) ``(scale, offset)``
    pairs, ``scale = gamma * rstd``, ``offset = beta - scale * mean`` -- the consumer
    contract of ``nax_conv3d``'s ``affine`` (_nax_conv.py:478-480, 131-133;
    mlx_model.py:328-335). Returns ``(B, C, 2)`` float64."""
    mean, var = group_norm_stats(x, groups)
    b, c = x.shape[:2]
    rstd = 1.0 / np.sqrt(var + eps)
    per = c // groups
    mean_c = np.repeat(mean, per, axis=1)
    rstd_c = np.repeat(rstd, per, axis=1)
    scale = np.asarray(gamma, np.float64)[None] * rstd_c
    offset = np.asarray(beta, np.float64)[None] - scale * mean_c
    return np.stack([scale, offset], axis=-1)


def apply_affine(x: np.ndarray, affine: np.ndarray) -> np.ndarray:
    """``x * scale + offset`` per (b, c) of NCDHW ``x``."""
    sh = (x.shape[0], x.shape[1]) + (1,) * (x.ndim - 2)
    return x * affine[..., 0].reshape(sh) + affine[..., 1].reshape(sh)


def group_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, *, groups: int,
               eps: float) -> np.ndarray:
    """Affine GroupNorm of NCDHW ``x`` in float64."""
    return apply_affine(np.asarray(x, np.float64), group_norm_affine(x, gamma, beta,
                                                                      groups=groups, eps=eps))


def silu(x: np.ndarray) -> np.ndarray:
    """``x / (1 + exp(-x))`` (_nax_conv.py:134)."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):   # exp(-x) = inf for x < -709 gives the limit -0
        return x / (1.0 + np.exp(-x))


def layer_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """Affine LayerNorm over the last axis, biased variance (mlx_model.py:360-367)."""
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(gamma, np.float64) + np.asarray(beta, np.float64)


_erf = np.vectorize(math.erf, otypes=[np.float64])


def gelu(x: np.ndarray) -> np.ndarray:
    """Exact erf GELU ``x * (1 + erf(x / sqrt(2))) / 2`` (mlx_model.py:369-374)."""
    x = np.asarray(x, dtype=np.float64)
    return x * (1.0 + _erf(x / math.sqrt(2.0))) * 0.5
