"""VQ codebook search oracle (test infrastructure only; see ``oracle/__init__.py``).

Restates the reference's four-channel nearest-codebook search (src/lesiondiffusion_mlx/
_vq.py:12-82) and the quantize step around it (mlx_model.py:742-803) in NumPy, with every
rounding point of the element type ``T`` (float16 or float32) explicit:

* squared norms: the squares rounded to T, summed in float32 in channel order, the sum
  rounded to T (mlx_model.py:775-778; ``_vq.py:77`` for the latent);
* dot products: float32 ``z0 * c0`` then three fused multiply-adds (``_vq.py:21-25``);
* distance: ``T(T(|z|^2 + |c|^2) - T(2 * T(dot)))`` (``_vq.py:28-30``);
* selection: the first NaN, else the first smallest distance -- NumPy's ``argmin`` order,
  which is MLX's (``_vq.py:31-45``);
* output: the straight-through ``z + (selected - z)`` in T (mlx_model.py:788-789).

NumPy has no fused multiply-add, so ``fma32`` forms it exactly: the product of two float32
values is exact in float64, the float64 sum carries its rounding error in a two-sum term,
and the float32 rounding uses that term where the float64 sum sits on a float32 midpoint.
"""

from __future__ import annotations

import numpy as np


def _round_to_f32(s: np.ndarray, err: np.ndarray) -> np.ndarray:
    """float32 value nearest the exact ``s + err`` (float64 ``s``, ``|err|`` below half
    an ulp of ``s``), ties to even."""
    r = s.astype(np.float32)
    back = r.astype(np.float64)
    # s exactly halfway between two float32 values: the sign of err picks the side.
    lo = np.nextafter(r, np.float32(-np.inf)).astype(np.float64)
    hi = np.nextafter(r, np.float32(np.inf)).astype(np.float64)
    mid_below = (s - lo) == (back - s)      # s halfway between lo and r
    mid_above = (hi - s) == (s - back)      # s halfway between r and hi
    on_mid = (back != s) & (mid_below | mid_above) & np.isfinite(s)
    if not np.any(on_mid & (err != 0)):
        return r
    out = r.copy()
    pick_low = on_mid & (err < 0)
    pick_high = on_mid & (err > 0)
    # the exact value lies on err's side of the midpoint
    low_side = np.where(mid_below, lo, back).astype(np.float32)
    high_side = np.where(mid_below, back, hi).astype(np.float32)
    out = np.where(pick_low, low_side, out)
    out = np.where(pick_high, high_side, out)
    return out


def fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded float32 ``a * b + c``."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64                       # exact: 24 + 24 significant bits
    s = p + c64
    bp = s - p                          # two-sum error of the float64 addition
    err = (p - (s - bp)) + (c64 - bp)
    with np.errstate(invalid="ignore"):
        return _round_to_f32(s, np.where(np.isfinite(err), err, 0.0))


def squared_norms4(x: np.ndarray, dtype) -> np.ndarray:
    """``T(sum_c float32(T(x_c * x_c)))`` over the last axis of ``(..., 4)`` values."""
    t = np.dtype(dtype)
    x = np.asarray(x, t)
    with np.errstate(over="ignore", invalid="ignore"):   # fp16 squares overflow to inf, as on the GPU
        sq = (x * x).astype(t).astype(np.float32)
        s = sq[..., 0]
        for c in range(1, 4):
            s = (s + sq[..., c]).astype(np.float32)
        return s.astype(t)


def distances4(z: np.ndarray, codebook: np.ndarray, dtype, *, z_norm: np.ndarray | None = None,
               codebook_norm: np.ndarray | None = None) -> np.ndarray:
    """``(P, E)`` distances of latent rows ``z (P, 4)`` to codebook rows ``(E, 4)`` with the
    reference's rounding points in ``dtype``."""
    t = np.dtype(dtype)
    z = np.asarray(z, t)
    cb = np.asarray(codebook, t)
    zn = squared_norms4(z, t) if z_norm is None else np.asarray(z_norm, t)
    cn = squared_norms4(cb, t) if codebook_norm is None else np.asarray(codebook_norm, t)
    zf = z.astype(np.float32)[:, None, :]
    cf = cb.astype(np.float32)[None, :, :]
    with np.errstate(over="ignore", invalid="ignore"):
        dot = (zf[..., 0] * cf[..., 0]).astype(np.float32)
        for c in range(1, 4):
            dot = fma32(zf[..., c], cf[..., c], dot)
        summed = (zn[:, None] + cn[None, :]).astype(t)
        doubled = (t.type(2) * dot.astype(t)).astype(t)
        return (summed - doubled).astype(t)


def nearest_codebook4(z: np.ndarray, codebook: np.ndarray, dtype, **norms) -> np.ndarray:
    """int32 index of the chosen code per latent row: the first NaN distance, else the first
    smallest one (``argmin``'s order)."""
    return np.argmin(distances4(z, codebook, dtype, **norms), axis=1).astype(np.int32)


def quantize4(z: np.ndarray, codebook: np.ndarray, dtype) -> tuple[np.ndarray, np.ndarray]:
    """(indices, straight-through ``z + (selected - z)`` in ``dtype``) for rows ``(P, 4)``."""
    t = np.dtype(dtype)
    z = np.asarray(z, t)
    idx = nearest_codebook4(z, codebook, t)
    sel = np.asarray(codebook, t)[idx]
    with np.errstate(over="ignore", invalid="ignore"):
        return idx, (z + (sel - z).astype(t)).astype(t)
