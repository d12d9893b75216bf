"""Float64 attention oracle (test infrastructure only)."""

from __future__ import annotations

import numpy as np


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
              mask: np.ndarray | None = None) -> np.ndarray:
    """``softmax(q k^T * scale + mask) v`` for ``(B, H, L, D)`` inputs in float64.

    Restates the float64 reference of tests/test_native_kernels.py:380-392 (row max
    subtracted before ``exp``) generalised to any head width, key length and an
    optional additive mask broadcastable to ``(B, H, L, LK)`` whose ``-inf`` entries
    remove keys (mlx_model.py:843-847, 860-862). A row whose keys are all masked
    yields zeros.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s = np.einsum("bhld,bhmd->bhlm", q, k) * scale
    if mask is not None:
        s = s + np.asarray(mask, np.float64)
    top = s.max(axis=-1, keepdims=True)
    top = np.where(np.isfinite(top), top, 0.0)
    p = np.exp(s - top)
    den = p.sum(axis=-1, keepdims=True)
    p = np.divide(p, den, out=np.zeros_like(p), where=den > 0)
    return np.einsum("bhlm,bhmd->bhld", p, v)


def attention_projected(q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int,
                        scale: float) -> np.ndarray:
    """Attention on head-interleaved projections ``(B, L, heads * d)`` (head ``h`` is
    columns ``h*d .. h*d+d-1``), returning the same layout (_attention.py:331-349)."""
    b, l, f = q.shape
    d = f // heads

    def split(t: np.ndarray) -> np.ndarray:
        return t.reshape(t.shape[0], t.shape[1], heads, d).transpose(0, 2, 1, 3)

    out = attention(split(q), split(k), split(v), scale)
    return out.transpose(0, 2, 1, 3).reshape(b, l, f)
