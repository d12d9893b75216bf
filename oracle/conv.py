"""Float64 convolution oracle (test infrastructure only; see ``oracle/__init__.py``).

All tensors here are channels-first NCDHW NumPy arrays, the reference's public
layout (src/lesiondiffusion_mlx/_nax_conv.py:471-495).
"""

from __future__ import annotations

import numpy as np


def f16(x: np.ndarray) -> np.ndarray:
    """Round to float16 and return float64 (one IEEE round-to-nearest-even)."""
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float64)


def output_extent(n: int, *, stride: int = 1, upsample: bool = False) -> int:
    """Spatial output size of the padding-1 3x3x3 conv.

    Follows _nax_conv.py:513-516, 552: ``n`` for stride 1, ``(n - 1) // 2 + 1`` for
    stride 2 and ``2 n`` when the input is nearest-2x upsampled first.
    """
    if upsample:
        return 2 * n
    if stride == 1:
        return n
    if stride == 2:
        return (n - 1) // 2 + 1
    raise ValueError("stride must be 1 or 2")


def conv3d(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None, *,
           stride: int = 1, padding: int | None = None) -> np.ndarray:
    """Cross-correlation of NCDHW ``x`` with Torch-layout ``w`` ``(O, C, K, K, K)``.

    Zero padding ``padding`` (default ``K // 2``) on every spatial side, equal
    ``stride`` on every axis; float64 arithmetic, bias ``(O,)`` or per batch item
    ``(B, O)`` added last. This is the float64 sliding-window convolution of
    tests/test_native_kernels.py:213-225, evaluated one tap at a time as a matrix
    product so that full-size configs finish in seconds.
    """
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    bsz, cin, d, h, wd = x.shape
    o, cw, k, k2, k3 = w.shape
    assert cw == cin and k == k2 == k3
    p = k // 2 if padding is None else padding
    xp = np.pad(x, [(0, 0), (0, 0), (p, p), (p, p), (p, p)])
    od = (d + 2 * p - k) // stride + 1
    oh = (h + 2 * p - k) // stride + 1
    ow = (wd + 2 * p - k) // stride + 1
    out = np.zeros((bsz, o, od, oh, ow), dtype=np.float64)
    for kd in range(k):
        for kh in range(k):
            for kw in range(k):
                xs = xp[:, :, kd:kd + stride * (od - 1) + 1:stride,
                        kh:kh + stride * (oh - 1) + 1:stride,
                        kw:kw + stride * (ow - 1) + 1:stride]
                # (O, C) x (B, C, od, oh, ow) -> (O, B, od, oh, ow)
                out += np.moveaxis(np.tensordot(w[:, :, kd, kh, kw], xs, axes=([1], [1])), 0, 1)
    if b is not None:
        b = np.asarray(b, dtype=np.float64)
        out += b[:, :, None, None, None] if b.ndim == 2 else b[None, :, None, None, None]
    return out


def conv3d_magnitude(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None, *,
                     stride: int = 1, padding: int | None = None) -> np.ndarray:
    """Sum of absolute terms of each output, the scale of the reference's error
    bound ``1/2 ulp_fp16 + 8 * 2^-23 * sum|terms|`` (tests/test_native_kernels.py:37-39,
    98-104)."""
    return conv3d(np.abs(x), np.abs(w), None if b is None else np.abs(b),
                  stride=stride, padding=padding)


def upsample_nearest2(x: np.ndarray) -> np.ndarray:
    """Nearest 2x upsampling of the three spatial axes: output ``i`` reads input
    ``floor(i / 2)`` (src/lesiondiffusion_mlx/_spatial.py:12-26)."""
    return x.repeat(2, axis=2).repeat(2, axis=3).repeat(2, axis=4)


def resize_nearest(x: np.ndarray, shape: tuple[int, int, int]) -> np.ndarray:
    """Nearest resize with index ``floor(i * in / out)`` per axis (_spatial.py:60-69)."""
    if len(shape) != 3:
        raise ValueError("nearest resizing needs three spatial axes")
    for axis, target in enumerate(shape, start=2):
        idx = np.floor(np.arange(target) * (x.shape[axis] / target)).astype(np.int64)
        x = np.take(x, idx, axis=axis)
    return x


def fold_upsample_weight(w: np.ndarray) -> np.ndarray:
    """Fold a ``(O, C, 3, 3, 3)`` weight into 8 parity 2x2x2 filters.

    After nearest 2x upsampling, output ``2 m + p`` of an axis reads source voxels
    ``m - 1, m, m`` (p = 0) or ``m, m, m + 1`` (p = 1), so the taps that read the
    same source voxel merge: p = 0 -> ``(k0, k1 + k2)``, p = 1 -> ``(k0 + k1, k2)``
    (_nax_conv.py:367-405). Sums are float32 as in the reference; the caller rounds.

    Returns ``(8, O, 2, 2, 2, C)`` float32 indexed ``[pd*4+ph*2+pw, o, td, th, tw, c]``;
    parity ``p`` tap ``t`` reads the source at offset ``p - 1 + t``.
    """
    w32 = np.asarray(w, dtype=np.float32)

    def fold(a: np.ndarray, axis: int) -> np.ndarray:
        k0, k1, k2 = (np.take(a, i, axis=axis) for i in range(3))
        p0 = np.stack([k0, k1 + k2], axis=axis)
        p1 = np.stack([k0 + k1, k2], axis=axis)
        return np.stack([p0, p1], axis=0)

    o, c = w32.shape[:2]
    out = np.zeros((2, 2, 2, o, c, 2, 2, 2), dtype=np.float32)
    fd = fold(w32, 2)                      # (pd, O, C, td, 3, 3)
    for pd in range(2):
        fh = fold(fd[pd], 3)               # (ph, O, C, td, th, 3)
        for ph in range(2):
            fw = fold(fh[ph], 4)           # (pw, O, C, td, th, tw)
            for pw in range(2):
                out[pd, ph, pw] = fw[pw]
    # -> (8, O, td, th, tw, C)
    return out.reshape(8, o, c, 2, 2, 2).transpose(0, 1, 3, 4, 5, 2)


def upsample_conv_folded(x: np.ndarray, folded: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """Convolution of the nearest 2x upsampling of ``x`` from folded parity weights
    (``fold_upsample_weight`` layout), computed parity by parity on the source grid
    without forming the upsampled tensor (_nax_conv.py:168-189, 246-253)."""
    x = np.asarray(x, dtype=np.float64)
    folded = np.asarray(folded, dtype=np.float64)
    bsz, c, d, h, wd = x.shape
    o = folded.shape[1]
    xp = np.pad(x, [(0, 0), (0, 0), (1, 1), (1, 1), (1, 1)])
    out = np.zeros((bsz, o, 2 * d, 2 * h, 2 * wd))
    for parity in range(8):
        pd, ph, pw = parity >> 2, (parity >> 1) & 1, parity & 1
        acc = np.zeros((bsz, o, d, h, wd))
        for td in range(2):
            for th in range(2):
                for tw in range(2):
                    # padded index of source m - 1 + p + t is m + p + t
                    xs = xp[:, :, pd + td:pd + td + d, ph + th:ph + th + h, pw + tw:pw + tw + wd]
                    acc += np.moveaxis(np.tensordot(folded[parity, :, td, th, tw, :], xs,
                                                    axes=([1], [1])), 0, 1)
        out[:, :, pd::2, ph::2, pw::2] = acc
    if b is not None:
        b = np.asarray(b, dtype=np.float64)
        out += b[:, :, None, None, None] if b.ndim == 2 else b[None, :, None, None, None]
    return out


def pack_weight_reference_layout(w: np.ndarray) -> np.ndarray:
    """The reference's packed 3x3x3 weight: ``(27 * C', O')`` with row ``tap * C' + c``,
    ``tap = kd * 9 + kh * 3 + kw``, ``C' = ceil(C / 16) * 16``, ``O' = 16`` if ``O <= 16``
    else ``ceil(O / 32) * 32``, zero padding (_nax_conv.py:331-364)."""
    o, c = w.shape[:2]
    op = 16 - o if o <= 16 else -o % 32
    cp = -c % 16
    wp = np.pad(w, [(0, op), (0, cp), (0, 0), (0, 0), (0, 0)])
    return np.ascontiguousarray(wp.transpose(2, 3, 4, 1, 0).reshape(27 * (c + cp), o + op))


def pack_upsample_weight_reference_layout(w: np.ndarray) -> np.ndarray:
    """The reference's folded weight ``(8, 8 * C', O')``: parity ``pd*4+ph*2+pw``, row
    ``(td*4+th*2+tw) * C' + c``, float32 sums rounded to float16 once
    (_nax_conv.py:367-405)."""
    o, c = w.shape[:2]
    op = 16 - o if o <= 16 else -o % 32
    cp = -c % 16
    wp = np.pad(np.asarray(w, np.float32), [(0, op), (0, cp), (0, 0), (0, 0), (0, 0)])
    folded = fold_upsample_weight(wp)        # (8, O', 2, 2, 2, C')
    rows = folded.transpose(0, 2, 3, 4, 5, 1).reshape(8, 8 * (c + cp), o + op)
    return rows.astype(np.float16)


def conv3d_planes(plane, depth: int, w: np.ndarray, b: np.ndarray | None = None, *, stride: int = 1,
                  planes: list[int]) -> np.ndarray:
    """Output D-planes ``planes`` of ``conv3d(x, w, b, stride=stride)`` (3x3x3, padding 1)
    for an input of ``depth`` planes that is only read plane by plane: ``plane(i)`` returns
    input plane ``i`` as ``(B, C, H, W)``. Output plane ``od`` reads input planes
    ``od * stride + kd - 1`` (zero outside ``[0, depth)``), the same sliding window as
    ``conv3d``; this lets a full-size layer be checked on a few planes without forming it.
    Returns ``(B, O, len(planes), H', W')`` float64."""
    w = np.asarray(w, dtype=np.float64)
    o, c = w.shape[:2]
    out = None
    for j, od in enumerate(planes):
        for kd in range(3):
            i = od * stride + kd - 1
            if not 0 <= i < depth:
                continue
            xp = np.pad(np.asarray(plane(i), np.float64), [(0, 0), (0, 0), (1, 1), (1, 1)])
            bsz, _, hp, wp = xp.shape
            oh = (hp - 3) // stride + 1
            ow = (wp - 3) // stride + 1
            if out is None:
                out = np.zeros((bsz, o, len(planes), oh, ow))
            for kh in range(3):
                for kw in range(3):
                    xs = xp[:, :, kh:kh + stride * (oh - 1) + 1:stride, kw:kw + stride * (ow - 1) + 1:stride]
                    out[:, :, j] += np.moveaxis(np.tensordot(w[:, :, kd, kh, kw], xs, axes=([1], [1])), 0, 1)
    if out is None:
        raise ValueError("no output plane reads an input plane")
    if b is not None:
        b = np.asarray(b, dtype=np.float64)
        out += b[:, :, None, None, None] if b.ndim == 2 else b[None, :, None, None, None]
    return out


def upsample_conv_folded_planes(plane, depth: int, folded: np.ndarray, b: np.ndarray | None = None, *,
                                planes: list[int]) -> np.ndarray:
    """Output D-planes ``planes`` (of the 2x grid) of ``upsample_conv_folded``, reading the
    source plane by plane (``plane(i)`` as in ``conv3d_planes``): output plane ``2 m + pd``
    reads source planes ``m - 1 + pd + td``, td = 0, 1, through parity pd's folded taps
    (_nax_conv.py:168-189, 246-253). Returns ``(B, O, len(planes), 2H, 2W)`` float64."""
    folded = np.asarray(folded, dtype=np.float64)
    o = folded.shape[1]
    out = None
    for j, od in enumerate(planes):
        pd, m = od % 2, od // 2
        for td in range(2):
            i = m - 1 + pd + td
            if not 0 <= i < depth:
                continue
            xp = np.pad(np.asarray(plane(i), np.float64), [(0, 0), (0, 0), (1, 1), (1, 1)])
            bsz, _, hp, wp = xp.shape
            h, wd = hp - 2, wp - 2
            if out is None:
                out = np.zeros((bsz, o, len(planes), 2 * h, 2 * wd))
            for ph in range(2):
                for pw in range(2):
                    parity = pd * 4 + ph * 2 + pw
                    for th in range(2):
                        for tw in range(2):
                            xs = xp[:, :, ph + th:ph + th + h, pw + tw:pw + tw + wd]
                            out[:, :, j, ph::2, pw::2] += np.moveaxis(
                                np.tensordot(folded[parity, :, td, th, tw, :], xs, axes=([1], [1])), 0, 1)
    if out is None:
        raise ValueError("no output plane reads a source plane")
    if b is not None:
        b = np.asarray(b, dtype=np.float64)
        out += b[:, :, None, None, None] if b.ndim == 2 else b[None, :, None, None, None]
    return out
