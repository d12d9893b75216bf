"""Source-order fp16 conv3d and GroupNorm oracle (test infrastructure only; see
``oracle/__init__.py``).

Restates the reference's Torch-CPU-ordered half-precision kernels
(src/lesiondiffusion_mlx/_source_half.py), every float32 rounding explicit:

``conv3d_half`` (``_CONV``, _source_half.py:19-104; host ``conv3d_half``, :327-384)
    Each output is the dot product of the im2col column with the weight row over
    ``k = c * KD*KH*KW + (kd * KH + kh) * KW + kw`` (channel-major, :38-45). Products of
    two fp16 values are exact in float32. They are summed into four float32 partials by
    ``k % 4`` for ``k < K - K % 4`` in increasing ``k`` (:64-73), the remaining ``k`` are
    appended to partial 0 (:76-95), the total is ``((p0 + p1) + p2) + p3`` (:96-97), plus
    ``float32(bias)`` (:98-104), rounded once to fp16 (the float32 result stored into the
    half output).

``group_norm_half`` (_source_half.py:120-300, host :387-544)
    Per (batch item, group) the ``SIZE = C/G * D*H*W`` values in NCDHW order are split
    into vectors of 8 and chunks of 16 vectors. Each chunk keeps Welford moments per
    vector lane (``_PARTIAL_MOMENTS``, :135-162); chunks are merged by a binary-counter
    cascade, 128-chunk blocks in parallel first (``_CASCADE``, :164-199) and then
    group-wide with the leftover chunks (``_MOMENTS``, :201-260); the elements past the
    last whole vector are a scalar Welford pass, and the lanes are folded into it last
    (:247-260). ``merge`` is :121-132. The affine: ``var = max(m2 / SIZE, 0)``,
    ``rstd = 1/sqrt(var + eps)`` taken in float64 and rounded to float32 -- the value
    the reference's compensated reciprocal root (:244-252, :267-275) reproduces, as
    Torch computes it -- ``scale = rstd * weight``, ``offset = fma(-scale, mean, bias)``;
    the output ``fp16(scale * x + offset)`` with two float32 roundings (:253-254,
    :292-299).

NumPy float32 arithmetic rounds each operation to nearest even, as the kernels do with
contraction off; fused multiply-adds use ``oracle.vq.fma32`` (exactly rounded).
"""

from __future__ import annotations

import numpy as np

from oracle.vq import fma32

F32 = np.float32
CHUNK_VECTORS = 16        # vectors per Welford chunk (kChunkSize)
VECTOR = 8                # halves per vector; two float32 lanes of 4
BLOCK_DEPTH = 7           # 128-chunk blocks cascaded in parallel (_source_half.py:486-490)
BLOCK_CHUNKS = 1 << BLOCK_DEPTH


# ----------------------------------------------------------------------------- conv3d


def conv_extent(n: int, k: int, padding: int, stride: int) -> int:
    return (n + 2 * padding - k) // stride + 1


def _columns(x: np.ndarray, ksize: tuple[int, int, int], padding: int, stride: int):
    """im2col of NCDHW ``x`` as float32 ``(B * OD*OH*OW, C * KD*KH*KW)``, channel-major
    columns, zeros outside the volume (_source_half.py:35-47)."""
    b, c, d, h, w = x.shape
    kd, kh, kw = ksize
    od, oh, ow = (conv_extent(n, k, padding, stride) for n, k in zip((d, h, w), ksize))
    xp = np.zeros((b, c, d + 2 * padding, h + 2 * padding, w + 2 * padding), F32)
    xp[:, :, padding:padding + d, padding:padding + h, padding:padding + w] = x.astype(F32)
    cols = np.empty((b, od, oh, ow, c, kd, kh, kw), F32)
    for a in range(kd):
        for e in range(kh):
            for f in range(kw):
                cols[..., a, e, f] = xp[:, :, a:a + stride * od:stride, e:e + stride * oh:stride,
                                        f:f + stride * ow:stride].transpose(0, 2, 3, 4, 1)
    return cols.reshape(b * od * oh * ow, c * kd * kh * kw), (b, od, oh, ow)


def conv3d_half(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None, *, padding: int,
                stride: int) -> np.ndarray:
    """Source-order half conv3d of NCDHW fp16 ``x`` with ``(O, C, KD, KH, KW)`` fp16 weights;
    returns NCDHW fp16."""
    x = np.asarray(x, np.float16)
    weight = np.asarray(weight, np.float16)
    o = weight.shape[0]
    cols, (b, od, oh, ow) = _columns(x, tuple(weight.shape[2:]), padding, stride)
    wf = weight.reshape(o, -1).astype(F32)
    k_total = wf.shape[1]
    complete = k_total - k_total % 4
    part = np.zeros((4, cols.shape[0], o), F32)
    for k in range(k_total):
        # fp16 x fp16 is exact in float32, so the product is the same fused or not
        part[k % 4 if k < complete else 0] += cols[:, k:k + 1] * wf[None, :, k]
    total = ((part[0] + part[1]) + part[2]) + part[3]
    if bias is not None:
        total = total + np.asarray(bias, np.float16).astype(F32)[None]
    return total.astype(np.float16).reshape(b, od, oh, ow, o).transpose(0, 4, 1, 2, 3)


# -------------------------------------------------------------------------- GroupNorm


def _merge(a, b):
    """``merge(a, b)`` (_source_half.py:121-132): b folded into a. A moment set is
    (count int64 ``(n,)``, mean float32 ``(n, 4)``, m2 float32 ``(n, 4)``)."""
    ac, am, am2 = a
    bc, bm, bm2 = b
    count = ac + bc
    ratio = np.where(count == 0, F32(0), bc.astype(F32) / np.maximum(count, 1).astype(F32)).astype(F32)
    delta = (bm - am).astype(F32)
    correction = (ratio[:, None] * delta).astype(F32)
    prior = (delta * ac.astype(F32)[:, None]).astype(F32)
    mean = (am + correction).astype(F32)
    m2 = fma32(prior, correction, (am2 + bm2).astype(F32))
    return count, mean, m2


def _empty(shape_lead: tuple[int, ...]):
    return (np.zeros(shape_lead, np.int64), np.zeros(shape_lead + (4,), F32), np.zeros(shape_lead + (4,), F32))


def _group_values(x: np.ndarray, groups: int) -> np.ndarray:
    """NCDHW ``x`` as float32 ``(B * G, SIZE)`` in the reference's element order."""
    b, c = x.shape[:2]
    return np.asarray(x, np.float16).reshape(b * groups, -1).astype(F32)


def chunk_partials(values: np.ndarray):
    """``_PARTIAL_MOMENTS`` (_source_half.py:135-162) for every (group, chunk): returns
    counts ``(chunks,)`` and float32 mean, m2 ``(BG, chunks, 8)``."""
    bg, size = values.shape
    vectors = size // VECTOR
    chunks = max(1, (vectors + CHUNK_VECTORS - 1) // CHUNK_VECTORS)
    counts = np.array([max(0, min(CHUNK_VECTORS, vectors - ch * CHUNK_VECTORS)) for ch in range(chunks)], np.int64)
    vec = np.zeros((bg, chunks * CHUNK_VECTORS, VECTOR), F32)
    vec[:, :vectors] = values[:, :vectors * VECTOR].reshape(bg, vectors, VECTOR)
    vec = vec.reshape(bg, chunks, CHUNK_VECTORS, VECTOR)
    mean = np.zeros((bg, chunks, VECTOR), F32)
    m2 = np.zeros((bg, chunks, VECTOR), F32)
    for j in range(CHUNK_VECTORS):
        active = (j < counts)[None, :, None]
        ratio = F32(1.0) / F32(j + 1)
        xj = vec[:, :, j]
        delta = (xj - mean).astype(F32)
        new_mean = fma32(delta, np.full_like(delta, ratio), mean)
        new_m2 = fma32(delta, (xj - new_mean).astype(F32), m2)
        mean = np.where(active, new_mean, mean)
        m2 = np.where(active, new_m2, m2)
    return counts, mean, m2


def _chunk_pair(counts, mean, m2, ch):
    """The (lo, hi) lane halves of chunk ``ch`` as two moment sets of that chunk's count."""
    bg = mean.shape[0]
    cnt = np.full((bg,), counts[ch], np.int64)
    return (cnt, mean[:, ch, :4], m2[:, ch, :4]), (cnt, mean[:, ch, 4:], m2[:, ch, 4:])


def block_cascades(counts, mean, m2):
    """``_CASCADE`` (_source_half.py:164-199): each full 128-chunk block cascaded to its
    level-6 result (the final carry left to the group pass). Returns mean, m2
    ``(BG, blocks, 4)``."""
    bg, chunks = mean.shape[:2]
    blocks = chunks // BLOCK_CHUNKS if chunks > BLOCK_CHUNKS else 0
    out_mean = np.zeros((bg, blocks, 4), F32)
    out_m2 = np.zeros((bg, blocks, 4), F32)
    for blk in range(blocks):
        stack = [_empty((bg,)) for _ in range(BLOCK_DEPTH)]
        for c in range(BLOCK_CHUNKS):
            lo, hi = _chunk_pair(counts, mean, m2, blk * BLOCK_CHUNKS + c)
            stack[0] = _merge(_merge(stack[0], lo), hi)
            mask = c + 1
            level = 1
            while level < BLOCK_DEPTH and (mask & 1) == 0:
                stack[level] = _merge(stack[level], stack[level - 1])
                stack[level - 1] = _empty((bg,))
                mask >>= 1
                level += 1
        out_mean[:, blk] = stack[BLOCK_DEPTH - 1][1]
        out_m2[:, blk] = stack[BLOCK_DEPTH - 1][2]
    return out_mean, out_m2


def group_moments(values: np.ndarray, *, blocked: bool = True):
    """Mean and ``m2`` per group (``_MOMENTS``, _source_half.py:201-260), float32 ``(BG,)``.

    ``blocked=False`` runs the same cascade as one sequential binary counter over every
    chunk (the form the blocks split up); the two agree bit for bit."""
    bg, size = values.shape
    vectors = size // VECTOR
    counts, mean, m2 = chunk_partials(values)
    chunks = counts.shape[0]
    depth = max(1, (chunks - 1).bit_length())
    stack = [_empty((bg,)) for _ in range(depth)]
    blocks = chunks // BLOCK_CHUNKS if (blocked and chunks > BLOCK_CHUNKS) else 0
    if blocks:
        c_mean, c_m2 = block_cascades(counts, mean, m2)
        for blk in range(blocks):
            n = 2 * min(BLOCK_CHUNKS * CHUNK_VECTORS, vectors - blk * BLOCK_CHUNKS * CHUNK_VECTORS)
            part = (np.full((bg,), n, np.int64), c_mean[:, blk], c_m2[:, blk])
            stack[BLOCK_DEPTH] = _merge(stack[BLOCK_DEPTH], part)
            mask = blk + 1
            level = BLOCK_DEPTH + 1
            while level < depth and (mask & 1) == 0:
                stack[level] = _merge(stack[level], stack[level - 1])
                stack[level - 1] = _empty((bg,))
                mask >>= 1
                level += 1
    for ch in range(blocks * BLOCK_CHUNKS, chunks):
        lo, hi = _chunk_pair(counts, mean, m2, ch)
        stack[0] = _merge(_merge(stack[0], lo), hi)
        mask = ch + 1
        level = 1
        while level < depth and (mask & 1) == 0:
            stack[level] = _merge(stack[level], stack[level - 1])
            stack[level - 1] = _empty((bg,))
            mask >>= 1
            level += 1
    for level in range(1, depth):
        stack[0] = _merge(stack[0], stack[level])
    # the scalar tail past the last whole vector (_source_half.py:240-246)
    count = np.zeros((bg,), np.int64)
    t_mean = np.zeros((bg,), F32)
    t_m2 = np.zeros((bg,), F32)
    for i in range(vectors * VECTOR, size):
        xv = values[:, i]
        delta = (xv - t_mean).astype(F32)
        count = count + 1
        t_mean = (t_mean + (delta / count.astype(F32)).astype(F32)).astype(F32)
        t_m2 = fma32(delta, (xv - t_mean).astype(F32), t_m2)
    # fold the four lanes in (_source_half.py:247-260)
    added = 2 * vectors
    for lane in range(4):
        n = count + added
        with np.errstate(invalid="ignore", divide="ignore"):
            ratio = np.where(n == 0, F32(0), (F32(added) / np.maximum(n, 1).astype(F32)).astype(F32)).astype(F32)
        delta = (stack[0][1][:, lane] - t_mean).astype(F32)
        t_mean = fma32(ratio, delta, t_mean)
        t_m2 = (t_m2 + fma32(((delta * delta).astype(F32) * ratio).astype(F32), count.astype(F32),
                             stack[0][2][:, lane])).astype(F32)
        count = n
    return t_mean, t_m2


def group_norm_affine_half(x: np.ndarray, weight: np.ndarray, bias: np.ndarray, *, groups: int,
                           eps: float, blocked: bool = True):
    """float32 ``(B, C, 2)`` = (scale, offset) per channel (``_NORM_PARAMETERS``,
    _source_half.py:263-278), plus the group mean and variance ``(B, G)``."""
    b, c = x.shape[:2]
    values = _group_values(x, groups)
    size = values.shape[1]
    mean, m2 = group_moments(values, blocked=blocked)
    var = np.maximum((m2 / F32(size)).astype(F32), F32(0))
    rstd = (1.0 / np.sqrt(var.astype(np.float64) + np.float64(F32(eps)))).astype(F32)
    cpg = c // groups
    w = np.asarray(weight, np.float16).astype(F32).reshape(groups, cpg)
    bb = np.asarray(bias, np.float16).astype(F32).reshape(groups, cpg)
    rstd_g = rstd.reshape(b, groups, 1)
    mean_g = mean.reshape(b, groups, 1)
    scale = (rstd_g * w[None]).astype(F32)
    offset = fma32(-scale, np.broadcast_to(mean_g, scale.shape), np.broadcast_to(bb[None], scale.shape))
    affine = np.stack([scale.reshape(b, c), offset.reshape(b, c)], axis=-1).astype(F32)
    return affine, mean.reshape(b, groups), var.reshape(b, groups)


def group_norm_half(x: np.ndarray, weight: np.ndarray, bias: np.ndarray, *, groups: int,
                    eps: float) -> np.ndarray:
    """Source-order half GroupNorm of NCDHW fp16 ``x``; returns fp16 of ``x``'s shape."""
    x = np.asarray(x, np.float16)
    affine, _, _ = group_norm_affine_half(x, weight, bias, groups=groups, eps=eps)
    b, c = x.shape[:2]
    xs = x.reshape(b, c, -1).astype(F32)
    scale = affine[..., 0][..., None]
    offset = affine[..., 1][..., None]
    y = ((scale * xs).astype(F32) + offset).astype(F32)
    return y.astype(np.float16).reshape(x.shape)
