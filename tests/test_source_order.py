"""Pin the source-order oracle (``oracle/source_order.py``) on the CPU.

conv3d: bit for bit against Torch-CPU's own fp16 ``F.conv3d`` -- the computation the
reference's source kernel reproduces -- on the reference's test shapes
(tests/test_source_model.py:198-242, seed 47). oneDNN is switched off for the comparison:
on CPUs with AVX512-FP16 Torch routes fp16 convolutions to oneDNN, whose reduction order
differs; without it Torch takes its portable slow_conv3d / BlasKernel path, the one the
reference's fixtures were recorded with.

GroupNorm: the reference's own test holds its source GroupNorm to Torch at atol 1e-3
(tests/test_source_model.py:262-316); Torch's x86 build vectorizes the moments over 32
halves instead of 8, so here the oracle is held to Torch within one fp16 ulp of the output
plus a few fp32 roundings of its two affine terms, its group moments to float64 within
Welford's rounding, and its 128-chunk block split to the plain sequential cascade, bit for
bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import source_order as so

# (channels, outputs, kernel, padding, stride, with_bias): tests/test_source_model.py:198-210
CONV_CASES = [
    (2, 31, (1, 1, 1), 0, 1, True),
    (1, 3, (3, 3, 3), 1, 1, True),
    (2, 5, (3, 3, 3), 1, 2, False),
    (3, 7, (3, 1, 3), 1, 1, True),
    (4, 9, (2, 3, 2), 0, 1, False),
    (95, 35, (3, 3, 3), 1, 1, True),
    (96, 32, (3, 3, 3), 1, 2, True),
    (128, 33, (1, 1, 1), 0, 1, True),
    (512, 5, (1, 1, 1), 0, 1, False),
]

# tests/test_source_model.py:245-259 (16 groups, eps 1e-6)
GN_SHAPES = [
    (1, 96, 8, 12, 16), (2, 96, 8, 32, 32), (2, 16, 1, 1, 1), (2, 16, 1, 1, 7),
    (1, 16, 1, 1, 16377), (1, 16, 1, 1, 16384), (1, 16, 1, 1, 16391), (1, 16, 1, 1, 16392),
    (1, 16, 1, 1, 32760), (1, 16, 1, 1, 32768), (1, 16, 1, 1, 32775), (1, 16, 1, 1, 32776),
]


def conv_case(channels, outputs, kernel, with_bias):
    """The reference's inputs for one case (tests/test_source_model.py:222-225)."""
    rng = np.random.default_rng(47)
    x = rng.normal(size=(2, channels, 5, 7, 9)).astype(np.float16)
    w = rng.normal(size=(outputs, channels, *kernel)).astype(np.float16)
    b = rng.normal(size=outputs).astype(np.float16) if with_bias else None
    return x, w, b


def torch_conv_half(x, w, b, padding, stride) -> np.ndarray:
    """Torch-CPU fp16 conv3d on its portable path (oneDNN off)."""
    with torch.no_grad(), torch.backends.mkldnn.flags(enabled=False):
        return F.conv3d(torch.from_numpy(x), torch.from_numpy(w), None if b is None else torch.from_numpy(b),
                        padding=padding, stride=stride).numpy()


def gn_case(shape):
    """The reference's inputs for one GroupNorm case (tests/test_source_model.py:268-271)."""
    rng = np.random.default_rng(42)
    x = rng.normal(size=shape).astype(np.float16)
    w = rng.normal(size=shape[1]).astype(np.float16)
    b = rng.normal(size=shape[1]).astype(np.float16)
    return x, w, b


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"c{c[0]}-o{c[1]}-k{''.join(map(str, c[2]))}-s{c[4]}")
def test_source_conv_oracle_is_torch_cpu_bit_for_bit(case) -> None:
    channels, outputs, kernel, padding, stride, with_bias = case
    x, w, b = conv_case(channels, outputs, kernel, with_bias)
    got = so.conv3d_half(x, w, b, padding=padding, stride=stride)
    want = torch_conv_half(x, w, b, padding, stride)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_source_conv_order_is_what_the_pin_checks() -> None:
    """One fp32 accumulator in k order (a plausible mistake) differs from Torch on the
    reference's 95-channel case, so the pin above does tell the orders apart."""
    x, w, b = conv_case(95, 35, (3, 3, 3), True)
    cols, (bb, od, oh, ow) = so._columns(x, (3, 3, 3), 1, 1)
    wf = w.reshape(35, -1).astype(np.float32)
    acc = np.zeros((cols.shape[0], 35), np.float32)
    for k in range(wf.shape[1]):
        acc += cols[:, k:k + 1] * wf[None, :, k]
    single = (acc + b.astype(np.float32)[None]).astype(np.float16).reshape(bb, od, oh, ow, 35).transpose(0, 4, 1, 2, 3)
    want = torch_conv_half(x, w, b, 1, 1)
    assert np.count_nonzero(single.view(np.uint16) != want.view(np.uint16)) > 0


@pytest.mark.parametrize("shape", GN_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_source_group_norm_oracle_near_torch(shape) -> None:
    x, w, b = gn_case(shape)
    got = so.group_norm_half(x, w, b, groups=16, eps=1e-6)
    want = F.group_norm(torch.from_numpy(x), 16, torch.from_numpy(w), torch.from_numpy(b), eps=1e-6).numpy()
    # one fp16 ulp of the output, plus a few fp32 roundings of scale * x and offset (the
    # two orders' fp32 moments differ in their last bits; near zero that shows)
    aff, _, _ = so.group_norm_affine_half(x, w, b, groups=16, eps=1e-6)
    xs = x.reshape(x.shape[0], x.shape[1], -1).astype(np.float64)
    terms = (np.abs(aff[..., :1] * xs) + np.abs(aff[..., 1:])).reshape(x.shape)
    bound = np.spacing(np.abs(want)).astype(np.float64) + 4 * 2.0 ** -24 * terms
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= bound), f"max excess {np.max(err - bound):.3e}"
    # and within the reference's own tolerance of float64 GroupNorm of the same values
    want64 = F.group_norm(torch.from_numpy(x).double(), 16, torch.from_numpy(w).double(),
                          torch.from_numpy(b).double(), eps=1e-6).numpy()
    assert np.abs(got.astype(np.float64) - want64).max() <= 2 * np.spacing(np.float16(8)).astype(np.float64)


@pytest.mark.parametrize("shape", [(1, 96, 8, 12, 16), (1, 16, 1, 1, 32775), (2, 64, 8, 40, 40)],
                         ids=lambda s: "x".join(map(str, s)))
def test_source_group_moments_against_float64_and_block_split(shape) -> None:
    groups = 16 if shape[1] < 64 or shape[1] == 96 else 32
    x, w, b = gn_case(shape)
    aff, mean, var = so.group_norm_affine_half(x, w, b, groups=groups, eps=1e-6)
    aff_seq, mean_seq, var_seq = so.group_norm_affine_half(x, w, b, groups=groups, eps=1e-6, blocked=False)
    np.testing.assert_array_equal(aff, aff_seq)
    np.testing.assert_array_equal(mean, mean_seq)
    xs = x.reshape(shape[0], groups, -1).astype(np.float64)
    # Welford in fp32 over n values: mean and variance within a few ulp times log2(n)
    n = xs.shape[-1]
    tol = 8 * np.log2(n) * 2.0 ** -24
    assert np.all(np.abs(mean - xs.mean(-1)) <= tol * np.abs(xs).mean(-1))
    assert np.all(np.abs(var / xs.var(-1) - 1) <= tol)
    # the affine from those moments: scale = rstd * weight, offset = bias - scale * mean
    cpg = shape[1] // groups
    rstd = 1 / np.sqrt(var.astype(np.float64) + np.float32(1e-6))
    scale = np.repeat(rstd, cpg, axis=1) * w.astype(np.float64)[None]
    np.testing.assert_allclose(aff[..., 0], scale, rtol=2 * 2.0 ** -24)
    offset = b.astype(np.float64)[None] - aff[..., 0].astype(np.float64) * np.repeat(mean, cpg, axis=1)
    np.testing.assert_allclose(aff[..., 1], offset, rtol=2.0 ** -23, atol=2.0 ** -24 * np.abs(offset).max())


def test_source_group_norm_closed_forms() -> None:
    """A group of equal values has mean exactly that value and m2 exactly 0; integer
    values small enough for exact fp32 sums give the exact mean."""
    x = np.full((1, 16, 2, 3, 5), 1.5, np.float16)
    w = np.ones(16, np.float16)
    b = np.zeros(16, np.float16)
    _, mean, var = so.group_norm_affine_half(x, w, b, groups=16, eps=1e-6)
    assert np.all(mean == np.float32(1.5)) and np.all(var == 0)
    xi = (np.arange(16 * 64).reshape(1, 16, 1, 1, 64) % 8).astype(np.float16)   # 0..7 repeating
    _, mean, var = so.group_norm_affine_half(xi, w, b, groups=16, eps=1e-6)
    assert np.all(mean == np.float32(3.5))
    np.testing.assert_allclose(var, 5.25, rtol=2.0 ** -20)
