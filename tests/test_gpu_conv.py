"""conv3d parity on the MI355X: the HIP implicit-GEMM kernel against the float64
oracle, at the reference's own error model (tests/test_native_kernels.py:37-39, 98-104:
``|err| <= 1/2 ulp_fp16 + 8 * 2^-23 * sum|terms|`` (+ ``2^-11 * sum|terms|`` for a
re-rounded operand)) and the fp16 bar (max abs <= 2e-2, rel L2 <= 1e-3)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as ocv
from oracle import norm as onm
from tests.conftest import ACCUMULATION_EPS, OPERAND_ROUNDING, assert_fp16_bar, half_spacing

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["default", "streamed", "streamed-split", "quad"])
def conv_path(request, monkeypatch):
    """Every case four times: with the library's own kernel choice; with the streamed
    3x3x3 kernel taking every shape it supports (its fill threshold lowered to one
    workgroup), so small cases cover its partial bricks, batches, concat and fusions;
    with that threshold out of reach, so every streamed shape with two or more channel
    chunks splits them over workgroups (fp32 partial sums, fixed-order reduce); and with
    the K-quarter kernel taking every shape it supports (64-channel input chunks and
    output tiles, no input transform)."""
    monkeypatch.delenv("LDX_CONV_STREAM_MIN_WG", raising=False)
    monkeypatch.delenv("LDX_CONV_QUAD", raising=False)
    if request.param == "streamed":
        monkeypatch.setenv("LDX_CONV_STREAM_MIN_WG", "1")
        monkeypatch.setenv("LDX_CONV_QUAD", "0")
    elif request.param == "streamed-split":
        monkeypatch.setenv("LDX_CONV_STREAM_MIN_WG", "1000000")
        monkeypatch.setenv("LDX_CONV_QUAD", "0")
    elif request.param == "quad":
        monkeypatch.setenv("LDX_CONV_QUAD", "1")
    return request.param


def ndhwc(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a.transpose(0, 2, 3, 4, 1))


def ncdhw(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a.transpose(0, 4, 1, 2, 3))


def case(shape, out_c, k, seed):
    """Seeded fp16 case (tests/test_native_kernels.py:52-67): x ~ N(0,1) NCDHW, weight
    ~ N(0, 1/(C k^3)), bias ~ N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    c = shape[1]
    x = rng.normal(size=shape).astype(np.float16)
    w = (rng.normal(size=(out_c, c, k, k, k)) * (c * k ** 3) ** -0.5).astype(np.float16)
    b = (rng.normal(size=(out_c,)) * 0.1).astype(np.float16)
    return x, w, b


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().astype(np.float64)


def check_single_rounding(actual_ndhwc, x, w, b, stride=1, extra_operand_rounding=False):
    expected = ocv.conv3d(x, w, b, stride=stride)
    mag = ocv.conv3d_magnitude(x, w, b, stride=stride)
    actual = ncdhw(actual_ndhwc)
    err = np.abs(actual - expected)
    bound = half_spacing(expected) + (ACCUMULATION_EPS + (OPERAND_ROUNDING if extra_operand_rounding else 0)) * mag
    assert np.all(err <= bound), f"max excess {np.max(err - bound):.3e}"
    assert_fp16_bar(actual, expected)


@pytest.mark.parametrize(("shape", "out_c", "stride"), [
    ((1, 16, 5, 7, 9), 32, 1),   # odd extents
    ((2, 32, 4, 6, 3), 128, 1),  # batched, 128 outputs
    ((1, 48, 9, 3, 5), 64, 1),
    ((1, 5, 6, 4, 7), 4, 1),     # C and O not multiples of 8 (scalar path)
    ((2, 24, 7, 6, 9), 40, 2),   # stride 2, odd and even extents
    ((1, 512, 4, 4, 4), 128, 1),  # large C, few bricks
    ((1, 64, 32, 40, 40), 64, 1),  # config 1
    ((1, 9, 8, 10, 10), 64, 1),   # 9-channel network input
    ((1, 64, 8, 10, 10), 1, 1),   # single output channel
    ((1, 256, 4, 5, 5), 256, 1),
    ((1, 128, 8, 10, 10), 128, 2),
])
def test_conv3d_matches_float64_and_rounds_once(pkg, dev, shape, out_c, stride) -> None:
    """tests/test_native_kernels.py:143-168, plus the config shapes."""
    x, w, b = case(shape, out_c, 3, sum(shape))
    y = pkg.ops.conv3d(to_dev(ndhwc(x), dev), to_dev(w, dev), to_dev(b, dev), stride=stride)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16
    ext = tuple(ocv.output_extent(n, stride=stride) for n in shape[2:])
    assert tuple(y.shape) == (shape[0], *ext, out_c)
    check_single_rounding(host(y), x.astype(np.float64), w.astype(np.float64), b.astype(np.float64), stride)


@pytest.mark.parametrize(("shape", "c0", "out_c"), [
    ((2, 128, 6, 7, 13), 64, 128),    # two inputs, two output tiles, partial bricks, batch 2
    ((1, 192, 5, 11, 21), 128, 64),   # three chunks (two from the first input)
    ((1, 64, 4, 5, 10), 64, 64),      # exactly one brick
])
def test_conv3d_fuses_concat_bias_shift_residual_scale(pkg, dev, shape, c0, out_c) -> None:
    """concat([x, skip]) read from two tensors without forming it, a per-batch-item fp32
    bias, an fp16 shift, output scale and residual, one rounding of the sum (no input
    transform: the shapes every 3x3x3 kernel takes)."""
    rng = np.random.default_rng(sum(shape) + c0)
    x, w, _ = case(shape, out_c, 3, sum(shape))
    bias = rng.normal(size=(shape[0], out_c)).astype(np.float32)
    shift = rng.normal(size=(shape[0], out_c)).astype(np.float16)
    res = rng.normal(size=(shape[0], out_c, *shape[2:])).astype(np.float16)
    scale = 0.5
    x0t, x1t = to_dev(ndhwc(x[:, :c0]), dev), to_dev(ndhwc(x[:, c0:]), dev)
    y = pkg.ops.nax_conv3d(x0t, pkg.ops.pack_weight(to_dev(w, dev)), to_dev(bias, dev), x1=x1t,
                           shift=to_dev(shift, dev), residual=to_dev(ndhwc(res), dev), output_scale=scale)
    torch.cuda.synchronize()
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    products = ocv.conv3d(x64, w64)
    add = bias.astype(np.float64) + shift.astype(np.float64)
    expected = (products + add[:, :, None, None, None]) * scale + res
    mag = ocv.conv3d_magnitude(x64, w64)
    err = np.abs(ncdhw(host(y)) - expected)
    assert np.all(err <= half_spacing(expected) + ACCUMULATION_EPS * mag * scale)
    assert_fp16_bar(ncdhw(host(y)), expected)


@pytest.mark.parametrize(("shape", "c0", "out_c", "silu_only"), [
    ((2, 128, 6, 7, 13), 64, 128, False),   # two inputs, two output tiles, partial bricks
    ((1, 192, 5, 11, 21), 128, 64, False),  # three chunks
    ((1, 64, 4, 5, 10), 64, 64, True),      # SiLU without an affine
])
def test_conv3d_fuses_norm_silu_concat_shift_residual(pkg, dev, shape, c0, out_c, silu_only) -> None:
    """The GroupNorm affine + SiLU prologue on 64-channel chunks (what the K-quarter kernel
    stages through registers) with a two-tensor concat, per-batch bias, shift, scale and
    residual: against float64 of the normalised input rounded once to fp16."""
    rng = np.random.default_rng(sum(shape) + 3)
    x, w, _ = case(shape, out_c, 3, sum(shape) + 1)
    c = shape[1]
    bias = rng.normal(size=(shape[0], out_c)).astype(np.float32)
    shift = rng.normal(size=(shape[0], out_c)).astype(np.float16)
    res = rng.normal(size=(shape[0], out_c, *shape[2:])).astype(np.float16)
    x0t = to_dev(ndhwc(x[:, :c0]), dev)
    x1t = to_dev(ndhwc(x[:, c0:]), dev) if c0 < c else None
    if silu_only:
        aff = None
        prep = onm.silu(x.astype(np.float64))
    else:
        gamma = rng.normal(size=(c,)).astype(np.float32)
        beta = rng.normal(size=(c,)).astype(np.float32)
        aff = pkg.ops.group_norm_affine(x0t, to_dev(gamma, dev), to_dev(beta, dev), groups=16, eps=1e-5, x1=x1t)
        a = aff.cpu().numpy().astype(np.float64)
        prep = onm.silu(x.astype(np.float64) * a[:, :, 0, None, None, None] + a[:, :, 1, None, None, None])
    y = pkg.ops.nax_conv3d(x0t, pkg.ops.pack_weight(to_dev(w, dev)), to_dev(bias, dev), x1=x1t, affine=aff,
                           silu=True, shift=to_dev(shift, dev), residual=to_dev(ndhwc(res), dev), output_scale=0.5)
    torch.cuda.synchronize()
    normalized = ocv.f16(prep)
    w64 = w.astype(np.float64)
    products = ocv.conv3d(normalized, w64)
    add = bias.astype(np.float64) + shift.astype(np.float64)
    expected = (products + add[:, :, None, None, None]) * 0.5 + res
    mag = ocv.conv3d_magnitude(normalized, w64)
    err = np.abs(ncdhw(host(y)) - expected)
    # the normalised operand is rounded to fp16 on the GPU from the same fp32 affine
    assert np.all(err <= half_spacing(expected) + (ACCUMULATION_EPS + OPERAND_ROUNDING) * mag * 0.5)
    assert_fp16_bar(ncdhw(host(y)), expected)


def test_conv3d_reads_a_strided_channel_slice(pkg, dev) -> None:
    """A channel slice of a wider NDHWC tensor (voxel pitch > C), as a view, not a copy."""
    x, w, b = case((1, 32, 5, 6, 7), 48, 3, 3)
    wide = np.zeros((1, 5, 6, 7, 72), np.float16)
    wide[..., 16:48] = ndhwc(x)
    xt = to_dev(wide, dev)[..., 16:48]
    out_wide = torch.zeros((1, 5, 6, 7, 64), dtype=torch.float16, device=dev)
    pk = pkg.ops.pack_weight(to_dev(w, dev))
    pkg.ops.nax_conv3d(xt, pk, to_dev(b, dev), out=out_wide[..., 8:56])
    torch.cuda.synchronize()
    o = host(out_wide)
    assert np.all(o[..., :8] == 0) and np.all(o[..., 56:] == 0)
    check_single_rounding(o[..., 8:56], x.astype(np.float64), w.astype(np.float64), b.astype(np.float64))


def test_conv3d_two_input_concat(pkg, dev) -> None:
    """concat([x, skip]) read from two tensors without forming it."""
    x, w, b = case((2, 48, 4, 5, 6), 32, 3, 4)
    a, s = x[:, :32], x[:, 32:]
    pk = pkg.ops.pack_weight(to_dev(w, dev))
    y = pkg.ops.nax_conv3d(to_dev(ndhwc(a), dev), pk, to_dev(b, dev), x1=to_dev(ndhwc(s), dev))
    torch.cuda.synchronize()
    check_single_rounding(host(y), x.astype(np.float64), w.astype(np.float64), b.astype(np.float64))


@pytest.mark.parametrize("output_scale", [1.0, 0.25])
@pytest.mark.parametrize("channels", [32, 512])
def test_conv3d_batch_bias_residual_scale(pkg, dev, output_scale, channels) -> None:
    """tests/test_native_kernels.py:171-193: ((conv + bias[b]) * scale + residual), one rounding."""
    x, w, _ = case((2, channels, 4, 4, 4), 64, 3, channels)
    rng = np.random.default_rng(1)
    bias = rng.normal(size=(2, 64)).astype(np.float32)
    res = rng.normal(size=(2, 64, 4, 4, 4)).astype(np.float16)
    y = pkg.ops.nax_conv3d(to_dev(ndhwc(x), dev), pkg.ops.pack_weight(to_dev(w, dev)), to_dev(bias, dev),
                           residual=to_dev(ndhwc(res), dev), output_scale=output_scale)
    torch.cuda.synchronize()
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    products = ocv.conv3d(x64, w64)
    mag = ocv.conv3d_magnitude(x64, w64)
    expected = (products + bias.astype(np.float64)[:, :, None, None, None]) * output_scale + res
    err = np.abs(ncdhw(host(y)) - expected)
    assert np.all(err <= half_spacing(expected) + ACCUMULATION_EPS * mag * output_scale)


@pytest.mark.parametrize("upsample", [False, True])
@pytest.mark.parametrize("with_residual", [False, True])
def test_conv3d_scales_overflowing_branch_before_store(pkg, dev, upsample, with_residual) -> None:
    """tests/test_native_kernels.py:113-140: a 75000 branch (beyond fp16) scaled by 0.25
    before the single store, residual unscaled: exactly 18750 (+ 8192)."""
    x = torch.zeros((1, 2, 2, 2, 16), dtype=torch.float16, device=dev)
    w = torch.zeros((1, 16, 3, 3, 3), dtype=torch.float16, device=dev)
    bias = torch.tensor([75000.0], dtype=torch.float32, device=dev)
    sp = 4 if upsample else 2
    res = torch.full((1, sp, sp, sp, 1), 8192.0, dtype=torch.float16, device=dev) if with_residual else None
    pk = (pkg.ops.pack_upsample_weight if upsample else pkg.ops.pack_weight)(w)
    y = pkg.ops.nax_conv3d(x, pk, bias, upsample=upsample, residual=res, output_scale=0.25)
    torch.cuda.synchronize()
    want = np.full((1, sp, sp, sp, 1), 75000.0 * 0.25 + (8192.0 if with_residual else 0), np.float16)
    np.testing.assert_array_equal(host(y), want.astype(np.float64))


@pytest.mark.parametrize("shape,out_c", [((2, 32, 3, 5, 4), 64), ((1, 256, 8, 10, 10), 256),
                                         ((1, 128, 16, 20, 20), 128)])
def test_upsample_conv_matches_conv_of_nearest_upsampling(pkg, dev, shape, out_c) -> None:
    """tests/test_native_kernels.py:196-210: folded weights round merged taps once."""
    x, w, b = case(shape, out_c, 3, 21)
    y = pkg.ops.nax_conv3d(to_dev(ndhwc(x), dev), pkg.ops.pack_upsample_weight(to_dev(w, dev)),
                           to_dev(b, dev), upsample=True)
    torch.cuda.synchronize()
    up = ocv.upsample_nearest2(x.astype(np.float64))
    w64, b64 = w.astype(np.float64), b.astype(np.float64)
    expected = ocv.conv3d(up, w64, b64)
    mag = ocv.conv3d_magnitude(up, w64, b64)
    actual = ncdhw(host(y))
    assert actual.shape == expected.shape
    err = np.abs(actual - expected)
    assert np.all(err <= half_spacing(expected) + (ACCUMULATION_EPS + OPERAND_ROUNDING) * mag)
    assert_fp16_bar(actual, expected)


def test_pack_weight_layout_is_the_reference_layout_transposed(pkg, dev) -> None:
    """Bit-exact: packed[o, tap, c] == reference_packed[tap * C' + c, o]."""
    rng = np.random.default_rng(9)
    w = rng.standard_normal((20, 5, 3, 3, 3)).astype(np.float16)
    packed = pkg.ops.pack_weight(to_dev(w, dev))
    ours = pkg.ops.unpack_weight(packed)[0]
    ref = ocv.pack_weight_reference_layout(w)
    assert ours.shape == (20, 27, 5)
    assert packed.data.numel() == 4 * 27 * 4 * 512  # zero-padded to 128 outputs, 64 channels
    for tap in range(27):
        np.testing.assert_array_equal(ours[:, tap, :].T, ref[tap * 16:tap * 16 + 5, :20])
    full = packed.data.cpu().numpy().reshape(4, 27, 4, 2, 32, 8)  # (ob, tap, kc, g, r, e)
    assert np.all(full[1:] == 0) and np.all(full[0, :, :, :, 20:, :] == 0) and np.all(full[0, :, 1:] == 0)
    assert np.all(full[0, :, 0, 0, :, 5:] == 0) and np.all(full[0, :, 0, 1] == 0)


def test_pack_upsample_weight_is_bit_exact(pkg, dev) -> None:
    rng = np.random.default_rng(10)
    w = rng.standard_normal((7, 12, 3, 3, 3)).astype(np.float16)
    ours = pkg.ops.unpack_weight(pkg.ops.pack_upsample_weight(to_dev(w, dev)))
    ref = ocv.pack_upsample_weight_reference_layout(w)  # (8, 8 * 16, 16)
    assert ours.shape == (8, 7, 8, 12)
    for par in range(8):
        for t in range(8):
            np.testing.assert_array_equal(ours[par, :, t, :].T, ref[par, t * 16:t * 16 + 12, :7])


def test_norm_silu_conv_fuses_normalisation_shift_and_residual(pkg, dev) -> None:
    """tests/test_native_kernels.py:309-338: fused GN-affine + SiLU prologue, shift and
    residual vs the separately normalised input, one rounding of the sum."""
    rng = np.random.default_rng(13)
    x, w, b = case((2, 32, 4, 5, 6), 64, 3, 13)
    gamma = rng.normal(size=(32,)).astype(np.float16)
    beta = rng.normal(size=(32,)).astype(np.float16)
    shift = rng.normal(size=(2, 64)).astype(np.float16)
    res = rng.normal(size=(2, 64, 4, 5, 6)).astype(np.float16)
    xt = to_dev(ndhwc(x), dev)
    aff = pkg.ops.group_norm_affine(xt, to_dev(gamma, dev), to_dev(beta, dev), groups=8, eps=1e-5)
    bias = to_dev(b, dev).float()[None] + to_dev(shift, dev).float()
    y = pkg.ops.nax_conv3d(xt, pkg.ops.pack_weight(to_dev(w, dev)), bias, affine=aff, silu=True,
                           residual=to_dev(ndhwc(res), dev))
    torch.cuda.synchronize()
    x64 = x.astype(np.float64)
    normalized = ocv.f16(onm.silu(onm.group_norm(x64, gamma, beta, groups=8, eps=1e-5)))
    w64 = w.astype(np.float64)
    expected = ocv.conv3d(normalized, w64, b.astype(np.float64)) + shift[:, :, None, None, None] + res
    mag = ocv.conv3d_magnitude(normalized, w64, b.astype(np.float64))
    err = np.abs(ncdhw(host(y)) - expected)
    assert np.all(err <= half_spacing(expected) + (ACCUMULATION_EPS + OPERAND_ROUNDING) * mag)


@pytest.mark.parametrize("shape,c0,out_c", [((2, 96, 5, 9, 11), 64, 128), ((1, 128, 6, 7, 18), 32, 64)])
def test_conv_fuses_concat_norm_shift_residual_scale(pkg, dev, shape, c0, out_c) -> None:
    """Everything a decoder ResBlock conv fuses (mlx_model.py:290-342, 644): concat([x, skip])
    read from two tensors, GroupNorm affine + SiLU prologue (rounded to fp16 once), a
    per-batch-item fp32 bias, an fp16 shift, output scale and a residual, one rounding of
    the sum; extents that leave partial bricks on every axis."""
    rng = np.random.default_rng(sum(shape))
    x, w, b = case(shape, out_c, 3, 31)
    c = shape[1]
    gamma = rng.normal(size=(c,)).astype(np.float16)
    beta = rng.normal(size=(c,)).astype(np.float16)
    bias = rng.normal(size=(shape[0], out_c)).astype(np.float32)
    shift = rng.normal(size=(shape[0], out_c)).astype(np.float16)
    res = rng.normal(size=(shape[0], out_c, *shape[2:])).astype(np.float16)
    scale = 0.5
    x0t, x1t = to_dev(ndhwc(x[:, :c0]), dev), to_dev(ndhwc(x[:, c0:]), dev)
    aff = pkg.ops.group_norm_affine(x0t, to_dev(gamma, dev), to_dev(beta, dev), groups=16, eps=1e-5, x1=x1t)
    y = pkg.ops.nax_conv3d(x0t, pkg.ops.pack_weight(to_dev(w, dev)), to_dev(bias, dev), x1=x1t, affine=aff,
                           silu=True, shift=to_dev(shift, dev), residual=to_dev(ndhwc(res), dev),
                           output_scale=scale)
    torch.cuda.synchronize()
    normalized = ocv.f16(onm.silu(onm.group_norm(x.astype(np.float64), gamma, beta, groups=16, eps=1e-5)))
    w64 = w.astype(np.float64)
    products = ocv.conv3d(normalized, w64)
    add = bias.astype(np.float64) + shift.astype(np.float64)
    expected = (products + add[:, :, None, None, None]) * scale + res
    mag = ocv.conv3d_magnitude(normalized, w64)
    err = np.abs(ncdhw(host(y)) - expected)
    # the normalised operand comes from the GPU's own statistics: allow its fp16 rounding
    assert np.all(err <= half_spacing(expected) + (ACCUMULATION_EPS + 2 * OPERAND_ROUNDING) * mag * scale)
    assert_fp16_bar(ncdhw(host(y)), expected)


@pytest.mark.parametrize("with_bias", [True, False])
def test_pointwise_conv(pkg, dev, with_bias) -> None:
    """tests/test_native_kernels.py:361-377 (this kernel rounds once, inside that bound)."""
    x, w, b = case((2, 48, 3, 5, 7), 40, 1, 11)
    y = pkg.ops.conv3d(to_dev(ndhwc(x), dev), to_dev(w, dev), to_dev(b, dev) if with_bias else None,
                       padding=0)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (2, 3, 5, 7, 40)
    x64, w64, b64 = x.astype(np.float64), w.astype(np.float64), b.astype(np.float64)
    products = ocv.conv3d(x64, w64, padding=0)
    expected = products + (b64[None, :, None, None, None] if with_bias else 0)
    mag = ocv.conv3d_magnitude(x64, w64, padding=0)
    bound = half_spacing(products) + ACCUMULATION_EPS * mag + (half_spacing(expected) if with_bias else 0)
    assert np.all(np.abs(ncdhw(host(y)) - expected) <= bound)


def test_dense_rounds_once_and_fuses_gelu(pkg, dev) -> None:
    """tests/test_native_kernels.py:341-358, plus the dense -> GELU pair."""
    rng = np.random.default_rng(17)
    x = rng.normal(size=(2, 33, 48)).astype(np.float16)
    w = (rng.normal(size=(40, 48)) / 7).astype(np.float16)
    b = rng.normal(size=(40,)).astype(np.float16)
    pk = pkg.ops.pack_weight(to_dev(w, dev))
    y = pkg.ops.dense(to_dev(x, dev), pk, to_dev(b, dev))
    g = pkg.ops.dense(to_dev(x, dev), pk, to_dev(b, dev), act="gelu")
    torch.cuda.synchronize()
    terms = x.astype(np.float64) @ w.astype(np.float64).T
    expected = terms + b
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T + np.abs(b.astype(np.float64))
    yy = host(y)
    assert np.all(np.abs(yy - expected) <= half_spacing(expected) + ACCUMULATION_EPS * mag)
    want = onm.gelu(yy)  # GELU of the stored half value, rounded once more
    assert np.all(np.abs(host(g) - want) <= half_spacing(want) * 1.001 + 1e-7)


@pytest.mark.parametrize(("rows", "c", "o", "act", "with_res"), [
    (800, 256, 768, None, False),    # LINet level-2 norm1 -> q/k/v
    (100, 256, 1024, "gelu", False),  # level-3 norm3 -> feed-forward with GELU
    (800, 256, 1024, "gelu", True),   # level-2 norm3 -> feed-forward (800 workgroups), residual
    (37, 512, 64, None, True),        # widest fused LayerNorm, ragged row block, residual
    (5, 16, 32, None, False),         # one k-step in total
])
def test_dense_layer_norm_matches_float64(pkg, dev, rows, c, o, act, with_res) -> None:
    """ldx_dense_ln: LayerNorm of each row (mlx_model.py:360-367) then the dense layer in
    one launch, against float64 (LayerNorm, one fp16 rounding of its output, product), and
    against the two separate kernels."""
    rng = np.random.default_rng(rows + c + o)
    x = (rng.normal(size=(1, rows, c)) * 2 + 0.5).astype(np.float16)
    g = rng.normal(size=c).astype(np.float32)
    bb = rng.normal(size=c).astype(np.float32)
    w = (rng.normal(size=(o, c)) / np.sqrt(c)).astype(np.float16)
    bias = rng.normal(size=(o,)).astype(np.float16)
    res = rng.normal(size=(1, rows, o)).astype(np.float16) if with_res else None
    pk = pkg.ops.pack_weight(to_dev(w, dev))
    gd, bd = to_dev(g, dev), to_dev(bb, dev)
    xd = to_dev(x, dev)
    rd = to_dev(res, dev) if with_res else None
    y = pkg.ops.dense(xd, pk, to_dev(bias, dev), residual=rd, act=act, ln=(gd, bd, 1e-5))
    sep = pkg.ops.dense(pkg.ops.layer_norm(xd, gd, bd, 1e-5), pk, to_dev(bias, dev), residual=rd, act=act)
    torch.cuda.synchronize()
    xn = onm.layer_norm(x.astype(np.float64), g, bb, 1e-5)
    w64 = w.astype(np.float64)
    pre = xn @ w64.T + bias.astype(np.float64) + (res.astype(np.float64) if with_res else 0)
    expected = onm.gelu(pre) if act == "gelu" else pre
    # one fp16 rounding of the normalized input (2^-11 relative each, 2^-10 allowed for the
    # fused statistics' summation order), the accumulation, one rounding of the output
    mag = np.abs(xn) @ np.abs(w64).T
    bound = 2 * half_spacing(expected) + 2.0 ** -10 * mag + ACCUMULATION_EPS * (mag + np.abs(pre))
    yy = host(y)
    assert np.all(np.isfinite(yy))
    assert np.all(np.abs(yy - expected) <= bound)
    assert np.all(np.abs(yy - host(sep)) <= bound)


def merged_moments(m: torch.Tensor) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Chan's merge, in float64, of every block's (count, mean, M2) per channel pair."""
    mm = m.double().cpu().numpy()
    n, mean, m2 = mm[..., 0], mm[..., 1], mm[..., 2]
    assert np.all(m2 >= 0) and np.all(n >= 0) and np.all(n % 2 == 0)
    tot = n.sum(1)
    mu = (n * mean).sum(1) / tot
    return tot, mu, (m2.sum(1) + (n * (mean - mu[:, None]) ** 2).sum(1)) / tot


def check_moments(pkg, dev, y: torch.Tensor, groups: int = 32, eps: float = 1e-5) -> None:
    """The moments a conv kept of y: every output voxel counted once per channel pair, the
    pairs' mean and variance those of the stored fp16 values (float64 reference), and
    group_norm_affine from them equal to GroupNorm's (scale, offset) of y."""
    m = pkg.ops.moments_of(y)
    assert m is not None, "this conv kept no moments"
    yv = host(y)
    b, o = yv.shape[0], yv.shape[-1]
    pairs = yv.reshape(b, -1, o // 2, 2)
    tot, mu, var = merged_moments(m)
    assert np.array_equal(tot, np.full((b, o // 2), 2.0 * pairs.shape[1]))
    np.testing.assert_allclose(mu, pairs.mean(axis=(1, 3)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(var, pairs.var(axis=(1, 3)), rtol=1e-4, atol=1e-7)
    rng = np.random.default_rng(o)
    gamma = rng.normal(size=(o,)).astype(np.float32)
    beta = rng.normal(size=(o,)).astype(np.float32)
    aff = host(pkg.ops.group_norm_affine(y, to_dev(gamma, dev), to_dev(beta, dev), groups=groups, eps=eps))
    grp = yv.reshape(b, -1, groups, o // groups)
    gm, gv = grp.mean(axis=(1, 3)), grp.var(axis=(1, 3))
    scale = gamma[None] / np.sqrt(np.repeat(gv, o // groups, axis=1) + eps)
    offset = beta[None] - scale * np.repeat(gm, o // groups, axis=1)
    np.testing.assert_allclose(aff[..., 0], scale, rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(aff[..., 1], offset, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize(("shape", "out_c", "stride", "upsample", "fused", "groups"), [
    ((2, 64, 5, 9, 11), 64, 1, False, True, 32),
    ((1, 32, 6, 7, 18), 128, 1, False, False, 32),
    ((1, 96, 4, 6, 5), 256, 1, False, True, 32),
    ((1, 32, 9, 10, 12), 64, 2, False, False, 32),
    ((2, 64, 3, 5, 4), 64, 1, True, False, 32),
    # More (pair, block) items per group than the merge's 256 threads take in one round of
    # four (1,024), so its loop runs several rounds with all 256 threads loaded: 8 pairs per
    # group on config 1's grid, and the VQ decoder's 64 x 80 x 80 level (1,600 .. 12,800
    # blocks per pair, depending on the kernel path).
    ((1, 64, 32, 40, 40), 64, 1, False, True, 4),
    ((1, 64, 64, 80, 80), 64, 1, False, False, 32),
])
def test_conv_keeps_group_norm_moments(pkg, dev, shape, out_c, stride, upsample, fused, groups) -> None:
    """ldx_conv3d_stats: the GroupNorm partial moments reduced in the conv's epilogue (or
    its split-K reduce) -- every path of the parametrised kernel choice -- match the
    stored output, and the output itself equals ldx_conv3d's."""
    x, w, b = case(shape, out_c, 3, 41)
    rng = np.random.default_rng(41)
    res = rng.normal(size=(shape[0], *([2 * s for s in shape[2:]] if upsample else
                                       [(s - 1) // stride + 1 for s in shape[2:]]), out_c)).astype(np.float16)
    xt = to_dev(ndhwc(x), dev)
    packed = pkg.ops.pack_upsample_weight(to_dev(w, dev)) if upsample else pkg.ops.pack_weight(to_dev(w, dev))
    kw = dict(stride=stride, upsample=upsample, residual=to_dev(res, dev), output_scale=0.5)
    if fused:
        gamma = rng.normal(size=(shape[1],)).astype(np.float32)
        beta = rng.normal(size=(shape[1],)).astype(np.float32)
        kw.update(affine=pkg.ops.group_norm_affine(xt, to_dev(gamma, dev), to_dev(beta, dev), groups=32,
                                                   eps=1e-5), silu=True)
    y = pkg.ops.nax_conv3d(xt, packed, to_dev(b, dev), moments="always", **kw)
    y_plain = pkg.ops.nax_conv3d(xt, packed, to_dev(b, dev), **kw)
    torch.cuda.synchronize()
    assert pkg.ops.moments_of(y_plain) is None
    assert torch.equal(y, y_plain)
    check_moments(pkg, dev, y, groups=groups)


def test_group_norm_of_a_concat_from_moments(pkg, dev) -> None:
    """The decoder's GroupNorm over concat([x, skip]) from both producers' moments, with
    groups that straddle the two tensors (C = 96 + 64, 32 groups of 5 channels would not be
    pairs: 16 groups of 10), against float64 GroupNorm of the concatenation."""
    xa, wa, ba = case((1, 32, 5, 6, 7), 96, 3, 51)
    xb, wb, bb = case((1, 32, 5, 6, 7), 64, 3, 52)
    ya = pkg.ops.nax_conv3d(to_dev(ndhwc(xa), dev), pkg.ops.pack_weight(to_dev(wa, dev)), to_dev(ba, dev),
                            moments="always")
    yb = pkg.ops.nax_conv3d(to_dev(ndhwc(xb), dev), pkg.ops.pack_weight(to_dev(wb, dev)), to_dev(bb, dev),
                            moments="always")
    assert pkg.ops.moments_of(ya) is not None and pkg.ops.moments_of(yb) is not None
    rng = np.random.default_rng(5)
    gamma = rng.normal(size=(160,)).astype(np.float32)
    beta = rng.normal(size=(160,)).astype(np.float32)
    aff = host(pkg.ops.group_norm_affine(ya, to_dev(gamma, dev), to_dev(beta, dev), groups=16, eps=1e-5, x1=yb))
    cat = np.concatenate([host(ya), host(yb)], axis=-1)
    grp = cat.reshape(1, -1, 16, 10)
    gm, gv = grp.mean(axis=(1, 3)), grp.var(axis=(1, 3))
    scale = gamma[None] / np.sqrt(np.repeat(gv, 10, axis=1) + 1e-5)
    np.testing.assert_allclose(aff[..., 0], scale, rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(aff[..., 1], beta[None] - scale * np.repeat(gm, 10, axis=1), rtol=2e-5, atol=2e-5)
