"""bf16 conv3d and attention on the MI355X (ldx_conv3d / ldx_attention with dtype
LDX_DTYPE_BF16: bf16 operands on v_mfma_f32_32x32x16_bf16, fp32 accumulation, one bf16
rounding) against the float64 oracle on the same bf16-valued inputs.

Bound: the reference's per-element error model (tests/test_native_kernels.py:37-39,
98-104) with bf16's output rounding -- 1/2 ulp of bf16 + 8 * 2^-23 * sum|terms| -- plus
2^-8 * sum|terms| where an operand is re-rounded to bf16 on the device (the GroupNorm /
SiLU prologue, LayerNorm in front of a dense layer, folded upsample weights). BASELINE's
fp16 bar (max abs 2e-2, relative L2 1e-3) scaled by the ratio of the two formats' unit
roundoffs (2^-8 / 2^-11 = 8): max abs 0.16, relative L2 8e-3. Attention: the reference's
fp16 tolerance (atol = rtol = 2e-3, test_native_kernels.py:448-450) scaled the same way."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import conv as ocv
from oracle import norm as onm
from tests.conftest import ACCUMULATION_EPS

pytestmark = pytest.mark.gpu

BF16_OPERAND_ROUNDING = 2.0 ** -8     # unit roundoff of bf16
BF16_BAR = dict(max_abs=0.16, rel_l2=8e-3)


def bf16_values(a: np.ndarray) -> np.ndarray:
    """``a`` rounded to bf16 (round to nearest even), as float64."""
    return torch.from_numpy(np.asarray(a, np.float32)).bfloat16().double().numpy()


def bf16_half_spacing(v: np.ndarray) -> np.ndarray:
    """Half the bf16 spacing at ``v`` (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 8)


def to_dev(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).bfloat16()


def host(t: torch.Tensor) -> np.ndarray:
    return t.double().cpu().numpy()


def assert_bf16_bar(actual: np.ndarray, expected: np.ndarray) -> None:
    err = np.abs(actual - expected)
    assert np.all(np.isfinite(actual))
    assert err.max() <= BF16_BAR["max_abs"], f"max abs error {err.max():.3e}"
    rel = np.linalg.norm(actual - expected) / max(np.linalg.norm(expected), 1e-30)
    assert rel <= BF16_BAR["rel_l2"], f"relative L2 {rel:.3e}"


def check_bound(actual, expected, mag, *, rerounded: bool) -> None:
    bound = bf16_half_spacing(expected) + (ACCUMULATION_EPS + (BF16_OPERAND_ROUNDING if rerounded else 0.0)) * mag
    err = np.abs(actual - expected)
    assert np.all(err <= bound), f"max excess {np.max(err - bound):.3e} (max err {err.max():.3e})"
    assert_bf16_bar(actual, expected)


@pytest.fixture(params=["default", "streamed", "streamed-split", "quad"])
def conv_path(request, monkeypatch):
    """The library's kernel choice; the streamed kernel for every shape it takes; that
    kernel with its reduction split over workgroups; the K-quarter kernel for every shape
    it takes (64-channel input chunks, 64-channel output tiles)."""
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


def _case(shape, out_c, k, seed, *, offset=0.0):
    rng = np.random.default_rng(seed)
    c = shape[1]
    x = bf16_values(rng.normal(size=shape) + offset)
    w = bf16_values(rng.normal(size=(out_c, c, k, k, k)) * (c * k ** 3) ** -0.5)
    b = rng.normal(size=(out_c,)) * 0.1
    return x, w, b


@pytest.mark.parametrize(("shape", "out_c", "stride"), [
    ((1, 64, 32, 40, 40), 64, 1),    # config 1's shape
    ((2, 32, 6, 7, 9), 128, 1),      # batched, partial bricks
    ((1, 96, 5, 6, 7), 64, 1),       # three channel chunks
    ((1, 24, 7, 6, 9), 40, 2),       # stride 2, odd sizes (general kernel)
    ((1, 512, 4, 4, 4), 128, 1),     # large C on a small grid (split-K)
    ((1, 5, 6, 4, 7), 4, 1),         # C and O not multiples of 8 (scalar staging)
])
def test_bf16_conv3d_matches_float64(pkg, dev, conv_path, shape, out_c, stride) -> None:
    x, w, b = _case(shape, out_c, 3, sum(shape) + out_c)
    xt = to_dev(x.transpose(0, 2, 3, 4, 1), dev)
    y = pkg.ops.nax_conv3d(xt, pkg.ops.pack_weight(to_dev(w, dev)), torch.from_numpy(b).float().to(dev),
                           stride=stride)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    expected = ocv.conv3d(x, w, b, stride=stride)
    mag = ocv.conv3d_magnitude(x, w, b, stride=stride)
    check_bound(host(y).transpose(0, 4, 1, 2, 3), expected, mag, rerounded=False)


@pytest.mark.parametrize(("c", "c0"), [(64, 32), (128, 64)])
def test_bf16_fused_prologue_epilogue_and_concat(pkg, dev, conv_path, c, c0) -> None:
    """concat([x, skip]) through the GroupNorm affine + SiLU prologue (one bf16 rounding of
    the prepared input), per-batch bias + bf16 shift, output scale and a bf16 residual. The
    64 + 64 split is one the K-quarter kernel takes."""
    x, w, _ = _case((2, c, 5, 8, 9), 64, 3, 7 + c, offset=0.4)
    rng = np.random.default_rng(8)
    gamma, beta = rng.normal(size=c), rng.normal(size=c) * 0.3
    aff = onm.group_norm_affine(x, gamma, beta, groups=32, eps=1e-5)
    bias = rng.normal(size=(2, 64)) * 0.1
    shift = bf16_values(rng.normal(size=(2, 64)) * 0.1)
    res = bf16_values(rng.normal(size=(2, 64, 5, 8, 9)))
    xd = x.transpose(0, 2, 3, 4, 1)
    y = pkg.ops.nax_conv3d(to_dev(xd[..., :c0], dev), pkg.ops.pack_weight(to_dev(w, dev)),
                           torch.from_numpy(bias).float().to(dev), x1=to_dev(xd[..., c0:], dev),
                           affine=torch.from_numpy(aff.astype(np.float32)).to(dev), silu=True,
                           shift=to_dev(shift, dev), residual=to_dev(res.transpose(0, 2, 3, 4, 1), dev),
                           output_scale=0.5)
    torch.cuda.synchronize()
    aff32 = aff.astype(np.float32).astype(np.float64)
    prep = bf16_values(onm.silu(onm.apply_affine(x, aff32)))
    conv = ocv.conv3d(prep, w, bias + shift)
    expected = conv * 0.5 + res
    mag = ocv.conv3d_magnitude(prep, w, bias + shift) * 0.5
    check_bound(host(y).transpose(0, 4, 1, 2, 3), expected, mag, rerounded=True)


def test_bf16_upsample_conv(pkg, dev) -> None:
    """The nearest-2x upsample fold with bf16 weights (fp32 sums, one bf16 rounding)."""
    x, w, b = _case((1, 64, 4, 5, 6), 64, 3, 11)
    y = pkg.ops.nax_conv3d(to_dev(x.transpose(0, 2, 3, 4, 1), dev), pkg.ops.pack_upsample_weight(to_dev(w, dev)),
                           torch.from_numpy(b).float().to(dev), upsample=True)
    torch.cuda.synchronize()
    folded = bf16_values(ocv.fold_upsample_weight(w.astype(np.float32)).astype(np.float64))
    expected = ocv.upsample_conv_folded(x, folded, b)
    mag = ocv.upsample_conv_folded(np.abs(x), np.abs(folded), np.abs(b))
    check_bound(host(y).transpose(0, 4, 1, 2, 3), expected, mag, rerounded=False)
    # and the fold stands for the conv of the upsampled input to the folded weights' rounding
    ref = ocv.conv3d(ocv.upsample_nearest2(x), w, b)
    check_bound(host(y).transpose(0, 4, 1, 2, 3), ref, ocv.conv3d_magnitude(ocv.upsample_nearest2(x), w, b),
                rerounded=True)


@pytest.mark.parametrize(("tokens", "c", "o", "ln", "act"), [
    (800, 256, 768, True, None),      # norm1 + q/k/v
    (800, 256, 1024, True, "gelu"),   # norm3 + ff with GELU
    (800, 1024, 256, False, None),    # ff 1024 -> 256 (k-split)
    (77, 768, 512, False, None),      # cross K/V projection
])
def test_bf16_dense(pkg, dev, tokens, c, o, ln, act) -> None:
    """Dense layers (pointwise GEMM over tokens) in bf16, with the fused LayerNorm and the
    GELU epilogue; a residual on the unfused ones."""
    rng = np.random.default_rng(tokens + c + o)
    x = bf16_values(rng.normal(size=(1, tokens, c)))
    w = bf16_values(rng.normal(size=(o, c)) * c ** -0.5)
    b = rng.normal(size=o) * 0.1
    g, bt = 1 + rng.normal(size=c) * 0.2, rng.normal(size=c) * 0.2
    res = None if ln else bf16_values(rng.normal(size=(1, tokens, o)))
    kw = {}
    if ln:
        kw["ln"] = (torch.from_numpy(g).float().to(dev), torch.from_numpy(bt).float().to(dev), 1e-5)
    y = pkg.ops.dense(to_dev(x, dev), pkg.ops.pack_weight(to_dev(w, dev)), torch.from_numpy(b).float().to(dev),
                      residual=None if res is None else to_dev(res, dev), act=act, **kw)
    torch.cuda.synchronize()
    xin = bf16_values(onm.layer_norm(x, g.astype(np.float32), bt.astype(np.float32), 1e-5)) if ln else x
    pre = xin @ w.T + b + (0 if res is None else res)
    mag = np.abs(xin) @ np.abs(w).T + np.abs(b)
    got = host(y)
    if act == "gelu":
        expected = onm.gelu(pre)
        bound = bf16_half_spacing(expected) + 1.13 * (2 * bf16_half_spacing(pre) + (ACCUMULATION_EPS + BF16_OPERAND_ROUNDING) * mag)
        assert np.all(np.abs(got - expected) <= bound)
        assert_bf16_bar(got, expected)
    else:
        check_bound(got, pre, mag, rerounded=ln)


def test_bf16_conv_keeps_group_norm_moments(pkg, dev) -> None:
    """The GroupNorm moments a bf16 conv keeps describe its stored bf16 output."""
    x, w, b = _case((1, 64, 8, 10, 12), 64, 3, 13)
    y = pkg.ops.nax_conv3d(to_dev(x.transpose(0, 2, 3, 4, 1), dev), pkg.ops.pack_weight(to_dev(w, dev)),
                           torch.from_numpy(b).float().to(dev), moments="always")
    torch.cuda.synchronize()
    m = pkg.ops.moments_of(y)
    assert m is not None
    mm = m.double().cpu().numpy()
    n, mean, m2 = mm[..., 0], mm[..., 1], mm[..., 2]
    tot = n.sum(1)
    mu = (n * mean).sum(1) / tot
    var = (m2.sum(1) + (n * (mean - mu[:, None]) ** 2).sum(1)) / tot
    pairs = host(y).reshape(1, -1, 32, 2)
    assert np.array_equal(tot, np.full((1, 32), 2.0 * pairs.shape[1]))
    np.testing.assert_allclose(mu, pairs.mean(axis=(1, 3)), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(var, pairs.var(axis=(1, 3)), rtol=1e-4, atol=1e-7)


def _check_attention(got, want) -> None:
    np.testing.assert_allclose(got, want, atol=1.6e-2, rtol=1.6e-2)
    assert_bf16_bar(got, want)


@pytest.mark.parametrize(("b", "h", "lq", "lk", "d"), [
    (1, 8, 1600, 1600, 64),    # config 2 self attention
    (1, 8, 1600, 77, 64),      # config 2 cross attention
    (1, 8, 800, 800, 32),      # config 5 level-2 attention
    (2, 2, 300, 300, 128),
    (1, 1, 1024, 1024, 256),
])
def test_bf16_attention_matches_float64(pkg, dev, b, h, lq, lk, d) -> None:
    rng = np.random.default_rng(lq + lk + d)
    q, k, v = (bf16_values(rng.normal(size=(b, h, n, d))) for n in (lq, lk, lk))
    o = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d ** -0.5)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16
    _check_attention(host(o), oatt.attention(q, k, v, d ** -0.5))


def test_bf16_attention_with_mask(pkg, dev) -> None:
    """An additive mask removing keys (and a fully masked query row, which gives zeros)."""
    rng = np.random.default_rng(5)
    q, k, v = (bf16_values(rng.normal(size=(1, 2, 96, 64))) for _ in range(3))
    mask = np.where(rng.random((1, 1, 96, 96)) < 0.3, -np.inf, 0.0)
    mask[0, 0, 5, :] = -np.inf
    o = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 0.125,
                          mask=torch.from_numpy(mask.astype(np.float32)).to(dev))
    torch.cuda.synchronize()
    want = oatt.attention(q, k, v, 0.125, mask)
    _check_attention(host(o), want)
    assert np.all(host(o)[:, :, 5] == 0)


def test_dtype_mismatch_is_rejected(pkg, dev) -> None:
    x = torch.zeros((1, 4, 4, 4, 32), dtype=torch.bfloat16, device=dev)
    pk16 = pkg.ops.pack_weight(torch.zeros((32, 32, 3, 3, 3), dtype=torch.float16, device=dev))
    with pytest.raises(ValueError, match="packed weight"):
        pkg.ops.nax_conv3d(x, pk16)
    q = torch.zeros((1, 1, 32, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        pkg.ops.attention(q, q.half(), q, 0.125)
