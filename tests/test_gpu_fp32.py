"""The FP32 networks on the MI355X: the exact split-fp16 conv / dense mode, fp32 GroupNorm,
LayerNorm and attention, and whole FP32 networks against the reference's recorded FP32
Torch-CPU outputs.

Per-op bound, the reference's own for its exact mode (tests/test_native_kernels.py:37-39,
232-236): |err| <= (8 * 2^-23 + 4 * 2^-22) * sum|terms| + 2^-23 * |expected| against
float64 (twice the magnitude where taps are summed before the split: the upsample conv,
test_native_kernels.py:271-290). Whole networks: the reference's FP32 fixture bound,
atol 2e-6 and rtol 2e-5 (tests/test_equivalence.py:62-73), against ``unet_mask`` (LMNet's
FP32 UNet with cross attention) and ``vq_float32`` (the FP32 decoder, quantized and not).
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import conv as ocv
from oracle import fixture_weights as ofw
from oracle import norm as onm
from tests.conftest import ACCUMULATION_EPS, load_fixture

pytestmark = pytest.mark.gpu

SPLIT_ERROR = 4 * 2.0 ** -22   # tests/test_native_kernels.py:39


def fp32_case(shape, out_c, seed, k=3):
    """tests/test_native_kernels.py:238-252: channel scales over several decades put many
    lo parts near fp16's subnormal range, which the 2^11 scaling must survive."""
    rng = np.random.default_rng(seed)
    scales = np.exp(rng.normal(size=(1, shape[1], 1, 1, 1)) * 2)
    x = (rng.normal(size=shape) * scales).astype(np.float32).astype(np.float64)
    w = (rng.normal(size=(out_c, shape[1], k, k, k)) * (k ** 3 * shape[1]) ** -0.5).astype(np.float32).astype(np.float64)
    b = (rng.normal(size=(out_c,)) * 0.1).astype(np.float32).astype(np.float64)
    return x, w, b


def dev32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def ndhwc(a):
    return np.ascontiguousarray(a.transpose(0, 2, 3, 4, 1))


def host(t):
    return t.double().cpu().numpy()


def assert_near_fp32(actual, expected, magnitude, extra=0.0):
    """``extra``: a relative error of the operands beyond their split (per unit magnitude)."""
    bound = (ACCUMULATION_EPS + SPLIT_ERROR + extra) * magnitude + 2.0 ** -23 * np.abs(expected)
    err = np.abs(actual - expected)
    assert np.all(err <= bound), f"max excess {np.max(err - bound):.3e} (max err {err.max():.3e})"


@pytest.mark.parametrize(("shape", "out_c", "stride"), [
    ((1, 4, 5, 7, 9), 16, 1),     # padded input channels
    ((1, 16, 6, 5, 4), 1, 1),     # a single output channel
    ((2, 24, 7, 6, 9), 40, 2),    # stride 2, padded output channels
    ((1, 64, 4, 6, 5), 128, 1),
    ((1, 32, 16, 20, 20), 64, 1),  # streamed kernel products (2C = 64, 2O = 128)
])
def test_fp32_exact_conv_matches_float64(pkg, dev, shape, out_c, stride) -> None:
    """tests/test_native_kernels.py:255-276."""
    x, w, b = fp32_case(shape, out_c, sum(shape))
    y = pkg.ops.nax_conv3d(dev32(ndhwc(x), dev), pkg.ops.pack_weight(dev32(w, dev)), dev32(b, dev), stride=stride)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    expected = ocv.conv3d(x, w, b, stride=stride)
    mag = ocv.conv3d_magnitude(x, w, b, stride=stride)
    assert_near_fp32(host(y).transpose(0, 4, 1, 2, 3), expected, mag)


def test_fp32_exact_conv_upsamples_with_bias_and_residual(pkg, dev) -> None:
    """tests/test_native_kernels.py:279-306: the conv of a nearest 2x upsampling with a
    per-batch bias and a residual, against float64 at twice the magnitude bound."""
    x, w, _ = fp32_case((2, 32, 3, 5, 4), 16, 23)
    rng = np.random.default_rng(23)
    bias = rng.normal(size=(2, 16)).astype(np.float32).astype(np.float64)
    res = rng.normal(size=(2, 16, 6, 10, 8)).astype(np.float32).astype(np.float64)
    y = pkg.ops.nax_conv3d(dev32(ndhwc(x), dev), pkg.ops.pack_upsample_weight(dev32(w, dev)), dev32(bias, dev),
                           upsample=True, residual=dev32(ndhwc(res), dev))
    torch.cuda.synchronize()
    up = ocv.upsample_nearest2(x)
    expected = ocv.conv3d(up, w) + bias[:, :, None, None, None] + res
    mag = ocv.conv3d_magnitude(up, w) + np.abs(bias)[:, :, None, None, None] + np.abs(res)
    assert_near_fp32(host(y).transpose(0, 4, 1, 2, 3), expected, 2 * mag)


def test_fp32_fused_prologue_shift_scale_and_concat(pkg, dev) -> None:
    """concat([x, skip]) through the fp32 GroupNorm affine + SiLU prologue, per-batch bias
    plus fp32 shift, output scale and residual."""
    x, w, _ = fp32_case((2, 48, 5, 6, 7), 32, 31)
    rng = np.random.default_rng(31)
    gamma, beta = rng.normal(size=48), rng.normal(size=48) * 0.3
    aff = onm.group_norm_affine(x, gamma, beta, groups=16, eps=1e-5).astype(np.float32).astype(np.float64)
    bias = rng.normal(size=(2, 32)).astype(np.float32).astype(np.float64)
    shift = rng.normal(size=(2, 32)).astype(np.float32).astype(np.float64)
    res = rng.normal(size=(2, 32, 5, 6, 7)).astype(np.float32).astype(np.float64)
    xd = ndhwc(x)
    y = pkg.ops.nax_conv3d(dev32(xd[..., :16], dev), pkg.ops.pack_weight(dev32(w, dev)), dev32(bias, dev),
                           x1=dev32(xd[..., 16:], dev), affine=dev32(aff, dev), silu=True, shift=dev32(shift, dev),
                           residual=dev32(ndhwc(res), dev), output_scale=0.5)
    torch.cuda.synchronize()
    prep = onm.silu(onm.apply_affine(x, aff))
    expected = ocv.conv3d(prep, w, bias + shift) * 0.5 + res
    mag = ocv.conv3d_magnitude(prep, w, bias + shift) * 0.5 + np.abs(res)
    # the prepared input is an fp32 value on the device (affine, SiLU) before its split:
    # a few more fp32 ulps per operand
    assert_near_fp32(host(y).transpose(0, 4, 1, 2, 3), expected, mag, extra=4 * 2.0 ** -23)


@pytest.mark.parametrize(("shape", "out_c"), [
    ((1, 64, 19, 32, 38), 64),    # LMNet's full-resolution grid: 128-voxel bricks, two k-groups
    ((1, 40, 16, 24, 32), 72),    # the same tiling with a partial chunk and partial row block
    ((2, 136, 3, 5, 6), 40),      # a small grid: 32-voxel bricks, four k-groups, 3 chunks
])
def test_fp32_exact_conv_tilings_with_group_norm_prologue(pkg, dev, shape, out_c) -> None:
    """The one-pass exact conv's tilings (chosen by grid size) through the fp32 GroupNorm
    affine + SiLU prologue and a residual, against float64 at the exact-mode bound."""
    x, w, b = fp32_case(shape, out_c, sum(shape) + out_c)
    rng = np.random.default_rng(out_c)
    c = shape[1]
    aff = np.stack([rng.normal(size=(shape[0], c)), rng.normal(size=(shape[0], c)) * 0.3], -1)
    aff = aff.astype(np.float32).astype(np.float64)
    res = rng.normal(size=(shape[0], out_c) + shape[2:]).astype(np.float32).astype(np.float64)
    y = pkg.ops.nax_conv3d(dev32(ndhwc(x), dev), pkg.ops.pack_weight(dev32(w, dev)), dev32(b, dev),
                           affine=dev32(aff, dev), silu=True, residual=dev32(ndhwc(res), dev))
    torch.cuda.synchronize()
    prep = onm.silu(onm.apply_affine(x, aff))
    expected = ocv.conv3d(prep, w, b) + res
    mag = ocv.conv3d_magnitude(prep, w, b) + np.abs(res)
    assert_near_fp32(host(y).transpose(0, 4, 1, 2, 3), expected, mag, extra=4 * 2.0 ** -23)


@pytest.mark.parametrize("k", [1, 3])
def test_fp32_unaligned_concat_with_batched_affine(pkg, dev, k) -> None:
    """Channel counts that are not multiples of 4 (element-wise input reads), two batch items
    with their own GroupNorm affine and bias through the pointwise (flattened) and 3x3x3
    tilings, a y slice of a wider tensor."""
    rng = np.random.default_rng(40 + k)
    x, w, _ = fp32_case((2, 19, 3, 9, 11), 37, 40 + k, k=k)
    aff = np.stack([rng.normal(size=(2, 19)), rng.normal(size=(2, 19)) * 0.3], -1).astype(np.float32)
    bias = rng.normal(size=(2, 37)).astype(np.float32).astype(np.float64)
    xd = ndhwc(x)
    out = torch.zeros((2, 3, 9, 11, 40), dtype=torch.float32, device=dev)
    pkg.ops.nax_conv3d(dev32(xd[..., :6], dev), pkg.ops.pack_weight(dev32(w, dev)), dev32(bias, dev),
                       x1=dev32(xd[..., 6:], dev), affine=dev32(aff, dev), silu=True, out=out[..., 1:38])
    torch.cuda.synchronize()
    prep = onm.silu(onm.apply_affine(x, aff.astype(np.float64)))
    expected = ocv.conv3d(prep, w, bias)
    mag = ocv.conv3d_magnitude(prep, w, bias)
    got = host(out)
    assert np.all(got[..., 0] == 0) and np.all(got[..., 38:] == 0)
    assert_near_fp32(got[..., 1:38].transpose(0, 4, 1, 2, 3), expected, mag, extra=4 * 2.0 ** -23)


@pytest.mark.parametrize("act", [None, "gelu", "silu"])
def test_fp32_dense(pkg, dev, act) -> None:
    """Dense layers in the exact mode, with the fp32 GELU / SiLU epilogue."""
    rng = np.random.default_rng(3)
    x = rng.normal(size=(1, 200, 96)).astype(np.float32).astype(np.float64)
    w = (rng.normal(size=(160, 96)) / np.sqrt(96)).astype(np.float32).astype(np.float64)
    b = (rng.normal(size=160) * 0.1).astype(np.float32).astype(np.float64)
    y = pkg.ops.dense(dev32(x, dev), pkg.ops.pack_weight(dev32(w, dev)), dev32(b, dev), act=act)
    torch.cuda.synchronize()
    pre = x @ w.T + b
    mag = np.abs(x) @ np.abs(w).T + np.abs(b)
    got = host(y)
    if act is None:
        assert_near_fp32(got, pre, mag)
    else:
        f = onm.gelu if act == "gelu" else onm.silu
        # the activation's slope is below 1.13; its fp32 evaluation adds a few ulps
        np.testing.assert_allclose(got, f(pre), rtol=4 * 2.0 ** -23, atol=1.13 * ((ACCUMULATION_EPS + SPLIT_ERROR) * mag.max() + 2.0 ** -22))


def test_fp32_group_norm_and_layer_norm(pkg, dev) -> None:
    rng = np.random.default_rng(4)
    x = (rng.normal(size=(2, 48, 5, 6, 7)) * 3 + 1).astype(np.float32).astype(np.float64)
    gamma, beta = rng.normal(size=48).astype(np.float32), rng.normal(size=48).astype(np.float32)
    xd = ndhwc(x)
    aff = host(pkg.ops.group_norm_affine(dev32(xd[..., :32], dev), dev32(gamma, dev), dev32(beta, dev), groups=16,
                                         eps=1e-5, x1=dev32(xd[..., 32:], dev)))
    want = onm.group_norm_affine(x, gamma.astype(np.float64), beta.astype(np.float64), groups=16, eps=1e-5)
    np.testing.assert_allclose(aff, want, rtol=1e-5, atol=1e-6)
    t = rng.normal(size=(300, 96)).astype(np.float32).astype(np.float64) * 2
    g, bb = rng.normal(size=96).astype(np.float32), rng.normal(size=96).astype(np.float32)
    got = host(pkg.ops.layer_norm(dev32(t, dev), dev32(g, dev), dev32(bb, dev), 1e-5))
    np.testing.assert_allclose(got, onm.layer_norm(t, g.astype(np.float64), bb.astype(np.float64), 1e-5),
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize(("lq", "lk", "d"), [(64, 3, 16), (300, 300, 32), (129, 77, 64), (8, 8, 16)])
def test_fp32_attention_matches_float64(pkg, dev, lq, lk, d) -> None:
    rng = np.random.default_rng(lq + lk + d)
    q, k, v = (rng.normal(size=(2, 3, n, d)).astype(np.float32).astype(np.float64) for n in (lq, lk, lk))
    o = pkg.ops.attention(dev32(q, dev), dev32(k, dev), dev32(v, dev), d ** -0.5)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32
    np.testing.assert_allclose(host(o), oatt.attention(q, k, v, d ** -0.5), rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize(("batch", "length", "keys", "heads"), [(1, 96, 64, 2), (2, 32, 160, 1), (1, 1056, 96, 2)])
def test_fp32_attention_reference_cases(pkg, dev, batch, length, keys, heads) -> None:
    """The reference's FP32 flash-attention cases (tests/test_native_kernels.py:395-458:
    32-wide heads, q and k scaled by 2 for peaked rows that move the running maximum) at
    its FP32 bound, atol 2e-5 -- here on the split-fp16 MFMA kernel."""
    rng = np.random.default_rng(length + keys)
    q, k, v = ((rng.normal(size=(batch, heads, n, 32)) * sc).astype(np.float32).astype(np.float64)
               for n, sc in ((length, 2.0), (keys, 2.0), (keys, 1.0)))
    o = pkg.ops.attention(dev32(q, dev), dev32(k, dev), dev32(v, dev), 32 ** -0.5)
    torch.cuda.synchronize()
    got = host(o)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, oatt.attention(q, k, v, 32 ** -0.5), rtol=0, atol=2e-5)


def test_fp32_attention_lmnet_length(pkg, dev) -> None:
    """LMNet's 23,104-token FP32 self-attention (two 32-wide heads; mlx_model.py:74-76,
    _attention.py:27-28) on the split-fp16 MFMA kernel, every 97th query row against float64
    at the reference's FP32 bound (atol 2e-5)."""
    n, heads = 23104, 2
    rng = np.random.default_rng(23104)
    q, k, v = ((rng.normal(size=(1, heads, n, 32)) * sc).astype(np.float32) for sc in (2.0, 2.0, 1.0))
    print(f"fp32 attention {n} tokens x {heads} heads", flush=True)
    o = pkg.ops.attention(dev32(q, dev), dev32(k, dev), dev32(v, dev), 32 ** -0.5)
    torch.cuda.synchronize()
    rows = np.arange(0, n, 97)
    got = host(o)[:, :, rows]
    want = oatt.attention(q[:, :, rows].astype(np.float64), k.astype(np.float64), v.astype(np.float64), 32 ** -0.5)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("d", [32, 64])
def test_fp32_attention_split_kernel_agrees_with_the_valu_kernel(pkg, dev, monkeypatch, d) -> None:
    """The split-fp16 MFMA kernel and the FP32 VALU flash kernel (LDX_ATTN_F32=valu) on the
    same ragged inputs: both within FP32 error of each other."""
    rng = np.random.default_rng(d)
    q, k, v = (rng.normal(size=(2, 3, n, d)).astype(np.float32) for n in (257, 333, 333))
    args = [dev32(t, dev) for t in (q, k, v)]
    mfma = host(pkg.ops.attention(*args, d ** -0.5))
    monkeypatch.setenv("LDX_ATTN_F32", "valu")
    valu = host(pkg.ops.attention(*args, d ** -0.5))
    torch.cuda.synchronize()
    np.testing.assert_allclose(mfma, valu, rtol=2e-5, atol=2e-6)


def test_fp32_unet_matches_recorded_torch(pkg, dev) -> None:
    """LMNet's FP32 network (the ``unet_mask`` recording: cross attention to a context, 16-wide
    heads) at the reference's FP32 bound, atol 2e-6, rtol 2e-5."""
    z = load_fixture("unet_mask")
    assert z["dtype"].item() == "float32"
    c = json.loads(z["config"].item())
    cfg = pkg.unet.UnetConfig(c["model_channels"], c["num_res_blocks"], tuple(c["attention_resolutions"]),
                              tuple(c["channel_mult"]), c["num_head_channels"], c["skip_context"])
    w = ofw.unet_fixture_weights(int(z["weight_seed"]), skip_context=cfg.skip_context)
    net = pkg.unet.LdmUnet(w, cfg, dtype=torch.float32)
    out = net(dev32(z["x"], dev), torch.from_numpy(z["timesteps"]).to(dev), dev32(z["context"], dev))
    torch.cuda.synchronize()
    got, rec = host(out), z["output"].astype(np.float64)
    print(f"unet_mask fp32: max abs {np.abs(got - rec).max():.3e}")
    np.testing.assert_allclose(got, rec, atol=2e-6, rtol=2e-5)


def test_fp32_vq_decoder_matches_recorded_torch(pkg, dev) -> None:
    """The FP32 VQ decoder: decode(z) (fp32 quantization, then the decoder) and the
    unquantized decode against the ``vq_float32`` recording at atol 2e-6, rtol 2e-5."""
    z = load_fixture("vq_float32")
    dec = pkg.vq.VqDecoder(ofw.vq_fixture_weights(int(z["weight_seed"])), dtype=torch.float32)
    zt = dev32(z["z"], dev)
    for key, quantize in (("decoded_unquantized", False), ("decoded", True)):
        got = host(dec(zt, quantize=quantize))
        rec = z[key].astype(np.float64)
        print(f"vq fp32 {key}: max abs {np.abs(got - rec).max():.3e}")
        np.testing.assert_allclose(got, rec, atol=2e-6, rtol=2e-5)
