"""Parity at the benchmark configurations' full workloads (configs 2-5), on the MI355X.

Every distinct layer of configs 3, 4 and 5 runs at its full size with the fusions the
networks use: the GroupNorm + SiLU prologue, the time-embedding shift, the residual, the
decoder's two-tensor concat, the upsample fold, LayerNorm in front of a dense layer and the
GELU epilogue. Its output is checked against the float64 oracle on a few output D-planes
(3x3x3 convs: the first, a middle and the last plane, so both borders count) or on sampled
rows (pointwise layers); only the input planes those outputs read are copied to the host.
The bound is the reference's per-element error model (tests/test_native_kernels.py:37-39,
98-104): 1/2 ulp of fp16 + 8 * 2^-23 * sum|terms|, + 2^-11 * sum|terms| where an fp16
operand is re-rounded (prologues, folded weights), plus BASELINE's fp16 bar (max abs
2e-2, relative L2 1e-3).

Attention at the configs' shapes is checked against float64 (config 4's 51,200 keys on 256
sampled query rows), with the cross-attention K/V projected from the 77 x 768 context by the
library's own dense layer. GroupNorm statistics run at config 4's largest tensors. The
whole networks of configs 3 and 5 run at full size against the oracle network, and every
network (config 4's decoder too) must repeat bit for bit; config 5's captured DDIM step
must equal the eager step bit for bit.
"""

from __future__ import annotations

import zlib
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import conv as ocv
from oracle import norm as onm
from oracle import unet as oun
from tests.conftest import ACCUMULATION_EPS, OPERAND_ROUNDING, assert_fp16_bar, half_spacing

pytestmark = pytest.mark.gpu

GELU_SLOPE_MAX = 1.13   # max |d gelu / dx| (1.1289 at x = 1.4142)


@dataclass(frozen=True)
class Layer:
    """One layer at its config size: input grid (B, D, H, W), channels c0 (+ c1 from a
    second tensor), O outputs, kernel k (3 or 1), stride / upsample, and its fusions."""

    name: str
    grid: tuple[int, int, int, int]
    c0: int
    out_c: int
    k: int = 3
    c1: int = 0
    stride: int = 1
    upsample: bool = False
    norm: str | None = None      # None, "gn" (GroupNorm affine), "gn_silu", "ln"
    groups: int = 32
    eps: float = 1e-5
    shift: bool = False
    residual: bool = False
    act: str | None = None


# Config 3 (encoder stack) and config 5 (LINet-style UNet, 9 input channels, attention at the
# 8x10x10 and 4x5x5 levels) -- levels 64/128/256/256 at 32x40x40 / 16x20x20 / 8x10x10 / 4x5x5.
UNET_LAYERS = [
    Layer("cfg3 conv_in 4->64", (1, 32, 40, 40), 4, 64),
    Layer("cfg5 conv_in 9->64", (1, 32, 40, 40), 9, 64),
    Layer("L0 in_layers 64->64", (1, 32, 40, 40), 64, 64, norm="gn_silu", shift=True),
    Layer("L0 out_layers 64->64", (1, 32, 40, 40), 64, 64, norm="gn_silu", residual=True),
    Layer("down0 64 stride 2", (1, 32, 40, 40), 64, 64, stride=2),
    Layer("L1 in_layers 64->128", (1, 16, 20, 20), 64, 128, norm="gn_silu", shift=True),
    Layer("L1 skip 64->128", (1, 16, 20, 20), 64, 128, k=1),
    Layer("L1 out_layers 128->128", (1, 16, 20, 20), 128, 128, norm="gn_silu", residual=True),
    Layer("down1 128 stride 2", (1, 16, 20, 20), 128, 128, stride=2),
    Layer("L2 in_layers 128->256", (1, 8, 10, 10), 128, 256, norm="gn_silu", shift=True),
    Layer("L2 skip 128->256", (1, 8, 10, 10), 128, 256, k=1),
    Layer("L2 out_layers 256->256", (1, 8, 10, 10), 256, 256, norm="gn_silu", residual=True),
    Layer("down2 256 stride 2", (1, 8, 10, 10), 256, 256, stride=2),
    Layer("L3 in_layers 256->256", (1, 4, 5, 5), 256, 256, norm="gn_silu", shift=True),
    Layer("L3 out_layers 256->256", (1, 4, 5, 5), 256, 256, norm="gn_silu", residual=True),
    # decoder: concat([x, skip]) read from two tensors, 1x1 skip projections of the concat
    Layer("dec L3 in 256+256->256", (1, 4, 5, 5), 256, 256, c1=256, norm="gn_silu", shift=True),
    Layer("dec L3 skip 256+256->256", (1, 4, 5, 5), 256, 256, c1=256, k=1),
    Layer("dec up 256 4x5x5->8x10x10", (1, 4, 5, 5), 256, 256, upsample=True),
    Layer("dec L2 in 256+128->256", (1, 8, 10, 10), 256, 256, c1=128, norm="gn_silu", shift=True),
    Layer("dec L2 skip 256+128->256", (1, 8, 10, 10), 256, 256, c1=128, k=1),
    Layer("dec up 256 8x10x10->16x20x20", (1, 8, 10, 10), 256, 256, upsample=True),
    Layer("dec L1 in 256+128->128", (1, 16, 20, 20), 256, 128, c1=128, norm="gn_silu", shift=True),
    Layer("dec L1 in 128+64->128", (1, 16, 20, 20), 128, 128, c1=64, norm="gn_silu", shift=True),
    Layer("dec L1 skip 128+64->128", (1, 16, 20, 20), 128, 128, c1=64, k=1),
    Layer("dec up 128 16x20x20->32x40x40", (1, 16, 20, 20), 128, 128, upsample=True),
    Layer("dec L0 in 128+64->64", (1, 32, 40, 40), 128, 64, c1=64, norm="gn_silu", shift=True),
    Layer("dec L0 skip 128+64->64", (1, 32, 40, 40), 128, 64, c1=64, k=1),
    Layer("dec L0 in 64+64->64", (1, 32, 40, 40), 64, 64, c1=64, norm="gn_silu", shift=True),
    Layer("out 64->4", (1, 32, 40, 40), 64, 4, norm="gn_silu"),
    # spatial transformer at 8x10x10 (800 tokens) and 4x5x5 (100 tokens), 256 channels
    Layer("xf proj_in 256 (GroupNorm affine)", (1, 8, 10, 10), 256, 256, k=1, norm="gn", eps=1e-6),
    Layer("xf norm1 + qkv 256->768", (1, 1, 1, 800), 256, 768, k=1, norm="ln"),
    Layer("xf to_out 256 + residual", (1, 1, 1, 800), 256, 256, k=1, residual=True),
    Layer("xf norm2 + to_q 256", (1, 1, 1, 100), 256, 256, k=1, norm="ln"),
    Layer("xf norm3 + ff 256->1024 GELU", (1, 1, 1, 800), 256, 1024, k=1, norm="ln", act="gelu"),
    Layer("xf ff 1024->256 + residual", (1, 1, 1, 800), 1024, 256, k=1, residual=True),
    Layer("xf proj_out 256 + residual", (1, 4, 5, 5), 256, 256, k=1, residual=True),
    Layer("context projection 768->768", (1, 1, 1, 77), 768, 768, k=1),
    Layer("cross K/V 768->512", (1, 1, 1, 77), 768, 512, k=1),
]

# Config 4: VQ decoder 8x32x40x40 -> 1x128x160x160, GroupNorm 16 groups, eps 1e-6.
VQ_LAYERS = [
    Layer("post_quant_conv 8->8", (1, 32, 40, 40), 8, 8, k=1),
    Layer("conv_in 8->256", (1, 32, 40, 40), 8, 256),
    Layer("mid 256->256", (1, 32, 40, 40), 256, 256, norm="gn_silu", groups=16, eps=1e-6),
    Layer("mid 256->256 + residual", (1, 32, 40, 40), 256, 256, norm="gn_silu", groups=16, eps=1e-6,
          residual=True),
    Layer("attn q/k/v 256->768 (GroupNorm affine)", (1, 32, 40, 40), 256, 768, k=1, norm="gn", groups=16,
          eps=1e-6),
    Layer("attn proj_out 256 + residual", (1, 32, 40, 40), 256, 256, k=1, residual=True),
    Layer("up 256 32x40x40->64x80x80", (1, 32, 40, 40), 256, 256, upsample=True),
    Layer("up.2 256->128", (1, 64, 80, 80), 256, 128, norm="gn_silu", groups=16, eps=1e-6),
    Layer("up.2 nin 256->128", (1, 64, 80, 80), 256, 128, k=1),
    Layer("up.2 128->128 + residual", (1, 64, 80, 80), 128, 128, norm="gn_silu", groups=16, eps=1e-6,
          residual=True),
    Layer("up 128 64x80x80->128x160x160", (1, 64, 80, 80), 128, 128, upsample=True),
    Layer("up.1 128->64", (1, 128, 160, 160), 128, 64, norm="gn_silu", groups=16, eps=1e-6),
    Layer("up.1 nin 128->64", (1, 128, 160, 160), 128, 64, k=1),
    Layer("up.1 64->64 + residual", (1, 128, 160, 160), 64, 64, norm="gn_silu", groups=16, eps=1e-6,
          residual=True),
    Layer("up.0 64->32", (1, 128, 160, 160), 64, 32, norm="gn_silu", groups=16, eps=1e-6),
    Layer("up.0 nin 64->32", (1, 128, 160, 160), 64, 32, k=1),
    Layer("up.0 32->32 + residual", (1, 128, 160, 160), 32, 32, norm="gn_silu", groups=16, eps=1e-6,
          residual=True),
    Layer("conv_out 32->1", (1, 128, 160, 160), 32, 1, norm="gn_silu", groups=16, eps=1e-6),
]


def _randn(gen, shape, dev, scale=1.0, offset=0.0, dtype=torch.float16):
    return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * scale + offset).to(dtype)


def _h64(t: torch.Tensor) -> np.ndarray:
    return t.double().cpu().numpy()


def run_layer(pkg, dev, layer: Layer, seed: int):
    """Run ``layer`` on seeded device inputs; returns what the check needs."""
    ops = pkg.ops
    g = torch.Generator(device=dev).manual_seed(seed)
    b, d, h, w = layer.grid
    cin = layer.c0 + layer.c1
    # Inputs offset from zero so that the GroupNorm affine does real work.
    x0 = _randn(g, (b, d, h, w, layer.c0), dev, 1.5, 0.3)
    x1 = _randn(g, (b, d, h, w, layer.c1), dev, 1.5, -0.2) if layer.c1 else None
    wt = _randn(g, (layer.out_c, cin, layer.k, layer.k, layer.k), dev, (cin * layer.k ** 3) ** -0.5)
    bias = _randn(g, (layer.out_c,), dev, 0.1, dtype=torch.float32)
    kw: dict = {}
    affine = ln = None
    gamma = _randn(g, (cin,), dev, 0.2, 1.0, dtype=torch.float32)
    beta = _randn(g, (cin,), dev, 0.2, dtype=torch.float32)
    if layer.norm in ("gn", "gn_silu"):
        affine = ops.group_norm_affine(x0, gamma, beta, groups=layer.groups, eps=layer.eps, x1=x1)
        kw.update(affine=affine, silu=layer.norm == "gn_silu")
    elif layer.norm == "ln":
        ln = (gamma.contiguous(), beta.contiguous(), 1e-5)
        kw.update(ln=ln)
    if layer.shift:
        kw["shift"] = _randn(g, (b, layer.out_c), dev, 0.1)
    out_grid = tuple((2 * n if layer.upsample else ocv.output_extent(n, stride=layer.stride)) for n in (d, h, w))
    res = _randn(g, (b, *out_grid, layer.out_c), dev) if layer.residual else None
    packed = ops.pack_upsample_weight(wt) if layer.upsample else ops.pack_weight(wt)
    y = ops.nax_conv3d(x0, packed, bias, stride=layer.stride, upsample=layer.upsample, residual=res, x1=x1,
                       act=layer.act, **kw)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (b, *out_grid, layer.out_c)
    return dict(x0=x0, x1=x1, w=wt, bias=bias, affine=affine, gamma=gamma, beta=beta, res=res, y=y,
                shift=kw.get("shift"))


def prepared_planes(layer: Layer, r: dict):
    """``plane(i)``: input plane i (B, C, H, W) float64 as the kernel consumes it -- the
    two tensors' channels concatenated, then the prologue (affine, SiLU, one fp16
    rounding) when the layer has one."""
    aff = None if r["affine"] is None else _h64(r["affine"])
    cache: dict[int, np.ndarray] = {}

    def plane(i: int) -> np.ndarray:
        if i not in cache:
            xs = [r["x0"][:, i]] + ([r["x1"][:, i]] if r["x1"] is not None else [])
            p = np.concatenate([_h64(t) for t in xs], axis=-1).transpose(0, 3, 1, 2)  # (B, C, H, W)
            if aff is not None:
                p = p * aff[..., 0][:, :, None, None] + aff[..., 1][:, :, None, None]
                if layer.norm == "gn_silu":
                    p = onm.silu(p)
                p = ocv.f16(p)
            cache[i] = p
        return cache[i]

    return plane


def check_conv_layer(layer: Layer, r: dict) -> None:
    """3x3x3 layer: output planes (first, middle, last) against the float64 oracle."""
    b, d = layer.grid[:2]
    od = r["y"].shape[1]
    planes = sorted({0, od // 2, od - 1})
    plane = prepared_planes(layer, r)
    w64 = _h64(r["w"])
    bias = _h64(r["bias"])[None].repeat(b, 0)
    if r["shift"] is not None:
        bias = bias + _h64(r["shift"])
    if layer.upsample:
        folded = ocv.f16(ocv.fold_upsample_weight(r["w"].float().cpu().numpy()).astype(np.float64))
        expected = ocv.upsample_conv_folded_planes(plane, d, folded, bias, planes=planes)
        mag = ocv.upsample_conv_folded_planes(lambda i: np.abs(plane(i)), d, np.abs(folded), np.abs(bias),
                                              planes=planes)
    else:
        expected = ocv.conv3d_planes(plane, d, w64, bias, stride=layer.stride, planes=planes)
        mag = ocv.conv3d_planes(lambda i: np.abs(plane(i)), d, np.abs(w64), np.abs(bias), stride=layer.stride,
                                planes=planes)
    if r["res"] is not None:
        expected = expected + _h64(r["res"][:, planes]).transpose(0, 4, 1, 2, 3)
    actual = _h64(r["y"][:, planes]).transpose(0, 4, 1, 2, 3)
    rounding = OPERAND_ROUNDING if layer.norm else 0.0
    bound = half_spacing(expected) + (ACCUMULATION_EPS + rounding) * mag
    err = np.abs(actual - expected)
    assert np.all(err <= bound), f"{layer.name}: max excess {np.max(err - bound):.3e} (max err {err.max():.3e})"
    assert_fp16_bar(actual, expected)


def check_pointwise_layer(layer: Layer, r: dict, rows: int = 768) -> None:
    """1x1 / dense layer: sampled output rows (voxels / tokens, first and last included)
    against float64, through the LayerNorm or GroupNorm prologue and the GELU epilogue."""
    b, d, h, w = layer.grid
    n = d * h * w
    rng = np.random.default_rng(n + layer.out_c)
    idx = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, size=min(rows, n))]))
    ti = torch.from_numpy(idx).to(r["y"].device)
    xs = [r["x0"].reshape(b, n, -1)[:, ti]] + ([r["x1"].reshape(b, n, -1)[:, ti]] if r["x1"] is not None else [])
    x = np.concatenate([_h64(t) for t in xs], axis=-1)                       # (B, rows, C)
    if layer.norm in ("gn", "gn_silu"):
        aff = _h64(r["affine"])
        x = x * aff[:, None, :, 0] + aff[:, None, :, 1]
        if layer.norm == "gn_silu":
            x = onm.silu(x)
        x = ocv.f16(x)
    elif layer.norm == "ln":
        x = ocv.f16(onm.layer_norm(x, _h64(r["gamma"]), _h64(r["beta"]), 1e-5))
    w64 = _h64(r["w"]).reshape(layer.out_c, -1)
    bias = _h64(r["bias"])
    pre = x @ w64.T + bias
    mag = np.abs(x) @ np.abs(w64).T + np.abs(bias)
    rounding = OPERAND_ROUNDING if layer.norm else 0.0
    if r["res"] is not None:
        pre = pre + _h64(r["res"].reshape(b, n, -1)[:, ti])
    actual = _h64(r["y"].reshape(b, n, -1)[:, ti])
    if layer.act == "gelu":
        expected = onm.gelu(pre)
        bound = half_spacing(expected) + GELU_SLOPE_MAX * (2 * half_spacing(pre) + (ACCUMULATION_EPS + rounding) * mag)
    else:
        expected = pre
        bound = half_spacing(expected) + (ACCUMULATION_EPS + rounding) * mag
    err = np.abs(actual - expected)
    assert np.all(err <= bound), f"{layer.name}: max excess {np.max(err - bound):.3e} (max err {err.max():.3e})"
    assert_fp16_bar(actual, expected)


@pytest.mark.parametrize("layer", UNET_LAYERS + VQ_LAYERS, ids=lambda l: l.name.replace(" ", "_"))
def test_config_layer_at_full_size(pkg, dev, layer: Layer) -> None:
    """One layer of configs 3, 4 or 5 at its full size, with its fusions."""
    r = run_layer(pkg, dev, layer, seed=zlib.crc32(layer.name.encode()))
    if layer.k == 3:
        check_conv_layer(layer, r)
    else:
        check_pointwise_layer(layer, r)


# ------------------------------------------------------------------------ GroupNorm

@pytest.mark.parametrize(("shape", "c1", "groups", "eps"), [
    ((1, 128, 160, 160, 64), 0, 16, 1e-6),   # config 4 full resolution, 64 channels
    ((1, 128, 160, 160, 32), 0, 16, 1e-6),   # config 4 full resolution, 32 channels
    ((1, 64, 80, 80, 256), 0, 16, 1e-6),     # config 4 up.2 input
    ((1, 32, 40, 40, 192), 64, 32, 1e-5),    # config 5 decoder level-0 concat [x (128), skip (64)]
])
def test_group_norm_at_config_size(pkg, dev, shape, c1, groups, eps) -> None:
    """GroupNorm statistics of config-size tensors (the two-pass path) against float64."""
    g = torch.Generator(device=dev).manual_seed(sum(shape))
    b, c = shape[0], shape[-1]
    x = _randn(g, shape, dev, 2.0, 0.7)
    gamma = _randn(g, (c,), dev, 0.3, 1.0, dtype=torch.float32)
    beta = _randn(g, (c,), dev, 0.3, dtype=torch.float32)
    c0 = c - c1
    x0, x1 = (x[..., :c0], x[..., c0:]) if c1 else (x, None)
    aff = _h64(pkg.ops.group_norm_affine(x0, gamma, beta, groups=groups, eps=eps, x1=x1))
    # float64 statistics per group, accumulated over voxel chunks
    flat = x.reshape(b, -1, groups, c // groups)
    s1 = np.zeros((b, groups))
    step = 1 << 18
    for v0 in range(0, flat.shape[1], step):
        s1 += _h64(flat[:, v0:v0 + step]).sum(axis=(1, 3))
    count = flat.shape[1] * (c // groups)
    mean = s1 / count
    m2 = np.zeros((b, groups))
    for v0 in range(0, flat.shape[1], step):
        m2 += ((_h64(flat[:, v0:v0 + step]) - mean[:, None, :, None]) ** 2).sum(axis=(1, 3))
    var = m2 / count
    scale = _h64(gamma)[None] / np.sqrt(np.repeat(var, c // groups, axis=1) + eps)
    offset = _h64(beta)[None] - scale * np.repeat(mean, c // groups, axis=1)
    np.testing.assert_allclose(aff[..., 0], scale, rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(aff[..., 1], offset, rtol=2e-5, atol=2e-5)


# ------------------------------------------------------------------------ attention

def _check_attention(got: np.ndarray, want: np.ndarray) -> None:
    """The reference's fp16 attention tolerance (tests/test_native_kernels.py:448-450) and
    BASELINE's fp16 bar."""
    np.testing.assert_allclose(got, want, atol=2e-3, rtol=2e-3)
    assert_fp16_bar(got, want)


@pytest.mark.parametrize(("tokens", "heads", "depth"), [(800, 8, 32), (100, 8, 32)])
def test_config5_self_attention(pkg, dev, tokens, heads, depth) -> None:
    """Config 5's self attention at the 8x10x10 and 4x5x5 levels (heads of 32 over 256
    channels), on the projection layout (B, L, heads * d)."""
    g = torch.Generator(device=dev).manual_seed(tokens)
    q, k, v = (_randn(g, (1, tokens, heads * depth), dev) for _ in range(3))
    o = pkg.ops.flash_attention(q, k, v, heads=heads, scale=depth ** -0.5)
    torch.cuda.synchronize()
    want = oatt.attention_projected(_h64(q), _h64(k), _h64(v), heads, depth ** -0.5)
    _check_attention(_h64(o), want)


def _cross_attention(pkg, dev, lq: int, heads: int, depth: int, seed: int, *, context_projection: bool):
    """Queries of width heads * depth against 77 context tokens of width 768 projected to
    K and V by the library's dense layers (the context linear projection first when
    ``context_projection``, as LINet's prepare_denoiser does, mlx_model.py:570-591).
    The projections are checked against float64 at the GEMM bound, and the attention
    against float64 attention of the projections the kernel consumed."""
    ops = pkg.ops
    c = heads * depth
    g = torch.Generator(device=dev).manual_seed(seed)
    ctx = _randn(g, (1, 77, 768), dev)
    q = _randn(g, (1, lq, c), dev)
    wc = _randn(g, (768, 768), dev, 768 ** -0.5)
    wk = _randn(g, (c, 768), dev, 768 ** -0.5)
    wv = _randn(g, (c, 768), dev, 768 ** -0.5)
    src = ops.dense(ctx, ops.pack_weight(wc)) if context_projection else ctx
    kv = ops.dense(src, ops.pack_weight(torch.cat([wk, wv]).contiguous()))
    k, v = kv[..., :c], kv[..., c:]
    o = ops.flash_attention(q, k, v, heads=heads, scale=depth ** -0.5)
    torch.cuda.synchronize()
    s64 = _h64(src)[0]
    w_kv = np.concatenate([_h64(wk), _h64(wv)])
    pre = s64 @ w_kv.T
    bound = half_spacing(pre) + ACCUMULATION_EPS * (np.abs(s64) @ np.abs(w_kv).T)
    assert np.all(np.abs(_h64(kv)[0] - pre) <= bound)
    if context_projection:
        c64 = _h64(ctx)[0]
        pre_c = c64 @ _h64(wc).T
        assert np.all(np.abs(s64 - pre_c) <= half_spacing(pre_c) + ACCUMULATION_EPS * (np.abs(c64) @ np.abs(_h64(wc)).T))
    want = oatt.attention_projected(_h64(q), _h64(k), _h64(v), heads, depth ** -0.5)
    _check_attention(_h64(o), want)


def test_config2_cross_attention_with_projection(pkg, dev) -> None:
    """Config 2's cross attention: 1,600 queries, 8 heads x 64, against 77 context tokens of
    768 channels projected by to_k / to_v (768 -> 512)."""
    _cross_attention(pkg, dev, 1600, 8, 64, 2, context_projection=False)


@pytest.mark.parametrize("tokens", [800, 100])
def test_config5_cross_attention_with_projection(pkg, dev, tokens) -> None:
    """Config 5's cross attention (heads of 32 over 256 channels) after the context linear
    projection (768 -> 768) and the K/V projection (768 -> 512)."""
    _cross_attention(pkg, dev, tokens, 8, 32, tokens, context_projection=True)


def test_config4_mid_attention_on_sampled_queries(pkg, dev) -> None:
    """Config 4's mid-block attention: one head of width 256 over 51,200 tokens. 256 query
    rows (the first, the last and 254 random ones) against all keys in float64."""
    g = torch.Generator(device=dev).manual_seed(4)
    n, c = 51200, 256
    qkv = _randn(g, (1, n, 3 * c), dev)
    q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
    o = pkg.ops.flash_attention(q, k, v, heads=1, scale=c ** -0.5)
    torch.cuda.synchronize()
    rng = np.random.default_rng(4)
    rows = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, 254)]))
    k64, v64 = _h64(k)[0], _h64(v)[0]
    q64 = _h64(q[0, torch.from_numpy(rows).to(dev)])
    want = oatt.attention(q64[None, None], k64[None, None], v64[None, None], c ** -0.5)[0, 0]
    _check_attention(_h64(o[0, torch.from_numpy(rows).to(dev)]), want)


# --------------------------------------------------------------------- whole networks

def _unet(pkg, in_channels, context_dim, attention):
    cfg = pkg.unet.UnetConfig(64, 2, attention, (1, 2, 4, 4), 32, context_dim is None)
    w = pkg.unet.unet_state_dict(cfg, in_channels=in_channels, out_channels=4, context_dim=context_dim, seed=0)
    w16 = {k: v.astype(np.float16) for k, v in w.items()}
    ocfg = oun.UnetConfig(64, 2, attention, (1, 2, 4, 4), 32, context_dim is None)
    return pkg.unet.LdmUnet(w16, cfg), w16, ocfg


def _as_accurate_as_reference_rounding(got: np.ndarray, exact: np.ndarray, half: np.ndarray, what: str) -> None:
    """The fused fp16 network against the float64 oracle network, with the reference's own
    fp16 rounding points (the oracle with half storage) as the yardstick: its relative L2
    error may exceed that scheme's by at most a quarter, and its max abs error stays within
    BASELINE's 2e-2."""
    rl2 = lambda a: float(np.linalg.norm(a - exact) / np.linalg.norm(exact))
    print(f"{what}: rel L2 vs float64 {rl2(got):.3e} (reference rounding {rl2(half):.3e}), "
          f"max abs {np.abs(got - exact).max():.3e} (reference rounding {np.abs(half - exact).max():.3e})")
    assert np.all(np.isfinite(got))
    assert rl2(got) <= 1.25 * rl2(half) + 1e-4, (rl2(got), rl2(half))
    assert np.abs(got - exact).max() <= 2e-2


def test_config3_encoder_stack_at_full_size(pkg, dev) -> None:
    """Config 3 (4-channel 32x40x40 latent, levels 64/128/256/256, two ResBlocks each,
    stride-2 convs) against the float64 oracle network; a rerun repeats bit for bit."""
    net, w16, ocfg = _unet(pkg, 4, None, ())
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 32, 40, 40, 4)).astype(np.float16)
    t = np.array([500], np.int32)
    xt = torch.from_numpy(x).to(dev)
    tt = torch.from_numpy(t).to(dev)
    y1 = net.encoder_stack(xt, tt).clone()
    y2 = net.encoder_stack(xt, tt)
    torch.cuda.synchronize()
    assert tuple(y1.shape) == (1, 4, 5, 5, 256)
    assert torch.equal(y1, y2), "config 3 rerun differs"
    xn = x.transpose(0, 4, 1, 2, 3)
    exact = oun.Unet(w16, ocfg, half=False).encoder_stack(xn, t)
    half = oun.Unet(w16, ocfg, half=True).encoder_stack(xn, t)
    _as_accurate_as_reference_rounding(_h64(y1).transpose(0, 4, 1, 2, 3), exact, half, "config 3")


def test_config5_unet_forward_at_full_size(pkg, dev) -> None:
    """Config 5's network (9 input channels, 32x40x40, self + cross attention at the two
    lowest levels and the middle, 77 x 768 context) against the float64 oracle network; a
    rerun repeats bit for bit."""
    net, w16, ocfg = _unet(pkg, 9, 768, (4, 8))
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 32, 40, 40, 9)).astype(np.float16)
    ctx = rng.standard_normal((1, 77, 768)).astype(np.float16)
    t = np.array([996], np.int32)
    den = net.prepare_denoiser(torch.from_numpy(ctx).to(dev))
    xt, tt = torch.from_numpy(x).to(dev), torch.from_numpy(t).to(dev)
    y1 = den(xt, tt).clone()
    y2 = den(xt, tt)
    torch.cuda.synchronize()
    assert tuple(y1.shape) == (1, 32, 40, 40, 4)
    assert torch.equal(y1, y2), "config 5 rerun differs"
    xn = x.transpose(0, 4, 1, 2, 3)
    exact = oun.Unet(w16, ocfg, half=False).forward(xn, t, ctx)
    half = oun.Unet(w16, ocfg, half=True).forward(xn, t, ctx)
    _as_accurate_as_reference_rounding(_h64(y1).transpose(0, 4, 1, 2, 3), exact, half, "config 5")


def test_config5_captured_step_equals_eager_step(pkg, dev) -> None:
    """Config 5's DDIM step at full size (masked conditioning, 200-step schedule): three
    replays of the captured step graph equal three eager steps bit for bit."""
    net, _, _ = _unet(pkg, 9, 768, (4, 8))
    rng = np.random.default_rng(55)
    ctx = torch.from_numpy(rng.standard_normal((1, 77, 768)).astype(np.float16)).to(dev)
    cond = torch.from_numpy(rng.standard_normal((1, 32, 40, 40, 4)).astype(np.float32)).to(dev)
    mask = np.zeros((1, 32, 40, 40), np.float32)
    mask[0, 10:16, 12:20, 20:28] = (rng.random((6, 8, 8)) < 0.05)
    betas = np.linspace(0.00085 ** 0.5, 0.012 ** 0.5, 1000) ** 2
    alphas = np.cumprod(1.0 - betas).astype(np.float16)
    sampler = pkg.sampling.DdimSampler(alphas, 200)
    prep = sampler.prepare(net.prepare_denoiser(ctx), cond, torch.from_numpy(mask).to(dev), masked_conditioning=True)
    init = torch.from_numpy(rng.standard_normal((1, 32, 40, 40, 4)).astype(np.float32)).to(dev)
    noise = torch.from_numpy(rng.standard_normal((200, 1, 32, 40, 40, 4)).astype(np.float32)).to(dev)
    prep.set_noise(init, noise)
    prep.step.zero_()
    eager = []
    for _ in range(3):
        prep._step()
        eager.append(prep.x.clone())
    prep.capture()
    prep.set_noise(init, noise)
    prep.step.zero_()
    for i in range(3):
        prep.graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(prep.x, eager[i]), f"replay {i} differs from the eager step"
    assert bool(torch.isfinite(prep.x).all())


def test_config4_decoder_at_full_size_repeats(pkg, dev) -> None:
    """Config 4's decoder end to end (8x32x40x40 -> 1x128x160x160): finite, the expected
    shape, and bit-identical on a rerun. Its layers are checked one by one above."""
    w, kw = pkg.vq.vq_decoder_state_dict(latent_channels=8, levels=[(3, 256, True), (2, 128, True), (1, 64, False),
                                                                    (0, 32, False)],
                                         mid_channels=256, mid_attention=True, seed=0)
    dec = pkg.vq.VqDecoder({k: v.astype(np.float16) for k, v in w.items()}, **kw)
    g = torch.Generator(device=dev).manual_seed(44)
    z = _randn(g, (1, 32, 40, 40, 8), dev)
    y1 = dec.decode(z, quantize=False).clone()
    y2 = dec.decode(z, quantize=False)
    torch.cuda.synchronize()
    assert tuple(y1.shape) == (1, 128, 160, 160, 1)
    assert bool(torch.isfinite(y1).all())
    assert torch.equal(y1, y2), "config 4 rerun differs"
