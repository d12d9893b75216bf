"""Pin the CPU oracle: against the reference's recorded Torch-CPU fixtures, against
independent implementations (torch CPU ops, brute-force loops) and closed forms."""

from __future__ import annotations

import json
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import conv as ocv
from oracle import fixture_weights as ofw
from oracle import norm as onm
from oracle import sampling as osm
from oracle import unet as oun
from tests.conftest import load_fixture


def fixture_tol(expected: np.ndarray) -> tuple[float, float]:
    """tests/test_equivalence.py:62-73: fp16 atol = rtol = 2e-3, fp32 2e-6 / 2e-5."""
    return (2e-3, 2e-3) if expected.dtype == np.float16 else (2e-6, 2e-5)


# ------------------------------------------------------------ recorded fixtures

@pytest.mark.parametrize("name", ["unet_mask", "unet_inpainting"])
def test_oracle_unet_matches_recorded_torch(name: str) -> None:
    z = load_fixture(name)
    c = json.loads(z["config"].item())
    cfg = oun.UnetConfig(c["model_channels"], c["num_res_blocks"], tuple(c["attention_resolutions"]),
                         tuple(c["channel_mult"]), c["num_head_channels"], c["skip_context"])
    w = ofw.unet_fixture_weights(int(z["weight_seed"]), skip_context=cfg.skip_context)
    half = z["dtype"].item() == "float16"
    if half:
        w = {k: v.astype(np.float16) for k, v in w.items()}
    x, ctx = z["x"], z["context"]
    if half:
        x, ctx = x.astype(np.float16), ctx.astype(np.float16)
    out = oun.Unet(w, cfg, half=half).forward(x, z["timesteps"], ctx)
    atol, rtol = fixture_tol(z["output"])
    np.testing.assert_allclose(out, z["output"].astype(np.float64), atol=atol, rtol=rtol)


def test_fixture_weight_recipe_changes_output() -> None:
    """A wrong draw order (a plausible mistake in the recipe) breaks the fixture match."""
    z = load_fixture("unet_mask")
    c = json.loads(z["config"].item())
    cfg = oun.UnetConfig(c["model_channels"], c["num_res_blocks"], tuple(c["attention_resolutions"]),
                         tuple(c["channel_mult"]), c["num_head_channels"], c["skip_context"])
    w = ofw.unet_fixture_weights(int(z["weight_seed"]) + 1, skip_context=cfg.skip_context)
    out = oun.Unet(w, cfg, half=False).forward(z["x"], z["timesteps"], z["context"])
    assert np.abs(out - z["output"]).max() > 1e-3


@pytest.mark.parametrize("dtype", ["float32", "float16"])
@pytest.mark.parametrize("half_rounding", [False, True])
def test_oracle_vq_decoder_matches_recorded_torch(dtype: str, half_rounding: bool) -> None:
    if dtype == "float32" and half_rounding:
        pytest.skip("float32 network has no half storage")
    z = load_fixture("vq_" + dtype)
    w = ofw.vq_fixture_weights(int(z["weight_seed"]))
    if dtype == "float16":
        w = {k: v.astype(np.float16) for k, v in w.items()}
    dec = oun.VqDecoder(w, half=half_rounding)
    zz = z["z"].astype(np.float16) if dtype == "float16" else z["z"]
    for key, inp in (("decoded_unquantized", zz), ("decoded", z["quantized"])):
        atol, rtol = fixture_tol(z[key])
        np.testing.assert_allclose(dec.decode(inp), z[key].astype(np.float64), atol=atol, rtol=rtol)


@pytest.mark.parametrize("name", ["ddim_mask", "ddim_inpainting"])
def test_oracle_ddim_matches_recorded_torch(name: str) -> None:
    z = load_fixture(name)
    c = osm.ddim_coefficients(z["alphas"], int(z["steps"]))
    assert np.array_equal(c["timesteps"], z["timesteps"])
    for ours, theirs in (("alphas", "alphas_selected"), ("previous", "previous"),
                         ("sqrt_one_minus", "sqrt_one_minus"), ("sigmas", "sigmas")):
        np.testing.assert_allclose(c[ours], z[theirs], atol=2e-6, rtol=2e-5)

    def denoiser(x, t, cond):  # tests/_fixture_models.py:200-211
        x = x[:, :1] if x.shape[1] == 4 else x
        return x * 0.125 + t[:, None, None, None, None].astype(np.float32) * 0.001 + cond.sum() * 0.01

    mask = z.get("mask")
    out = osm.ddim_sample(denoiser, c, z["condition"], z["image"], z["initial"], z["noise"], mask)
    np.testing.assert_allclose(out, z["output"], atol=2e-6, rtol=2e-5)


def test_oracle_silu_matches_recorded_half_activation() -> None:
    """One fp32 SiLU rounded once to half: <= 1 ulp, RMS <= 0.1 ulp
    (tests/test_equivalence.py:131-148)."""
    z = load_fixture("unet_activations")
    ours = onm.silu(z["silu_input"].astype(np.float64)).astype(np.float16)
    exp = z["silu_output"]
    ulps = np.abs(ours.astype(np.float32) - exp.astype(np.float32)) / np.abs(np.spacing(exp)).astype(np.float32)
    assert ulps.max() <= 1 and np.sqrt(np.mean(ulps ** 2)) <= 0.1


def test_oracle_softmax_matches_recorded_half_softmax() -> None:
    z = load_fixture("unet_activations")
    s = z["softmax_input"].astype(np.float64)
    p = np.exp(s - s.max(-1, keepdims=True))
    ours = (p / p.sum(-1, keepdims=True)).astype(np.float16)
    exp = z["softmax_output"]
    ulps = np.abs(ours.astype(np.float32) - exp.astype(np.float32)) / np.abs(np.spacing(exp)).astype(np.float32)
    assert ulps.max() <= 1


# ---------------------------------------------------------------- conv oracle

@pytest.mark.parametrize("stride", [1, 2])
@pytest.mark.parametrize("shape", [(1, 5, 6, 4, 7), (2, 8, 5, 7, 9)])
def test_conv_oracle_matches_torch(shape, stride) -> None:
    rng = np.random.default_rng(0)
    x = rng.standard_normal(shape)
    w = rng.standard_normal((6, shape[1], 3, 3, 3))
    b = rng.standard_normal(6)
    ours = ocv.conv3d(x, w, b, stride=stride)
    ref = F.conv3d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b), stride=stride,
                   padding=1).numpy()
    np.testing.assert_allclose(ours, ref, rtol=1e-12, atol=1e-12)
    assert ours.shape[2:] == tuple(ocv.output_extent(n, stride=stride) for n in shape[2:])


def test_conv_oracle_brute_force_tiny() -> None:
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 2, 3, 2, 3))
    w = rng.standard_normal((2, 2, 3, 3, 3))
    ours = ocv.conv3d(x, w, stride=1)
    ref = np.zeros_like(ours)
    for o in range(2):
        for d in range(3):
            for h in range(2):
                for ww in range(3):
                    s = 0.0
                    for c in range(2):
                        for kd in range(3):
                            for kh in range(3):
                                for kw in range(3):
                                    i, j, k = d + kd - 1, h + kh - 1, ww + kw - 1
                                    if 0 <= i < 3 and 0 <= j < 2 and 0 <= k < 3:
                                        s += x[0, c, i, j, k] * w[o, c, kd, kh, kw]
                    ref[0, o, d, h, ww] = s
    np.testing.assert_allclose(ours, ref, rtol=1e-12, atol=1e-12)


def test_output_extent_rule() -> None:
    assert [ocv.output_extent(n, stride=2) for n in range(1, 8)] == [1, 1, 2, 2, 3, 3, 4]
    assert ocv.output_extent(5, upsample=True) == 10
    with pytest.raises(ValueError):
        ocv.output_extent(4, stride=3)


def test_upsample_fold_equals_conv_of_nearest_upsampling() -> None:
    """Folded parity filters reproduce conv(upsample(x)) (tests/test_native_kernels.py:196-210)."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 3, 3, 4, 2))
    w = rng.standard_normal((4, 3, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4)
    folded = ocv.fold_upsample_weight(w).astype(np.float64)
    ours = ocv.upsample_conv_folded(x, folded, b)
    ref = ocv.conv3d(ocv.upsample_nearest2(x), w.astype(np.float64), b)
    np.testing.assert_allclose(ours, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("stride", [1, 2])
def test_conv_plane_slabs_equal_torch_planes(stride) -> None:
    """``conv3d_planes`` (input read plane by plane) gives torch's F.conv3d output planes,
    boundary planes included, for odd and even depths."""
    rng = np.random.default_rng(3)
    for shape in ((2, 5, 7, 6, 5), (1, 3, 6, 5, 8)):
        x = rng.standard_normal(shape)
        w = rng.standard_normal((4, shape[1], 3, 3, 3))
        b = rng.standard_normal((shape[0], 4))
        ref = F.conv3d(torch.from_numpy(x), torch.from_numpy(w), None, stride=stride, padding=1).numpy()
        ref = ref + b[:, :, None, None, None]
        od = ref.shape[2]
        planes = [0, od // 2, od - 1]
        ours = ocv.conv3d_planes(lambda i: x[:, :, i], shape[2], w, b, stride=stride, planes=planes)
        np.testing.assert_allclose(ours, ref[:, :, planes], rtol=1e-12, atol=1e-12)


def test_upsample_plane_slabs_equal_conv_of_nearest_upsampling() -> None:
    """``upsample_conv_folded_planes`` gives the planes of ``upsample_conv_folded`` exactly and
    of conv(upsample(x)) to the fold's float32 rounding, for both parities at the borders."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 3, 4, 3, 5))
    w = rng.standard_normal((5, 3, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(5)
    folded = ocv.fold_upsample_weight(w).astype(np.float64)
    planes = [0, 1, 4, 7]
    ours = ocv.upsample_conv_folded_planes(lambda i: x[:, :, i], 4, folded, b, planes=planes)
    np.testing.assert_allclose(ours, ocv.upsample_conv_folded(x, folded, b)[:, :, planes], rtol=1e-12, atol=1e-12)
    ref = ocv.conv3d(ocv.upsample_nearest2(x), w.astype(np.float64), b)[:, :, planes]
    np.testing.assert_allclose(ours, ref, rtol=1e-5, atol=1e-5)


def test_nearest_rules() -> None:
    x = np.arange(2 * 3 * 2).reshape(1, 1, 2, 3, 2).astype(np.float64)
    up = ocv.upsample_nearest2(x)
    for i in range(4):
        for j in range(6):
            for k in range(4):
                assert up[0, 0, i, j, k] == x[0, 0, i // 2, j // 2, k // 2]
    np.testing.assert_array_equal(ocv.resize_nearest(x, (4, 6, 4)), up)
    r = ocv.resize_nearest(x, (3, 2, 5))
    assert r.shape == (1, 1, 3, 2, 5)
    assert r[0, 0, 2, 1, 4] == x[0, 0, math.floor(2 * 2 / 3), math.floor(1 * 3 / 2), math.floor(4 * 2 / 5)]


def test_reference_pack_layout_brute_force() -> None:
    rng = np.random.default_rng(3)
    w = rng.standard_normal((20, 5, 3, 3, 3)).astype(np.float16)
    p = ocv.pack_weight_reference_layout(w)
    assert p.shape == (27 * 16, 32)
    for o in range(32):
        for c in range(16):
            for kd in range(3):
                for kh in range(3):
                    for kw in range(3):
                        tap = kd * 9 + kh * 3 + kw
                        want = w[o, c, kd, kh, kw] if o < 20 and c < 5 else 0
                        assert p[tap * 16 + c, o] == want
    assert ocv.pack_weight_reference_layout(w[:4]).shape == (27 * 16, 16)


def test_reference_upsample_pack_layout_brute_force() -> None:
    rng = np.random.default_rng(4)
    w = rng.standard_normal((3, 2, 3, 3, 3)).astype(np.float16)
    p = ocv.pack_upsample_weight_reference_layout(w)
    assert p.shape == (8, 8 * 16, 16)
    sets = {(0, 0): [0], (0, 1): [1, 2], (1, 0): [0, 1], (1, 1): [2]}
    for par in range(8):
        pd, ph, pw = par >> 2, (par >> 1) & 1, par & 1
        for t in range(8):
            td, th, tw = t >> 2, (t >> 1) & 1, t & 1
            for o in range(3):
                for c in range(2):
                    tot = np.float32(0)
                    for kw in sets[(pw, tw)]:
                        hs = np.float32(0)
                        for kh in sets[(ph, th)]:
                            ds = np.float32(0)
                            for kd in sets[(pd, td)]:
                                ds = np.float32(ds + np.float32(w[o, c, kd, kh, kw]))
                            hs = np.float32(hs + ds)
                        tot = np.float32(tot + hs)
                    assert p[par, t * 16 + c, o] == np.float16(tot)


# --------------------------------------------------------- norm / activations

def test_group_norm_oracle_matches_torch() -> None:
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 8, 3, 4, 5)) * 3 + 1
    g, b = rng.standard_normal(8), rng.standard_normal(8)
    ours = onm.group_norm(x, g, b, groups=4, eps=1e-5)
    ref = F.group_norm(torch.from_numpy(x), 4, torch.from_numpy(g), torch.from_numpy(b), eps=1e-5).numpy()
    np.testing.assert_allclose(ours, ref, rtol=1e-10, atol=1e-10)


def test_layer_norm_and_gelu_oracles_match_torch() -> None:
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 7, 16)) * 2
    g, b = rng.standard_normal(16), rng.standard_normal(16)
    np.testing.assert_allclose(onm.layer_norm(x, g, b, 1e-5),
                               F.layer_norm(torch.from_numpy(x), (16,), torch.from_numpy(g),
                                            torch.from_numpy(b), 1e-5).numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(onm.gelu(x), F.gelu(torch.from_numpy(x)).numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(onm.silu(x), F.silu(torch.from_numpy(x)).numpy(), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ attention

@pytest.mark.parametrize("lk", [5, 77])
def test_attention_oracle_matches_torch_sdpa(lk: int) -> None:
    rng = np.random.default_rng(7)
    q = rng.standard_normal((2, 3, 11, 16))
    k = rng.standard_normal((2, 3, lk, 16))
    v = rng.standard_normal((2, 3, lk, 16))
    mask = np.where(rng.random((2, 1, 11, lk)) < 0.2, -np.inf, 0.0)
    mask[..., 0] = 0.0
    for m in (None, mask):
        ours = oatt.attention(q, k, v, 0.3, m)
        ref = F.scaled_dot_product_attention(
            torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
            attn_mask=None if m is None else torch.from_numpy(m), scale=0.3).numpy()
        np.testing.assert_allclose(ours, ref, rtol=1e-10, atol=1e-10)


def test_attention_oracle_closed_forms() -> None:
    rng = np.random.default_rng(8)
    k = rng.standard_normal((1, 1, 9, 4))
    v = rng.standard_normal((1, 1, 9, 4))
    # zero queries: uniform weights -> mean of v (the reference's tie case)
    out = oatt.attention(np.zeros((1, 1, 3, 4)), k, v, 1.0)
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(axis=2, keepdims=True), out.shape), atol=1e-12)
    # fully masked row -> zeros
    m = np.full((1, 1, 3, 9), -np.inf)
    assert np.all(oatt.attention(np.ones((1, 1, 3, 4)), k, v, 1.0, m) == 0)


# ------------------------------------------------------------------- schedule

def test_timestep_schedule() -> None:
    t = osm.lesion_diffusion_timesteps(200)
    assert len(t) == 200 and t[0] == 1 and t[-1] == 996 and t[1] - t[0] == 5
    assert len(osm.lesion_diffusion_timesteps(6)) == 7
    for bad in (3, 1000, 0, True):
        with pytest.raises(ValueError):
            osm.lesion_diffusion_timesteps(bad)


def test_timestep_embedding_closed_form() -> None:
    e = oun.timestep_embedding(np.array([0, 17]), 8)
    np.testing.assert_allclose(e[0], [1, 1, 1, 1, 0, 0, 0, 0], atol=0)
    f = np.exp(-math.log(10000) * np.arange(4) / 4)
    np.testing.assert_allclose(e[1], np.concatenate([np.cos(17 * f), np.sin(17 * f)]), rtol=1e-5, atol=1e-6)


# -------------------------------------------------- torch fp32 CPU baseline networks

def test_torch_cpu_unet_matches_float64_oracle() -> None:
    """The benchmark's torch-fp32 CPU network (oracle/torch_cpu.py) computes the oracle
    network: the recorded ``unet_mask`` architecture with cross attention to a context (both
    attentions, the concat decoder, upsampling) and its encoder stack agree with the float64
    oracle to fp32 accuracy."""
    import importlib
    import json

    from oracle import fixture_weights as ofw
    from oracle import unet as oun

    tcpu = importlib.import_module("oracle.torch_cpu")
    z = load_fixture("unet_mask")
    c = json.loads(z["config"].item())
    cfg = oun.UnetConfig(c["model_channels"], c["num_res_blocks"], tuple(c["attention_resolutions"]),
                         tuple(c["channel_mult"]), c["num_head_channels"], False)
    w = ofw.unet_fixture_weights(101, skip_context=False)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 4, 8, 8, 8))
    ctx = rng.standard_normal((1, 3, 6))
    t = np.array([417], np.int32)
    want = oun.Unet(w, cfg, half=False).forward(x, t, ctx)
    got = tcpu.TorchUnet(w, cfg).forward(x, t, ctx).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    want_e = oun.Unet(w, cfg, half=False).encoder_stack(x, t)
    got_e = tcpu.TorchUnet(w, cfg).encoder_stack(x, t).numpy()
    np.testing.assert_allclose(got_e, want_e, rtol=1e-4, atol=1e-5)


def test_torch_cpu_vq_decoder_matches_float64_oracle() -> None:
    """The torch-fp32 CPU VQ decoder (mid attention, two upsamplings) against the oracle."""
    import importlib

    lay = importlib.import_module("oracle.torch_cpu")
    from oracle import fixture_weights as ofw
    from oracle import unet as oun

    w = ofw.vq_fixture_weights(201)
    rng = np.random.default_rng(10)
    z = rng.standard_normal((1, 4, 2, 3, 2))
    want = oun.VqDecoder(w, half=False).decode(z)
    got = lay.TorchVqDecoder(w).decode(z).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------- VQ codebook search

def _round_fraction_f32(x) -> np.float32:
    """The float32 nearest the exact rational ``x`` (ties to even), by comparing neighbours."""
    from fractions import Fraction

    f = np.float32(float(x))
    cands = [f, np.nextafter(f, np.float32(-np.inf)), np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - x),
                                     int(np.frombuffer(np.float32(c).tobytes(), np.uint32)[0]) & 1))
    return np.float32(best)


def test_fma32_is_correctly_rounded() -> None:
    """``oracle.vq.fma32`` equals the exactly rounded a * b + c: on random operands of mixed
    magnitudes and on hand-built cases whose product is a float32 midpoint and whose addend
    is too small for the float64 sum (plain float64 evaluation rounds those the wrong way)."""
    from fractions import Fraction

    from oracle import vq as ovq

    rng = np.random.default_rng(21)
    a = (rng.standard_normal(400) * 2.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    b = (rng.standard_normal(400) * 2.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    c = (-(a.astype(np.float64) * b) * (1 + rng.standard_normal(400) * 1e-6)).astype(np.float32)
    # a * b = 24929 * (673 / 2^24) = 1 + 2^-24 exactly, halfway between 1 and 1 + 2^-23.
    ma, mb = np.float32(24929.0), np.float32(673.0 * 2.0 ** -24)
    a = np.concatenate([a, [ma, ma, ma]]).astype(np.float32)
    b = np.concatenate([b, [mb, mb, mb]]).astype(np.float32)
    c = np.concatenate([c, [2.0 ** -80, -(2.0 ** -80), 0.0]]).astype(np.float32)
    got = ovq.fma32(a, b, c)
    want = np.array([_round_fraction_f32(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
                     for x, y, z in zip(a, b, c)], np.float32)
    np.testing.assert_array_equal(got, want)
    assert got[-3] == np.float32(1 + 2.0 ** -23) and got[-2] == np.float32(1.0) and got[-1] == np.float32(1.0)


def test_vq_selection_rule_closed_forms() -> None:
    """The selection is the first NaN, else the first smallest distance: ties keep the lower
    index, -0 equals +0, +inf rows give index 0."""
    from oracle import vq as ovq

    d = np.array([[3, 1, 1, 2], [3, np.nan, 1, np.nan], [np.inf, np.inf, np.inf, np.inf],
                  [0.0, -0.0, -1, -1], [5, 4, 3, np.nan]], np.float32)
    assert np.argmin(d, axis=1).tolist() == [1, 1, 0, 2, 3]
    # a two-code book where the latent sits exactly between the codes: a tie, index 0
    cb = np.array([[0, 0, 0, 0], [2, 0, 0, 0]], np.float32)
    for t in (np.float16, np.float32):
        assert ovq.nearest_codebook4(np.array([[1, 0, 0, 0]], t), cb, t).tolist() == [0]
        assert ovq.nearest_codebook4(np.array([[1.75, 0, 0, 0]], t), cb, t).tolist() == [1]


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_vq_oracle_matches_recorded_quantize_bit_for_bit(dtype: str) -> None:
    """The recorded source quantize of the fixture latent (tests/test_equivalence.py:164,
    ``assert_bits``) with the fixture codebook, reproduced exactly."""
    from oracle import vq as ovq

    z = load_fixture("vq_" + dtype)
    t = np.dtype(dtype)
    cb = ofw.vq_fixture_weights(int(z["weight_seed"]))["quantize.embedding.weight"].astype(t)
    flat = z["z"].astype(t).transpose(0, 2, 3, 4, 1).reshape(-1, 4)
    _, q = ovq.quantize4(flat, cb, t)
    want = z["quantized"].transpose(0, 2, 3, 4, 1).reshape(-1, 4)
    assert q.dtype == want.dtype
    np.testing.assert_array_equal(q.view(np.uint16 if t == np.float16 else np.uint32),
                                  want.view(np.uint16 if t == np.float16 else np.uint32))
