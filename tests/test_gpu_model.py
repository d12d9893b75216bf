"""Whole-network parity on the MI355X: the fp16 UNet and VQ decoder against the
reference's recorded Torch-CPU fixtures (tests/test_equivalence.py:62-96, 151-166:
fp16 atol = rtol = 2e-3), larger random-weight networks against the float64 oracle,
and the graph-captured DDIM loop against the oracle loop."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import fixture_weights as ofw
from oracle import sampling as osm
from oracle import unet as oun
from oracle import vq as ovq
from tests.conftest import assert_fp16_bar, load_fixture

pytestmark = pytest.mark.gpu


def fixture_unet(pkg, name):
    z = load_fixture(name)
    c = json.loads(z["config"].item())
    cfg = dict(model_channels=c["model_channels"], num_res_blocks=c["num_res_blocks"],
               attention_resolutions=tuple(c["attention_resolutions"]), channel_mult=tuple(c["channel_mult"]),
               num_head_channels=c["num_head_channels"], skip_context=c["skip_context"])
    w = ofw.unet_fixture_weights(int(z["weight_seed"]), skip_context=cfg["skip_context"])
    w16 = {k: v.astype(np.float16) for k, v in w.items()}
    net = pkg.unet.LdmUnet(w16, pkg.unet.UnetConfig(**cfg))
    return z, cfg, w16, net


def assert_matches_recording(got: np.ndarray, recorded: np.ndarray, oracle_half: np.ndarray) -> None:
    """A fused-path fp16 network against a Torch-CPU fp16 recording. The recording
    rounds after every op of the source arithmetic (GroupNorm, sigmoid, product, conv,
    residual sum, similarity, softmax); the fused path rounds once per fused op, and
    its attention sums in a different order, so outputs differ by a few fp16 ulps of the
    inner activations. The reference calls its own 2e-3 cross-framework bound
    provisional (tests/test_equivalence.py:66-68). Held here: 3e-3 absolute + 2e-3
    relative per element and the fp16 parity bar against the recording, and 2e-3 against
    the oracle evaluated with the fused path's storage points."""
    rec = recorded.astype(np.float64)
    excess = lambda a: float(np.max(np.abs(a - rec) - (2e-3 + 2e-3 * np.abs(rec))))
    print(f"vs recording: max abs {np.abs(got - rec).max():.3e}, excess over 2e-3 + 2e-3|rec| {excess(got):.3e}; "
          f"reference rounding (oracle): max abs {np.abs(oracle_half - rec).max():.3e}, excess "
          f"{excess(oracle_half):.3e}")
    np.testing.assert_allclose(got, rec, atol=3e-3, rtol=2e-3)
    assert_fp16_bar(got, rec, rel_l2=1e-2)
    np.testing.assert_allclose(got, oracle_half, atol=2e-3, rtol=2e-3)


def test_unet_inpainting_matches_recorded_torch(pkg, dev) -> None:
    """The fp16 fixture UNet (16-wide heads, skip_context) against Torch-CPU upstream."""
    z, cfg, w16, net = fixture_unet(pkg, "unet_inpainting")
    x = torch.from_numpy(z["x"].astype(np.float16)).to(dev)
    out = net(x, torch.from_numpy(z["timesteps"]).to(dev), None)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ora = oun.Unet(w16, oun.UnetConfig(**cfg), half=True).forward(z["x"].astype(np.float16), z["timesteps"], None)
    assert_matches_recording(got, z["output"], ora)


def assert_as_accurate_as_reference_rounding(got: np.ndarray, exact: np.ndarray, half: np.ndarray) -> None:
    """The fused fp16 path against the float64 oracle, with the reference's own fp16
    rounding points (the oracle with half storage) as the yardstick: its error may not
    exceed the reference scheme's by more than a quarter, and it stays within the fp16
    max-abs bar. The two schemes round at different points (the fused path once per
    fused op), so they differ from each other by about the noise each carries."""
    rl2 = lambda a: float(np.linalg.norm(a - exact) / np.linalg.norm(exact))
    assert rl2(got) <= 1.25 * rl2(half) + 1e-4, (rl2(got), rl2(half))
    assert np.abs(got - exact).max() <= 2e-2
    np.testing.assert_allclose(got, half, atol=4e-3, rtol=2e-3)


def test_unet_with_context_matches_oracle(pkg, dev) -> None:
    """The fixture architecture with cross-attention to a context (unet_mask's layout),
    fp16 weights, against the float64 oracle with and without the reference's half
    storage points."""
    z = load_fixture("unet_mask")
    c = json.loads(z["config"].item())
    cfg = dict(model_channels=c["model_channels"], num_res_blocks=c["num_res_blocks"],
               attention_resolutions=tuple(c["attention_resolutions"]), channel_mult=tuple(c["channel_mult"]),
               num_head_channels=c["num_head_channels"], skip_context=False)
    w16 = {k: v.astype(np.float16) for k, v in ofw.unet_fixture_weights(101, skip_context=False).items()}
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 4, 8, 8, 8)).astype(np.float16)
    ctx = rng.standard_normal((2, 3, 6)).astype(np.float16)
    t = np.array([17, 503], np.int32)
    net = pkg.unet.LdmUnet(w16, pkg.unet.UnetConfig(**cfg))
    got = net(torch.from_numpy(x).to(dev), torch.from_numpy(t).to(dev), torch.from_numpy(ctx).to(dev))
    torch.cuda.synchronize()
    half = oun.Unet(w16, oun.UnetConfig(**cfg), half=True).forward(x, t, ctx)
    exact = oun.Unet(w16, oun.UnetConfig(**cfg), half=False).forward(x, t, ctx)
    assert_as_accurate_as_reference_rounding(got.float().cpu().numpy().astype(np.float64), exact, half)


def test_linet_style_unet_matches_oracle(pkg, dev) -> None:
    """A LINet-style network (channels 32/64/128/128, two ResBlocks per level,
    self + cross attention at the two lowest levels, 9 input channels, 64-wide context)
    with random weights at 16x16x16, against the float64 oracle (no half storage): the
    fp16 bar of the whole forward."""
    cfg = pkg.unet.UnetConfig(32, 2, (4, 8), (1, 2, 4, 4), 32, False)
    w = pkg.unet.unet_state_dict(cfg, in_channels=9, out_channels=4, context_dim=64, seed=3)
    w16 = {k: v.astype(np.float16) for k, v in w.items()}
    rng = np.random.default_rng(6)
    x = rng.standard_normal((1, 9, 16, 16, 16)).astype(np.float16)
    ctx = rng.standard_normal((1, 7, 64)).astype(np.float16)
    t = np.array([996], np.int32)
    net = pkg.unet.LdmUnet(w16, cfg)
    got = net(torch.from_numpy(x).to(dev), torch.from_numpy(t).to(dev), torch.from_numpy(ctx).to(dev))
    torch.cuda.synchronize()
    ocfg = oun.UnetConfig(32, 2, (4, 8), (1, 2, 4, 4), 32, False)
    exact = oun.Unet(w16, ocfg, half=False).forward(x, t, ctx)
    half = oun.Unet(w16, ocfg, half=True).forward(x, t, ctx)
    g = got.float().cpu().numpy()
    np.testing.assert_allclose(g, half, atol=2e-2, rtol=2e-2)
    assert_fp16_bar(g, exact, rel_l2=5e-3)


@pytest.mark.parametrize("dtype", ["float16"])
def test_vq_decoder_matches_recorded_torch(pkg, dev, dtype) -> None:
    """decode(z) (nearest-codebook quantization, then the decoder) and decode(z,
    quantize=False) of the fixture decoder (tests/test_equivalence.py:151-166), held as in
    ``assert_matches_recording``."""
    z = load_fixture("vq_" + dtype)
    w16 = {k: v.astype(np.float16) for k, v in ofw.vq_fixture_weights(int(z["weight_seed"])).items()}
    dec = pkg.vq.VqDecoder(w16)
    ora = oun.VqDecoder(w16, half=True)
    z16 = z["z"].astype(np.float16)
    _, q = ovq.quantize4(z16.transpose(0, 2, 3, 4, 1).reshape(-1, 4), w16["quantize.embedding.weight"], np.float16)
    q = q.reshape(1, 2, 2, 2, 4).transpose(0, 4, 1, 2, 3)
    for key, quantize, oracle_in in (("decoded_unquantized", False, z16), ("decoded", True, q)):
        got = dec(torch.from_numpy(z16).to(dev), quantize=quantize)
        torch.cuda.synchronize()
        assert_matches_recording(got.float().cpu().numpy(), z[key], ora.decode(oracle_in))


@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_vq_quantize_matches_recorded_torch_bit_for_bit(pkg, dev, dtype) -> None:
    """The quantize step on the GPU equals the recorded source quantize bit for bit
    (tests/test_equivalence.py:164, ``assert_bits``), in fp16 and in fp32."""
    z = load_fixture("vq_" + dtype)
    t = getattr(torch, dtype)
    w = ofw.vq_fixture_weights(int(z["weight_seed"]))
    dec = pkg.vq.VqDecoder({k: v.astype(np.float16) for k, v in w.items()})
    dec.set_codebook(w["quantize.embedding.weight"].astype(dtype))
    zz = torch.from_numpy(z["z"].transpose(0, 2, 3, 4, 1).copy()).to(dev)
    got = dec.quantize(zz, t)
    torch.cuda.synchronize()
    assert got.dtype == t
    want = z["quantized"].transpose(0, 2, 3, 4, 1)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16 if dtype == "float16" else np.uint32),
                                  want.view(np.uint16 if dtype == "float16" else np.uint32))


def test_scaled_vq_decoder_matches_fp32_decoder(pkg, dev) -> None:
    """The scaled fp16 decoder (_scaled_vq.py) against the recorded fp32 decoder outputs: the
    unquantized decode, and decode(z) with the latent quantized in fp32 against an fp32
    codebook first (_scaled_vq.py:45-49)."""
    z = load_fixture("vq_float32")
    w = ofw.vq_fixture_weights(int(z["weight_seed"]))
    w16 = {k: v.astype(np.float16) for k, v in w.items()}
    dec = pkg.vq.ScaledVqDecoder(w16)
    dec.set_codebook(w["quantize.embedding.weight"].astype(np.float32))
    zt = torch.from_numpy(z["z"]).to(dev)
    got = dec(zt.half(), quantize=False)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.float().cpu().numpy(), z["decoded_unquantized"], atol=2e-3, rtol=2e-3)
    got = dec(zt)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.float().cpu().numpy(), z["decoded"], atol=2e-3, rtol=2e-3)


def test_vq_decoder_with_mid_attention_matches_oracle(pkg, dev) -> None:
    """The generalised decoder (two upsamplings, single-head mid attention at head width
    64) at a small grid against the oracle."""
    w, kw = pkg.vq.vq_decoder_state_dict(latent_channels=8, levels=[(3, 64, True), (2, 32, True), (1, 16, False)],
                                         mid_channels=64, mid_attention=True, seed=4)
    w16 = {k: v.astype(np.float16) for k, v in w.items()}
    rng = np.random.default_rng(8)
    zz = rng.standard_normal((1, 8, 4, 5, 6)).astype(np.float16)
    got = pkg.vq.VqDecoder(w16, **kw)(torch.from_numpy(zz).to(dev), quantize=False)
    torch.cuda.synchronize()
    ora = oun.VqDecoder(w16, half=True, levels=kw["levels"], upsample_levels=kw["upsample_levels"]).decode(zz)
    assert got.shape == ora.shape == (1, 1, 16, 20, 24)
    np.testing.assert_allclose(got.float().cpu().numpy(), ora, atol=2e-2, rtol=2e-2)
    exact = oun.VqDecoder(w16, half=False, levels=kw["levels"], upsample_levels=kw["upsample_levels"]).decode(zz)
    assert_fp16_bar(got.float().cpu().numpy(), exact, rel_l2=5e-3)


def test_graph_captured_ddim_matches_oracle_loop(pkg, dev) -> None:
    """DDIM with the recorded fp16 schedule of the inpainting case (20 alphas, 4 steps)
    driving the fp16 fixture UNet on a seeded 4x4x4 latent (the recorded case's 2x2x2
    latent leaves the UNet's second level 1x1x1, where GroupNorm normalises groups of two
    values and even the float64 and fp16 oracles disagree by 0.2). Every graph replay
    equals the eager loop bit for bit; each step equals the oracle update
    (mlx_sampling.py:116-136) applied to that step's own input state with the oracle
    denoiser, so the bar is the denoiser's fp16 error times the step's coefficients."""
    zd = load_fixture("ddim_inpainting")
    zu, cfg, w16, net = fixture_unet(pkg, "unet_inpainting")
    rng = np.random.default_rng(11)
    img = rng.standard_normal((1, 4, 4, 4, 4)).astype(np.float32)
    m = (rng.random((1, 1, 4, 4, 4)) < 0.5).astype(np.float32)
    initial = rng.standard_normal((1, 4, 4, 4, 4)).astype(np.float32)
    noise_all = rng.standard_normal((4, 1, 4, 4, 4, 4)).astype(np.float32)
    sampler = pkg.sampling.DdimSampler(zd["alphas"], int(zd["steps"]))
    cond = torch.from_numpy(img.transpose(0, 2, 3, 4, 1).copy()).to(dev)
    mask = torch.from_numpy(m[:, 0].copy()).to(dev)
    prep = sampler.prepare(net.prepare_denoiser(None), cond, mask)
    init = torch.from_numpy(initial.transpose(0, 2, 3, 4, 1).copy()).to(dev)
    noise = torch.from_numpy(noise_all.transpose(0, 1, 3, 4, 5, 2).copy()).to(dev)

    onet = oun.Unet(w16, oun.UnetConfig(**cfg), half=True)
    c = osm.ddim_coefficients(zd["alphas"], int(zd["steps"]))
    n = len(c["timesteps"])
    prep.set_noise(init, noise)
    prep.step.zero_()
    m64, img64 = m.astype(np.float64), img.astype(np.float64)
    for it, idx in enumerate(reversed(range(n))):
        x_prev = prep.x.cpu().numpy().astype(np.float64).transpose(0, 4, 1, 2, 3)
        prep._step()
        torch.cuda.synchronize()
        x_new = prep.x.cpu().numpy().astype(np.float64).transpose(0, 4, 1, 2, 3)
        xm = x_prev * m64 + (1 - m64) * img64
        net_in = np.concatenate([xm, m64], axis=1).astype(np.float16)
        eps = onet.forward(net_in, np.array([c["timesteps"][idx]], np.int32), None)[:, :4]
        want = osm.ddim_update(xm, eps, float(c["alphas"][idx]), float(c["previous"][idx]),
                               float(c["sigmas"][idx]), float(c["sqrt_one_minus"][idx]), noise_all[it])
        np.testing.assert_allclose(x_new, want, atol=1e-2, rtol=1e-2)
    # the final blend resets the known region to the conditioning latent
    prep.set_noise(init, noise)
    eager = prep.run(use_graph=False).clone()
    got = eager.cpu().numpy().transpose(0, 4, 1, 2, 3)
    keep = m.repeat(4, axis=1) == 0
    np.testing.assert_array_equal(got[keep], img[keep])
    prep.set_noise(init, noise)
    prep.capture()
    for _ in range(3):
        prep.set_noise(init, noise)
        r = prep.run(use_graph=True).clone()
        torch.cuda.synchronize()
        assert torch.equal(r, eager), "graph replay differs from the eager loop"
    # Noise handed over as host tensors after the capture: copied into the buffer the graph
    # reads, so replays still see it.
    prep.set_noise(init.cpu(), noise.cpu())
    r = prep.run(use_graph=True).clone()
    torch.cuda.synchronize()
    assert torch.equal(r, eager), "graph replay after set_noise with host tensors differs"
