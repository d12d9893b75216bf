"""GroupNorm statistics, LayerNorm, timestep features, SiLU, nearest upsampling,
channel copies and the DDIM step on the MI355X, against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import conv as ocv
from oracle import norm as onm
from oracle import sampling as osm
from oracle import unet as oun
from tests.conftest import half_spacing, load_fixture

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize(("shape", "groups", "split"), [
    ((2, 5, 6, 7, 64), 32, 0), ((1, 32, 40, 40, 64), 32, 0), ((1, 4, 5, 5, 9), 9, 0),
    ((2, 3, 4, 5, 96), 32, 64), ((1, 8, 10, 10, 512), 32, 256), ((1, 2, 2, 2, 4), 4, 0),
    # one-launch path at the config-5 coarse levels: 8 channels per group, several passes of
    # eight voxels per thread, a concat boundary, and 24 channels per group
    ((1, 8, 10, 10, 256), 32, 0), ((2, 4, 5, 5, 256), 32, 0), ((1, 16, 20, 20, 256), 32, 128),
    ((1, 4, 5, 5, 768), 32, 0),
])
def test_group_norm_affine_matches_oracle(pkg, dev, shape, groups, split) -> None:
    rng = np.random.default_rng(sum(shape))
    x = (rng.normal(size=shape) * 2 + 0.5).astype(np.float16)
    c = shape[-1]
    gamma, beta = rng.normal(size=c).astype(np.float32), rng.normal(size=c).astype(np.float32)
    if split:
        aff = pkg.ops.group_norm_affine(to_dev(x[..., :split], dev), to_dev(gamma, dev), to_dev(beta, dev),
                                        groups=groups, eps=1e-5, x1=to_dev(x[..., split:], dev))
    else:
        aff = pkg.ops.group_norm_affine(to_dev(x, dev), to_dev(gamma, dev), to_dev(beta, dev),
                                        groups=groups, eps=1e-5)
    torch.cuda.synchronize()
    ref = onm.group_norm_affine(x.astype(np.float64).transpose(0, 4, 1, 2, 3), gamma, beta, groups=groups,
                                eps=1e-5)
    np.testing.assert_allclose(host(aff), ref, rtol=2e-5, atol=2e-5)
    # deterministic: a second run is bit-identical
    aff2 = pkg.ops.group_norm_affine(to_dev(x, dev), to_dev(gamma, dev), to_dev(beta, dev), groups=groups,
                                     eps=1e-5) if not split else aff
    torch.cuda.synchronize()
    assert torch.equal(aff, aff2)


def _merged(n, mean, m2, axis):
    """Pairwise-free closed form of merging (count, mean, M2) blocks along ``axis``:
    N = sum n, mean = sum n mean / N, M2 = sum M2 + sum n (mean - mean_total)^2."""
    tot = n.sum(axis=axis)
    mu = (n * mean).sum(axis=axis) / tot
    return tot, mu, m2.sum(axis=axis) + (n * (mean - np.expand_dims(mu, axis)) ** 2).sum(axis=axis)


@pytest.mark.parametrize(("n0", "c0", "n1", "c1", "groups"), [
    (3000, 64, 0, 0, 8),       # 12,000 (pair, block) items per group: folded first
    (20000, 32, 0, 0, 16),     # one pair per group, 20,000 blocks
    (2500, 64, 600, 32, 8),    # concat: x0's blocks folded, x1's (3,600 items) merged as they are
])
def test_group_norm_from_many_moment_blocks(pkg, dev, n0, c0, n1, c1, groups) -> None:
    """ldx_group_norm_affine_moments_ws: moments of many blocks folded on many workgroups,
    then merged per group -- against the closed-form merge of the same blocks in float64
    and against the one-pass merge (fp32 rounding apart)."""
    import ctypes

    lib = pkg._lib
    rng = np.random.default_rng(n0 + c0)
    b = 2

    def blocks(n, c):
        cnt = np.full((b, n, c // 2), 2.0 * 32)
        mean = rng.normal(size=(b, n, c // 2)) * 0.5 + 1.0
        m2 = rng.uniform(0.5, 2.0, size=(b, n, c // 2)) * cnt
        return np.stack([cnt, mean, m2], -1)

    m0 = blocks(n0, c0)
    m1 = blocks(n1, c1) if c1 else None
    c = c0 + c1
    gamma, beta = rng.normal(size=c).astype(np.float32), rng.normal(size=c).astype(np.float32)
    d_m0 = to_dev(m0.astype(np.float32), dev)
    d_m1 = to_dev(m1.astype(np.float32), dev) if c1 else None
    g, bt = to_dev(gamma, dev), to_dev(beta, dev)
    ws_bytes = lib.lib.ldx_group_norm_moments_workspace_bytes(n0, c0, n1, c1, b, groups)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    aff = torch.empty((b, c, 2), dtype=torch.float32, device=dev)
    aff1 = torch.empty((b, c, 2), dtype=torch.float32, device=dev)
    p1 = d_m1.data_ptr() if c1 else None
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    lib.check(lib.lib.ldx_group_norm_affine_moments_ws(d_m0.data_ptr(), n0, c0, p1, n1, c1, b, groups, g.data_ptr(),
                                                       bt.data_ptr(), 1e-5, aff.data_ptr(), ws.data_ptr(), ws_bytes, s),
              "moments_ws")
    lib.check(lib.lib.ldx_group_norm_affine_moments(d_m0.data_ptr(), n0, c0, p1, n1, c1, b, groups, g.data_ptr(),
                                                    bt.data_ptr(), 1e-5, aff1.data_ptr(), s), "moments")
    torch.cuda.synchronize()
    # float64 closed form: the group's pairs over every block of both inputs
    gs = c // groups
    scale = np.empty((b, c)); offset = np.empty((b, c))
    for gi in range(groups):
        parts = []
        for lo_pair in range(gi * gs // 2, (gi + 1) * gs // 2):
            if lo_pair < c0 // 2:
                parts.append(m0[:, :, lo_pair].astype(np.float32).astype(np.float64))
            else:
                parts.append(m1[:, :, lo_pair - c0 // 2].astype(np.float32).astype(np.float64))
        allb = np.concatenate(parts, axis=1)
        tot, mu, m2 = _merged(allb[..., 0], allb[..., 1], allb[..., 2], 1)
        rstd = 1.0 / np.sqrt(m2 / tot + 1e-5)
        for ch in range(gi * gs, (gi + 1) * gs):
            scale[:, ch] = gamma[ch] * rstd
            offset[:, ch] = beta[ch] - gamma[ch] * rstd * mu
    a = host(aff)
    np.testing.assert_allclose(a[..., 0], scale, rtol=2e-5, atol=1e-6)
    np.testing.assert_allclose(a[..., 1], offset, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(a, host(aff1), rtol=2e-5, atol=2e-6)


def test_layer_norm_matches_oracle(pkg, dev) -> None:
    rng = np.random.default_rng(2)
    for f in (16, 256, 768):
        x = (rng.normal(size=(3, 37, f)) * 3).astype(np.float16)
        g, b = rng.normal(size=f).astype(np.float32), rng.normal(size=f).astype(np.float32)
        y = pkg.ops.layer_norm(to_dev(x, dev), to_dev(g, dev), to_dev(b, dev), 1e-5)
        torch.cuda.synchronize()
        ref = onm.layer_norm(x.astype(np.float64), g, b, 1e-5)
        assert np.all(np.abs(host(y) - ref) <= 2 * half_spacing(ref) + 1e-5)


def test_timestep_embedding_and_silu(pkg, dev) -> None:
    t = np.array([1, 17, 996], np.int32)
    e = pkg.ops.timestep_embedding(to_dev(t, dev), 64)
    torch.cuda.synchronize()
    ref = oun.timestep_embedding(t, 64)
    assert np.all(np.abs(host(e) - ref) <= 2 * half_spacing(ref) + 1e-6)
    z = load_fixture("unet_activations")
    s = pkg.ops.silu(to_dev(z["silu_input"], dev)).cpu().numpy()
    exp = z["silu_output"]
    ulps = np.abs(s.astype(np.float32) - exp.astype(np.float32)) / np.abs(np.spacing(exp)).astype(np.float32)
    assert ulps.max() <= 1 and np.sqrt(np.mean(ulps ** 2)) <= 0.1


def test_upsample_nearest_and_copy_channels(pkg, dev) -> None:
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 3, 4, 5, 6)).astype(np.float16)
    up = pkg.ops.upsample_nearest2(to_dev(x, dev))
    torch.cuda.synchronize()
    ref = ocv.upsample_nearest2(x.transpose(0, 4, 1, 2, 3)).transpose(0, 2, 3, 4, 1)
    np.testing.assert_array_equal(up.cpu().numpy(), ref)
    dst = torch.zeros((2, 3, 4, 5, 16), dtype=torch.float16, device=dev)
    rc = pkg._lib.lib.ldx_copy_channels(to_dev(x, dev).data_ptr(), 6, 2, dst.data_ptr(), 16, 9, 2 * 3 * 4 * 5,
                                        4, None)
    assert rc == 0
    torch.cuda.synchronize()
    d = dst.cpu().numpy()
    np.testing.assert_array_equal(d[..., 9:13], x[..., 2:6])
    assert np.all(d[..., :9] == 0) and np.all(d[..., 13:] == 0)


def test_ddim_step_kernels_match_oracle(pkg, dev) -> None:
    """The fused prepare/update kernels reproduce the reference DDIM loop on the
    recorded inpainting case (identity-like denoiser evaluated on the host)."""
    z = load_fixture("ddim_inpainting")
    c = osm.ddim_coefficients(z["alphas"], int(z["steps"]))
    img = z["image"].transpose(0, 2, 3, 4, 1).reshape(-1, 4)
    mask = z["mask"].reshape(-1)
    x = to_dev(z["initial"].transpose(0, 2, 3, 4, 1).reshape(-1, 4).astype(np.float32), dev)
    cond, m = to_dev(img.astype(np.float32), dev), to_dev(mask.astype(np.float32), dev)
    net = torch.zeros((8, 9), dtype=torch.float16, device=dev)
    lib = pkg._lib.lib
    xs = z["initial"].astype(np.float64)
    for it, idx in enumerate(reversed(range(len(c["timesteps"])))):
        assert lib.ldx_ddim_prepare(x.data_ptr(), cond.data_ptr(), m.data_ptr(), 8, 4, 4, net.data_ptr(), 9,
                                    None) == 0
        torch.cuda.synchronize()
        n = net.float().cpu().numpy()
        xm = xs * z["mask"] + (1 - z["mask"]) * z["image"]
        np.testing.assert_allclose(n[:, :4], ocv.f16(xm.transpose(0, 2, 3, 4, 1).reshape(-1, 4)), atol=1e-3)
        np.testing.assert_array_equal(n[:, 8], mask.astype(np.float16))
        eps = (np.arange(32, dtype=np.float64).reshape(8, 4) / 50.0).astype(np.float16)
        out = torch.zeros((8, 9), dtype=torch.float16, device=dev)
        out[:, :4] = to_dev(eps, dev)
        coef = to_dev(np.array([c["alphas"][idx], c["previous"][idx], c["sigmas"][idx],
                                c["sqrt_one_minus"][idx]], np.float32), dev)
        noise = to_dev(z["noise"][it].transpose(0, 2, 3, 4, 1).reshape(-1, 4).astype(np.float32), dev)
        assert lib.ldx_ddim_update(x.data_ptr(), out.data_ptr(), 9, noise.data_ptr(), coef.data_ptr(), None,
                                   8, 4, None) == 0
        torch.cuda.synchronize()
        eps_n = eps.astype(np.float64).reshape(1, 2, 2, 2, 4).transpose(0, 4, 1, 2, 3)
        xs = osm.ddim_update(xm, eps_n, float(c["alphas"][idx]), float(c["previous"][idx]),
                             float(c["sigmas"][idx]), float(c["sqrt_one_minus"][idx]), z["noise"][it])
        got = x.cpu().numpy().reshape(1, 2, 2, 2, 4).transpose(0, 4, 1, 2, 3)
        np.testing.assert_allclose(got, xs, rtol=1e-5, atol=1e-5)
