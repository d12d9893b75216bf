"""Source-order fp16 conv3d and GroupNorm on the GPU (``ldx_conv3d_source_half``,
``ldx_group_norm_source_half`` through ``ops.conv3d_half`` / ``ops.group_norm_half``).

conv3d must equal the oracle and Torch-CPU's fp16 ``F.conv3d`` (oneDNN off) bit for bit --
the reference's own test of its source kernel (tests/test_source_model.py:198-242) -- on the
reference's shapes, on channels-last inputs, and on the first and last output planes of the
config-1 conv. GroupNorm must equal the oracle's restatement of the reference's cascade bit
for bit (affine and output) on the reference's shapes and at config sizes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import source_order as so
from tests.test_source_order import CONV_CASES, GN_SHAPES, conv_case, gn_case, torch_conv_half

pytestmark = pytest.mark.gpu


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint16)


def _dev(a, dev):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"c{c[0]}-o{c[1]}-k{''.join(map(str, c[2]))}-s{c[4]}")
def test_source_conv_is_torch_cpu_bit_for_bit(pkg, dev, case) -> None:
    channels, outputs, kernel, padding, stride, with_bias = case
    x, w, b = conv_case(channels, outputs, kernel, with_bias)
    print(f"conv3d_source_half case {case}", flush=True)
    y = pkg.ops.conv3d_half(_dev(x, dev), _dev(w, dev), _dev(b, dev), padding=padding, stride=stride)
    got = y.cpu().numpy()
    np.testing.assert_array_equal(_bits(got), _bits(so.conv3d_half(x, w, b, padding=padding, stride=stride)))
    np.testing.assert_array_equal(_bits(got), _bits(torch_conv_half(x, w, b, padding, stride)))


def test_source_conv_channels_last_gives_the_same_bits(pkg, dev) -> None:
    x, w, b = conv_case(95, 35, (3, 3, 3), True)
    xd = _dev(x, dev)
    y0 = pkg.ops.conv3d_half(xd, _dev(w, dev), _dev(b, dev), padding=1, stride=2)
    y1 = pkg.ops.conv3d_half(xd.contiguous(memory_format=torch.channels_last_3d), _dev(w, dev), _dev(b, dev),
                             padding=1, stride=2)
    assert y1.is_contiguous(memory_format=torch.channels_last_3d)
    assert torch.equal(y0, y1.contiguous())


def test_source_conv_config1_end_planes(pkg, dev) -> None:
    """The config-1 conv (1 x 64 x 32 x 40 x 40, 3x3x3, padding 1) at full size; output
    planes 0-2 and 29-31 checked bit for bit against the oracle on the input planes they
    read (a 3x3x3 output plane reads the input planes next to it)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 64, 32, 40, 40)).astype(np.float16)
    w = (rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(1728)).astype(np.float16)
    b = (rng.standard_normal(64) * 0.01).astype(np.float16)
    got = pkg.ops.conv3d_half(_dev(x, dev), _dev(w, dev), _dev(b, dev), padding=1, stride=1).cpu().numpy()
    assert got.shape == (1, 64, 32, 40, 40)
    lo = so.conv3d_half(x[:, :, :4], w, b, padding=1, stride=1)[:, :, :3]
    hi = so.conv3d_half(x[:, :, 28:], w, b, padding=1, stride=1)[:, :, 1:]
    np.testing.assert_array_equal(_bits(got[:, :, :3]), _bits(lo))
    np.testing.assert_array_equal(_bits(got[:, :, 29:]), _bits(hi))
    assert np.all(np.isfinite(got.astype(np.float32)))


def test_source_conv_rejects_bad_arguments(pkg, dev) -> None:
    x = torch.zeros((1, 4, 2, 2, 2), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="input channels differ"):
        pkg.ops.conv3d_half(x, torch.zeros((3, 5, 3, 3, 3), dtype=torch.float16, device=dev), None, padding=1,
                            stride=1)
    with pytest.raises(ValueError, match="exceeds the padded input"):
        pkg.ops.conv3d_half(x, torch.zeros((3, 4, 5, 5, 5), dtype=torch.float16, device=dev), None, padding=0,
                            stride=1)
    with pytest.raises(ValueError, match="one value per output channel"):
        pkg.ops.conv3d_half(x, torch.zeros((3, 4, 1, 1, 1), dtype=torch.float16, device=dev),
                            torch.zeros(4, dtype=torch.float16, device=dev), padding=0, stride=1)


def _gn_check(pkg, dev, x, w, b, groups, eps, *, channels_last=False):
    xd = _dev(x, dev)
    if channels_last:
        xd = xd.contiguous(memory_format=torch.channels_last_3d)
    y, aff = pkg.ops.group_norm_half(xd, _dev(w, dev), _dev(b, dev), groups=groups, eps=eps, return_affine=True)
    want_aff, _, _ = so.group_norm_affine_half(x, w, b, groups=groups, eps=eps)
    np.testing.assert_array_equal(aff.cpu().numpy().view(np.uint32), want_aff.view(np.uint32))
    want = so.group_norm_half(x, w, b, groups=groups, eps=eps)
    np.testing.assert_array_equal(_bits(y.contiguous().cpu().numpy()), _bits(want))


@pytest.mark.parametrize("shape", GN_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_source_group_norm_matches_oracle_bit_for_bit(pkg, dev, shape) -> None:
    x, w, b = gn_case(shape)
    print(f"group_norm_source_half shape {shape}", flush=True)
    _gn_check(pkg, dev, x, w, b, 16, 1e-6)


@pytest.mark.parametrize("shape,groups,eps", [((1, 64, 32, 40, 40), 32, 1e-5), ((2, 96, 8, 32, 32), 32, 1e-5),
                                              ((1, 256, 8, 10, 10), 32, 1e-6)],
                         ids=["config1", "strided-groups", "coarse"])
def test_source_group_norm_config_sizes(pkg, dev, shape, groups, eps) -> None:
    x, w, b = gn_case(shape)
    print(f"group_norm_source_half shape {shape} groups {groups}", flush=True)
    _gn_check(pkg, dev, x, w, b, groups, eps)


def test_source_group_norm_channels_last(pkg, dev) -> None:
    x, w, b = gn_case((2, 96, 8, 12, 16))
    _gn_check(pkg, dev, x, w, b, 32, 1e-5, channels_last=True)


def test_source_group_norm_rejects_bad_arguments(pkg, dev) -> None:
    x = torch.zeros((1, 6, 2, 2, 2), dtype=torch.float16, device=dev)
    w = torch.ones(6, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="divisible by num_groups"):
        pkg.ops.group_norm_half(x, w, w, groups=4, eps=1e-6)
    with pytest.raises(ValueError, match="one value per channel"):
        pkg.ops.group_norm_half(x, w[:5], w, groups=3, eps=1e-6)
