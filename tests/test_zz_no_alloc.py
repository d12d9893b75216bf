"""ldx_group_norm_affine_noalloc (GroupNorm statistics whose partials live in the library's
per-GPU device array instead of a caller workspace) against ldx_group_norm_affine on the
same inputs: bit for bit, on two calls in a row with the second smaller than the first,
and against the float64 oracle. Calls go through the C ABI."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import norm as onm

pytestmark = pytest.mark.gpu


def _affine_both_ways(pkg, dev, shape, c1, groups, seed):
    """(workspace result, no-alloc result, float64 oracle) for NDHWC ``shape`` whose last
    ``c1`` channels come from a second tensor."""
    lib = pkg._lib.lib
    rng = np.random.default_rng(seed)
    b, d, h, w, c = shape
    c0 = c - c1
    x = (rng.standard_normal(shape) * 2 + 0.5).astype(np.float16)
    gamma = rng.standard_normal(c).astype(np.float32)
    beta = rng.standard_normal(c).astype(np.float32)
    x0 = torch.from_numpy(np.ascontiguousarray(x[..., :c0])).to(dev)
    x1 = torch.from_numpy(np.ascontiguousarray(x[..., c0:])).to(dev) if c1 else None
    g, bt = torch.from_numpy(gamma).to(dev), torch.from_numpy(beta).to(dev)
    voxels = d * h * w
    ws_bytes = lib.ldx_group_norm_workspace_bytes(b, voxels, c, groups)
    assert 0 < ws_bytes <= pkg._lib.GROUP_NORM_SCRATCH_BYTES
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    # Outputs start as NaN so that an entry left unwritten cannot pass as equal.
    want = torch.full((b, c, 2), float("nan"), dtype=torch.float32, device=dev)
    got = torch.full((b, c, 2), float("nan"), dtype=torch.float32, device=dev)
    x1p = x1.data_ptr() if x1 is not None else None
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.ldx_group_norm_affine(x0.data_ptr(), c0, c0, x1p, c1, c1, b, voxels, groups, g.data_ptr(),
                                   bt.data_ptr(), 1e-5, want.data_ptr(), ws.data_ptr(), st)
    assert rc == 0, pkg._lib.last_error()
    rc = lib.ldx_group_norm_affine_noalloc(x0.data_ptr(), c0, c0, x1p, c1, c1, b, voxels, groups, g.data_ptr(),
                                           bt.data_ptr(), 1e-5, got.data_ptr(), st)
    assert rc == 0, pkg._lib.last_error()
    torch.cuda.synchronize()
    ref = onm.group_norm_affine(x.astype(np.float64).transpose(0, 4, 1, 2, 3), gamma.astype(np.float64),
                                beta.astype(np.float64), groups=groups, eps=1e-5)
    return want.cpu().numpy(), got.cpu().numpy(), ref


@pytest.mark.parametrize("order", ["large-then-small"])
def test_noalloc_group_norm_equals_workspace_group_norm(pkg, dev, order) -> None:
    """Two calls in a row through the shared device array: config 1's 64-channel grid at
    batch 2 (256 chunk partials per group), then a smaller 2-tensor concat (32 chunks). The
    second call's partials overwrite a prefix of the first's; both results equal the
    workspace entry point's bit for bit and the float64 GroupNorm to 2e-5."""
    for shape, c1, groups, seed in (((2, 32, 40, 40, 64), 0, 32, 1), ((1, 8, 16, 16, 32), 16, 8, 2)):
        want, got, ref = _affine_both_ways(pkg, dev, shape, c1, groups, seed)
        assert np.all(np.isfinite(got))
        np.testing.assert_array_equal(got, want)
        np.testing.assert_allclose(got.astype(np.float64), ref, rtol=2e-5, atol=2e-5)


def test_noalloc_group_norm_rejects_a_shape_past_its_scratch(pkg, dev) -> None:
    """A shape whose partials would exceed the device array is refused on the host (no
    launch), with a message that names the limit."""
    lib = pkg._lib.lib
    x = torch.zeros(16, dtype=torch.float16, device=dev)
    g = torch.zeros(64, dtype=torch.float32, device=dev)
    out = torch.zeros(2 * 64, dtype=torch.float32, device=dev)
    voxels = 1 << 24
    batch = 8
    assert lib.ldx_group_norm_workspace_bytes(batch, voxels, 64, 32) > pkg._lib.GROUP_NORM_SCRATCH_BYTES
    rc = lib.ldx_group_norm_affine_noalloc(x.data_ptr(), 64, 64, None, 0, 0, batch, voxels, 32, g.data_ptr(),
                                           g.data_ptr(), 1e-5, out.data_ptr(), None)
    assert rc == pkg._lib.LDX_EINVAL
    assert "scratch" in pkg._lib.last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
