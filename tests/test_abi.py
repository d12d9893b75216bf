"""The C ABI on the CPU: libldx.so loads, exports every function ``include/ldx.h``
declares, the ctypes structs match the C layout, and argument errors are rejected
before any device work (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from tests.conftest import REPO

HEADER = REPO / "include" / "ldx.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ldx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(pkg) -> None:
    names = declared_functions()
    assert len(names) >= 14
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg._lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\b(ldx_[a-z0-9_]+)\b", out))
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    assert set(names) == set(pkg._lib.SIGNATURES), "ctypes signature table out of sync with ldx.h"


def test_ctypes_structs_match_c_layout(pkg, tmp_path) -> None:
    lib = pkg._lib
    fields = {"ldx_conv3d_args": lib.ConvArgs, "ldx_attention_args": lib.AttnArgs,
              "ldx_conv3d_source_args": lib.SourceConvArgs}
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "ldx.h"', "int main(void) {"]
    for cname, cls in fields.items():
        src.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            src.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    src.append("return 0; }")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(REPO / "include"), str(c), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, got):
        cname, what, val = line.split()
        cls = fields[cname]
        want = ctypes.sizeof(cls) if what == "size" else getattr(cls, what).offset
        assert int(val) == want, f"{cname}.{what}: C {val} != ctypes {want}"


def test_abi_version(pkg) -> None:
    assert pkg._lib.lib.ldx_abi_version() == pkg._lib.ABI_VERSION


def _conv_args(lib, **kw):
    a = lib.ConvArgs()
    a.batch, a.in_d, a.in_h, a.in_w = 1, 4, 4, 4
    a.c0, a.c1, a.out_c, a.ksize, a.stride = 8, 0, 8, 3, 1
    a.x0, a.x0_pitch, a.weight, a.y, a.y_pitch = 16, 8, 16, 16, 8
    a.output_scale = 1.0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("bad", [
    {"ksize": 5}, {"stride": 3}, {"batch": 0}, {"in_d": 0}, {"c0": 0}, {"out_c": 0},
    {"ksize": 1, "stride": 2}, {"upsample": 1, "stride": 2}, {"x0": None}, {"weight": None},
    {"c1": 8}, {"x0_pitch": 4}, {"y_pitch": 4}, {"act": 7}, {"residual": 16, "residual_pitch": 2},
    {"dtype": 3}, {"dtype": 7},
])
def test_conv3d_rejects_bad_arguments_before_launch(pkg, bad) -> None:
    lib = pkg._lib
    a = _conv_args(lib, **bad)
    rc = lib.lib.ldx_conv3d(ctypes.byref(a), None)
    assert rc == lib.LDX_EINVAL
    assert "conv3d" in lib.last_error()


def test_attention_rejects_bad_arguments_before_launch(pkg) -> None:
    lib = pkg._lib
    a = lib.AttnArgs()
    a.batch, a.heads, a.q_len, a.kv_len, a.head_dim = 1, 1, 8, 8, 48
    a.q = a.k = a.v = a.o = 256
    assert lib.lib.ldx_attention(ctypes.byref(a), None) == lib.LDX_EINVAL
    assert "head_dim" in lib.last_error()
    a.head_dim = 64
    a.q_stride[1] = 12
    assert lib.lib.ldx_attention(ctypes.byref(a), None) == lib.LDX_EINVAL
    a.q_stride[1] = 64
    a.kv_len = 0
    assert lib.lib.ldx_attention(ctypes.byref(a), None) == lib.LDX_EINVAL
    a.kv_len = 8
    a.dtype = 5   # not an element type
    assert lib.lib.ldx_attention(ctypes.byref(a), None) == lib.LDX_EINVAL
    assert "dtype" in lib.last_error()


def test_small_ops_reject_bad_arguments(pkg) -> None:
    l = pkg._lib.lib
    E = pkg._lib.LDX_EINVAL
    assert l.ldx_pack_weight(16, 0, 4, 3, 16, None) == E
    assert l.ldx_pack_weight(16, 4, 4, 2, 16, None) == E
    assert l.ldx_pack_upsample_weight(None, 4, 4, 0, 16, None) == E
    assert l.ldx_pack_upsample_weight(16, 4, 4, 7, 16, None) == E   # unknown dtype
    assert l.ldx_group_norm_affine(16, 8, 12, None, 0, 0, 1, 10, 5, 16, 16, 1e-5, 16, 16, None) == E
    assert l.ldx_layer_norm(16, 8, 1, 2000, 16, 16, 1e-5, 16, 2000, None) == E
    assert l.ldx_timestep_embedding(16, 1, 7, 16, None) == E
    assert l.ldx_copy_channels(16, 8, 4, 16, 8, 0, 10, 8, None) == E
    assert l.ldx_ddim_prepare(16, 16, 16, 10, 4, 2, 16, 9, None) == E
    assert l.ldx_upsample_nearest2(16, 2, 1, 1, 1, 1, 4, 16, 4, None) == E
    assert l.ldx_group_norm_workspace_bytes(0, 10, 8, 2) == 0
    assert l.ldx_group_norm_workspace_bytes(1, 51200, 64, 32) > 0


@pytest.mark.parametrize("bad", [
    {"x": None}, {"weight": None}, {"y": None}, {"batch": 0}, {"in_c": 0}, {"out_c": 0}, {"kd": 0},
    {"stride": 0}, {"padding": -1}, {"kd": 9, "padding": 0},
])
def test_source_conv_rejects_bad_arguments_before_launch(pkg, bad) -> None:
    lib = pkg._lib
    a = lib.SourceConvArgs(batch=1, in_c=4, in_d=4, in_h=4, in_w=4, out_c=4, kd=3, kh=3, kw=3, stride=1, padding=1,
                           x=16, x_batch_stride=256, x_channel_stride=64, x_voxel_stride=1, weight=16, y=16,
                           y_batch_stride=256, y_channel_stride=64, y_voxel_stride=1)
    for k, v in bad.items():
        setattr(a, k, v)
    assert lib.lib.ldx_conv3d_source_half(ctypes.byref(a), None) == lib.LDX_EINVAL
    assert "conv3d" in lib.last_error()


def test_source_group_norm_rejects_bad_arguments_before_launch(pkg) -> None:
    l = pkg._lib.lib
    E = pkg._lib.LDX_EINVAL
    gn = l.ldx_group_norm_source_half
    # channels not divisible by groups; no weight; an empty tensor; too small a workspace
    assert gn(16, 96, 8, 1, 1, 12, 8, 5, 16, 16, 1e-6, 16, 16, 96, 8, 1, 16, 1 << 20, None) == E
    assert gn(16, 96, 8, 1, 1, 12, 8, 4, None, 16, 1e-6, 16, 16, 96, 8, 1, 16, 1 << 20, None) == E
    assert gn(16, 96, 8, 1, 1, 12, 0, 4, 16, 16, 1e-6, 16, 16, 96, 8, 1, 16, 1 << 20, None) == E
    assert gn(16, 96, 8, 1, 1, 12, 8, 4, 16, 16, 1e-6, 16, 16, 96, 8, 1, 16, 4, None) == E
    assert "workspace" in pkg._lib.last_error()
    ws = l.ldx_group_norm_source_workspace_bytes
    assert ws(1, 12, 8, 5) == 0 and ws(0, 12, 8, 4) == 0
    # chunks of 16 vectors of 8: (1, 64, 51200 voxels, 32 groups) -> 800 chunks, 6 blocks
    assert ws(1, 64, 51200, 32) == 32 * 800 * 16 * 4 + 32 * 6 * 8 * 4


def test_ops_fail_loudly_on_cpu_tensors(pkg) -> None:
    import torch

    x = torch.zeros((1, 2, 2, 2, 8), dtype=torch.float16)
    w = torch.zeros((8, 8, 3, 3, 3), dtype=torch.float16)
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.ops.conv3d(x, w)
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.ops.attention(torch.zeros(1, 1, 4, 64, dtype=torch.float16),
                          torch.zeros(1, 1, 4, 64, dtype=torch.float16),
                          torch.zeros(1, 1, 4, 64, dtype=torch.float16), 0.125)


def test_group_norm_moments_travel_with_the_tensor_the_conv_wrote(pkg) -> None:
    """Host logic of the GroupNorm-moments hand-off (no kernel runs): moments attach to the
    conv's output, are found only for a tensor of matching batch and channel pairs, and are
    cleared when that tensor is written again without them."""
    import torch

    t = torch.zeros(2, 3, 4, 5, 16)
    m = torch.zeros(2, 7, 8, 3)
    assert pkg.ops.moments_of(t) is None
    pkg.ops._set_moments(t, m)
    assert pkg.ops.moments_of(t) is m
    assert pkg.ops.moments_of(t.view(2, 60, 16)) is None           # a view is another tensor
    other = torch.zeros(2, 3, 4, 5, 8)
    pkg.ops._set_moments(other, m)                                  # 8 channels != 2 * 8 pairs
    assert pkg.ops.moments_of(other) is None
    pkg.ops._set_moments(t, None)
    assert pkg.ops.moments_of(t) is None
    assert pkg.ops.moments_of(None) is None


def test_group_norm_moments_are_dropped_after_any_later_write(pkg) -> None:
    """Moments are tagged with the storage's write version: a torch in-place op on the
    tensor, a write through another view of its storage, or a library op writing it via
    ``out=`` (which bumps the shared counter) all make ``moments_of`` return None."""
    import torch

    m = torch.zeros(1, 3, 8, 3)
    t = torch.zeros(1, 2, 2, 2, 16)
    pkg.ops._set_moments(t, m)
    assert pkg.ops.moments_of(t) is m
    t.add_(1.0)
    assert pkg.ops.moments_of(t) is None

    base = torch.zeros(1, 2, 2, 2, 48)
    t = base[..., 16:32]
    pkg.ops._set_moments(t, m)
    assert pkg.ops.moments_of(t) is m
    base[..., 40:].fill_(2.0)                                   # another slice of the same storage
    assert pkg.ops.moments_of(t) is None

    t = torch.zeros(1, 2, 2, 2, 16)
    pkg.ops._set_moments(t, m)
    pkg.ops._wrote(t.view(1, 8, 16))                           # what every out= writer does
    assert pkg.ops.moments_of(t) is None


def test_group_norm_moments_helpers_accept_inference_tensors(pkg) -> None:
    """Under ``torch.inference_mode`` tensors have no version counter: recording a write
    must not raise, and no moments are kept of (or found for) such a tensor, since a later
    torch write to it could not be detected."""
    import torch

    m = torch.zeros(1, 3, 8, 3)
    with torch.inference_mode():
        t = torch.zeros(1, 2, 2, 2, 16)
        assert t.is_inference()
        pkg.ops._wrote(t)
        pkg.ops._set_moments(t, m)
        assert pkg.ops.moments_of(t) is None
        pkg.ops._set_moments(t, None)
        assert pkg.ops.moments_of(t) is None
    pkg.ops._set_moments(t, m)            # outside the mode the tensor is still an inference tensor
    assert pkg.ops.moments_of(t) is None


def test_network_rejects_bf16_at_construction(pkg) -> None:
    """bf16 is an op-level type; a bf16 network (whose GroupNorm / LayerNorm / timestep
    kernels take fp16 or fp32) fails at construction with a clear message, not on its
    first forward."""
    import torch

    with pytest.raises(ValueError, match="network dtype"):
        pkg.layers.SourceLayers({}, device="cpu", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="network dtype"):
        pkg.unet.LdmUnet({}, None, device="cpu", dtype=torch.bfloat16)
