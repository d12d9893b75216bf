"""ctypes binding of ``libldx.so`` (the C ABI declared in ``include/ldx.h``).

The library is loaded from this package directory; if it is missing, or a symbol the
header declares is absent, import fails loudly -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_NAME = "libldx.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

LDX_OK = 0
LDX_EINVAL = -1
LDX_EHIP = -2
ACT_NONE = 0
ACT_GELU = 1
ACT_SILU = 2
DTYPE_F16 = 0
DTYPE_F32 = 1
DTYPE_BF16 = 2
GROUP_NORM_SCRATCH_BYTES = 4 << 20   # LDX_GROUP_NORM_SCRATCH_BYTES

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p
c_fp = ctypes.POINTER(ctypes.c_float)


class ConvArgs(ctypes.Structure):
    """Mirror of ``ldx_conv3d_args``."""

    _fields_ = [
        ("batch", c_i32), ("in_d", c_i32), ("in_h", c_i32), ("in_w", c_i32),
        ("c0", c_i32), ("c1", c_i32), ("out_c", c_i32), ("ksize", c_i32),
        ("stride", c_i32), ("upsample", c_i32),
        ("x0", c_vp), ("x0_pitch", c_i64),
        ("x1", c_vp), ("x1_pitch", c_i64),
        ("weight", c_vp),
        ("bias", c_vp), ("bias_batched", c_i32),
        ("shift", c_vp), ("shift_pitch", c_i64),
        ("affine", c_vp), ("silu", c_i32),
        ("residual", c_vp), ("residual_pitch", c_i64),
        ("output_scale", c_f32), ("act", c_i32),
        ("y", c_vp), ("y_pitch", c_i64),
        ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t),
        ("dtype", c_i32),
    ]


class AttnArgs(ctypes.Structure):
    """Mirror of ``ldx_attention_args``."""

    _fields_ = [
        ("batch", c_i32), ("heads", c_i32), ("q_len", c_i32), ("kv_len", c_i32),
        ("head_dim", c_i32),
        ("q", c_vp), ("q_stride", c_i64 * 3),
        ("k", c_vp), ("k_stride", c_i64 * 3),
        ("v", c_vp), ("v_stride", c_i64 * 3),
        ("o", c_vp), ("o_stride", c_i64 * 3),
        ("scale", c_f32),
        ("mask", c_vp), ("mask_stride", c_i64 * 4),
        ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t),
        ("dtype", c_i32),
    ]


class SourceConvArgs(ctypes.Structure):
    """Mirror of ``ldx_conv3d_source_args``."""

    _fields_ = [
        ("batch", c_i32), ("in_c", c_i32), ("in_d", c_i32), ("in_h", c_i32), ("in_w", c_i32),
        ("out_c", c_i32), ("kd", c_i32), ("kh", c_i32), ("kw", c_i32),
        ("stride", c_i32), ("padding", c_i32),
        ("x", c_vp), ("x_batch_stride", c_i64), ("x_channel_stride", c_i64), ("x_voxel_stride", c_i64),
        ("weight", c_vp), ("bias", c_vp),
        ("y", c_vp), ("y_batch_stride", c_i64), ("y_channel_stride", c_i64), ("y_voxel_stride", c_i64),
    ]


# name -> (restype, argtypes); every function declared in include/ldx.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ldx_last_error": (ctypes.c_char_p, []),
    "ldx_abi_version": (c_i32, []),
    "ldx_conv3d_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(ConvArgs)]),
    "ldx_conv3d": (c_i32, [ctypes.POINTER(ConvArgs), c_vp]),
    "ldx_conv3d_stats_chunks": (c_i64, [ctypes.POINTER(ConvArgs)]),
    "ldx_conv3d_stats": (c_i32, [ctypes.POINTER(ConvArgs), c_vp, c_vp]),
    "ldx_dense_ln": (c_i32, [ctypes.POINTER(ConvArgs), c_vp, c_vp, c_f32, c_vp]),
    "ldx_packed_weight_elems": (ctypes.c_size_t, [c_i32, c_i32, c_i32, c_i32]),
    "ldx_pack_weight": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "ldx_pack_upsample_weight": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "ldx_group_norm_workspace_bytes": (ctypes.c_size_t, [c_i32, c_i64, c_i32, c_i32]),
    "ldx_group_norm_affine_noalloc": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_i64, c_i32,
                                              c_vp, c_vp, c_f32, c_vp, c_vp]),
    "ldx_group_norm_affine_moments": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_i32,
                                               c_vp, c_vp, c_f32, c_vp, c_vp]),
    "ldx_group_norm_moments_workspace_bytes": (ctypes.c_size_t, [c_i64, c_i32, c_i64, c_i32, c_i32, c_i32]),
    "ldx_group_norm_affine_moments_ws": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_i32,
                                                 c_vp, c_vp, c_f32, c_vp, c_vp, ctypes.c_size_t, c_vp]),
    "ldx_group_norm_affine": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_i64, c_i32,
                                      c_vp, c_vp, c_f32, c_vp, c_vp, c_vp]),
    "ldx_layer_norm": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_i64, c_vp]),
    "ldx_attention_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(AttnArgs)]),
    "ldx_attention": (c_i32, [ctypes.POINTER(AttnArgs), c_vp]),
    "ldx_timestep_embedding": (c_i32, [c_vp, c_i32, c_i32, c_vp, c_vp]),
    "ldx_silu": (c_i32, [c_vp, c_i64, c_vp, c_vp]),
    "ldx_copy_channels": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i64, c_i32, c_vp]),
    "ldx_upsample_nearest2": (c_i32, [c_vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp]),
    "ldx_ddim_prepare": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_i64, c_vp]),
    "ldx_ddim_update": (c_i32, [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_i32, c_vp]),
    "ldx_ddim_timestep": (c_i32, [c_vp, c_vp, c_i32, c_vp, c_vp]),
    "ldx_step_advance": (c_i32, [c_vp, c_vp]),
    "ldx_vq_squared_norms4": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_vp]),
    "ldx_pack_weight_exact": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "ldx_packed_weight_exact_elems": (ctypes.c_size_t, [c_i32, c_i32, c_i32]),
    "ldx_group_norm_affine_f32": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_i64, c_i32,
                                          c_vp, c_vp, c_f32, c_vp, c_vp]),
    "ldx_layer_norm_f32": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_vp, c_vp, c_f32, c_vp, c_i64, c_vp]),
    "ldx_timestep_embedding_f32": (c_i32, [c_vp, c_i32, c_i32, c_vp, c_vp]),
    "ldx_vq_nearest4": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "ldx_conv3d_source_half": (c_i32, [ctypes.POINTER(SourceConvArgs), c_vp]),
    "ldx_group_norm_source_workspace_bytes": (ctypes.c_size_t, [c_i32, c_i32, c_i64, c_i32]),
    "ldx_group_norm_source_half": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_i32, c_i32, c_i64, c_i32, c_vp, c_vp,
                                           c_f32, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, ctypes.c_size_t,
                                           c_vp]),
}

ABI_VERSION = 12


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_NAME} not found at {LIB_PATH}; build it with __graft_entry__.build() "
            "(hipcc --offload-arch=gfx950). There is no CPU fallback.")
    # torch first: its HIP runtime (soname libamdhip64.so.7) then satisfies the library's
    # dependency, so the process holds one runtime and the library sees torch's device
    # and streams. Loaded the other way round, two runtimes coexist and the library's
    # reports no device.
    import torch  # noqa: F401
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the library lacks a declared symbol
        fn.restype = res
        fn.argtypes = args
    if lib.ldx_abi_version() != ABI_VERSION:
        raise ImportError(f"{LIB_NAME} ABI version {lib.ldx_abi_version()} != {ABI_VERSION}")
    return lib


lib = _load()


def last_error() -> str:
    msg = lib.ldx_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Raise ``ValueError`` for a rejected argument and ``RuntimeError`` for a HIP error,
    the split the reference makes between its own checks and Metal failures
    (_nax_conv.py:506-510, 553-554; medmlx.py:761-763)."""
    if rc == LDX_OK:
        return
    if rc == LDX_EINVAL:
        raise ValueError(f"{what}: {last_error()}")
    raise RuntimeError(f"{what}: {last_error()}")
