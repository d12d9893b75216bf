"""Op-level API over ``libldx.so``: the drop-in replacements for the reference's
``nax_conv3d`` / ``pack_weight`` / ``pack_upsample_weight`` / ``conv3d_ncdhw`` /
``flash_attention`` / ``mx.fast.scaled_dot_product_attention`` /
``group_norm_affine`` / ``mx.fast.layer_norm``.

Tensors are ``torch`` CUDA (HIP) tensors used only as device memory; every op runs a
hand-written gfx950 kernel through the C ABI on torch's current stream. Activations
are channels-last NDHWC ``(B, D, H, W, C)`` float16, optionally a channel slice of a
wider tensor (the voxel pitch is read from the strides). Argument errors raise
``ValueError`` before anything is launched; HIP errors raise ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch
from torch.autograd.graph import increment_version

from . import _lib
from ._lib import ACT_GELU, ACT_NONE, ACT_SILU, AttnArgs, ConvArgs, SourceConvArgs, check, lib

__all__ = [
    "PackedWeight", "pack_weight", "pack_upsample_weight", "nax_conv3d", "conv3d", "dense",
    "group_norm_affine", "layer_norm", "attention", "flash_attention", "timestep_embedding",
    "silu", "upsample_nearest2", "resize_nearest", "output_extent", "count_flops", "squared_norms4",
    "nearest_codebook4", "conv3d_half", "group_norm_half",
]


class count_flops:
    """Context manager tallying the algorithmic FLOPs (2 x real multiply-adds, no
    padding; a folded upsample conv counts its 8 taps) of the convs, dense layers and
    attention launched inside it -- for throughput figures."""

    active: "count_flops | None" = None

    def __init__(self) -> None:
        self.conv = 0.0
        self.dense = 0.0
        self.attention = 0.0

    @property
    def total(self) -> float:
        return self.conv + self.dense + self.attention

    def __enter__(self) -> "count_flops":
        count_flops.active = self
        return self

    def __exit__(self, *exc) -> None:
        count_flops.active = None


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# Element types of the conv / attention kernels (the C ABI's LDX_DTYPE_*): fp16 and bf16, and
# fp32 for the FP32 networks (the exact split-fp16 mode).
ELEM_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}
ALL_DTYPES = {**ELEM_DTYPES, torch.float32: _lib.DTYPE_F32}


def _require_cuda(t: torch.Tensor, name: str, dtype: torch.dtype | tuple | None = torch.float16) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (got {t.device}); there is no CPU path")
    allowed = dtype if isinstance(dtype, tuple) else (dtype,)
    if dtype is not None and t.dtype not in allowed:
        raise ValueError(f"{name} must be {' or '.join(str(d) for d in allowed)}, got {t.dtype}")


def _same_elem(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    """``t`` is a device tensor of the call's element type ``dtype``."""
    _require_cuda(t, name, dtype)


def voxel_pitch(x: torch.Tensor, name: str = "x") -> int:
    """Voxel pitch (elements) of an NDHWC tensor whose voxels are evenly spaced and
    whose channels are contiguous -- a contiguous tensor or a channel slice of one."""
    if x.dim() != 5:
        raise ValueError(f"{name} must be NDHWC (B, D, H, W, C), got shape {tuple(x.shape)}")
    b, d, h, w, c = x.shape
    st = x.stride()
    if c > 1 and st[4] != 1:
        raise ValueError(f"{name}: channels must be contiguous")
    pitch = st[3] if w > 1 else (st[2] // max(w, 1) if h > 1 else (st[1] // (h * w) if d > 1 else (
        st[0] // (d * h * w) if b > 1 else c)))
    if pitch < c:
        raise ValueError(f"{name}: voxel pitch {pitch} < channels {c}")
    if ((w > 1 and st[3] != pitch) or (h > 1 and st[2] != w * pitch)
            or (d > 1 and st[1] != h * w * pitch) or (b > 1 and st[0] != d * h * w * pitch)):
        raise ValueError(f"{name}: voxels must be evenly spaced (strides {st})")
    return int(pitch)


def output_extent(n: int, *, stride: int = 1, upsample: bool = False) -> int:
    """``n`` (stride 1), ``(n - 1) // 2 + 1`` (stride 2), ``2 n`` (upsample)
    (_nax_conv.py:513-516, 552)."""
    if upsample:
        return 2 * n
    if stride == 1:
        return n
    if stride == 2:
        return (n - 1) // 2 + 1
    raise ValueError("stride must be 1 or 2")


# ------------------------------------------------------------------ weights

@dataclass
class PackedWeight:
    """A conv/dense weight in the kernel's fragment-major layout (a flat fp16 tensor of
    ``ldx_packed_weight_elems`` values; see ``include/ldx.h``), or folded into the
    8 parity filters of a nearest-2x-upsampled conv."""

    data: torch.Tensor
    out_channels: int
    in_channels: int
    ksize: int
    upsample: bool = False
    # FP32 weight in the exact mode's split: hi and lo fp16 planes
    # (``ldx_packed_weight_exact_elems`` values; an upsample conv keeps its unfolded 3x3x3
    # taps and runs on the upsampled grid).
    exact: bool = False


def pack_weight(weight: torch.Tensor) -> PackedWeight:
    """Pack a Torch-layout ``(O, C, K, K, K)`` (K = 1 or 3) or dense ``(O, C)`` fp16 or
    bf16 weight (the reference's ``pack_weight``, _nax_conv.py:350-364, in this library's
    layout); the packed tensor keeps the weight's dtype. An fp32 weight is packed for the
    exact mode (its hi / lo fp16 split, _nax_conv.py:343-364)."""
    _require_cuda(weight, "weight", tuple(ALL_DTYPES))
    if weight.dim() == 2:
        weight = weight.reshape(*weight.shape, 1, 1, 1)
    if weight.dim() != 5 or weight.shape[2] != weight.shape[3] or weight.shape[3] != weight.shape[4] \
            or weight.shape[2] not in (1, 3):
        raise ValueError(f"weight must be (O, C, K, K, K) with K in (1, 3), got {tuple(weight.shape)}")
    o, c, k = int(weight.shape[0]), int(weight.shape[1]), int(weight.shape[2])
    w = weight.contiguous()
    if w.dtype == torch.float32:
        return _pack_exact(w, o, c, k, False)
    out = torch.empty(lib.ldx_packed_weight_elems(o, c, k, 0), dtype=w.dtype, device=weight.device)
    check(lib.ldx_pack_weight(_ptr(w), o, c, k, _ptr(out), _stream()), "pack_weight")
    return PackedWeight(out, o, c, k, False)


def _pack_exact(w: torch.Tensor, o: int, c: int, k: int, upsample: bool) -> PackedWeight:
    out = torch.empty(lib.ldx_packed_weight_exact_elems(o, c, k), dtype=torch.float16, device=w.device)
    check(lib.ldx_pack_weight_exact(_ptr(w), o, c, k, _ptr(out), _stream()), "pack_weight_exact")
    return PackedWeight(out, o, c, k, upsample, exact=True)


def pack_upsample_weight(weight: torch.Tensor) -> PackedWeight:
    """Fold a ``(O, C, 3, 3, 3)`` fp16 weight into 8 parity 2x2x2 filters for a conv of a
    nearest 2x upsampling (_nax_conv.py:367-405), in the weight's dtype (fp16 or bf16). An
    fp32 weight keeps its 3x3x3 taps, split for the exact mode (the conv runs on the
    upsampled grid)."""
    _require_cuda(weight, "weight", tuple(ALL_DTYPES))
    if weight.dim() != 5 or tuple(weight.shape[2:]) != (3, 3, 3):
        raise ValueError(f"weight must be (O, C, 3, 3, 3), got {tuple(weight.shape)}")
    o, c = int(weight.shape[0]), int(weight.shape[1])
    w = weight.contiguous()
    if w.dtype == torch.float32:
        return _pack_exact(w, o, c, 3, True)
    out = torch.empty(lib.ldx_packed_weight_elems(o, c, 3, 1), dtype=w.dtype, device=weight.device)
    check(lib.ldx_pack_upsample_weight(_ptr(w), o, c, ELEM_DTYPES[w.dtype], _ptr(out), _stream()),
          "pack_upsample_weight")
    return PackedWeight(out, o, c, 3, True)


def unpack_weight(packed: PackedWeight) -> "np.ndarray":
    """Host copy of a packed weight in the plain ``(parities, O, taps, C)`` order (a test
    and debugging aid; the kernels read the fragment-major form)."""
    import numpy as np

    taps = 8 if packed.upsample else packed.ksize ** 3
    par = 8 if packed.upsample else 1
    nob = -(-packed.out_channels // 128) * 4
    nkc = -(-packed.in_channels // 64) * 4
    f = packed.data.cpu().numpy().reshape(par, nob, taps, nkc, 2, 32, 8)  # lane = g*32 + r
    # -> (par, ob, r, taps, kc, g, e) -> (par, O', taps, C')
    full = f.transpose(0, 1, 5, 2, 3, 4, 6).reshape(par, nob * 32, taps, nkc * 16)
    return full[:, :packed.out_channels, :, :packed.in_channels]


def _bias32(bias: torch.Tensor | None, batch: int, out_c: int) -> tuple[torch.Tensor | None, int]:
    if bias is None:
        return None, 0
    if not bias.is_cuda:
        raise ValueError("bias must be a device tensor")
    if bias.shape[-1] != out_c or bias.dim() not in (1, 2) or (bias.dim() == 2 and bias.shape[0] != batch):
        raise ValueError(f"bias shape {tuple(bias.shape)} does not fit ({batch}, {out_c})")
    return bias.to(torch.float32).contiguous(), int(bias.dim() == 2)


# ------------------------------------------------------------------ conv3d

MOMENTS_MAX_BLOCKS = 16384


def nax_conv3d(x: torch.Tensor, packed: PackedWeight, bias: torch.Tensor | None = None, *,
               affine: torch.Tensor | None = None, silu: bool = False, stride: int = 1,
               upsample: bool = False, output_scale: float = 1.0,
               residual: torch.Tensor | None = None, x1: torch.Tensor | None = None,
               act: str | None = None, out: torch.Tensor | None = None,
               shift: torch.Tensor | None = None,
               ln: tuple[torch.Tensor, torch.Tensor, float] | None = None,
               moments: bool | str = False) -> torch.Tensor:
    """Fused conv of NDHWC ``x`` (optionally ``concat([x, x1], channels)``) with a packed
    weight: ``half((conv(prep(x)) + bias + shift) * output_scale + residual)``, ``prep`` =
    the per-(b, c) ``affine`` then SiLU, rounded to fp16 once (nax_conv3d,
    _nax_conv.py:451-500). ``shift`` is an fp16 ``(B, O)`` per-batch term (a row slice of
    a wider tensor is fine). ``act="gelu"`` / ``"silu"`` additionally stores
    ``half(act(y))``. ``ln = (gamma, beta, eps)`` (pointwise convs of one input only)
    layer-normalizes each input row first, in the same launch (ldx_dense_ln).
    ``moments=True`` also keeps the GroupNorm partial moments of the output, reduced in
    the conv's epilogue (ldx_conv3d_stats), where the plan allows it and pays (not on
    split-K plans; ``moments="always"`` keeps them there too): a later
    ``group_norm_affine`` of the returned tensor then merges them instead of reading it.

    Element type: fp16 or bf16 (``x``'s dtype; ``x1``, the packed weight, ``shift``,
    ``residual`` and ``out`` must share it; bias and affine are fp32 either way), or fp32:
    the exact split-fp16 mode of the FP32 networks (a weight packed from fp32; no moments,
    no fused LayerNorm).

    Returns NDHWC ``(B, D', H', W', O)`` in ``x``'s dtype (written into ``out`` when given,
    which may be a channel slice of a wider tensor).
    """
    _require_cuda(x, "x", tuple(ALL_DTYPES))
    et = x.dtype
    exact = et == torch.float32
    if packed.exact != exact or (not exact and packed.data.dtype != et):
        raise ValueError(f"packed weight is {'an fp32 (exact) packing' if packed.exact else packed.data.dtype} "
                         f"but x is {et}")
    if exact and (ln is not None or moments == "always"):
        raise ValueError("the fp32 mode has no fused LayerNorm and keeps no moments")
    xp = voxel_pitch(x, "x")
    b, d, h, w, c0 = (int(s) for s in x.shape)
    c1, x1p = 0, 0
    if x1 is not None:
        _same_elem(x1, "x1", et)
        x1p = voxel_pitch(x1, "x1")
        if tuple(x1.shape[:4]) != (b, d, h, w):
            raise ValueError(f"x1 grid {tuple(x1.shape[:4])} != x grid {(b, d, h, w)}")
        c1 = int(x1.shape[4])
    if packed.in_channels != c0 + c1:
        raise ValueError(f"packed weight expects {packed.in_channels} input channels, got {c0 + c1}")
    if packed.upsample != bool(upsample):
        raise ValueError("upsample convs need pack_upsample_weight weights (and only they)")
    if packed.ksize == 1 and (stride != 1 or upsample):
        raise ValueError("pointwise conv supports stride 1 only")
    o = packed.out_channels
    if upsample:
        grid = (2 * d, 2 * h, 2 * w)
    elif packed.ksize == 3:
        grid = tuple(output_extent(n, stride=stride) for n in (d, h, w))
    else:
        grid = (d, h, w)
    bias32, batched = _bias32(bias, b, o)
    aff = None
    if affine is not None:
        if affine.dtype != torch.float32 or not affine.is_cuda or affine.numel() != b * (c0 + c1) * 2:
            raise ValueError("affine must be device float32 with batch * C * 2 values")
        aff = affine.contiguous()
    resp = 0
    if residual is not None:
        _same_elem(residual, "residual", et)
        if tuple(residual.shape) != (b, *grid, o):
            raise ValueError(f"residual shape {tuple(residual.shape)} != output {(b, *grid, o)}")
        resp = voxel_pitch(residual, "residual")
    if out is None:
        out = torch.empty((b, *grid, o), dtype=et, device=x.device)
    else:
        _same_elem(out, "out", et)
        if tuple(out.shape) != (b, *grid, o):
            raise ValueError(f"out shape {tuple(out.shape)} != {(b, *grid, o)}")
    yp = voxel_pitch(out, "out")
    a = ConvArgs()
    a.batch, a.in_d, a.in_h, a.in_w = b, d, h, w
    a.c0, a.c1, a.out_c = c0, c1, o
    a.ksize, a.stride, a.upsample = packed.ksize, stride, int(bool(upsample))
    a.x0, a.x0_pitch = x.data_ptr(), xp
    a.x1, a.x1_pitch = (x1.data_ptr() if x1 is not None else None), x1p
    a.weight = packed.data.data_ptr()
    a.bias, a.bias_batched = (bias32.data_ptr() if bias32 is not None else None), batched
    a.affine, a.silu = (aff.data_ptr() if aff is not None else None), int(bool(silu))
    a.residual, a.residual_pitch = (residual.data_ptr() if residual is not None else None), resp
    a.output_scale = float(output_scale)
    a.act = {None: ACT_NONE, "gelu": ACT_GELU, "silu": ACT_SILU}[act]
    a.dtype = ALL_DTYPES[et]
    if shift is not None:
        _same_elem(shift, "shift", et)
        if shift.dim() != 2 or tuple(shift.shape) != (b, o) or shift.stride(1) != 1:
            raise ValueError(f"shift must be (B, O) = {(b, o)} with contiguous channels")
        a.shift, a.shift_pitch = shift.data_ptr(), shift.stride(0) if b > 1 else o
    a.y, a.y_pitch = out.data_ptr(), yp
    if count_flops.active is not None:
        taps = 8 if upsample else packed.ksize ** 3
        flops = 2.0 * b * grid[0] * grid[1] * grid[2] * o * (c0 + c1) * taps
        if packed.ksize == 1 and d == 1 and h == 1:
            count_flops.active.dense += flops
        else:
            count_flops.active.conv += flops
    ws_bytes = lib.ldx_conv3d_workspace_bytes(ctypes.byref(a))
    ws = None
    if ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
    if ln is not None:
        gamma, beta, eps = ln
        for t, name in ((gamma, "ln gamma"), (beta, "ln beta")):
            if t.dtype != torch.float32 or not t.is_cuda or t.numel() != c0 or not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous device float32 with {c0} values")
        check(lib.ldx_dense_ln(ctypes.byref(a), gamma.data_ptr(), beta.data_ptr(), float(eps), _stream()),
              "dense_ln")
        _set_moments(out, None)
        return out
    # Split-K plans (a workspace was asked for) keep no moments here: on the small tensors
    # that split, the reduce with moments (6.5 us) and their merge cost more than the
    # plain reduce plus a one-launch GroupNorm pass (measured on MI355X, config 5).
    # Nor do outputs of more than MOMENTS_MAX_BLOCKS moment blocks per batch item (the VQ
    # decoder's 32-channel full-resolution convs, 10^5 blocks): one workgroup per group
    # merges the blocks, which there costs more (90 us) than the two-pass GroupNorm over
    # the tensor (measured on MI355X, config 4: caps of 2048 / 4096 / 16384 blocks gave
    # 19.67 / 19.70 / 19.59 ms).
    if exact:
        check(lib.ldx_conv3d(ctypes.byref(a), _stream()), "conv3d (fp32)")
        _set_moments(out, None)
        return out
    # An inference-mode output keeps no moments (see _set_moments), so none are taken.
    want = (moments == "always" or (moments is True and not ws_bytes)) and not out.is_inference()
    chunks = lib.ldx_conv3d_stats_chunks(ctypes.byref(a)) if want else 0
    if moments != "always" and chunks > MOMENTS_MAX_BLOCKS:
        chunks = 0
    if chunks > 0:
        m = torch.empty((b, chunks, o // 2, 3), dtype=torch.float32, device=x.device)
        check(lib.ldx_conv3d_stats(ctypes.byref(a), m.data_ptr(), _stream()), "conv3d_stats")
        _set_moments(out, m)
        return out
    check(lib.ldx_conv3d(ctypes.byref(a), _stream()), "conv3d")
    _set_moments(out, None)
    return out


def _wrote(t: torch.Tensor) -> None:
    """Record that a kernel wrote ``t`` through its data pointer. Torch counts in-place
    writes in a version counter shared by every view of the same storage, but a write by
    a kernel launched through the C ABI is invisible to it; bumping the counter here
    makes every write -- by this library or by torch -- invalidate moments kept of any
    view of that storage. Inference tensors (``torch.inference_mode``) carry no version
    counter; nothing is recorded for them, and no moments are kept of them."""
    if not t.is_inference():
        increment_version(t)


def _set_moments(t: torch.Tensor, m: torch.Tensor | None) -> None:
    """Attach (or clear) the GroupNorm partial moments a conv kept of ``t`` as written,
    tagged with the storage's write version after that write. An inference tensor has no
    write version to validate moments against later, so none are kept of it (its
    GroupNorm then reduces the tensor itself)."""
    _wrote(t)
    if m is None or t.is_inference():
        if hasattr(t, "_ldx_moments"):
            del t._ldx_moments
    else:
        t._ldx_moments = (m, t._version)


def moments_of(t: torch.Tensor | None) -> torch.Tensor | None:
    """The ``(B, chunks, C / 2, 3)`` moments a conv kept of ``t`` (``nax_conv3d(...,
    moments=True)``), or None -- also when anything has written to ``t``'s storage since
    (a torch in-place op, another op's ``out=``, a write through another view)."""
    kept = getattr(t, "_ldx_moments", None) if t is not None else None
    if kept is None or t.is_inference():
        return None
    m, version = kept
    if t._version != version or t.dim() != 5 or m.shape[0] != t.shape[0] or 2 * m.shape[2] != t.shape[4]:
        return None
    return m


def conv3d(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           stride: int = 1, padding: int | None = None) -> torch.Tensor:
    """The reference's op-level ``conv3d(x, w, b, stride, pad)`` on NDHWC ``x`` with a
    Torch-layout ``(O, C, K, K, K)`` weight: K = 3 with padding 1, or K = 1 with
    padding 0 (mlx_model.py:159-202). Packs the weight on each call; modules prepack."""
    k = int(weight.shape[2]) if weight.dim() == 5 else 1
    pad = k // 2 if padding is None else padding
    if pad != k // 2:
        raise ValueError(f"only padding {k // 2} is supported for a {k}x{k}x{k} kernel")
    return nax_conv3d(x, pack_weight(weight), bias, stride=stride)


def dense(x: torch.Tensor, packed: PackedWeight, bias: torch.Tensor | None = None, *,
          residual: torch.Tensor | None = None, act: str | None = None,
          out: torch.Tensor | None = None, affine: torch.Tensor | None = None,
          ln: tuple[torch.Tensor, torch.Tensor, float] | None = None) -> torch.Tensor:
    """``half(x @ W^T + bias (+ residual))`` over the last axis of fp16 ``x`` with fp32
    accumulation and one rounding (SourceLayers.dense native path, mlx_model.py:204-217).
    ``ln = (gamma, beta, eps)`` applies ``layer_norm`` to ``x`` first, in the same launch."""
    if packed.ksize != 1:
        raise ValueError("dense needs a (O, C) weight packed with pack_weight")
    lead = x.shape[:-1]
    rows = math.prod(lead)
    x5 = x.reshape(1, 1, 1, rows, x.shape[-1])
    r5 = None if residual is None else residual.reshape(1, 1, 1, rows, packed.out_channels)
    o5 = None if out is None else out.reshape(1, 1, 1, rows, packed.out_channels)
    y = nax_conv3d(x5, packed, bias, residual=r5, act=act, out=o5, affine=affine, ln=ln)
    return y.reshape(*lead, packed.out_channels)


# ------------------------------------------------------------ normalisation

def group_norm_affine(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, *, groups: int,
                      eps: float, x1: torch.Tensor | None = None) -> torch.Tensor:
    """Per-(b, c) ``(scale, offset)`` fp32 ``(B, C, 2)`` of GroupNorm over NDHWC ``x``
    (optionally ``concat([x, x1])``), ``scale = gamma * rsqrt(var + eps)``, ``offset =
    beta - scale * mean`` (medmlx_core group_norm_affine; mlx_model.py:328-335)."""
    _require_cuda(x, "x", (torch.float16, torch.float32))
    xp = voxel_pitch(x, "x")
    b, d, h, w, c0 = (int(s) for s in x.shape)
    c1, x1p = 0, 0
    if x1 is not None:
        _require_cuda(x1, "x1", x.dtype)
        x1p = voxel_pitch(x1, "x1")
        c1 = int(x1.shape[4])
    c = c0 + c1
    if c % groups:
        raise ValueError(f"groups {groups} must divide channels {c}")
    g32 = gamma.to(torch.float32).contiguous()
    b32 = beta.to(torch.float32).contiguous()
    if x.dtype == torch.float32:
        out = torch.empty((b, c, 2), dtype=torch.float32, device=x.device)
        check(lib.ldx_group_norm_affine_f32(_ptr(x), xp, c0, _ptr(x1), x1p, c1, b, d * h * w, groups, _ptr(g32),
                                            _ptr(b32), float(eps), _ptr(out), _stream()), "group_norm_affine_f32")
        return out
    m0, m1 = moments_of(x), moments_of(x1)
    if m0 is not None and (x1 is None or m1 is not None) and (c // groups) % 2 == 0 and c0 % 2 == 0 \
            and c1 % 2 == 0:
        # Moments the producing convs kept: no pass over x.
        out = torch.empty((b, c, 2), dtype=torch.float32, device=x.device)
        n1 = int(m1.shape[1]) if m1 is not None else 0
        # Many blocks per group: the blocks are first folded by a pass over whole rows.
        ws_bytes = lib.ldx_group_norm_moments_workspace_bytes(int(m0.shape[1]), c0, n1, c1, b, groups)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        check(lib.ldx_group_norm_affine_moments_ws(
            _ptr(m0), int(m0.shape[1]), c0, _ptr(m1), n1, c1, b, groups, _ptr(g32), _ptr(b32), float(eps),
            _ptr(out), _ptr(ws), ws_bytes, _stream()), "group_norm_affine_moments")
        return out
    voxels = d * h * w
    ws = torch.empty(max(1, lib.ldx_group_norm_workspace_bytes(b, voxels, c, groups)),
                     dtype=torch.uint8, device=x.device)
    out = torch.empty((b, c, 2), dtype=torch.float32, device=x.device)
    check(lib.ldx_group_norm_affine(_ptr(x), xp, c0, _ptr(x1), x1p, c1, b, voxels, groups,
                                    _ptr(g32), _ptr(b32), float(eps), _ptr(out), _ptr(ws), _stream()),
          "group_norm_affine")
    return out


def layer_norm(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float = 1e-5,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """LayerNorm over the last axis of fp16 or fp32 ``x`` (mx.fast.layer_norm,
    mlx_model.py:360-367)."""
    _require_cuda(x, "x", (torch.float16, torch.float32))
    f = int(x.shape[-1])
    x2 = x.reshape(-1, f)
    if x2.stride(-1) != 1:
        raise ValueError("layer_norm: features must be contiguous")
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _require_cuda(out, "out", x.dtype)
    o2 = out.reshape(-1, f)
    fn = lib.ldx_layer_norm_f32 if x.dtype == torch.float32 else lib.ldx_layer_norm
    check(fn(_ptr(x2), x2.stride(0), x2.shape[0], f, _ptr(gamma.to(torch.float32).contiguous()),
             _ptr(beta.to(torch.float32).contiguous()), float(eps), _ptr(o2), o2.stride(0), _stream()),
          "layer_norm")
    _wrote(out)
    return out


# ----------------------------------------------------------------- attention

def _attn_args(q4: torch.Tensor, k4: torch.Tensor, v4: torch.Tensor, o4: torch.Tensor,
               scale: float, mask: torch.Tensor | None) -> AttnArgs:
    """Build the C arguments from (B, L, H, D) views."""
    a = AttnArgs()
    b, lq, h, d = (int(s) for s in q4.shape)
    a.batch, a.heads, a.q_len, a.kv_len, a.head_dim = b, h, lq, int(k4.shape[1]), d
    for name, t in (("q", q4), ("k", k4), ("v", v4), ("o", o4)):
        if t.stride(3) != 1:
            raise ValueError(f"attention: {name} head_dim must be contiguous")
        setattr(a, name, t.data_ptr())
        getattr(a, name + "_stride")[:] = [t.stride(0), t.stride(1), t.stride(2)]
    a.scale = float(scale)
    a.dtype = ALL_DTYPES[q4.dtype]
    a.mask = None
    if mask is not None:
        a.mask = mask.data_ptr()
        a.mask_stride[:] = [mask.stride(0), mask.stride(1), mask.stride(2), mask.stride(3)]
    ws_bytes = lib.ldx_attention_workspace_bytes(ctypes.byref(a))
    if ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q4.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
        a._keep = ws  # the buffer lives as long as the argument block
    return a


def _prepare_mask(mask: torch.Tensor | None, b: int, h: int, lq: int, lk: int,
                  device: torch.device) -> torch.Tensor | None:
    if mask is None:
        return None
    if not mask.is_cuda:
        raise ValueError("mask must be a device tensor")
    if mask.dtype == torch.bool:
        mask = torch.zeros(mask.shape, dtype=torch.float32, device=device).masked_fill(~mask, -math.inf)
    mask = mask.to(torch.float32)
    while mask.dim() < 4:
        mask = mask.unsqueeze(0)
    return mask.expand(b, h, lq, lk)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
              mask: torch.Tensor | None = None) -> torch.Tensor:
    """``softmax(q k^T * scale + mask) v`` for fp16 ``(B, H, L, D)`` tensors, the contract
    of ``mx.fast.scaled_dot_product_attention`` (mlx_model.py:485-487, 860-862). ``mask``
    is additive (``-inf`` removes a key) or boolean (``True`` keeps a key), broadcast to
    ``(B, H, L, LK)``. fp16 or bf16 (all three alike; the probabilities are rounded to
    that type for the P V product), or fp32 (head widths 16 / 32 / 64, no mask; FP32
    throughout). Returns ``(B, H, L, D)``."""
    _require_cuda(q, "q", tuple(ALL_DTYPES))
    for name, t in (("q", q), ("k", k), ("v", v)):
        _same_elem(t, name, q.dtype)
        if t.dim() != 4:
            raise ValueError(f"{name} must be (B, H, L, D)")
    b, h, lq, d = (int(s) for s in q.shape)
    lk = int(k.shape[2])
    if tuple(k.shape) != (b, h, lk, d) or tuple(v.shape) != (b, h, lk, d):
        raise ValueError(f"k/v shapes {tuple(k.shape)}, {tuple(v.shape)} do not fit q {tuple(q.shape)}")
    out = torch.empty((b, h, lq, d), dtype=q.dtype, device=q.device)
    m = _prepare_mask(mask, b, h, lq, lk, q.device)
    a = _attn_args(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), out.transpose(1, 2), scale, m)
    if count_flops.active is not None:
        count_flops.active.attention += 4.0 * b * h * lq * lk * d
    check(lib.ldx_attention(ctypes.byref(a), _stream()), "attention")
    return out


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, heads: int, scale: float,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Multi-head attention on head-interleaved projections ``(B, L, heads * d)``
    (head ``h`` = columns ``h*d .. h*d+d-1``), returning that layout
    (flash_attention, _attention.py:331-351). Key length may differ from query length.
    fp16, bf16 or fp32 (as ``attention``)."""
    _require_cuda(q, "q", tuple(ALL_DTYPES))
    for name, t in (("q", q), ("k", k), ("v", v)):
        _same_elem(t, name, q.dtype)
        if t.dim() != 3:
            raise ValueError(f"{name} must be (B, L, heads * d)")
    b, lq, f = (int(s) for s in q.shape)
    if f % heads:
        raise ValueError(f"features {f} not divisible by heads {heads}")
    d = f // heads
    lk = int(k.shape[1])
    if tuple(k.shape) != (b, lk, f) or tuple(v.shape) != (b, lk, f):
        raise ValueError("k/v must be (B, LK, heads * d) matching q")
    if out is None:
        out = torch.empty((b, lq, f), dtype=q.dtype, device=q.device)
    else:
        _same_elem(out, "out", q.dtype)
    a = _attn_args(q.view(b, lq, heads, d) if q.is_contiguous() else q.unflatten(2, (heads, d)),
                   k.unflatten(2, (heads, d)), v.unflatten(2, (heads, d)), out.unflatten(2, (heads, d)),
                   scale, None)
    if count_flops.active is not None:
        count_flops.active.attention += 4.0 * b * heads * lq * lk * d
    check(lib.ldx_attention(ctypes.byref(a), _stream()), "attention")
    _wrote(out)
    return out


# ---------------------------------------------------------------- small ops

def timestep_embedding(timesteps: torch.Tensor, channels: int, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """``[cos(t f), sin(t f)]`` (mlx_model.py:609-612) for int32 ``timesteps``, fp16 (computed
    in fp32, rounded once) or fp32."""
    _require_cuda(timesteps, "timesteps", torch.int32)
    if dtype not in (torch.float16, torch.float32):
        raise ValueError(f"timestep features are fp16 or fp32, not {dtype}")
    t = timesteps.contiguous()
    out = torch.empty((t.shape[0], channels), dtype=dtype, device=t.device)
    fn = lib.ldx_timestep_embedding_f32 if dtype == torch.float32 else lib.ldx_timestep_embedding
    check(fn(_ptr(t), t.shape[0], channels, _ptr(out), _stream()), "timestep_embedding")
    return out


def silu(x: torch.Tensor) -> torch.Tensor:
    """``half(silu(float(x)))`` (LdmUnet.silu, mlx_model.py:409-413)."""
    _require_cuda(x, "x")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    check(lib.ldx_silu(_ptr(xc), xc.numel(), _ptr(out), _stream()), "silu")
    return out


def upsample_nearest2(x: torch.Tensor) -> torch.Tensor:
    """Nearest 2x upsampling of NDHWC ``x`` (_spatial.py:41-57)."""
    _require_cuda(x, "x")
    xp = voxel_pitch(x)
    b, d, h, w, c = (int(s) for s in x.shape)
    out = torch.empty((b, 2 * d, 2 * h, 2 * w, c), dtype=torch.float16, device=x.device)
    check(lib.ldx_upsample_nearest2(_ptr(x), xp, b, d, h, w, c, _ptr(out), c, _stream()),
          "upsample_nearest2")
    return out


def resize_nearest(x: torch.Tensor, shape: tuple[int, int, int]) -> torch.Tensor:
    """Nearest resize of NDHWC ``x`` to spatial ``shape``; only the factor-two case the
    model uses runs on the device (_spatial.py:60-69)."""
    if len(shape) != 3:
        raise ValueError("nearest resizing needs three spatial axes")
    if tuple(shape) == tuple(2 * int(s) for s in x.shape[1:4]):
        return upsample_nearest2(x)
    raise ValueError("only nearest 2x resizing is supported")


# ------------------------------------------------------------ VQ codebook search

_VQ_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def _vq_rows(t: torch.Tensor, name: str) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor; there is no CPU path")
    if t.dtype not in _VQ_DTYPES:
        raise ValueError(f"{name} must be float16 or float32, got {t.dtype}")
    if t.dim() != 2 or t.shape[1] != 4 or not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous (rows, 4), got {tuple(t.shape)}")
    if t.shape[0] < 1:
        raise ValueError(f"{name} is empty")
    return int(t.shape[0])


def squared_norms4(x: torch.Tensor) -> torch.Tensor:
    """Per-row ``T(sum float32(T(x * x)))`` of ``(rows, 4)`` vectors, the squared norm the
    reference keeps per codebook entry (mlx_model.py:775-778)."""
    n = _vq_rows(x, "x")
    out = torch.empty(n, dtype=x.dtype, device=x.device)
    check(lib.ldx_vq_squared_norms4(_ptr(x), n, _VQ_DTYPES[x.dtype], _ptr(out), _stream()), "vq_squared_norms4")
    return out


def nearest_codebook4(z: torch.Tensor, codebook: torch.Tensor, codebook_norm: torch.Tensor, *,
                      quantized: torch.Tensor | None = None) -> torch.Tensor:
    """int32 index of the nearest codebook row for each ``(positions, 4)`` latent row:
    the reference's distance and rounding points, the first NaN distance else the first
    smallest (nearest_codebook4, _vq.py:63-82). ``quantized`` (same shape and dtype as
    ``z``), when given, receives the straight-through ``z + (selected - z)``."""
    p = _vq_rows(z, "z")
    e = _vq_rows(codebook, "codebook")
    if codebook.dtype != z.dtype or codebook_norm.dtype != z.dtype:
        raise ValueError("z, codebook and codebook_norm must share one dtype")
    if not codebook_norm.is_cuda or tuple(codebook_norm.shape) != (e,) or not codebook_norm.is_contiguous():
        raise ValueError(f"codebook_norm must be a contiguous device vector of {e} values")
    if quantized is not None and (tuple(quantized.shape) != (p, 4) or quantized.dtype != z.dtype
                                  or not quantized.is_contiguous() or not quantized.is_cuda):
        raise ValueError("quantized must be a contiguous device tensor shaped and typed like z")
    idx = torch.empty(p, dtype=torch.int32, device=z.device)
    check(lib.ldx_vq_nearest4(_ptr(z), None, _ptr(codebook), _ptr(codebook_norm), p, e, _VQ_DTYPES[z.dtype],
                              _ptr(idx), _ptr(quantized), _stream()), "vq_nearest4")
    if quantized is not None:
        _wrote(quantized)
    return idx


# --------------------------------------------------------------- source-order arithmetic


def _ncdhw_strides(x: torch.Tensor, name: str) -> tuple[int, int, int]:
    """(batch, channel, voxel) element strides of a logical NCDHW tensor whose voxels are
    evenly spaced: NCDHW-contiguous (voxel stride 1) or channels-last 3-D (voxel stride C)."""
    if x.dim() != 5:
        raise ValueError(f"{name} must be NCDHW (B, C, D, H, W), got shape {tuple(x.shape)}")
    _, _, d, h, w = x.shape
    st = x.stride()
    sv = st[4] if w > 1 else (st[3] // w if h > 1 else (st[2] // (h * w) if d > 1 else 1))
    if (w > 1 and st[4] != sv) or (h > 1 and st[3] != w * sv) or (d > 1 and st[2] != h * w * sv):
        raise ValueError(f"{name}: voxels must be evenly spaced (strides {st})")
    return int(st[0]), int(st[1]), int(sv)


def _like(x: torch.Tensor, shape: tuple[int, ...]) -> torch.Tensor:
    """An empty fp16 tensor of ``shape`` in ``x``'s memory format (NCDHW or channels-last)."""
    fmt = (torch.channels_last_3d if not x.is_contiguous() and x.is_contiguous(memory_format=torch.channels_last_3d)
           else torch.contiguous_format)
    return torch.empty(shape, dtype=torch.float16, device=x.device, memory_format=fmt)


def conv3d_half(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, *, padding: int,
                stride: int) -> torch.Tensor:
    """Source-order fp16 conv3d (conv3d_half, _source_half.py:327-384): four fp32 partial
    sums in Torch-CPU's channel-major order, bias added, one fp16 rounding -- Torch-CPU's
    result bit for bit. ``x`` is NCDHW ``(B, C, D, H, W)`` (contiguous or channels-last),
    ``weight`` ``(O, C, KD, KH, KW)``, ``bias`` ``(O,)`` or None, all fp16; returns
    ``(B, O, OD, OH, OW)`` in ``x``'s memory format."""
    _require_cuda(x, "x")
    _require_cuda(weight, "weight")
    xs = _ncdhw_strides(x, "conv3d input")
    if weight.dim() != 5:
        raise ValueError(f"weight must be (O, C, KD, KH, KW), got {tuple(weight.shape)}")
    b, c, d, h, w = x.shape
    o, wc, kd, kh, kw = weight.shape
    if wc != c:
        raise ValueError("conv3d input channels differ from source weights")
    if bias is not None:
        _require_cuda(bias, "bias")
        if tuple(bias.shape) != (o,):
            raise ValueError("conv3d bias must have one value per output channel")
        bias = bias.contiguous()
    ext = [(n + 2 * padding - k) // stride + 1 for n, k in zip((d, h, w), (kd, kh, kw))]
    if min(ext) < 1:
        raise ValueError("conv3d kernel exceeds the padded input")
    weight = weight.contiguous()
    y = _like(x, (b, o, *ext))
    ys = _ncdhw_strides(y, "y")
    a = SourceConvArgs(batch=b, in_c=c, in_d=d, in_h=h, in_w=w, out_c=o, kd=kd, kh=kh, kw=kw, stride=stride,
                       padding=padding, x=_ptr(x), x_batch_stride=xs[0], x_channel_stride=xs[1],
                       x_voxel_stride=xs[2], weight=_ptr(weight), bias=_ptr(bias), y=_ptr(y),
                       y_batch_stride=ys[0], y_channel_stride=ys[1], y_voxel_stride=ys[2])
    check(lib.ldx_conv3d_source_half(ctypes.byref(a), _stream()), "conv3d_source_half")
    fc = count_flops.active
    if fc is not None:
        fc.conv += 2.0 * b * o * c * kd * kh * kw * ext[0] * ext[1] * ext[2]
    return y


def group_norm_half(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, *, groups: int, eps: float,
                    return_affine: bool = False):
    """Source-order fp16 GroupNorm (group_norm_half, _source_half.py:387-544): Torch-CPU's
    chunked Welford cascade per group, then ``fp16(scale * x + offset)`` with the
    per-channel fp32 affine. ``x`` is NCDHW (contiguous or channels-last) fp16, ``weight``
    and ``bias`` fp16 ``(C,)``. Returns the normalized tensor in ``x``'s memory format, and
    with ``return_affine`` also the fp32 ``(B, C, 2)`` (scale, offset)."""
    _require_cuda(x, "x")
    xs = _ncdhw_strides(x, "group_norm input")
    b, c = x.shape[:2]
    if groups < 1 or c % groups:
        raise ValueError(f"group_norm channels {c} must be divisible by num_groups {groups}")
    for t, nm in ((weight, "weight"), (bias, "bias")):
        _require_cuda(t, nm)
        if tuple(t.shape) != (c,):
            raise ValueError("group_norm affine must have one value per channel")
    weight, bias = weight.contiguous(), bias.contiguous()
    voxels = int(x.shape[2] * x.shape[3] * x.shape[4])
    y = _like(x, tuple(x.shape))
    ys = _ncdhw_strides(y, "y")
    affine = torch.empty((b, c, 2), dtype=torch.float32, device=x.device)
    ws_bytes = lib.ldx_group_norm_source_workspace_bytes(b, c, voxels, groups)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=x.device)
    check(lib.ldx_group_norm_source_half(_ptr(x), xs[0], xs[1], xs[2], b, c, voxels, groups, _ptr(weight),
                                         _ptr(bias), float(eps), _ptr(affine), _ptr(y), ys[0], ys[1], ys[2],
                                         _ptr(ws), int(ws.numel()), _stream()), "group_norm_source_half")
    return (y, affine) if return_affine else y
