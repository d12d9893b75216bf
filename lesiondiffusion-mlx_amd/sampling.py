"""Uniform DDIM sampling of the conditioned (masked) denoiser on the device
(src/lesiondiffusion_mlx/mlx_sampling.py:17-200, _schedules.py:11-39).

The per-step coefficients are computed once on the host exactly as the reference does
(including its float16 schedule arithmetic), then live in device tables indexed by a
device-side step counter, so one DDIM step -- mask blend, network input assembly,
timestep lookup, UNet forward, update -- can be captured once as a HIP graph and
replayed for every step.
"""

from __future__ import annotations

import ctypes
from collections.abc import Callable

import numpy as np
import torch

from ._lib import check, lib


def lesion_diffusion_timesteps(steps: int, total: int = 1000) -> tuple[int, ...]:
    """``value + 1`` for ``value`` in ``range(0, total, total // steps)``; an index that
    would reach ``total`` is an error (_schedules.py:11-39)."""
    if not isinstance(steps, int) or isinstance(steps, bool) or steps < 1:
        raise ValueError(f"DDIM step count must be an int >= 1, got {steps!r}")
    if not isinstance(total, int) or isinstance(total, bool) or total < steps:
        raise ValueError(f"a {total!r}-entry noise schedule cannot hold {steps} DDIM steps")
    timesteps = tuple(v + 1 for v in range(0, total, total // steps))
    if timesteps[-1] >= total:
        raise ValueError(f"{steps} DDIM steps would index timestep {timesteps[-1]}, past the end of the "
                         f"{total}-entry schedule; pick a step count for which it stays below {total}")
    return timesteps


def _vp(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class DdimSampler:
    """Coefficients of the uniform DDIM schedule (mlx_sampling.py:27-60). ``alphas_cumprod``
    keeps its dtype (float16 for LINet): the selected values, ``1 - a`` and its
    reciprocal are evaluated in it before promotion to float32, as the reference does."""

    def __init__(self, alphas_cumprod: np.ndarray, steps: int, *, eta: float = 1.0, device="cuda"):
        ac = np.asarray(alphas_cumprod)
        self.timesteps = lesion_diffusion_timesteps(steps, int(ac.shape[0]))
        sel = ac[np.array(self.timesteps)]
        prev = np.concatenate([ac[:1], sel[:-1]])
        one = np.ones((), ac.dtype)
        self.alphas = sel.astype(np.float32)
        self.previous = prev.astype(np.float32)
        self.sqrt_one_minus = np.sqrt(one - sel).astype(np.float32)
        inv = (one / (one - sel)).astype(np.float32)
        self.sigmas = (np.float32(eta) * np.sqrt((1 - self.previous) * inv * (1 - self.alphas / self.previous))
                       ).astype(np.float32)
        self.device = torch.device(device)
        order = list(reversed(range(len(self.timesteps))))  # largest timestep first
        coef = np.stack([self.alphas, self.previous, self.sigmas, self.sqrt_one_minus], 1)[order]
        self.coef_table = torch.from_numpy(np.ascontiguousarray(coef)).to(self.device)
        self.t_table = torch.tensor([self.timesteps[i] for i in order], dtype=torch.int32, device=self.device)

    def prepare(self, denoiser: Callable[[torch.Tensor, torch.Tensor], torch.Tensor],
                conditioning: torch.Tensor, mask: torch.Tensor | None = None, *,
                masked_conditioning: bool = False) -> "PreparedDdim":
        """Bind a context-bound NDHWC denoiser, the clean latent ``conditioning`` (fp32 NDHWC
        ``(B, D, H, W, C)``) and a generation mask (fp32 ``(B, D, H, W)``, 1 = generate).
        The network input per voxel is ``[x, mask]`` (mlx_sampling.py:175-176), or
        ``[x, conditioning * (1 - mask), mask]`` with ``masked_conditioning``."""
        return PreparedDdim(self, denoiser, conditioning, mask, masked_conditioning)


class PreparedDdim:
    """A bound DDIM trajectory runner (mlx_sampling.py:138-200)."""

    def __init__(self, sampler: DdimSampler, denoiser, conditioning: torch.Tensor, mask: torch.Tensor | None,
                 masked_conditioning: bool):
        self.s = sampler
        self.denoiser = denoiser
        dev = sampler.device
        self.cond = conditioning.to(device=dev, dtype=torch.float32).contiguous()
        self.b, self.d, self.h, self.w, self.c = (int(v) for v in self.cond.shape)
        self.voxels = self.b * self.d * self.h * self.w
        self.mask = None if mask is None else mask.to(device=dev, dtype=torch.float32).contiguous()
        if self.mask is not None and self.mask.numel() != self.voxels:
            raise ValueError("mask must have one value per latent voxel")
        self.cc = self.c if (masked_conditioning and mask is not None) else (0 if mask is not None else self.c)
        self.in_channels = self.c + self.cc + (1 if mask is not None else 0)
        self.net_in = torch.zeros((self.b, self.d, self.h, self.w, self.in_channels), dtype=torch.float16, device=dev)
        self.x = torch.zeros_like(self.cond)
        self.step = torch.zeros(1, dtype=torch.int32, device=dev)
        self.t = torch.zeros(self.b, dtype=torch.int32, device=dev)
        self.noise: torch.Tensor | None = None
        self.graph: torch.cuda.CUDAGraph | None = None

    @property
    def num_steps(self) -> int:
        return len(self.s.timesteps)

    def _step(self) -> None:
        """One DDIM step on the current stream (capturable)."""
        st = _stream()
        check(lib.ldx_ddim_prepare(_vp(self.x), _vp(self.cond), _vp(self.mask), self.voxels, self.c, self.cc,
                                   _vp(self.net_in), self.in_channels, st), "ddim_prepare")
        check(lib.ldx_ddim_timestep(_vp(self.step), _vp(self.s.t_table), self.b, _vp(self.t), st),
              "ddim_timestep")
        eps = self.denoiser(self.net_in, self.t)
        pitch = int(eps.shape[-1])
        if pitch < self.c or not eps.is_contiguous():
            raise ValueError("denoiser output must be contiguous NDHWC with at least C channels")
        check(lib.ldx_ddim_update(_vp(self.x), _vp(eps), pitch, _vp(self.noise), _vp(self.s.coef_table),
                                  _vp(self.step), self.voxels, self.c, st), "ddim_update")
        check(lib.ldx_step_advance(_vp(self.step), st), "step_advance")

    def set_noise(self, initial: torch.Tensor, step_noise: torch.Tensor) -> None:
        """``initial`` (B, D, H, W, C) and ``step_noise`` (steps, B, D, H, W, C), fp32, in the
        order the steps run (largest timestep first)."""
        if tuple(step_noise.shape) != (self.num_steps, *self.cond.shape):
            raise ValueError(f"step noise must be {(self.num_steps, *self.cond.shape)}")
        self.x.copy_(initial.to(self.x.device, torch.float32))
        if self.noise is None:
            self.noise = torch.empty(step_noise.shape, dtype=torch.float32, device=self.x.device)
        # In place: a captured step graph holds this buffer's device address, so the table
        # must never be rebound once it exists (any dtype / device / layout is copied in).
        self.noise.copy_(step_noise)

    def capture(self) -> None:
        """Capture one step (the step counter advances inside it) as a HIP graph."""
        if self.noise is None:
            raise ValueError("set_noise first")
        self.step.zero_()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        saved_x = self.x.clone()
        with torch.cuda.stream(s):
            self._step()  # warm-up outside capture (allocations, kernel loading)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._step()
        torch.cuda.synchronize()
        self.x.copy_(saved_x)
        self.step.zero_()
        self.graph = g

    def run(self, *, use_graph: bool = True) -> torch.Tensor:
        """Run every step from the current ``x`` and step counter 0; returns the final
        latent with the known region reset (mlx_sampling.py:192-198)."""
        self.step.zero_()
        for _ in range(self.num_steps):
            if use_graph and self.graph is not None:
                self.graph.replay()
            else:
                self._step()
        if self.mask is not None:
            scratch = torch.empty_like(self.net_in)
            check(lib.ldx_ddim_prepare(_vp(self.x), _vp(self.cond), _vp(self.mask), self.voxels, self.c, self.cc,
                                       _vp(scratch), self.in_channels, _stream()), "ddim_prepare")
        return self.x
