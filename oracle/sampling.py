"""DDIM schedule and step oracle (test infrastructure only)."""

from __future__ import annotations

import numpy as np


def lesion_diffusion_timesteps(steps: int, total: int = 1000) -> tuple[int, ...]:
    """``value + 1`` for ``value`` in ``range(0, total, total // steps)``, rejecting an
    out-of-range last index (src/lesiondiffusion_mlx/_schedules.py:11-39)."""
    if not isinstance(steps, int) or isinstance(steps, bool) or steps < 1:
        raise ValueError(f"step count {steps!r} is not an int >= 1")
    if not isinstance(total, int) or isinstance(total, bool) or total < steps:
        raise ValueError(f"schedule of {total!r} entries is shorter than {steps} steps")
    t = tuple(v + 1 for v in range(0, total, total // steps))
    if t[-1] >= total:
        raise ValueError(f"last timestep {t[-1]} of {steps} steps is outside a {total}-entry schedule")
    return t


def ddim_coefficients(alphas_cumprod: np.ndarray, steps: int, eta: float = 1.0) -> dict[str, np.ndarray]:
    """Per-step DDIM coefficients in schedule order (mlx_sampling.py:27-60).

    ``alphas`` are the selected cumulative products, ``previous`` the value one
    schedule entry earlier (entry 0 for the first), ``sigma = eta * sqrt((1 - prev)
    * (1 / (1 - a)) * (1 - a / prev))`` with the reciprocal evaluated in the
    schedule's own dtype (float16 for LINet) before promotion, as the reference does.
    """
    ac = np.asarray(alphas_cumprod)
    ts = lesion_diffusion_timesteps(steps, ac.shape[0])
    sel = ac[np.array(ts)]
    prev = np.concatenate([ac[:1], sel[:-1]])
    inv = (np.ones((), ac.dtype) / (np.ones((), ac.dtype) - sel)).astype(np.float32)
    a32 = sel.astype(np.float32)
    p32 = prev.astype(np.float32)
    sqrt_one_minus = np.sqrt(np.ones((), ac.dtype) - sel).astype(np.float32)
    sig = (np.float32(eta) * np.sqrt((1 - p32) * inv * (1 - a32 / p32))).astype(np.float32)
    return {"timesteps": np.array(ts), "alphas": a32, "previous": p32,
            "sqrt_one_minus": sqrt_one_minus, "sigmas": sig}


def ddim_update(x: np.ndarray, eps: np.ndarray, alpha: float, previous: float, sigma: float,
                sqrt_one_minus: float, noise: np.ndarray) -> np.ndarray:
    """One DDIM update ``sqrt(prev) * x0 + sqrt(1 - prev - sigma^2) * eps + sigma * noise``
    with ``x0 = (x - sqrt(1 - a) * eps) / sqrt(a)`` (mlx_sampling.py:128-132, 182-185)."""
    x = np.asarray(x, np.float64)
    eps = np.asarray(eps, np.float64)
    pred = (x - sqrt_one_minus * eps) / np.sqrt(alpha)
    direction = np.sqrt(1.0 - previous - sigma ** 2) * eps
    return np.sqrt(previous) * pred + direction + sigma * np.asarray(noise, np.float64)


def ddim_sample(denoiser, coeffs: dict[str, np.ndarray], condition, image: np.ndarray,
                initial: np.ndarray, noise: np.ndarray, mask: np.ndarray | None = None) -> np.ndarray:
    """The reference DDIM loop (mlx_sampling.py:105-136): largest timestep first; with a
    mask the known region is reset to ``image`` before every step and at the end."""
    x = np.asarray(initial, np.float64)
    n = len(coeffs["timesteps"])
    for it, idx in enumerate(reversed(range(n))):
        t = np.full((x.shape[0],), coeffs["timesteps"][idx], dtype=np.int32)
        if mask is not None:
            x = x * mask + (1 - mask) * image
            net_in = np.concatenate([x, mask], axis=1)
        else:
            net_in = np.concatenate([x, image], axis=1)
        eps = denoiser(net_in, t, condition)
        if mask is not None:
            eps = eps[:, :image.shape[1]]
        x = ddim_update(x, eps, float(coeffs["alphas"][idx]), float(coeffs["previous"][idx]),
                        float(coeffs["sigmas"][idx]), float(coeffs["sqrt_one_minus"][idx]), noise[it])
    if mask is not None:
        x = x * mask + (1 - mask) * image
    return x
