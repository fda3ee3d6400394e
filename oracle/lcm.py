"""Closed-form pieces of the denoise loop (CPU oracle).

* ``time_proj``  -- the 320-d sinusoid, VulkanUnetPipeline.kt:36-46
  (also LcmScheduler.kt:87-96): ``[cos(t f_i) (160) | sin(t f_i) (160)]``,
  ``f_i = exp(-ln(1e4) i / 160)``, evaluated in float64 and rounded to float32.
* ``LcmSchedule`` -- LcmScheduler.kt:15-82: scaled-linear betas, LCM timesteps,
  boundary-condition coefficients and the per-step update, in float64.
* ``cfg_combine`` -- VulkanUnetPipeline.kt:86: ``u + s (c - u)``.
"""
from __future__ import annotations

import math

import numpy as np


def time_proj(t: float, dim: int = 320) -> np.ndarray:
    """VulkanUnetPipeline.kt:36-46 (flip_sin_to_cos, shift 0)."""
    half = dim // 2
    out = np.empty(dim, np.float32)
    for i in range(half):
        a = t * math.exp(-math.log(10000.0) * i / half)
        out[i] = math.cos(a)
        out[half + i] = math.sin(a)
    return out


class LcmSchedule:
    """LcmScheduler.kt:15-82 (epsilon prediction, 1000 train steps, 50 original
    steps, timestep scaling 10, sigma_data 0.5)."""

    def __init__(self, steps: int, n_train: int = 1000, n_orig: int = 50,
                 timestep_scaling: float = 10.0):
        self.steps = steps
        beta0, beta1 = 0.00085, 0.0120
        acc = 1.0
        ac = np.empty(n_train, np.float64)
        for i in range(n_train):  # LcmScheduler.kt:27-37
            b = (math.sqrt(beta0) + (math.sqrt(beta1) - math.sqrt(beta0)) * i / (n_train - 1)) ** 2
            acc *= 1.0 - b
            ac[i] = acc
        self.alphas_cumprod = ac
        k = n_train // n_orig  # LcmScheduler.kt:39-46
        origin = [(j + 1) * k - 1 for j in range(n_orig)]
        rev = origin[::-1]
        self.timesteps = [rev[int(math.floor(j * len(rev) / steps))] for j in range(steps)]
        self.timestep_scaling = timestep_scaling
        self.sigma_data = 0.5

    def coeffs(self, idx: int):
        """Per-step scalars (LcmScheduler.kt:57-68)."""
        t = self.timesteps[idx]
        a_t = self.alphas_cumprod[t]
        st = t * self.timestep_scaling
        sd2 = self.sigma_data ** 2
        c_skip = sd2 / (st * st + sd2)
        c_out = st / math.sqrt(st * st + sd2)
        last = idx == self.steps - 1
        a_prev = 1.0 if last else self.alphas_cumprod[self.timesteps[idx + 1]]
        return dict(t=t, sqrt_alpha=math.sqrt(a_t), sqrt_beta=math.sqrt(1.0 - a_t),
                    c_skip=c_skip, c_out=c_out, sqrt_alpha_prev=math.sqrt(a_prev),
                    sqrt_beta_prev=math.sqrt(1.0 - a_prev), last=last)

    def step(self, idx: int, latents: np.ndarray, eps: np.ndarray, noise) -> np.ndarray:
        """LcmScheduler.kt:56-82, element loop :70-79, float64 then float32."""
        c = self.coeffs(idx)
        x = latents.astype(np.float64)
        x0 = (x - c["sqrt_beta"] * eps.astype(np.float64)) / c["sqrt_alpha"]
        den = c["c_out"] * x0 + c["c_skip"] * x
        if c["last"]:
            return den.astype(np.float32)
        return (c["sqrt_alpha_prev"] * den
                + c["sqrt_beta_prev"] * noise.astype(np.float64)).astype(np.float32)


def cfg_combine(cond: np.ndarray, uncond: np.ndarray, scale: float) -> np.ndarray:
    """VulkanUnetPipeline.kt:86 (float32 arithmetic, as in the Kotlin loop)."""
    cond = cond.astype(np.float32)
    uncond = uncond.astype(np.float32)
    return uncond + np.float32(scale) * (cond - uncond)
