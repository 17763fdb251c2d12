"""Rotary position embedding described by its inverse frequencies.

The reference's RoPE modules all reduce to ``mlx.core.fast.rope``: pair ``i``
of the first ``dims`` dims -- ``(i, i + dims/2)``, or ``(2i, 2i+1)`` when
``traditional`` -- turns by ``theta = position * inv_freq[i]``.  ``nn.RoPE``
uses ``inv_freq[i] = scale * base^(-2i/dims)``; ``Llama3RoPE``, ``SuScaledRoPE``
and ``YarnRoPE`` pass their own periods (``freqs``, ``inv_freq = 1 / freqs``),
lib/python/easymlx/layers/rotary/_rotary.py:134-221.

``RotaryEmbedding`` is callable like those modules (``rope(x, offset=...)``
on ``[..., seq, dims]``) with plain torch arithmetic, and an affine page cache
recognises it in ``concatenate_to_cache`` to rotate K inside the
quantize-on-write kernel and Q with one launch.
"""

from __future__ import annotations

import math

import torch


class RotaryEmbedding:
    """RoPE with ``inv_freq`` float32 ``[dims // 2]``."""

    def __init__(self, dims: int, *, traditional: bool = False, base: float | None = 10000.0, scale: float = 1.0,
                 freqs=None):
        if dims <= 0 or dims % 2:
            raise ValueError(f"dims must be a positive even number, got {dims}")
        self.dims = int(dims)
        self.traditional = bool(traditional)
        if freqs is not None:
            periods = torch.as_tensor(freqs, dtype=torch.float32).reshape(-1)
            if periods.numel() != dims // 2:
                raise ValueError(f"freqs must hold dims // 2 = {dims // 2} periods, got {periods.numel()}")
            self._inv = (1.0 / periods).to(torch.float32)
        else:
            if base is None:
                raise ValueError("base or freqs is required")
            i = torch.arange(0, dims, 2, dtype=torch.float64)
            self._inv = (scale * torch.pow(torch.tensor(float(base), dtype=torch.float64), -i / dims)).to(
                torch.float32)
        self._dev: dict = {}

    @classmethod
    def llama3(cls, dims: int, *, base: float = 10000.0, factor: float = 8.0, low_freq_factor: float = 1.0,
               high_freq_factor: float = 4.0, original_max_position_embeddings: int = 8192,
               traditional: bool = False) -> "RotaryEmbedding":
        """Llama-3 piecewise scaled periods, as ``Llama3RoPE`` builds them (``_rotary.py:175-190``)."""
        f32 = torch.float32
        freqs = torch.pow(torch.tensor(float(base), dtype=f32), torch.arange(0, dims, 2, dtype=f32) / dims)
        wavelens = 2 * math.pi * freqs
        low_wl = original_max_position_embeddings / low_freq_factor
        high_wl = original_max_position_embeddings / high_freq_factor
        freqs = torch.where(wavelens > low_wl, freqs * factor, freqs)
        medium = (wavelens > high_wl) & (wavelens < low_wl)
        smooth = (original_max_position_embeddings / wavelens - low_freq_factor) / (high_freq_factor - low_freq_factor)
        smooth_freqs = freqs / ((1 - smooth) / factor + smooth)
        return cls(dims, traditional=traditional, base=None, freqs=torch.where(medium, smooth_freqs, freqs))

    @property
    def inv_freq_cpu(self) -> torch.Tensor:
        return self._inv

    def inv_freq(self, device) -> torch.Tensor:
        dev = torch.device(device)
        t = self._dev.get(dev)
        if t is None:
            t = self._inv.to(dev)
            self._dev[dev] = t
        return t

    def rotate(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """``x [..., seq, D]`` with ``positions`` broadcastable to ``[..., seq]``; fp32 math, x's dtype out."""
        half = self.dims // 2
        th = positions.to(torch.float32)[..., None] * self.inv_freq(x.device)  # [..., seq, half]
        cs, sn = torch.cos(th), torch.sin(th)
        xf = x.to(torch.float32)
        if self.traditional:
            x0, x1 = xf[..., 0:self.dims:2], xf[..., 1:self.dims:2]
        else:
            x0, x1 = xf[..., :half], xf[..., half:self.dims]
        y0 = x0 * cs - x1 * sn
        y1 = x0 * sn + x1 * cs
        out = xf.clone()
        if self.traditional:
            out[..., 0:self.dims:2], out[..., 1:self.dims:2] = y0, y1
        else:
            out[..., :half], out[..., half:self.dims] = y0, y1
        return out.to(x.dtype)

    def __call__(self, x: torch.Tensor, offset=0) -> torch.Tensor:
        """Like the reference's RoPE modules: ``x [..., seq, dims]``; ``offset`` an int or one per leading row."""
        seq = x.shape[-2]
        ar = torch.arange(seq, device=x.device)
        if isinstance(offset, torch.Tensor) and offset.numel() > 1:
            off = offset.to(x.device).reshape((-1,) + (1,) * (x.ndim - 2))  # [B, 1, ..., 1]
            pos = off + ar
        else:
            pos = ar + int(offset)
        return self.rotate(x, pos)
