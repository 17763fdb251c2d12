"""GPU affine quantize in MLX's layout (``mlx.core.quantize(mode="affine")`` on MI355X)."""

from __future__ import annotations

import torch

from . import _native


def affine_quantize(x: torch.Tensor, group_size: int = 64, bits: int = 4):
    """Quantize fp16 ``[..., D]`` -> ``(codes int32 [..., D*bits/32], scales fp16 [..., D/g], biases)``.

    Same arithmetic as the fused cache write; output layout is MLX's
    (``lib/python/easymlx/infra/mixins/bridge.py:304``).  ``codes`` holds the
    uint32 words in an int32 tensor.
    """
    if x.dtype != torch.float16:
        raise NotImplementedError("affine_quantize takes fp16 input")
    if x.device.type != "cuda":
        raise RuntimeError("affine_quantize runs on the GPU only")
    x = x.contiguous()
    d = int(x.shape[-1])
    if d % group_size:
        raise ValueError(f"last dim {d} must be a multiple of group_size {group_size}")
    rows = x.numel() // d if d else 0
    lead = tuple(x.shape[:-1])
    codes = torch.empty(lead + (d * bits // 32,), dtype=torch.int32, device=x.device)
    scales = torch.empty(lead + (d // group_size,), dtype=torch.float16, device=x.device)
    biases = torch.empty_like(scales)
    lib = _native.load()
    _native.check(
        lib.emx_affine_quantize(
            x.data_ptr(), rows, d, int(group_size), int(bits), codes.data_ptr(), scales.data_ptr(),
            biases.data_ptr(), torch.cuda.current_stream(x.device).cuda_stream,
        )
    )
    return codes, scales, biases
