"""Weight layouts the kernels read in place.

AITER's (16, 16) preshuffle (the layout SGLang's ROCm MoE path leaves its FP8 / MXFP4
expert weights in, read in place by the reference: sgl_amd_mono/glm53/gfx950/
kernel.py:787-808 ``ld_fp8_chunk(shuffled)``): an ``[N, K]`` byte matrix becomes
``[N/16, K/32, 2, 16, 16]``, i.e. for every 16-row group and 32-byte column chunk,
two 256-byte halves holding 16 bytes of each of the 16 rows. A lane's MFMA operand
(16 rows x 32 bytes of K) is then two 16-byte loads, and a wave's load pair covers
2 KB of contiguous memory.
"""

from __future__ import annotations

import torch


def shuffle_16x16(w: torch.Tensor) -> torch.Tensor:
    """Row-major ``[..., N, K]`` bytes (uint8 / float8) -> AITER (16, 16) layout, same
    shape and dtype (a new contiguous tensor). N % 16 == 0 and K % 32 == 0."""
    *lead, n, k = w.shape
    if n % 16 or k % 32:
        raise ValueError(f"shuffle_16x16: need N % 16 == 0 and K % 32 == 0, got N={n} K={k}")
    dt = w.dtype
    b = w.contiguous().view(torch.uint8).reshape(*lead, n // 16, 16, k // 32, 2, 16)
    nd = len(lead)
    perm = list(range(nd)) + [nd, nd + 2, nd + 3, nd + 1, nd + 4]
    return b.permute(*perm).contiguous().reshape(*lead, n, k).view(dt)
