"""GGUF Q4_0 weight format on the host side of the decode path.

The interface format is GGUF's own: a [n, k] Q4_0 tensor is n rows of k/32
blocks of 18 bytes (fp16 scale, 16 nibble bytes), exactly what
``gguf.GGUFReader`` exposes as ``tensor.data`` and what the reference's
``unpack_q4`` consumes (src/spark_vllm_ascend/integration/weights.py:34-40).
The HIP kernels stream this layout directly, so loading a checkpoint never
repacks weights (the reference's own repack, weights.py:42-54, assumes
bf16-exact scales and would reject general fp16 scales).

Synthetic weights follow the recipe of the single-GEMV workload: d =
fp16(|N(0,1)| * 0.02), codes uniform in 0..15, qs[j] = code[j] | code[j+16]
<< 4.  They are generated on the device with a seeded torch generator.
"""
from __future__ import annotations

import torch

from ..native import torch_ops

QK4_0 = 32
BLOCK_BYTES = 18
GGML_TYPE_Q4_0 = 2


def row_bytes(k: int) -> int:
    if k % QK4_0:
        raise ValueError(f"Q4_0 rows need k % 32 == 0, got {k}")
    return k // QK4_0 * BLOCK_BYTES


def pack_q4_0(scales_f16: torch.Tensor, codes_u4: torch.Tensor) -> torch.Tensor:
    """scales fp16 [n, nb], codes uint8 0..15 [n, nb, 32] -> uint8 [n, nb*18]."""
    n, nb = scales_f16.shape
    out = torch.empty((n, nb, BLOCK_BYTES), dtype=torch.uint8, device=scales_f16.device)
    out[:, :, 0:2] = scales_f16.contiguous().view(torch.uint8).view(n, nb, 2)
    out[:, :, 2:] = (codes_u4[:, :, :16] & 15) | ((codes_u4[:, :, 16:] & 15) << 4)
    return out.view(n, nb * BLOCK_BYTES)


def synthetic_q4_0(n: int, k: int, seed: int, device, scale: float = 0.02,
                   chunk_rows: int = 8192) -> torch.Tensor:
    """Seeded random Q4_0 weights [n, k/32*18] generated on `device`."""
    nb = k // QK4_0
    row_bytes(k)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out = torch.empty((n, nb * BLOCK_BYTES), dtype=torch.uint8, device=device)
    for r0 in range(0, n, chunk_rows):
        r1 = min(n, r0 + chunk_rows)
        d = (torch.randn((r1 - r0, nb), generator=gen, device=device).abs_() * scale).half()
        codes = torch.randint(0, 16, (r1 - r0, nb, QK4_0), generator=gen, device=device,
                              dtype=torch.uint8)
        out[r0:r1] = pack_q4_0(d, codes)
    return out


def unpack_q4_0(blocks: torch.Tensor, n: int, k: int):
    """(codes int8 [n, k] in [-8, 7], scales fp16 [n, k/32]) on the blocks'
    device -- the reference's unpack_q4 on torch tensors."""
    b = blocks.reshape(n, k // QK4_0, BLOCK_BYTES)
    s = b[:, :, :2].contiguous().view(torch.float16).reshape(n, k // QK4_0)
    v = b[:, :, 2:]
    q = torch.cat((v & 15, v >> 4), dim=-1).reshape(n, k).to(torch.int8) - 8
    return q, s


def dequantize_bf16(blocks: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """bf16 weights RNE(d * q), computed by the HIP dequant kernel (bit-exact
    with gguf dequantize followed by .bfloat16())."""
    return torch_ops.q4_0_dequant_bf16(blocks.reshape(-1), n, k)
