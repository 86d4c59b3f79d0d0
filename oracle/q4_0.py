"""GGUF Q4_0 (ggml type 2) for the oracle -- test infrastructure.

Two independent restatements of the block decode of
src/spark_vllm_ascend/integration/weights.py:34-40:
  * numpy (this file), using numpy's float16 for the scale;
  * C (q4_0_ref.c, loaded through ctypes), using an ldexp decode of binary16.
tests/test_oracle_q4_0.py checks them against each other and against
known-answer blocks (d = 1.0, -0.0, a subnormal, 65504, +-inf, NaN; the
nibble order byte 0x1F -> element 0 = 7, element 16 = -7).

repack() restates the packed layout of the batched MFMA GEMM
(smx_q4_0_repack): the reference repacks its own weights for its kernel at
load time (src/spark_vllm_ascend/integration/weights.py:42-54); this is the
MFMA layout's counterpart, pinned by literal known-answer bytes in
tests/test_oracle_q4_0.py and, on the GPU, by the packed GEMM matching the
layout-independent float64 GEMV and selecting exact weights for one-hot
activations.

The third-party routine the reference calls, gguf-py ``dequantize``
(gguf==0.19.0, deployment/requirements.txt:5), is not installed here; for
Q4_0 its published algorithm is exactly this closed form: d * (nibble - 8).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .bf16 import f32_to_bf16_bits

BLOCK = 32
BLOCK_BYTES = 18

_LIB_PATH = Path(__file__).resolve().parent / "_build" / "liboracle.so"
_lib = None


def c_lib() -> ctypes.CDLL:
    """The C restatement (built by oracle/Makefile)."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(f"{_LIB_PATH} missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(_LIB_PATH))
        P, I = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_to_f32.restype = ctypes.c_float
        lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
        for name in ("oracle_q4_0_unpack",):
            getattr(lib, name).argtypes = [P, I, I, P, P]
        for name in ("oracle_q4_0_dequant_f32", "oracle_q4_0_dequant_bf16"):
            getattr(lib, name).argtypes = [P, I, I, P]
        for name in ("oracle_q4_0_gemv_f64", "oracle_q4_0_gemv_bf16w"):
            getattr(lib, name).argtypes = [P, P, I, I, P]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def row_bytes(k: int) -> int:
    return k // BLOCK * BLOCK_BYTES


def make_blocks(n: int, k: int, seed: int, scale: float = 0.02) -> np.ndarray:
    """Synthetic Q4_0 weights, the recipe of the single-GEMV workload:
    d = fp16(|N(0,1)| * scale), 4-bit codes uniform in 0..15, byte j of qs =
    code[j] | code[j + 16] << 4.  Returns uint8 [n, k/32*18]."""
    assert k % BLOCK == 0
    rng = np.random.default_rng(seed)
    nb = k // BLOCK
    d = (np.abs(rng.standard_normal((n, nb))) * scale).astype(np.float16)
    codes = rng.integers(0, 16, size=(n, nb, BLOCK), dtype=np.uint8)
    return pack_blocks(d, codes)


def pack_blocks(d: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """d: fp16 [n, nb]; codes: uint8 in 0..15 [n, nb, 32] -> uint8 [n, nb*18]."""
    n, nb = d.shape
    out = np.empty((n, nb, BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = np.ascontiguousarray(d, dtype="<f2").view(np.uint8).reshape(n, nb, 2)
    out[:, :, 2:] = (codes[:, :, :16] & 15) | ((codes[:, :, 16:] & 15) << 4)
    return out.reshape(n, nb * BLOCK_BYTES)


def unpack(blocks: np.ndarray, n: int, k: int):
    """-> (codes int8 [n, k] in [-8, 7], scales fp16 [n, k/32]).
    weights.py:36-40: s = bytes 0-1 as '<f2'; q = concat(v & 15, v >> 4) - 8."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(n, k // BLOCK, BLOCK_BYTES)
    s = b[:, :, :2].copy().view("<f2").reshape(n, k // BLOCK)
    v = b[:, :, 2:]
    q = np.concatenate((v & 15, v >> 4), axis=-1).reshape(n, k).astype(np.int8) - 8
    return q, s


def dequant_f32(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """Exact fp32 weights d * q (an 11-bit significand times a 4-bit integer)."""
    q, s = unpack(blocks, n, k)
    return (q.reshape(n, k // BLOCK, BLOCK).astype(np.float32)
            * s.astype(np.float32)[:, :, None]).reshape(n, k)


def dequant_bf16_bits(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """bf16 weights as the reference deploys them: RNE(d * q), uint16 bits."""
    return f32_to_bf16_bits(dequant_f32(blocks, n, k))


def c_unpack(blocks: np.ndarray, n: int, k: int):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    q = np.empty((n, k), dtype=np.int8)
    s = np.empty((n, k // BLOCK), dtype=np.uint16)
    c_lib().oracle_q4_0_unpack(_ptr(blocks), n, k, _ptr(q), _ptr(s))
    return q, s.view(np.float16)


def c_dequant_f32(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty((n, k), dtype=np.float32)
    c_lib().oracle_q4_0_dequant_f32(_ptr(blocks), n, k, _ptr(out))
    return out


def c_dequant_bf16_bits(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty((n, k), dtype=np.uint16)
    c_lib().oracle_q4_0_dequant_bf16(_ptr(blocks), n, k, _ptr(out))
    return out


def gemv_f64(x_bits: np.ndarray, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """y = W x in float64 over the exact weights (C restatement)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(k)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, dtype=np.float64)
    c_lib().oracle_q4_0_gemv_f64(_ptr(x_bits), _ptr(blocks), n, k, _ptr(y))
    return y


def gemv_bf16w_bits(x_bits: np.ndarray, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """The reference kernel's rounding points (bf16 weights, fp32 FMA, bf16 out)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(k)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, dtype=np.uint16)
    c_lib().oracle_q4_0_gemv_bf16w(_ptr(x_bits), _ptr(blocks), n, k, _ptr(y))
    return y


def gemv_np_f64(x_f32: np.ndarray, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """numpy restatement of gemv_f64 (independent of the C code)."""
    w = dequant_f32(blocks, n, k).astype(np.float64)
    return w @ np.asarray(x_f32, dtype=np.float64).reshape(k)


def packed_groups(n: int, gated: bool) -> int:
    return -(-n // 8) if gated else -(-n // 16)


def packed_bytes(n: int, k: int, gated: bool = False) -> int:
    return packed_groups(n, gated) * (k // 256) * 2304


def repack(blocks: np.ndarray, n: int, k: int, gated: bool = False) -> np.ndarray:
    """The packed layout of smx_q4_0_repack, uint8 [packed_bytes(n, k, gated)].

    Per row group G (16 rows; gated: gate rows 8G..8G+7 then the matching up
    rows d + 8G..) and 256-k chunk c, 2304 bytes at (G * k/256 + c) * 2304:
    lane l = 16 g + r (row r of the group, k-group g) owns 16 bytes at
    16 l (blocks 0-3 of the chunk) and 1024 + 16 l (blocks 4-7); in them
    byte 4 i + b holds the codes of elements 8 g + b (low nibble) and
    8 g + 4 + b (high nibble) of block i; row r's 8 fp16 scales follow at
    2048 + 16 r.  Rows past the end repeat the last row.  blocks holds n
    rows (gated: 2n, gate then up)."""
    assert k % 256 == 0 and k > 0
    nb, nc = k // BLOCK, k // 256
    rows_total = 2 * n if gated else n
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(rows_total, nb, BLOCK_BYTES)
    qs = b[:, :, 2:]
    codes = np.concatenate((qs & 15, qs >> 4), axis=-1)       # [rows, nb, 32] element order
    G = packed_groups(n, gated)
    r = np.arange(16)
    if gated:
        row = np.minimum(8 * np.arange(G)[:, None] + (r & 7)[None, :], n - 1) + n * (r >= 8)[None, :]
    else:
        row = np.minimum(16 * np.arange(G)[:, None] + r[None, :], n - 1)
    cg = codes[row].reshape(G, 16, nc, 8, 4, 8)                # [G, r, c, blk, g, e8]
    byte = cg[..., :4] | (cg[..., 4:] << 4)                    # [G, r, c, blk, g, b]
    byte = byte.reshape(G, 16, nc, 2, 4, 4, 4)                 # blk -> (part, i)
    lanes = byte.transpose(0, 2, 3, 5, 1, 4, 6)                # [G, c, part, g, r, i, b]
    sc = b[row][:, :, :, :2].reshape(G, 16, nc, 8, 2).transpose(0, 2, 1, 3, 4)  # [G, c, r, blk, 2]
    out = np.concatenate((lanes.reshape(G, nc, 2048), sc.reshape(G, nc, 256)), axis=-1)
    return np.ascontiguousarray(out).reshape(-1)
