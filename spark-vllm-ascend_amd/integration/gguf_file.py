"""GGUF (version 2/3) reader and writer for local files, and the mapping of a
Qwen3-style decoder's tensors onto DecodeModel's weights.

The reference reads its checkpoint with gguf-py's ``GGUFReader`` and decodes
Q4_0 tensors from ``t.data`` reshaped to ``[n, k/32, 18]`` with ``(n, k) =
reversed(t.shape)`` (src/spark_vllm_ascend/integration/weights.py:10-40;
src/tools/deployment/prepare_model.py:46-64).  gguf-py is not a dependency
here; this module reads the same file format directly:

  header    magic "GGUF", uint32 version, uint64 tensor count, uint64
            metadata count (little endian throughout)
  metadata  key (uint64 length + UTF-8), uint32 value type, value
            (scalars, strings, typed arrays)
  tensors   name, uint32 n_dims, uint64 dims[n_dims] (dims[0] varies
            fastest), uint32 ggml type, uint64 offset into the data section
  data      starts at the first multiple of ``general.alignment`` (default
            32) after the tensor infos; each tensor at its offset

Tensor bytes are memory-mapped, never copied until a tensor is used; Q4_0
tensors come back as uint8 ``[n, k/32*18]`` -- the layout the kernels stream.
Only local paths are accepted (nothing is fetched).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types
T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, \
    T_UINT64, T_INT64, T_FLOAT64 = range(13)
_SCALAR = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I",
           T_INT32: "<i", T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q",
           T_FLOAT64: "<d"}

# ggml tensor types: (elements per block, bytes per block)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q5_0, GGML_Q5_1, GGML_Q8_0 = 0, 1, 2, 3, 6, 7, 8
GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_Q8_K = 10, 11, 12, 13, 14, 15
GGML_BF16 = 30
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q4_1: (32, 20),
         GGML_Q5_0: (32, 22), GGML_Q5_1: (32, 24), GGML_Q8_0: (32, 34), GGML_Q2_K: (256, 84),
         GGML_Q3_K: (256, 110), GGML_Q4_K: (256, 144), GGML_Q5_K: (256, 176),
         GGML_Q6_K: (256, 210), GGML_Q8_K: (256, 292), GGML_BF16: (1, 2)}


@dataclass
class GGUFTensor:
    name: str
    dims: tuple            # gguf order: dims[0] varies fastest
    ggml_type: int
    offset: int            # relative to the data section
    nbytes: int
    data: np.ndarray       # uint8 view of the tensor's bytes (memory-mapped)

    @property
    def shape(self) -> tuple:
        """Row-major (torch) shape: reversed gguf dims."""
        return tuple(reversed(self.dims))

    def q4_0_blocks(self) -> np.ndarray:
        """uint8 [n, k/32*18] for a 2-D Q4_0 tensor of torch shape [n, k]."""
        if self.ggml_type != GGML_Q4_0:
            raise ValueError(f"{self.name}: ggml type {self.ggml_type} is not Q4_0 (2)")
        if len(self.dims) != 2:
            raise ValueError(f"{self.name}: expected a 2-D tensor")
        n, k = self.shape
        return self.data.reshape(n, k // 32 * 18)

    def float32(self) -> np.ndarray:
        """F32 / F16 / BF16 tensor as float32 in its torch shape."""
        if self.ggml_type == GGML_F32:
            a = self.data.view("<f4")
        elif self.ggml_type == GGML_F16:
            a = self.data.view("<f2").astype(np.float32)
        elif self.ggml_type == GGML_BF16:
            a = (self.data.view("<u2").astype(np.uint32) << 16).view(np.float32)
        else:
            raise ValueError(f"{self.name}: ggml type {self.ggml_type} is not a float type")
        return a.reshape(self.shape)


def tensor_nbytes(dims, ggml_type: int) -> int:
    if ggml_type not in BLOCK:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    per, size = BLOCK[ggml_type]
    n = int(np.prod(dims, dtype=np.int64)) if dims else 1
    if dims and dims[0] % per:
        raise ValueError(f"row length {dims[0]} is not a multiple of the block size {per}")
    return n // per * size


class _Cursor:
    def __init__(self, buf):
        self.buf = buf
        self.pos = 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise ValueError("truncated GGUF file")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar("<Q")
        if n > (1 << 31):
            raise ValueError("implausible GGUF string length")
        return self.take(n).decode("utf-8")

    def value(self, vtype: int):
        if vtype in _SCALAR:
            return self.scalar(_SCALAR[vtype])
        if vtype == T_STRING:
            return self.string()
        if vtype == T_ARRAY:
            itype = self.scalar("<I")
            count = self.scalar("<Q")
            if count > (1 << 31):
                raise ValueError("implausible GGUF array length")
            if itype in _SCALAR and itype != T_BOOL:
                fmt = _SCALAR[itype]
                size = struct.calcsize(fmt)
                return np.frombuffer(self.take(size * count), dtype=np.dtype(fmt)).copy()
            return [self.value(itype) for _ in range(count)]
        raise ValueError(f"unknown GGUF metadata type {vtype}")


class GGUFFile:
    """A parsed GGUF file: ``metadata`` (dict), ``tensors`` (list, file
    order), ``tensor(name)``."""

    def __init__(self, path):
        self.path = Path(path)
        self._mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        cur = _Cursor(self._mm)
        if cur.take(4) != GGUF_MAGIC:
            raise ValueError(f"{self.path}: not a GGUF file")
        self.version = cur.scalar("<I")
        if self.version not in (2, 3):
            raise ValueError(f"{self.path}: GGUF version {self.version} is not supported")
        n_tensors = cur.scalar("<Q")
        n_kv = cur.scalar("<Q")
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = cur.string()
            self.metadata[key] = cur.value(cur.scalar("<I"))
        infos = []
        for _ in range(n_tensors):
            name = cur.string()
            n_dims = cur.scalar("<I")
            if n_dims > 8:
                raise ValueError(f"{name}: {n_dims} dimensions")
            dims = tuple(cur.scalar("<Q") for _ in range(n_dims))
            infos.append((name, dims, cur.scalar("<I"), cur.scalar("<Q")))
        align = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if align <= 0 or align & (align - 1):
            raise ValueError(f"general.alignment {align} is not a power of two")
        self.alignment = align
        self.data_offset = -(-cur.pos // align) * align
        self.tensors: list[GGUFTensor] = []
        self._by_name: dict[str, GGUFTensor] = {}
        for name, dims, gtype, off in infos:
            nbytes = tensor_nbytes(dims, gtype)
            start = self.data_offset + off
            if off % align or start + nbytes > len(self._mm):
                raise ValueError(f"{name}: data out of bounds or misaligned")
            t = GGUFTensor(name, dims, gtype, off, nbytes, self._mm[start:start + nbytes])
            self.tensors.append(t)
            self._by_name[name] = t

    def tensor(self, name: str) -> GGUFTensor:
        if name not in self._by_name:
            raise KeyError(f"{self.path}: no tensor {name!r}")
        return self._by_name[name]

    def __contains__(self, name: str) -> bool:
        return name in self._by_name


def _pack_value(v) -> tuple[int, bytes]:
    if isinstance(v, bool):
        return T_BOOL, struct.pack("<?", v)
    if isinstance(v, int):
        return (T_UINT32, struct.pack("<I", v)) if 0 <= v < 2 ** 32 else (T_INT64, struct.pack("<q", v))
    if isinstance(v, float):
        return T_FLOAT32, struct.pack("<f", v)
    if isinstance(v, str):
        b = v.encode("utf-8")
        return T_STRING, struct.pack("<Q", len(b)) + b
    if isinstance(v, np.ndarray):
        code = {np.dtype("<i4"): T_INT32, np.dtype("<f4"): T_FLOAT32, np.dtype("<u4"): T_UINT32,
                np.dtype("<i8"): T_INT64, np.dtype("<u1"): T_UINT8}[v.dtype.newbyteorder("<")]
        return T_ARRAY, struct.pack("<IQ", code, v.size) + v.astype(v.dtype.newbyteorder("<")).tobytes()
    if isinstance(v, (list, tuple)) and all(isinstance(s, str) for s in v):
        body = b"".join(struct.pack("<Q", len(s.encode())) + s.encode() for s in v)
        return T_ARRAY, struct.pack("<IQ", T_STRING, len(v)) + body
    raise TypeError(f"cannot store {type(v)} in GGUF metadata")


def write_gguf(path, metadata: dict, tensors: list[tuple[str, int, tuple, np.ndarray]],
               alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file.  tensors: (name, ggml_type, torch_shape, bytes
    as a uint8 array); shapes are given row-major and stored reversed."""
    md = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        md["general.alignment"] = alignment
    head = bytearray(GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(md)))
    for k, v in md.items():
        kb = k.encode("utf-8")
        vt, vb = _pack_value(v)
        head += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", vt) + vb
    offsets, off = [], 0
    for name, gtype, shape, data in tensors:
        dims = tuple(reversed(shape))
        if tensor_nbytes(dims, gtype) != data.nbytes:
            raise ValueError(f"{name}: {data.nbytes} bytes for shape {shape} type {gtype}")
        nb = name.encode("utf-8")
        head += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", gtype, off)
        offsets.append(off)
        off = -(-(off + data.nbytes) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (-len(head) % alignment))
        pos = 0
        for (name, gtype, shape, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(np.ascontiguousarray(data).view(np.uint8).tobytes())
            pos = o + data.nbytes


# ----------------------------------------------------------------- decoder
def decoder_config(g: GGUFFile) -> dict:
    """DecoderConfig fields from llama.cpp-style metadata (``{arch}.*``)."""
    arch = g.metadata.get("general.architecture", "qwen3")
    m = g.metadata
    hidden = int(m[f"{arch}.embedding_length"])
    n_q = int(m[f"{arch}.attention.head_count"])
    head_dim = int(m.get(f"{arch}.attention.key_length", hidden // n_q))
    emb = g.tensor("token_embd.weight") if "token_embd.weight" in g else g.tensor("output.weight")
    return dict(hidden=hidden, n_layers=int(m[f"{arch}.block_count"]), n_q=n_q,
                n_kv=int(m.get(f"{arch}.attention.head_count_kv", n_q)), head_dim=head_dim,
                intermediate=int(m[f"{arch}.feed_forward_length"]), vocab=int(emb.shape[0]),
                eps=float(m.get(f"{arch}.attention.layer_norm_rms_epsilon", 1e-6)),
                rope_theta=float(m.get(f"{arch}.rope.freq_base", 1e6)))


def decoder_weights(g: GGUFFile, n_layers: int) -> dict:
    """numpy weights keyed as DecodeModel expects: Q4_0 blocks (uint8) for
    qkv / o_proj / gate_up / down / head, float32 norms.  q, k, v rows are
    concatenated into one QKV tensor and gate, up into one gate|up tensor
    (gate rows first); a fused ``attn_qkv`` tensor is taken as is.  The
    head is ``output.weight`` when present, else the tied ``token_embd``."""
    w = {}
    for i in range(n_layers):
        b = f"blk.{i}."
        if b + "attn_qkv.weight" in g:
            w[f"layers.{i}.qkv"] = g.tensor(b + "attn_qkv.weight").q4_0_blocks()
        else:
            w[f"layers.{i}.qkv"] = np.concatenate(
                [g.tensor(b + f"attn_{x}.weight").q4_0_blocks() for x in ("q", "k", "v")])
        w[f"layers.{i}.o_proj"] = g.tensor(b + "attn_output.weight").q4_0_blocks()
        w[f"layers.{i}.gate_up"] = np.concatenate(
            [g.tensor(b + f"ffn_{x}.weight").q4_0_blocks() for x in ("gate", "up")])
        w[f"layers.{i}.down"] = g.tensor(b + "ffn_down.weight").q4_0_blocks()
        for j, name in enumerate(("attn_norm", "ffn_norm", "attn_q_norm", "attn_k_norm")):
            w[f"layers.{i}.norm{j}"] = g.tensor(b + name + ".weight").float32()
    w["final_norm"] = g.tensor("output_norm.weight").float32()
    head = g.tensor("output.weight") if "output.weight" in g else g.tensor("token_embd.weight")
    w["head"] = head.q4_0_blocks()
    return w
