"""ctypes binding of libsmx_probe.so, the streaming-read probe the
benchmark measures HBM ceilings with (csrc/probe/read_probe.h).  A
measurement instrument, not part of the decode path: the product library
(libsmx.so, include/smx.h) does not contain it and nothing on the decode
path loads this module."""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

PROBE_LIB_PATH = Path(__file__).resolve().parent / "libsmx_probe.so"
PROBE_ABI_VERSION = 1
_lib = None


def load() -> ctypes.CDLL:
    """Load libsmx_probe.so once (after torch, so it binds to torch's HIP
    runtime)."""
    global _lib
    if _lib is None:
        if not PROBE_LIB_PATH.exists():
            raise RuntimeError(f"{PROBE_LIB_PATH} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(PROBE_LIB_PATH))
        lib.smx_probe_abi_version.restype = ctypes.c_int32
        lib.smx_read_probe_sink_size.argtypes = [ctypes.c_int64, ctypes.c_int32]
        lib.smx_read_probe_sink_size.restype = ctypes.c_int64
        lib.smx_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32]
        lib.smx_read_probe.restype = ctypes.c_int
        if lib.smx_probe_abi_version() != PROBE_ABI_VERSION:
            raise RuntimeError("libsmx_probe.so ABI mismatch")
        _lib = lib
    return _lib


def read_probe_sink_size(nbytes: int, loads_per_lane: int) -> int:
    """Sink words (one per wave) of read_probe over nbytes; -1 if invalid."""
    return int(load().smx_read_probe_sink_size(nbytes, loads_per_lane))


def read_probe(src: torch.Tensor, nbytes: int, sink: torch.Tensor, loads_per_lane: int = 8) -> None:
    """Streaming read of the first nbytes of src on the current stream: the
    HBM ceiling of a kernel moving the same bytes; sink (int32) receives one
    XOR word per wave."""
    if not (src.is_cuda and src.is_contiguous()):
        raise ValueError("src must be a contiguous device tensor")
    if not 0 < nbytes <= src.numel() * src.element_size():
        raise ValueError("nbytes exceeds src")
    if src.data_ptr() % 16 or nbytes % 16:
        raise ValueError("src and nbytes must be 16-byte aligned")
    n = read_probe_sink_size(nbytes, loads_per_lane)
    if n <= 0:
        raise ValueError("loads_per_lane must be 1, 2, 4, 8 or 16")
    if not (sink.is_cuda and sink.is_contiguous() and sink.dtype == torch.int32
            and sink.numel() == n and sink.device == src.device):
        raise ValueError(f"sink must be a contiguous int32 device tensor of {n} words")
    rc = load().smx_read_probe(ctypes.c_void_p(torch.cuda.current_stream(src.device).cuda_stream),
                               src.data_ptr(), nbytes, sink.data_ptr(), n, loads_per_lane)
    if rc != 0:
        raise RuntimeError(f"smx_read_probe failed with code {rc}")
