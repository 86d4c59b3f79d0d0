"""ctypes binding of libsmx.so, the C ABI declared in include/smx.h.

The library is loaded after torch, so it binds to the HIP runtime torch
already mapped (both carry the soname libamdhip64.so.7): device pointers and
stream handles from torch are then valid in the library.  Nothing here falls
back to another implementation: if the library is missing, every op raises.

Wrappers validate devices, dtypes, contiguity and sizes the way the
reference's TORCH_CHECK wrapper does (src/spark_vllm_ascend/native/head/
extension.cpp:8-10), enqueue on the current stream and raise RuntimeError on
a non-zero return code.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsmx.so"
#: load() requires a validation record (written by
#: spark-vllm-ascend_amd/native/validate.py after a passing GPU test run) to
#: vouch for the library about to be loaded: the one this variable names, or
#: DEFAULT_RECORD beside the library
VALIDATION_ENV = "SMX_VALIDATION_RECORD"
DEFAULT_RECORD = LIB_PATH.with_name("libsmx.validation.json")
#: set to 1 to load a library no record vouches for: the test suite, the
#: benchmark and the build check do (they are what validates and measures the
#: library as built); a record named by SMX_VALIDATION_RECORD is still checked
UNVALIDATED_ENV = "SMX_ALLOW_UNVALIDATED"
ABI_VERSION = 10
SMX_EINVAL = 10001
SMX_EUNSUPPORTED = 10002

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float
_F64 = ctypes.c_double

# name -> argument types (all return int)
SIGNATURES = {
    "smx_abi_version": [],
    "smx_q4_0_dequant_bf16": [_P, _P, _P, _I64, _I64],
    "smx_q4_0_gemv": [_P, _P, _P, _P, _I64, _I64],
    "smx_q4_0_gemv_swiglu": [_P, _P, _P, _P, _I64, _I64],
    "smx_q4_0_gemv_gelu": [_P, _P, _P, _P, _P, _I64, _I64],
    "smx_splitkv_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32,
                           _I32, _I32, _F32],
    "smx_splitkv_decode_merged": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                  _I32, _I32, _I32, _I32, _F32],
    "smx_splitkv_decode_merged_noalloc": [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                          _I32, _I32, _I32, _I32, _F32],
    "smx_qknorm_rope_splitkv_decode_merged": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                              _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                              _I32, _F32, _F32],
    "smx_lse_merge": [_P, _P, _P, _P, _I32, _I32, _I32, _I32],
    "smx_splitkv_plan": [_P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32],
    "smx_splitkv_decode_planned_merged": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                          _I32, _I32, _I32, _I32, _I32, _I32, _F32],
    "smx_qknorm_rope_splitkv_decode_planned_merged": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                      _P, _I32, _I32, _I32, _I32, _I32, _I32,
                                                      _I32, _I32, _I32, _I32, _F32, _F32],
    "smx_q4_0_gemm": [_P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_swiglu": [_P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_gelu": [_P, _P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_argmax": [_P, _P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_keys_per_row": [_I64],
    "smx_q4_0_packed_bytes": [_I64, _I64, _I32],
    "smx_q4_0_repack": [_P, _P, _P, _I64, _I64, _I32],
    "smx_q4_0_gemm_packed": [_P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_packed_swiglu": [_P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_packed_gelu": [_P, _P, _P, _P, _P, _I64, _I64, _I64],
    "smx_q4_0_gemm_packed_argmax": [_P, _P, _P, _P, _P, _I64, _I64, _I64],
    "smx_compute_slot_mapping": [_P, _P, _I32, _P, _P, _P, _I32, _I32, _I32, _I32],
    "smx_add_rmsnorm": [_P, _P, _P, _P, _P, _P, _I64, _I64, _F32],
    "smx_qknorm_rope_kv_write": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
                                 _I32, _I32, _I32, _F32],
    "smx_silu_mul": [_P, _P, _P, _I64, _I64],
    "smx_gelu_mul": [_P, _P, _P, _P, _I64, _I64],
    "smx_embedding": [_P, _P, _P, _P, _I64, _I64, _I64],
    "smx_argmax_bf16": [_P, _P, _I64, _I64, _P],
    "smx_reshape_and_cache": [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32],
    "smx_decode_advance": [_P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                           _I32, _P, _P, _I64, _I64],
    "smx_q4_0_add_rmsnorm_gemv": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F32],
    "smx_q4_0_add_rmsnorm_gemv_swiglu": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F32],
    "smx_q4_0_add_rmsnorm_gemv_gelu": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F32],
    "smx_q4_0_add_rmsnorm_gemv_argmax": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F32],
    "smx_q4_0_argmax_keys_size": [_I64, _I64],
    "smx_runner_create": [ctypes.POINTER(ctypes.c_char_p), _I32, ctypes.POINTER(_P)],
    "smx_runner_begin": [_P],
    "smx_runner_end": [_P],
    "smx_runner_num_packets": [_P, ctypes.POINTER(_I64)],
    "smx_runner_replay": [_P, _I32, _I32],
    "smx_runner_wait": [_P, _F64],
    "smx_runner_elapsed": [_P, ctypes.POINTER(_F64)],
    "smx_runner_destroy": [_P],
    "smx_runner_set_drain_timeout": [_P, _F64],
    "smx_graph_num_nodes": [_P, ctypes.POINTER(_I64)],
}

#: fence modes of smx_runner_replay (include/smx.h)
RUNNER_FENCES_AGENT = 0
RUNNER_FENCES_ACQUIRE_ONLY = 1

# return types other than int
RESTYPES = {"smx_q4_0_argmax_keys_size": ctypes.c_int64,
            "smx_q4_0_gemm_keys_per_row": ctypes.c_int64,
            "smx_q4_0_packed_bytes": ctypes.c_int64,
            "smx_runner_destroy": None}

_lib = None
_record = None  # the validation record load() checked (None: unvalidated load)


class SmxError(RuntimeError):
    """A C-ABI call returned a non-zero code."""

    def __init__(self, func: str, code: int, detail: str):
        self.code = code
        super().__init__(f"{func} failed with code {code}: {detail}")


def library_sha256(path: Path = LIB_PATH) -> str:
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def _file_sha256(path) -> str:
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def check_code_objects(record_path, paths) -> None:
    """Raise RuntimeError unless the validation record at record_path holds
    the sha256 of every device code object in paths: the step runner loads
    them beside the library, so the record vouches for them too."""
    try:
        rec = json.loads(Path(record_path).read_text())
    except (OSError, ValueError) as exc:
        raise RuntimeError(f"validation record {record_path} unreadable: {exc}") from exc
    want = rec.get("code_objects_sha256") if isinstance(rec, dict) else None
    want = want if isinstance(want, dict) else {}
    bad = [Path(p).name for p in paths
           if not Path(p).exists() or want.get(Path(p).name) != _file_sha256(p)]
    if bad:
        raise RuntimeError(f"validation record {record_path} rejected: code objects {bad} "
                           "are not the ones it validated")


def check_validation_record(record_path, lib_path: Path = LIB_PATH) -> str:
    """Raise RuntimeError unless the JSON validation record at record_path
    vouches for the library at lib_path: a complete GPU test run of this ABI
    version with no failure and at least one passed test, and the library's
    sha256.  Returns the digest.  The reference gates its kernel library the
    same way (src/spark_vllm_ascend/integration/head.py:22-27: a complete
    validation record whose library_sha256 matches, before load_library)."""
    try:
        rec = json.loads(Path(record_path).read_text())
    except (OSError, ValueError) as exc:
        raise RuntimeError(f"validation record {record_path} unreadable: {exc}") from exc
    res = rec.get("pytest", {}) if isinstance(rec, dict) else {}
    problems = []
    if rec.get("complete") is not True:
        problems.append("not complete")
    if rec.get("abi_version") != ABI_VERSION:
        problems.append(f"ABI {rec.get('abi_version')} != {ABI_VERSION}")
    if res.get("exit") != 0 or res.get("failed", 1) != 0 or res.get("errors", 1) != 0:
        problems.append("the GPU tests did not all pass")
    if not res.get("passed", 0) > 0:
        problems.append("no GPU test passed")
    digest = library_sha256(lib_path) if Path(lib_path).exists() else None
    if digest is None or rec.get("library_sha256") != digest:
        problems.append("library_sha256 does not match the library")
    if problems:
        raise RuntimeError(f"validation record {record_path} rejected: " + "; ".join(problems))
    return digest


def validation_record() -> Path | None:
    """The validation record load() checks: SMX_VALIDATION_RECORD if set,
    else DEFAULT_RECORD -- or None when SMX_ALLOW_UNVALIDATED=1 and no
    record is named."""
    named = os.environ.get(VALIDATION_ENV)
    if named:
        return Path(named)
    if os.environ.get(UNVALIDATED_ENV, "") == "1":
        return None
    return DEFAULT_RECORD


def checked_record() -> Path | None:
    """The record the loaded library was checked against (None: unvalidated)."""
    return _record


def load() -> ctypes.CDLL:
    """Load libsmx.so once (after torch) and declare its signatures.  A
    validation record must vouch for the library first
    (check_validation_record), as the reference refuses its kernel library
    without one (src/spark_vllm_ascend/integration/head.py:22-27): the record
    SMX_VALIDATION_RECORD names, else DEFAULT_RECORD; with
    SMX_ALLOW_UNVALIDATED=1 and no record named, the library loads
    unchecked."""
    global _lib, _record
    if _lib is not None:
        return _lib
    try:  # bind to the HIP runtime torch uses when torch is present
        import torch  # noqa: F401
    except ImportError:
        pass
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() or "
            "python spark-vllm-ascend_amd/native/build.py")
    record = validation_record()
    if record is not None:
        if not record.exists():
            raise RuntimeError(
                f"no validation record at {record}: validate the library on the GPU first "
                f"(python spark-vllm-ascend_amd/native/validate.py --record {record}), name a "
                f"record with {VALIDATION_ENV}, or set {UNVALIDATED_ENV}=1 to load it "
                "unvalidated")
        check_validation_record(record, LIB_PATH)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    lib.smx_last_error.argtypes = []
    lib.smx_last_error.restype = ctypes.c_char_p
    version = lib.smx_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libsmx.so ABI {version} != expected {ABI_VERSION}")
    _lib = lib
    _record = record
    return lib


def call(name: str, *args) -> None:
    """Invoke a C-ABI function and raise SmxError on a non-zero return."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        if rc in (SMX_EINVAL, SMX_EUNSUPPORTED):
            detail = lib.smx_last_error().decode()
        else:
            detail = f"HIP error {rc}"
        raise SmxError(name, rc, detail)
