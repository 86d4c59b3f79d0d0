"""CPU-only checks of the C ABI: the library loads, exports every function
include/smx.h declares, reports its ABI version, and rejects invalid
arguments with SMX_EINVAL before any GPU work (these calls never reach a
kernel, so they run without a GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

from _util import pkg

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / "include" / "smx.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smx_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "smx_q4_0_gemv" in names and "smx_splitkv_decode" in names
    assert len(names) >= 12


def test_library_exports_every_declared_symbol():
    native = pkg("native")
    lib = native.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert lib.smx_abi_version() == native.ABI_VERSION


def test_bindings_cover_header():
    native = pkg("native")
    declared = set(declared_functions()) - {"smx_last_error"}
    assert declared == set(native.SIGNATURES), declared ^ set(native.SIGNATURES)


@pytest.mark.parametrize("call,args", [
    ("smx_q4_0_gemv", (None, None, None, None, 64, 256)),
    ("smx_q4_0_gemv", (None, 16, 16, 16, 64, 255)),
    ("smx_q4_0_gemv", (None, 16, 16, 16, 0, 256)),
    ("smx_q4_0_gemv", (None, 17, 16, 16, 64, 256)),
    ("smx_q4_0_gemv_swiglu", (None, 16, 16, 16, 64, 100)),
    ("smx_q4_0_gemv_gelu", (None, 16, 16, None, 16, 64, 256)),
    ("smx_q4_0_gemv_gelu", (None, 16, 16, 17, 16, 64, 256)),
    ("smx_q4_0_gemv_gelu", (None, 16, 16, 16, 16, 64, 100)),
    ("smx_q4_0_add_rmsnorm_gemv_gelu", (None, 16, 32, 16, 64, 16, None, 16, 64, 2560, 1e-6)),
    ("smx_q4_0_add_rmsnorm_gemv_gelu", (None, 16, 32, 16, 64, 16, 16, 16, 64, 2560, -1.0)),
    ("smx_q4_0_gemm_gelu", (None, 16, 16, None, 16, 4, 64, 256)),
    ("smx_q4_0_gemm_gelu", (None, 16, 16, 16, 16, 17, 64, 256)),
    ("smx_gelu_mul", (None, 16, None, 16, 1, 10)),
    ("smx_gelu_mul", (None, 16, 16, 16, 0, 10)),
    ("smx_gelu_mul", (None, 16, 15, 16, 1, 10)),
    ("smx_q4_0_dequant_bf16", (None, 16, 16, 64, 33)),
    ("smx_splitkv_decode", (None, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 128, 32, 8, 64, 0.1)),
    ("smx_splitkv_decode", (None, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 128, 32, 16, 128, 0.1)),
    ("smx_splitkv_decode", (None, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 96, 32, 8, 128, 0.1)),
    ("smx_splitkv_decode", (None, 16, 16, 16, 16, 16, 16, 16, 1, 0, 8, 8, 128, 32, 8, 128, 0.1)),
    ("smx_splitkv_decode", (None, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 128, 32, 8, 128, -1.0)),
    ("smx_splitkv_decode", (None, 16, 16, 16, 16, 16, 16, 16, 1, 4, 1 << 20, 8, 4096, 32, 8, 128, 0.1)),
    ("smx_lse_merge", (None, 16, 16, 16, 1, 0, 32, 128)),
    ("smx_lse_merge", (None, 16, 16, 16, 1, 4, 32, 64)),
    ("smx_splitkv_decode_merged", (None, 16, 16, 16, 16, 16, 16, 16, None, 1, 4, 8, 8, 128, 32, 8, 128, 0.1)),
    ("smx_splitkv_decode_merged", (None, 16, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 100, 32, 8, 128, 0.1)),
    ("smx_add_rmsnorm", (None, 16, 16, 16, 16, 16, 1, 2561, 1e-6)),
    ("smx_add_rmsnorm", (None, 16, 16, 16, 16, 16, 1, 32768, 1e-6)),
    ("smx_add_rmsnorm", (None, 8, 16, 16, 16, 16, 1, 2560, 1e-6)),
    ("smx_qknorm_rope_kv_write", (None, 16, 16, 16, 16, 16, 16, 16, 16, 16, 1, 32, 8, 64, 8, 128, 100, 1e-6)),
    ("smx_silu_mul", (None, 16, 16, 0, 10)),
    ("smx_embedding", (None, 16, 16, 16, 0, 10, 10)),
    ("smx_argmax_bf16", (None, 16, 0, 10, 16)),
    ("smx_decode_advance", (None, 16, None, 0, None, None, 16, 16, 16, 16, 16, None, 0, 1, 1, 0, None, None, 0, 0)),
    ("smx_decode_advance", (None, 16, None, 0, None, 16, 16, 16, 16, 16, 16, None, 1, 1, 1, 0, None, None, 0, 0)),
    ("smx_decode_advance", (None, 16, None, 0, 16, 16, 16, 16, 16, 16, 16, None, 1, 1, 1, 0, None, None, 0, 0)),
    ("smx_decode_advance", (None, 16, 16, 0, None, None, 16, 16, 16, 16, 16, None, 1, 1, 1, 0, None, None, 0, 0)),
    ("smx_decode_advance", (None, 16, None, 0, None, None, 16, 16, 16, 16, 16, None, 1, 1, 1, 0, 16, None, 8, 8)),
    ("smx_decode_advance", (None, 16, None, 0, None, None, 16, 16, 16, 16, 16, None, 1, 1, 1, 0, 16, 16, 0, 8)),
    ("smx_q4_0_add_rmsnorm_gemv", (None, 16, 16, 16, 16, 16, 16, 64, 96, 1e-6)),
    ("smx_q4_0_add_rmsnorm_gemv", (None, 16, 16, 16, 16, 16, 16, 64, 256, 1e-6)),
    ("smx_q4_0_add_rmsnorm_gemv", (None, 16, 32, 16, 32, 16, 16, 64, 256, 1e-6)),
    ("smx_q4_0_add_rmsnorm_gemv_swiglu", (None, 16, 32, 16, 64, 16, 16, 64, 2560, -1.0)),
    ("smx_q4_0_add_rmsnorm_gemv_argmax", (None, 16, 32, 16, 16, 16, 16, 3, 64, 256, 1e-6)),
    ("smx_reshape_and_cache", (None, 16, 16, 16, 16, 16, 0, 8, 128, 4, 128)),
    ("smx_compute_slot_mapping", (None, 16, 1, 16, 16, 16, 5, 4, 8, 128)),
    ("smx_q4_0_gemm", (None, 16, 16, 16, 17, 64, 256)),
    ("smx_q4_0_gemm", (None, 16, 16, 16, 4, 64, 96)),
    ("smx_q4_0_gemm_swiglu", (None, 12, 16, 16, 4, 64, 256)),
    ("smx_compute_slot_mapping", (None, 16, 0, 16, 16, 16, 1, 4, 8, 128)),
    ("smx_qknorm_rope_splitkv_decode_merged",
     (None, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 128, 32, 8, 128, 0, 1e-6, 0.1)),
    ("smx_qknorm_rope_splitkv_decode_merged",
     (None, 16, 16, 16, 16, 12, 16, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 128, 32, 8, 128, 100, 1e-6, 0.1)),
    ("smx_qknorm_rope_splitkv_decode_merged",
     (None, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, None, 1, 4, 8, 8, 128, 32, 8, 128, 100, 1e-6, 0.1)),
    ("smx_qknorm_rope_splitkv_decode_merged",
     (None, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, 128, 32, 8, 64, 100, 1e-6, 0.1)),
    ("smx_runner_create", (None, 0, None)),
    ("smx_runner_begin", (None,)),
    ("smx_runner_end", (None,)),
    ("smx_runner_num_packets", (None, None)),
    ("smx_runner_replay", (None, 1, 0)),
    ("smx_runner_wait", (None, 1.0)),
    ("smx_runner_elapsed", (None, None)),
])
def test_invalid_arguments_rejected_on_host(call, args):
    native = pkg("native")
    lib = native.load()
    rc = getattr(lib, call)(*args)
    assert rc == native.SMX_EINVAL
    assert lib.smx_last_error().decode().startswith(call)


def test_argmax_keys_size():
    native = pkg("native")
    lib = native.load()
    assert lib.smx_q4_0_argmax_keys_size(151936, 2560) == 151936 // 16
    assert lib.smx_q4_0_argmax_keys_size(1000, 256) == 125
    assert lib.smx_q4_0_argmax_keys_size(1000, 96) == -1


def test_call_raises_with_message():
    native = pkg("native")
    with pytest.raises(native.SmxError, match="k must be a multiple of 32"):
        native.call("smx_q4_0_gemv", None, 16, 16, 16, 64, 100)


def test_argmax_keys_follow_launch_shape():
    """One key per workgroup: 16 rows per workgroup for the 151936 x 2560 head,
    8 above K = 16384 (the norm + argmax GEMV takes one row group there, two
    would need more than 256 VGPRs); -1 for K not a multiple of 64."""
    lib = pkg("native").load()
    assert lib.smx_q4_0_argmax_keys_size(151936, 2560) == 151936 // 16
    assert lib.smx_q4_0_argmax_keys_size(4096, 20480) == 4096 // 8
    assert lib.smx_q4_0_argmax_keys_size(2056, 32768) == 2056 // 8
    assert lib.smx_q4_0_argmax_keys_size(1000, 100) == -1


def test_read_probe_sizes():
    """The benchmark's streaming-read probe lives in libsmx_probe.so, not in
    the decode path's library or header."""
    lib = pkg("native.probe").load()
    assert lib.smx_read_probe_sink_size(14_008_320, 8) == 4 * -(-14_008_320 // 32768)
    assert lib.smx_read_probe_sink_size(100, 8) == -1   # not a multiple of 16
    assert lib.smx_read_probe_sink_size(4096, 3) == -1  # loads not a power of two <= 16
    assert lib.smx_read_probe(None, 16, 4096, 16, 2, 1) == 10001  # sink size
    assert not hasattr(pkg("native").load(), "smx_read_probe")
    assert "read_probe" not in (ROOT / "include" / "smx.h").read_text()


def test_graph_num_nodes_rejects_null():
    native = pkg("native")
    n = ctypes.c_int64(-1)
    assert native.load().smx_graph_num_nodes(None, ctypes.byref(n)) == native.SMX_EINVAL


def test_packed_layout_sizes_and_host_checks():
    """smx_q4_0_packed_bytes: whole 16-row groups (gated: 8 gate + 8 up rows) of
    2304 bytes per 256-k chunk, -1 off the supported shapes; smx_q4_0_repack
    and the packed GEMMs refuse bad shapes on the host, before any launch
    (the pointers below are never dereferenced)."""
    native = pkg("native")
    lib = native.load()
    assert lib.smx_q4_0_packed_bytes(16, 256, 0) == 2304
    assert lib.smx_q4_0_packed_bytes(17, 256, 0) == 2 * 2304
    assert lib.smx_q4_0_packed_bytes(9728, 2560, 1) == 1216 * 10 * 2304
    assert lib.smx_q4_0_packed_bytes(2560, 9728, 0) == 2560 * 9728 // 32 * 18
    for n, k in ((0, 256), (16, 0), (16, 320), (16, 128), (16, 1 << 21), ((1 << 30) + 1, 256)):
        assert lib.smx_q4_0_packed_bytes(n, k, 0) == -1, (n, k)
    E = native.SMX_EINVAL
    assert lib.smx_q4_0_repack(None, 16, 32, 16, 320, 0) == E      # k not a multiple of 256
    assert lib.smx_q4_0_repack(None, 16, 40, 16, 256, 0) == E      # wp not 16-byte aligned
    assert lib.smx_q4_0_repack(None, None, 32, 16, 256, 0) == E
    assert lib.smx_q4_0_repack(None, 16, 32, 1 << 30, 1 << 20, 0) == E  # grid beyond one launch
    assert lib.smx_q4_0_gemm_packed(None, 32, 32, 32, 17, 16, 256) == E   # m > 16
    assert lib.smx_q4_0_gemm_packed(None, 40, 32, 32, 2, 16, 256) == E    # x not 16-byte aligned
    assert lib.smx_q4_0_gemm_packed_swiglu(None, 32, 32, 32, 2, 16, 320) == E
    assert lib.smx_q4_0_gemm_packed_gelu(None, 32, 32, None, 32, 2, 16, 256) == E  # no table
    assert lib.smx_q4_0_gemm_packed_argmax(None, 32, 32, 32, None, 2, 16, 256) == E  # no keys
