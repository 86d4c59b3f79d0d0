"""smx_splitkv_decode_merged_noalloc: split-KV decode + LSE merge with the
split partials in the library's own device array (no caller workspace).

Called through the C ABI and compared bit for bit with
smx_splitkv_decode_merged on caller-allocated partials (same kernels, so the
bar is exact equality), on two calls in a row -- the second smaller -- and
through a captured graph replayed with eager work in between.  The host-side
size limit is checked without a GPU.
"""
import ctypes

import numpy as np
import pytest

from _util import pkg

N_Q, N_KV, HD, BS = 32, 8, 128, 128
SCRATCH = 8 << 20


def _native():
    return pkg("native")


def _call_noalloc(q, kc, vc, table, lens, out, num_splits, stream=None):
    import torch
    s = torch.cuda.current_stream().cuda_stream if stream is None else stream
    _native().call("smx_splitkv_decode_merged_noalloc", s, q.data_ptr(), kc.data_ptr(),
                   vc.data_ptr(), table.data_ptr(), lens.data_ptr(), out.data_ptr(),
                   q.shape[0], num_splits, table.shape[1], kc.shape[0], BS, N_Q, N_KV, HD,
                   HD ** -0.5)


def _call_buffers(q, kc, vc, table, lens, out, num_splits):
    import torch
    dev = q.device
    po = torch.empty((q.shape[0], num_splits, N_Q, HD), dtype=torch.float32, device=dev)
    pl = torch.empty((q.shape[0], num_splits, N_Q), dtype=torch.float32, device=dev)
    _native().call("smx_splitkv_decode_merged", torch.cuda.current_stream().cuda_stream,
                   q.data_ptr(), kc.data_ptr(), vc.data_ptr(), table.data_ptr(), lens.data_ptr(),
                   po.data_ptr(), pl.data_ptr(), out.data_ptr(), q.shape[0], num_splits,
                   table.shape[1], kc.shape[0], BS, N_Q, N_KV, HD, HD ** -0.5)


def _case(dev, seed, lens, max_blocks):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    seqs = len(lens)
    nblk = seqs * max_blocks + 1
    kc = torch.randn((nblk, BS, N_KV, HD), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((nblk, BS, N_KV, HD), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((seqs, N_Q, HD), generator=g, device=dev).to(torch.bfloat16)
    perm = torch.randperm(nblk, generator=torch.Generator().manual_seed(seed))
    table = perm[:seqs * max_blocks].to(torch.int32).view(seqs, max_blocks).to(dev)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
    return q, kc, vc, table, lens_t


@pytest.mark.gpu
def test_noalloc_matches_buffered_entry_twice():
    import torch
    dev = torch.device("cuda:0")
    # first call: 3 sequences (one empty), 48 splits of a 6144-token capacity
    # (3 * 48 * 32 * 516 = 2.4 MB of scratch); second call smaller: one
    # sequence of 300 tokens, 4 splits
    for seed, lens, max_blocks, splits in ((1, [6000, 0, 1337], 48, 48), (2, [300], 4, 4)):
        q, kc, vc, table, lens_t = _case(dev, seed, lens, max_blocks)
        ref = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        _call_buffers(q, kc, vc, table, lens_t, ref, splits)
        _call_noalloc(q, kc, vc, table, lens_t, got, splits)
        torch.cuda.synchronize()
        print(f"noalloc call: lens {lens} splits {splits}", flush=True)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"lens {lens}"
        assert bool(torch.isfinite(ref.float()).all())


@pytest.mark.gpu
def test_noalloc_under_graph_capture():
    """Recorded into a graph (the caller it exists for), replayed three times
    with other eager attention calls on the same scratch in between: every
    replay equals the eager result."""
    import torch
    dev = torch.device("cuda:0")
    q, kc, vc, table, lens_t = _case(dev, 3, [4000], 40)
    ref = torch.empty_like(q)
    _call_buffers(q, kc, vc, table, lens_t, ref, 32)
    out = torch.empty_like(q)
    _call_noalloc(q, kc, vc, table, lens_t, out, 32)  # resolves the scratch address
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        _call_noalloc(q, kc, vc, table, lens_t, out, 32)
    q2, kc2, vc2, table2, lens2 = _case(dev, 4, [900, 77], 8)
    other = torch.empty_like(q2)
    for i in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        _call_noalloc(q2, kc2, vc2, table2, lens2, other, 8)  # reuses the same scratch
        torch.cuda.synchronize()


@pytest.mark.parametrize("seqs,splits", [(16, 32), (1, 4096), (600, 1)])
def test_noalloc_rejects_beyond_scratch(seqs, splits):
    """More partials than SMX_NOALLOC_SCRATCH_BYTES hold: SMX_EINVAL on the
    host, before any GPU call (runs without a GPU)."""
    lib = _native().load()
    need = seqs * splits * N_Q * (4 * HD + 4)
    assert need > SCRATCH
    rc = lib.smx_splitkv_decode_merged_noalloc(None, 16, 16, 16, 16, 16, 16, seqs, splits, 64,
                                               64, BS, N_Q, N_KV, HD, 0.1)
    assert rc == _native().SMX_EINVAL
    assert b"SMX_NOALLOC_SCRATCH_BYTES" in lib.smx_last_error()


def test_noalloc_argument_checks():
    lib = _native().load()
    # null out, bad head_dim: rejected like the buffered entry
    assert lib.smx_splitkv_decode_merged_noalloc(None, 16, 16, 16, 16, 16, None, 1, 4, 8, 8, BS,
                                                 N_Q, N_KV, HD, 0.1) == _native().SMX_EINVAL
    assert lib.smx_splitkv_decode_merged_noalloc(None, 16, 16, 16, 16, 16, 16, 1, 4, 8, 8, BS,
                                                 N_Q, N_KV, 64, 0.1) == _native().SMX_EINVAL
