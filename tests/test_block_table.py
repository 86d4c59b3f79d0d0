"""Block allocation (CPU) and the slot-mapping kernel (GPU) against the
closed form slot = table[p // bs] * bs + p % bs, with the reference's own
validation cases (src/tools/validation/test_slot_mapping.py:11-53): flipped
tables per block size 128/256/512/1024, token counts 0 / 1 / 1025 / 2048 /
4096 at offsets, padding to 32768 entries, and graph replay with the
position changed between replays."""
import numpy as np
import pytest

from _util import pkg


def bm(**kw):
    import torch
    args = dict(num_blocks=10, block_size=4, max_seqs=3, max_blocks_per_seq=5, device="cpu")
    args.update(kw)
    return pkg("integration.block_table").BlockManager(**args)


def test_allocation_and_free_reuse():
    m = bm()
    m.add_sequence(7, 9)  # 3 pages
    m.add_sequence(8, 4)  # 1 page
    assert m.pages(7) == [0, 1, 2] and m.pages(8) == [3]
    assert m.num_free_blocks == 6
    m.append_tokens(8)  # 5 tokens -> 2 pages
    assert m.pages(8) == [3, 4]
    assert m.slot(7, 5) == 1 * 4 + 1
    t = m.table_host
    assert t[m.row(7)].tolist() == [0, 1, 2, -1, -1]
    m.free(7)
    assert m.num_free_blocks == 8
    m.add_sequence(9, 2)
    assert m.pages(9) == [5]  # FIFO free list
    assert m.table_host[m.row(9)].tolist()[:1] == [5]


def test_limits():
    m = bm()
    with pytest.raises(ValueError):
        m.add_sequence(1, 21)  # > 5 blocks per sequence
    assert m.num_free_blocks == 10
    m.add_sequence(1, 20)  # 5 blocks
    m.add_sequence(2, 16)  # 4 blocks
    with pytest.raises(MemoryError):
        m.add_sequence(3, 8)  # needs 2, 1 free; the row is released again
    m.add_sequence(3, 4)
    assert m.num_free_blocks == 0
    with pytest.raises(MemoryError):
        m.append_tokens(2)  # a 5th block for sequence 2
    with pytest.raises(ValueError):
        m.append_tokens(1)  # a 6th block for sequence 1
    assert m.length(1) == 20 and m.length(2) == 16


def test_decode_batch_metadata():
    m = bm()
    m.add_sequence(1, 6)
    m.add_sequence(2, 1)
    md = m.decode_batch([2, 1])
    assert md["positions"].tolist() == [0, 5]
    assert md["seq_lens"].tolist() == [1, 6]
    assert md["query_start_loc"].tolist() == [0, 1, 2]
    assert md["block_table"][0, 0].item() == m.pages(2)[0]


MAXIMUM = 32768
SIZES = [128, 256, 512, 1024]


def _expected(table, size, positions):
    exp = np.full(MAXIMUM, -1, dtype=np.int64)
    exp[:positions.size] = table[positions // size].astype(np.int64) * size + positions % size
    return exp


@pytest.mark.gpu
def test_slot_mapping_reference_cases():
    import torch
    ops = pkg("native.torch_ops")
    dev = torch.device("cuda:0")
    tables = [np.arange(320, dtype=np.int32)[::-1] + i * 400 for i in range(4)]
    out = torch.full((MAXIMUM,), -99, dtype=torch.int64, device=dev)
    for count, offset in [(0, 0), (1, 127), (1025, 63), (2048, 3072), (4096, 0)]:
        pos = np.arange(count, dtype=np.int64) + offset
        q = torch.tensor([0, count], dtype=torch.int32, device=dev)
        for table, size in zip(tables, SIZES):
            t = torch.from_numpy(table.copy()).view(1, -1).to(dev)
            ops.compute_slot_mapping(q, torch.from_numpy(pos).to(dev), t, size, MAXIMUM, out=out)
            np.testing.assert_array_equal(out.cpu().numpy(), _expected(table, size, pos),
                                          err_msg=f"count {count} offset {offset} size {size}")


@pytest.mark.gpu
def test_slot_mapping_graph_replay():
    import torch
    ops = pkg("native.torch_ops")
    dev = torch.device("cuda:0")
    table = np.arange(320, dtype=np.int32)[::-1].copy()
    t = torch.from_numpy(table).view(1, -1).to(dev)
    pos = torch.tensor([4095], dtype=torch.int64, device=dev)
    q = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    out = torch.full((MAXIMUM,), -99, dtype=torch.int64, device=dev)
    ops.compute_slot_mapping(q, pos, t, 128, MAXIMUM, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.compute_slot_mapping(q, pos, t, 128, MAXIMUM, out=out)
    for p in (4096, 127, 8192):
        pos.fill_(p)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), _expected(table, 128, np.array([p])))


@pytest.mark.gpu
def test_slot_mapping_ragged_batch_and_out_of_table():
    import torch
    ops = pkg("native.torch_ops")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(5)
    table = rng.permutation(64).astype(np.int32).reshape(4, 16)
    starts = np.array([0, 3, 3, 10, 12], dtype=np.int32)  # request 1 is empty
    pos = rng.integers(0, 16 * 32, starts[-1]).astype(np.int64)
    pos[11] = 16 * 32 + 5  # past the table -> -1
    pos[0] = -1            # negative -> -1
    out = ops.compute_slot_mapping(torch.from_numpy(starts).to(dev), torch.from_numpy(pos).to(dev),
                                   torch.from_numpy(table).to(dev), 32, 20).cpu().numpy()
    exp = np.full(20, -1, dtype=np.int64)
    for r in range(4):
        for t in range(starts[r], starts[r + 1]):
            p = pos[t]
            if 0 <= p < 16 * 32:
                exp[t] = int(table[r, p // 32]) * 32 + p % 32
    np.testing.assert_array_equal(out, exp)
