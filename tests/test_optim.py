"""The optimizer kernels' tensor table (naju_amd.optim.build_table) on the
CPU: record layout, chunk ownership and the chunk -> tensor map."""
import numpy as np
import pytest

from naju_amd.optim import CHUNK, TENSOR_DTYPE, build_table


def test_record_layout_matches_the_c_struct():
    # naju_adamw_tensor: four pointers, numel, first_chunk, group, reserved
    assert TENSOR_DTYPE.itemsize == 56
    assert [TENSOR_DTYPE.fields[n][1] for n in ("numel", "first_chunk", "group")] == [32, 40, 48]


def test_chunks_cover_every_element_once():
    sizes = [1, CHUNK, CHUNK + 1, 3 * CHUNK, 17, 2 * CHUNK - 1]
    entries = [(16 * i, 16 * i + 1, 16 * i + 2, 16 * i + 3, n, i % 2) for i, n in enumerate(sizes)]
    rec, cmap = build_table(entries)
    want_chunks = [(n + CHUNK - 1) // CHUNK for n in sizes]
    assert cmap.dtype == np.int32 and cmap.size == sum(want_chunks)
    assert list(rec["first_chunk"]) == list(np.concatenate(([0], np.cumsum(want_chunks)[:-1])))
    covered = np.zeros(len(sizes), dtype=np.int64)
    for c, t in enumerate(cmap):
        off = (c - rec["first_chunk"][t]) * CHUNK
        assert 0 <= off < rec["numel"][t]
        covered[t] += min(CHUNK, rec["numel"][t] - off)
    assert list(covered) == sizes
    assert list(rec["group"]) == [i % 2 for i in range(len(sizes))]


def test_empty_tensors_are_refused_and_empty_table_is_empty():
    rec, cmap = build_table([])
    assert rec.size == 0 and cmap.size == 0
    with pytest.raises(ValueError):
        build_table([(0, 0, 0, 0, 0, 0)])
