"""Packed layout construction on the CPU: the reference's table, offsets and validation texts
(dism_v3/src/frontend.cpp:259-280, dism_v3/include/varlen/layout.cuh:29-47)."""
import pytest
import torch

from dism_amd import VarlenLayout


def test_layout_table_and_counts():
    layout = VarlenLayout.from_cu_seqlens(
        torch.tensor([0, 0, 256, 512, 1024, 1024, 2048], dtype=torch.int32), 2048)
    assert layout.lengths == (0, 256, 256, 512, 0, 1024)
    assert layout.tokens == layout.padded_tokens == 2048
    t = layout.table
    assert t.dtype == torch.int64 and tuple(t.shape) == (6, 7)
    assert t[:, 0].tolist() == [0, 0, 256, 512, 1024, 1024]
    assert t[:, 1].tolist() == t[:, 3].tolist() == [0, 256, 256, 512, 0, 1024]
    f = v = r = 0
    for row, n in zip(t.tolist(), layout.lengths):
        assert row[4:] == [f, v, r]
        f += ((n - 1) // 32 if n else 0) * n
        v += ((n - 1) // 16 if n else 0) * n
        r += (n + 31) // 32 * n
    assert (layout.forward_elements, layout.vertical_elements, layout.backward_elements) == \
        (f, v, r)
    assert layout.longest == 1024 and layout.documents == 6
    assert layout.spans() == [(0, 256), (256, 256), (512, 512), (1024, 1024)]
    assert layout.checkpoint_bytes(2) == 4 * 2 * (f + v + 3 * r)
    # the kernels receive only the non-empty documents
    assert layout.offsets("cpu").tolist() == [0, 256, 512, 1024, 2048]


@pytest.mark.parametrize("offsets,total,match", [
    ([0, 300], 300, "aligned"),
    ([0, 256], 512, "endpoints"),
    ([256, 512], 512, "endpoints"),
    ([0, 512, 256, 768], 768, "monotonic"),
])
def test_layout_validation(offsets, total, match):
    with pytest.raises(RuntimeError, match=match):
        VarlenLayout.from_cu_seqlens(torch.tensor(offsets, dtype=torch.int32), total)


def test_layout_rejects_bad_offsets_tensor():
    with pytest.raises(RuntimeError, match="cu_seqlens must be contiguous int32"):
        VarlenLayout.from_cu_seqlens(torch.tensor([0, 256], dtype=torch.int64), 256)
    empty = VarlenLayout.from_cu_seqlens(torch.tensor([0, 0, 0], dtype=torch.int32), 0)
    assert empty.tokens == 0 and empty.forward_elements == 0 and empty.spans() == []
    with pytest.raises(NotImplementedError):
        VarlenLayout.for_graph(empty.table, 0)
