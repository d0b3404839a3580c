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
    with pytest.raises(ValueError, match="owned CUDA Graph layout"):
        VarlenLayout.for_graph(empty.table, 0)


# ---- fixed-capacity graph layouts (dism_v3/src/host/graph_layout.h, varlen.py:28-36) ----

def _cu(offsets):
    return torch.tensor(offsets, dtype=torch.int32)


def test_graph_layout_table_offsets_and_capacities():
    from dism_amd import graph_layout_maximum, layout_from_table, make_graph_layout
    table = make_graph_layout(_cu([0, 0, 256, 512, 1024, 1024, 2048]), 2048, 1024, 1024)
    assert table.dtype == torch.int64 and tuple(table.shape) == (8, 7)
    # non-empty documents first (empty ones have no row), then padding rows at `tokens`
    assert table[:, :4].tolist() == [[0, 256, 0, 256], [256, 256, 256, 256],
                                     [512, 512, 512, 512], [1024, 1024, 1024, 1024]] + \
        [[2048, 0, 2048, 0]] * 4
    f = v = b = 0
    for row in table.tolist():
        assert row[4:] == [f, v, b]
        n = row[1]
        if n:
            f, v, b = f + (n - 1) // 32 * n, v + (n - 1) // 16 * n, b + n // 32 * n
    assert graph_layout_maximum(table) == 1024
    assert graph_layout_maximum(table.view(-1, 7)) == 1024   # views share the state
    assert graph_layout_maximum(table.clone()) == 0          # clones do not
    plain = VarlenLayout.from_cu_seqlens(_cu([0, 1024, 2048]), 2048)
    assert graph_layout_maximum(plain.table) == 0
    layout = VarlenLayout.for_graph(table, 2048)
    # capacities follow max_seqlen, not the current pack
    assert (layout.forward_elements, layout.vertical_elements, layout.backward_elements) == \
        (2048 * (1023 // 32), 2048 * (1023 // 16), 2048 * (1024 // 32))
    assert layout.longest == layout.max_length == 1024 and layout.documents == 8
    assert layout.spans() == [(0, 256), (256, 256), (512, 512), (1024, 1024)]
    # the kernels' offsets: fixed size tokens/256 + 1, padding repeats `tokens`
    assert layout.offsets("cpu").tolist() == [0, 256, 512, 1024] + [2048] * 5
    again = layout_from_table(table.view(-1), 2048)
    assert again.max_length == 1024 and again.forward_elements == layout.forward_elements
    same = layout_from_table(plain.table, 2048)
    assert (same.lengths, same.forward_elements, same.vertical_elements,
            same.backward_elements) == (plain.lengths, plain.forward_elements,
                                        plain.vertical_elements, plain.backward_elements)
    assert layout_from_table(None, 0) is None


def test_graph_layout_update_in_place():
    from dism_amd import make_graph_layout, update_graph_layout
    table = make_graph_layout(_cu([0, 512, 1024]), 1024, 512, 512)
    layout = VarlenLayout.for_graph(table, 1024)
    ptr = table.data_ptr()
    update_graph_layout(table, _cu([0, 256, 512, 768, 1024]))
    assert table.data_ptr() == ptr
    assert layout.spans() == [(0, 256), (256, 256), (512, 256), (768, 256)]
    assert layout.offsets("cpu").tolist() == [0, 256, 512, 768, 1024]
    update_graph_layout(table.view(-1, 7), _cu([0, 0, 512, 1024]))
    assert layout.spans() == [(0, 512), (512, 512)]
    assert layout.offsets("cpu").tolist() == [0, 512, 1024, 1024, 1024]


def test_graph_rejects_changed_invalid_boundaries():
    """Reference nanochat/tests/test_cuda_graph.py:142-150: invalid updates raise and leave
    the table unchanged."""
    from dism_amd import make_graph_layout, update_graph_layout
    table = make_graph_layout(_cu([0, 512, 1024]), 1024, 512, 512)
    before = table.clone()
    for bounds in ([0, 255, 512, 1024], [0, 768, 1024], [0, 256, 768, 1024], [0, 512, 512]):
        with pytest.raises(RuntimeError):
            update_graph_layout(table, _cu(bounds))
        assert torch.equal(table, before)
    with pytest.raises(RuntimeError, match="contiguous CPU int32"):
        update_graph_layout(table, torch.tensor([0, 1024], dtype=torch.int64))
    with pytest.raises(RuntimeError, match="expected an owned graph layout"):
        update_graph_layout(before, _cu([0, 1024]))


@pytest.mark.parametrize("tokens,maximum,row,match", [
    (1000, 256, 256, "capacities"),
    (1024, 2048, 1024, "capacities"),
    (1024, 512, 256, "capacities"),
    (1024, 256, 768, "capacities"),
    (1 << 20, 256, 256, "document-tag range"),
])
def test_graph_layout_capacity_validation(tokens, maximum, row, match):
    from dism_amd import make_graph_layout
    with pytest.raises(RuntimeError, match=match):
        make_graph_layout(_cu([0, tokens]), tokens, maximum, row)


def test_pack_vectors_is_a_view_and_metadata_is_document_head_major():
    """VarlenLayout.pack (reference varlen.py:42-47; pack kernel
    src/probe/varlen_pack.cu:10-24): vectors return the squeezed view; per-token metadata
    [1,H,T] becomes, per document, a head-major block of its tokens -- checked against an
    explicit loop over documents, heads and tokens."""
    layout = VarlenLayout.from_cu_seqlens(_cu([0, 256, 256, 768, 1024]), 1024)
    x = torch.zeros((1, 1024, 3, 8), dtype=torch.bfloat16)
    assert layout.pack(x, vectors=True).data_ptr() == x.data_ptr()
    assert tuple(layout.pack(x, vectors=True).shape) == (1024, 3, 8)
    with pytest.raises(RuntimeError, match="token count"):
        layout.pack(x[:, :512].contiguous(), vectors=True)
    with pytest.raises(RuntimeError, match="metadata"):
        layout.pack(x, vectors=False)
    labels = torch.randint(0, 1 << 20, (1, 3, 1024), dtype=torch.int32)
    got = layout.pack(labels, vectors=False)
    want = torch.empty(1024 * 3, dtype=torch.int32)
    for begin, n in ((0, 256), (256, 512), (768, 256)):
        for h in range(3):
            for t in range(n):
                want[begin * 3 + h * n + t] = labels[0, h, begin + t]
    assert got.dtype == torch.int32 and torch.equal(got, want)
    # an exact permutation: every element once
    assert torch.equal(torch.sort(got).values, torch.sort(labels.reshape(-1)).values)
