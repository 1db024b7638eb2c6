"""Host logic of the padded LM head's gradient layout (naju_amd.xent): the
logits' gradient keeps a padded row stride with zero padding columns, and
only such buffers are handed back as whole padded rows. CPU tensors: no
kernel runs."""
import torch

from naju_amd import xent


def test_padded_rows_keep_their_stride_with_zero_padding():
    x = torch.empty(6, 136)[:, :130]
    g = xent._grad_buffer(x, 6, 130)
    assert g.shape == (6, 130) and g.stride() == (136, 1)
    full = xent.zero_padded_rows(g, 136)
    assert full is not None and full.shape == (6, 136) and full.data_ptr() == g.data_ptr()
    assert torch.all(full[:, 130:] == 0)
    # another stride, a slice or a foreign tensor of the same layout: no
    assert xent.zero_padded_rows(g, 140) is None
    assert xent.zero_padded_rows(g[1:], 136) is None
    assert xent.zero_padded_rows(torch.empty(6, 136)[:, :130], 136) is None


def test_contiguous_and_wide_strides_get_contiguous_gradients():
    g = xent._grad_buffer(torch.empty(4, 100), 4, 100)
    assert g.is_contiguous() and xent.zero_padded_rows(g, 100) is None
    wide = torch.empty(4, 100 + xent._MAX_PAD + 8)[:, :100]
    g = xent._grad_buffer(wide, 4, 100)
    assert g.is_contiguous()


def test_registry_entry_ends_with_its_buffer():
    import gc
    g = xent._grad_buffer(torch.empty(3, 72)[:, :70], 3, 70)
    ptr = g.data_ptr()
    assert ptr in xent._ZERO_PADDED
    del g
    gc.collect()
    assert ptr not in xent._ZERO_PADDED


def test_weight_copy_layout_and_table():
    """naju_amd.wcast: a group's weights back to back, padding rows as
    zero-fill entries (src 0), groups 64-element aligned, chunks per entry."""
    from naju_amd import wcast
    a, b, c = torch.empty(3, 8), torch.empty(5, 8), torch.empty(7, 16)
    total, mats, entries = wcast.layout([((a, b), 0), ((c,), 4)])
    assert mats == [(0, 8, 8), (64, 8, 16)]
    assert total == 64 + 128
    assert entries == [(a.data_ptr(), 0, 24), (b.data_ptr(), 24, 40), (c.data_ptr(), 64, 112), (0, 176, 16)]
    rec, cmap = wcast.build_table([(1, 0, 8192), (2, 8192, 8193), (0, 20000, 5)])
    assert list(rec["first_chunk"]) == [0, 1, 3] and list(cmap) == [0, 1, 1, 2]
    assert not wcast.servable([((a,), 0)])  # CPU tensors


def test_weight_copy_lookup_is_scoped():
    from naju_amd import wcast
    w = torch.empty(2, 2)
    assert wcast.lookup((w,), torch.bfloat16) is None
    with wcast.active(None, [], None):
        assert wcast.lookup((w,), torch.bfloat16) is None
