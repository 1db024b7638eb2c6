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
