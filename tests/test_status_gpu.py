"""Failed carry hand-offs reach the caller without a synchronisation.

The N = 1 kernels hand chunk carries between workgroups with bounded waits; a
wait that gives up writes NaN outputs and sets the workspace's status word.
naju_scan_hip copies that word to pinned host memory asynchronously after
each N = 1 call, and the next call (or backward) on the same stream raises
NajuScanError once the copy has landed, clearing the word so the workspace
is usable again. The failures are forced from the host with the library's
NAJU_DEBUG_SPIN_LIMIT=0 test hook (every hand-off gives up at once, every
kernel still exits normally)."""
import pytest
import torch

from tests._helpers import NAMES, rand_inputs

pytestmark = pytest.mark.gpu


def _inputs(dev, grad=False):
    ins = rand_inputs(2, 4096, 256, 1, seed=23, dtype=torch.float32)
    xs = [ins[k].to(dev).requires_grad_(grad) for k in NAMES]
    return xs, ins["dy"].to(dev)


def test_failed_forward_handoff_raises_at_the_next_call(gpu, monkeypatch):
    from naju_amd import naju_scan_hip
    from naju_amd._lib import NajuScanError
    xs, _ = _inputs(gpu)
    with torch.no_grad():
        y_ok = naju_scan_hip(*xs)
        monkeypatch.setenv("NAJU_DEBUG_SPIN_LIMIT", "0")
        y_bad = naju_scan_hip(*xs)
        monkeypatch.delenv("NAJU_DEBUG_SPIN_LIMIT")
        torch.cuda.synchronize()
        assert bool(torch.isnan(y_bad[:, 128:]).all()) and bool(torch.isfinite(y_bad[:, :128]).all())
        with pytest.raises(NajuScanError, match="earlier scan call") as ei:
            naju_scan_hip(*xs)
        assert ei.value.code == 1
        # cleared: the same workspace serves correct calls again
        y2 = naju_scan_hip(*xs)
        torch.cuda.synchronize()
    torch.testing.assert_close(y2, y_ok, rtol=1e-6, atol=1e-6)


def test_failed_backward_handoff_raises_at_the_next_call(gpu, monkeypatch):
    from naju_amd import naju_scan_hip
    from naju_amd._lib import NajuScanError
    xs, dy = _inputs(gpu, grad=True)
    y = naju_scan_hip(*xs)
    monkeypatch.setenv("NAJU_DEBUG_SPIN_LIMIT", "0")
    y.backward(dy)
    monkeypatch.delenv("NAJU_DEBUG_SPIN_LIMIT")
    torch.cuda.synchronize()
    assert bool(torch.isnan(xs[0].grad).any())
    with pytest.raises(NajuScanError) as ei:
        naju_scan_hip(*xs)
    assert ei.value.code == 1
    for x in xs:
        x.grad = None
    y = naju_scan_hip(*xs)
    y.backward(dy)
    torch.cuda.synchronize()
    assert all(bool(torch.isfinite(x.grad).all()) for x in xs)


def test_healthy_calls_never_raise(gpu):
    """Many N = 1 calls in a row on one stream without synchronisation: the
    status copies of healthy calls read 0."""
    from naju_amd import naju_scan_hip
    xs, dy = _inputs(gpu, grad=True)
    for _ in range(20):
        y = naju_scan_hip(*xs)
        y.backward(dy)
    torch.cuda.synchronize()
    naju_scan_hip(*xs)
    torch.cuda.synchronize()
