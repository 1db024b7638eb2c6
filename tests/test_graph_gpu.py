"""The C ABI under HIP-graph capture: naju_scan_fwd + naju_scan_bwd issue only
kernel launches on the caller's stream (no allocation, host sync or memset),
and the kernels return the workspace's ticket counters to zero themselves, so
one captured forward + backward replays like the eager calls. Each test
replays the graph several times, with eager work and synchronisations in
between, and checks every replay bitwise against the eager result (fixed-order
carries: NAJU_FLAG_DETERMINISTIC) and the workspace status word."""
import ctypes

import pytest
import torch

from tests._helpers import _DTC, rand_inputs

pytestmark = pytest.mark.gpu


def _setup(ins, dev):
    from naju_amd import _lib
    L = _lib.lib()
    t = {k: (v.to(dev).contiguous() if v is not None else None) for k, v in ins.items()}
    u, Bm = t["u"], t["B"]
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    dts = (_DTC[u.dtype], _DTC[t["f_logit"].dtype], _DTC[Bm.dtype])
    bufs = {
        "y": torch.empty_like(u),
        "ck": torch.empty(max(1, L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts)), dtype=torch.float32, device=dev),
        "du": torch.empty_like(u), "dfl": torch.empty_like(t["f_logit"]), "dil": torch.empty_like(t["i_logit"]),
        "dB": torch.empty_like(Bm), "dC": torch.empty_like(t["C"]),
        "dD": torch.empty(D, dtype=torch.float32, device=dev),
        "dh0": torch.empty_like(t["h0"]) if t.get("h0") is not None else None,
        "ws": torch.zeros(max(256, L.naju_scan_workspace_bytes(Bsz, T, D, N, *dts)), dtype=torch.uint8, device=dev),
        "_inputs": t,
    }
    p = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    flags = _lib.FLAG_DETERMINISTIC

    def step():
        st = torch.cuda.current_stream(dev).cuda_stream
        b = bufs
        _lib.check(L.naju_scan_fwd(p(t["u"]), p(t["f_logit"]), p(t["i_logit"]), p(t["B"]), p(t["C"]),
                                   p(t["D_skip"]), p(t.get("h0")), p(b["y"]), p(b["ck"]), None, Bsz, T, D, N, *dts,
                                   flags, p(b["ws"]), b["ws"].numel(), st))
        _lib.check(L.naju_scan_bwd(p(t["u"]), p(t["f_logit"]), p(t["i_logit"]), p(t["B"]), p(t["C"]),
                                   p(t["D_skip"]), p(b["ck"]), p(t["dy"]), p(b["du"]), p(b["dfl"]), p(b["dil"]),
                                   p(b["dB"]), p(b["dC"]), p(b["dD"]), p(b["dh0"]), Bsz, T, D, N, *dts, flags,
                                   p(b["ws"]), b["ws"].numel(), st))

    def status():
        s = ctypes.c_uint32(7)
        _lib.check(L.naju_scan_workspace_status(p(bufs["ws"]), torch.cuda.current_stream(dev).cuda_stream,
                                                ctypes.byref(s)))
        return s.value

    return bufs, step, status


@pytest.mark.parametrize("N,shape,dtype", [(1, (2, 1000, 256), torch.bfloat16), (16, (2, 300, 128), torch.float32)])
def test_graph_replay_matches_eager(gpu, N, shape, dtype):
    ins = rand_inputs(*shape, N, seed=40 + N, dtype=dtype, h0_std=0.2)
    bufs, step, status = _setup(ins, gpu)
    outs = ("y", "du", "dfl", "dil", "dB", "dC", "dD", "dh0")
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        ref = {k: bufs[k].clone() for k in outs if bufs[k] is not None}
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    for rep in range(3):
        for k in ref:
            bufs[k].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for k, v in ref.items():
            assert torch.equal(bufs[k], v), f"replay {rep}: {k} differs from the eager call"
        assert status() == 0
        # eager work on the same buffers between replays
        with torch.cuda.stream(s):
            step()
        torch.cuda.synchronize()
        assert torch.equal(bufs["y"], ref["y"])


@pytest.mark.parametrize("N,shape,dtype", [(1, (2, 1000, 256), torch.bfloat16), (1, (1, 4096, 128), torch.float32),
                                           (16, (2, 300, 128), torch.float32)])
def test_graph_back_to_back_replays_with_new_inputs(gpu, N, shape, dtype):
    """Replays follow each other with no eager call in between, each on new
    inputs copied into the captured buffers. Every replay must equal an eager
    call on its own inputs (run afterwards, on a second workspace): a replay
    that accepted the previous replay's cross-workgroup hand-off words would
    carry the previous inputs' states into its outputs."""
    ins0 = rand_inputs(*shape, N, seed=70 + N, dtype=dtype, h0_std=0.2)
    bufs, step, status = _setup(ins0, gpu)
    outs = ("y", "du", "dfl", "dil", "dB", "dC", "dD", "dh0")
    t_in = bufs["_inputs"]
    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    sets, got = [], []
    for rep in range(4):
        # the last replay repeats the inputs of the one before it
        ins = sets[-1] if rep == 3 else rand_inputs(*shape, N, seed=100 * rep + N, dtype=dtype, h0_std=0.2)
        sets.append(ins)
        for k, v in ins.items():
            if v is not None and k in t_in:
                t_in[k].copy_(v.to(gpu))
        for k in outs:
            if bufs[k] is not None:
                bufs[k].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got.append({k: bufs[k].clone() for k in outs if bufs[k] is not None})
        assert status() == 0
    for rep, ins in enumerate(sets):
        ref_bufs, ref_step, ref_status = _setup(ins, gpu)
        ref_step()
        torch.cuda.synchronize()
        assert ref_status() == 0
        for k, v in got[rep].items():
            assert torch.equal(v, ref_bufs[k]), f"replay {rep}: {k} differs from an eager call on its inputs"


@pytest.mark.parametrize("N,shape,dtype", [(1, (2, 1000, 256), torch.bfloat16), (16, (2, 300, 128), torch.float32)])
def test_wrapper_inference_forward_captures(gpu, N, shape, dtype):
    """naju_scan_hip's no-grad forward captured into a graph through the
    Python wrapper: its asynchronous status watching stays out of the capture
    (no copy recorded, no event queried while capturing), and every replay on
    new inputs equals an eager call on them bitwise (with torch's
    deterministic mode on, which selects fixed-order N = 1 carries)."""
    from naju_amd import naju_scan_hip
    names = ("u", "f_logit", "i_logit", "B", "C", "D_skip", "h0")
    ins = rand_inputs(*shape, N, seed=90 + N, dtype=dtype, h0_std=0.2)
    t = {k: ins[k].to(gpu) for k in names}
    s = torch.cuda.Stream(gpu)
    was = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        with torch.no_grad(), torch.cuda.stream(s):
            naju_scan_hip(*[t[k] for k in names])  # the workspace exists before capture
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                y = naju_scan_hip(*[t[k] for k in names])
        torch.cuda.synchronize()
        for rep in range(3):
            new = rand_inputs(*shape, N, seed=200 + 10 * rep + N, dtype=dtype, h0_std=0.2)
            for k in names:
                t[k].copy_(new[k].to(gpu))
            g.replay()
            torch.cuda.synchronize()
            with torch.no_grad():
                ref = naju_scan_hip(*[new[k].to(gpu) for k in names])
            torch.cuda.synchronize()
            assert torch.equal(y, ref), f"replay {rep} differs from an eager call on its inputs"
    finally:
        torch.use_deterministic_algorithms(was)
