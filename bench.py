"""Benchmark of the fused fwd+bwd Naju scan on one MI355X.

A step is one forward (naju_scan_fwd) plus one backward (naju_scan_bwd) of the
scan over one batch of synthetic input resident in HBM, through the C ABI on
preallocated buffers (the hot path itself, no autograd bookkeeping). The
default workload is benchmark configuration c2 (naju_amd.workloads.CONFIGS): B=8, L=4096, D=1024, bf16
streams with fp32 state, N=1 (B=C=1), h0 ~ N(0, 0.1^2), dy ~ N(0,1).

value = algorithmic bytes of fwd+bwd per step * K / wall time of K steps
(GB/s). The roofline object reports the dominant kernel (the backward) from
HIP events recorded on the launch stream inside the timed region. The
cpu_baseline leg times the sequential torch-CPU restatement of the
reference's scan (oracle/scan_ref.py: scan_loop_torch, the algorithm of
reference naju/scan.py:79-93) with autograd on a bounded sample of the same
workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--N 1]
"""
import argparse
import gc
import json
import os
import sys
import time

_ROOT = os.path.dirname(os.path.abspath(__file__))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

HBM_PEAK_GBS = 8000.0
VALU_PEAK_TFLOPS = 157.3 / 2  # fp32 FMA without packed-FP32 instructions
METRIC = "fwd+bwd scan GB/s (% of HBM peak) at B8 L4096 D1024; LM tokens/s"


def _dt_size(dt):
    import torch
    return 4 if dt == torch.float32 else 2


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"],
                    help="c1-c4: the scan itself; c5: the LM training step (tokens/s)")
    ap.add_argument("--N", type=int, default=1, help="state size (d_state)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--flush", action="store_true",
                    help="also time steps with a 1 GiB cache-flush write before each step")
    ap.add_argument("--tune-gemms", default=None, metavar="CSV",
                    help="c5: time the GEMM solutions during the warmup and record them in CSV "
                         "(default: read naju_amd/tunableop_mi355x_lm.csv)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run 3 plain 512 MiB device copies (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)

    if args.config == "c5":
        _bench_lm(args)
        return

    import ctypes
    import torch
    from naju_amd import _lib
    from naju_amd.workloads import CONFIGS, algorithmic_bytes, config_inputs

    L = _lib.lib()
    dev = torch.device("cuda", 0)
    if args.calib_copy:
        src = torch.ones(1 << 27, dtype=torch.float32, device=dev)   # 512 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"calib-copy: 3 x copy of {src.numel() * 4} bytes", file=sys.stderr, flush=True)
        del src, dst
    cfg = CONFIGS[args.config]
    Bsz, T, D, N = cfg["batch"], cfg["T"], cfg["D"], args.N
    ins = config_inputs(args.config, N=N, seed=0, device=dev)
    xdt = ins["u"].dtype
    DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
    dts = (DT[xdt], DT[ins["f_logit"].dtype], DT[ins["B"].dtype])
    u, fl, il, Bm, Cm, Dk, h0, dy = (ins[k] for k in ("u", "f_logit", "i_logit", "B", "C", "D_skip", "h0", "dy"))
    y = torch.empty_like(u)
    ck = torch.empty(L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts), dtype=torch.float32, device=dev)
    du, dfl, dil = torch.empty_like(u), torch.empty_like(fl), torch.empty_like(il)
    dB, dC = torch.empty_like(Bm), torch.empty_like(Cm)
    dD = torch.empty(D, dtype=torch.float32, device=dev)
    dh0 = torch.empty_like(h0) if h0 is not None else None
    ws_bytes = L.naju_scan_workspace_bytes(Bsz, T, D, N, *dts)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def fwd():
        _lib.check(L.naju_scan_fwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(h0), p(y), p(ck), None,
                                   Bsz, T, D, N, *dts, 0, p(ws), ws_bytes, sh))

    def bwd():
        _lib.check(L.naju_scan_bwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(ck), p(dy), p(du), p(dfl),
                                   p(dil), p(dB), p(dC), p(dD), p(dh0), Bsz, T, D, N, *dts, 0, p(ws),
                                   ws_bytes, sh))

    s_x, s_g, s_bc = _dt_size(xdt), _dt_size(fl.dtype), _dt_size(Bm.dtype)
    has_h0 = h0 is not None
    bytes_fwd = algorithmic_bytes(Bsz, T, D, N, s_x, s_g, s_bc, has_h0, fwd=True, bwd=False)
    bytes_bwd = algorithmic_bytes(Bsz, T, D, N, s_x, s_g, s_bc, has_h0, fwd=False, bwd=True)
    bytes_step = bytes_fwd + bytes_bwd

    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()

    K = args.steps
    # the timed region: K steps back to back, nothing else on the stream
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        fwd()
        bwd()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / K
    # per-call durations (the roofline): K more steps with HIP events around
    # each call, on the stream the kernels run on
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(K)]
    for k in range(K):
        ev[k][0].record(stream)
        fwd()
        ev[k][1].record(stream)
        bwd()
        ev[k][2].record(stream)
    torch.cuda.synchronize()
    t_fwd = sorted(e[0].elapsed_time(e[1]) for e in ev)
    t_bwd = sorted(e[1].elapsed_time(e[2]) for e in ev)
    avg_fwd = sum(t_fwd) / K
    avg_bwd = sum(t_bwd) / K
    med = lambda xs: xs[len(xs) // 2]  # noqa: E731

    st = ctypes.c_uint32(0)
    _lib.check(L.naju_scan_workspace_status(p(ws), sh, ctypes.byref(st)))
    if st.value != 0:
        raise RuntimeError("workspace status nonzero: a carry hand-off timed out")

    value = bytes_step / (ms_step * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float32: "f32", torch.float16: "f16"}[xdt]
        + " streams, f32 state/accum",
        "data": "synthetic (seeded; the c2 gate/input recipe of naju_amd.workloads)",
        "config": {"workload": f"naju scan fwd+bwd {args.config}: B={Bsz} L={T} D={D} N={N}"
                   + (" B=C=1" if N == 1 else " B,C~N(0,1/N)") + (" with h0" if has_h0 else ""),
                   "batch": Bsz, "seq_len": T, "channels": D, "d_state": N,
                   "parallelism": "single GPU", "cache_flush": False},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "elements_per_s": round(Bsz * T * D / (ms_step * 1e-3), 1),
        "algorithmic_bytes_per_step": bytes_step,
        "fwd_ms_avg": round(avg_fwd, 5), "fwd_ms_median": round(med(t_fwd), 5),
        "bwd_ms_avg": round(avg_bwd, 5), "bwd_ms_median": round(med(t_bwd), 5),
        "fwd_GBs": round(bytes_fwd / (avg_fwd * 1e-3) / 1e9, 1),
        "roofline": {
            "kernel": "naju_scan_bwd call = n1_bwd_kernel + fold_kernel" if N == 1 else "naju_scan_bwd call",
            "bound": "hbm",
            "achieved": round(bytes_bwd / (avg_bwd * 1e-3) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bytes_bwd / (avg_bwd * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": _traffic(args.config, N),
        },
    }
    if N > 1:
        # General N is compute-bound: the recurrence, readout and adjoint are
        # about 19N flop per element (5N forward, 14N backward), fp32 FMA on
        # the VALU. Packed-FP32 ops are disabled in this build, so the peak is
        # half of MI355X's 157.3 TFLOP/s vector fp32.
        E = Bsz * T * D
        fl_bwd = 14.0 * N * E
        ach = fl_bwd / (avg_bwd * 1e-3) / 1e12
        out["roofline_compute"] = {"kernel": "naju_scan_bwd call", "bound": "valu", "achieved": round(ach, 2),
                                   "peak": VALU_PEAK_TFLOPS, "unit": "TFLOP/s",
                                   "frac": round(ach / VALU_PEAK_TFLOPS, 4),
                                   "fwd_achieved": round(5.0 * N * E / (avg_fwd * 1e-3) / 1e12, 2)}
    if args.flush:
        scratch = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        tf = []
        for k in range(min(K, 20)):
            scratch.fill_(k & 0xFF)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fwd()
            bwd()
            e1.record(stream)
            torch.cuda.synchronize()
            tf.append(e0.elapsed_time(e1))
        tf.sort()
        out["flushed_ms_median"] = round(med(tf), 5)
        out["flushed_GBs"] = round(bytes_step / (med(tf) * 1e-3) / 1e9, 1)
        del scratch
    out["cpu_baseline"] = None if args.no_cpu else _cpu_baseline(args.config, N)
    print(json.dumps(out), flush=True)


def _bench_lm(args):
    """Benchmark configuration c5: one training step of the Naju LM (12 layers,
    d_model 768, vocab 50257, N = 64) on a batch of 8 x 2048 uniformly random
    token ids: bf16 autocast forward, cross-entropy (the fused HIP kernels of
    naju_amd.xent on the bf16 logits), backward, gradient
    clipping at 1.0 and an AdamW step, with every mixer's scan on the HIP
    kernels. value = tokens per second."""
    import torch
    from naju_amd.mixer import NajuLM, build_optimizer
    from naju_amd.xent import cross_entropy
    from naju_amd import gemm_tuning
    dev = torch.device("cuda", 0)
    # GEMM solutions: the recorded choice for these shapes (PyTorch
    # TunableOp), or time them now with --tune-gemms (during the warmup)
    if args.tune_gemms:
        gemm_tuning.tune(args.tune_gemms)
        tuned = args.tune_gemms
    else:
        tuned = gemm_tuning.DEFAULT if gemm_tuning.load() else None
    V, d_model, n_layers, T, Bsz = 50257, 768, 12, 2048, 8
    torch.manual_seed(0)
    model = NajuLM(V, d_model=d_model, n_layers=n_layers, dropout=0.1, scan_backend="hip").to(dev)
    opt = build_optimizer(model, lr=1e-3, weight_decay=0.1)
    ids = torch.randint(0, V, (Bsz, T + 1), device=dev)
    x, y = ids[:, :-1].contiguous(), ids[:, 1:].contiguous()
    n_params = sum(p.numel() for p in model.parameters())

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(x)
            loss = cross_entropy(logits.view(-1, V), y.view(-1))
        opt.zero_grad(set_to_none=True)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Python's cyclic collector: a full collection walks every live object and
    # stalls the launching thread for tens of ms (the GPU queue drains
    # meanwhile); the objects alive after the warmup are moved out of its way
    gc.collect()
    gc.freeze()
    K = args.steps
    t0 = time.perf_counter()
    for _ in range(K):
        loss = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / K
    tokens = Bsz * T
    tflops = 6.0 * n_params * tokens / dt / 1e12
    out = {
        "metric": METRIC, "value": round(tokens / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 autocast (scan in f32 state)",
        "data": "synthetic (uniform random token ids; random init)",
        "config": {"workload": "naju LM training step c5: 12 layers, d_model 768, vocab 50257, N=64, "
                               "batch 8 x seq 2048, AdamW + clip 1.0",
                   "parameters": n_params, "parallelism": "single GPU",
                   "gemm_choices": os.path.basename(tuned) if tuned else "library default"},
        "loss_last": round(float(loss.detach()), 4),
        "roofline": {"kernel": "whole training step (6 x parameters x tokens)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def _traffic(config, N):
    """HBM bytes per launch of the backward kernel, from the committed
    rocprofv3 --pmc summary (profiles/traffic.json), or None."""
    path = os.path.join(_ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(f"{config}_N{N}_bwd")
    except (OSError, ValueError):
        return None


def _cpu_baseline(config, N):
    """The reference's sequential scan algorithm (torch CPU, autograd) on a
    bounded sample of the workload: all batch rows and channels, the first
    T_s timesteps. GB/s with the same algorithmic-byte formula."""
    import torch
    from naju_amd.workloads import CONFIGS, algorithmic_bytes, make_inputs
    from oracle.scan_ref import scan_loop_torch
    cfg = CONFIGS[config]
    Bsz, D = cfg["batch"], cfg["D"]
    Ts = 1024 if config in ("c1", "c2") else 256
    Ts = min(Ts, cfg["T"])
    cores = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(cores)
    ins = make_inputs(Bsz, Ts, D, N=N, dtype=torch.float32, gate=cfg["gate"], h0_std=cfg["h0_std"], seed=0,
                      device="cpu")
    names = ("u", "f_logit", "i_logit", "B", "C", "D_skip")
    xs = [ins[k].requires_grad_(True) for k in names]
    h0 = ins["h0"].requires_grad_(True) if ins["h0"] is not None else None
    t0 = time.perf_counter()
    yv = scan_loop_torch(*xs, h0=h0)
    yv.backward(ins["dy"])
    dt = time.perf_counter() - t0
    s = 4 if cfg["dtype"] == torch.float32 else 2
    nbytes = algorithmic_bytes(Bsz, Ts, D, N, s, s, s, h0 is not None)
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "seconds": round(dt, 2),
            "sample": f"{config} fwd+bwd, all {Bsz} batch rows x {D} channels, first {Ts} of {cfg['T']} "
                      f"timesteps, N={N}; torch-CPU loop restating naju/scan.py:79-93 with autograd, fp32 "
                      f"arithmetic; bytes counted at the workload's dtypes"}


if __name__ == "__main__":
    main()
