"""Benchmark of the fused fwd+bwd Naju scan on one MI355X.

A step is one forward (naju_scan_fwd) plus one backward (naju_scan_bwd) of the
scan over one batch of synthetic input resident in HBM, through the C ABI on
preallocated buffers (the hot path itself, no autograd bookkeeping). The
default workload is benchmark configuration c2 (naju_amd.workloads.CONFIGS): B=8, L=4096, D=1024, bf16
streams with fp32 state, N=1 (B=C=1), h0 ~ N(0, 0.1^2), dy ~ N(0,1).

value = algorithmic bytes of fwd+bwd per step * K / wall time of K steps
(GB/s), after W untimed warmup steps continued until at least WARM_MS of
warmup have passed (the GPU's clocks ramp over the first milliseconds of
work). The roofline object reports the dominant kernel (the backward) from
HIP events recorded on the launch stream inside the timed region. The same
line carries the step timed after a 1 GiB cache-flush write, and (default
c2, N = 1 run) a "configs" table: c1, c3 and c4 at N = 1 (c3 / c4 against the
70%-of-HBM step times), c2, c3 and c4 at N = 64 (HBM fraction and the
roofline of the instructions the kernels issue) and the c5 LM training step
(tokens/s and peak memory, at the default and a 128-row checkpoint
interval); an "inference" table (the no-grad forward at c2, N = 1 and 64);
and "reference_bench_shapes", the reference's own scan benchmark shapes
(naju/tests/bench_scan.py) in fp32 and bf16: forward under no_grad, forward
+ backward, peak memory. The cpu_baseline leg times the sequential torch-CPU
restatement of the reference's scan (oracle/scan_ref.py: scan_loop_torch,
the algorithm of reference naju/scan.py:79-93) on the host cores: c1 forward
and forward + backward at N = 1 and 64, and the benchmarked workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--N 1]
                       [--no-extras] [--no-cpu] [--no-flush]
"""
import argparse
import ctypes
import gc
import json
import os
import sys
import time

_ROOT = os.path.dirname(os.path.abspath(__file__))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

HBM_PEAK_GBS = 8000.0


CLOCK_GHZ = 2.4     # MI355X peak engine clock
N_SIMDS = 256 * 4   # 256 CUs x 4 SIMDs


def issue_roof(key, E, n, ms_step):
    """The compute roofline of a general-N step from the instructions its
    kernels issue (profiles/issue.json: rocprofv3 counters of the same
    workload): the VALU pipe needs 4 cycles per wave-instruction (16 lanes,
    no packed FP32) and the matrix-core pipe its busy cycles, the two pipes
    run concurrently, so the step needs at least the busier pipe's share per
    SIMD at the peak clock. frac = that time / the measured step; peak = the
    recurrence's 19n flop per element delivered at that rate. None without a
    record for this workload."""
    path = os.path.join(_ROOT, "profiles", "issue.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(key)
    except (OSError, ValueError):
        rec = None
    if not rec:
        return None
    valu_ms = 4.0 * rec["valu_wave_insts_per_step"] / N_SIMDS / (CLOCK_GHZ * 1e9) * 1e3
    mfma_ms = rec["mfma_busy_cycles_per_step"] / N_SIMDS / (CLOCK_GHZ * 1e9) * 1e3
    t_issue_ms = max(valu_ms, mfma_ms)
    work = 19.0 * n * E
    return {"bound": "instruction issue, the busier of the VALU and matrix-core pipes at 2.4 GHz",
            "work": "19N flop per element", "unit": "TFLOP/s",
            "achieved": round(work / (ms_step * 1e-3) / 1e12, 2),
            "peak": round(work / (t_issue_ms * 1e-3) / 1e12, 2),
            "valu_pipe_ms": round(valu_ms, 5), "mfma_pipe_ms": round(mfma_ms, 5),
            "frac": round(t_issue_ms / ms_step, 4), "source": "profiles/issue.json"}


METRIC = "fwd+bwd scan GB/s (% of HBM peak) at B8 L4096 D1024; LM tokens/s"


def _dt_size(dt):
    import torch
    return 4 if dt == torch.float32 else 2


# rooflines of the per-config lines: %-of-HBM targets from the survey's
# measurement plan (70% of 8 TB/s on the fused fwd+bwd at N = 1)
TARGET_FRAC = 0.70
# minimum wall time of the headline's untimed warmup (besides its W steps)
WARM_MS = 100.0


def _scan_case(L, config, N, dev, seed=0):
    """Inputs, outputs and workspace of one scan configuration, plus the two
    C-ABI calls of a step (forward, backward) as closures."""
    import torch
    from naju_amd import _lib
    from naju_amd.workloads import CONFIGS, algorithmic_bytes, config_inputs
    cfg = CONFIGS[config]
    Bsz, T, D = cfg["batch"], cfg["T"], cfg["D"]
    ins = config_inputs(config, N=N, seed=seed, device=dev)
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
    sh = torch.cuda.current_stream(dev).cuda_stream
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def fwd():
        _lib.check(L.naju_scan_fwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(h0), p(y), p(ck), None,
                                   Bsz, T, D, N, *dts, 0, p(ws), ws_bytes, sh))

    def fwd_infer():
        # the forward as under no_grad: no checkpoint is written
        _lib.check(L.naju_scan_fwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(h0), p(y), None, None,
                                   Bsz, T, D, N, *dts, 0, p(ws), ws_bytes, sh))

    def bwd():
        _lib.check(L.naju_scan_bwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(ck), p(dy), p(du), p(dfl),
                                   p(dil), p(dB), p(dC), p(dD), p(dh0), Bsz, T, D, N, *dts, 0, p(ws),
                                   ws_bytes, sh))

    def status():
        st = ctypes.c_uint32(0)
        _lib.check(L.naju_scan_workspace_status(p(ws), sh, ctypes.byref(st)))
        return st.value

    s_x, s_g, s_bc = _dt_size(xdt), _dt_size(fl.dtype), _dt_size(Bm.dtype)
    has_h0 = h0 is not None
    bf = algorithmic_bytes(Bsz, T, D, N, s_x, s_g, s_bc, has_h0, fwd=True, bwd=False)
    bb = algorithmic_bytes(Bsz, T, D, N, s_x, s_g, s_bc, has_h0, fwd=False, bwd=True)
    dname = {torch.bfloat16: "bf16", torch.float32: "f32", torch.float16: "f16"}[xdt]
    return dict(fwd=fwd, bwd=bwd, fwd_infer=fwd_infer, status=status, bytes_fwd=bf, bytes_bwd=bb, E=Bsz * T * D, dtype=dname,
                shape=(Bsz, T, D, N), has_h0=has_h0, gate=cfg["gate"], _keep=(ins, y, ck, du, dfl, dil, dB, dC,
                                                                              dD, dh0, ws))


def _time_case(case, steps, warmup, stream, min_warm_ms=0.0):
    """K steps back to back (wall clock between synchronisations), then K
    more with HIP events on the launch stream around each call. Untimed
    warmup: `warmup` steps, continued until min_warm_ms of wall time have
    passed (the GPU's clocks ramp up over the first milliseconds of work: a
    C2 N=1 step measures 0.192 ms after 10 warmup steps, 0.186 ms after 200)."""
    import torch
    # the first step (code loading, first-touch allocations) is not counted
    # towards min_warm_ms
    case["fwd"]()
    case["bwd"]()
    torch.cuda.synchronize()
    t_w = time.perf_counter()
    k = 1
    while k < warmup or (time.perf_counter() - t_w) * 1e3 < min_warm_ms:
        case["fwd"]()
        case["bwd"]()
        k += 1
        if k >= warmup and min_warm_ms > 0 and k % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    n_warm = k
    t0 = time.perf_counter()
    for _ in range(steps):
        case["fwd"]()
        case["bwd"]()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for k in range(steps):
        ev[k][0].record(stream)
        case["fwd"]()
        ev[k][1].record(stream)
        case["bwd"]()
        ev[k][2].record(stream)
    torch.cuda.synchronize()
    t_fwd = sorted(e[0].elapsed_time(e[1]) for e in ev)
    t_bwd = sorted(e[1].elapsed_time(e[2]) for e in ev)
    if case["status"]() != 0:
        raise RuntimeError("workspace status nonzero: a carry hand-off timed out")
    return dict(ms_step=ms_step, fwd_avg=sum(t_fwd) / steps, bwd_avg=sum(t_bwd) / steps,
                fwd_med=t_fwd[len(t_fwd) // 2], bwd_med=t_bwd[len(t_bwd) // 2], warmup_run=n_warm)


def _config_entry(L, config, N, dev, steps, warmup, target_ms=None):
    """One line of the per-configuration table: GB/s, % of HBM peak,
    elements/s and roofline fractions of the fused fwd+bwd step."""
    import torch
    case = _scan_case(L, config, N, dev)
    t = _time_case(case, steps, warmup, torch.cuda.current_stream(dev), min_warm_ms=100.0)
    b, T, D, n = case["shape"]
    step_bytes = case["bytes_fwd"] + case["bytes_bwd"]
    gbs = step_bytes / (t["ms_step"] * 1e-3) / 1e9
    e = {
        "workload": f"naju scan fwd+bwd {config}: B={b} L={T} D={D} N={n} {case['dtype']} streams, "
                    f"gates '{case['gate']}'" + (" with h0" if case["has_h0"] else ""),
        "steps": steps, "ms_per_step": round(t["ms_step"], 5),
        "GBs": round(gbs, 1), "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "elements_per_s": round(case["E"] / (t["ms_step"] * 1e-3), 1),
        "algorithmic_bytes_per_step": step_bytes,
        "fwd_ms_avg": round(t["fwd_avg"], 5), "bwd_ms_avg": round(t["bwd_avg"], 5),
        "roofline_frac_step": round(gbs / HBM_PEAK_GBS, 4),
        "roofline_frac_bwd": round(case["bytes_bwd"] / (t["bwd_avg"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }
    if n > 1:
        e["roofline_compute"] = issue_roof(f"{config}_N{n}", case["E"], n, t["ms_step"])
    if target_ms is not None:
        e["target_ms"] = target_ms
        e["meets_target"] = bool(t["ms_step"] <= target_ms)
    del case
    torch.cuda.empty_cache()
    return e


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps (default: 200 scan steps, 3 LM steps for --config c5); "
                         "the scan's warmup also lasts at least WARM_MS = 100 ms")
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"],
                    help="c1-c4: the scan itself; c5: the LM training step (tokens/s)")
    ap.add_argument("--N", type=int, default=1, help="state size (d_state)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the other configurations (c1, c3, c4 at N=1; c2-c4 at N=64; the c5 LM step), "
                         "the inference entries and the reference's benchmark shapes")
    ap.add_argument("--no-flush", action="store_true",
                    help="skip the steps timed with a 1 GiB cache-flush write before each step")
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

    if args.warmup is None:
        args.warmup = 3 if args.config == "c5" else 200
    if args.config == "c5":
        print(json.dumps(_bench_lm(args.steps, args.warmup, args.tune_gemms, line=True)), flush=True)
        return

    import torch
    from naju_amd import _lib

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
    N = args.N
    case = _scan_case(L, args.config, N, dev)
    stream = torch.cuda.current_stream(dev)
    # at least W warmup steps, and at least 100 ms of them: the clocks ramp
    # over the first milliseconds of work whatever W is
    t = _time_case(case, args.steps, args.warmup, stream, min_warm_ms=WARM_MS)
    Bsz, T, D, _ = case["shape"]
    bytes_fwd, bytes_bwd = case["bytes_fwd"], case["bytes_bwd"]
    bytes_step = bytes_fwd + bytes_bwd
    ms_step = t["ms_step"]
    K = args.steps
    value = bytes_step / (ms_step * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "warmup_steps_run": t["warmup_run"],
        "warmup_min_ms": WARM_MS,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": case["dtype"] + " streams, f32 state/accum",
        "data": f"synthetic (seeded; the {args.config} gate/input recipe of naju_amd.workloads)",
        "config": {"workload": f"naju scan fwd+bwd {args.config}: B={Bsz} L={T} D={D} N={N}"
                   + (" B=C=1" if N == 1 else " B,C~N(0,1/N)") + (" with h0" if case["has_h0"] else ""),
                   "batch": Bsz, "seq_len": T, "channels": D, "d_state": N,
                   "parallelism": "single GPU", "cache_flush": False},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "elements_per_s": round(case["E"] / (ms_step * 1e-3), 1),
        "algorithmic_bytes_per_step": bytes_step,
        "fwd_ms_avg": round(t["fwd_avg"], 5), "fwd_ms_median": round(t["fwd_med"], 5),
        "bwd_ms_avg": round(t["bwd_avg"], 5), "bwd_ms_median": round(t["bwd_med"], 5),
        "fwd_GBs": round(bytes_fwd / (t["fwd_avg"] * 1e-3) / 1e9, 1),
        "roofline": {
            "kernel": "naju_scan_bwd call = n1_bwd_kernel + fold_kernel" if N == 1 else "naju_scan_bwd call",
            "bound": "hbm",
            "achieved": round(bytes_bwd / (t["bwd_avg"] * 1e-3) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bytes_bwd / (t["bwd_avg"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": _traffic(args.config, N),
        },
    }
    if N > 1:
        # General N is compute-bound (about 19N flop per element against
        # 22-44 bytes): the roofline of the instructions the kernels issue
        out["roofline_compute"] = issue_roof(f"{args.config}_N{N}", case["E"], N, ms_step)
    if not args.no_flush:
        # the same step with a 1 GiB write before it: nothing of the step's
        # inputs is left in the 256 MB last-level cache
        scratch = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        tf = []
        for k in range(min(K, 20)):
            scratch.fill_(k & 0xFF)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            case["fwd"]()
            case["bwd"]()
            e1.record(stream)
            torch.cuda.synchronize()
            tf.append(e0.elapsed_time(e1))
        tf.sort()
        out["flushed_ms_median"] = round(tf[len(tf) // 2], 5)
        out["flushed_GBs"] = round(bytes_step / (tf[len(tf) // 2] * 1e-3) / 1e9, 1)
        out["flushed_pct_hbm_peak"] = round(100.0 * out["flushed_GBs"] / HBM_PEAK_GBS, 2)
        del scratch
    del case
    torch.cuda.empty_cache()
    if not args.no_extras and args.config == "c2" and N == 1:
        # every other configuration, each with its own GB/s and roofline
        # fraction; c3 / c4 against the 70%-of-HBM targets
        ks, ws = max(5, min(K, 20)), max(2, min(args.warmup, 5))
        tgt = lambda c: round(_step_bytes_of(c, 1) / (TARGET_FRAC * HBM_PEAK_GBS * 1e9) * 1e3, 4)  # noqa: E731
        ex = {}
        for name, cfg, n, target in (("c1_n1", "c1", 1, None), ("c3_n1", "c3", 1, tgt("c3")),
                                     ("c4_n1", "c4", 1, tgt("c4")), ("c2_n64", "c2", 64, None),
                                     ("c3_n64", "c3", 64, None), ("c4_n64", "c4", 64, None)):
            ex[name] = _config_entry(L, cfg, n, dev, ks, ws, target)
            print(f"bench: {name} {ex[name]['ms_per_step']} ms/step {ex[name]['GBs']} GB/s", file=sys.stderr,
                  flush=True)
        out["target_ms_c2_n1"] = tgt("c2")
        ex["stream_reference"] = _stream_reference(dev)
        print(f"bench: stream reference {ex['stream_reference']}", file=sys.stderr, flush=True)
        # 5 warmup and up to 30 timed steps: the first steps after the
        # warmup run about 2% slower than the steady state
        ex["c5_lm_step"] = _bench_lm(max(10, min(K, 30)), 5, None, line=False)
        print(f"bench: c5 {ex['c5_lm_step']['tokens_per_s']} tokens/s", file=sys.stderr, flush=True)
        ex["c5_lm_step_ckpt128"] = _bench_lm(max(10, min(K, 30)), 5, None, line=False, ckpt_rows=128)
        print(f"bench: c5 (128-row checkpoint interval) {ex['c5_lm_step_ckpt128']['tokens_per_s']} tokens/s",
              file=sys.stderr, flush=True)
        out["configs"] = ex
        out["inference"] = {name: _inference_entry(L, cfg, n, dev, ks)
                            for name, cfg, n in (("c2_n1", "c2", 1), ("c2_n64", "c2", 64))}
        print(f"bench: inference {out['inference']}", file=sys.stderr, flush=True)
        out["reference_bench_shapes"] = _reference_bench(dev)
        print("bench: reference bench shapes done", file=sys.stderr, flush=True)
    out["cpu_baseline"] = None if args.no_cpu else _cpu_baseline(args.config, N)
    print(json.dumps(out), flush=True)


def _inference_entry(L, config, N, dev, steps):
    """The no-grad forward (naju_scan_fwd with no checkpoint, what
    naju_scan_hip runs under torch.no_grad; the role of the reference's
    inference backend, naju/cuda/bw.py:36-38): GB/s of the forward's
    algorithmic bytes (read u, f_logit, i_logit, B, C, h0; write y) and % of
    HBM peak, HIP events around each call on the launch stream after at least
    100 ms of warmup."""
    import torch
    case = _scan_case(L, config, N, dev)
    stream = torch.cuda.current_stream(dev)
    t_w = time.perf_counter()
    while (time.perf_counter() - t_w) < 0.1:
        for _ in range(8):
            case["fwd_infer"]()
        torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in ev:
        e0.record(stream)
        case["fwd_infer"]()
        e1.record(stream)
    torch.cuda.synchronize()
    ts = sorted(e0.elapsed_time(e1) for e0, e1 in ev)
    ms = sum(ts) / len(ts)
    b, T, D, n = case["shape"]
    gbs = case["bytes_fwd"] / (ms * 1e-3) / 1e9
    out = {"workload": f"naju scan forward, no grad (no checkpoint): {config} B={b} L={T} D={D} N={n} "
                       f"{case['dtype']} streams" + (" with h0" if case["has_h0"] else ""),
           "steps": steps, "ms_avg": round(ms, 5), "ms_median": round(ts[len(ts) // 2], 5),
           "algorithmic_bytes": case["bytes_fwd"], "GBs": round(gbs, 1),
           "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
           "elements_per_s": round(case["E"] / (ms * 1e-3), 1)}
    del case
    torch.cuda.empty_cache()
    return out


# The reference's own scan benchmark shapes (naju/tests/bench_scan.py:112):
# (batch, T, d_inner, N)
REF_BENCH_SHAPES = ((8, 2048, 512, 64), (8, 8192, 512, 64), (2, 32768, 512, 64))


def _reference_bench(dev, iters=30, warmup=10):
    """The reference's scan benchmark (naju/tests/bench_scan.py:24-80) run
    on these kernels through the backend callable naju_scan_hip, as it runs
    each of its backends: its input recipe (u ~ N(0,1), f_logit ~ N(0,1)+2,
    i_logit ~ N(0,1)-1, B, C ~ N(0,1)/sqrt(N), D_skip ~ 0.01 N(0,1)), in
    float32 (its default) and bfloat16 (its --dtype bf16); forward under
    no_grad and forward + backward (y.backward(dy)), CUDA events around each
    call after `warmup` calls, median / p10 / p90 of `iters`; peak memory =
    torch.cuda.max_memory_allocated over the run, inputs included, with this
    package's workspace cache emptied first (so its workspace counts). The
    training step also at the 128-row checkpoint interval (the memory-light
    mode). GB/s and % of HBM use the algorithmic bytes of the pass (fwd: read
    u, f_logit, i_logit, B, C; write y)."""
    import torch
    from naju_amd import naju_scan_hip
    from naju_amd import scan as scan_mod
    from naju_amd.workloads import algorithmic_bytes

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        ts.sort()
        n = len(ts)
        return ts[n // 2], ts[max(0, n // 10)], ts[min(n - 1, 9 * n // 10)]

    def one(b, T, D, N, dtype, mode, rows):
        # everything of the measurement is local, so it is freed on return
        s = 4 if dtype == torch.float32 else 2
        scan_mod._WS._bufs.clear()
        scan_mod._WS._status.clear()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        base = torch.cuda.memory_allocated(dev)
        torch.cuda.reset_peak_memory_stats(dev)
        g = torch.Generator(device=dev).manual_seed(0)

        def r(*shape, add=0.0, scale=1.0):
            # one float32 temporary at a time
            return (torch.randn(*shape, generator=g, device=dev) * scale + add).to(dtype)
        ins = [r(b, T, D), r(b, T, D, add=2.0), r(b, T, D, add=-1.0), r(b, T, N, scale=N ** -0.5),
               r(b, T, N, scale=N ** -0.5), r(D, scale=0.01)]
        in_bytes = sum(x.numel() * x.element_size() for x in ins)
        if mode == "fwd":
            with torch.no_grad():
                med, p10, p90 = timed(lambda: naju_scan_hip(*ins))
            nbytes = algorithmic_bytes(b, T, D, N, s, s, s, False, fwd=True, bwd=False)
        else:
            for x in ins:
                x.requires_grad_(True)
            dy = torch.randn(b, T, D, device=dev, generator=g).to(dtype)

            def step():
                naju_scan_hip(*ins, ckpt_rows=rows).backward(dy)
                for x in ins:
                    x.grad = None
            med, p10, p90 = timed(step)
            nbytes = algorithmic_bytes(b, T, D, N, s, s, s, False)
        peak = torch.cuda.max_memory_allocated(dev) - base
        gbs = nbytes / (med * 1e-3) / 1e9
        return {"ms_median": round(med, 4), "ms_p10": round(p10, 4), "ms_p90": round(p90, 4),
                "peak_GiB": round(peak / 2 ** 30, 3), "inputs_GiB": round(in_bytes / 2 ** 30, 3),
                "Mtok_per_s": round(b * T / (med * 1e-3) / 1e6, 2),
                "GBs": round(gbs, 1), "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2)}

    res = {}
    for dtype, dname in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        for (b, T, D, N) in REF_BENCH_SHAPES:
            res[f"{dname} B={b} T={T} d_inner={D} N={N}"] = {
                mode: one(b, T, D, N, dtype, mode, rows)
                for mode, rows in (("fwd", None), ("fwd+bwd", None), ("fwd+bwd ckpt128", 128))}
    scan_mod._WS._bufs.clear()
    scan_mod._WS._status.clear()
    torch.cuda.empty_cache()
    return res


def _stream_reference(dev):
    """What plain streaming reaches on this GPU: torch.addcmul over three bf16
    input streams and one output stream (the forward's streams, contiguous,
    no scan), at the c2 size (inputs fit the 256 MB last-level cache, so
    repeated passes partly hit it) and at the c4 size (working set far above
    it). GB/s of algorithmic traffic, median of 10 timed passes."""
    import torch

    res = {}
    for name, (b, t, d) in (("c2_size", (8, 4096, 1024)), ("c4_size", (32, 8192, 4096))):
        x = [torch.randn(b, t, d, device=dev, dtype=torch.bfloat16) for _ in range(3)]
        y = torch.empty_like(x[0])
        nbytes = 4 * x[0].numel() * 2
        for _ in range(3):
            torch.addcmul(x[0], x[1], x[2], out=y)
        ts = []
        for _ in range(10):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            torch.addcmul(x[0], x[1], x[2], out=y)
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        ts.sort()
        res[name] = round(nbytes / (ts[len(ts) // 2] * 1e-3) / 1e9, 1)
        del x, y
        torch.cuda.empty_cache()
    res["unit"] = "GB/s"
    return res


def _step_bytes_of(config, N):
    import torch
    from naju_amd.workloads import CONFIGS, algorithmic_bytes
    c = CONFIGS[config]
    s = 4 if c["dtype"] == torch.float32 else 2
    return algorithmic_bytes(c["batch"], c["T"], c["D"], N, s, s, s, c["h0_std"] > 0)


def _bench_lm(steps, warmup, tune_gemms=None, line=True, ckpt_rows=None):
    """Benchmark configuration c5: one training step of the Naju LM (12 layers,
    d_model 768, vocab 50257, N = 64) on a batch of 8 x 2048 uniformly random
    token ids: bf16 autocast forward, cross-entropy (the fused HIP kernels of
    naju_amd.xent on the bf16 logits), backward, gradient
    clipping at 1.0 and an AdamW step (one fused HIP pass for both,
    naju_amd.optim), with every mixer's scan on the HIP kernels. value = tokens per second. line=True: the whole bench line;
    else the entry of the per-configuration table. ckpt_rows: the scans'
    checkpoint interval (NAJU_CKPT_ROWS for the run; None = the default).
    peak_GiB: torch.cuda.max_memory_allocated over the timed steps."""
    if ckpt_rows:
        os.environ["NAJU_CKPT_ROWS"] = str(int(ckpt_rows))
    try:
        return _bench_lm_run(steps, warmup, tune_gemms, line, ckpt_rows)
    finally:
        os.environ.pop("NAJU_CKPT_ROWS", None)


def _bench_lm_run(steps, warmup, tune_gemms, line, ckpt_rows):
    import torch
    from naju_amd.mixer import NajuLM, build_optimizer
    from naju_amd.optim import AdamW as NajuAdamW
    from naju_amd.xent import cross_entropy
    from naju_amd import gemm_tuning
    dev = torch.device("cuda", 0)
    # GEMM solutions: the recorded choice for these shapes (PyTorch
    # TunableOp), or time them now with --tune-gemms (during the warmup)
    if tune_gemms:
        gemm_tuning.tune(tune_gemms)
        tuned = tune_gemms
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
        if isinstance(opt, NajuAdamW):
            # clip_grad_norm_(params, 1.0) + step(), the clip inside the update
            opt.step(max_grad_norm=1.0)
        else:
            torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
            opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # Python's cyclic collector: a full collection walks every live object and
    # stalls the launching thread for tens of ms (the GPU queue drains
    # meanwhile); the objects alive after the warmup are moved out of its way
    gc.collect()
    gc.freeze()
    torch.cuda.reset_peak_memory_stats(dev)
    K = steps
    t0 = time.perf_counter()
    for _ in range(K):
        loss = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / K
    peak_gib = round(torch.cuda.max_memory_allocated(dev) / 2 ** 30, 3)
    gc.unfreeze()
    tokens = Bsz * T
    tflops = 6.0 * n_params * tokens / dt / 1e12
    workload = ("naju LM training step c5: 12 layers, d_model 768, vocab 50257, N=64, "
                "batch 8 x seq 2048, AdamW + clip 1.0"
                + (f", scan checkpoint every {ckpt_rows} rows" if ckpt_rows else ""))
    roof = {"kernel": "whole training step (6 x parameters x tokens)", "bound": "mfma",
            "achieved": round(tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
            "frac": round(tflops / 2500.0, 4), "traffic": None}
    loss_last = round(float(loss.detach()), 4)
    del model, opt, ids, x, y, loss
    torch.cuda.empty_cache()
    if not line:
        return {"workload": workload, "steps": K, "ms_per_step": round(dt * 1e3, 3),
                "tokens_per_s": round(tokens / dt, 1), "model_TFLOPs": round(tflops, 1),
                "roofline": roof, "loss_last": loss_last, "peak_GiB": peak_gib,
                "gemm_choices": os.path.basename(tuned) if tuned else "library default"}
    return {
        "metric": METRIC, "value": round(tokens / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": K,
        "warmup": warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 autocast (scan in f32 state)",
        "data": "synthetic (uniform random token ids; random init)",
        "config": {"workload": workload, "parameters": n_params, "parallelism": "single GPU",
                   "gemm_choices": os.path.basename(tuned) if tuned else "library default"},
        "loss_last": loss_last, "peak_GiB": peak_gib, "roofline": roof, "cpu_baseline": None,
    }


def _traffic(config, N):
    """HBM bytes per launch of the backward kernel, from the committed
    rocprofv3 --pmc summary (profiles/traffic.json), or None."""
    path = os.path.join(_ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(f"{config}_N{N}_bwd")
    except (OSError, ValueError):
        return None


def _cpu_info():
    """Host facts for the CPU baseline: core counts, model, SMT state."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    info["cpu_model"] = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    for key, path in (("smt_active", "/sys/devices/system/cpu/smt/active"),
                      ("smt_control", "/sys/devices/system/cpu/smt/control"),
                      ("cgroup_cpu_max", "/sys/fs/cgroup/cpu.max")):
        try:
            with open(path) as f:
                info[key] = f.read().strip()
        except OSError:
            pass
    return info


def _cpu_time(fn, runs=3):
    """1 warmup, then the median of `runs` timed runs (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts


def _cpu_baseline(config, N):
    """The reference's sequential scan algorithm (oracle/scan_ref.py:
    scan_loop_torch, restating naju/scan.py:79-93) on the host cores, torch
    intra-op threads = os.cpu_count(): 1 warmup + the median of 3 runs of
      * configuration c1 (2 x 1024 x 256, fp32) forward under no_grad and
        forward + backward (autograd), each at N = 1 and N = 64;
      * a bounded sample of the benchmarked workload, forward + backward:
        all batch rows and channels, the first timesteps up to 8 M elements
        (1024 of c2's 4096), whose GB/s (same algorithmic-byte formula) is
        the baseline value. The loop's backward costs O(T^2): each step's
        u[:, t]-style selection writes a full-size gradient in its backward,
        so the whole c2 length would be slower per element than the sample.
    """
    import torch
    from naju_amd.workloads import CONFIGS, algorithmic_bytes, make_inputs
    from oracle.scan_ref import scan_loop_torch
    info = _cpu_info()
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    info["torch_threads"] = torch.get_num_threads()
    names = ("u", "f_logit", "i_logit", "B", "C", "D_skip")

    def case(cfg_name, T, n, grad):
        cfg = CONFIGS[cfg_name]
        Bsz, D = cfg["batch"], cfg["D"]
        ins = make_inputs(Bsz, T, D, N=n, dtype=torch.float32, gate=cfg["gate"], h0_std=cfg["h0_std"], seed=0,
                          device="cpu")

        def run():
            if grad:
                xs = [ins[k].clone().requires_grad_(True) for k in names]
                h0 = ins["h0"].clone().requires_grad_(True) if ins["h0"] is not None else None
                scan_loop_torch(*xs, h0=h0).backward(ins["dy"])
            else:
                with torch.no_grad():
                    scan_loop_torch(*[ins[k] for k in names], h0=ins["h0"])

        med, ts = _cpu_time(run)
        s = 4 if cfg["dtype"] == torch.float32 else 2
        nbytes = algorithmic_bytes(Bsz, T, D, n, s, s, s, ins["h0"] is not None, fwd=True, bwd=grad)
        return {"seconds_median": round(med, 4), "seconds": [round(t, 4) for t in ts],
                "GBs": round(nbytes / med / 1e9, 5), "elements_per_s": round(Bsz * T * D / med, 1)}

    c1 = {}
    for n in (1, 64):
        c1[f"fwd_nograd_N{n}"] = case("c1", 1024, n, False)
        c1[f"fwd_bwd_N{n}"] = case("c1", 1024, n, True)
    cfg = CONFIGS[config]
    Ts = min(cfg["T"], max(1, (8 << 20) // (cfg["batch"] * cfg["D"] * max(1, N // 16))))
    main_case = case(config, Ts, N, True)
    part = "the whole workload" if Ts == cfg["T"] else f"first {Ts} of {cfg['T']} timesteps"
    return {"value": main_case["GBs"], "unit": "GB/s", "cores": info["torch_threads"], "kind": "port",
            "seconds": main_case["seconds_median"],
            "sample": f"{config} fwd+bwd, all {cfg['batch']} batch rows x {cfg['D']} channels, {part}, N={N}; "
                      f"torch-CPU loop restating naju/scan.py:79-93 with autograd (its backward is O(T^2)), fp32 "
                      f"arithmetic, bytes counted at the workload's dtypes; 1 warmup + median of 3",
            "elements_per_s": main_case["elements_per_s"], "c1": c1, "host": info}


if __name__ == "__main__":
    main()
