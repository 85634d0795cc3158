"""Benchmark of the MI355X Mamba-3 hot path (one JSON line on stdout).

Headline (`value`): the SSD scan forward at BASELINE config 1 -- B=8, L=2048,
H=12, P=64, N=128, chunk 64, bf16 storage with f32 accumulation, Rotational
dynamics with a learned trapezoid -- as whole-job tokens/s on one GPU.  A step
is one m3_scan call over the batch with every input already resident in HBM.

The scan runs as the library's chunk-parallel path over a workspace from
torch's allocator, allocated outside the timed region: at config 1 the fused
single launch (--scan-path three selects the three launches); the
single-pass kernel's time on the same inputs is reported beside it.

Also reported on the same line:
  roofline       the scan call's algorithmic bytes (its inputs and outputs)
                 over the average duration of one call (HIP events on the launch
                 stream), against the 8 TB/s HBM peak, plus its MFMA fraction;
  prefill        BASELINE config 4: the whole Mamba3Lm prefill (B=16, L=2048,
                 24 layers, int8 projections): tokens/s and matrix TFLOP/s;
  decode         BASELINE config 3: one token for 256 sequences through
                 24 layers x 24 heads (P=64, N=128) of f32 state cache, in place,
                 timed over consecutive steps: us per step, GB/s, fraction of HBM peak;
  decode_factored the same steps on the second cache format (m3_step_factored:
                 last_u carried as the previous token's x and b), on its own bytes;
  backward       config 1's scan backward (every input gradient from dL/dy):
                 us per call, fwd+bwd tokens/s, HBM fraction of its minimum bytes;
  decode_lm      the whole Mamba3Lm decode step around it (d_model 1536, int8
                 projections, head): us per step, tokens/s, GB/s over the state,
                 weight and logit bytes;
  decode_lm_default the same with the reference's default mixer (conv_kernel 4,
                 bc_bias): the convolution history joins the in-place caches;
  cpu_baseline  the CPU restatement of the reference's composed algorithm
                 (oracle/, OpenMP) on the same config-1 workload, on the host.

Inputs are synthetic (seeded torch RNG on the device, the distributions of
BASELINE.json).  `--gpus N` with N > 1 exits: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import dataclasses
import ctypes as C
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mamba-trainer_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA, TFLOP/s

# HBM-side bytes of one headline scan call and the MFMA-busy fraction of its
# kernel, from profiles/scan_config1_kernels.txt (rocprofv3 FETCH_SIZE /
# WRITE_SIZE per dispatch scaled by a 256 MiB copy, SQ_VALU_MFMA_BUSY_CYCLES
# over GRBM_GUI_ACTIVE).  At config 1 the library runs the fused single
# launch (chunk_scan_fused_kernel): 205.4 MB read + 107.0 MB written.
# Counters cannot be read inside this process; re-measured when the kernels
# change.
SCAN_TRAFFIC_BYTES = 312_500_000
SCAN_MFMA_BUSY = {"chunk_scan_fused_kernel": 0.052}

# BASELINE config 1 (the headline) and config 3 (decode)
SCAN = dict(B=8, L=2048, H=12, P=64, N=128, R=1, Q=64)
DECODE = dict(B=256, layers=24, H=24, P=64, N=128, R=1, sets=4)


def scan_algorithmic(B, L, H, P, N, R, Q, s_io=2, theta_per_token=True, want_state=True):
    """Algorithmic HBM bytes and MFMA-contractible FLOPs of one scan launch.

    Per (token, head): x, b, c (and theta, materialised per token) read at s_io
    bytes, dt and lambda read as f32, y written at s_io bytes; plus the outgoing
    state h, last_u [B,H,P,N] f32 and angle [B,H,N/2] f32 when wanted.
    FLOPs per (token, head): 2*Q*R^2*(N+P) (the masked C B^T and its product
    with X) + 4*R*P*N (chunk state and carry-in output).
    """
    per_tok = (P * R + 2 * N * R + (N // 2 if theta_per_token else 0)) * s_io + 8 + P * R * s_io
    nbytes = B * L * H * per_tok
    if want_state:
        nbytes += B * H * (2 * P * N + N // 2) * 4
    flops = B * L * H * (2 * Q * R * R * (N + P) + 4 * R * P * N)
    return nbytes, flops


def decode_algorithmic(B, H, P, N, R):
    """Bytes per layer step: h and last_u read + written (16 B per state element)
    plus x, b, c, theta, dt, lambda read, angle read + written, y written (f32)."""
    state = 16 * B * H * P * N
    io = B * H * (P * R + 2 * N * R + N // 2 + 2 + 2 * (N // 2) + P * R) * 4
    return state + io


def decode_factored_algorithmic(B, H, P, N, R):
    """Bytes per layer step of the factored form (m3_step_factored): h read +
    written (8 B per state element), the inputs and outputs of
    decode_algorithmic, and the previous token's x and b read + written."""
    state = 8 * B * H * P * N
    io = B * H * (P * R + 2 * N * R + N // 2 + 2 + 2 * (N // 2) + P * R) * 4
    prev = B * H * 2 * (P * R + N * R) * 4
    return state + io + prev


def make_scan_inputs(torch, dev, B, L, H, P, N, R, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    x = torch.randn(B, L, H, P, R, device=dev, generator=g).to(bf)
    b = (torch.randn(B, L, H, N, R, device=dev, generator=g) / math.sqrt(N)).to(bf)
    c = (torch.randn(B, L, H, N, R, device=dev, generator=g) / math.sqrt(N)).to(bf)
    dt = torch.nn.functional.softplus(torch.randn(B, L, H, device=dev, generator=g) - 3.0
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, L, H, device=dev, generator=g))
    a_log = torch.rand(H, device=dev, generator=g) * math.log(16.0)
    # theta ~ U(0, pi) per head per state pair, materialised per token
    theta = (torch.rand(1, 1, H, N // 2, device=dev, generator=g) * math.pi).expand(
        B, L, H, N // 2).contiguous().to(bf)
    return dict(x=x, b=b, c=c, dt=dt, lam=lam, a_log=a_log, theta=theta)


def bench_scan(torch, lib, L_, args, chunk_parallel=True, inp=None, sets=None):
    """Config 1's scan through m3_scan.  Step i runs on input/output set
    i % sets: with several sets (their inputs total well over the 256 MB
    Infinity Cache) no call finds the previous call's inputs cached, so the
    figure is HBM-bound as a fresh batch would be; sets=1 re-reads one resident
    set (the cache-assisted figure, reported beside it)."""
    dev = "cuda:0"
    s = SCAN
    B, L, H, P, N, R, Q = s["B"], s["L"], s["H"], s["P"], s["N"], s["R"], s["Q"]
    K = args.scan_sets if sets is None else sets
    if inp is None:
        inp = [make_scan_inputs(torch, dev, B, L, H, P, N, R, 0x4D414D43 + k) for k in range(K)]
    calls, keep = [], []
    ws = None
    for k in range(K):
        d = inp[k]
        y = torch.empty_like(d["x"])
        h = torch.empty(B, H, P, N, device=dev)
        lu = torch.empty(B, H, P, N, device=dev)
        ang = torch.empty(B, H, N // 2, device=dev)
        cin = L_.ScanInputsC(B, L, H, P, N, R, L_.M3_BF16, d["x"].data_ptr(), d["b"].data_ptr(),
                             d["c"].data_ptr(), d["dt"].data_ptr(), d["a_log"].data_ptr(),
                             d["lam"].data_ptr(), d["theta"].data_ptr(), None, None, Q, 1,
                             None, 0)
        if chunk_parallel:
            need = int(lib.m3_scan_workspace_bytes(C.byref(cin)))
            if ws is None:
                ws = torch.empty(need, dtype=torch.uint8, device=dev)
            cin.workspace, cin.workspace_bytes = ws.data_ptr(), need
        cout = L_.ScanOutputC(y.data_ptr(), L_.SsmStateC(h.data_ptr(), lu.data_ptr(),
                                                         ang.data_ptr()))
        keep.append((cin, cout, y, h, lu, ang))
        calls.append((C.byref(cin), C.byref(cout)))
    stream = torch.cuda.current_stream()
    sp = C.c_void_p(stream.cuda_stream)
    fn = lib.m3_scan

    def step(i):
        pin, pout = calls[i % K]
        st = fn(pin, pout, sp)
        if st != 0:
            L_.check(st)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1) / args.steps
    for kp in keep:
        assert torch.isfinite(kp[2].float()).all(), "non-finite scan output"
    in_bytes = sum(t.numel() * t.element_size() for d in inp[:K] for t in d.values())
    return dict(wall_ms=wall * 1e3 / args.steps, kernel_ms=ev_ms, tokens=B * L, inp=inp,
                sets=K, input_MB=round(in_bytes / 1e6, 1),
                workspace_bytes=0 if ws is None else ws.numel())


def cpu_model():
    """The host CPU's model name and logical core count (lscpu's fields, read
    from /proc/cpuinfo)."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": name, "host_logical_cpus": os.cpu_count()}


def _pause_for_trace(args):
    """With --only, a 0.5 s idle gap separates a leg's warm-up (weight
    quantisation, GEMM plan probes) from its timed passes, so a kernel trace
    can tell them apart."""
    if args.only:
        time.sleep(0.5)


# Mamba3Lm prefill (next-row workload, reported beside the headline)
PREFILL = dict(B=16, L=2048, vocab=32000, d_model=768, layers=24, H=12, P=64, N=128, G=12)


def prefill_flops(p):
    """Matrix FLOPs of one prefill: per layer in_proj and out_proj, then the head
    (the scan's own MFMA work is counted in scan_algorithmic)."""
    d, H, P, N, G = p["d_model"], p["H"], p["P"], p["N"], p["G"]
    din = H * P
    width = 2 * din + 2 * G * N + H + H + H * N // 2
    m = p["B"] * p["L"]
    per_layer = 2 * m * d * width + 2 * m * din * d
    return per_layer * p["layers"] + 2 * m * d * p["vocab"]


def bench_prefill(torch, args):
    """Config 4 end to end: embedding, 24 x (RMSNorm, int8 in_proj, prologue,
    scan, gate, int8 out_proj + residual), final norm, head; random init."""
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    p = PREFILL
    dev = "cuda:0"
    ssm = SsmConfig(d_model=p["d_model"], n_heads=p["H"], head_dim=p["P"], d_state=p["N"],
                    n_groups=p["G"], discretization=Discretization.LearnedTrapezoid,
                    dynamics=StateDynamics.Rotational, mode=SsmMode(1), chunk_size=64,
                    conv_kernel=None, bc_norm=True)
    lm = Mamba3Lm(Mamba3LmConfig(vocab_size=p["vocab"], d_model=p["d_model"],
                                 n_layers=p["layers"], ssm=ssm, int8_weights=True, seed=4), dev)
    g = torch.Generator(device=dev).manual_seed(0x4D414D46)
    ids = torch.randint(0, p["vocab"], (p["B"], p["L"]), device=dev, generator=g)
    for _ in range(2):
        logits = lm.forward(ids)
    torch.cuda.synchronize()
    _pause_for_trace(args)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.prefill_steps):
        logits = lm.forward(ids)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.prefill_steps
    assert torch.isfinite(logits[0, :4].float()).all(), "non-finite logits"
    flops = prefill_flops(p)
    toks = p["B"] * p["L"]
    return {"workload": "config 4: Mamba3Lm prefill B=16 L=2048, vocab 32000, d_model 768, "
                        "24 layers x 12 heads x 64, N 128, groups 12, bc_norm, no conv, int8 "
                        "per-output-channel fake-quant projections, bf16 activations",
            "tokens_per_s": round(toks / (ms * 1e-3), 1), "ms_per_prefill": round(ms, 3),
            "matrix_tflop": round(flops / 1e12, 3),
            "matrix_tflops_achieved": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_bf16_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}


def bench_ingest(torch, args):
    """Row (f4): a checkpoint of config 4's model in the reference's JSON format
    written, parsed and restored (checkpoint.rs:54-83, module.rs:249-285); the
    parse is timed beside Python's json module on one layer's in_proj."""
    import json as _json
    import tempfile
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    from mamba3.checkpoint import Checkpoint
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    p = PREFILL
    dev = "cuda:0"
    ssm = SsmConfig(d_model=p["d_model"], n_heads=p["H"], head_dim=p["P"], d_state=p["N"],
                    n_groups=p["G"], discretization=Discretization.LearnedTrapezoid,
                    dynamics=StateDynamics.Rotational, mode=SsmMode(1), chunk_size=64,
                    conv_kernel=None, bc_norm=True)
    cfg = Mamba3LmConfig(vocab_size=p["vocab"], d_model=p["d_model"], n_layers=p["layers"],
                         ssm=ssm, int8_weights=True, seed=6)
    src = Mamba3Lm(cfg, dev)
    ck = Checkpoint.capture(src, 1).with_metadata({"d_model": p["d_model"]})
    values = ck.num_values()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "config4.json")
        t0 = time.perf_counter()
        ck.save(path)
        t_save = time.perf_counter() - t0
        nbytes = os.path.getsize(path)
        t0 = time.perf_counter()
        loaded = Checkpoint.load(path)
        t_load = time.perf_counter() - t0
        dst = Mamba3Lm(dataclasses.replace(cfg, seed=7), dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loaded.restore(dst, strict=True)
        torch.cuda.synchronize()
        t_restore = time.perf_counter() - t0
        ids = torch.randint(0, p["vocab"], (1, 64), device=dev)
        same = bool(torch.equal(src.forward(ids), dst.forward(ids)))
        # Python's json on one layer's in_proj (a bounded sample of the same text)
        e = loaded.state.entries["stack.layers.0.mixer.in_proj.weight"]
        sample = _json.dumps({"entries": {"w": {"shape": e.shape, "data": e.data.tolist()}}})
        t0 = time.perf_counter()
        _json.loads(sample)
        t_py = time.perf_counter() - t0
    return {"workload": "config-4 Mamba3Lm checkpoint (24 layers, vocab 32000, d_model 768) in "
                        "the reference's JSON format",
            "values": values, "file_MB": round(nbytes / 1e6, 1),
            "save_s": round(t_save, 3), "load_s": round(t_load, 3),
            "load_MBps": round(nbytes / 1e6 / t_load, 1), "restore_s": round(t_restore, 3),
            "restored_logits_identical": same, "threads": min(os.cpu_count() or 1, 16),
            "python_json_MBps": round(len(sample) / 1e6 / t_py, 1),
            "python_json_sample": "one layer's in_proj (4.1 M values) through json.loads"}


# Row (f2): the whole Mamba3Lm decode step at config 3's mixer shapes
DECODE_LM = dict(B=256, vocab=32000, d_model=1536, layers=24, H=24, P=64, N=128, G=24)


def scan_backward_algorithmic(B, L, H, P, N, R, s_io=2):
    """HBM bytes of one backward call at the algorithm's minimum: x, b, c,
    theta (per token), dy read at s_io bytes and dt, lambda as f32; dx, db, dc,
    dtheta written at s_io bytes and ddt, dlambda as f32."""
    per_tok = (2 * P * R + 2 * N * R + N // 2) * s_io + 8 + (P * R + 2 * N * R + N // 2) * s_io + 8
    return B * L * H * per_tok


def scan_backward_flops(B, L, H, P, N, R, Q=32):
    """MFMA-contractible FLOPs of one backward call, counted like the forward
    (full Q x Q band products): per row (token, rank), the band products C~B~^T,
    dY X^T, M^T dY, (dM o K) B~ and (dM o K)^T C~ (2 Q (3N + 2P)), and the five
    P x N products B~ Gh^T, dY S, X Gh, the V-state and the recompute of U
    (10 P N).  Q is the backward's chunk length in rows."""
    return B * L * H * R * (2 * Q * (3 * N + 2 * P) + 10 * P * N)


def bench_backward(torch, lib, L_, args, inp, fwd_ms):
    """Config 1's scan backward (m3_scan_backward): dL/dy -> every input
    gradient, the forward chunk states recomputed inside the call."""
    import ctypes as C
    dev = "cuda:0"
    s = SCAN
    B, L, H, P, N, R = s["B"], s["L"], s["H"], s["P"], s["N"], s["R"]
    g = torch.Generator(device=dev).manual_seed(0x4D414D45)
    dy = torch.randn(B, L, H, P, R, device=dev, generator=g).to(torch.bfloat16)
    cin = L_.ScanInputsC(B, L, H, P, N, R, L_.M3_BF16, inp["x"].data_ptr(), inp["b"].data_ptr(),
                         inp["c"].data_ptr(), inp["dt"].data_ptr(), inp["a_log"].data_ptr(),
                         inp["lam"].data_ptr(), inp["theta"].data_ptr(), None, None, s["Q"], 0,
                         None, 0)
    need = int(lib.m3_scan_backward_workspace_bytes(C.byref(cin)))
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    cin.workspace, cin.workspace_bytes = ws.data_ptr(), need
    gx, gb, gc, gth = (torch.empty_like(inp[k]) for k in ("x", "b", "c", "theta"))
    gdt, glam = torch.empty_like(inp["dt"]), torch.empty_like(inp["lam"])
    ga = torch.empty(H, device=dev)
    gr = L_.ScanGradsC(dy.data_ptr(), None, None, gx.data_ptr(), gb.data_ptr(), gc.data_ptr(),
                       gdt.data_ptr(), glam.data_ptr(), ga.data_ptr(), gth.data_ptr(), None, None,
                       None, None)
    stream = torch.cuda.current_stream()
    call = lambda: L_.check(lib.m3_scan_backward(C.byref(cin), C.byref(gr),
                                                 C.c_void_p(stream.cuda_stream)))
    for _ in range(max(2, args.warmup // 4)):
        call()
    torch.cuda.synchronize()
    steps = max(5, args.steps // 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / steps * 1e3
    assert bool(torch.isfinite(gx.float()).all()) and bool(torch.isfinite(ga).all())
    nbytes = scan_backward_algorithmic(B, L, H, P, N, R)
    flops = scan_backward_flops(B, L, H, P, N, R)
    tokens = B * L
    tflops = flops / (us * 1e-6) / 1e12
    out = {"us_per_call": round(us, 2), "calls": steps,
           "tokens_per_s_bwd": round(tokens / (us * 1e-6), 1),
           "algorithmic_bytes": nbytes, "achieved_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
           "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_flops": flops, "mfma_f32_tflops": round(tflops, 2),
           "frac_mfma_f32_peak": round(tflops / MFMA_F32_PEAK_TFLOPS, 4),
           "bound": "mfma_f32", "workspace_MB": round(need / 1e6, 1),
           "note": "bf16 storage, f32 arithmetic (MFMA f32 16x16x4); includes the recompute "
                   "of the forward chunk states"}
    if fwd_ms is not None:
        out["tokens_per_s_fwd_bwd"] = round(tokens / ((us * 1e-3 + fwd_ms) * 1e-3), 1)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_backward_baseline(args)
    return out


def cpu_backward_baseline(args):
    """The oracle's f64 reverse mode of the scan recurrence on the host (OpenMP
    over batch x head), on a sample of config 1: batch 1, every head, full
    length, bf16-rounded inputs."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle
    from cases import baseline_inputs
    s = SCAN
    rng = np.random.default_rng(0x4D414D45)
    inp = baseline_inputs(rng, 1, s["L"], s["H"], s["P"], s["N"], 1, theta=True, dtype="bf16")
    dy = rng.standard_normal((1, s["L"], s["H"], s["P"], 1)).astype(np.float32)
    run = lambda: oracle.scan_backward_f64(inp["x"], inp["b"], inp["c"], inp["dt"], inp["a_log"],
                                           inp["lam"], dy, inp["theta"])
    run()   # warmup
    times = []
    for _ in range(args.cpu_reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(s["L"] / med, 1), "unit": "tokens/s", "cores": oracle.num_threads(),
            "kind": "port", **cpu_model(),
            "sample": (f"config 1 at batch 1 (L=2048, H=12, P=64, N=128, Rotational, bf16-rounded "
                       f"inputs), f64 reverse mode of the recurrence (oracle/mamba3_oracle.c "
                       f"m3o_scan_backward_f64), 1 warmup + median of {args.cpu_reps}: "
                       f"{med:.3f} s per pass")}


def bench_decode_lm(torch, args):
    """One token per sequence through the 24-layer stack with the state cache
    updated in place: embedding, 24 x (RMSNorm, int8 in_proj, prologue, decode
    step, gate, int8 out_proj + residual), final norm, head (lm.rs:337-353)."""
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    p = DECODE_LM
    dev = "cuda:0"
    B, H, P, N = p["B"], p["H"], p["P"], p["N"]
    ssm = SsmConfig(d_model=p["d_model"], n_heads=H, head_dim=P, d_state=N, n_groups=p["G"],
                    discretization=Discretization.LearnedTrapezoid,
                    dynamics=StateDynamics.Rotational, mode=SsmMode(1), chunk_size=64,
                    conv_kernel=None, bc_norm=True)
    lm = Mamba3Lm(Mamba3LmConfig(vocab_size=p["vocab"], d_model=p["d_model"],
                                 n_layers=p["layers"], ssm=ssm, int8_weights=True, seed=5), dev)
    g = torch.Generator(device=dev).manual_seed(0x4D414D47)
    cache = lm.empty_cache(B, dev)
    for c in cache:                        # config 3's state: N(0, 0.1), angles U(-pi, pi)
        c.ssm.h.normal_(0.0, 0.1, generator=g)
        c.ssm.last_u.normal_(0.0, 0.1, generator=g)
        c.ssm.angle.uniform_(-math.pi, math.pi, generator=g)
    ids = torch.randint(0, p["vocab"], (16, B, 1), device=dev, generator=g)
    for i in range(4):
        logits = lm.forward_cached(ids[i], cache)
    torch.cuda.synchronize()
    _pause_for_trace(args)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    steps = args.decode_lm_steps
    e0.record(stream)
    for i in range(steps):
        logits = lm.forward_cached(ids[i % 16], cache)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_eager = e0.elapsed_time(e1) / steps
    assert torch.isfinite(logits.float()).all(), "non-finite logits"
    # the same step captured once as a HIP graph and replayed (the serving form)
    graph = lm.capture_decode(cache, B)
    for i in range(2):
        graph.step(ids[i])
    torch.cuda.synchronize()
    _pause_for_trace(args)
    e0.record(stream)
    for i in range(steps):
        logits = graph.step(ids[i % 16])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert torch.isfinite(logits.float()).all(), "non-finite logits (graph)"
    # at batch 1 the eager step is bound by the host issuing its launches; the
    # graph replay is not
    small = {}
    cache1 = lm.empty_cache(1, dev)
    ids1 = ids[:, :1]
    for i in range(4):
        lm.forward_cached(ids1[i], cache1)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        lm.forward_cached(ids1[i % 16], cache1)
    e1.record(stream)
    torch.cuda.synchronize()
    small["us_per_step_eager"] = round(e0.elapsed_time(e1) / steps * 1e3, 1)
    graph1 = lm.capture_decode(cache1, 1)
    for i in range(2):
        graph1.step(ids1[i])
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        graph1.step(ids1[i % 16])
    e1.record(stream)
    torch.cuda.synchronize()
    small["us_per_step_graph"] = round(e0.elapsed_time(e1) / steps * 1e3, 1)
    d, NL = p["d_model"], p["layers"]
    width = ssm.in_proj_width()
    weights = NL * (d * width * 2 + width * 4 + d * d * 2 + d * 4) + d * p["vocab"] * 2
    nbytes = NL * decode_algorithmic(B, H, P, N, 1) + weights + B * p["vocab"] * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    # the same model on factored caches (h plus the previous token's x and b
    # per layer; decode steps stream h only), as a graph replay
    cache_f = lm.empty_cache(B, dev, factored=True)
    for c in cache_f:
        c.ssm.h.normal_(0.0, 0.1, generator=g)
        c.ssm.x_prev.normal_(0.0, 1.0, generator=g)
        c.ssm.b_prev.normal_(0.0, 1.0 / math.sqrt(N), generator=g)
        c.ssm.angle.uniform_(-math.pi, math.pi, generator=g)
    graph_f = lm.capture_decode(cache_f, B)
    for i in range(2):
        graph_f.step(ids[i])
    torch.cuda.synchronize()
    _pause_for_trace(args)
    e0.record(stream)
    for i in range(steps):
        logits = graph_f.step(ids[i % 16])
    e1.record(stream)
    torch.cuda.synchronize()
    ms_f = e0.elapsed_time(e1) / steps
    assert torch.isfinite(logits.float()).all(), "non-finite logits (factored caches)"
    nbytes_f = NL * decode_factored_algorithmic(B, H, P, N, 1) + weights + B * p["vocab"] * 2
    factored = {"us_per_step": round(ms_f * 1e3, 1), "tokens_per_s": round(B / (ms_f * 1e-3), 1),
                "bytes_per_step": nbytes_f,
                "frac_hbm_peak": round(nbytes_f / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "cache": "factored (Mamba3Lm.empty_cache(factored=True)), graph replay"}
    return {"workload": "Mamba3Lm decode step, batch 256 x 1 token, vocab 32000, d_model 1536, "
                        "24 layers x 24 heads x 64, N 128, groups 24, bc_norm, no conv, int8 "
                        "per-output-channel fake-quant projections, f32 state cache in place",
            "us_per_step": round(ms * 1e3, 1), "tokens_per_s": round(B / (ms * 1e-3), 1),
            "bytes_per_step": nbytes, "achieved_GBps": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "steps": steps,
            "launch": "one HIP graph replay per step (Mamba3Lm.capture_decode)",
            "us_per_step_eager": round(ms_eager * 1e3, 1), "batch1": small,
            "factored_cache": factored}


def bench_decode_lm_default(torch, args):
    """The decode step of bench_decode_lm with the reference's default mixer
    (config.rs:131-156: conv_kernel 4, bc_bias, bc_norm, D skip, no post-gate
    norm) at the same widths: each layer's cache adds the convolution history
    [256, 3, 7680] bf16, read and rewritten in place by the fused mixer step
    (m3_mixer_step_conv, one launch a layer).  Graph replay on full-format
    and on factored caches."""
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    p = DECODE_LM
    dev = "cuda:0"
    B, H, P, N, K = p["B"], p["H"], p["P"], p["N"], 4
    ssm = SsmConfig(d_model=p["d_model"], n_heads=H, head_dim=P, d_state=N, n_groups=p["G"],
                    discretization=Discretization.LearnedTrapezoid,
                    dynamics=StateDynamics.Rotational, mode=SsmMode(1), chunk_size=64,
                    conv_kernel=K, bc_norm=True, bc_bias=True, post_gate_norm=False)
    lm = Mamba3Lm(Mamba3LmConfig(vocab_size=p["vocab"], d_model=p["d_model"],
                                 n_layers=p["layers"], ssm=ssm, int8_weights=True, seed=5), dev)
    g = torch.Generator(device=dev).manual_seed(0x4D414D48)
    ids = torch.randint(0, p["vocab"], (16, B, 1), device=dev, generator=g)
    d, NL = p["d_model"], p["layers"]
    width = ssm.in_proj_width()
    chans = H * P + 2 * p["G"] * N
    weights = NL * (d * width * 2 + width * 4 + d * d * 2 + d * 4) + d * p["vocab"] * 2
    conv_bytes = NL * (2 * B * (K - 1) * chans * 2 + (K + 1) * chans * 4)
    steps = args.decode_lm_steps
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {"workload": "Mamba3Lm decode step, batch 256 x 1 token, vocab 32000, d_model 1536, "
                       "24 layers x 24 heads x 64, N 128, groups 24, the reference's default "
                       "mixer (conv_kernel 4, bc_bias, bc_norm), int8 per-output-channel "
                       "fake-quant projections, state and history caches in place",
           "steps": steps, "launch": "one HIP graph replay per step (Mamba3Lm.capture_decode)"}
    for factored in (False, True):
        cache = lm.empty_cache(B, dev, factored=factored)
        for c in cache:
            c.ssm.h.normal_(0.0, 0.1, generator=g)
            if factored:
                c.ssm.x_prev.normal_(0.0, 1.0, generator=g)
                c.ssm.b_prev.normal_(0.0, 1.0 / math.sqrt(N), generator=g)
            else:
                c.ssm.last_u.normal_(0.0, 0.1, generator=g)
            c.ssm.angle.uniform_(-math.pi, math.pi, generator=g)
            c.conv.normal_(0.0, 1.0, generator=g)
        graph = lm.capture_decode(cache, B)
        for i in range(2):
            graph.step(ids[i])
        torch.cuda.synchronize()
        _pause_for_trace(args)
        e0.record(stream)
        for i in range(steps):
            logits = graph.step(ids[i % 16])
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        assert torch.isfinite(logits.float()).all(), "non-finite logits (default mixer)"
        per_layer = (decode_factored_algorithmic if factored else decode_algorithmic)(B, H, P, N, 1)
        nbytes = NL * per_layer + conv_bytes + weights + B * p["vocab"] * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        leg = {"us_per_step": round(ms * 1e3, 1), "tokens_per_s": round(B / (ms * 1e-3), 1),
               "bytes_per_step": nbytes, "achieved_GBps": round(gbs, 1),
               "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        if factored:
            out["factored_cache"] = leg
        else:
            out.update(leg)
        del graph, cache
    return out


# BASELINE configs 0 and 2 (parity cases; their forward scans are reported beside
# the headline): name -> (B, L, H, P, N, R, bf16, rotational)
OTHER_SCANS = {"config0": (2, 512, 4, 64, 64, 1, False, False),
               "config2": (4, 4096, 24, 64, 128, 4, True, True)}


def bench_other_scans(torch, lib, L_, args):
    """Forward scans of configs 0 (f32, Real, SISO) and 2 (bf16, Rotational,
    MIMO rank 4) through m3_scan with the workspace the library asks for,
    rotating over --scan-sets input/output sets as the headline does (config 2
    takes three: one set is 1.26 GB already)."""
    dev = "cuda:0"
    out = {}
    for name, (B, L, H, P, N, R, bf16, rot) in OTHER_SCANS.items():
        K = min(args.scan_sets, 3) if name == "config2" else args.scan_sets
        st = torch.bfloat16 if bf16 else torch.float32
        calls, keep = [], []
        ws = None
        for k in range(K):
            g = torch.Generator(device=dev).manual_seed(0x4D414D43 + k)
            x = torch.randn(B, L, H, P, R, device=dev, generator=g).to(st)
            b = (torch.randn(B, L, H, N, R, device=dev, generator=g) / math.sqrt(N)).to(st)
            c = (torch.randn(B, L, H, N, R, device=dev, generator=g) / math.sqrt(N)).to(st)
            dt = torch.nn.functional.softplus(torch.randn(B, L, H, device=dev, generator=g) - 3.0
                                              ).clamp(1e-3, 0.1)
            lam = torch.sigmoid(torch.randn(B, L, H, device=dev, generator=g))
            a_log = torch.rand(H, device=dev, generator=g) * math.log(16.0)
            th = ((torch.rand(1, 1, H, N // 2, device=dev, generator=g) * math.pi)
                  .expand(B, L, H, N // 2).contiguous().to(st)) if rot else None
            y = torch.empty_like(x)
            h = torch.empty(B, H, P, N, device=dev)
            lu = torch.empty_like(h)
            ang = torch.empty(B, H, N // 2, device=dev) if rot else None
            cin = L_.ScanInputsC(B, L, H, P, N, R, L_.M3_BF16 if bf16 else L_.M3_F32,
                                 x.data_ptr(), b.data_ptr(), c.data_ptr(), dt.data_ptr(),
                                 a_log.data_ptr(), lam.data_ptr(), th.data_ptr() if rot else None,
                                 None, None, 64, 1, None, 0)
            need = int(lib.m3_scan_workspace_bytes(C.byref(cin)))
            if ws is None:
                ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
            if need:
                cin.workspace, cin.workspace_bytes = ws.data_ptr(), need
            cout = L_.ScanOutputC(y.data_ptr(), L_.SsmStateC(h.data_ptr(), lu.data_ptr(),
                                                             ang.data_ptr() if rot else None))
            keep.append((cin, cout, x, b, c, dt, lam, a_log, th, y, h, lu, ang))
            calls.append((C.byref(cin), C.byref(cout)))
        stream = torch.cuda.current_stream()
        sp = C.c_void_p(stream.cuda_stream)
        call = lambda i: L_.check(lib.m3_scan(calls[i % K][0], calls[i % K][1], sp))
        for i in range(5):
            call(i)
        torch.cuda.synchronize()
        steps = max(12, args.steps // 4)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            call(i)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / steps * 1e3
        for kp in keep:
            assert bool(torch.isfinite(kp[9].float()).all())
        nbytes, flops = scan_algorithmic(B, L, H, P, N, R, 64, s_io=2 if bf16 else 4,
                                         theta_per_token=rot)
        out[name] = {"workload": f"B={B} L={L} H={H} P={P} N={N} R={R} "
                                 f"{'bf16' if bf16 else 'f32'} {'Rotational' if rot else 'Real'}",
                     "us_per_call": round(us, 2), "tokens_per_s": round(B * L / (us * 1e-6), 1),
                     "path": "chunk-parallel" if need else "single pass", "input_sets": K,
                     "achieved_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "mfma_tflops": round(flops / (us * 1e-6) / 1e12, 2),
                     "frac_bf16_mfma_peak": round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}
        del keep, calls, ws
        torch.cuda.empty_cache()
    return out


def bench_decode(torch, lib, L_, args, factored=False):
    """Config 3: 24 layers x one step each per pass over the f32 cache, in
    place, rotating over `sets` input sets.  factored: the same steps through
    m3_step_factored, the cache holding h and the previous token's x and b
    (a second cache format, reported on its own byte count)."""
    dev = "cuda:0"
    d = DECODE
    B, NL, H, P, N, R, K = d["B"], d["layers"], d["H"], d["P"], d["N"], d["R"], d["sets"]
    g = torch.Generator(device=dev).manual_seed(0x4D414D45)
    h = torch.randn(NL, B, H, P, N, device=dev, generator=g) * 0.1
    if factored:
        xp = torch.randn(NL, B, H, P, R, device=dev, generator=g)
        bp = torch.randn(NL, B, H, N, R, device=dev, generator=g) / math.sqrt(N)
    else:
        lu = torch.randn(NL, B, H, P, N, device=dev, generator=g) * 0.1
    ang = (torch.rand(NL, B, H, N // 2, device=dev, generator=g) * 2 - 1) * math.pi
    a_log = torch.rand(NL, H, device=dev, generator=g) * math.log(16.0)
    d_skip = torch.ones(H, device=dev)
    sets = []
    for _ in range(K):
        x = torch.randn(B, H, P, R, device=dev, generator=g)
        b = torch.randn(B, H, N, R, device=dev, generator=g) / math.sqrt(N)
        c = torch.randn(B, H, N, R, device=dev, generator=g) / math.sqrt(N)
        th = torch.rand(B, H, N // 2, device=dev, generator=g) * math.pi
        dt = torch.nn.functional.softplus(torch.randn(B, H, device=dev, generator=g) - 3.0
                                          ).clamp(1e-3, 0.1)
        lam = torch.sigmoid(torch.randn(B, H, device=dev, generator=g))
        sets.append((x, b, c, th, dt, lam))
    y = torch.empty(B, H, P, R, device=dev)
    calls = []
    for k in range(K):
        x, b, c, th, dt, lam = sets[k]
        per_layer = []
        for l in range(NL):
            args_c = L_.StepInputsC(B, H, P, N, R, L_.M3_F32, x.data_ptr(), b.data_ptr(),
                                    c.data_ptr(), dt.data_ptr(), lam.data_ptr(),
                                    a_log[l].data_ptr(), th.data_ptr(), d_skip.data_ptr())
            if factored:
                st = L_.SsmStateFactoredC(h[l].data_ptr(), xp[l].data_ptr(), bp[l].data_ptr(),
                                          ang[l].data_ptr())
            else:
                st = L_.SsmStateC(h[l].data_ptr(), lu[l].data_ptr(), ang[l].data_ptr())
            per_layer.append((args_c, st))
        calls.append(per_layer)
    stream = torch.cuda.current_stream()
    sp = C.c_void_p(stream.cuda_stream)
    fn = lib.m3_step_factored if factored else lib.m3_step
    yp = C.c_void_p(y.data_ptr())
    refs = [[(C.byref(a), C.byref(s)) for a, s in per] for per in calls]

    def step(i):
        for pa, ps in refs[i % K]:
            st = fn(pa, ps, yp, sp)
            if st != 0:
                L_.check(st)

    for i in range(args.decode_warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.decode_steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.decode_steps
    assert torch.isfinite(h).all(), "non-finite decode state"
    nbytes = NL * (decode_factored_algorithmic if factored else decode_algorithmic)(B, H, P, N, R)
    gbs = nbytes / (ms * 1e-3) / 1e9
    # the same passes with all 24 layers in one launch (m3_step_layers)
    tabs = []
    for per in calls:
        ins = (L_.StepInputsC * NL)(*[a for a, _ in per])
        sts = ((L_.SsmStateFactoredC if factored else L_.SsmStateC) * NL)(*[s for _, s in per])
        ysa = (C.c_void_p * NL)(*([y.data_ptr()] * NL))
        tabs.append((ins, sts, ysa))
    fl = lib.m3_step_layers

    def step_one(i):
        ins, sts, ysa = tabs[i % K]
        st = (fl(NL, ins, None, sts, ysa, sp) if factored else fl(NL, ins, sts, None, ysa, sp))
        if st != 0:
            L_.check(st)

    for i in range(args.decode_warmup):
        step_one(i)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.decode_steps):
        step_one(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_one = e0.elapsed_time(e1) / args.decode_steps
    assert torch.isfinite(h).all(), "non-finite decode state"
    if factored:
        return dict(us_per_step=round(ms * 1e3, 2), steps=args.decode_steps, layers=NL,
                    bytes_per_step=nbytes, achieved_GBps=round(gbs, 1),
                    frac_hbm_peak=round(gbs / HBM_PEAK_GBS, 4),
                    us_per_layer=round(ms * 1e3 / NL, 2),
                    us_per_step_one_launch=round(ms_one * 1e3, 2),
                    frac_hbm_peak_one_launch=round(nbytes / (ms_one * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    cache="h f32 [B,H,P,N] + the previous token's x [B,H,P,R] and b [B,H,N,R] "
                          "(m3_step_factored; last_u formed in registers)")
    # a practical stream ceiling beside it: torch's device copy of one layer's
    # h and last_u (the same bytes read and written as one layer's update)
    src = torch.cat([h[0].reshape(-1), lu[0].reshape(-1)])
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    reps = 20
    e0.record(stream)
    for _ in range(reps):
        dst.copy_(src)
    e1.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * 4 / (e0.elapsed_time(e1) / reps * 1e-3) / 1e9
    return dict(us_per_step=round(ms * 1e3, 2), steps=args.decode_steps, layers=NL,
                bytes_per_step=nbytes, achieved_GBps=round(gbs, 1),
                frac_hbm_peak=round(gbs / HBM_PEAK_GBS, 4),
                us_per_layer=round(ms * 1e3 / NL, 2),
                launch="one m3_step launch per layer, 24 per pass",
                us_per_step_one_launch=round(ms_one * 1e3, 2),
                frac_hbm_peak_one_launch=round(nbytes / (ms_one * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                device_copy_GBps=round(copy_gbs, 1))


def cpu_baseline(args):
    """The oracle's f32 restatement of the reference's composed scan on the host
    (OpenMP over batch x head), on config 1's full workload, bf16-rounded inputs."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle
    from cases import baseline_inputs
    s = SCAN
    B = args.cpu_batch
    rng = np.random.default_rng(0x4D414D43)
    inp = baseline_inputs(rng, B, s["L"], s["H"], s["P"], s["N"], 1, theta=True, dtype="bf16")
    run = lambda: oracle.scan_composed_f32(inp["x"], inp["b"], inp["c"], inp["dt"],
                                           inp["a_log"], inp["lam"], inp["theta"],
                                           chunk=s["Q"], want_state=True)
    run()   # warmup
    times = []
    for _ in range(args.cpu_reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    tokens = B * s["L"]
    return {"value": round(tokens / med, 1), "unit": "tokens/s",
            "cores": oracle.num_threads(), "kind": "port", **cpu_model(),
            "sample": (f"config 1 at batch {B} (L=2048, H=12, P=64, N=128, Q=64, Rotational, "
                       f"bf16-rounded inputs, f32 math), composed reference algorithm "
                       f"(oracle/mamba3_oracle.c m3o_scan_composed_f32), 1 warmup + median "
                       f"of {args.cpu_reps}: {med:.3f} s per pass")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--decode-steps", type=int, default=512,
                    help="timed decode steps (BASELINE config 3: 512 consecutive steps)")
    ap.add_argument("--decode-warmup", type=int, default=8)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-4 prefill leg")
    ap.add_argument("--prefill-steps", type=int, default=5)
    ap.add_argument("--no-decode-lm", action="store_true", help="skip the LM decode-step leg")
    ap.add_argument("--decode-lm-steps", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-backward", action="store_true", help="skip the scan backward leg")
    ap.add_argument("--scan-sets", type=int, default=4,
                    help="input/output sets the scan legs rotate over (4 x 152 MB at config 1)")
    ap.add_argument("--cpu-batch", type=int, default=8)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--only", choices=("prefill", "decode_lm", "decode_lm_default", "ingest",
                                       "backward", "other_scans", "decode", "decode_factored"),
                    default=None,
                    help="run one model leg alone and print its object (for kernel traces)")
    ap.add_argument("--scan-only", action="store_true",
                    help="run only the headline scan --steps times (for counter runs)")
    ap.add_argument("--scan-path", choices=("fused", "three"), default="fused",
                    help="the chunk-parallel scan's form for bf16 at rank 1: the fused single "
                         "launch (the library's default) or the three launches")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="copy MIB MiB device to device --steps times and exit (the known-size "
                         "kernel that scales FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every GPU box in this build has one, and the path "
              "has no multi-GPU leg (sharding is designed, not built). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs the MI355X (no ROCm device visible)", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n * 4, "copies": args.steps}), flush=True)
        return
    from mamba3 import _lib as L_
    lib = L_.lib()
    L_.check(lib.m3_debug_scan_options(0 if args.scan_path == "fused" else 1, 0, 0))

    torch.cuda.synchronize()
    if args.only == "backward":
        s = SCAN
        inp = make_scan_inputs(torch, "cuda:0", s["B"], s["L"], s["H"], s["P"], s["N"], s["R"],
                               0x4D414D43)
        torch.cuda.synchronize()
        _pause_for_trace(args)
        print(json.dumps({"backward": bench_backward(torch, lib, L_, args, inp, None)}),
              flush=True)
        return
    if args.only in ("other_scans", "decode", "decode_factored"):
        if args.only == "decode_factored":
            leg = bench_decode(torch, lib, L_, args, factored=True)
        else:
            leg = (bench_other_scans if args.only == "other_scans" else bench_decode)(
                torch, lib, L_, args)
        print(json.dumps({args.only: leg}), flush=True)
        return
    if args.only:
        leg = {"prefill": bench_prefill, "decode_lm": bench_decode_lm,
               "decode_lm_default": bench_decode_lm_default,
               "ingest": bench_ingest}[args.only](torch, args)
        print(json.dumps({args.only: leg}), flush=True)
        return
    if args.scan_only:
        sc = bench_scan(torch, lib, L_, args, chunk_parallel=True)
        print(json.dumps({"scan_us": round(sc["kernel_ms"] * 1e3, 2), "sets": sc["sets"]}),
              flush=True)
        return
    sc = bench_scan(torch, lib, L_, args, chunk_parallel=True)
    sc_res = bench_scan(torch, lib, L_, args, chunk_parallel=True, inp=sc["inp"], sets=1)
    sc1 = bench_scan(torch, lib, L_, args, chunk_parallel=False, inp=sc["inp"])
    s = SCAN
    nbytes, flops = scan_algorithmic(s["B"], s["L"], s["H"], s["P"], s["N"], s["R"], s["Q"])
    k_s = sc["kernel_ms"] * 1e-3
    achieved = nbytes / k_s / 1e9
    tflops = flops / k_s / 1e12
    ms_step = sc["wall_ms"]
    value = sc["tokens"] / (ms_step * 1e-3)

    bwd = None if args.no_backward else bench_backward(torch, lib, L_, args, sc["inp"][0],
                                                       sc["kernel_ms"])
    other = bench_other_scans(torch, lib, L_, args)
    dec = None if args.no_decode else bench_decode(torch, lib, L_, args)
    dec_f = None if args.no_decode else bench_decode(torch, lib, L_, args, factored=True)
    pre = None if args.no_prefill else bench_prefill(torch, args)
    dlm = None if args.no_decode_lm else bench_decode_lm(torch, args)
    dlm_def = None if args.no_decode_lm else bench_decode_lm_default(torch, args)
    cpu = None if args.no_cpu else cpu_baseline(args)

    line = {
        "metric": "SSD scan fwd tokens/s (config 1) + % roofline; decode-step us & HBM GB/s "
                  "at batch 256",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded device RNG, BASELINE.json distributions)",
        "config": {"workload": "mamba3_scan config 1: B=8 L=2048 H=12 P=64 N=128 chunk=64, "
                               "bf16 storage f32 accumulate, Rotational, LearnedTrapezoid, "
                               "SISO, want_state",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": SCAN_TRAFFIC_BYTES,
                     "kernel": "m3_scan: chunk_scan_fused_kernel (one launch a call: each "
                               "128-token segment's state, the look-back for the state "
                               "entering it, its outputs)",
                     "kernel_us": round(sc["kernel_ms"] * 1e3, 2),
                     "input_sets": sc["sets"], "input_MB_total": sc["input_MB"],
                     "kernel_us_resident_inputs": round(sc_res["kernel_ms"] * 1e3, 2),
                     "workspace_MB": round(sc["workspace_bytes"] / 1e6, 1),
                     "algorithmic_bytes": nbytes, "algorithmic_flops": flops,
                     "mfma_busy": SCAN_MFMA_BUSY,
                     "mfma_tflops": round(tflops, 2),
                     "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4)},
        "scan_single_pass_us": round(sc1["kernel_ms"] * 1e3, 2),
        "scan_rotated_sets": sc["sets"],
        "other_scans": other,
        "backward": bwd,
        "decode": dec,
        "decode_factored": dec_f,
        "prefill": pre,
        "decode_lm": dlm,
        "decode_lm_default": dlm_def,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
