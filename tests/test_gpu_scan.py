"""GPU parity of the chunked scan (m3_scan / m3_ssd_chunked through the C ABI)
against the CPU oracle on the same seeded inputs.

Bars: f32 rel-L2 <= 1e-5 against the f64 recurrence (and the reference test
metric, worst |a-e|/(1+|e|), at the reference's own tolerances against its
own oracle); bf16 storage rel-L2 <= 1e-2 against the f64 recurrence evaluated
on the same bf16-rounded inputs.
"""
import math
import zlib

import numpy as np
import pytest
import torch

import oracle
from cases import Case, assert_close, baseline_inputs, rel_l2
from gpu_util import dev, host, oracle_scan, run_scan

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 1e-2


def angle_err(a, b):
    d = np.asarray(a, np.float64) - np.asarray(b, np.float64)
    d = (d + math.pi) % (2 * math.pi) - math.pi
    return float(np.max(np.abs(d))) if d.size else 0.0


def test_mfma_lane_layouts():
    import mamba3
    assert mamba3.selftest_mfma() == 0


# ---------------------------------------------------------------- the reference's own cases

@pytest.mark.parametrize("chunk", [1, 2, 3, 4, 8, 16])
def test_chunked_scan_matches_the_recurrence(chunk):
    """tests/ssm.rs:187-205 through m3_ssd_chunked."""
    from mamba3.ssm import ssd_chunked
    case = Case(2, 12, 3, 4, 6)
    a, g, w = case.weights()
    y, st = ssd_chunked(dev(case.x), dev(case.b), dev(case.c), dev(a), dev(g), dev(w), None,
                        chunk, True)
    want_y, want_h = case.reference()
    assert_close(host(y), want_y, 2e-4, f"y (chunk={chunk})")
    assert_close(host(st), want_h, 2e-4, f"final state (chunk={chunk})")
    y64, h64, _, _ = oracle.scan_recurrence_f64(*[v[..., None] for v in (case.x, case.b, case.c)],
                                                case.dt, case.a_log, case.lam)
    assert rel_l2(host(y), y64[..., 0]) <= F32_TOL
    assert rel_l2(host(st), h64) <= F32_TOL


@pytest.mark.parametrize("seq", [1, 5, 7, 13])
def test_chunked_scan_handles_ragged_lengths(seq):
    """tests/ssm.rs:207-220."""
    from mamba3.ssm import ssd_chunked
    case = Case(1, seq, 2, 3, 4)
    a, g, w = case.weights()
    y, st = ssd_chunked(dev(case.x), dev(case.b), dev(case.c), dev(a), dev(g), dev(w), None, 4,
                        True)
    want_y, want_h = case.reference()
    assert_close(host(y), want_y, 2e-4, f"y (seq={seq})")
    assert_close(host(st), want_h, 2e-4, f"state (seq={seq})")


def test_euler_mode_reproduces_mamba2():
    """tests/ssm.rs:222-236: want_state=false returns no state."""
    from mamba3.ssm import ssd_chunked
    case = Case(1, 8, 2, 3, 4)
    case.lam = np.ones_like(case.lam)
    a, g, w = case.weights()
    assert np.abs(w - g).max() <= 1e-6
    y, st = ssd_chunked(dev(case.x), dev(case.b), dev(case.c), dev(a), dev(g), dev(w), None, 4,
                        False)
    assert st is None
    want_y, _ = case.reference()
    assert_close(host(y), want_y, 2e-4, "euler y")


def test_split_windows_match_a_single_pass():
    """tests/ssm.rs:238-310: rotation plus state carried across a cut at t=5."""
    case = Case(2, 12, 2, 3, 4)
    theta = case.theta()
    x, b, c = case.rank1()
    full = dict(x=x, b=b, c=c, dt=case.dt, a_log=case.a_log, lam=case.lam, theta=theta)

    def part(sl):
        return {k: (v[:, sl] if k not in ("a_log",) else v) for k, v in full.items()}

    y_full, h_full, _, _ = run_scan(full, chunk=4)
    y1, h1, l1, a1 = run_scan(part(slice(0, 5)), chunk=4)
    y2, h2, _, _ = run_scan(part(slice(5, 12)), chunk=4, state=(h1, l1, a1))
    assert_close(np.concatenate([y1, y2], axis=1), y_full, 3e-4, "split vs full")
    assert_close(h2, h_full, 3e-4, "split final state")
    y64, h64, _, _ = oracle_scan(full)
    assert rel_l2(y_full, y64) <= F32_TOL and rel_l2(h_full, h64) <= F32_TOL


# ---------------------------------------------------------------- every ScanInputs feature

FEATURE_CASES = [
    # B, T, H, P, N, R, theta, skip, state, dtype
    (2, 37, 3, 16, 32, 1, True, True, True, "f32"),
    (1, 100, 2, 64, 64, 1, False, False, False, "f32"),
    (1, 129, 2, 64, 128, 1, True, True, True, "f32"),
    (2, 70, 2, 24, 16, 2, True, True, True, "f32"),
    (1, 50, 2, 32, 32, 3, True, False, True, "f32"),
    (1, 40, 1, 16, 32, 4, True, True, False, "f32"),
    (2, 37, 3, 16, 32, 1, True, True, True, "bf16"),
    (1, 200, 2, 64, 128, 1, True, True, True, "bf16"),
    (1, 130, 2, 64, 128, 4, True, True, True, "bf16"),
    (1, 65, 1, 128, 256, 1, True, False, True, "bf16"),
    (1, 33, 1, 48, 256, 2, True, True, True, "f32"),
    (1, 9, 2, 3, 6, 1, True, True, True, "f32"),
    (1, 1, 2, 5, 4, 2, True, True, True, "f32"),
    (2, 150, 3, 64, 64, 1, True, True, True, "f32"),
    (1, 77, 2, 64, 128, 2, True, True, True, "f32"),
    (1, 70, 2, 64, 64, 4, True, True, True, "f32"),
    (1, 90, 2, 64, 64, 2, True, True, True, "bf16"),
    (2, 129, 2, 64, 64, 4, False, True, False, "bf16"),
    (1, 64, 3, 64, 128, 1, True, False, True, "bf16"),
]


@pytest.mark.parametrize("chunk_parallel", [True, False], ids=["chunk_parallel", "single_pass"])
@pytest.mark.parametrize("B,T,H,P,N,R,theta,skip,state,dtype", FEATURE_CASES)
def test_scan_features_against_f64(B, T, H, P, N, R, theta, skip, state, dtype, chunk_parallel):
    rng = np.random.default_rng(zlib.crc32(repr((B, T, H, P, N, R, theta, skip, state,
                                                  dtype)).encode()))
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=theta, dtype=dtype,
                          theta_per_head=False, state=state)
    d_skip = rng.uniform(-1, 1, H).astype(np.float32) if skip else None
    st = (inp["h0"], inp["last_u0"], inp.get("angle0")) if state else None
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    y, h, lu, ang = run_scan(inp, dtype=tdt, theta=theta, skip=d_skip, state=st,
                             chunk_parallel=chunk_parallel)
    y64, h64, lu64, ang64 = oracle_scan(inp, theta=theta, skip=d_skip, state=st)
    tol = BF16_TOL if dtype == "bf16" else F32_TOL
    assert rel_l2(y, y64) <= tol, ("y", rel_l2(y, y64))
    assert rel_l2(h, h64) <= tol, ("h", rel_l2(h, h64))
    assert rel_l2(lu, lu64) <= tol, ("last_u", rel_l2(lu, lu64))
    if theta:
        assert angle_err(ang, ang64) <= (1e-4 if dtype == "f32" else 1e-3)


# Shapes beyond the scan kernels' tiles (head_dim over 128, d_state over 256,
# rank over the rows of a chunk): the scan runs token by token on the step
# kernel's generic body, which the reference's mamba3_scan (no shape limits,
# scan.rs:458-618) is held to through the f64 recurrence.
BEYOND_CASES = [
    # B, T, H, P, N, R, theta, skip, state, want_state, dtype
    (2, 40, 2, 160, 64, 1, True, True, True, True, "f32"),      # head_dim 160
    (1, 30, 2, 32, 320, 1, True, False, True, True, "bf16"),    # d_state 320
    (2, 20, 1, 16, 16, 72, True, True, False, True, "f32"),     # rank 72 (32 rows a chunk)
    (1, 25, 2, 16, 16, 80, False, True, True, False, "bf16"),   # rank 80 (64 rows), no state out
    (4, 1, 3, 192, 16, 1, True, True, True, True, "f32"),       # one token, head_dim 192
]


@pytest.mark.parametrize("B,T,H,P,N,R,theta,skip,state,want_state,dtype", BEYOND_CASES)
def test_shapes_beyond_the_scan_kernels_against_f64(B, T, H, P, N, R, theta, skip, state,
                                                     want_state, dtype):
    from mamba3 import _lib
    rng = np.random.default_rng(zlib.crc32(repr(("beyond", B, T, H, P, N, R)).encode()))
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=theta, dtype=dtype,
                          theta_per_head=False, state=state)
    d_skip = rng.uniform(-1, 1, H).astype(np.float32) if skip else None
    st = (inp["h0"], inp["last_u0"], inp.get("angle0")) if state else None
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    before = _lib.lib().m3_launch_count()
    y, h, lu, ang = run_scan(inp, dtype=tdt, theta=theta, skip=d_skip, state=st,
                             want_state=want_state)
    launches = _lib.lib().m3_launch_count() - before
    assert launches >= T, launches           # one step launch per token
    y64, h64, lu64, ang64 = oracle_scan(inp, theta=theta, skip=d_skip, state=st)
    tol = BF16_TOL if dtype == "bf16" else F32_TOL
    print(f"beyond the scan kernels (P {P}, N {N}, R {R}, {dtype}): rel-L2 y {rel_l2(y, y64):.2e}",
          flush=True)
    assert rel_l2(y, y64) <= tol, ("y", rel_l2(y, y64))
    if want_state:
        assert rel_l2(h, h64) <= tol, ("h", rel_l2(h, h64))
        assert rel_l2(lu, lu64) <= tol, ("last_u", rel_l2(lu, lu64))
        if theta:
            assert angle_err(ang, ang64) <= (1e-4 if dtype == "f32" else 1e-3)


def test_gated_scan_beyond_the_scan_kernels():
    """m3_scan_gated at a shape the scan kernels do not cover: the steps, then
    the gate kernel, equal to m3_scan followed by m3_mixer_gate."""
    import ctypes as C
    from mamba3 import _lib
    from mamba3.ssm import ScanInputs, mamba3_scan, mamba3_scan_gated
    B, T, H, P, N, R = 2, 24, 2, 160, 32, 1
    rng = np.random.default_rng(4242)
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=True, dtype="bf16")
    bf = torch.bfloat16
    si = ScanInputs(dev(inp["x"], bf), dev(inp["b"], bf), dev(inp["c"], bf), dev(inp["dt"]),
                    dev(inp["a_log"]), dev(inp["lam"])).with_theta(dev(inp["theta"], bf))
    d = H * P * R
    proj = torch.randn(B, T, d + 40, device="cuda:0").to(bf)
    ref = mamba3_scan(si)
    gated = torch.empty(B, T, d, dtype=bf, device="cuda:0")
    _lib.check(_lib.lib().m3_mixer_gate(B * T, d, ref.y.data_ptr(), proj.data_ptr(), d + 40, None,
                                        C.c_float(1e-5), gated.data_ptr(), None))
    got = mamba3_scan_gated(si, proj)
    torch.cuda.synchronize()
    assert torch.equal(got.y.view(B, T, d), gated)


# chunk_size sets the shortest segment of the chunk-parallel path (the state
# passes between segments; inside one it advances in registers sub-chunk by
# sub-chunk): segments of 1 to 64 sub-chunks, every rank, both storage types
SEGMENT_CASES = [
    # B, T, H, N, R, dtype, chunk_size
    (1, 700, 2, 128, 1, "bf16", 128),
    (1, 700, 2, 128, 1, "bf16", 256),
    (2, 700, 1, 128, 1, "bf16", 448),
    (1, 1000, 2, 64, 1, "bf16", 512),
    (1, 576, 1, 128, 1, "bf16", 4096),
    (1, 513, 2, 128, 2, "bf16", 192),
    (1, 300, 2, 128, 4, "bf16", 256),
    (1, 300, 1, 64, 4, "bf16", 1024),
    (1, 333, 2, 128, 1, "f32", 160),
    (1, 300, 1, 64, 4, "f32", 128),
    (1, 257, 2, 64, 2, "f32", 96),
]


@pytest.mark.parametrize("B,T,H,N,R,dtype,chunk", SEGMENT_CASES)
def test_segments_against_f64(B, T, H, N, R, dtype, chunk):
    import ctypes as C
    from mamba3 import _lib
    rng = np.random.default_rng(zlib.crc32(repr((B, T, H, N, R, dtype, chunk)).encode()))
    P = 64
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=True, dtype=dtype,
                          theta_per_head=False, state=True)
    d_skip = rng.uniform(-1, 1, H).astype(np.float32)
    st = (inp["h0"], inp["last_u0"], inp.get("angle0"))
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    # the chunk-parallel form runs, and longer segments need less workspace
    need = lambda q: _lib.lib().m3_scan_workspace_bytes(C.byref(_lib.ScanInputsC(
        B, T, H, P, N, R, _lib.M3_BF16 if dtype == "bf16" else _lib.M3_F32, 16, 16, 16, 16, 16,
        16, 16, None, None, q, 1, None, 0)))
    assert need(chunk) > 0
    assert need(chunk) <= need(64)
    y, h, lu, ang = run_scan(inp, dtype=tdt, chunk=chunk, skip=d_skip, state=st)
    y64, h64, lu64, ang64 = oracle_scan(inp, skip=d_skip, state=st)
    tol = BF16_TOL if dtype == "bf16" else F32_TOL
    errs = dict(y=rel_l2(y, y64), h=rel_l2(h, h64), last_u=rel_l2(lu, lu64))
    print(f"segments of >= {chunk} tokens, {dtype} R={R} N={N} T={T}: rel-L2 "
          + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()) + f" (bar {tol:g})")
    for k, v in errs.items():
        assert v <= tol, (k, v)
    assert angle_err(ang, ang64) <= (1e-4 if dtype == "f32" else 1e-3)


def test_want_state_false_writes_no_state():
    rng = np.random.default_rng(5)
    inp = baseline_inputs(rng, 1, 20, 1, 16, 32, 1, theta=True)
    y, h, lu, ang = run_scan(inp, want_state=False)
    assert h is None and lu is None
    y64, _, _, _ = oracle_scan(inp)
    assert rel_l2(y, y64) <= F32_TOL


def test_empty_window_passes_the_state_through():
    """seq = 0: empty y; the carried state comes back unchanged."""
    rng = np.random.default_rng(6)
    inp = baseline_inputs(rng, 2, 0, 2, 16, 32, 1, theta=True, state=True)
    st = (inp["h0"], inp["last_u0"], inp["angle0"])
    y, h, lu, ang = run_scan(inp, state=st)
    assert y.shape == (2, 0, 2, 16, 1)
    assert np.array_equal(h, inp["h0"]) and np.array_equal(lu, inp["last_u0"])
    assert np.array_equal(ang, inp["angle0"])


def test_errors_surface_as_reference_errors():
    from mamba3 import ConfigError, UnsupportedError
    rng = np.random.default_rng(8)
    inp = baseline_inputs(rng, 1, 8, 1, 16, 6, 1, theta=True)
    inp["b"] = inp["b"][:, :, :, :5]
    inp["c"] = inp["c"][:, :, :, :5]
    inp["theta"] = inp["theta"][..., :2]
    with pytest.raises(ConfigError, match="even d_state"):
        run_scan(inp)
    # rank 40 is past a chunk's rows but runs token by token on the step
    # kernel; rank 300 is past that kernel's LDS as well
    inp = baseline_inputs(rng, 1, 8, 1, 16, 32, 300, theta=False)
    with pytest.raises(UnsupportedError, match="exceed both"):
        run_scan(inp, dtype=torch.float32, theta=False)


# ---------------------------------------------------------------- BASELINE configs

def test_config0_f32_full_size():
    """B2 L512 H4 P64 N64, f32, Real, LearnedTrapezoid."""
    rng = np.random.default_rng(0x4D414D42)
    inp = baseline_inputs(rng, 2, 512, 4, 64, 64, 1, theta=False)
    y, h, lu, _ = run_scan(inp, theta=False)
    y64, h64, lu64, _ = oracle_scan(inp, theta=False)
    assert rel_l2(y, y64) <= F32_TOL
    assert rel_l2(h, h64) <= F32_TOL
    assert rel_l2(lu, lu64) <= F32_TOL
    # and the composed f32 restatement of the reference algorithm agrees as well
    yc, hc, _, _ = oracle.scan_composed_f32(inp["x"], inp["b"], inp["c"], inp["dt"],
                                            inp["a_log"], inp["lam"], chunk=64)
    assert rel_l2(y, yc) <= 1e-5


def test_config1_bf16_two_heads_full_length():
    """BASELINE config 1 shapes (L2048, P64, N128, bf16, Rotational) on 2 heads."""
    rng = np.random.default_rng(0x4D414D43)
    inp = baseline_inputs(rng, 1, 2048, 2, 64, 128, 1, theta=True, dtype="bf16")
    y, h, lu, ang = run_scan(inp, dtype=torch.bfloat16)
    y64, h64, lu64, ang64 = oracle_scan(inp)
    print(f"config 1, 2 heads, L=2048: rel-L2 y {rel_l2(y, y64):.2e}, h {rel_l2(h, h64):.2e}, "
          f"last_u {rel_l2(lu, lu64):.2e} (bar {BF16_TOL:g})")
    assert rel_l2(y, y64) <= BF16_TOL
    assert rel_l2(h, h64) <= BF16_TOL
    assert angle_err(ang, ang64) <= 1e-3


def test_config2_mimo_bf16_one_head():
    """BASELINE config 2 shapes (MIMO R=4, L4096, P64, N128, bf16) on one head."""
    rng = np.random.default_rng(0x4D414D44)
    inp = baseline_inputs(rng, 1, 4096, 1, 64, 128, 4, theta=True, dtype="bf16")
    y, h, lu, ang = run_scan(inp, dtype=torch.bfloat16)
    y64, h64, lu64, ang64 = oracle_scan(inp)
    assert rel_l2(y, y64) <= BF16_TOL
    assert rel_l2(h, h64) <= BF16_TOL


@pytest.mark.parametrize("B,T,H,R", [(8, 512, 12, 1), (4, 256, 24, 4), (24, 200, 12, 1)],
                         ids=["config1", "config2", "288_sequences"])
def test_chunk_parallel_matches_single_pass_at_benchmark_shapes(B, T, H, R):
    """Configs 1 and 2 at full batch and head count (shorter sequence), and 288
    sequences (past one round of the single pass's one sequence per CU, where
    the chunked launches are chosen again): the chunk-parallel kernels and the
    single-pass kernel agree, and both match the f64 recurrence on two of the
    sequences."""
    import ctypes as C
    from mamba3 import _lib
    from mamba3.ssm import ScanInputs, mamba3_scan
    g = torch.Generator(device="cuda").manual_seed(7 + R + B)
    P, N = 64, 128
    cin = _lib.ScanInputsC(B, T, H, P, N, R, _lib.M3_BF16, 16, 16, 16, 16, 16, 16, 16, None,
                           None, 64, 1, None, 0)
    assert _lib.lib().m3_scan_workspace_bytes(C.byref(cin)) > 0   # the chunked form runs
    x = torch.randn(B, T, H, P, R, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(B, T, H, N, R, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    c = (torch.randn(B, T, H, N, R, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=g) - 3
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    a_log = torch.rand(H, device="cuda", generator=g) * math.log(16)
    th = (torch.rand(B, T, H, N // 2, device="cuda", generator=g) * math.pi).to(torch.bfloat16)
    mk = lambda two: mamba3_scan(ScanInputs(x, b, c, dt, a_log, lam).with_theta(th)
                                 .with_chunk_parallel(two))
    two, one = mk(True), mk(False)
    assert rel_l2(host(two.y), host(one.y)) <= BF16_TOL
    assert rel_l2(host(two.state.h), host(one.state.h)) <= BF16_TOL
    assert rel_l2(host(two.state.last_u), host(one.state.last_u)) <= BF16_TOL
    assert angle_err(host(two.state.angle), host(one.state.angle)) <= 1e-3
    for bb, hh in ((0, 0), (B - 1, H - 1)):
        sl = lambda t: host(t[bb:bb + 1, :, hh:hh + 1])
        y64, h64, _, _ = oracle.scan_recurrence_f64(
            sl(x), sl(b), sl(c), sl(dt), host(a_log[hh:hh + 1]), sl(lam), sl(th))
        assert rel_l2(host(two.y[bb:bb + 1, :, hh:hh + 1]), y64) <= BF16_TOL
        assert rel_l2(host(two.state.h[bb:bb + 1, hh:hh + 1]), h64) <= BF16_TOL


def test_config1_full_size_split_window_property():
    """Full config 1 (B8 L2048 H12): scan(x) == scan(x[:1024]) then scan(x[1024:])
    carrying the state -- a size-independent check at the benchmark shape."""
    g = torch.Generator(device="cuda").manual_seed(1)
    B, T, H, P, N = 8, 2048, 12, 64, 128
    from mamba3.ssm import ScanInputs, mamba3_scan
    x = torch.randn(B, T, H, P, 1, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(B, T, H, N, 1, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    c = (torch.randn(B, T, H, N, 1, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=g) - 3
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    a_log = torch.rand(H, device="cuda", generator=g) * math.log(16)
    th = (torch.rand(1, 1, H, N // 2, device="cuda", generator=g) * math.pi).expand(
        B, T, H, N // 2).contiguous().to(torch.bfloat16)
    full = mamba3_scan(ScanInputs(x, b, c, dt, a_log, lam).with_theta(th))
    cut = 1000
    s = slice(0, cut)
    first = mamba3_scan(ScanInputs(x[:, s], b[:, s], c[:, s], dt[:, s], a_log, lam[:, s])
                        .with_theta(th[:, s]))
    s = slice(cut, T)
    second = mamba3_scan(ScanInputs(x[:, s], b[:, s], c[:, s], dt[:, s], a_log, lam[:, s])
                         .with_theta(th[:, s]).with_state(first.state))
    joined = torch.cat([first.y, second.y], dim=1).float()
    ey, eh = rel_l2(host(joined), host(full.y)), rel_l2(host(second.state.h), host(full.state.h))
    print(f"config 1 full size, split at {cut}: rel-L2 y {ey:.2e}, h {eh:.2e} (bar {BF16_TOL:g})")
    assert ey <= BF16_TOL
    assert eh <= BF16_TOL
    assert torch.isfinite(full.y.float()).all()


def test_config1_full_size_every_sequence_against_f64():
    """Full config 1 (B8 L2048 H12 P64 N128, bf16, rotational with per-token
    theta, LearnedTrapezoid, skip D) through the benchmark's chunk-parallel
    plan, every one of the 96 sequences against the f64 recurrence: y, h,
    last_u and the angle.  Margins are printed."""
    from mamba3.ssm import ScanInputs, mamba3_scan
    g = torch.Generator(device="cuda").manual_seed(11)
    B, T, H, P, N = 8, 2048, 12, 64, 128
    x = torch.randn(B, T, H, P, 1, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(B, T, H, N, 1, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    c = (torch.randn(B, T, H, N, 1, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=g) - 3
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    a_log = torch.rand(H, device="cuda", generator=g) * math.log(16)
    th = (torch.rand(B, T, H, N // 2, device="cuda", generator=g) * math.pi).to(torch.bfloat16)
    d_skip = torch.rand(H, device="cuda", generator=g) * 2 - 1
    out = mamba3_scan(ScanInputs(x, b, c, dt, a_log, lam).with_theta(th).with_skip(d_skip)
                      .with_state_output(True))
    torch.cuda.synchronize()
    hx, hb, hc, hdt, hlam, hth = (host(t) for t in (x, b, c, dt, lam, th))
    hy, hh, hlu, hang = (host(t) for t in (out.y, out.state.h, out.state.last_u, out.state.angle))
    worst = np.zeros(4)
    for bb in range(B):
        sl = lambda a: a[bb:bb + 1]
        y64, h64, lu64, a64 = oracle.scan_recurrence_f64(sl(hx), sl(hb), sl(hc), sl(hdt),
                                                         host(a_log), sl(hlam), sl(hth),
                                                         d_skip=host(d_skip))
        e = np.array([rel_l2(sl(hy), y64), rel_l2(sl(hh), h64), rel_l2(sl(hlu), lu64),
                      angle_err(sl(hang), a64)])
        worst = np.maximum(worst, e)
    print(f"config 1 full size, all {B * H} sequences against f64: worst rel-L2 y {worst[0]:.2e}, "
          f"h {worst[1]:.2e}, last_u {worst[2]:.2e} (bar {BF16_TOL:g}); angle {worst[3]:.1e}",
          flush=True)
    assert max(worst[:3]) <= BF16_TOL
    assert worst[3] <= 1e-3


# ------------------------------------------------------- the fused single launch
def _scan_options(path, lookback_mode=0, spin=0):
    from mamba3 import _lib
    _lib.check(_lib.lib().m3_debug_scan_options(path, lookback_mode, spin))


def _fused_inputs(seed, B, T, H, N, theta=True, state=True, skip=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    P = 64
    x = torch.randn(B, T, H, P, 1, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(B, T, H, N, 1, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    c = (torch.randn(B, T, H, N, 1, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=g) - 3
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    a_log = torch.rand(H, device="cuda", generator=g) * math.log(16)
    th = ((torch.rand(B, T, H, N // 2, device="cuda", generator=g) * math.pi).to(torch.bfloat16)
          if theta else None)
    d = (torch.rand(H, device="cuda", generator=g) * 2 - 1) if skip else None
    st = None
    if state:
        st = (0.1 * torch.randn(B, H, P, N, device="cuda", generator=g),
              0.1 * torch.randn(B, H, P, N, device="cuda", generator=g),
              (torch.rand(B, H, N // 2, device="cuda", generator=g) - 0.5) * 6 if theta else None)
    return x, b, c, dt, a_log, lam, th, d, st


def _run_inputs(t):
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan
    x, b, c, dt, a_log, lam, th, d, st = t
    si = ScanInputs(x, b, c, dt, a_log, lam)
    if th is not None:
        si = si.with_theta(th)
    if d is not None:
        si = si.with_skip(d)
    if st is not None:
        si = si.with_state(SsmState(*st))
    out = mamba3_scan(si.with_state_output(True).with_chunk_parallel(True))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("B,T,H,N,theta,state,skip", [
    (8, 2048, 12, 128, True, False, True),   # config 1: segments of 128 tokens, 16 a sequence
    (2, 700, 3, 128, True, True, True),      # ragged end, carried state
    (1, 64, 4, 128, True, True, False),      # one sub-chunk: one segment
    (1, 130, 5, 128, True, False, False),    # a last segment of one sub-chunk
    (2, 1000, 3, 64, True, True, True),      # d_state 64
    (2, 513, 4, 128, False, True, True),     # real dynamics
])
def test_fused_launch_matches_the_three_launches_and_f64(B, T, H, N, theta, state, skip):
    """The fused single launch (default for bf16 at rank 1) against the three
    launches (m3_debug_scan_options path 1) on the same inputs, and both
    against the f64 recurrence on two sequences; the fused launch's outputs
    repeat bit for bit."""
    t = _fused_inputs(B * 1000 + T, B, T, H, N, theta, state, skip)
    fused = _run_inputs(t)
    again = _run_inputs(t)
    _scan_options(1)
    try:
        three = _run_inputs(t)
    finally:
        _scan_options(0)
    assert torch.equal(fused.y, again.y) and torch.equal(fused.state.h, again.state.h)
    assert torch.equal(fused.state.last_u, again.state.last_u)
    e = [_device_rel_l2(fused.y, three.y), _device_rel_l2(fused.state.h, three.state.h),
         _device_rel_l2(fused.state.last_u, three.state.last_u)]
    x, b, c, dt, a_log, lam, th, d, st = t
    worst = 0.0
    for bb, hh in ((0, 0), (B - 1, H - 1)):
        sl = lambda v: host(v[bb:bb + 1, :, hh:hh + 1])
        y64, h64, lu64, a64 = oracle.scan_recurrence_f64(
            sl(x), sl(b), sl(c), sl(dt), host(a_log[hh:hh + 1]), sl(lam),
            None if th is None else sl(th), None if d is None else host(d[hh:hh + 1]),
            None if st is None else host(st[0][bb:bb + 1, hh:hh + 1]),
            None if st is None else host(st[1][bb:bb + 1, hh:hh + 1]),
            None if (st is None or st[2] is None) else host(st[2][bb:bb + 1, hh:hh + 1]))
        ys = host(fused.y[bb:bb + 1, :, hh:hh + 1])
        worst = max(worst, rel_l2(ys, y64), rel_l2(host(fused.state.h[bb:bb + 1, hh:hh + 1]), h64))
        if th is not None:
            assert angle_err(host(fused.state.angle[bb:bb + 1, hh:hh + 1]), a64) <= 1e-3
    print(f"fused vs three launches B{B} T{T} H{H} N{N}: rel-L2 y {e[0]:.2e} h {e[1]:.2e} "
          f"last_u {e[2]:.2e}; fused vs f64 worst {worst:.2e} (bar {BF16_TOL:g})", flush=True)
    assert max(e) <= BF16_TOL
    assert worst <= BF16_TOL


def test_fused_lookback_give_up_surfaces_as_nan():
    """A segment whose look-back gives up (forced from the host: every segment
    after a sequence's first gives up at once) takes NaN for the state
    entering it: its outputs, those of every later segment and the boundary
    state come out NaN, never stale; the first segment's outputs (the first
    128 tokens) are the normal run's; every kernel exits, and the next call
    is normal again."""
    B, T, H, N = 2, 700, 3, 128
    t = _fused_inputs(5, B, T, H, N)
    normal = _run_inputs(t)
    _scan_options(0, 1, 0)
    try:
        gave = _run_inputs(t)
    finally:
        _scan_options(0)
    after = _run_inputs(t)
    assert torch.equal(after.y, normal.y) and torch.equal(after.state.h, normal.state.h)
    assert torch.equal(gave.y[:, :128], normal.y[:, :128])
    assert torch.isnan(gave.y[:, 128:].float()).all()
    assert torch.isnan(gave.state.h).all() and torch.isnan(gave.state.angle).all()
    assert torch.isfinite(normal.y.float()).all()


def _device_rel_l2(a, b):
    """rel-L2 of two device tensors, accumulated in f64 on the device."""
    a, b = a.double(), b.double()
    return float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))


def test_config2_full_size_split_window_and_f64():
    """Full config 2 (B4 L4096 H24 P64 N128, MIMO R4, bf16, rotational, per-token
    theta): scan(x) == scan(x[:2000]) then scan(x[2000:]) carrying the state
    (tests/ssm.rs:238-310 at the benchmark shape; the cut is not a chunk or
    segment multiple), and two whole sequences (all 24 heads) against the f64
    recurrence.  Margins are printed."""
    from mamba3.ssm import ScanInputs, mamba3_scan
    g = torch.Generator(device="cuda").manual_seed(2)
    B, T, H, P, N, R = 4, 4096, 24, 64, 128, 4
    x = torch.randn(B, T, H, P, R, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(B, T, H, N, R, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    c = (torch.randn(B, T, H, N, R, device="cuda", generator=g) / math.sqrt(N)).to(torch.bfloat16)
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=g) - 3
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    a_log = torch.rand(H, device="cuda", generator=g) * math.log(16)
    th = (torch.rand(B, T, H, N // 2, device="cuda", generator=g) * math.pi).to(torch.bfloat16)
    full = mamba3_scan(ScanInputs(x, b, c, dt, a_log, lam).with_theta(th))
    cut = 2000
    s = slice(0, cut)
    first = mamba3_scan(ScanInputs(x[:, s], b[:, s], c[:, s], dt[:, s], a_log, lam[:, s])
                        .with_theta(th[:, s]))
    s = slice(cut, T)
    second = mamba3_scan(ScanInputs(x[:, s], b[:, s], c[:, s], dt[:, s], a_log, lam[:, s])
                         .with_theta(th[:, s]).with_state(first.state))
    torch.cuda.synchronize()
    ey = _device_rel_l2(torch.cat([first.y, second.y], dim=1), full.y)
    eh = _device_rel_l2(second.state.h, full.state.h)
    eu = _device_rel_l2(second.state.last_u, full.state.last_u)
    ea = angle_err(host(second.state.angle), host(full.state.angle))
    print(f"config 2 full size, split at {cut}: rel-L2 y {ey:.2e}, h {eh:.2e}, last_u {eu:.2e}, "
          f"angle {ea:.1e} (bar {BF16_TOL:g})", flush=True)
    assert ey <= BF16_TOL and eh <= BF16_TOL and eu <= BF16_TOL and ea <= 1e-3
    assert torch.isfinite(full.y.float()).all()
    for bb in (0, B - 1):
        sl = lambda t: host(t[bb:bb + 1])
        y64, h64, lu64, _ = oracle.scan_recurrence_f64(sl(x), sl(b), sl(c), sl(dt), host(a_log),
                                                       sl(lam), sl(th))
        e = (rel_l2(sl(full.y), y64), rel_l2(sl(full.state.h), h64),
             rel_l2(sl(full.state.last_u), lu64))
        print(f"config 2 full size, sequence {bb} (24 heads, L=4096) against f64: rel-L2 y "
              f"{e[0]:.2e}, h {e[1]:.2e}, last_u {e[2]:.2e} (bar {BF16_TOL:g})", flush=True)
        assert max(e) <= BF16_TOL


# ------------------------------------------------------------------ gated scan
@pytest.mark.parametrize("B,T,H,N,R,theta,skip,state,chunk_parallel,extra", [
    (2, 300, 3, 128, 1, True, True, True, True, 72),     # chunk-parallel, rank 1: the gate in its last kernel
    # a z row of width 4 mod 8 (a fixed-lambda in_proj row): the fused gate
    # and the composed gate's scalar kernel
    (2, 300, 3, 128, 1, True, True, True, True, 68),
    (8, 2048, 12, 128, 1, True, True, False, True, 72),  # config 1's shape: segments of several sub-chunks
    (1, 700, 2, 64, 1, True, False, False, True, 72),    # d_state 64, ragged end
    (2, 256, 2, 128, 1, False, True, False, True, 72),   # real dynamics
    (1, 300, 2, 128, 2, True, True, False, True, 72),    # MIMO chunk-parallel: the gate as a second launch
    (2, 300, 3, 128, 1, True, True, True, False, 72),    # single pass: a second launch
])
def test_gated_scan_equals_scan_then_gate(B, T, H, N, R, theta, skip, state, chunk_parallel, extra):
    """m3_scan_gated gives m3_scan's y through m3_mixer_gate (no post-gate
    norm) bit for bit, with the same output state, on every path."""
    import ctypes as C
    from mamba3 import _lib
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan, mamba3_scan_gated
    P = 64
    rng = np.random.default_rng(zlib.crc32(repr((B, T, H, N, R)).encode()))
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=theta, dtype="bf16", state=state)
    bf = torch.bfloat16
    si = ScanInputs(dev(inp["x"], bf), dev(inp["b"], bf), dev(inp["c"], bf), dev(inp["dt"]),
                    dev(inp["a_log"]), dev(inp["lam"]))
    if theta:
        si = si.with_theta(dev(inp["theta"], bf))
    if skip:
        si = si.with_skip(dev(rng.uniform(-1, 1, H).astype(np.float32)))
    if state:
        si = si.with_state(SsmState(dev(inp["h0"]), dev(inp["last_u0"]),
                                    dev(inp["angle0"]) if theta else None))
    si = si.with_state_output(True).with_chunk_parallel(chunk_parallel)
    d = H * P * R
    width = d + extra                    # z leads a wider row, as in the in_proj output
    proj = torch.randn(B, T, width, device="cuda:0").to(bf)
    ref = mamba3_scan(si)
    gated = torch.empty(B, T, d, dtype=bf, device="cuda:0")
    _lib.check(_lib.lib().m3_mixer_gate(B * T, d, ref.y.data_ptr(), proj.data_ptr(), width, None,
                                        C.c_float(1e-5), gated.data_ptr(), None))
    got = mamba3_scan_gated(si, proj)
    torch.cuda.synchronize()
    assert torch.equal(got.y.view(B, T, d), gated)
    assert torch.equal(got.state.h, ref.state.h) and torch.equal(got.state.last_u, ref.state.last_u)
    if theta:
        assert torch.equal(got.state.angle, ref.state.angle)


@pytest.mark.parametrize("B,T,H,N,R,state,chunk_parallel,path,extra", [
    (2, 300, 3, 128, 1, True, True, 0, 72),      # the fused single launch, gated
    (16, 512, 12, 128, 1, True, True, 1, 4632 - 768),   # config 4's row, the three launches
    (1, 700, 2, 64, 1, False, True, 1, 72),      # d_state 64, ragged end
    (1, 300, 2, 128, 2, True, True, 1, 72),      # MIMO rank 2
    (2, 300, 2, 128, 4, True, True, 1, 72),      # MIMO rank 4 (its own bf16 kernels)
    (2, 300, 3, 128, 1, True, False, 0, 72),     # single pass
    (2, 300, 3, 128, 1, True, True, 0, 68),      # theta not 16-byte aligned: made contiguous
])
def test_gated_scan_reads_theta_in_place(B, T, H, N, R, state, chunk_parallel, path, extra):
    """theta as a view of the in_proj rows' last H*N/2 columns (read by the
    kernels at the row stride) gives the same bytes as a contiguous copy:
    y and the whole output state, on every path that takes it.  A row whose
    theta pieces are not 16-byte aligned is copied first (one call with the
    stride, refused before any launch, then one without)."""
    from mamba3 import _lib
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan_gated
    P = 64
    rng = np.random.default_rng(zlib.crc32(repr(("in place", B, T, H, N, R)).encode()))
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=True, dtype="bf16", state=state)
    bf = torch.bfloat16
    d, NH = H * P * R, N // 2
    width = d + extra + H * NH           # [z | ... | theta], theta last as in the in_proj row
    proj = torch.randn(B, T, width, device="cuda:0").to(bf)
    proj[..., width - H * NH:] = dev(inp["theta"], bf).view(B, T, H * NH)
    view = proj[..., width - H * NH:].unflatten(-1, (H, NH))
    assert not view.is_contiguous()

    def run(theta):
        si = ScanInputs(dev(inp["x"], bf), dev(inp["b"], bf), dev(inp["c"], bf), dev(inp["dt"]),
                        dev(inp["a_log"]), dev(inp["lam"])).with_theta(theta)
        si = si.with_skip(dev(np.linspace(-1, 1, H).astype(np.float32)))
        if state:
            si = si.with_state(SsmState(dev(inp["h0"]), dev(inp["last_u0"]), dev(inp["angle0"])))
        return mamba3_scan_gated(si.with_state_output(True).with_chunk_parallel(chunk_parallel), proj)

    L = _lib.lib()
    orig, strides = L.m3_scan_gated, []

    def spy(*a):
        strides.append(a[4])
        return orig(*a)

    _lib.check(L.m3_debug_scan_options(path, 0, 0))
    L.m3_scan_gated = spy
    try:
        ref = run(view.contiguous())
        got = run(view)
    finally:
        L.m3_scan_gated = orig
        _lib.check(L.m3_debug_scan_options(0, 0, 0))
    torch.cuda.synchronize()
    aligned = (width - H * NH) * 2 % 16 == 0
    assert strides == ([0, width] if aligned else [0, width, 0])
    assert torch.equal(got.y, ref.y)
    for f in ("h", "last_u", "angle"):
        assert torch.equal(getattr(got.state, f), getattr(ref.state, f)), f
