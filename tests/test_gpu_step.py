"""GPU parity of the decode step (m3_step through the C ABI) against the oracle:
the reference's step-vs-scan test, the f64 recurrence, the f32 restatement of
mamba3_step, in-place semantics, and BASELINE config 3's shape (f32 state,
rel-L2 <= 1e-5)."""
import math
import zlib

import numpy as np
import pytest
import torch

import oracle
from cases import Case, assert_close, baseline_inputs, rel_l2
from gpu_util import dev, host

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def test_step_matches_the_chunked_scan():
    """tests/ssm.rs:312-380: stepwise mamba3_step (theta, D) vs the scan."""
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan, mamba3_step
    case = Case(2, 9, 2, 3, 4)
    theta = case.theta()
    d_skip = np.array([0.3, -0.2], np.float32)
    x, b, c = case.rank1()
    par = mamba3_scan(ScanInputs(dev(x), dev(b), dev(c), dev(case.dt), dev(case.a_log),
                                 dev(case.lam)).with_theta(dev(theta)).with_skip(dev(d_skip))
                      .with_chunk_size(4))
    state = SsmState.zeros(case.batch, case.heads, case.head_dim, case.state, True, "cuda")
    steps = []
    for t in range(case.seq):
        y, state = mamba3_step(dev(x[:, t]), dev(b[:, t]), dev(c[:, t]), dev(case.dt[:, t]),
                               dev(case.lam[:, t]), dev(case.a_log), dev(theta[:, t]),
                               dev(d_skip), state)
        steps.append(host(y))
    stepwise = np.stack(steps, axis=1)
    assert_close(stepwise, host(par.y), 3e-4, "step vs chunked")
    y64, h64, lu64, a64 = oracle.scan_recurrence_f64(x, b, c, case.dt, case.a_log, case.lam,
                                                     theta, d_skip)
    assert rel_l2(stepwise, y64) <= F32_TOL
    assert rel_l2(host(state.h), h64) <= F32_TOL
    assert rel_l2(host(state.last_u), lu64) <= F32_TOL


STEP_CASES = [
    # B, H, P, N, R, theta, skip, dtype
    (3, 4, 64, 128, 1, True, True, "f32"),
    (2, 3, 64, 64, 1, False, True, "f32"),
    (2, 2, 32, 32, 2, True, False, "f32"),
    (2, 2, 16, 128, 4, True, True, "f32"),
    (1, 2, 8, 6, 1, True, True, "f32"),
    (1, 2, 5, 256, 3, True, True, "f32"),
    (2, 2, 64, 128, 1, True, True, "bf16"),
    (1, 1, 4, 512, 1, True, False, "f32"),
]


@pytest.mark.parametrize("B,H,P,N,R,theta,skip,dtype", STEP_CASES)
def test_step_in_place_against_oracle(B, H, P, N, R, theta, skip, dtype):
    from cases import bf16_round
    from mamba3.ssm import SsmState, mamba3_step_
    rng = np.random.default_rng(zlib.crc32(repr((B, H, P, N, R, theta, skip, dtype)).encode()))
    f = np.float32
    x = rng.standard_normal((B, H, P, R), dtype=f)
    b = (rng.standard_normal((B, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f)
    c = (rng.standard_normal((B, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f)
    th = rng.uniform(0, math.pi, (B, H, N // 2)).astype(f) if theta else None
    if dtype == "bf16":
        x, b, c = bf16_round(x), bf16_round(b), bf16_round(c)
        th = bf16_round(th) if theta else None
    dt = np.clip(np.log1p(np.exp(rng.standard_normal((B, H)) - 3)), 1e-3, 0.1).astype(f)
    lam = (1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(f)
    a_log = rng.uniform(0, math.log(16), H).astype(f)
    d_skip = rng.uniform(-1, 1, H).astype(f) if skip else None
    h = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
    lu = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
    ang = rng.uniform(-math.pi, math.pi, (B, H, N // 2)).astype(f) if theta else None
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    state = SsmState(dev(h), dev(lu), dev(ang) if theta else None)
    y = mamba3_step_(dev(x, tdt), dev(b, tdt), dev(c, tdt), dev(dt), dev(lam), dev(a_log),
                     dev(th, tdt) if theta else None, dev(d_skip), state)
    torch.cuda.synchronize()
    # the f32 restatement of mamba3_step and the f64 recurrence (one token, carried state)
    yo, ho, luo, ango = oracle.step_f32(x, b, c, dt, lam, a_log, th, d_skip, h, lu, ang)
    y64, h64, lu64, a64 = oracle.scan_recurrence_f64(
        x[:, None], b[:, None], c[:, None], dt[:, None], a_log, lam[:, None],
        th[:, None] if theta else None, d_skip, h, lu, ang)
    tol = 1e-2 if dtype == "bf16" else F32_TOL
    assert rel_l2(host(y), y64[:, 0]) <= tol
    assert rel_l2(host(state.h), h64) <= tol
    assert rel_l2(host(state.last_u), lu64) <= tol
    assert rel_l2(host(y), yo) <= tol
    if theta:
        d = host(state.angle) - a64
        d = (d + math.pi) % (2 * math.pi) - math.pi
        assert np.abs(d).max() <= 1e-5


def test_config3_shape_one_layer_many_steps():
    """BASELINE config 3 per-layer shape (batch 256, 24 heads, P64, N128, f32 cache):
    8 consecutive in-place steps on the GPU against 8 oracle steps."""
    from mamba3.ssm import SsmState, mamba3_step_
    B, H, P, N = 256, 24, 64, 128
    rng = np.random.default_rng(3)
    f = np.float32
    h = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
    lu = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
    ang = rng.uniform(-math.pi, math.pi, (B, H, N // 2)).astype(f)
    a_log = rng.uniform(0, math.log(16), H).astype(f)
    d_skip = np.ones(H, f)
    state = SsmState(dev(h), dev(lu), dev(ang))
    ho, luo, ango = h.copy(), lu.copy(), ang.copy()
    for step in range(8):
        x = rng.standard_normal((B, H, P, 1), dtype=f)
        b = (rng.standard_normal((B, H, N, 1), dtype=f) / f(math.sqrt(N))).astype(f)
        c = (rng.standard_normal((B, H, N, 1), dtype=f) / f(math.sqrt(N))).astype(f)
        th = rng.uniform(0, math.pi, (B, H, N // 2)).astype(f)
        dt = np.clip(np.log1p(np.exp(rng.standard_normal((B, H)) - 3)), 1e-3, 0.1).astype(f)
        lam = (1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(f)
        y = mamba3_step_(dev(x), dev(b), dev(c), dev(dt), dev(lam), dev(a_log), dev(th),
                         dev(d_skip), state)
        yo, ho, luo, ango = oracle.step_f32(x, b, c, dt, lam, a_log, th, d_skip, ho, luo, ango)
        assert rel_l2(host(y), yo) <= F32_TOL, step
    assert rel_l2(host(state.h), ho) <= F32_TOL
    assert rel_l2(host(state.last_u), luo) <= F32_TOL


# ------------------------------------------------------------------ factored last_u
def _step_inputs(rng, B, H, P, N, R, theta, dtype):
    f = np.float32
    x = rng.standard_normal((B, H, P, R), dtype=f)
    b = (rng.standard_normal((B, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f)
    c = (rng.standard_normal((B, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f)
    th = rng.uniform(0, math.pi, (B, H, N // 2)).astype(f) if theta else None
    dt = np.clip(np.log1p(np.exp(rng.standard_normal((B, H)) - 3)), 1e-3, 0.1).astype(f)
    lam = (1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(f)
    st = torch.bfloat16 if dtype == "bf16" else torch.float32
    return (dev(x).to(st), dev(b).to(st), dev(c).to(st), dev(dt), dev(lam),
            None if th is None else dev(th).to(st))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,H,P,N,R,theta,skip", [(3, 2, 64, 128, 1, True, True),
                                                   (2, 3, 16, 32, 2, True, False),
                                                   (2, 2, 8, 16, 4, False, True),
                                                   (1, 2, 24, 64, 8, True, True),
                                                   (2, 1, 5, 4, 3, True, False)])
def test_factored_step_equals_the_full_step_bit_for_bit(B, H, P, N, R, theta, skip, dtype):
    """m3_step_factored against m3_step over five steps from the same state
    (last_u zero, the previous token zero): y, h and the angle equal bit for
    bit at every step (the factored form forms last_u from the same f32
    products the full form stored), and x_prev / b_prev hold the last
    token's x and b."""
    from mamba3.ssm import SsmState, SsmStateFactored, mamba3_step_, mamba3_step_factored_
    rng = np.random.default_rng(B * 100 + N + R)
    f = np.float32
    st = torch.bfloat16 if dtype == "bf16" else torch.float32
    h0 = dev((rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f))
    ang = dev(rng.uniform(-math.pi, math.pi, (B, H, N // 2)).astype(f)) if theta else None
    full = SsmState(h0.clone(), torch.zeros_like(h0), None if ang is None else ang.clone())
    fac = SsmStateFactored.zeros(B, H, P, N, R, theta, "cuda", dtype=st)
    fac.h.copy_(h0)
    if theta:
        fac.angle.copy_(ang)
    a_log = dev(rng.uniform(0, math.log(16), H).astype(f))
    d_skip = dev(rng.uniform(0.5, 1.5, H).astype(f)) if skip else None
    for step in range(5):
        x, b, c, dt, lam, th = _step_inputs(rng, B, H, P, N, R, theta, dtype)
        y1 = mamba3_step_(x, b, c, dt, lam, a_log, th, d_skip, full)
        y2 = mamba3_step_factored_(x, b, c, dt, lam, a_log, th, d_skip, fac)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), step
        assert torch.equal(full.h, fac.h), step
        if theta:
            assert torch.equal(full.angle, fac.angle), step
        assert torch.equal(fac.x_prev, x) and torch.equal(fac.b_prev, b), step


def test_factored_step_continues_a_window():
    """A window through m3_scan, then steps: from SsmStateFactored.after_window
    (the scan's h and angle, the window's last x and b) the factored steps
    follow the full steps from the scan's own state (whose last_u the scan
    formed from the same token)."""
    from mamba3.ssm import (ScanInputs, SsmStateFactored, mamba3_scan, mamba3_step_,
                            mamba3_step_factored_)
    rng = np.random.default_rng(5)
    inp = baseline_inputs(rng, 2, 130, 3, 64, 128, 1, theta=True, dtype="bf16")
    st = torch.bfloat16
    si = (ScanInputs(dev(inp["x"]).to(st), dev(inp["b"]).to(st), dev(inp["c"]).to(st),
                     dev(inp["dt"]), dev(inp["a_log"]), dev(inp["lam"]))
          .with_theta(dev(inp["theta"]).to(st)).with_state_output(True))
    out = mamba3_scan(si)
    full = out.state.clone()
    fac = SsmStateFactored.after_window(si, out).clone()
    assert torch.equal(fac.x_prev, si.x[:, -1]) and torch.equal(fac.b_prev, si.b[:, -1])
    for step in range(4):
        x, b, c, dt, lam, th = _step_inputs(rng, 2, 3, 64, 128, 1, True, "bf16")
        y1 = mamba3_step_(x, b, c, dt, lam, si.a_log, th, None, full)
        y2 = mamba3_step_factored_(x, b, c, dt, lam, si.a_log, th, None, fac)
        assert rel_l2(host(y2), host(y1)) <= 1e-5, step
        assert rel_l2(host(fac.h), host(full.h)) <= 1e-5, step


def test_factored_step_config3_shape_against_oracle():
    """The config-3 layer shape (batch 256, 24 heads, P64, N128, bf16 inputs):
    eight factored steps against the f32 restatement of mamba3_step carrying
    the full last_u, from h ~ N(0, 0.1) and last_u zero."""
    from mamba3.ssm import SsmStateFactored, mamba3_step_factored_
    B, H, P, N = 256, 24, 64, 128
    rng = np.random.default_rng(33)
    f = np.float32
    h = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
    ang = rng.uniform(-math.pi, math.pi, (B, H, N // 2)).astype(f)
    a_log = rng.uniform(0, math.log(16), H).astype(f)
    d_skip = np.ones(H, f)
    fac = SsmStateFactored.zeros(B, H, P, N, 1, True, "cuda")
    fac.h.copy_(dev(h))
    fac.angle.copy_(dev(ang))
    ho, luo, ango = h.copy(), np.zeros_like(h), ang.copy()
    for step in range(8):
        x, b, c, dt, lam, th = _step_inputs(rng, B, H, P, N, 1, True, "bf16")
        y = mamba3_step_factored_(x, b, c, dt, lam, dev(a_log), th, dev(d_skip), fac)
        yo, ho, luo, ango = oracle.step_f32(host(x), host(b), host(c), host(dt), host(lam), a_log,
                                            host(th), d_skip, ho, luo, ango)
        assert rel_l2(host(y), yo) <= 1e-2, step
    assert rel_l2(host(fac.h), ho) <= 1e-5


@pytest.mark.parametrize("theta", [True, False])
def test_unfactored_last_u_equals_the_stored_one(theta):
    """SsmStateFactored.to_full (m3_state_unfactor) after three steps gives
    the last_u the full form stored, bit for bit."""
    from mamba3.ssm import SsmState, SsmStateFactored, mamba3_step_, mamba3_step_factored_
    rng = np.random.default_rng(12)
    B, H, P, N, R = 3, 2, 16, 32, 2
    full = SsmState.zeros(B, H, P, N, theta, "cuda")
    fac = SsmStateFactored.zeros(B, H, P, N, R, theta, "cuda", dtype=torch.bfloat16)
    a_log = dev(rng.uniform(0, 2, H).astype(np.float32))
    for _ in range(3):
        x, b, c, dt, lam, th = _step_inputs(rng, B, H, P, N, R, theta, "bf16")
        mamba3_step_(x, b, c, dt, lam, a_log, th, None, full)
        mamba3_step_factored_(x, b, c, dt, lam, a_log, th, None, fac)
    back = fac.to_full()
    torch.cuda.synchronize()
    assert torch.equal(back.last_u, full.last_u)
    assert torch.equal(back.h, full.h)


def test_factored_step_errors():
    import ctypes as C
    from mamba3 import _lib
    from mamba3.error import ArgumentError, UnsupportedError
    from mamba3.ssm import SsmStateFactored, mamba3_step_factored_
    rng = np.random.default_rng(1)
    x, b, c, dt, lam, th = _step_inputs(rng, 2, 2, 8, 12, 1, True, "f32")
    a_log = dev(np.zeros(2, np.float32))
    fac = SsmStateFactored.zeros(2, 2, 8, 12, 1, True, "cuda", dtype=torch.float32)
    with pytest.raises(UnsupportedError, match="factored step needs"):
        mamba3_step_factored_(x, b, c, dt, lam, a_log, th, None, fac)   # d_state 12: 12/4 = 3
    x, b, c, dt, lam, th = _step_inputs(rng, 2, 2, 8, 16, 1, True, "f32")
    fac = SsmStateFactored.zeros(2, 2, 8, 16, 1, True, "cuda", dtype=torch.float32)
    alias = SsmStateFactored(fac.h, x, fac.b_prev, fac.angle)          # x_prev is the input x
    with pytest.raises(ArgumentError, match="must not overlap"):
        mamba3_step_factored_(x, b, c, dt, lam, a_log, th, None, alias)


def test_factored_state_cache_steps_like_the_full_one():
    """StateCache(factored=True): three steps of layer 1 equal the full cache's
    bit for bit (both from zero), and the other layers stay untouched."""
    from mamba3 import StateCache
    rng = np.random.default_rng(9)
    full = StateCache(3, 2, 2, 16, 32, True, "cuda")
    fac = StateCache(3, 2, 2, 16, 32, True, "cuda", factored=True, rank=1,
                     dtype=torch.float32)
    assert fac.num_bytes() < full.num_bytes()
    a_log = dev(rng.uniform(0, 2, 2).astype(np.float32))
    for _ in range(3):
        x, b, c, dt, lam, th = _step_inputs(rng, 2, 2, 16, 32, 1, True, "f32")
        y1 = full.step_layer(1, x, b, c, dt, lam, a_log, th)
        y2 = fac.step_layer(1, x, b, c, dt, lam, a_log, th)
        assert torch.equal(y1, y2)
    assert torch.equal(full.h, fac.h) and torch.equal(full.angle, fac.angle)
    assert not fac.h[0].any() and not fac.h[2].any()


@pytest.mark.parametrize("factored", [False, True])
@pytest.mark.parametrize("layers,B,H,P,N,R", [(3, 4, 3, 64, 128, 1), (26, 2, 2, 8, 16, 2)])
def test_all_layers_in_one_launch_equal_layer_by_layer(layers, B, H, P, N, R, factored):
    """StateCache.step_all (m3_step_layers: every layer's step in one launch,
    split at 24 layers) against step_layer on each layer in turn: y, h,
    last_u (or the previous token) and the angle equal bit for bit over
    three steps."""
    from mamba3 import StateCache
    rng = np.random.default_rng(layers + R)
    g = torch.Generator(device="cuda").manual_seed(4)
    kw = dict(factored=True, rank=R, dtype=torch.float32) if factored else {}
    one = StateCache(layers, B, H, P, N, True, "cuda", init_std=0.1, generator=g, **kw)
    g = torch.Generator(device="cuda").manual_seed(4)
    per = StateCache(layers, B, H, P, N, True, "cuda", init_std=0.1, generator=g, **kw)
    a_logs = [dev(rng.uniform(0, 2, H).astype(np.float32)) for _ in range(layers)]
    skip = dev(np.ones(H, np.float32))
    for _ in range(3):
        inputs = []
        for l in range(layers):
            x, b, c, dt, lam, th = _step_inputs(rng, B, H, P, N, R, True, "f32")
            inputs.append((x, b, c, dt, lam, a_logs[l], th, skip))
        ys = one.step_all(inputs)
        for l in range(layers):
            y = per.step_layer(l, *inputs[l])
            assert torch.equal(ys[l], y), l
    assert torch.equal(one.h, per.h) and torch.equal(one.angle, per.angle)
    if factored:
        assert torch.equal(one.x_prev, per.x_prev) and torch.equal(one.b_prev, per.b_prev)
    else:
        assert torch.equal(one.last_u, per.last_u)


def test_step_layers_rejects_mixed_shapes():
    import ctypes as C
    from mamba3 import _lib
    from mamba3.error import ShapeError
    from mamba3.ssm.scan import _step_args
    rng = np.random.default_rng(2)
    a_log = dev(np.zeros(2, np.float32))
    args = (_lib.StepInputsC * 2)()
    keep = []
    for l, n in enumerate((16, 32)):
        x, b, c, dt, lam, th = _step_inputs(rng, 2, 2, 8, n, 1, True, "f32")
        a, k = _step_args(x, b, c, dt, lam, a_log, th, None)
        args[l] = a
        keep.append(k)
    st = (_lib.SsmStateC * 2)()
    ys = (C.c_void_p * 2)()
    with pytest.raises(ShapeError, match="layer 1's shapes"):
        _lib.check(_lib.lib().m3_step_layers(2, args, st, None, ys, None))


@pytest.mark.parametrize("mismatch", ["dtype", "rank", "batch"])
def test_step_all_checks_every_layer_state_before_any_launch(mismatch):
    """StateCache.step_all on a factored cache (bf16, rank 1) with inputs that
    do not fit it (f32 storage, rank 2, or a larger batch) raises before any
    launch: the kernel would step each layer's slice at the inputs' element
    size and shape, past the slices.  The cache is left untouched."""
    from mamba3 import StateCache
    from mamba3.error import ArgumentError, ShapeError
    rng = np.random.default_rng(7)
    layers, B, H, P, N = 3, 2, 2, 16, 32
    cache = StateCache(layers, B, H, P, N, True, "cuda", init_std=0.1,
                       generator=torch.Generator(device="cuda").manual_seed(1), factored=True,
                       rank=1, dtype=torch.bfloat16)
    before = (cache.h.clone(), cache.x_prev.clone(), cache.b_prev.clone(), cache.angle.clone())
    R = 2 if mismatch == "rank" else 1
    Bi = B + 1 if mismatch == "batch" else B
    dtype = "f32" if mismatch == "dtype" else "bf16"
    a_log = dev(np.zeros(H, np.float32))
    inputs = []
    for _ in range(layers):
        x, b, c, dt, lam, th = _step_inputs(rng, Bi, H, P, N, R, True, dtype)
        inputs.append((x, b, c, dt, lam, a_log, th, None))
    with pytest.raises((ArgumentError, ShapeError)):
        cache.step_all(inputs)
    torch.cuda.synchronize()
    assert torch.equal(cache.h, before[0]) and torch.equal(cache.x_prev, before[1])
    assert torch.equal(cache.b_prev, before[2]) and torch.equal(cache.angle, before[3])


def test_state_cache_layers_are_independent():
    """infer::StateCache: stepping one layer leaves the others untouched."""
    from mamba3 import StateCache
    cache = StateCache(3, 2, 2, 16, 32, True, "cuda", init_std=0.1,
                       generator=torch.Generator(device="cuda").manual_seed(0))
    before = cache.h.clone()
    x = torch.randn(2, 2, 16, 1, device="cuda")
    b = torch.randn(2, 2, 32, 1, device="cuda")
    dt = torch.full((2, 2), 0.05, device="cuda")
    lam = torch.full((2, 2), 0.5, device="cuda")
    a_log = torch.zeros(2, device="cuda")
    th = torch.rand(2, 2, 16, device="cuda")
    cache.step_layer(1, x, b, b, dt, lam, a_log, th)
    cache.advance(1)
    torch.cuda.synchronize()
    assert torch.equal(cache.h[0], before[0]) and torch.equal(cache.h[2], before[2])
    assert not torch.equal(cache.h[1], before[1])
    assert cache.position() == 1
