"""f16 storage (the reference's FloatElem for half::f16, src/backend.rs:86-98)
through the C ABI.  An f16 call runs the f32 kernels on widened copies of its
f16 tensors and narrows its f16 outputs back, so each case checks that
contract exactly: the f16 call equals the f32 call on the same (f16-valued)
inputs with its f16 outputs rounded to f16, bit for bit (the backward to f32
rounding, since its LDS atomics make two calls agree only that far), and one
scan case is held against the f64 recurrence on the f16 inputs."""
import math
import zlib

import numpy as np
import pytest
import torch

import oracle
from cases import baseline_inputs, rel_l2
from gpu_util import dev, host

pytestmark = pytest.mark.gpu

H16, F32 = torch.float16, torch.float32


def _f16(a):
    """numpy f32 -> device f16 tensor (rounded to nearest even)."""
    return None if a is None else dev(a).to(H16)


@pytest.mark.parametrize("B,T,H,P,N,R,theta,skip,state,chunk_parallel", [
    (2, 300, 3, 64, 128, 1, True, True, True, True),     # chunk-parallel (three launches)
    (1, 200, 2, 64, 64, 2, True, False, True, False),    # single pass, rank 2
    (1, 100, 2, 32, 16, 1, False, True, False, True),    # generic kernel
    (1, 30, 2, 160, 32, 1, True, True, True, True),      # head_dim 160: token by token
])
def test_f16_scan_is_the_f32_scan_rounded(B, T, H, P, N, R, theta, skip, state, chunk_parallel):
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan
    rng = np.random.default_rng(zlib.crc32(repr(("f16", B, T, H, P, N, R)).encode()))
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=theta, dtype="f32", state=state)
    x16, b16, c16 = _f16(inp["x"]), _f16(inp["b"]), _f16(inp["c"])
    th16 = _f16(inp["theta"]) if theta else None
    d_skip = dev(rng.uniform(-1, 1, H).astype(np.float32)) if skip else None

    def run(x, b, c, th):
        si = ScanInputs(x, b, c, dev(inp["dt"]), dev(inp["a_log"]), dev(inp["lam"]))
        if th is not None:
            si = si.with_theta(th)
        if d_skip is not None:
            si = si.with_skip(d_skip)
        if state:
            si = si.with_state(SsmState(dev(inp["h0"]), dev(inp["last_u0"]),
                                        dev(inp["angle0"]) if theta else None))
        return mamba3_scan(si.with_state_output(True).with_chunk_parallel(chunk_parallel))

    got = run(x16, b16, c16, th16)
    ref = run(x16.float(), b16.float(), c16.float(), None if th16 is None else th16.float())
    torch.cuda.synchronize()
    assert got.y.dtype == H16
    assert torch.equal(got.y, ref.y.to(H16))
    assert torch.equal(got.state.h, ref.state.h) and torch.equal(got.state.last_u, ref.state.last_u)
    if theta:
        assert torch.equal(got.state.angle, ref.state.angle)
    if chunk_parallel and R == 1:
        # against the f64 recurrence on the f16 inputs: the f16 rounding of y
        # (2^-11 relative at most) is the error
        y64, h64, _, _ = oracle.scan_recurrence_f64(
            host(x16), host(b16), host(c16), inp["dt"], inp["a_log"], inp["lam"],
            host(th16) if theta else None, host(d_skip) if skip else None,
            inp["h0"] if state else None, inp["last_u0"] if state else None,
            inp["angle0"] if (state and theta) else None)
        e = rel_l2(host(got.y), y64)
        print(f"f16 scan against f64: rel-L2 y {e:.2e}, h {rel_l2(host(got.state.h), h64):.2e}",
              flush=True)
        assert e <= 1e-3
        assert rel_l2(host(got.state.h), h64) <= 1e-4


def test_f16_ssd_chunked_is_the_f32_form_rounded():
    from mamba3.ssm import ssd_chunked
    rng = np.random.default_rng(161)
    B, T, H, P, N = 2, 150, 2, 32, 16
    f = np.float32
    x = _f16(rng.standard_normal((B, T, H, P), dtype=f))
    b = _f16((rng.standard_normal((B, T, H, N), dtype=f) / f(4)).astype(f))
    c = _f16((rng.standard_normal((B, T, H, N), dtype=f) / f(4)).astype(f))
    a = dev(-rng.uniform(0.001, 0.1, (B, T, H)).astype(f))
    g = dev(rng.uniform(0.1, 1, (B, T, H)).astype(f))
    w = dev(rng.uniform(0.1, 1, (B, T, H)).astype(f))
    s0 = dev((rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f))
    y16, h16 = ssd_chunked(x, b, c, a, g, w, s0, chunk_size=32)
    y32, h32 = ssd_chunked(x.float(), b.float(), c.float(), a, g, w, s0, chunk_size=32)
    torch.cuda.synchronize()
    assert y16.dtype == H16
    assert torch.equal(y16, y32.to(H16)) and torch.equal(h16, h32)


@pytest.mark.parametrize("B,H,P,N,R,theta,skip", [(2, 2, 64, 128, 1, True, True),
                                                   (2, 3, 16, 32, 2, True, False),
                                                   (1, 2, 8, 16, 4, False, True)])
def test_f16_steps_are_the_f32_steps_rounded(B, H, P, N, R, theta, skip):
    """Full and factored caches, four steps each from the same state: y
    rounded to f16 bit for bit, h and the angle equal, the factored cache's
    x_prev / b_prev the last token's f16 x and b, and its unfactored last_u
    the f32 form's."""
    from mamba3.ssm import SsmState, SsmStateFactored, mamba3_step_, mamba3_step_factored_
    rng = np.random.default_rng(B * 1000 + N * 10 + R)
    f = np.float32
    h0 = dev((rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f))
    lu0 = dev((rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f))
    ang = dev(rng.uniform(-math.pi, math.pi, (B, H, N // 2)).astype(f)) if theta else None
    clone = lambda t: None if t is None else t.clone()
    full16, full32 = (SsmState(h0.clone(), lu0.clone(), clone(ang)) for _ in range(2))
    fac16 = SsmStateFactored.zeros(B, H, P, N, R, theta, "cuda", dtype=H16)
    fac32 = SsmStateFactored.zeros(B, H, P, N, R, theta, "cuda", dtype=F32)
    for fac in (fac16, fac32):
        fac.h.copy_(h0)
        if theta:
            fac.angle.copy_(ang)
    a_log = dev(rng.uniform(0, math.log(16), H).astype(f))
    d_skip = dev(rng.uniform(0.5, 1.5, H).astype(f)) if skip else None
    for step in range(4):
        x = _f16(rng.standard_normal((B, H, P, R), dtype=f))
        b = _f16((rng.standard_normal((B, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f))
        c = _f16((rng.standard_normal((B, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f))
        th = _f16(rng.uniform(0, math.pi, (B, H, N // 2)).astype(f)) if theta else None
        dt = dev(np.clip(np.log1p(np.exp(rng.standard_normal((B, H)) - 3)), 1e-3, 0.1).astype(f))
        lam = dev((1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(f))
        up = lambda t: None if t is None else t.float()
        y16 = mamba3_step_(x, b, c, dt, lam, a_log, th, d_skip, full16)
        y32 = mamba3_step_(up(x), up(b), up(c), dt, lam, a_log, up(th), d_skip, full32)
        z16 = mamba3_step_factored_(x, b, c, dt, lam, a_log, th, d_skip, fac16)
        z32 = mamba3_step_factored_(up(x), up(b), up(c), dt, lam, a_log, up(th), d_skip, fac32)
        torch.cuda.synchronize()
        assert y16.dtype == H16 and z16.dtype == H16
        assert torch.equal(y16, y32.to(H16)) and torch.equal(z16, z32.to(H16)), step
        assert torch.equal(full16.h, full32.h) and torch.equal(full16.last_u, full32.last_u), step
        assert torch.equal(fac16.h, fac32.h), step
        if theta:
            assert torch.equal(full16.angle, full32.angle) and torch.equal(fac16.angle, fac32.angle)
        assert torch.equal(fac16.x_prev, x) and torch.equal(fac16.b_prev, b), step
    assert torch.equal(fac16.to_full().last_u, fac32.to_full().last_u)


@pytest.mark.parametrize("theta,skip,state,P,N,R", [(True, True, True, 64, 64, 1),
                                                   (False, False, False, 64, 64, 1),
                                                   (True, True, True, 48, 32, 2)])   # token walk
def test_f16_backward_is_the_f32_backward_rounded(theta, skip, state, P, N, R):
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan_backward
    B, T, H = 1, 160, 2
    rng = np.random.default_rng(1616 + theta + 2 * state + P)
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=theta, dtype="f32", state=state)
    x16, b16, c16 = _f16(inp["x"]), _f16(inp["b"]), _f16(inp["c"])
    th16 = _f16(inp["theta"]) if theta else None
    dy16 = _f16(rng.standard_normal((B, T, H, P, R)).astype(np.float32))
    d_skip = dev(rng.uniform(-1, 1, H).astype(np.float32)) if skip else None
    dh = dev((rng.standard_normal((B, H, P, N)) * 0.1).astype(np.float32)) if state else None

    def run(x, b, c, th, dy):
        si = ScanInputs(x, b, c, dev(inp["dt"]), dev(inp["a_log"]), dev(inp["lam"]))
        if th is not None:
            si = si.with_theta(th)
        if d_skip is not None:
            si = si.with_skip(d_skip)
        if state:
            si = si.with_state(SsmState(dev(inp["h0"]), dev(inp["last_u0"]),
                                        dev(inp["angle0"]) if theta else None))
        return mamba3_scan_backward(si, dy, dh)

    g16 = run(x16, b16, c16, th16, dy16)
    up = lambda t: None if t is None else t.float()
    g32 = run(up(x16), up(b16), up(c16), up(th16), up(dy16))
    torch.cuda.synchronize()
    for name in ("x", "b", "c") + (("theta",) if theta else ()):
        a, r = getattr(g16, name), getattr(g32, name)
        assert a.dtype == H16, name
        # the f32 grads rounded to f16; two backward calls agree to f32 rounding
        assert rel_l2(host(a), host(r.to(H16))) <= 1e-5, name
    for name in ("dt", "lam", "a_log"):
        assert rel_l2(host(getattr(g16, name)), host(getattr(g32, name))) <= 1e-5, name


def test_f16_empty_window_passes_the_state_through():
    """seq = 0 with f16 storage: nothing is widened, the state passes through."""
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan
    B, H, P, N = 2, 3, 64, 64
    g = torch.Generator(device="cuda:0").manual_seed(3)
    x = torch.empty(B, 0, H, P, 1, dtype=H16, device="cuda:0")
    b = torch.empty(B, 0, H, N, 1, dtype=H16, device="cuda:0")
    st = SsmState(torch.randn(B, H, P, N, device="cuda:0", generator=g),
                  torch.randn(B, H, P, N, device="cuda:0", generator=g), None)
    si = ScanInputs(x, b, b.clone(), torch.empty(B, 0, H, device="cuda:0"),
                    torch.zeros(H, device="cuda:0"), torch.empty(B, 0, H, device="cuda:0"))
    out = mamba3_scan(si.with_state(st).with_state_output(True))
    torch.cuda.synchronize()
    assert out.y.shape == x.shape and out.y.dtype == H16
    assert torch.equal(out.state.h, st.h) and torch.equal(out.state.last_u, st.last_u)
