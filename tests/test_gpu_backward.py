"""GPU parity of the scan backward (m3_scan_backward through the C ABI, and the
autograd node of the Python mirror) against the f64 reverse-mode oracle
(oracle.scan_backward_f64, itself pinned by central differences of the f64
recurrence and by the reference's scan_is_differentiable case).

Bars: rel-L2 <= 1e-5 per gradient for f32 storage; <= 1e-2 for bf16 storage
(the oracle runs on the same bf16-rounded inputs and dy; dx, db, dc and dtheta
are returned in bf16).
"""
import math
import zlib

import numpy as np
import pytest
import torch

import oracle
from cases import baseline_inputs, bf16_round, rel_l2
from gpu_util import dev, host

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 1e-2

CASES = [
    # B, T, H, P, N, R, theta, skip, state, dtype
    (1, 100, 2, 64, 64, 1, True, True, True, "f32"),
    (2, 70, 1, 64, 128, 1, True, False, False, "f32"),
    (1, 50, 2, 64, 64, 2, True, True, False, "f32"),
    (1, 45, 1, 64, 128, 4, True, True, True, "f32"),
    (1, 96, 2, 64, 128, 1, False, True, False, "f32"),
    (1, 33, 1, 64, 128, 2, False, False, True, "f32"),
    (1, 1, 2, 64, 64, 1, True, True, True, "f32"),
    (1, 200, 2, 64, 128, 1, True, True, True, "bf16"),
    (1, 130, 2, 64, 64, 1, True, False, False, "bf16"),
    (1, 90, 1, 64, 64, 2, True, True, True, "bf16"),
    (2, 60, 1, 64, 128, 4, True, True, False, "bf16"),
    (1, 65, 2, 64, 64, 4, False, True, True, "bf16"),
]

NAMES = ("x", "b", "c", "dt", "lam", "a_log", "theta", "d_skip", "h0", "last_u0", "angle0")


def _run(case, upstream=True):
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan_backward
    B, T, H, P, N, R, theta, skip, state, dtype = case
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=theta, dtype=dtype,
                          theta_per_head=False, state=state)
    d_skip = rng.uniform(-1, 1, H).astype(np.float32) if skip else None
    dy = rng.standard_normal((B, T, H, P, R)).astype(np.float32)
    if dtype == "bf16":
        dy = bf16_round(dy)
    dh = (rng.standard_normal((B, H, P, N)) * 0.1).astype(np.float32) if (state and upstream) else None
    dang = (rng.standard_normal((B, H, N // 2)) * 0.1).astype(np.float32) \
        if (state and theta and upstream) else None
    # dL/d(output last_u): flows into x, b and the last token's angle
    dlu = (rng.standard_normal((B, H, P, N)) * 0.1).astype(np.float32) if upstream else None
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    si = ScanInputs(dev(inp["x"], tdt), dev(inp["b"], tdt), dev(inp["c"], tdt), dev(inp["dt"]),
                    dev(inp["a_log"]), dev(inp["lam"]))
    if theta:
        si = si.with_theta(dev(inp["theta"], tdt))
    if skip:
        si = si.with_skip(dev(d_skip))
    if state:
        si = si.with_state(SsmState(dev(inp["h0"]), dev(inp["last_u0"]),
                                    dev(inp["angle0"]) if theta else None))
    g = mamba3_scan_backward(si, dev(dy, tdt), None if dh is None else dev(dh),
                             None if dang is None else dev(dang),
                             None if dlu is None else dev(dlu))
    torch.cuda.synchronize()
    ref = oracle.scan_backward_f64(
        inp["x"], inp["b"], inp["c"], inp["dt"], inp["a_log"], inp["lam"], dy,
        inp["theta"] if theta else None, d_skip, inp.get("h0") if state else None,
        inp.get("last_u0") if state else None, inp.get("angle0") if (state and theta) else None,
        dh, dlu, dang)
    return g, ref


@pytest.mark.parametrize("case", CASES, ids=[repr(c) for c in CASES])
def test_backward_against_f64_reverse_mode(case):
    g, ref = _run(case)
    tol = BF16_TOL if case[-1] == "bf16" else F32_TOL
    checked = 0
    for k in NAMES:
        mine = getattr(g, k)
        if mine is None or ref.get(k) is None:
            continue
        err = rel_l2(host(mine), ref[k])
        assert err <= tol, (k, err)
        checked += 1
    assert checked >= 6


# Shapes the chunk kernels do not take (head_dim other than 64, d_state other
# than 64 / 128, rank other than 1, 2, 4): the reverse mode of the recurrence,
# token by token, against the same f64 reverse mode.
GENERIC_CASES = [
    # B, T, H, P, N, R, theta, skip, state, dtype
    (1, 40, 2, 48, 32, 1, True, True, True, "f32"),
    (2, 33, 1, 16, 16, 3, True, False, True, "f32"),
    (1, 50, 1, 160, 64, 1, False, True, False, "f32"),
    (1, 70, 2, 32, 96, 2, True, True, True, "bf16"),
    (1, 37, 1, 24, 8, 5, True, True, False, "bf16"),
    (3, 1, 2, 40, 16, 1, True, True, True, "f32"),        # one token
]


@pytest.mark.parametrize("case", GENERIC_CASES, ids=[repr(c) for c in GENERIC_CASES])
def test_generic_backward_against_f64_reverse_mode(case):
    from mamba3 import _lib
    before = _lib.lib().m3_launch_count()
    g, ref = _run(case)
    assert _lib.lib().m3_launch_count() - before == 2   # the token walk and the head sums
    tol = BF16_TOL if case[-1] == "bf16" else F32_TOL
    checked = 0
    for k in NAMES:
        mine = getattr(g, k)
        if mine is None or ref.get(k) is None:
            continue
        err = rel_l2(host(mine), ref[k])
        assert err <= tol, (k, err)
        checked += 1
    assert checked >= 6


def test_upstream_state_gradient_only():
    """dy = 0 with dL/dh and dL/dangle of the output state: the whole gradient
    flows back through the reverse state pass alone."""
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan_backward
    rng = np.random.default_rng(21)
    B, T, H, P, N = 1, 150, 2, 64, 128
    inp = baseline_inputs(rng, B, T, H, P, N, 1, theta=True, theta_per_head=False, state=True)
    dy = np.zeros((B, T, H, P, 1), np.float32)
    dh = rng.standard_normal((B, H, P, N)).astype(np.float32)
    dang = rng.standard_normal((B, H, N // 2)).astype(np.float32)
    si = (ScanInputs(dev(inp["x"]), dev(inp["b"]), dev(inp["c"]), dev(inp["dt"]),
                     dev(inp["a_log"]), dev(inp["lam"])).with_theta(dev(inp["theta"]))
          .with_state(SsmState(dev(inp["h0"]), dev(inp["last_u0"]), dev(inp["angle0"]))))
    g = mamba3_scan_backward(si, dev(dy), dev(dh), dev(dang))
    ref = oracle.scan_backward_f64(inp["x"], inp["b"], inp["c"], inp["dt"], inp["a_log"],
                                   inp["lam"], dy, inp["theta"], None, inp["h0"], inp["last_u0"],
                                   inp["angle0"], dh, None, dang)
    for k in ("x", "b", "c", "dt", "lam", "a_log", "theta", "h0", "last_u0", "angle0"):
        assert rel_l2(host(getattr(g, k)), ref[k]) <= F32_TOL, k


def test_autograd_node_matches_the_direct_backward():
    """loss = <w, y> through mamba3_scan with requires_grad: torch's backward
    calls m3_scan_backward and returns the same gradients."""
    from mamba3.ssm import ScanInputs, mamba3_scan, mamba3_scan_backward
    rng = np.random.default_rng(3)
    B, T, H, P, N = 2, 80, 2, 64, 64
    inp = baseline_inputs(rng, B, T, H, P, N, 1, theta=True, theta_per_head=False)
    ts = {k: dev(inp[k]).requires_grad_(True) for k in ("x", "b", "c", "dt", "a_log", "lam",
                                                          "theta")}
    d_skip = dev(rng.uniform(-1, 1, H).astype(np.float32)).requires_grad_(True)
    wgt = dev(rng.standard_normal((B, T, H, P, 1)).astype(np.float32))
    out = mamba3_scan(ScanInputs(ts["x"], ts["b"], ts["c"], ts["dt"], ts["a_log"], ts["lam"])
                      .with_theta(ts["theta"]).with_skip(d_skip).with_state_output(False))
    assert out.state is None
    (out.y * wgt).sum().backward()
    with torch.no_grad():
        g = mamba3_scan_backward(
            ScanInputs(ts["x"], ts["b"], ts["c"], ts["dt"], ts["a_log"], ts["lam"])
            .with_theta(ts["theta"]).with_skip(d_skip), wgt)
    for k, mine in (("x", g.x), ("b", g.b), ("c", g.c), ("dt", g.dt), ("a_log", g.a_log),
                    ("lam", g.lam), ("theta", g.theta)):
        assert rel_l2(host(ts[k].grad), host(mine)) <= 1e-6, k
    assert rel_l2(host(d_skip.grad), host(g.d_skip)) <= 1e-6


@pytest.mark.parametrize("dtype,R,rot,P,N", [("f32", 1, True, 64, 64), ("f32", 2, False, 64, 64),
                                             ("bf16", 1, True, 64, 64), ("bf16", 4, True, 64, 64),
                                             # the backward's token walk; the second
                                             # with the forward token by token too
                                             ("f32", 3, True, 48, 32), ("f32", 1, True, 160, 32)])
def test_two_windows_chained_through_the_state(dtype, R, rot, P, N):
    """Two windows joined through SsmState (the second starts from the first's
    h, last_u and angle), differentiated end to end by autograd: the
    gradients equal those of the single window over the whole sequence.  The
    first window's output last_u reaches the loss only through the second
    window's carried state S = h + (1 - lambda_0) dt_0 last_u, so this needs
    the last_u adjoint (scan.rs:521-535, 599-618)."""
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan, mamba3_scan_backward
    rng = np.random.default_rng(11 + R)
    B, T, H, cut = 1, 150, 2, 70
    inp = baseline_inputs(rng, B, T, H, P, N, R, theta=rot, dtype=dtype, theta_per_head=False)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    keys = ("x", "b", "c", "dt", "lam") + (("theta",) if rot else ())
    full = {k: dev(inp[k], tdt if k in ("x", "b", "c", "theta") else torch.float32) for k in keys}
    a_log = dev(inp["a_log"])
    w = dev(rng.standard_normal((B, T, H, P, R)).astype(np.float32), tdt)
    wh = dev(rng.standard_normal((B, H, P, N)).astype(np.float32) * 0.1)
    parts = [{k: full[k][:, s].clone().requires_grad_(True) for k in keys}
             for s in (slice(0, cut), slice(cut, T))]
    al = a_log.clone().requires_grad_(True)

    def inputs(d):
        si = ScanInputs(d["x"], d["b"], d["c"], d["dt"], al, d["lam"])
        return si.with_theta(d["theta"]) if rot else si

    o1 = mamba3_scan(inputs(parts[0]))
    o2 = mamba3_scan(inputs(parts[1]).with_state(o1.state))
    loss = ((o1.y.float() * w[:, :cut].float()).sum() + (o2.y.float() * w[:, cut:].float()).sum()
            + (o2.state.h * wh).sum())
    loss.backward()
    with torch.no_grad():
        si = ScanInputs(full["x"], full["b"], full["c"], full["dt"], a_log, full["lam"])
        if rot:
            si = si.with_theta(full["theta"])
        g = mamba3_scan_backward(si, w, wh)
    tol = BF16_TOL if dtype == "bf16" else 1e-4
    for k in keys:
        joined = torch.cat([parts[0][k].grad.float(), parts[1][k].grad.float()], dim=1)
        err = rel_l2(host(joined), host(getattr(g, k if k != "lam" else "lam")))
        assert err <= tol, (k, err)
    assert rel_l2(host(al.grad), host(g.a_log)) <= tol


@pytest.mark.parametrize("what", ["dt", "lam", "a_log", "theta", "d_skip", "dh", "dangle",
                                  "dlast_u", "state.h", "state.angle"])
def test_backward_rejects_mis_shaped_tensors_before_any_launch(what):
    """mamba3_scan_backward checks every tensor's shape on the host: a wrong
    one raises ShapeError and no kernel runs."""
    from mamba3 import ShapeError, _lib
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan_backward
    B, T, H, P, N = 1, 40, 2, 64, 64
    t = lambda *s: torch.zeros(s, device="cuda")
    ok = dict(dt=t(B, T, H), lam=t(B, T, H), a_log=t(H), theta=t(B, T, H, N // 2), d_skip=t(H),
              dh=t(B, H, P, N), dangle=t(B, H, N // 2), dlast_u=t(B, H, P, N),
              h=t(B, H, P, N), angle=t(B, H, N // 2))
    bad = {"dt": t(B, T + 1, H), "lam": t(B, T, H + 1), "a_log": t(H + 1),
           "theta": t(B, T, H, N // 2 - 1), "d_skip": t(1), "dh": t(B, H, P, N - 1),
           "dangle": t(B, H, N), "dlast_u": t(B, H, P + 1, N), "state.h": t(B, H, P, N + 2),
           "state.angle": t(B, H, 3)}[what]
    k = what.split(".")[-1]
    args = dict(ok)
    args["h" if what == "state.h" else ("angle" if what == "state.angle" else k)] = bad
    si = (ScanInputs(t(B, T, H, P, 1), t(B, T, H, N, 1), t(B, T, H, N, 1), args["dt"],
                     args["a_log"], args["lam"]).with_theta(args["theta"]).with_skip(args["d_skip"])
          .with_state(SsmState(args["h"], t(B, H, P, N), args["angle"])))
    before = _lib.lib().m3_launch_count()
    with pytest.raises(ShapeError, match=what.split(".")[-1] if what != "lam" else "lambda"):
        mamba3_scan_backward(si, t(B, T, H, P, 1), args["dh"], args["dangle"], args["dlast_u"])
    assert _lib.lib().m3_launch_count() == before


def test_step_rejects_mis_shaped_theta_and_skip():
    from mamba3 import ShapeError
    from mamba3.ssm import SsmState, mamba3_step_
    B, H, P, N = 2, 3, 64, 64
    t = lambda *s: torch.zeros(s, device="cuda")
    st = SsmState(t(B, H, P, N), t(B, H, P, N), t(B, H, N // 2))
    x, b = t(B, H, P, 1), t(B, H, N, 1)
    with pytest.raises(ShapeError, match="theta"):
        mamba3_step_(x, b, b, t(B, H), t(B, H), t(H), t(B, H, N // 2 + 1), None, st)
    with pytest.raises(ShapeError, match="d_skip"):
        mamba3_step_(x, b, b, t(B, H), t(B, H), t(H), t(B, H, N // 2), t(H + 1), st)


def test_config1_shape_two_heads_full_length():
    """BASELINE config 1 shapes (L2048, P64, N128, bf16, Rotational) on two heads."""
    case = (1, 2048, 2, 64, 128, 1, True, False, False, "bf16")
    g, ref = _run(case)
    for k in ("x", "b", "c", "dt", "lam", "a_log", "theta"):
        assert rel_l2(host(getattr(g, k)), ref[k]) <= BF16_TOL, k


def test_backward_errors_surface_as_reference_errors():
    from mamba3 import ArgumentError, UnsupportedError
    from mamba3.ssm import ScanInputs, mamba3_scan_backward
    rng = np.random.default_rng(4)
    # head_dim 9000: its x and dy rows alone exceed the token walk's 64 KB
    inp = baseline_inputs(rng, 1, 10, 1, 9000, 16, 1, theta=True)
    si = (ScanInputs(dev(inp["x"]), dev(inp["b"]), dev(inp["c"]), dev(inp["dt"]),
                     dev(inp["a_log"]), dev(inp["lam"])).with_theta(dev(inp["theta"])))
    with pytest.raises(UnsupportedError, match="fit 64 KB"):
        mamba3_scan_backward(si, dev(np.zeros((1, 10, 1, 9000, 1), np.float32)))
    # a gradient buffer off the 16-byte grid
    from mamba3 import _lib
    import ctypes as C
    inp2 = baseline_inputs(rng, 1, 40, 1, 64, 64, 1, theta=False)
    xs = dev(inp2["x"])
    cin = _lib.ScanInputsC(1, 40, 1, 64, 64, 1, _lib.M3_F32, xs.data_ptr(),
                           dev(inp2["b"]).data_ptr(), dev(inp2["c"]).data_ptr(),
                           dev(inp2["dt"]).data_ptr(), dev(inp2["a_log"]).data_ptr(),
                           dev(inp2["lam"]).data_ptr(), None, None, None, 64, 0, None, 0)
    ws = torch.zeros(int(_lib.lib().m3_scan_backward_workspace_bytes(C.byref(cin))),
                     dtype=torch.uint8, device="cuda")
    cin.workspace, cin.workspace_bytes = ws.data_ptr(), ws.numel()
    big = torch.zeros(xs.numel() + 4, device="cuda")
    gb, gc = torch.zeros(2, 40 * 64, device="cuda")
    gdt, glam, ga = torch.zeros(40, device="cuda"), torch.zeros(40, device="cuda"), \
        torch.zeros(1, device="cuda")
    gr = _lib.ScanGradsC(xs.data_ptr(), None, None, big.data_ptr() + 4, gb.data_ptr(),
                         gc.data_ptr(), gdt.data_ptr(), glam.data_ptr(), ga.data_ptr(), None,
                         None, None, None, None)
    st = _lib.lib().m3_scan_backward(C.byref(cin), C.byref(gr),
                                     C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.M3_ERR_UNSUPPORTED
    x = torch.zeros(1, 10, 1, 64, 1, device="cuda")
    with pytest.raises(ArgumentError):
        mamba3_scan_backward(ScanInputs(x, dev(inp["b"]), dev(inp["c"]), dev(inp["dt"]),
                                        dev(inp["a_log"]), dev(inp["lam"])), x.cpu())
