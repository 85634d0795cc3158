"""The checks that pin the CPU oracle (oracle/mamba3_oracle.c).

Each check returns its worst error; a check passes when that error is within
its tolerance.  `run_all()` is used twice by tests/test_oracle.py: once on the
oracle as built (every check must pass) and once per planted mistake
(`oracle.fault(...)`), where at least one check must fail -- which shows that
the checks can see a dropped term, a wrong sign or index, or a transposed
operand.

Sources of expected values, none of them a retyping of the oracle's own code:
  * literal known answers from the reference tests (tests/tensor.rs:183-200);
  * the reference tests' own inputs and composed forms (tests/autograd.rs:518-823);
  * the reference test-suite's own oracle `reference()` (tests/ssm.rs:58-106);
  * closed forms of the recurrence for structured inputs (one token, pure decay,
    pure rotation = complex eigenvalue exp(i*theta*dt) per config.rs:50-53,
    constant-input trapezoid sums);
  * invariants: chunk-size independence, split windows, step == scan,
    MIMO == sum of SISO systems, Euler == Mamba-2.
"""
from __future__ import annotations

import math

import numpy as np

import oracle
from cases import Case, worst_rel

CHECKS = []


def check(tol):
    def deco(fn):
        CHECKS.append((fn.__name__, fn, tol))
        return fn
    return deco


# --------------------------------------------------------------------------- KATs

@check(1e-6)
def cumsum_known_answers():
    """tests/tensor.rs:183-200."""
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    errs = [
        worst_rel(oracle.cumsum(x, 1), [1, 3, 6, 10]),
        worst_rel(oracle.cumsum(x, 1, exclusive=True), [0, 1, 3, 6]),
        worst_rel(oracle.cumsum(x, 1, reverse=True), [10, 9, 7, 4]),
        worst_rel(oracle.cumsum(x, 1, reverse=True, exclusive=True), [9, 7, 4, 0]),
    ]
    return max(errs)


@check(1e-6)
def trapezoid_matches_composed_shift():
    """tests/autograd.rs:781-806: fused weights vs lambda*dt + shift_left((1-lambda)*dt)."""
    batch, seq, heads = 2, 4, 3
    n = batch * seq * heads
    lam = np.array([0.1 + 0.8 * ((i * 5 % 9) / 9.0) for i in range(n)], np.float32)
    dt = np.array([0.05 + (i * 3 % 7) * 0.12 for i in range(n)], np.float32)
    lam, dt = lam.reshape(batch, seq, heads), dt.reshape(batch, seq, heads)
    g, w = oracle.trapezoid_weights(lam, dt)
    g_c = lam * dt
    nxt = (np.float32(1.0) - lam) * dt
    shifted = np.concatenate([nxt[:, 1:], np.zeros((batch, 1, heads), np.float32)], axis=1)
    w_c = g_c + shifted
    return max(float(np.max(np.abs(g - g_c))), float(np.max(np.abs(w - w_c))))


@check(1e-7)
def trapezoid_euler_collapse():
    """Euler (lambda = 1) gives w == g (tests/ssm.rs:222-230)."""
    case = Case(1, 8, 2, 3, 4)
    lam = np.ones_like(case.lam)
    g, w = oracle.trapezoid_weights(lam, case.dt)
    return float(np.max(np.abs(w - g)))


@check(1e-5)
def coefficients_closed_form():
    """tests/autograd.rs:518-549 inputs; alpha, beta, gamma closed forms."""
    heads, batch = 3, 2
    a_log = np.array([0.2, -0.5, 0.8], np.float32)
    dt = np.array([0.2 + 0.1 * i for i in range(batch * heads)], np.float32)
    lam = np.array([0.3 + 0.05 * i for i in range(batch * heads)], np.float32)
    got = oracle.ssm_coefficients(a_log, dt, lam)
    worst = 0.0
    for i in range(batch * heads):
        a = -math.exp(a_log[i % heads])
        alpha = math.exp(dt[i] * a)
        want = [alpha, (1 - lam[i]) * dt[i] * alpha, lam[i] * dt[i]]
        for k in range(3):
            worst = max(worst, abs(got[k, i] - want[k]))
    return worst


@check(1e-5)
def angle_wrap_closed_form():
    """tests/autograd.rs:577-588: phi = raw - round(raw / 2pi) * 2pi, raw = prev + dt*theta."""
    batch, heads = 2, 3
    dt = np.array([0.2 + 0.1 * i for i in range(batch * heads)], np.float32)
    theta = np.array([0.4 + 0.3 * i for i in range(batch * heads * 2)], np.float32)
    prev = np.array([1.1 - 0.2 * i for i in range(batch * heads * 2)], np.float32)
    got = oracle.ssm_angle(dt.reshape(batch, heads), theta.reshape(batch, heads, 2),
                           prev.reshape(batch, heads, 2)).ravel()
    worst = 0.0
    for i in range(theta.size):
        raw = prev[i] + dt[i // 2] * theta[i]
        want = raw - round(raw / (2 * math.pi)) * 2 * math.pi
        worst = max(worst, abs(got[i] - want))
    # the result must lie in [-pi, pi]
    assert np.all(np.abs(got) <= math.pi + 1e-6)
    return worst


@check(1e-6)
def rotation_quarter_turn():
    """Closed form: rotating (1, 0) by -pi/2 gives (0, -1); (0, 1) gives (1, 0)."""
    x = np.array([[1.0, 0.0], [0.0, 1.0]], np.float32)
    phi = np.array([math.pi / 2], np.float32)
    out = oracle.rotate_by_angle(x, phi, repeat=2)
    return worst_rel(out, [[0.0, -1.0], [1.0, 0.0]])


@check(1e-5)
def rotation_composed_cos_sin_form():
    """tests/autograd.rs:590-601 inputs: direct rotation vs the (cos phi, -sin phi) composed form."""
    batch, heads = 2, 3
    field = np.array([((i % 9) - 4.0) * 0.2 for i in range(batch * heads * 4)], np.float32)
    theta = np.array([0.4 + 0.3 * i for i in range(batch * heads * 2)], np.float32)
    x = field.reshape(batch * heads, 4)
    phi = theta.reshape(batch * heads, 2)
    out = oracle.rotate_by_angle(x, phi, repeat=1)
    cs, sn = np.cos(phi), -np.sin(phi)   # composed: rotate_halves(cos, -sin)
    want = np.concatenate([x[:, :2] * cs - x[:, 2:] * sn, x[:, :2] * sn + x[:, 2:] * cs], axis=1)
    return float(np.max(np.abs(out - want)))


@check(1e-6)
def band_closed_form():
    """fused.rs:2044-2070: zero above the diagonal, g on it, w*exp(clamp(.)) below;
    one pair lies past the -60 floor (tests/autograd.rs:611-618 spread)."""
    acum = np.array([[0.0, -1.5, -40.0, -75.0]], np.float32)
    w = np.array([[0.3, 0.5, 0.7, 0.9]], np.float32)
    g = np.array([[0.2, 0.4, 0.6, 0.8]], np.float32)
    band = oracle.ssd_band(acum, w, g)[0]
    want = np.zeros((4, 4))
    for t in range(4):
        for s in range(t + 1):
            d = max(min(float(acum[0, t] - acum[0, s]), 0.0), -60.0)
            want[t, s] = (g[0, s] if s == t else w[0, s]) * math.exp(d)
    return worst_rel(band, want)


# -------------------------------------------------------- the reference's own oracle

def _ref_case(B, T, H, P, N):
    return Case(B, T, H, P, N)


@check(1e-5)
def f64_recurrence_matches_reference_oracle():
    """tests/ssm.rs:58-106 (f32, the reference's oracle) vs the f64 recurrence."""
    worst = 0.0
    for dims in [(2, 12, 3, 4, 6), (1, 13, 2, 3, 4), (2, 9, 2, 3, 4)]:
        case = _ref_case(*dims)
        y_ref, h_ref = case.reference()
        x, b, c = case.rank1()
        y, h, _, _ = oracle.scan_recurrence_f64(x, b, c, case.dt, case.a_log, case.lam)
        worst = max(worst, worst_rel(y[..., 0], y_ref), worst_rel(h, h_ref))
    return worst


@check(2e-4)
def chunked_scan_matches_the_recurrence():
    """tests/ssm.rs:187-205: ssd_chunked for chunk in {1,2,3,4,8,16} vs reference()."""
    worst = 0.0
    for chunk in [1, 2, 3, 4, 8, 16]:
        case = Case(2, 12, 3, 4, 6)
        a, g, w = case.weights()
        y, st = oracle.ssd_chunked_f32(case.x, case.b, case.c, a, g, w, None, chunk, True)
        want_y, want_h = case.reference()
        worst = max(worst, worst_rel(y, want_y), worst_rel(st, want_h))
    return worst


@check(2e-4)
def chunked_scan_handles_ragged_lengths():
    """tests/ssm.rs:207-220."""
    worst = 0.0
    for seq in [1, 5, 7, 13]:
        case = Case(1, seq, 2, 3, 4)
        a, g, w = case.weights()
        y, st = oracle.ssd_chunked_f32(case.x, case.b, case.c, a, g, w, None, 4, True)
        want_y, want_h = case.reference()
        worst = max(worst, worst_rel(y, want_y), worst_rel(st, want_h))
    return worst


@check(2e-4)
def euler_mode_reproduces_mamba2():
    """tests/ssm.rs:222-236; also the explicit Mamba-2 recurrence h = alpha h + dt B x^T."""
    case = Case(1, 8, 2, 3, 4)
    case.lam = np.ones_like(case.lam)
    a, g, w = case.weights()
    y, st = oracle.ssd_chunked_f32(case.x, case.b, case.c, a, g, w, None, 4, False)
    assert st is None
    want_y, _ = case.reference()
    # Mamba-2: h_t = exp(dt A) h_{t-1} + dt_t B_t x_t^T, y = C h (no trapezoid term)
    B, T, H, P, N = case.batch, case.seq, case.heads, case.head_dim, case.state
    y2 = np.zeros((B, T, H, P))
    for bb in range(B):
        for hh in range(H):
            hst = np.zeros((P, N))
            for t in range(T):
                d = float(case.dt[bb, t, hh])
                hst = math.exp(d * float(case.a_head[hh])) * hst + d * np.outer(
                    case.x[bb, t, hh].astype(np.float64), case.b[bb, t, hh].astype(np.float64))
                y2[bb, t, hh] = hst @ case.c[bb, t, hh].astype(np.float64)
    return max(worst_rel(y, want_y), worst_rel(y, y2))


def _scan_full(case, theta=None, d_skip=None, chunk=4, f64=False, **state):
    x, b, c = case.rank1()
    if f64:
        return oracle.scan_recurrence_f64(x, b, c, case.dt, case.a_log, case.lam, theta,
                                          d_skip, state.get("h0"), state.get("last_u0"),
                                          state.get("angle0"))
    return oracle.scan_composed_f32(x, b, c, case.dt, case.a_log, case.lam, theta, d_skip,
                                    state.get("h0"), state.get("last_u0"), state.get("angle0"),
                                    chunk, True)


def _split(case, theta, cut, f64):
    full = _scan_full(case, theta, f64=f64)
    x, b, c = case.rank1()
    T = case.seq

    def run(sl, st):
        kw = {}
        if st is not None:
            kw = dict(h0=np.asarray(st[1], np.float32), last_u0=np.asarray(st[2], np.float32),
                      angle0=np.asarray(st[3], np.float32))
        if f64:
            return oracle.scan_recurrence_f64(x[:, sl], b[:, sl], c[:, sl], case.dt[:, sl],
                                              case.a_log, case.lam[:, sl], theta[:, sl], None,
                                              kw.get("h0"), kw.get("last_u0"), kw.get("angle0"))
        return oracle.scan_composed_f32(x[:, sl], b[:, sl], c[:, sl], case.dt[:, sl],
                                        case.a_log, case.lam[:, sl], theta[:, sl], None,
                                        kw.get("h0"), kw.get("last_u0"), kw.get("angle0"), 4,
                                        True)

    first = run(slice(0, cut), None)
    second = run(slice(cut, T), first)
    joined = np.concatenate([first[0], second[0]], axis=1)
    return max(worst_rel(joined, full[0]), worst_rel(second[1], full[1]))


@check(3e-4)
def split_windows_match_a_single_pass():
    """tests/ssm.rs:238-310, for the composed algorithm and the f64 recurrence."""
    case = Case(2, 12, 2, 3, 4)
    theta = case.theta()
    return max(_split(case, theta, 5, False), _split(case, theta, 5, True))


@check(3e-4)
def step_matches_the_chunked_scan():
    """tests/ssm.rs:312-380: stepwise mamba3_step vs mamba3_scan (theta and D)."""
    case = Case(2, 9, 2, 3, 4)
    theta = case.theta()
    d_skip = np.array([0.3, -0.2], np.float32)
    par = _scan_full(case, theta, d_skip)
    par64 = _scan_full(case, theta, d_skip, f64=True)
    B, H, P, N = case.batch, case.heads, case.head_dim, case.state
    h = np.zeros((B, H, P, N), np.float32)
    lu = np.zeros_like(h)
    ang = np.zeros((B, H, N // 2), np.float32)
    ys = []
    for t in range(case.seq):
        y, h, lu, ang = oracle.step_f32(case.x[:, t, :, :, None], case.b[:, t, :, :, None],
                                        case.c[:, t, :, :, None], case.dt[:, t], case.lam[:, t],
                                        case.a_log, theta[:, t], d_skip, h, lu, ang)
        ys.append(y)
    step = np.stack(ys, axis=1)
    return max(worst_rel(step, par[0]), worst_rel(step, par64[0]),
               worst_rel(par[0], par64[0]))


@check(3e-4)
def composed_matches_f64_with_state_theta_skip_mimo():
    """Every ScanInputs feature at once, ranks 1-3, against the f64 recurrence."""
    rng = np.random.default_rng(1234)
    worst = 0.0
    for (B, T, H, P, N, R, chunk) in [(2, 11, 2, 3, 4, 1, 4), (1, 10, 2, 4, 6, 2, 3),
                                      (1, 9, 1, 3, 4, 3, 4)]:
        x = rng.uniform(-1, 1, (B, T, H, P, R)).astype(np.float32)
        b = rng.uniform(-1, 1, (B, T, H, N, R)).astype(np.float32)
        c = rng.uniform(-1, 1, (B, T, H, N, R)).astype(np.float32)
        dt = rng.uniform(0.05, 0.55, (B, T, H)).astype(np.float32)
        lam = rng.uniform(0.01, 0.99, (B, T, H)).astype(np.float32)
        a_log = rng.uniform(-0.5, 1.0, H).astype(np.float32)
        th = rng.uniform(-1, 1, (B, T, H, N // 2)).astype(np.float32)
        sk = rng.uniform(-1, 1, H).astype(np.float32)
        h0 = rng.uniform(-0.5, 0.5, (B, H, P, N)).astype(np.float32)
        l0 = rng.uniform(-0.5, 0.5, (B, H, P, N)).astype(np.float32)
        a0 = rng.uniform(-3, 3, (B, H, N // 2)).astype(np.float32)
        got = oracle.scan_composed_f32(x, b, c, dt, a_log, lam, th, sk, h0, l0, a0, chunk, True)
        want = oracle.scan_recurrence_f64(x, b, c, dt, a_log, lam, th, sk, h0, l0, a0)
        for gg, ww in zip(got, want):
            worst = max(worst, worst_rel(gg, ww))
    return worst


@check(1e-9)
def mimo_is_the_sum_of_siso_systems():
    """scan.rs:538-541: y_i = sum_j SISO(x_j, B_j, C_i), h = sum_j h^(j) (f64)."""
    rng = np.random.default_rng(7)
    B, T, H, P, N, R = 1, 7, 2, 3, 4, 3
    x = rng.uniform(-1, 1, (B, T, H, P, R)).astype(np.float32)
    b = rng.uniform(-1, 1, (B, T, H, N, R)).astype(np.float32)
    c = rng.uniform(-1, 1, (B, T, H, N, R)).astype(np.float32)
    dt = rng.uniform(0.05, 0.55, (B, T, H)).astype(np.float32)
    lam = rng.uniform(0.01, 0.99, (B, T, H)).astype(np.float32)
    a_log = rng.uniform(-0.5, 1.0, H).astype(np.float32)
    th = rng.uniform(-1, 1, (B, T, H, N // 2)).astype(np.float32)
    y, h, lu, _ = oracle.scan_recurrence_f64(x, b, c, dt, a_log, lam, th)
    ys = np.zeros_like(y)
    hs = np.zeros_like(h)
    for i in range(R):
        for j in range(R):
            yij, hij, _, _ = oracle.scan_recurrence_f64(
                x[..., j:j + 1], b[..., j:j + 1], c[..., i:i + 1], dt, a_log, lam, th)
            ys[..., i] += yij[..., 0]
            if i == 0:
                hs += hij
    return max(float(np.max(np.abs(ys - y))), float(np.max(np.abs(hs - h))))


# -------------------------------------------------------------- closed forms

@check(1e-12)
def one_token_closed_form():
    """T = 1: y = lambda dt (C . B) x + alpha C.h0 + beta C.last_u0 + D x (f64)."""
    rng = np.random.default_rng(3)
    B, T, H, P, N = 1, 1, 1, 3, 4
    x = rng.uniform(-1, 1, (B, T, H, P, 1)).astype(np.float32)
    b = rng.uniform(-1, 1, (B, T, H, N, 1)).astype(np.float32)
    c = rng.uniform(-1, 1, (B, T, H, N, 1)).astype(np.float32)
    dt = np.array([[[0.3]]], np.float32)
    lam = np.array([[[0.7]]], np.float32)
    a_log = np.array([0.4], np.float32)
    sk = np.array([0.25], np.float32)
    h0 = rng.uniform(-1, 1, (B, H, P, N)).astype(np.float32)
    l0 = rng.uniform(-1, 1, (B, H, P, N)).astype(np.float32)
    y, h, lu, _ = oracle.scan_recurrence_f64(x, b, c, dt, a_log, lam, None, sk, h0, l0)
    d, l = float(dt[0, 0, 0]), float(lam[0, 0, 0])
    alpha = math.exp(-d * math.exp(float(a_log[0])))
    cv, bv, xv = (c[0, 0, 0, :, 0].astype(np.float64), b[0, 0, 0, :, 0].astype(np.float64),
                  x[0, 0, 0, :, 0].astype(np.float64))
    want = (l * d * float(cv @ bv) * xv + alpha * (h0[0, 0].astype(np.float64) @ cv)
            + (1 - l) * d * alpha * (l0[0, 0].astype(np.float64) @ cv) + float(sk[0]) * xv)
    want_h = (l * d * np.outer(xv, bv) + alpha * h0[0, 0].astype(np.float64)
              + (1 - l) * d * alpha * l0[0, 0].astype(np.float64))
    return max(float(np.max(np.abs(y[0, 0, 0, :, 0] - want))),
               float(np.max(np.abs(h[0, 0] - want_h))),
               float(np.max(np.abs(lu[0, 0] - np.outer(xv, bv)))))


@check(1e-12)
def pure_decay_closed_form():
    """x = 0 with an initial state: y_t = exp(A sum_{s<=t} dt_s) C_t . h0 + beta term at t=0."""
    rng = np.random.default_rng(5)
    B, T, H, P, N = 1, 6, 2, 2, 3
    x = np.zeros((B, T, H, P, 1), np.float32)
    b = rng.uniform(-1, 1, (B, T, H, N, 1)).astype(np.float32)
    c = rng.uniform(-1, 1, (B, T, H, N, 1)).astype(np.float32)
    dt = rng.uniform(0.1, 0.5, (B, T, H)).astype(np.float32)
    lam = rng.uniform(0.1, 0.9, (B, T, H)).astype(np.float32)
    a_log = np.array([0.1, -0.3], np.float32)
    h0 = rng.uniform(-1, 1, (B, H, P, N)).astype(np.float32)
    l0 = rng.uniform(-1, 1, (B, H, P, N)).astype(np.float32)
    y, _, _, _ = oracle.scan_recurrence_f64(x, b, c, dt, a_log, lam, None, None, h0, l0)
    worst = 0.0
    for hh in range(H):
        A = -math.exp(float(a_log[hh]))
        S = h0[0, hh].astype(np.float64) + (1 - float(lam[0, 0, hh])) * float(dt[0, 0, hh]) * \
            l0[0, hh].astype(np.float64)
        cum = 0.0
        for t in range(T):
            cum += float(dt[0, t, hh])
            want = math.exp(A * cum) * (S @ c[0, t, hh, :, 0].astype(np.float64))
            worst = max(worst, float(np.max(np.abs(y[0, t, hh, :, 0] - want))))
    return worst


@check(1e-9)
def pure_rotation_closed_form():
    """Rotational dynamics are the complex eigenvalue exp(dt (A + i theta)) (config.rs:50-53).

    With A -> 0, Euler weights, dt = 1, an impulse x_0 = 1, B = (1, 0) and
    C = (0, 1): y_t = Im(exp(i theta t)) = sin(theta t)."""
    T, omega = 7, 0.9
    x = np.zeros((1, T, 1, 1, 1), np.float32)
    x[0, 0] = 1.0
    b = np.zeros((1, T, 1, 2, 1), np.float32)
    b[0, :, 0, 0, 0] = 1.0
    c = np.zeros((1, T, 1, 2, 1), np.float32)
    c[0, :, 0, 1, 0] = 1.0
    dt = np.ones((1, T, 1), np.float32)
    lam = np.ones((1, T, 1), np.float32)
    a_log = np.array([-60.0], np.float32)   # A = -exp(-60): no decay
    th = np.full((1, T, 1, 1), omega, np.float32)
    y, _, _, ang = oracle.scan_recurrence_f64(x, b, c, dt, a_log, lam, th)
    omega32 = float(np.float32(omega))
    want = np.array([math.sin(omega32 * t) for t in range(T)])
    wrapped = (omega32 * T + math.pi) % (2 * math.pi) - math.pi
    return max(float(np.max(np.abs(y[0, :, 0, 0, 0] - want))), abs(float(ang[0, 0, 0]) - wrapped))


@check(1e-12)
def constant_input_trapezoid_sum():
    """A = 0, P = N = 1, B = C = x = 1: y_t = sum_{s<=t} lambda_s dt_s + sum_{1<=s<=t} (1-lambda_s) dt_s."""
    rng = np.random.default_rng(11)
    T = 9
    x = np.ones((1, T, 1, 1, 1), np.float32)
    b = np.ones((1, T, 1, 1, 1), np.float32)
    c = np.ones((1, T, 1, 1, 1), np.float32)
    dt = rng.uniform(0.1, 0.5, (1, T, 1)).astype(np.float32)
    lam = rng.uniform(0.1, 0.9, (1, T, 1)).astype(np.float32)
    a_log = np.array([-80.0], np.float32)
    y, _, _, _ = oracle.scan_recurrence_f64(x, b, c, dt, a_log, lam)
    d = dt[0, :, 0].astype(np.float64)
    l = lam[0, :, 0].astype(np.float64)
    want = np.cumsum(l * d) + np.concatenate([[0.0], np.cumsum(((1 - l) * d)[1:])])
    return float(np.max(np.abs(y[0, :, 0, 0, 0] - want)))


@check(1e-12)
def outer_product_orientation():
    """last_u = x B^T is [P, N] with P != N: element [p][n] = x_p * B_n (scan.rs:620-638)."""
    x = np.zeros((1, 1, 1, 2, 1), np.float32)
    x[0, 0, 0, :, 0] = [2.0, 3.0]
    b = np.zeros((1, 1, 1, 2, 1), np.float32)
    b[0, 0, 0, :, 0] = [5.0, 7.0]
    c = np.zeros_like(b)
    dt = np.full((1, 1, 1), 0.5, np.float32)
    lam = np.full((1, 1, 1), 0.5, np.float32)
    _, h, lu, _ = oracle.scan_recurrence_f64(x, b, c, dt, np.zeros(1, np.float32), lam)
    want = np.array([[10.0, 14.0], [15.0, 21.0]])
    return max(float(np.max(np.abs(lu[0, 0] - want))), float(np.max(np.abs(h[0, 0] - 0.25 * want))))


# --------------------------------------------------------------------------- backward

def _loss_f64(inp, seeds):
    """L = <dy, y> + <dh, h> + <dlu, last_u> + <dang, angle> on the f64 recurrence."""
    y, h, lu, ang = oracle.scan_recurrence_f64(
        inp["x"], inp["b"], inp["c"], inp["dt"], inp["a_log"], inp["lam"], inp.get("theta"),
        inp.get("d_skip"), inp.get("h0"), inp.get("last_u0"), inp.get("angle0"))
    L = float(np.sum(seeds["dy"] * y))
    if seeds.get("dh") is not None:
        L += float(np.sum(seeds["dh"] * h)) + float(np.sum(seeds["dlu"] * lu))
    if seeds.get("dang") is not None and ang is not None:
        L += float(np.sum(seeds["dang"] * ang))
    return L


def _directional_errors(inp, seeds, eps=2e-5, seed=0):
    """For every input, |<grad, d> - (L(+) - L(-))/2| / scale, where d is half
    the f32 difference of the two perturbed inputs (central differences).  The
    error of a correct gradient is the O(eps^2) truncation term: about 4e-9
    at eps = 2e-5 (it falls 100x per 10x smaller eps)."""
    g = oracle.scan_backward_f64(
        inp["x"], inp["b"], inp["c"], inp["dt"], inp["a_log"], inp["lam"], seeds["dy"],
        inp.get("theta"), inp.get("d_skip"), inp.get("h0"), inp.get("last_u0"),
        inp.get("angle0"), seeds.get("dh"), seeds.get("dlu"), seeds.get("dang"))
    rng = np.random.default_rng(seed)
    errs = []
    for k in ("x", "b", "c", "dt", "lam", "a_log", "theta", "d_skip", "h0", "last_u0", "angle0"):
        if inp.get(k) is None:
            continue
        v = inp[k].astype(np.float64)
        direction = rng.standard_normal(v.shape)
        step = eps * (np.abs(v) + 0.1)
        plus = dict(inp)
        minus = dict(inp)
        plus[k] = (v + step * direction).astype(np.float32)
        minus[k] = (v - step * direction).astype(np.float32)
        d = (plus[k].astype(np.float64) - minus[k].astype(np.float64)) / 2.0
        numeric = (_loss_f64(plus, seeds) - _loss_f64(minus, seeds)) / 2.0
        analytic = float(np.sum(g[k] * d))
        errs.append(abs(analytic - numeric) / (abs(numeric) + 1e-3 * np.linalg.norm(d) + 1e-30))
    return max(errs)


def _bwd_case(B, T, H, P, N, R, theta, skip, state, seed):
    rng = np.random.default_rng(seed)
    inp = dict(baseline_like(rng, B, T, H, P, N, R, theta, state))
    if skip:
        inp["d_skip"] = rng.uniform(-1, 1, H).astype(np.float32)
    seeds = dict(dy=rng.standard_normal((B, T, H, P, R)))
    if state:
        seeds["dh"] = rng.standard_normal((B, H, P, N))
        seeds["dlu"] = rng.standard_normal((B, H, P, N))
        if theta:
            seeds["dang"] = rng.standard_normal((B, H, N // 2))
    return inp, seeds


def baseline_like(rng, B, T, H, P, N, R, theta, state):
    f = np.float32
    out = dict(
        x=rng.standard_normal((B, T, H, P, R)).astype(f),
        b=(rng.standard_normal((B, T, H, N, R)) / math.sqrt(N)).astype(f),
        c=(rng.standard_normal((B, T, H, N, R)) / math.sqrt(N)).astype(f),
        dt=rng.uniform(0.02, 0.3, (B, T, H)).astype(f),
        a_log=rng.uniform(-0.5, 1.5, H).astype(f),
        lam=rng.uniform(0.1, 0.9, (B, T, H)).astype(f))
    if theta:
        out["theta"] = rng.uniform(0.0, math.pi, (B, T, H, N // 2)).astype(f)
    if state:
        out["h0"] = (0.3 * rng.standard_normal((B, H, P, N))).astype(f)
        out["last_u0"] = (0.3 * rng.standard_normal((B, H, P, N))).astype(f)
        if theta:
            out["angle0"] = rng.uniform(-3.0, 3.0, (B, H, N // 2)).astype(f)
    return out


@check(1e-7)
def backward_directional_derivatives_rotational_state_skip():
    """Every gradient against central differences of the f64 recurrence:
    rotating frame, skip, carried-in state and upstream state gradients,
    two checkpoint segments (T = 37)."""
    inp, seeds = _bwd_case(1, 37, 2, 3, 4, 1, True, True, True, 1)
    return _directional_errors(inp, seeds, seed=1)


@check(1e-7)
def backward_directional_derivatives_mimo():
    """MIMO rank 2 (the R^2 cross terms, scan.rs:538-589), rotating frame."""
    inp, seeds = _bwd_case(2, 20, 1, 2, 6, 2, True, False, False, 2)
    return _directional_errors(inp, seeds, seed=2)


@check(1e-7)
def backward_directional_derivatives_real_long():
    """Real dynamics over three checkpoint segments (T = 70), no state."""
    inp, seeds = _bwd_case(1, 70, 2, 4, 2, 1, False, True, False, 3)
    return _directional_errors(inp, seeds, seed=3)


@check(2e-2)
def backward_reference_differentiable_case():
    """tests/ssm.rs:382-426: Case::new(1, 6, 2, 3, 4), loss = sum(y^2), dx at
    coordinates 0, 5, 17, 30 against central differences (eps 1e-3) at the
    reference's own tolerance 2e-2 * (1 + |numeric|)."""
    case = Case(1, 6, 2, 3, 4)
    x, b, c = case.rank1()
    args = (b, c, case.dt, case.a_log, case.lam)
    y, _, _, _ = oracle.scan_recurrence_f64(x, *args)
    g = oracle.scan_backward_f64(x, b, c, case.dt, case.a_log, case.lam, 2.0 * y)
    worst = 0.0
    for i in (0, 5, 17, 30):
        def run(data):
            yy, _, _, _ = oracle.scan_recurrence_f64(data.reshape(x.shape), *args)
            return float(np.sum(yy.astype(np.float32) ** 2))
        plus = x.ravel().copy()
        minus = x.ravel().copy()
        plus[i] += np.float32(1e-3)
        minus[i] -= np.float32(1e-3)
        numeric = (run(plus) - run(minus)) / (2e-3)
        worst = max(worst, abs(g["x"].ravel()[i] - numeric) / (1.0 + abs(numeric)))
    return worst


def run_all():
    """Run every check; returns {name: (passed, worst_error)}."""
    out = {}
    for name, fn, tol in CHECKS:
        try:
            err = fn()
            out[name] = (bool(err <= tol), err)
        except AssertionError as e:   # a structural assertion inside a check
            out[name] = (False, str(e))
    return out
