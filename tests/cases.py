"""Input cases shared by the oracle and GPU parity tests.

`Case` restates the reference test fixture of tests/ssm.rs:108-185 (the LCG
`noise` of tests/ssm.rs:26-34 and its distributions), so the parity tests run
on exactly the inputs the reference's own tests use.  `baseline_inputs`
draws the BASELINE.json config distributions with numpy.
"""
from __future__ import annotations

import math

import numpy as np

import oracle


def assert_close(actual, expected, eps, what=""):
    """tests/ssm.rs:36-53: worst |a - e| / (1 + |e|) <= eps."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    assert a.shape == e.shape, f"{what}: length mismatch {a.shape} vs {e.shape}"
    if a.size == 0:
        return 0.0
    err = np.abs(a - e) / (1.0 + np.abs(e))
    at = int(np.argmax(err))
    worst = float(err[at])
    assert worst <= eps, (f"{what}: worst relative error {worst} at index {at} "
                          f"(got {a[at]}, want {e[at]})")
    return worst


def worst_rel(actual, expected):
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - e) / (1.0 + np.abs(e))))


def rel_l2(actual, expected):
    """The north-star parity metric ||a - e||_2 / ||e||_2."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    den = float(np.linalg.norm(e))
    num = float(np.linalg.norm(a - e))
    return num / den if den > 0 else num


class Case:
    """tests/ssm.rs:108-185 -- `Case::new(batch, seq, heads, head_dim, state)`."""

    def __init__(self, batch, seq, heads, head_dim, state):
        self.batch, self.seq, self.heads = batch, seq, heads
        self.head_dim, self.state = head_dim, state
        bt = batch * seq * heads
        f = np.float32
        self.dt = (f(0.05) + f(0.25) * (oracle.noise(bt, 7) + f(1.0))).astype(f)
        self.lam = (f(0.5) * (oracle.noise(bt, 11) + f(1.0)) * f(0.98) + f(0.01)).astype(f)
        self.a_head = np.array([-(f(1.0) + f(i) * f(0.7)) for i in range(heads)], f)
        self.x = oracle.noise(batch * seq * heads * head_dim, 1)
        self.b = oracle.noise(batch * seq * heads * state, 2)
        self.c = oracle.noise(batch * seq * heads * state, 3)
        self.reshape()

    def reshape(self):
        B, T, H, P, N = self.batch, self.seq, self.heads, self.head_dim, self.state
        self.x = self.x.reshape(B, T, H, P)
        self.b = self.b.reshape(B, T, H, N)
        self.c = self.c.reshape(B, T, H, N)
        self.dt = self.dt.reshape(B, T, H)
        self.lam = self.lam.reshape(B, T, H)

    @property
    def a_log(self):
        """`vars()` passes ln(-A) as a_log (tests/ssm.rs:168-171)."""
        return np.log(-self.a_head).astype(np.float32)

    def theta(self, seed=5):
        """tests/ssm.rs:242-245: noise(B*T*H*N/2, 5)."""
        B, T, H, N = self.batch, self.seq, self.heads, self.state
        return oracle.noise(B * T * H * (N // 2), seed).reshape(B, T, H, N // 2)

    def weights(self):
        """tests/ssm.rs:175-184: a = dt*A, g = lambda*dt, w = g + shift_left((1-lambda) dt)."""
        a = (self.dt * self.a_head.reshape(1, 1, -1)).astype(np.float32)
        g = (self.lam * self.dt).astype(np.float32)
        nxt = ((np.float32(1.0) - self.lam) * self.dt).astype(np.float32)
        shifted = np.zeros_like(nxt)
        shifted[:, :-1] = nxt[:, 1:]
        w = (g + shifted).astype(np.float32)
        return a, g, w

    def reference(self):
        return oracle.test_reference_f32(self.x, self.b, self.c, self.dt, self.lam, self.a_head)

    def rank1(self):
        """The `expand` closure: [.., last] -> [.., last, 1] (tests/ssm.rs:247-250)."""
        return self.x[..., None], self.b[..., None], self.c[..., None]


def baseline_inputs(rng, B, T, H, P, N, R=1, theta=False, dtype="f32", theta_per_head=True,
                    state=False):
    """BASELINE.json config distributions.

    x ~ N(0,1); dt = clamp(softplus(N(-3,1)), 1e-3, 0.1); a_log ~ U(0, ln 16);
    B, C ~ N(0,1)/sqrt(N); lambda = sigmoid(N(0,1)); theta ~ U(0, pi) per head
    per state pair (broadcast over batch and time) or per token.
    bf16 storage: x/b/c/theta are rounded to bf16 (round-to-nearest-even).
    """
    f = np.float32
    x = rng.standard_normal((B, T, H, P, R), dtype=f)
    b = (rng.standard_normal((B, T, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f)
    c = (rng.standard_normal((B, T, H, N, R), dtype=f) / f(math.sqrt(N))).astype(f)
    raw = rng.standard_normal((B, T, H), dtype=f) - f(3.0)
    dt = np.clip(np.log1p(np.exp(raw.astype(np.float64))), 1e-3, 0.1).astype(f)
    a_log = rng.uniform(0.0, math.log(16.0), H).astype(f)
    lam = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H)).astype(np.float64)))).astype(f)
    th = None
    if theta:
        if theta_per_head:
            th = np.broadcast_to(rng.uniform(0.0, math.pi, (1, 1, H, N // 2)).astype(f),
                                 (B, T, H, N // 2)).copy()
        else:
            th = rng.uniform(0.0, math.pi, (B, T, H, N // 2)).astype(f)
    out = dict(x=x, b=b, c=c, dt=dt, a_log=a_log, lam=lam, theta=th)
    if dtype == "bf16":
        for k in ("x", "b", "c", "theta"):
            if out[k] is not None:
                out[k] = bf16_round(out[k])
    if state:
        out["h0"] = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
        out["last_u0"] = (rng.standard_normal((B, H, P, N), dtype=f) * f(0.1)).astype(f)
        if theta:
            out["angle0"] = rng.uniform(-math.pi, math.pi, (B, H, N // 2)).astype(f)
    return out


def bf16_round(a):
    """Round f32 to the nearest bf16 (ties to even), returned as f32."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    nan = np.isnan(a)
    out = r.astype(np.uint32).view(np.float32).copy()
    out[nan] = a[nan]
    return out


def bf16_bits(a):
    """f32 (already bf16-representable or not) -> uint16 bf16 bit patterns (RNE)."""
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)
