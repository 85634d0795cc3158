"""ctypes binding of the CPU oracle (oracle/mamba3_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the reported CPU
baseline, never as the thing measured or shipped.  The product library
(mamba3 / libmamba3_hip.so) never imports this module.

Every function mirrors one C entry point; see the C file for the reference
citations (file:line) each one restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmamba3_oracle.so")
_lib = None

# Planted-mistake codes understood by m3o_set_fault (see mamba3_oracle.c).
FAULTS = {
    "drop_beta": 1,
    "rot_sign": 2,
    "transpose_u": 3,
    "lambda_index": 4,
    "decay_sign": 5,
    "mimo_diag": 6,
    "skip_sign": 7,
    "carry_beta": 8,
    "chunk_state_w": 9,
    "bwd_rot_sign": 10,
}


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_F = C.POINTER(C.c_float)
_D = C.POINTER(C.c_double)
_Z = C.c_size_t


def _declare(L):
    L.m3o_set_fault.argtypes = [C.c_int]
    L.m3o_get_fault.restype = C.c_int
    L.m3o_num_threads.restype = C.c_int
    L.m3o_noise.argtypes = [_Z, C.c_uint64, _F]
    L.m3o_test_reference_f32.argtypes = [_Z] * 5 + [_F] * 8
    L.m3o_scan_recurrence_f64.argtypes = [_Z] * 6 + [_F] * 11 + [_D] * 4
    L.m3o_scan_backward_f64.argtypes = [_Z] * 6 + [_F] * 11 + [_D] * 15
    L.m3o_cumsum.argtypes = [_F, _F, _Z, _Z, _Z, C.c_int, C.c_int]
    L.m3o_wrap_to.argtypes = [C.c_float, C.c_float]
    L.m3o_wrap_to.restype = C.c_float
    L.m3o_trapezoid_weights.argtypes = [_F, _F, _F, _F, _Z, _Z, _Z]
    L.m3o_ssd_band.argtypes = [_F, _F, _F, _F, _Z, _Z]
    L.m3o_exp_decay1.argtypes = [C.c_float] * 3
    L.m3o_exp_decay1.restype = C.c_float
    L.m3o_ssm_coefficients.argtypes = [_F, _F, _F, _F, _Z, _Z]
    L.m3o_ssm_angle.argtypes = [_F, _F, _F, _F, _Z, _Z]
    L.m3o_rotate_by_angle.argtypes = [_F, _F, _F, _Z, _Z, _Z, _Z]
    L.m3o_ssd_chunked_f32.argtypes = [_Z] * 5 + [_F] * 7 + [_Z, C.c_int, _F, _F]
    L.m3o_scan_composed_f32.argtypes = ([_Z] * 6 + [_F] * 11 + [_Z, C.c_int] + [_F] * 4)
    L.m3o_step_f32.argtypes = [_Z] * 5 + [_F] * 12


def _f32(a):
    if a is None:
        return None
    return np.ascontiguousarray(a, dtype=np.float32)


def _pf(a):
    return None if a is None else a.ctypes.data_as(_F)


def _pd(a):
    return None if a is None else a.ctypes.data_as(_D)


class fault:
    """Context manager that plants one mistake in the oracle (CPU only)."""

    def __init__(self, name: str):
        self.code = FAULTS[name]

    def __enter__(self):
        lib().m3o_set_fault(self.code)
        return self

    def __exit__(self, *exc):
        lib().m3o_set_fault(0)
        return False


def num_threads() -> int:
    return int(lib().m3o_num_threads())


def noise(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().m3o_noise(n, seed, _pf(out))
    return out


def test_reference_f32(x, b, c, dt, lam, a_head):
    """tests/ssm.rs:58-106. x [B,T,H,P], b/c [B,T,H,N] -> (y, h)."""
    x, b, c, dt, lam, a_head = map(_f32, (x, b, c, dt, lam, a_head))
    B, T, H, P = x.shape
    N = b.shape[3]
    y = np.empty_like(x)
    h = np.empty((B, H, P, N), np.float32)
    lib().m3o_test_reference_f32(B, T, H, P, N, _pf(x), _pf(b), _pf(c), _pf(dt),
                                 _pf(lam), _pf(a_head), _pf(y), _pf(h))
    return y, h


def scan_recurrence_f64(x, b, c, dt, a_log, lam, theta=None, d_skip=None,
                        h0=None, last_u0=None, angle0=None):
    """f64 recurrence. x [B,T,H,P,R], b/c [B,T,H,N,R].

    Returns (y [B,T,H,P,R], h, last_u [B,H,P,N], angle [B,H,N/2] or None), f64.
    """
    x, b, c, dt, a_log, lam = map(_f32, (x, b, c, dt, a_log, lam))
    theta, d_skip, h0, last_u0, angle0 = map(_f32, (theta, d_skip, h0, last_u0, angle0))
    B, T, H, P, R = x.shape
    N = b.shape[3]
    y = np.zeros((B, T, H, P, R), np.float64)
    h = np.zeros((B, H, P, N), np.float64)
    lu = np.zeros((B, H, P, N), np.float64)
    ang = np.zeros((B, H, N // 2), np.float64) if theta is not None else None
    lib().m3o_scan_recurrence_f64(B, T, H, P, N, R, _pf(x), _pf(b), _pf(c), _pf(dt),
                                  _pf(a_log), _pf(lam), _pf(theta), _pf(d_skip), _pf(h0),
                                  _pf(last_u0), _pf(angle0), _pd(y), _pd(h), _pd(lu),
                                  _pd(ang))
    return y, h, lu, ang


def scan_backward_f64(x, b, c, dt, a_log, lam, dy, theta=None, d_skip=None, h0=None,
                      last_u0=None, angle0=None, dh_out=None, dlast_u_out=None,
                      dangle_out=None):
    """Reverse mode of scan_recurrence_f64 for the loss sum(dy * y) (+ the
    upstream state gradients).  Returns a dict of f64 gradients: x, b, c, dt,
    lam, a_log, theta, d_skip, h0, last_u0, angle0 (None where the input is
    absent)."""
    x, b, c, dt, a_log, lam = map(_f32, (x, b, c, dt, a_log, lam))
    theta, d_skip, h0, last_u0, angle0 = map(_f32, (theta, d_skip, h0, last_u0, angle0))
    d64 = lambda a: None if a is None else np.ascontiguousarray(a, np.float64)
    dy, dh_out, dlast_u_out, dangle_out = map(d64, (dy, dh_out, dlast_u_out, dangle_out))
    B, T, H, P, R = x.shape
    N = b.shape[3]
    z = lambda *shape: np.zeros(shape, np.float64)
    g = dict(x=z(B, T, H, P, R), b=z(B, T, H, N, R), c=z(B, T, H, N, R), dt=z(B, T, H),
             lam=z(B, T, H), a_log=z(H), theta=z(B, T, H, N // 2) if theta is not None else None,
             d_skip=z(H), h0=z(B, H, P, N), last_u0=z(B, H, P, N), angle0=z(B, H, N // 2))
    lib().m3o_scan_backward_f64(B, T, H, P, N, R, _pf(x), _pf(b), _pf(c), _pf(dt), _pf(a_log),
                                _pf(lam), _pf(theta), _pf(d_skip), _pf(h0), _pf(last_u0),
                                _pf(angle0), _pd(dy), _pd(dh_out), _pd(dlast_u_out),
                                _pd(dangle_out), _pd(g["x"]), _pd(g["b"]), _pd(g["c"]),
                                _pd(g["dt"]), _pd(g["lam"]), _pd(g["theta"]), _pd(g["a_log"]),
                                _pd(g["d_skip"]), _pd(g["h0"]), _pd(g["last_u0"]),
                                _pd(g["angle0"]))
    return g


def cumsum(x, axis, reverse=False, exclusive=False):
    x = _f32(x)
    outer = int(np.prod(x.shape[:axis], dtype=np.int64))
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    out = np.empty_like(x)
    lib().m3o_cumsum(_pf(x), _pf(out), outer, x.shape[axis], inner, int(reverse),
                     int(exclusive))
    return out


def wrap_to(v: float, a: float) -> float:
    return float(lib().m3o_wrap_to(v, a))


def trapezoid_weights(lam, dt):
    """[B,T,H] -> (g, w) (fused.rs:2483-2503)."""
    lam, dt = _f32(lam), _f32(dt)
    B, T, H = lam.shape
    g, w = np.empty_like(lam), np.empty_like(lam)
    lib().m3o_trapezoid_weights(_pf(lam), _pf(dt), _pf(g), _pf(w), B, T, H)
    return g, w


def ssd_band(acum, w, g):
    """[rows, chunk] x3 -> [rows, chunk, chunk] (fused.rs:2044-2070)."""
    acum, w, g = map(_f32, (acum, w, g))
    rows, chunk = acum.shape
    out = np.empty((rows, chunk, chunk), np.float32)
    lib().m3o_ssd_band(_pf(acum), _pf(w), _pf(g), _pf(out), rows, chunk)
    return out


def exp_decay1(a: float, b: float, m: float) -> float:
    return float(lib().m3o_exp_decay1(a, b, m))


def ssm_coefficients(a_log, dt, lam):
    """a_log [H], dt/lambda [B,H] -> packed [3, B*H] (fused.rs:1679-1697)."""
    a_log, dt, lam = map(_f32, (a_log, dt, lam))
    lanes = dt.size
    out = np.empty(3 * lanes, np.float32)
    lib().m3o_ssm_coefficients(_pf(a_log), _pf(dt), _pf(lam), _pf(out), a_log.size, lanes)
    return out.reshape(3, lanes)


def ssm_angle(dt, theta, prev=None):
    """dt [B,H], theta/prev [B,H,K] -> phi [B,H,K] (fused.rs:1534-1555)."""
    dt, theta, prev = _f32(dt), _f32(theta), _f32(prev)
    inner = theta.shape[-1]
    out = np.empty_like(theta)
    lib().m3o_ssm_angle(_pf(dt), _pf(theta), _pf(prev), _pf(out), inner, theta.size)
    return out


def rotate_by_angle(x, phi, repeat=1):
    """Rotate rows of x (last axis 2*half) by -phi (fused.rs:588-619)."""
    x, phi = _f32(x), _f32(phi)
    half = x.shape[-1] // 2
    rows = x.size // (2 * half)
    table_rows = phi.size // half
    out = np.empty_like(x)
    lib().m3o_rotate_by_angle(_pf(x), _pf(phi), _pf(out), rows, half, repeat, table_rows)
    return out


def ssd_chunked_f32(x, b, c, a, g, w, init=None, chunk=64, want_state=True):
    """scan.rs:116-291. x [B,T,H,P], b/c [B,T,H,N], a/g/w [B,T,H]."""
    x, b, c, a, g, w, init = map(_f32, (x, b, c, a, g, w, init))
    B, T, H, P = x.shape
    N = b.shape[3]
    y = np.zeros_like(x)
    fs = np.zeros((B, H, P, N), np.float32) if want_state else None
    lib().m3o_ssd_chunked_f32(B, T, H, P, N, _pf(x), _pf(b), _pf(c), _pf(a), _pf(g), _pf(w),
                              _pf(init), chunk, int(want_state), _pf(y), _pf(fs))
    return y, fs


def scan_composed_f32(x, b, c, dt, a_log, lam, theta=None, d_skip=None, h0=None,
                      last_u0=None, angle0=None, chunk=64, want_state=True):
    """scan.rs:458-638. Returns (y, h, last_u, angle) in f32."""
    x, b, c, dt, a_log, lam = map(_f32, (x, b, c, dt, a_log, lam))
    theta, d_skip, h0, last_u0, angle0 = map(_f32, (theta, d_skip, h0, last_u0, angle0))
    B, T, H, P, R = x.shape
    N = b.shape[3]
    y = np.zeros_like(x)
    h = np.zeros((B, H, P, N), np.float32) if want_state else None
    lu = np.zeros((B, H, P, N), np.float32) if want_state else None
    ang = (np.zeros((B, H, N // 2), np.float32)
           if (want_state and theta is not None) else None)
    lib().m3o_scan_composed_f32(B, T, H, P, N, R, _pf(x), _pf(b), _pf(c), _pf(dt),
                                _pf(a_log), _pf(lam), _pf(theta), _pf(d_skip), _pf(h0),
                                _pf(last_u0), _pf(angle0), chunk, int(want_state), _pf(y),
                                _pf(h), _pf(lu), _pf(ang))
    return y, h, lu, ang


def step_f32(x, b, c, dt, lam, a_log, theta, d_skip, h, last_u, angle):
    """scan.rs:649-712, in place on copies. x [B,H,P,R], b/c [B,H,N,R].

    Returns (y, h, last_u, angle) -- new arrays; the inputs are not modified.
    """
    x, b, c, dt, lam, a_log, theta, d_skip = map(_f32, (x, b, c, dt, lam, a_log, theta, d_skip))
    h = np.array(h, np.float32, copy=True)
    last_u = np.array(last_u, np.float32, copy=True)
    angle = None if angle is None else np.array(angle, np.float32, copy=True)
    B, H, P, R = x.shape
    N = b.shape[2]
    y = np.zeros_like(x)
    lib().m3o_step_f32(B, H, P, N, R, _pf(x), _pf(b), _pf(c), _pf(dt), _pf(lam), _pf(a_log),
                       _pf(theta), _pf(d_skip), _pf(h), _pf(last_u), _pf(angle), _pf(y))
    return y, h, last_u, angle
