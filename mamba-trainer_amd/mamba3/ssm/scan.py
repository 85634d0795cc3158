"""The chunked scan and the decode step (src/ssm/scan.rs), on the gfx950 kernels.

Same names, argument meanings and errors as the reference's `ssm::scan`
module; every call goes through the C ABI of libmamba3_hip.so
(include/mamba3_ssm.h).  torch tensors are used only as device buffers: the
arithmetic is in the HIP kernels, and there is no CPU or torch fallback --
tensors that are not on a ROCm device are rejected.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from .. import _lib
from ..error import ArgumentError, RankError, ShapeError, UnsupportedError

_DTYPES = {torch.float32: _lib.M3_F32, torch.bfloat16: _lib.M3_BF16, torch.float16: _lib.M3_F16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise UnsupportedError(f"unsupported: storage dtype {t.dtype}; use float32, bfloat16 or "
                               "float16")


def _dev(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ArgumentError(f"{what} must be a ROCm device tensor (got {t.device}); "
                            "the scan has no CPU path")
    return t.contiguous()


def _f32(t: Optional[torch.Tensor], what: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    t = _dev(t, what)
    return t if t.dtype == torch.float32 else t.float()


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _expect_shape(t: torch.Tensor, shape, what: str):
    if tuple(t.shape) != tuple(shape):
        raise ShapeError(f"shape error: {what} has shape {list(t.shape)}, expected {list(shape)}")


@dataclass
class SsmState:
    """scan.rs:293-358: h and last_u [B, H, P, N] (f32), angle [B, H, N/2] or None."""
    h: torch.Tensor
    last_u: torch.Tensor
    angle: Optional[torch.Tensor] = None

    def num_elements(self) -> int:
        return self.h.numel() + self.last_u.numel() + (
            self.angle.numel() if self.angle is not None else 0)

    @staticmethod
    def zeros(batch, heads, head_dim, d_state, rotational, device) -> "SsmState":
        shape = (batch, heads, head_dim, d_state)
        return SsmState(
            torch.zeros(shape, dtype=torch.float32, device=device),
            torch.zeros(shape, dtype=torch.float32, device=device),
            torch.zeros((batch, heads, d_state // 2), dtype=torch.float32, device=device)
            if rotational else None)

    def clone(self) -> "SsmState":
        return SsmState(self.h.clone(), self.last_u.clone(),
                        None if self.angle is None else self.angle.clone())

    def detach(self) -> "SsmState":
        return SsmState(self.h.detach(), self.last_u.detach(),
                        None if self.angle is None else self.angle.detach())

    def _c(self) -> _lib.SsmStateC:
        return _lib.SsmStateC(self.h.data_ptr(), self.last_u.data_ptr(),
                              None if self.angle is None else self.angle.data_ptr())


class ScanInputs:
    """scan.rs:360-443, with the same builder methods and defaults."""

    def __init__(self, x, b, c, dt, a_log, lam):
        self.x, self.b, self.c = x, b, c
        self.dt, self.a_log, self.lam = dt, a_log, lam
        self.theta = None
        self.d_skip = None
        self.state: Optional[SsmState] = None
        self.chunk_size = 64
        self.want_state = True
        self.chunk_parallel = True   # the three chunk-parallel kernels, where they apply

    def with_theta(self, theta):
        self.theta = theta
        return self

    def with_skip(self, d_skip):
        self.d_skip = d_skip
        return self

    def with_state(self, state: SsmState):
        self.state = state
        return self

    def with_chunk_size(self, chunk_size: int):
        self.chunk_size = chunk_size
        return self

    def with_state_output(self, want_state: bool):
        self.want_state = want_state
        return self

    def with_chunk_parallel(self, chunk_parallel: bool):
        """Select the chunk-parallel kernels (default; they take a workspace from
        torch's allocator) or the single-pass kernel, which allocates nothing;
        the results agree to rounding.  No reference counterpart."""
        self.chunk_parallel = chunk_parallel
        return self


@dataclass
class ScanOutput:
    """scan.rs:445-452."""
    y: torch.Tensor
    state: Optional[SsmState]


def mamba3_scan(inputs: ScanInputs) -> ScanOutput:
    """scan.rs:454-618: the Mamba-3 selective scan.

    Differentiable like the reference's Var-based scan: when autograd is on and
    an input requires grad, the backward is m3_scan_backward (the gradient the
    reference gets by autodiff through the composed scan)."""
    tensors = _scan_tensors(inputs)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        cfg = (inputs.chunk_size, inputs.want_state, inputs.chunk_parallel)
        y, h, lu, ang = _ScanFn.apply(cfg, *tensors)
        return ScanOutput(y, SsmState(h, lu, ang) if inputs.want_state else None)
    return _scan_forward(inputs)


def _scan_tensors(inputs: ScanInputs):
    st = inputs.state
    return (inputs.x, inputs.b, inputs.c, inputs.dt, inputs.a_log, inputs.lam, inputs.theta,
            inputs.d_skip, st.h if st else None, st.last_u if st else None,
            st.angle if st else None)


def _inputs_of(cfg, x, b, c, dt, a_log, lam, theta, d_skip, h0, last_u0, angle0) -> ScanInputs:
    si = ScanInputs(x, b, c, dt, a_log, lam)
    si.theta, si.d_skip = theta, d_skip
    si.state = SsmState(h0, last_u0, angle0) if h0 is not None else None
    si.chunk_size, si.want_state, si.chunk_parallel = cfg
    return si


class _ScanFn(torch.autograd.Function):
    """mamba3_scan as one differentiable node: forward m3_scan, backward
    m3_scan_backward (which recomputes the chunk states it needs)."""

    @staticmethod
    def forward(ctx, cfg, *tensors):
        with torch.no_grad():
            out = _scan_forward(_inputs_of(cfg, *tensors))
        ctx.cfg = cfg
        ctx.save_for_backward(*tensors)
        ctx.set_materialize_grads(False)
        st = out.state
        return (out.y, st.h if st else None, st.last_u if st else None,
                st.angle if st else None)

    @staticmethod
    def backward(ctx, dy, dh, dlu, dang):
        tensors = ctx.saved_tensors
        x = tensors[0]
        if dy is None:
            dy = torch.zeros_like(x)
        g = mamba3_scan_backward(_inputs_of(ctx.cfg, *tensors), dy, dh, dang, dlu)
        order = (g.x, g.b, g.c, g.dt, g.a_log, g.lam, g.theta, g.d_skip, g.h0, g.last_u0,
                 g.angle0)
        grads = [None if (t is None or gt is None) else gt.to(t.dtype).view_as(t)
                 for t, gt in zip(tensors, order)]
        return (None, *grads)


@dataclass
class ScanGrads:
    """Gradients of mamba3_scan's inputs (None where the input is absent)."""
    x: torch.Tensor
    b: torch.Tensor
    c: torch.Tensor
    dt: torch.Tensor
    a_log: torch.Tensor
    lam: torch.Tensor
    theta: Optional[torch.Tensor]
    d_skip: Optional[torch.Tensor]
    h0: Optional[torch.Tensor]
    last_u0: Optional[torch.Tensor]
    angle0: Optional[torch.Tensor]


def mamba3_scan_backward(inputs: ScanInputs, dy: torch.Tensor, dh: Optional[torch.Tensor] = None,
                         dangle: Optional[torch.Tensor] = None,
                         dlast_u: Optional[torch.Tensor] = None) -> ScanGrads:
    """Gradients of the scan's inputs for dL/dy = dy (and dL/d state.h, dL/d
    state.angle, dL/d state.last_u of the output state), through
    m3_scan_backward.  Every tensor's shape is checked before any launch."""
    x = _dev(inputs.x, "x")
    if x.dim() != 5:
        raise RankError(5, x.dim(), x.shape)
    B, T, H, P, R = x.shape
    if inputs.b.dim() != 5:
        raise RankError(5, inputs.b.dim(), inputs.b.shape)
    N = inputs.b.shape[3]
    code = _dtype_code(x)
    b, c = _dev(inputs.b, "b"), _dev(inputs.c, "c")
    _expect_shape(b, (B, T, H, N, R), "b")
    _expect_shape(c, (B, T, H, N, R), "c")
    dt, lam, a_log = _f32(inputs.dt, "dt"), _f32(inputs.lam, "lambda"), _f32(inputs.a_log, "a_log")
    _expect_shape(dt, (B, T, H), "dt")
    _expect_shape(lam, (B, T, H), "lambda")
    _expect_shape(a_log, (H,), "a_log")
    theta = None if inputs.theta is None else _dev(inputs.theta, "theta").to(x.dtype)
    if theta is not None:
        _expect_shape(theta, (B, T, H, N // 2), "theta")
    d_skip = _f32(inputs.d_skip, "d_skip")
    if d_skip is not None:
        _expect_shape(d_skip, (H,), "d_skip")
    dy = _dev(dy, "dy").to(x.dtype)
    _expect_shape(dy, (B, T, H, P, R), "dy")
    dh = _f32(dh, "dh")
    if dh is not None:
        _expect_shape(dh, (B, H, P, N), "dh")
    dlast_u = _f32(dlast_u, "dlast_u")
    if dlast_u is not None:
        _expect_shape(dlast_u, (B, H, P, N), "dlast_u")
    dangle = _f32(dangle, "dangle") if theta is not None else None
    if dangle is not None:
        _expect_shape(dangle, (B, H, N // 2), "dangle")
    st = inputs.state
    st_c, h0, l0, a0 = None, None, None, None
    if st is not None:
        h0, l0 = _f32(st.h, "state.h"), _f32(st.last_u, "state.last_u")
        _expect_shape(h0, (B, H, P, N), "state.h")
        _expect_shape(l0, (B, H, P, N), "state.last_u")
        a0 = _f32(st.angle, "state.angle") if (st.angle is not None and theta is not None) else None
        if a0 is not None:
            _expect_shape(a0, (B, H, N // 2), "state.angle")
        st_c = _lib.SsmStateC(h0.data_ptr(), l0.data_ptr(), None if a0 is None else a0.data_ptr())
    cin = _lib.ScanInputsC(
        B, T, H, P, N, R, code, x.data_ptr(), b.data_ptr(), c.data_ptr(), dt.data_ptr(),
        a_log.data_ptr(), lam.data_ptr(), None if theta is None else theta.data_ptr(),
        None if d_skip is None else d_skip.data_ptr(),
        C.pointer(st_c) if st_c is not None else None, int(inputs.chunk_size), 0, None, 0)
    need = int(_lib.lib().m3_scan_backward_workspace_bytes(C.byref(cin)))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    cin.workspace, cin.workspace_bytes = ws.data_ptr(), ws.numel()
    f32 = lambda *shape: torch.empty(shape, dtype=torch.float32, device=x.device)
    g = ScanGrads(torch.empty_like(x), torch.empty_like(b), torch.empty_like(c), f32(B, T, H),
                  f32(H), f32(B, T, H), None if theta is None else torch.empty_like(theta),
                  None if d_skip is None else f32(H), None if st is None else f32(B, H, P, N),
                  None if st is None else f32(B, H, P, N), None if a0 is None else f32(B, H, N // 2))
    gc = _lib.ScanGradsC(dy.data_ptr(), _ptr(dh), _ptr(dangle), g.x.data_ptr(), g.b.data_ptr(),
                         g.c.data_ptr(), g.dt.data_ptr(), g.lam.data_ptr(), g.a_log.data_ptr(),
                         _ptr(g.theta), _ptr(g.d_skip), _ptr(g.h0), _ptr(g.last_u0),
                         _ptr(g.angle0), _ptr(dlast_u))
    _lib.check(_lib.lib().m3_scan_backward(C.byref(cin), C.byref(gc), _stream(x)))
    return g


def mamba3_scan_gated(inputs: ScanInputs, z: torch.Tensor) -> ScanOutput:
    """mamba3_scan followed by the mixer's gate (mamba3.rs:468-477, no
    post-gate norm): the returned y is bf16(y) * silu(z).  z holds B*T rows
    whose first H*P*R columns are the gate (e.g. the in_proj output, z its
    leading columns).  theta may be a view of rows at a token stride (the
    in_proj output's last H*N/2 columns): the kernels read it in place.
    Inference only: no autograd node."""
    return _scan_forward(inputs, z)


def _theta_rows(theta: torch.Tensor, B: int, T: int, H: int, NH: int) -> int:
    """The token stride (elements) of a bf16 [B, T, H, NH] theta whose tokens'
    rows are contiguous and evenly spaced, as a view into wider rows is;
    0 for anything else (then it is made contiguous)."""
    if (theta.dtype != torch.bfloat16 or theta.dim() != 4 or tuple(theta.shape) != (B, T, H, NH)
            or theta.is_contiguous()):
        return 0
    st = theta.stride()
    if st[3] != 1 or st[2] != NH or st[1] < H * NH or (B > 1 and st[0] != T * st[1]):
        return 0
    return st[1]


def _scan_forward(inputs: ScanInputs, gate: Optional[torch.Tensor] = None) -> ScanOutput:
    x = inputs.x
    if x.dim() != 5:
        raise RankError(5, x.dim(), x.shape)
    B, T, H, P, R = x.shape
    if inputs.b.dim() != 5:
        raise RankError(5, inputs.b.dim(), inputs.b.shape)
    N = inputs.b.shape[3]
    code = _dtype_code(x)
    x = _dev(x, "x")
    b = _dev(inputs.b, "b")
    c = _dev(inputs.c, "c")
    for t, what in ((b, "b"), (c, "c")):
        if t.dtype != x.dtype:
            raise ShapeError(f"shape error: {what} is {t.dtype} but x is {x.dtype}")
    _expect_shape(b, (B, T, H, N, R), "b")
    _expect_shape(c, (B, T, H, N, R), "c")
    dt = _f32(inputs.dt, "dt")
    lam = _f32(inputs.lam, "lambda")
    a_log = _f32(inputs.a_log, "a_log")
    _expect_shape(dt, (B, T, H), "dt")
    _expect_shape(lam, (B, T, H), "lambda")
    _expect_shape(a_log, (H,), "a_log")
    theta = None
    theta_stride = 0
    if inputs.theta is not None and gate is not None and inputs.theta.is_cuda and N % 2 == 0:
        theta_stride = _theta_rows(inputs.theta, B, T, H, N // 2)
        if theta_stride and x.dtype == torch.bfloat16:
            theta = inputs.theta
    if inputs.theta is not None and theta is None:
        theta_stride = 0
        theta = _dev(inputs.theta, "theta")
        if theta.dtype != x.dtype:
            theta = theta.to(x.dtype)
        if N % 2 == 0:
            _expect_shape(theta, (B, T, H, N // 2), "theta")
    d_skip = _f32(inputs.d_skip, "d_skip")
    if d_skip is not None:
        _expect_shape(d_skip, (H,), "d_skip")
    st = inputs.state
    st_c = None
    keep = []
    if st is not None:
        h0, l0 = _f32(st.h, "state.h"), _f32(st.last_u, "state.last_u")
        _expect_shape(h0, (B, H, P, N), "state.h")
        _expect_shape(l0, (B, H, P, N), "state.last_u")
        a0 = _f32(st.angle, "state.angle") if (st.angle is not None and theta is not None) else None
        keep += [h0, l0, a0]
        st_c = _lib.SsmStateC(h0.data_ptr(), l0.data_ptr(),
                              None if a0 is None else a0.data_ptr())

    y = torch.empty_like(x)
    out_state = None
    if inputs.want_state:
        out_state = SsmState(
            torch.empty((B, H, P, N), dtype=torch.float32, device=x.device),
            torch.empty((B, H, P, N), dtype=torch.float32, device=x.device),
            torch.empty((B, H, N // 2), dtype=torch.float32, device=x.device)
            if theta is not None else None)
    cin = _lib.ScanInputsC(
        B, T, H, P, N, R, code, x.data_ptr(), b.data_ptr(), c.data_ptr(), dt.data_ptr(),
        a_log.data_ptr(), lam.data_ptr(), None if theta is None else theta.data_ptr(),
        None if d_skip is None else d_skip.data_ptr(),
        C.pointer(st_c) if st_c is not None else None,
        int(inputs.chunk_size), int(bool(inputs.want_state)), None, 0)
    ws = None
    if inputs.chunk_parallel:
        need = int(_lib.lib().m3_scan_workspace_bytes(C.byref(cin)))
        if need > 0:
            # stream-ordered by torch's caching allocator: freed after this
            # call's kernels, reused by later work on the same stream
            ws = torch.empty(need, dtype=torch.uint8, device=x.device)
            cin.workspace = ws.data_ptr()
            cin.workspace_bytes = need
    cout = _lib.ScanOutputC(y.data_ptr(), out_state._c() if out_state else _lib.SsmStateC())
    if gate is None:
        _lib.check(_lib.lib().m3_scan(C.byref(cin), C.byref(cout), _stream(x)))
    else:
        zt = _dev(gate, "z")
        if zt.dtype != torch.bfloat16 or zt.stride(-1) != 1 or zt.dim() < 2:
            raise ShapeError("shape error: z must be bf16 rows with unit column stride")
        rows = zt.numel() // zt.shape[-1] if zt.is_contiguous() else None
        if rows != B * T or zt.shape[-1] < H * P * R:
            raise ShapeError(f"shape error: z must hold {B * T} rows of at least {H * P * R} columns, "
                             f"got {tuple(zt.shape)}")
        st = _lib.lib().m3_scan_gated(C.byref(cin), C.byref(cout), zt.data_ptr(), zt.shape[-1],
                                      theta_stride, _stream(x))
        if st == _lib.M3_ERR_UNSUPPORTED and theta_stride:
            # a shape the kernels that read theta in place do not cover (the
            # call checks this before any launch): theta made contiguous
            theta = theta.contiguous()
            cin.theta = theta.data_ptr()
            st = _lib.lib().m3_scan_gated(C.byref(cin), C.byref(cout), zt.data_ptr(),
                                          zt.shape[-1], 0, _stream(x))
        _lib.check(st)
    return ScanOutput(y, out_state)


def ssd_chunked(x, b, c, a, g, w, initial_state=None, chunk_size=64,
                want_state=True) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """scan.rs:98-291: x [B,T,H,P]; b, c [B,T,H,N]; a, g, w [B,T,H]."""
    if x.dim() != 4:
        raise RankError(4, x.dim(), x.shape)
    if b.dim() != 4:
        raise RankError(4, b.dim(), b.shape)
    B, T, H, P = x.shape
    N = b.shape[3]
    code = _dtype_code(x)
    x, b, c = _dev(x, "x"), _dev(b, "b"), _dev(c, "c")
    _expect_shape(b, (B, T, H, N), "b")
    _expect_shape(c, (B, T, H, N), "c")
    a, g, w = _f32(a, "a"), _f32(g, "g"), _f32(w, "w")
    for t, what in ((a, "a"), (g, "g"), (w, "w")):
        _expect_shape(t, (B, T, H), what)
    init = _f32(initial_state, "initial_state")
    if init is not None:
        _expect_shape(init, (B, H, P, N), "initial_state")
    y = torch.empty_like(x)
    fs = torch.empty((B, H, P, N), dtype=torch.float32, device=x.device) if want_state else None
    args = _lib.SsdArgsC(B, T, H, P, N, code, x.data_ptr(), b.data_ptr(), c.data_ptr(),
                         a.data_ptr(), g.data_ptr(), w.data_ptr(),
                         None if init is None else init.data_ptr(), int(chunk_size),
                         int(bool(want_state)))
    _lib.check(_lib.lib().m3_ssd_chunked(C.byref(args), C.c_void_p(y.data_ptr()),
                                         _ptr(fs), _stream(x)))
    return y, fs


def _step_args(x, b, c, dt, lam, a_log, theta, d_skip):
    if x.dim() != 4:
        raise RankError(4, x.dim(), x.shape)
    B, H, P, R = x.shape
    N = b.shape[2]
    code = _dtype_code(x)
    x, b, c = _dev(x, "x"), _dev(b, "b"), _dev(c, "c")
    _expect_shape(b, (B, H, N, R), "b")
    _expect_shape(c, (B, H, N, R), "c")
    dt, lam, a_log = _f32(dt, "dt"), _f32(lam, "lambda"), _f32(a_log, "a_log")
    _expect_shape(dt.reshape(-1), (B * H,), "dt")
    _expect_shape(lam.reshape(-1), (B * H,), "lambda")
    _expect_shape(a_log, (H,), "a_log")
    if theta is not None:
        theta = _dev(theta, "theta")
        if theta.dtype != x.dtype:
            theta = theta.to(x.dtype)
        _expect_shape(theta.reshape(-1), (B * H * (N // 2),), "theta")
    d_skip = _f32(d_skip, "d_skip")
    if d_skip is not None:
        _expect_shape(d_skip, (H,), "d_skip")
    keep = (x, b, c, dt, lam, a_log, theta, d_skip)
    args = _lib.StepInputsC(B, H, P, N, R, code, x.data_ptr(), b.data_ptr(), c.data_ptr(),
                            dt.data_ptr(), lam.data_ptr(), a_log.data_ptr(),
                            None if theta is None else theta.data_ptr(),
                            None if d_skip is None else d_skip.data_ptr())
    return args, keep


def check_step_state(keep, rotational: bool, state) -> None:
    """The checks every in-place step runs on its state before a launch: h
    (and last_u, or the factored cache's x_prev / b_prev in the inputs'
    dtype) contiguous device tensors of the step inputs' [B, H, P, N] (x
    [B, H, P, R], b [B, H, N, R]) shape, and the angle when theta is given.
    keep is _step_args' tensors (x, b, ...)."""
    B, H, P, R = keep[0].shape
    N = keep[1].shape[2]
    t = state.h
    if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
        raise ArgumentError("state.h must be a contiguous float32 device tensor")
    _expect_shape(t, (B, H, P, N), "state.h")
    if isinstance(state, SsmStateFactored):
        for t, shape, what in ((state.x_prev, (B, H, P, R), "state.x_prev"),
                               (state.b_prev, (B, H, N, R), "state.b_prev")):
            if t.dtype != keep[0].dtype or not t.is_contiguous() or not t.is_cuda:
                raise ArgumentError(f"{what} must be a contiguous {keep[0].dtype} device tensor")
            _expect_shape(t, shape, what)
    else:
        t = state.last_u
        if t is None or t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
            raise ArgumentError("state.last_u must be a contiguous float32 device tensor")
        _expect_shape(t, (B, H, P, N), "state.last_u")
    if rotational:
        if state.angle is None:
            raise ArgumentError("theta needs the state's angle tensor (updated in place)")
        a = state.angle
        if a.dtype != torch.float32 or not a.is_contiguous() or not a.is_cuda:
            raise ArgumentError("state.angle must be a contiguous float32 device tensor")
        _expect_shape(a, (B, H, N // 2), "state.angle")


def mamba3_step_(x, b, c, dt, lam, a_log, theta, d_skip, state: SsmState) -> torch.Tensor:
    """mamba3_step with the state updated IN PLACE (the C ABI's semantics); returns y."""
    args, keep = _step_args(x, b, c, dt, lam, a_log, theta, d_skip)
    check_step_state(keep, theta is not None, state)
    y = torch.empty_like(keep[0])
    st_c = state._c()
    _lib.check(_lib.lib().m3_step(C.byref(args), C.byref(st_c), C.c_void_p(y.data_ptr()),
                                  _stream(keep[0])))
    return y


@dataclass
class SsmStateFactored:
    """The decode cache with last_u factored (m3_ssm_state_factored; no
    reference counterpart).  last_u is always the last token's outer product
    sum_r x_r B~_r^T (scan.rs:599-618, 683-691), so the state keeps that
    token's x [B, H, P, R] and unrotated b [B, H, N, R] (in the inputs'
    dtype) with h and the angle, and a step streams h alone."""
    h: torch.Tensor
    x_prev: torch.Tensor
    b_prev: torch.Tensor
    angle: Optional[torch.Tensor] = None

    @staticmethod
    def zeros(batch, heads, head_dim, d_state, rank, rotational, device,
              dtype=torch.bfloat16) -> "SsmStateFactored":
        return SsmStateFactored(
            torch.zeros((batch, heads, head_dim, d_state), dtype=torch.float32, device=device),
            torch.zeros((batch, heads, head_dim, rank), dtype=dtype, device=device),
            torch.zeros((batch, heads, d_state, rank), dtype=dtype, device=device),
            torch.zeros((batch, heads, d_state // 2), dtype=torch.float32, device=device)
            if rotational else None)

    @staticmethod
    def after_window(inputs: "ScanInputs", out: "ScanOutput") -> "SsmStateFactored":
        """The factored state a window leaves: the scan's h and angle, and
        the window's last x and b (copies)."""
        st = out.state
        return SsmStateFactored(st.h, inputs.x[:, -1].contiguous(), inputs.b[:, -1].contiguous(),
                                st.angle)

    def clone(self) -> "SsmStateFactored":
        return SsmStateFactored(self.h.clone(), self.x_prev.clone(), self.b_prev.clone(),
                                None if self.angle is None else self.angle.clone())

    def to_full(self) -> SsmState:
        """The reference-format SsmState this stands for (m3_state_unfactor
        forms last_u = x_prev (R(-angle) b_prev)^T; h and the angle are
        shared, not copied)."""
        B, H, P, N = self.h.shape
        R = self.x_prev.shape[-1]
        last_u = torch.empty_like(self.h)
        _lib.check(_lib.lib().m3_state_unfactor(
            B, H, P, N, R, _dtype_code(self.x_prev), self.x_prev.data_ptr(),
            self.b_prev.data_ptr(), None if self.angle is None else self.angle.data_ptr(),
            last_u.data_ptr(), _stream(self.h)))
        return SsmState(self.h, last_u, self.angle)


def mamba3_step_factored_(x, b, c, dt, lam, a_log, theta, d_skip,
                          state: SsmStateFactored) -> torch.Tensor:
    """mamba3_step on the factored cache, in place (m3_step_factored);
    returns y.  Equal to mamba3_step_ on the full state it stands for."""
    args, keep = _step_args(x, b, c, dt, lam, a_log, theta, d_skip)
    check_step_state(keep, theta is not None, state)
    y = torch.empty_like(keep[0])
    st_c = _lib.SsmStateFactoredC(state.h.data_ptr(), state.x_prev.data_ptr(),
                                  state.b_prev.data_ptr(),
                                  None if theta is None else state.angle.data_ptr())
    _lib.check(_lib.lib().m3_step_factored(C.byref(args), C.byref(st_c), C.c_void_p(y.data_ptr()),
                                           _stream(keep[0])))
    return y


def mamba3_step(x, b, c, dt, lam, a_log, theta, d_skip,
                state: SsmState) -> Tuple[torch.Tensor, SsmState]:
    """scan.rs:640-712: one decoding step; returns (y, new SsmState) like the reference."""
    new = state.clone()
    if theta is not None and new.angle is None:
        B, H = x.shape[0], x.shape[1]
        new.angle = torch.zeros((B, H, b.shape[2] // 2), dtype=torch.float32, device=x.device)
    y = mamba3_step_(x, b, c, dt, lam, a_log, theta, d_skip, new)
    if theta is None:
        new.angle = None
    return y, new


def shift_left(x: torch.Tensor, axis: int) -> torch.Tensor:
    """scan.rs:59-75: shift towards smaller indices along `axis`, zero-filling the end."""
    n = x.shape[axis]
    if n == 0:
        return x.clone()
    out = torch.zeros_like(x)
    if n > 1:
        out.narrow(axis, 0, n - 1).copy_(x.narrow(axis, 1, n - 1))
    return out
