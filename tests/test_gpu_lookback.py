"""GPU checks specific to the single-launch look-back scan (the opt-in
chunk-parallel path for bf16 storage, M3_SCAN_CHUNKED=lookback): its control
words, forced aggregate folding, agreement with the three-launch form and the
single pass, and repeated calls on one workspace.

Parity bar as for every bf16 scan: rel-L2 <= 1e-2 against the f64 recurrence
on the same bf16-rounded inputs.  The look-back takes a predecessor's prefix
or folds its aggregate depending on timing, so two runs differ by f32
rounding (then bf16 rounding of y): run-to-run agreement is checked at 2e-3.
"""
import ctypes as C
import math
import os

import numpy as np
import pytest
import torch

import oracle
from cases import baseline_inputs, rel_l2
from gpu_util import dev, host, oracle_scan, run_scan

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
RUN_TOL = 2e-3


def _inputs(B, T, H, N, R, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    P = 64
    bf = torch.bfloat16
    x = torch.randn(B, T, H, P, R, device="cuda", generator=g).to(bf)
    b = (torch.randn(B, T, H, N, R, device="cuda", generator=g) / math.sqrt(N)).to(bf)
    c = (torch.randn(B, T, H, N, R, device="cuda", generator=g) / math.sqrt(N)).to(bf)
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=g) - 3
                                      ).clamp(1e-3, 0.1)
    lam = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g))
    a_log = torch.rand(H, device="cuda", generator=g) * math.log(16)
    th = (torch.rand(B, T, H, N // 2, device="cuda", generator=g) * math.pi).to(bf)
    return x, b, c, dt, lam, a_log, th


@pytest.fixture(autouse=True)
def _lookback(monkeypatch):
    monkeypatch.setenv("M3_SCAN_CHUNKED", "lookback")


def _scan_c(x, b, c, dt, lam, a_log, th, ws=None):
    """m3_scan through the C structs with an explicit workspace (or none)."""
    from mamba3 import _lib
    B, T, H, P, R = x.shape
    N = b.shape[3]
    y = torch.empty_like(x)
    h = torch.empty(B, H, P, N, device="cuda")
    lu = torch.empty(B, H, P, N, device="cuda")
    ang = torch.empty(B, H, N // 2, device="cuda")
    cin = _lib.ScanInputsC(B, T, H, P, N, R, _lib.M3_BF16, x.data_ptr(), b.data_ptr(),
                           c.data_ptr(), dt.data_ptr(), a_log.data_ptr(), lam.data_ptr(),
                           th.data_ptr(), None, None, 64, 1, None, 0)
    if ws is not None:
        cin.workspace, cin.workspace_bytes = ws.data_ptr(), ws.numel()
    cout = _lib.ScanOutputC(y.data_ptr(), _lib.SsmStateC(h.data_ptr(), lu.data_ptr(),
                                                         ang.data_ptr()))
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.lib().m3_scan(C.byref(cin), C.byref(cout), C.c_void_p(stream)))
    torch.cuda.synchronize()
    return y, h, lu, ang


def _workspace(x, b, th):
    from mamba3 import _lib
    B, T, H, P, R = x.shape
    N = b.shape[3]
    cin = _lib.ScanInputsC(B, T, H, P, N, R, _lib.M3_BF16, x.data_ptr(), b.data_ptr(),
                           b.data_ptr(), None, None, None, th.data_ptr(), None, None, 64, 1,
                           None, 0)
    need = int(_lib.lib().m3_scan_workspace_bytes(C.byref(cin)))
    assert need > 0
    return torch.zeros(need, dtype=torch.uint8, device="cuda")


def _check_against_f64(inp, out, pairs):
    x, b, c, dt, lam, a_log, th = inp
    y, h, lu, ang = out
    for bb, hh in pairs:
        sl = lambda t: host(t[bb:bb + 1, :, hh:hh + 1])
        y64, h64, lu64, _ = oracle.scan_recurrence_f64(
            sl(x), sl(b), sl(c), sl(dt), host(a_log[hh:hh + 1]), sl(lam), sl(th))
        assert rel_l2(host(y[bb:bb + 1, :, hh:hh + 1]), y64) <= BF16_TOL
        assert rel_l2(host(h[bb:bb + 1, hh:hh + 1]), h64) <= BF16_TOL
        assert rel_l2(host(lu[bb:bb + 1, hh:hh + 1]), lu64) <= BF16_TOL


@pytest.mark.parametrize("N,R,T", [(128, 1, 1000), (64, 1, 640), (128, 4, 300), (64, 2, 257)])
def test_control_words_and_repeat_calls(N, R, T):
    """Every workgroup took exactly one ticket, no wait was abandoned, and three
    calls on one workspace agree with each other and with the recurrence."""
    B, H = 3, 5
    inp = _inputs(B, T, H, N, R, seed=11 + N + R)
    x, b, c, dt, lam, a_log, th = inp
    ws = _workspace(x, b, th)
    qt = 64 // R
    bhk = B * H * ((T + qt - 1) // qt)
    outs = []
    for _ in range(3):
        outs.append(_scan_c(*inp, ws=ws))
        ctl = ws[:8].cpu().numpy().view(np.uint32)
        assert int(ctl[0]) == bhk, ("tickets", int(ctl[0]), bhk)
        assert int(ctl[1]) == 0, ("abandoned waits", int(ctl[1]))
    for o in outs[1:]:
        for a_, b_ in zip(o, outs[0]):
            assert rel_l2(host(a_), host(b_)) <= RUN_TOL
    _check_against_f64(inp, outs[0], ((0, 0), (B - 1, H - 1), (1, 2)))


@pytest.mark.parametrize("fold", [1, 2, 5, 1000])
def test_forced_aggregate_folds(fold, monkeypatch):
    """Every chunk folds at least `fold` predecessor aggregates before it uses a
    prefix (1000: all the way back to chunk 0): the fold algebra
    G o T_j = (R(Theta + Phi_j) E e_j, V + E R(Theta + Phi_j) U_j) gives the
    same scan as the chained prefixes."""
    B, H, T, N, R = 2, 3, 1500, 128, 1
    inp = _inputs(B, T, H, N, R, seed=5)
    x, b, c, dt, lam, a_log, th = inp
    ws = _workspace(x, b, th)
    base = _scan_c(*inp, ws=ws)
    monkeypatch.setenv("M3_SCAN_LOOKBACK_FOLD", str(fold))
    out = _scan_c(*inp, ws=ws)
    monkeypatch.delenv("M3_SCAN_LOOKBACK_FOLD")
    ctl = ws[:8].cpu().numpy().view(np.uint32)
    assert int(ctl[1]) == 0
    for a_, b_ in zip(out, base):
        assert rel_l2(host(a_), host(b_)) <= RUN_TOL
    _check_against_f64(inp, out, ((0, 0), (1, 2)))


@pytest.mark.parametrize("N,R", [(128, 1), (128, 2), (64, 4)])
def test_lookback_matches_three_launches_and_single_pass(N, R, monkeypatch):
    B, H, T = 4, 6, 700
    inp = _inputs(B, T, H, N, R, seed=3 + R)
    x, b, c, dt, lam, a_log, th = inp
    look = _scan_c(*inp, ws=_workspace(x, b, th))
    monkeypatch.setenv("M3_SCAN_CHUNKED", "three")
    three = _scan_c(*inp, ws=_workspace(x, b, th))
    monkeypatch.setenv("M3_SCAN_CHUNKED", "lookback")
    single = _scan_c(*inp, ws=None)
    for o in (three, single):
        for a_, b_ in zip(look, o):
            assert rel_l2(host(a_), host(b_)) <= BF16_TOL
    _check_against_f64(inp, look, ((0, 0), (B - 1, H - 1)))


def test_carried_state_and_skip_through_the_lookback():
    """Incoming state (h, last_u, angle) and the skip path with many chunks."""
    rng = np.random.default_rng(77)
    inp = baseline_inputs(rng, 2, 900, 3, 64, 128, 1, theta=True, dtype="bf16",
                          theta_per_head=False, state=True)
    d_skip = rng.uniform(-1, 1, 3).astype(np.float32)
    st = (inp["h0"], inp["last_u0"], inp["angle0"])
    y, h, lu, ang = run_scan(inp, dtype=torch.bfloat16, skip=d_skip, state=st)
    y64, h64, lu64, ang64 = oracle_scan(inp, skip=d_skip, state=st)
    assert rel_l2(y, y64) <= BF16_TOL
    assert rel_l2(h, h64) <= BF16_TOL
    assert rel_l2(lu, lu64) <= BF16_TOL
    d = (ang - ang64 + math.pi) % (2 * math.pi) - math.pi
    assert float(np.max(np.abs(d))) <= 1e-3


def test_config1_full_size_against_three_launches(monkeypatch):
    """BASELINE config 1 at full size: the look-back scan and the three-launch
    form agree, and two sequences match the f64 recurrence."""
    inp = _inputs(8, 2048, 12, 128, 1, seed=0x4D414D43)
    x, b, c, dt, lam, a_log, th = inp
    ws = _workspace(x, b, th)
    look = _scan_c(*inp, ws=ws)
    ctl = ws[:8].cpu().numpy().view(np.uint32)
    assert int(ctl[0]) == 8 * 12 * 32 and int(ctl[1]) == 0
    monkeypatch.setenv("M3_SCAN_CHUNKED", "three")
    three = _scan_c(*inp, ws=_workspace(x, b, th))
    monkeypatch.setenv("M3_SCAN_CHUNKED", "lookback")
    for a_, b_ in zip(look, three):
        assert rel_l2(host(a_), host(b_)) <= BF16_TOL
    assert torch.isfinite(look[0].float()).all()
    _check_against_f64(inp, look, ((0, 0), (7, 11)))
