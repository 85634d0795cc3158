"""m3_scan_no_alloc (the allocation-free m3_scan over the library's static
device scratch) against m3_scan with a caller workspace, through the C ABI.

Both run the same chunk-parallel kernels, so every output must agree bit for
bit.  Two calls in a row, the second on a smaller input, check that the
scratch left by the first call does not leak into the second.
"""
import ctypes as C

import pytest
import torch

DEV = "cuda:0"


def _inputs(seed, B, L, H, N, R, dtype, rot=True, skip=True, state=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    P = 64
    x = torch.randn((B, L, H, P, R), generator=g, device=DEV).to(dtype)
    b = (torch.randn((B, L, H, N, R), generator=g, device=DEV) / N ** 0.5).to(dtype)
    c = (torch.randn((B, L, H, N, R), generator=g, device=DEV) / N ** 0.5).to(dtype)
    dt = torch.nn.functional.softplus(torch.randn((B, L, H), generator=g, device=DEV) - 3.0)
    dt = dt.clamp(1e-3, 0.1)
    a_log = torch.rand((H,), generator=g, device=DEV) * 2.772588722
    lam = torch.sigmoid(torch.randn((B, L, H), generator=g, device=DEV))
    theta = (torch.rand((B, L, H, N // 2), generator=g, device=DEV) * 3.14159).to(dtype) if rot else None
    d_skip = torch.randn((H,), generator=g, device=DEV) if skip else None
    st = None
    if state:
        st = (0.1 * torch.randn((B, H, P, N), generator=g, device=DEV),
              0.1 * torch.randn((B, H, P, N), generator=g, device=DEV),
              (torch.rand((B, H, N // 2), generator=g, device=DEV) - 0.5) * 6.0 if rot else None)
    return dict(B=B, L=L, H=H, P=P, N=N, R=R, dtype=dtype, x=x, b=b, c=c, dt=dt, a_log=a_log,
                lam=lam, theta=theta, d_skip=d_skip, state=st)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _call(inp, no_alloc):
    """One scan through the C ABI; returns (y, h, last_u, angle, workspace bytes)."""
    from mamba3 import _lib
    L = _lib.lib()
    B, T, H, P, N, R = (inp[k] for k in ("B", "L", "H", "P", "N", "R"))
    dt_code = _lib.M3_BF16 if inp["dtype"] == torch.bfloat16 else _lib.M3_F32
    keep = []
    st_c = None
    if inp["state"] is not None:
        h0, u0, a0 = inp["state"]
        st_c = _lib.SsmStateC(h0.data_ptr(), u0.data_ptr(), _ptr(a0))
        keep.append(st_c)
    cin = _lib.ScanInputsC(B, T, H, P, N, R, dt_code, inp["x"].data_ptr(), inp["b"].data_ptr(),
                           inp["c"].data_ptr(), inp["dt"].data_ptr(), inp["a_log"].data_ptr(),
                           inp["lam"].data_ptr(), _ptr(inp["theta"]), _ptr(inp["d_skip"]),
                           C.pointer(st_c) if st_c is not None else None, 64, 1, None, 0)
    need = int(L.m3_scan_workspace_bytes(C.byref(cin)))
    ws = None
    if not no_alloc and need > 0:
        ws = torch.empty(need + 256, dtype=torch.uint8, device=DEV)
        off = (-ws.data_ptr()) % 256
        cin.workspace = ws.data_ptr() + off
        cin.workspace_bytes = need
    y = torch.full((B, T, H, P, R), float("nan"), device=DEV).to(inp["dtype"])
    h = torch.full((B, H, P, N), float("nan"), device=DEV)
    u = torch.full((B, H, P, N), float("nan"), device=DEV)
    ang = torch.full((B, H, N // 2), float("nan"), device=DEV) if inp["theta"] is not None else None
    cout = _lib.ScanOutputC(y.data_ptr(), _lib.SsmStateC(h.data_ptr(), u.data_ptr(), _ptr(ang)))
    stream = torch.cuda.current_stream().cuda_stream
    fn = L.m3_scan_no_alloc if no_alloc else L.m3_scan
    _lib.check(fn(C.byref(cin), C.byref(cout), stream))
    torch.cuda.synchronize()
    return y, h, u, ang, need


def _same(a, b):
    if a is None or b is None:
        return a is None and b is None
    return torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_no_alloc_matches_the_workspace_scan_on_two_calls(dtype):
    # the second input is smaller: stale scratch from the first call must not
    # reach its outputs
    # f32 keeps U and S in f32 over 32-row chunks: four times the bf16 scratch
    # per token, so its first case is shorter to stay within the 32 MiB
    first = _inputs(71, B=2, L=700 if dtype == torch.bfloat16 else 330, H=12, N=128, R=1,
                    dtype=dtype)
    second = _inputs(72, B=1, L=130, H=8, N=128, R=1, dtype=dtype, skip=False)
    for inp in (first, second):
        print(f"no-alloc case B={inp['B']} L={inp['L']} H={inp['H']} N={inp['N']} {inp['dtype']}",
              flush=True)
        ref = _call(inp, no_alloc=False)
        got = _call(inp, no_alloc=True)
        assert ref[4] > 0, "the case must take the chunk-parallel path (which uses the scratch)"
        assert ref[4] <= 32 << 20
        for name, r, g in zip(("y", "h", "last_u", "angle"), ref[:4], got[:4]):
            assert _same(r, g), name
        assert torch.isfinite(got[0].float()).all()


@pytest.mark.gpu
def test_no_alloc_mimo_and_real_dynamics():
    inp = _inputs(73, B=2, L=256, H=6, N=64, R=4, dtype=torch.bfloat16, rot=False, state=False)
    ref = _call(inp, no_alloc=False)
    got = _call(inp, no_alloc=True)
    assert ref[4] > 0
    for name, r, g in zip(("y", "h", "last_u"), ref[:3], got[:3]):
        assert _same(r, g), name


@pytest.mark.gpu
def test_no_alloc_refuses_an_overlapping_call_on_another_stream():
    """Two eager calls on different streams would share the GPU's scratch: the
    second is refused with M3_ERR_ARGUMENT while the first may still run (here
    it is queued behind a long product on its stream), and accepted once the
    first has finished; the accepted call gives the workspace scan's bytes."""
    from mamba3 import _lib
    L = _lib.lib()
    inp = _inputs(31, 2, 512, 4, 128, 1, torch.bfloat16)
    B, T, H, P, N, R = (inp[k] for k in ("B", "L", "H", "P", "N", "R"))
    st_c = _lib.SsmStateC(inp["state"][0].data_ptr(), inp["state"][1].data_ptr(),
                          _ptr(inp["state"][2]))
    cin = _lib.ScanInputsC(B, T, H, P, N, R, _lib.M3_BF16, inp["x"].data_ptr(),
                           inp["b"].data_ptr(), inp["c"].data_ptr(), inp["dt"].data_ptr(),
                           inp["a_log"].data_ptr(), inp["lam"].data_ptr(), _ptr(inp["theta"]),
                           _ptr(inp["d_skip"]), C.pointer(st_c), 64, 1, None, 0)
    assert L.m3_scan_workspace_bytes(C.byref(cin)) > 0   # the scratch is used
    y = torch.empty((B, T, H, P, R), device=DEV, dtype=torch.bfloat16)
    h, u = torch.empty((B, H, P, N), device=DEV), torch.empty((B, H, P, N), device=DEV)
    ang = torch.empty((B, H, N // 2), device=DEV)
    cout = _lib.ScanOutputC(y.data_ptr(), _lib.SsmStateC(h.data_ptr(), u.data_ptr(), ang.data_ptr()))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        m = torch.randn(4096, 4096, device=DEV)
        for _ in range(24):
            m = torch.mm(m, m) * 1e-3
    assert L.m3_scan_no_alloc(C.byref(cin), C.byref(cout), C.c_void_p(s1.cuda_stream)) == _lib.M3_OK
    assert L.m3_scan_no_alloc(C.byref(cin), C.byref(cout),
                              C.c_void_p(s2.cuda_stream)) == _lib.M3_ERR_ARGUMENT
    assert b"another stream" in L.m3_last_error()
    torch.cuda.synchronize()
    y.fill_(float("nan"))
    assert L.m3_scan_no_alloc(C.byref(cin), C.byref(cout), C.c_void_p(s2.cuda_stream)) == _lib.M3_OK
    torch.cuda.synchronize()
    ref = _call(inp, False)
    assert torch.equal(y, ref[0]) and torch.equal(h, ref[1]) and torch.equal(u, ref[2])
