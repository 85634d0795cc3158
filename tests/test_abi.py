"""CPU checks of the C ABI: the library loads, exports every declared symbol,
and its host-only entry points (config validation, widths, argument checks
that fail before any device work) behave like the reference.  No GPU needed.
"""
import ctypes as C
import math
import os
import re

import pytest

from conftest import ROOT

HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared_symbols():
    syms = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        syms.update(re.findall(r"\b(m3_[a-z0-9_]+)\s*\(", text))
    return sorted(syms)


def test_library_exports_every_declared_symbol():
    from mamba3 import _lib
    L = _lib.lib()
    syms = declared_symbols()
    assert len(syms) >= 24
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding declares a signature for each of them
    assert set(syms) == set(_lib.SIGNATURES), set(syms) ^ set(_lib.SIGNATURES)


def test_status_strings():
    from mamba3 import _lib
    L = _lib.lib()
    assert L.m3_status_string(0) == b"M3_OK"
    assert L.m3_status_string(4) == b"M3_ERR_UNSUPPORTED"


def test_config_defaults_match_reference():
    """config.rs:130-156."""
    from mamba3.ssm import Discretization, SsmConfig, StateDynamics
    c = SsmConfig.default_from_abi()
    assert (c.d_model, c.n_heads, c.head_dim, c.d_state, c.n_groups) == (768, 24, 64, 64, 24)
    assert c.discretization == Discretization.LearnedTrapezoid
    assert c.dynamics == StateDynamics.Rotational
    assert c.mode.rank() == 1 and c.chunk_size == 64 and c.conv_kernel == 4
    assert c.bc_norm and c.bc_bias and not c.post_gate_norm and c.skip_connection
    assert math.isclose(c.dt_min, 0.001, rel_tol=1e-6) and math.isclose(c.dt_max, 0.1, rel_tol=1e-6)
    assert (c.a_init_min, c.a_init_max) == (1.0, 16.0)


def test_config_widths():
    """config.rs:164-200."""
    from mamba3.ssm import Discretization, SsmConfig, SsmMode, StateDynamics
    c = SsmConfig(n_heads=12, n_groups=12, head_dim=64, d_state=128, mode=SsmMode.mimo(4))
    assert c.d_inner() == 12 * 64 * 4
    assert c.bc_width() == 12 * 128 * 4
    assert c.theta_width() == 12 * 64
    assert c.lambda_width() == 12
    assert c.in_proj_width() == 2 * c.d_inner() + 2 * c.bc_width() + 12 + 12 + 12 * 64
    c.dynamics = StateDynamics.Real
    c.discretization = Discretization.Euler
    assert c.theta_width() == 0 and c.lambda_width() == 0
    assert Discretization.Euler.fixed_lambda() == 1.0
    assert Discretization.Trapezoid.fixed_lambda() == 0.5
    assert Discretization.LearnedTrapezoid.fixed_lambda() is None


@pytest.mark.parametrize("change,message", [
    (dict(d_state=0), "SSM dimensions must all be positive"),
    (dict(n_heads=6, n_groups=4), "n_heads (6) must be a multiple of n_groups (4)"),
    (dict(d_state=7), "d_state must be even, got 7"),
    (dict(chunk_size=0), "chunk_size must be positive"),
    (dict(mode="rank0"), "MIMO rank must be positive"),
    (dict(dt_min=0.2, dt_max=0.1), "expected 0 < dt_min < dt_max"),
    (dict(a_init_min=0.0), "expected 0 < a_init_min <= a_init_max"),
    (dict(conv_kernel=1), "conv_kernel must be at least 2"),
])
def test_config_validation_rules(change, message):
    """config.rs:203-245, rule by rule, with the reference's messages."""
    from mamba3 import ConfigError
    from mamba3.ssm import SsmConfig, SsmMode
    c = SsmConfig()
    for k, v in change.items():
        if v == "rank0":
            c.mode = SsmMode(0)
        else:
            setattr(c, k, v)
    with pytest.raises(ConfigError) as e:
        c.validate()
    assert message in str(e.value)
    assert str(e.value).startswith("invalid configuration: ")


def test_builder_expand_and_build():
    """config.rs:331-347."""
    from mamba3.ssm import SsmConfig
    c = SsmConfig.builder().d_model(256).head_dim(32).expand(2.0).build()
    assert c.n_heads == 16 and c.n_groups == 16


def _scan_inputs(**kw):
    from mamba3 import _lib
    base = dict(batch=1, seq=4, heads=1, head_dim=4, d_state=4, rank=1, dtype=0, x=None,
                b=None, c=None, dt=None, a_log=None, lambda_=None, theta=None, d_skip=None,
                state=None, chunk_size=4, want_state=0)
    base.update(kw)
    return _lib.ScanInputsC(**base)


@pytest.mark.parametrize("kw,status,message", [
    (dict(rank=0), 1, "MIMO rank must be positive"),
    (dict(d_state=5, theta=1), 1, "rotational dynamics require an even d_state"),
    (dict(head_dim=0), 1, "SSM dimensions must all be positive"),
    # beyond the scan kernels the scan runs on the step kernel, so only shapes
    # beyond that one's LDS are refused
    (dict(head_dim=20000), 4, "head_dim 20000, d_state 4 and rank 1 exceed both"),
    (dict(d_state=8192), 4, "d_state 8192 and rank 1 exceed both"),
    (dict(rank=2000, dtype=1), 4, "and rank 2000 exceed both"),
    (dict(dtype=7), 6, "unknown dtype"),
    (dict(want_state=1), 6, "want_state needs output h and last_u"),
])
def test_scan_argument_validation_before_device_work(kw, status, message):
    """Reference rules (scan.rs:462, 485-489; config.rs:203-245) rejected on the host."""
    from mamba3 import _lib
    L = _lib.lib()
    cin = _scan_inputs(**kw)
    cout = _lib.ScanOutputC()
    st = L.m3_scan(C.byref(cin), C.byref(cout), None)
    assert st == status, L.m3_last_error()
    assert message in L.m3_last_error().decode()


@pytest.mark.parametrize("kw,status,message", [
    (dict(rank=0), 1, "MIMO rank must be positive"),
    (dict(d_state=5, theta=1), 1, "rotational dynamics require an even d_state"),
    (dict(head_dim=20000), 4, "exceed both the scan kernels"),
    (dict(want_state=1), 6, "want_state needs output h and last_u"),
    (dict(x=None, seq=8), 6, "x, b, c, dt, a_log, lambda and y are required"),
])
def test_f16_storage_validates_before_any_copy(kw, status, message):
    """f16 storage (M3_F16) takes the same checks as f32 and bf16, all of them
    before its widening copies: a rejected call allocates and launches nothing
    (the pointers are stand-ins that are never dereferenced)."""
    from mamba3 import _lib
    L = _lib.lib()
    fake = 1 << 20
    args = dict(dtype=_lib.M3_F16, x=fake, b=fake, c=fake, dt=fake, a_log=fake, lambda_=fake)
    args.update(kw)
    cin = _scan_inputs(**args)
    before = L.m3_launch_count()
    st = L.m3_scan(C.byref(cin), C.byref(_lib.ScanOutputC()), None)
    assert st == status, L.m3_last_error()
    assert message in L.m3_last_error().decode()
    assert L.m3_launch_count() == before


def test_f16_storage_entry_points_that_do_not_take_it():
    """m3_scan_no_alloc (which may not allocate) and m3_scan_gated refuse f16
    storage before any device work; the workspace query sizes an f16 scan as
    the f32 one it runs."""
    from mamba3 import _lib
    L = _lib.lib()
    fake = 1 << 20
    before = L.m3_launch_count()
    cin = _lib.ScanInputsC(1, 64, 2, 64, 128, 1, _lib.M3_F16, fake, fake, fake, fake, fake, fake,
                           None, None, None, 64, 0, None, 0)
    cout = _lib.ScanOutputC(fake, _lib.SsmStateC())
    assert L.m3_scan_no_alloc(C.byref(cin), C.byref(cout), None) == _lib.M3_ERR_UNSUPPORTED
    assert b"f16" in L.m3_last_error()
    assert L.m3_scan_gated(C.byref(cin), C.byref(cout), fake, 128, 0, None) == _lib.M3_ERR_UNSUPPORTED
    assert L.m3_launch_count() == before
    q = lambda dt: L.m3_scan_workspace_bytes(C.byref(_lib.ScanInputsC(
        8, 2048, 12, 64, 128, 1, dt, None, None, None, None, None, None, None, None, None, 64, 1,
        None, 0)))
    assert q(_lib.M3_F16) == q(_lib.M3_F32) > 0


def test_no_alloc_refuses_shapes_beyond_the_scan_kernels():
    """Shapes beyond the scan kernels' tiles run token by token on the step
    kernel, with temporaries for the carried state when it is not wanted, so
    m3_scan_no_alloc refuses them before any device work."""
    from mamba3 import _lib
    L = _lib.lib()
    fake = 1 << 20
    before = L.m3_launch_count()
    for P, N, R in ((192, 64, 1), (64, 320, 1), (16, 16, 80)):
        cin = _lib.ScanInputsC(1, 64, 2, P, N, R, _lib.M3_F32, fake, fake, fake, fake, fake, fake,
                               None, None, None, 64, 0, None, 0)
        cout = _lib.ScanOutputC(fake, _lib.SsmStateC())
        assert L.m3_scan_no_alloc(C.byref(cin), C.byref(cout), None) == _lib.M3_ERR_UNSUPPORTED
        assert b"beyond the scan kernels" in L.m3_last_error()
        assert L.m3_scan_workspace_bytes(C.byref(cin)) == 0
    assert L.m3_launch_count() == before


def test_python_api_rejects_host_tensors():
    """The product path has no CPU fallback: host tensors fail loudly."""
    import torch
    from mamba3 import ArgumentError, RankError
    from mamba3.ssm import ScanInputs, mamba3_scan
    x = torch.zeros(1, 4, 1, 4, 1)
    b = torch.zeros(1, 4, 1, 4, 1)
    dt = torch.zeros(1, 4, 1)
    a_log = torch.zeros(1)
    with pytest.raises(ArgumentError, match="no CPU path"):
        mamba3_scan(ScanInputs(x, b, b, dt, a_log, dt))
    with pytest.raises(RankError):
        mamba3_scan(ScanInputs(x[..., 0], b, b, dt, a_log, dt))


def test_scan_workspace_query():
    """m3_scan_workspace_bytes: the chunk-parallel kernels cover head_dim 64,
    d_state 64/128, rank 1/2/4; other shapes run single-pass and need none."""
    import ctypes as C
    from mamba3 import _lib
    L = _lib.lib()

    def need(B, T, H, P, N, R, dtype, chunk=64):
        cin = _lib.ScanInputsC(B, T, H, P, N, R, dtype, None, None, None, None, None, None,
                               None, None, None, chunk, 1, None, 0)
        return int(L.m3_scan_workspace_bytes(C.byref(cin)))

    # bf16 at rank 1 runs the fused single launch: per segment of two 64-token
    # sub-chunks a flag (8 bytes), U (bf16 64 x 128), the decay, the angle
    # total / cosine / sine per pair (3 x 64 f32), the state after the segment
    # (f32 64 x 128) and its angle (64 f32), each section 256-byte aligned
    def fused(segs, n=128):
        a = lambda v: (v + 255) // 256 * 256
        return (a(segs * 8) + a(segs * 64 * n * 2) + a(segs * 4) + 3 * a(segs * n // 2 * 4)
                + a(segs * 64 * n * 4) + a(segs * n // 2 * 4))
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_BF16) == fused(8 * 12 * 16)
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_BF16, chunk=512) == fused(8 * 12 * 16)
    assert need(2, 700, 3, 64, 64, 1, _lib.M3_BF16) == fused(2 * 3 * 6, 64)
    # 192 sequences: the fused grid would take six rounds of two workgroups a
    # CU, so the three launches run (segments of 256 tokens; 75 % of a
    # single-pass round)
    three = 2 * 64 * 128 * 2 + 4 + 3 * 64 * 4
    assert need(16, 2048, 12, 64, 128, 1, _lib.M3_BF16) == 16 * 12 * 4 * three
    assert need(20, 2048, 12, 64, 128, 1, _lib.M3_BF16) == 0   # 240 sequences: single pass
    _lib.check(L.m3_debug_scan_options(1, 0, 0))   # the three launches everywhere
    try:
        _three_launch_sizes(need, _lib)
    finally:
        _lib.check(L.m3_debug_scan_options(0, 0, 0))
    from mamba3.error import ArgumentError
    with pytest.raises(ArgumentError):
        _lib.check(L.m3_debug_scan_options(2, 0, 0))
    assert need(1, 100, 2, 48, 128, 1, _lib.M3_BF16) == 0      # head_dim 48
    assert need(1, 100, 2, 64, 96, 1, _lib.M3_BF16) == 0       # d_state 96
    assert need(1, 100, 2, 64, 128, 3, _lib.M3_BF16) == 0      # rank 3
    assert need(1, 0, 2, 64, 128, 1, _lib.M3_BF16) == 0        # empty window


def _three_launch_sizes(need, _lib):
    # per segment: U and S (bf16 64x128 each), the segment decay, and angle
    # total / cosine / sine per pair (3 x 64 f32).  At config 1 (96 sequences
    # of 32 sub-chunks of 64 tokens) segments of 4 sub-chunks give 768
    # chunk_scan workgroups: one round of three per CU on the 256 CUs the
    # query assumes without a device
    record = 2 * 64 * 128 * 2 + 4 + 3 * 64 * 4
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_BF16) == 8 * 12 * 8 * record
    # chunk_size is the shortest segment: 512 tokens -> 4 segments per sequence
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_BF16, chunk=512) == 8 * 12 * 4 * record
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_BF16, chunk=1) == 8 * 12 * 8 * record
    # f32 storage: 32-token sub-chunks, 8 per segment, and f32 U and S
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_F32) == 8 * 12 * 8 * (64 * 128 * 8 + 4 + 3 * 64 * 4)
    # bf16 rank 4 (config 2: 96 sequences of 256 sub-chunks of 16 tokens): one
    # round of three chunk_scan workgroups per CU, 768 segments of 32
    # sub-chunks, 8 per sequence
    assert need(4, 4096, 24, 64, 128, 4, _lib.M3_BF16) == 4 * 24 * 8 * record
    # rank 2 keeps six rounds of two per CU: 3072 segments of 4 sub-chunks of
    # 32 tokens
    assert need(4, 4096, 24, 64, 128, 2, _lib.M3_BF16) == 4 * 24 * 32 * record
    # the single pass runs one sequence per CU (256 CUs here, the CPU
    # fallback of the query): it is the faster form once its last round of
    # sequences fills 85 % of the CUs
    assert need(16, 2048, 12, 64, 128, 1, _lib.M3_BF16) == 8 * 12 * 2 * 4 * record  # 192: 75 %
    assert need(20, 2048, 12, 64, 128, 1, _lib.M3_BF16) == 0   # 240 sequences: 94 %
    assert need(14, 2048, 12, 64, 128, 1, _lib.M3_BF16) > 0    # 168
    assert need(24, 2048, 12, 64, 128, 1, _lib.M3_BF16) > 0    # 288: 1.13 rounds
    assert need(40, 2048, 12, 64, 128, 1, _lib.M3_BF16) == 0   # 480: 1.88 rounds


@pytest.mark.parametrize("kw,grads,status,message", [
    (dict(rank=0), {}, 1, "MIMO rank must be positive"),
    (dict(d_state=5, theta=1), {}, 1, "rotational dynamics require an even d_state"),
    (dict(dtype=7), {}, 6, "unknown dtype"),
    (dict(x=16, b=16, c=16, dt=16, a_log=16, lambda_=16), dict(dx=None), 6,
     "dy, dx, db, dc, ddt, dlambda and da_log are required"),
    (dict(x=16, b=16, c=16, dt=16, a_log=16, lambda_=16, theta=16, d_state=4), {}, 6,
     "dtheta is required"),
    (dict(x=16, b=16, c=16, dt=16, a_log=16, lambda_=16, head_dim=20000), {}, 4,
     "the scan backward covers shapes whose per-token vectors fit 64 KB"),
])
def test_scan_backward_argument_validation_before_device_work(kw, grads, status, message):
    """m3_scan_backward rejects bad arguments with the reference's rules and
    messages before any device work (the pointers here are never read)."""
    from mamba3 import _lib
    fields = dict(dy=16, dh=None, dangle=None, dx=16, db=16, dc=16, ddt=16, dlambda=16, da_log=16,
                  dtheta=None, dd_skip=None, dh0=None, dlast_u0=None, dangle0=None)
    fields.update(grads)
    g = _lib.ScanGradsC(**fields)
    st = _lib.lib().m3_scan_backward(C.byref(_scan_inputs(**kw)), C.byref(g), None)
    assert st == status
    assert message in _lib.lib().m3_last_error().decode()


def test_scan_backward_workspace_query():
    """m3_scan_backward_workspace_bytes: the state entering each chunk and
    the state gradient leaving it (f32 records at the backward's chunk length)
    plus per-chunk and per-token sections; 0 for shapes the backward does not
    cover."""
    from mamba3 import _lib
    L = _lib.lib()

    def need(B, T, H, P, N, R, dtype):
        cin = _lib.ScanInputsC(B, T, H, P, N, R, dtype, None, None, None, None, None, None,
                               None, None, None, 64, 0, None, 0)
        return int(L.m3_scan_backward_workspace_bytes(C.byref(cin)))

    w1 = need(8, 2048, 12, 64, 128, 1, _lib.M3_BF16)
    bhk = 8 * 12 * (2048 // 32)
    # S and Gh (f32 [P][N] records) per chunk; the chunk terms U and V are
    # formed inside the passes and never stored
    rec = bhk * 64 * 128 * 4
    assert 2 * rec <= w1 < 3 * rec
    assert w1 % 256 == 0
    assert need(8, 2048, 12, 64, 128, 1, _lib.M3_F32) == w1
    assert need(2, 100, 3, 64, 64, 2, _lib.M3_BF16) > 0
    # other shapes take the token walk (its own workspace), up to 64 KB of
    # per-token vectors
    assert need(1, 100, 2, 48, 128, 1, _lib.M3_BF16) > 0      # head_dim 48
    assert need(1, 100, 2, 64, 96, 1, _lib.M3_BF16) > 0       # d_state 96
    assert need(1, 100, 2, 64, 128, 3, _lib.M3_BF16) > 0      # rank 3
    assert need(1, 100, 2, 20000, 64, 1, _lib.M3_BF16) == 0   # beyond 64 KB of LDS


def test_no_alloc_scan_rejects_beyond_its_scratch():
    """m3_scan_no_alloc: a shape whose chunk-parallel workspace exceeds the
    static scratch fails with M3_ERR_UNSUPPORTED before any device work (the
    pointers below are stand-ins that are never dereferenced)."""
    from mamba3 import _lib
    L = _lib.lib()
    fake = 1 << 20
    # f32 keeps U and S in f32: ~64 KB per segment record at d_state 128
    cin = _lib.ScanInputsC(1, 65536, 12, 64, 128, 1, _lib.M3_F32, fake, fake, fake, fake, fake,
                           fake, fake, None, None, 64, 0, None, 0)
    need = int(L.m3_scan_workspace_bytes(C.byref(cin)))
    assert need > 32 << 20
    cout = _lib.ScanOutputC(fake, _lib.SsmStateC())
    st = L.m3_scan_no_alloc(C.byref(cin), C.byref(cout), None)
    assert st == _lib.M3_ERR_UNSUPPORTED
    msg = L.m3_last_error().decode()
    assert "static scratch holds 33554432 (32 MiB)" in msg and str(need) in msg
    assert L.m3_scan_no_alloc(None, C.byref(cout), None) == _lib.M3_ERR_ARGUMENT


def test_mixer_step_shape_cover_and_argument_checks():
    """m3_mixer_step's host-side checks (an empty call launches nothing): the
    shapes it covers, the ones it leaves to the composed calls, and its
    argument errors."""
    import ctypes as C
    from mamba3 import _lib
    L = _lib.lib()

    def call(H=4, P=64, N=128, R=1, G=4, state=True, factored=False, rot=True):
        d = _lib.MixerDimsC(0, H, P, N, R, G, 2, 1 if rot else 0, 1e-5)   # learned lambda
        st = C.byref(_lib.SsmStateC()) if state else None
        fc = C.byref(_lib.SsmStateFactoredC()) if factored else None
        return int(L.m3_mixer_step(C.byref(d), None, None, None, None, None, None, None, st, fc,
                                   None, None))

    assert call() == _lib.M3_OK
    assert call(R=2, N=64, P=32) == _lib.M3_OK
    assert call(state=False, factored=True) == _lib.M3_OK
    assert call(N=256) == _lib.M3_ERR_UNSUPPORTED      # d_state above 128
    assert call(N=96) == _lib.M3_ERR_UNSUPPORTED       # d_state / 8 not a power of two
    assert call(R=3) == _lib.M3_ERR_UNSUPPORTED
    assert call(P=4) == _lib.M3_ERR_UNSUPPORTED        # head_dim * rank not a multiple of 8
    assert call(state=True, factored=True) == _lib.M3_ERR_ARGUMENT
    assert call(state=False, factored=False) == _lib.M3_ERR_ARGUMENT
    assert call(H=4, G=3) == _lib.M3_ERR_CONFIG
    assert call(N=9) == _lib.M3_ERR_CONFIG               # odd d_state, rotational
    # the 16-byte prologue's rows: an in_proj width of 1796 (fixed lambda, H=4)
    d = _lib.MixerDimsC(0, 4, 64, 128, 1, 4, 1, 1, 1e-5)
    assert int(L.m3_mixer_in_proj_width(C.byref(d))) % 8 == 4
    assert int(L.m3_mixer_step(C.byref(d), None, None, None, None, None, None, None,
                               C.byref(_lib.SsmStateC()), None, None, None)) == _lib.M3_ERR_UNSUPPORTED


def test_conv_mixer_step_history_rules_before_any_launch():
    """m3_mixer_step_conv's host-side checks on an empty call (the pointers are
    stand-ins that are never dereferenced): one position per sequence, a
    history updated in place only where every channel belongs to one head
    (groups == heads), at most 4 taps, 16-byte aligned convolution buffers,
    and a non-negative post-gate norm eps."""
    import ctypes as C
    from mamba3 import _lib
    L = _lib.lib()
    H, P, N = 4, 16, 32
    chans = H * P + 2 * H * N          # groups == heads

    def call(G=H, k=4, seq=1, hist=1 << 20, new=1 << 20, w=1 << 16, bias=None, norm=None,
             eps=1e-5, conv=True):
        d = _lib.MixerDimsC(0, H, P, N, 1, G, 2, 1, 1e-5)
        cv = _lib.Conv1dC(k, seq, w, bias, hist, new)
        return int(L.m3_mixer_step_conv(C.byref(d), C.byref(cv) if conv else None, None, None,
                                        None, None, None, None, None, norm, C.c_float(eps),
                                        C.byref(_lib.SsmStateC()), None, None, None))

    assert call() == _lib.M3_OK                                   # in place, G == H
    assert call(conv=False, norm=1 << 12) == _lib.M3_OK           # post-gate norm alone
    assert call(G=2) == _lib.M3_ERR_UNSUPPORTED                   # in place, groups < heads
    assert "n_groups == n_heads" in L.m3_last_error().decode()
    assert call(G=2, new=(1 << 20) + 3 * chans * 2 * 4) == _lib.M3_OK   # separate, G < H
    assert call(seq=2) == _lib.M3_ERR_SHAPE
    assert call(k=1) == _lib.M3_ERR_CONFIG
    assert call(k=5) == _lib.M3_ERR_UNSUPPORTED                   # more taps than it holds
    assert call(w=None) == _lib.M3_ERR_ARGUMENT
    assert call(bias=(1 << 12) + 4) == _lib.M3_ERR_ARGUMENT       # unaligned bias
    assert call(conv=False, norm=1 << 12, eps=-1.0) == _lib.M3_ERR_CONFIG


def test_gated_scan_argument_checks_before_any_launch():
    """m3_scan_gated rejects f32 storage, a NULL z, a z row shorter than
    heads*head_dim*rank, a theta stride shorter than a token's heads*d_state/2
    angles and one whose rows are not whole 16-byte pieces, before any device
    work (the pointers are stand-ins that are never dereferenced)."""
    from mamba3 import _lib
    L = _lib.lib()
    fake = 1 << 20
    before = L.m3_launch_count()

    def call(dtype=_lib.M3_BF16, z=fake, stride=64 * 3, theta=None, theta_stride=0):
        cin = _lib.ScanInputsC(1, 8, 3, 64, 128, 1, dtype, fake, fake, fake, fake, fake, fake,
                               theta, None, None, 64, 0, None, 0)
        cout = _lib.ScanOutputC(fake, _lib.SsmStateC())
        return L.m3_scan_gated(C.byref(cin), C.byref(cout), z, stride, theta_stride, None)

    assert call(dtype=_lib.M3_F32) == _lib.M3_ERR_UNSUPPORTED
    assert call(z=None) == _lib.M3_ERR_ARGUMENT
    assert call(stride=64 * 3 - 1) == _lib.M3_ERR_SHAPE
    assert call(theta=fake, theta_stride=3 * 64 - 1) == _lib.M3_ERR_SHAPE
    assert call(theta=fake, theta_stride=3 * 64 + 4) == _lib.M3_ERR_UNSUPPORTED   # 392-byte rows
    assert b"16-byte pieces" in L.m3_last_error()
    assert L.m3_launch_count() == before
