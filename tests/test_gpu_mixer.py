"""GPU parity of the mixer and language-model path (mamba3_mixer.h + the scan)
against the CPU oracle (oracle/mixer_oracle.py) on identical inputs.

Bars: bf16 storage, f32 accumulation.  Kernel outputs are compared with the
oracle rounded at the same storage points; rel-L2 <= 1e-2 (the north-star bar
for bf16) unless stated, and bit-exact for the int8 grid and the embedding
gather.  f32 outputs (dt, lambda) at 1e-5.
"""
import dataclasses

import numpy as np
import pytest
import torch

import mixer_oracle as mo
from cases import rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def t_bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(DEV).to(torch.bfloat16)


def t_f32(a):
    return None if a is None else torch.from_numpy(np.asarray(a, np.float32)).to(DEV)


def host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def lib():
    from mamba3 import _lib
    return _lib


# ------------------------------------------------------------------ kernels
@pytest.mark.parametrize("rows,dim,stride", [(37, 768, 768), (5, 4, 4), (9, 24, 40), (3, 130, 130)])
def test_rms_norm_rows(rows, dim, stride):
    import ctypes as C
    rng = np.random.default_rng(rows * dim)
    x = mo.bf16(rng.normal(0, 3, (rows, stride)))
    w = rng.uniform(0.5, 1.5, dim)
    xd = t_bf16(x)
    y = torch.zeros((rows, stride), dtype=torch.bfloat16, device=DEV)
    L = lib()
    wd = t_f32(w)
    L.check(L.lib().m3_rms_norm(rows, dim, xd.data_ptr(), stride, wd.data_ptr(),
                                C.c_float(1e-5), y.data_ptr(), stride, None))
    torch.cuda.synchronize()
    ref = mo.rms_norm(x[:, :dim], w, 1e-5)
    assert rel_l2(host(y)[:, :dim], ref) <= 4e-3
    assert np.all(host(y)[:, dim:] == 0)                       # outside the row untouched


def test_quantize_columns_matches_the_grid_bit_for_bit():
    rng = np.random.default_rng(7)
    w = rng.normal(0, 0.02, (768, 300)).astype(np.float32)
    w[:, 11] = 0.0
    codes = torch.empty((768, 300), dtype=torch.bfloat16, device=DEV)
    scales = torch.empty(300, dtype=torch.float32, device=DEV)
    L = lib()
    wd = t_f32(w)
    L.check(L.lib().m3_quantize_int8_columns(768, 300, wd.data_ptr(), codes.data_ptr(),
                                             scales.data_ptr(), None))
    torch.cuda.synchronize()
    rc, rs = mo.quantize_int8_columns(w)
    assert np.array_equal(host(codes), rc.astype(np.float64))
    assert np.array_equal(scales.cpu().numpy(), rs)


@pytest.mark.parametrize("m,k,n,int8,resid", [(100, 64, 300, True, True), (33, 16, 7, False, False),
                                              (4096, 768, 5400, True, False),
                                              (2048, 768, 768, True, True)])
def test_linear_against_f64(m, k, n, int8, resid):
    from mamba3.nn import Linear
    rng = np.random.default_rng(m + n)
    x = mo.bf16(rng.normal(0, 1, (m, k)))
    w = rng.normal(0, 0.02, (k, n)).astype(np.float32)
    lin = Linear(t_f32(w), int8_weights=int8)
    if int8:
        c, s = mo.quantize_int8_columns(w)
        w_eff = c.astype(np.float64) * s
    else:
        w_eff = mo.bf16(w)
    r = mo.bf16(rng.normal(0, 1, (m, n))) if resid else None
    out = t_bf16(r) if resid else None
    y = lin.apply(t_bf16(x), residual=out, out=out)
    ref = x @ w_eff + (r if resid else 0.0)
    assert rel_l2(host(y), ref) <= 1e-2


# The first, second, fourth and fifth shapes take the 16-byte path (ranks 1, 4
# and 2); the third (d_state 4) and the last (width 2*8*3 + 2*3*8 + 3 + 12, not
# a multiple of 8) take the element-wise one.  `plain` drops biases and norm.
@pytest.mark.parametrize("H,G,P,N,R,learned,rot,plain", [(4, 2, 4, 8, 1, True, True, False),
                                                         (12, 12, 64, 128, 1, True, True, False),
                                                         (2, 1, 4, 4, 2, False, False, False),
                                                         (4, 4, 16, 32, 4, True, True, False),
                                                         (8, 4, 8, 64, 2, False, False, True),
                                                         (3, 3, 8, 8, 1, False, True, True)])
def test_prologue_against_oracle(H, G, P, N, R, learned, rot, plain):
    import ctypes as C
    from mamba3 import Discretization, StateDynamics
    rng = np.random.default_rng(H * N + R)
    cfg = dict(heads=H, head_dim=P, d_state=N, rank=R, groups=G, learned_lambda=learned,
               fixed_lambda=0.5, rotational=rot, eps=1e-5)
    din, bcw, lw, tw = mo.widths(cfg)
    width = 2 * din + 2 * bcw + H + lw + tw
    M = 37
    proj = mo.bf16(rng.normal(0, 1.5, (M, width)))
    p = dict(dt_bias=rng.normal(-2, 1, H).astype(np.float32),
             b_bias=rng.normal(0, 0.3, (H, N)).astype(np.float32),
             c_bias=rng.normal(0, 0.3, (H, N)).astype(np.float32),
             bc_norm=rng.uniform(0.5, 1.5, N).astype(np.float32))
    if plain:
        p.update(b_bias=None, c_bias=None, bc_norm=None)
    ref = mo.mixer_project(proj, cfg, p, rnd=True)
    L = lib()
    disc = Discretization.LearnedTrapezoid if learned else Discretization.Trapezoid
    dyn = StateDynamics.Rotational if rot else StateDynamics.Real
    dims = L.MixerDimsC(M, H, P, N, R, G, int(disc), int(dyn), 1e-5)
    assert L.lib().m3_mixer_in_proj_width(C.byref(dims)) == width
    x = torch.empty((M, H, P, R), dtype=torch.bfloat16, device=DEV)
    b = torch.empty((M, H, N, R), dtype=torch.bfloat16, device=DEV)
    c = torch.empty_like(b)
    dt = torch.empty((M, H), device=DEV)
    lam = torch.empty_like(dt)
    th = torch.empty((M, H, N // 2), dtype=torch.bfloat16, device=DEV) if rot else None
    keep = [t_f32(p[k]) for k in ("dt_bias", "b_bias", "c_bias", "bc_norm")]
    projd = t_bf16(proj)                              # held until the launch has run
    L.check(L.lib().m3_mixer_prologue(C.byref(dims), projd.data_ptr(),
                                      *[None if k is None else k.data_ptr() for k in keep],
                                      x.data_ptr(), b.data_ptr(),
                                      c.data_ptr(), dt.data_ptr(), lam.data_ptr(),
                                      None if th is None else th.data_ptr(), None))
    torch.cuda.synchronize()
    assert rel_l2(host(x), ref["x"]) <= 1e-2
    assert rel_l2(host(b), ref["b"]) <= 1e-2
    assert rel_l2(host(c), ref["c"]) <= 1e-2
    assert rel_l2(host(dt), ref["dt"]) <= 1e-5
    assert rel_l2(host(lam), ref["lam"]) <= 1e-5
    if rot:
        assert np.array_equal(host(th), ref["theta"])


# z stride 200 takes the 16-byte path, 201 the element-wise one.
@pytest.mark.parametrize("zs", [200, 201])
@pytest.mark.parametrize("norm", [False, True])
def test_gate_against_oracle(norm, zs):
    import ctypes as C
    rng = np.random.default_rng(11 + norm)
    T, d = 29, 96
    y = mo.bf16(rng.normal(0, 1, (T, d)))
    z = mo.bf16(rng.normal(0, 2, (T, zs)))
    w = rng.uniform(0.5, 1.5, d) if norm else None
    out = torch.empty((T, d), dtype=torch.bfloat16, device=DEV)
    L = lib()
    wt, yd, zd = t_f32(w), t_bf16(y), t_bf16(z)      # held until the launch has run
    L.check(L.lib().m3_mixer_gate(T, d, yd.data_ptr(), zd.data_ptr(), zs,
                                  None if wt is None else wt.data_ptr(), C.c_float(1e-5),
                                  out.data_ptr(), None))
    torch.cuda.synchronize()
    ref = mo.mixer_finish(y, z[:, :d], {"post_gate_norm": w}, dict(eps=1e-5), rnd=False)
    assert rel_l2(host(out), ref) <= 4e-3


def test_embedding_gather_is_exact_and_zeroes_unknown_ids():
    from mamba3.nn import Embedding
    rng = np.random.default_rng(12)
    table = mo.bf16(rng.normal(0, 1, (50, 24)))
    emb = Embedding(t_f32(table))
    ids = np.array([[0, 49, 7, 7], [3, -1, 50, 12]])
    out = host(emb.lookup(torch.from_numpy(ids).to(DEV)))
    for i in range(2):
        for j in range(4):
            want = table[ids[i, j]] if 0 <= ids[i, j] < 50 else np.zeros(24)
            assert np.array_equal(out[i, j], want)


# ------------------------------------------------------------------ mixer / LM
def gpu_lm_from_oracle(model, int8, learned=True, rot=True):
    """A mamba3.lm.Mamba3Lm carrying the oracle model's weights."""
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    from mamba3.nn import Embedding, Linear
    cfg = model["cfg"]
    ssm = SsmConfig(d_model=model["embed"].shape[1], n_heads=cfg["heads"], head_dim=cfg["head_dim"],
                    d_state=cfg["d_state"], n_groups=cfg["groups"],
                    discretization=Discretization.LearnedTrapezoid if learned else Discretization.Trapezoid,
                    dynamics=StateDynamics.Rotational if rot else StateDynamics.Real,
                    mode=SsmMode(cfg["rank"]), chunk_size=64, conv_kernel=None)
    lmc = Mamba3LmConfig(vocab_size=model["embed"].shape[0], d_model=model["embed"].shape[1],
                         n_layers=len(model["layers"]), ssm=ssm, int8_weights=int8)
    lm = Mamba3Lm(lmc, DEV)
    lm.embed = Embedding(t_f32(model["embed"]))
    lm.norm_f.weight = t_f32(model["norm_f"])
    lm.head = Linear(t_f32(model["head"]))
    for (norm, mixer), layer in zip(lm.layers, model["layers"]):
        norm.weight = t_f32(layer["norm"])
        mixer.in_proj = Linear(t_f32(layer["in_proj_master"]), int8_weights=int8)
        mixer.out_proj = Linear(t_f32(layer["out_proj_master"]), int8_weights=int8)
        mixer.dt_bias = t_f32(layer["dt_bias"])
        mixer.a_log = t_f32(layer["a_log"])
        mixer.d_skip = t_f32(layer["d_skip"])
        mixer.b_bias = t_f32(layer["b_bias"])
        mixer.c_bias = t_f32(layer["c_bias"])
        mixer.bc_norm.weight = t_f32(layer["bc_norm"])
    return lm


@pytest.mark.parametrize("int8,rot,learned,rank", [(True, True, True, 1), (False, True, True, 1),
                                                   (True, False, False, 1), (True, True, True, 2)])
def test_lm_forward_against_oracle(int8, rot, learned, rank):
    rng = np.random.default_rng(20 + int8 + 2 * rot + 4 * rank)
    model = mo.random_model(rng, vocab=32, d_model=32, n_layers=2, heads=2, head_dim=8,
                            d_state=8, rank=rank, rotational=rot, learned_lambda=learned,
                            fixed_lambda=0.5, int8=int8, bias_scale=0.3)
    lm = gpu_lm_from_oracle(model, int8, learned, rot)
    ids = rng.integers(0, 32, (2, 45))
    got = host(lm.forward(torch.from_numpy(ids).to(DEV)))
    ref = mo.lm_forward(ids, model, rnd=True)
    assert rel_l2(got, ref) <= 1e-2, rel_l2(got, ref)


def test_cached_decoding_matches_the_parallel_pass_on_device():
    """tests/model.rs:99-139 on the gfx950 path: one token at a time, and a
    prefill of 5 followed by steps, reproduce the parallel pass."""
    rng = np.random.default_rng(31)
    model = mo.random_model(rng, vocab=16, d_model=32, n_layers=2, heads=2, head_dim=8,
                            d_state=8, int8=True, bias_scale=0.3)
    lm = gpu_lm_from_oracle(model, True)
    seq = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6]], device=DEV)
    full = host(lm.forward(seq))
    for split in (0, 5):
        cache = lm.empty_cache(1, DEV)
        outs = []
        if split:
            outs.append(host(lm.forward_cached(seq[:, :split], cache)))
        for t in range(split, seq.shape[1]):
            outs.append(host(lm.forward_cached(seq[:, t:t + 1], cache)))
        step = np.concatenate(outs, axis=1)
        assert rel_l2(step, full) <= 1e-2, (split, rel_l2(step, full))
    ref = mo.lm_forward_stepwise(seq.cpu().numpy(), model, 5, rnd=True)
    assert rel_l2(step, ref) <= 1e-2


def test_config4_layer_shapes_against_oracle():
    """One layer of BASELINE config 4 (d_model 768, 12 x 64 heads, N 128, groups
    12, int8 projections, bc_norm) at batch 2 x 256 tokens."""
    rng = np.random.default_rng(40)
    model = mo.random_model(rng, vocab=64, d_model=768, n_layers=1, heads=12, head_dim=64,
                            d_state=128, int8=True, bias_scale=0.1)
    for layer in model["layers"]:                   # the reference's init scale at this width
        layer["in_proj_master"] = (layer["in_proj_master"] * (0.02 / 0.3)).astype(np.float32)
        c, s = mo.quantize_int8_columns(layer["in_proj_master"])
        layer["in_proj"] = c.astype(np.float64) * s
    lm = gpu_lm_from_oracle(model, True)
    ids = rng.integers(0, 64, (2, 256))
    got = host(lm.forward(torch.from_numpy(ids).to(DEV)))
    ref = mo.lm_forward(ids, model, rnd=True)
    assert rel_l2(got, ref) <= 1e-2, rel_l2(got, ref)


def test_decode_graph_replays_match_eager_steps():
    """Mamba3Lm.capture_decode: a captured decode step replayed six times, with
    eager steps and host synchronisation between the replays; every replay's
    logits and states equal the eager step's bit for bit (the same kernels on
    the same inputs), and capturing leaves the states where they were."""
    from mamba3.mixer import MixerCache
    rng = np.random.default_rng(61)
    model = mo.random_model(rng, vocab=64, d_model=64, n_layers=2, heads=4, head_dim=16,
                            d_state=16, int8=True, bias_scale=0.3)
    lm = gpu_lm_from_oracle(model, True)
    B = 8
    gen = torch.Generator(device=DEV).manual_seed(62)
    cache_e = lm.empty_cache(B, DEV)
    for c in cache_e:
        c.ssm.h.normal_(0.0, 0.1, generator=gen)
        c.ssm.last_u.normal_(0.0, 0.1, generator=gen)
        c.ssm.angle.uniform_(-3.0, 3.0, generator=gen)
    cache_g = [MixerCache(c.ssm.clone()) for c in cache_e]
    graph = lm.capture_decode(cache_g, B)
    torch.cuda.synchronize()
    for ce, cg in zip(cache_e, cache_g):
        assert torch.equal(ce.ssm.h, cg.ssm.h) and torch.equal(ce.ssm.angle, cg.ssm.angle)
    for step in range(6):
        ids = torch.randint(0, 64, (B, 1), device=DEV, generator=gen)
        want = lm.forward_cached(ids, cache_e).clone()
        torch.cuda.synchronize()
        got = graph.step(ids).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), step
        for ce, cg in zip(cache_e, cache_g):
            assert torch.equal(ce.ssm.h, cg.ssm.h), step
            assert torch.equal(ce.ssm.last_u, cg.ssm.last_u), step
            assert torch.equal(ce.ssm.angle, cg.ssm.angle), step
    assert torch.isfinite(got.float()).all()
