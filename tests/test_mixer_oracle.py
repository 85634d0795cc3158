"""Pins of the mixer / language-model oracle (oracle/mixer_oracle.py), CPU only.

Each check fixes the oracle by something other than its own formula:
known values of the activations, closed forms of RMSNorm, the int8 grid's
guarantees (the reference's tests/model.rs:318-361 adapted to per-channel
int8), how the projection row splits (perturbing one piece moves only its
own output), the rank-last layout, and the reference's decoding invariant
(tests/model.rs:99-139: one token at a time through the carried state equals
the parallel pass).  The causal convolution is pinned by a delta input (which
reads the taps back), by numpy.convolve per channel, and by windows chained
through the carried history (including windows shorter than the history).
test_planted_mistakes_are_caught plants each fault in the oracle and requires
that some check fails.
"""
import math

import numpy as np
import pytest

import mixer_oracle as mo


def _cfg(heads=2, head_dim=4, d_state=4, rank=1, groups=2, learned=True, rot=True):
    return dict(heads=heads, head_dim=head_dim, d_state=d_state, rank=rank, groups=groups,
                learned_lambda=learned, fixed_lambda=0.5, rotational=rot, eps=1e-5)


def _params(rng, cfg, bias=0.3):
    H, N = cfg["heads"], cfg["d_state"]
    return dict(dt_bias=rng.normal(0, 1, H).astype(np.float32),
                b_bias=rng.normal(0, bias, (H, N)).astype(np.float32),
                c_bias=rng.normal(0, bias, (H, N)).astype(np.float32),
                bc_norm=np.ones(N), post_gate_norm=None)


# ------------------------------------------------------------------ checks
def check_bf16_rounding():
    assert mo.bf16(1.0) == 1.0
    assert mo.bf16(1.0 + 2.0 ** -8) == 1.0                      # tie -> even
    assert mo.bf16(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6       # tie -> even (up)
    assert mo.bf16(1.0 + 2.0 ** -8 + 2.0 ** -12) == 1.0 + 2.0 ** -7


def check_activation_values():
    assert math.isclose(mo.silu(np.float64(1.0)), 0.7310585786300049, rel_tol=1e-14)
    assert mo.silu(np.float64(0.0)) == 0.0
    assert math.isclose(mo.softplus(np.float64(0.0)), math.log(2.0), rel_tol=1e-14)
    assert math.isclose(mo.softplus(np.float64(50.0)), 50.0, rel_tol=1e-14)
    assert mo.sigmoid(np.float64(0.0)) == 0.5


def check_rms_norm_closed_forms():
    y = mo.rms_norm(np.array([3.0, 4.0]), None, 0.0)
    assert np.allclose(y, np.array([3.0, 4.0]) / math.sqrt(12.5), rtol=1e-14)
    c = np.full((3, 8), -2.5)
    assert np.allclose(mo.rms_norm(c, np.arange(1, 9), 0.0), -np.arange(1, 9), rtol=1e-14)


def check_quantizer_grid():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (64, 24)).astype(np.float32)
    w[:, 3] = 0.0
    w[:, 5] = (np.arange(64) - 32) / 32.0                      # the reference test's ramp
    codes, scale = mo.quantize_int8_columns(w)
    assert np.all(codes == np.rint(codes)) and np.all(np.abs(codes) <= 127)
    for j in range(w.shape[1]):
        col = codes[:, j]
        assert len(np.unique(col)) <= 255
        if j != 3:
            assert np.abs(col).max() == 127                     # the column max hits the grid edge
        assert np.all(np.abs(col.astype(np.float64) * scale[j] - w[:, j]) <= scale[j] * 0.5 + 1e-12)
    assert np.all(codes[:, 3] == 0)
    assert math.isclose(float(scale[5]), 1.0 / 127.0, rel_tol=1e-6)


def check_projection_pieces():
    """Perturbing one piece of the projection row moves only its own output."""
    rng = np.random.default_rng(2)
    cfg = _cfg(heads=4, groups=2, rank=1)
    p = _params(rng, cfg)
    din, bcw, lw, tw = mo.widths(cfg)
    H = cfg["heads"]
    width = 2 * din + 2 * bcw + H + lw + tw
    base = rng.normal(0, 1, (3, width))
    ref = mo.mixer_project(base, cfg, p)
    spans = {"z": (0, din), "x": (din, 2 * din), "b": (2 * din, 2 * din + bcw),
             "c": (2 * din + bcw, 2 * din + 2 * bcw), "dt": (2 * din + 2 * bcw, 2 * din + 2 * bcw + H),
             "lam": (2 * din + 2 * bcw + H, 2 * din + 2 * bcw + 2 * H), "theta": (width - tw, width)}
    for piece, (lo, hi) in spans.items():
        pert = base.copy()
        pert[:, lo:hi] += 0.5
        out = mo.mixer_project(pert, cfg, p)
        for key in ("z", "x", "b", "c", "dt", "lam", "theta"):
            same = np.allclose(out[key], ref[key])
            assert same == (key != piece), (piece, key)
    # group g of B feeds heads [g * H/G, (g+1) * H/G) only
    pert = base.copy()
    lo = 2 * din + 1 * (bcw // cfg["groups"])
    pert[:, lo:lo + bcw // cfg["groups"]] += 0.5
    out = mo.mixer_project(pert, cfg, p)
    moved = [not np.allclose(out["b"][:, h], ref["b"][:, h]) for h in range(H)]
    assert moved == [False, False, True, True]


def check_rank_last_layout():
    rng = np.random.default_rng(3)
    cfg = _cfg(heads=2, groups=2, rank=2)
    p = _params(rng, cfg)
    din, bcw, lw, tw = mo.widths(cfg)
    width = 2 * din + 2 * bcw + 2 + lw + tw
    base = rng.normal(0, 1, (2, width))
    ref = mo.mixer_project(base, cfg, p)
    N = cfg["d_state"]
    pert = base.copy()
    pert[:, 2 * din + (0 * 2 + 1) * N + 2] += 0.7          # group 0, rank 1, state 2
    out = mo.mixer_project(pert, cfg, p)
    assert out["b"].shape == (2, 2, N, 2)
    assert np.allclose(out["b"][:, :, :, 0], ref["b"][:, :, :, 0])
    assert np.allclose(out["b"][:, 1], ref["b"][:, 1])
    assert not np.allclose(out["b"][:, 0, :, 1], ref["b"][:, 0, :, 1])


def check_bc_norm_unit_rms():
    rng = np.random.default_rng(4)
    cfg = _cfg(heads=3, groups=3, rank=2, d_state=8)
    p = _params(rng, cfg)
    p["b_bias"] = None
    din, bcw, lw, tw = mo.widths(cfg)
    base = rng.normal(0, 2, (5, 2 * din + 2 * bcw + 3 + lw + tw))
    out = mo.mixer_project(base, cfg, p)
    ms = np.mean(out["b"] ** 2, axis=2)                      # over the state axis
    assert np.allclose(ms, 1.0, atol=1e-3)


def check_known_mixer_values():
    """One token with hand-picked pieces: x = silu(1), dt = softplus(0 + bias),
    lambda = sigmoid(0), and the gate y * silu(z) at y = 1, z = 1."""
    cfg = _cfg(heads=1, groups=1, head_dim=1, d_state=2, rot=False)
    p = dict(dt_bias=np.array([0.0], np.float32), b_bias=None, c_bias=None, bc_norm=None)
    din, bcw, lw, tw = mo.widths(cfg)
    row = np.zeros((1, 2 * din + 2 * bcw + 1 + lw + tw))
    row[0, din] = 1.0
    out = mo.mixer_project(row, cfg, p)
    assert math.isclose(float(out["x"][0, 0, 0, 0]), 0.7310585786300049, rel_tol=1e-12)
    assert math.isclose(float(out["dt"][0, 0]), math.log(2.0), rel_tol=1e-6)
    assert float(out["lam"][0, 0]) == 0.5
    p["dt_bias"] = np.array([1.5], np.float32)
    out = mo.mixer_project(row, cfg, p)
    assert math.isclose(float(out["dt"][0, 0]), math.log1p(math.exp(1.5)), rel_tol=1e-6)
    g = mo.mixer_finish(np.ones((1, 1)), np.ones((1, 1)), {"post_gate_norm": None}, cfg)
    assert math.isclose(float(g[0, 0]), 0.7310585786300049, rel_tol=1e-12)


def check_zero_projection_is_silent():
    rng = np.random.default_rng(5)
    model = mo.random_model(rng, n_layers=1)
    layer = model["layers"][0]
    layer = dict(layer, in_proj=np.zeros_like(layer["in_proj"]))
    out, _ = mo.mixer_apply(rng.normal(0, 1, (1, 6, 16)), layer, model["cfg"])
    assert np.allclose(out, 0.0)


def check_cached_decoding_matches_parallel():
    """tests/model.rs:99-139: stepwise and prefill + steps equal the parallel pass."""
    for rot, learned, conv in ((True, True, None), (False, False, None), (True, True, 4)):
        rng = np.random.default_rng(6)
        model = mo.random_model(rng, rotational=rot, learned_lambda=learned, fixed_lambda=0.5,
                                bias_scale=0.3, conv_kernel=conv)
        ids = np.array([[3, 1, 4, 1, 5, 9, 2, 6]]) % 16
        full = mo.lm_forward(ids, model)
        for split in (0, 5):
            step = mo.lm_forward_stepwise(ids, model, split)
            assert np.max(np.abs(step - full)) < 2e-3, (rot, conv, split,
                                                        np.max(np.abs(step - full)))
    # the pieces really move the logits (the invariant is not vacuous)
    assert np.std(full) > 1e-2


def check_conv_delta_reproduces_taps():
    """A unit impulse at position s0 of channel c gives bias + w[k-1-d, c] at
    position s0 + d for d < k, and the bias everywhere else."""
    rng = np.random.default_rng(7)
    k, S, C = 4, 9, 3
    w = rng.normal(0, 1, (k, C))
    bias = rng.normal(0, 1, C)
    x = np.zeros((1, S, C))
    x[0, 2, 1] = 1.0
    out, _ = mo.causal_conv1d(x, w, bias)
    want = np.broadcast_to(bias, (1, S, C)).copy()
    for d in range(k):
        want[0, 2 + d, 1] += w[k - 1 - d, 1]
    assert np.allclose(out, want, rtol=0, atol=1e-15)


def check_conv_matches_numpy_convolve():
    """Per channel, the causal convolution is numpy's full convolution of
    history ++ x with the reversed taps, read at the positions of x."""
    rng = np.random.default_rng(8)
    for k, S, hist in ((2, 7, False), (4, 11, True), (5, 3, True)):
        B, C = 2, 5
        w = rng.normal(0, 1, (k, C))
        bias = rng.normal(0, 1, C)
        x = rng.normal(0, 1, (B, S, C))
        h = rng.normal(0, 1, (B, k - 1, C)) if hist else None
        out, _ = mo.causal_conv1d(x, w, bias, h)
        for b in range(B):
            for c in range(C):
                seq = np.concatenate([np.zeros(k - 1) if h is None else h[b, :, c], x[b, :, c]])
                full = np.convolve(seq, w[::-1, c])
                assert np.allclose(out[b, :, c], full[k - 1:k - 1 + S] + bias[c], rtol=1e-13,
                                   atol=1e-13), (k, S, b, c)


def check_conv_history_chains_windows():
    """The convolution of a sequence equals the convolution of its pieces, each
    started from the history the previous piece returned; pieces of one
    position and pieces shorter than the history included."""
    rng = np.random.default_rng(9)
    k, S, B, C = 4, 12, 2, 3
    w = rng.normal(0, 1, (k, C))
    bias = rng.normal(0, 1, C)
    x = rng.normal(0, 1, (B, S, C))
    whole, last = mo.causal_conv1d(x, w, bias)
    for cuts in ((5,), (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11), (2, 7), (10,)):
        hist, outs, lo = None, [], 0
        for hi in list(cuts) + [S]:
            o, hist = mo.causal_conv1d(x[:, lo:hi], w, bias, hist)
            outs.append(o)
            lo = hi
        assert np.allclose(np.concatenate(outs, axis=1), whole, rtol=1e-13, atol=1e-13), cuts
        assert np.allclose(hist, last, rtol=0, atol=0), cuts
    assert np.array_equal(last, x[:, S - (k - 1):])           # the last k-1 inputs


CHECKS = [check_bf16_rounding, check_activation_values, check_rms_norm_closed_forms,
          check_quantizer_grid, check_projection_pieces, check_rank_last_layout,
          check_bc_norm_unit_rms, check_known_mixer_values, check_zero_projection_is_silent,
          check_cached_decoding_matches_parallel, check_conv_delta_reproduces_taps,
          check_conv_matches_numpy_convolve, check_conv_history_chains_windows]


@pytest.mark.parametrize("check", CHECKS, ids=[c.__name__ for c in CHECKS])
def test_mixer_oracle_pin(check):
    mo.FAULT = None
    check()


@pytest.mark.parametrize("fault", mo.FAULTS)
def test_planted_mistakes_are_caught(fault):
    mo.FAULT = fault
    try:
        failed = []
        for check in CHECKS:
            try:
                check()
            except AssertionError:
                failed.append(check.__name__)
        assert failed, f"planted fault {fault!r} passed every check"
    finally:
        mo.FAULT = None
