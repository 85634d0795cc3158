"""CPU restatement of the Mamba-3 mixer and the all-Mamba language model.

TEST INFRASTRUCTURE ONLY: imported by tests/ (and nothing else) as the
checker of the gfx950 mixer / LM path.  It never runs on the product path.

Follows BectorVoom/mamba-trainer:
  rms_norm               src/nn/norm.rs:70-105, src/tensor/ops/fused.rs:140-185
  quantize_int8_columns  src/nn/quant.rs:95-103 (int8_weights), 231-245 (PerChannel
                         symmetric quantize), 282-330 (solve_scale, channel_scales)
  causal_conv1d          src/nn/conv.rs:60-225 (weight [k, channels], tap j on the input
                         delayed by k-1-j), src/tensor/ops/fused.rs:780-865 (history
                         ++ input window, new history = its last k-1 positions)
  mixer_project          src/models/mamba3.rs:350-466 (split, the convolution over
                         [x | B | C] (386-400), silu, group -> head broadcast, B/C
                         bias, bc_norm, rank-last, softplus, sigmoid)
  mixer_finish           src/models/mamba3.rs:468-477
  mixer_apply            src/models/mamba3.rs:498-567 (the scan is the pinned f64
                         recurrence of oracle.scan_recurrence_f64)
  lm_forward             src/models/lm.rs:295-327, src/models/hybrid.rs:446-456
  lm_forward_stepwise    src/models/lm.rs:337-353, hybrid.rs:459-493 (one token
                         at a time through the carried state)

Arithmetic is f64.  With `rnd=True` every tensor the device path stores in
bf16 (normed rows, the projection, x/B/C/theta, y, the gated rows, the residual
stream, the logits) is rounded to bf16 at the same point, so a comparison with
the device differs only by accumulation order.

Planted mistakes (tests only): set FAULT to one of FAULTS to check that the
pins catch it.
"""
from __future__ import annotations

import numpy as np

import oracle as _scan

FAULTS = ("bc_swap", "no_silu_x", "norm_axis", "gate_sign", "dt_bias_sign", "quant_scale",
          "conv_flip", "conv_no_history", "conv_history_head")
FAULT = None


def bf16(a):
    """Round to the nearest bf16 (ties to even), returned as f64."""
    f = np.ascontiguousarray(np.asarray(a, np.float64).astype(np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def _r(a, rnd):
    return bf16(a) if rnd else np.asarray(a, np.float64)


def silu(v):
    return v / (1.0 + np.exp(-v))


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def softplus(v):
    """max(v, 0) + ln(1 + exp(-|v|))  (fused.rs:1291-1293)."""
    return np.maximum(v, 0.0) + np.log1p(np.exp(-np.abs(v)))


def rms_norm(x, w=None, eps=1e-5):
    """y = x * rsqrt(mean(x^2) + eps) * w over the last axis."""
    x = np.asarray(x, np.float64)
    s = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * s
    return y if w is None else y * np.asarray(w, np.float64)


def quantize_int8_columns(w):
    """w [in, out] f32 -> (codes [in, out], scales [out]) in f32 arithmetic:
    scale = max(max|w|, 1e-12) / 127; code = clamp(round(w / scale), -127, 127)."""
    w = np.asarray(w, np.float32)
    m = np.max(np.abs(w), axis=0)
    scale = (np.maximum(m, np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    if FAULT == "quant_scale":
        scale = (np.maximum(m, np.float32(1e-12)) / np.float32(128.0)).astype(np.float32)
    codes = np.clip(np.rint(w / scale), -127, 127).astype(np.float32)
    return codes, scale


def causal_conv1d(x, w, bias=None, history=None):
    """x [B, S, C], w [k, C], bias [C] or None, history [B, k-1, C] or None
    (zeros) -> (out [B, S, C], new_history [B, k-1, C]).  With the window
    win = history ++ x along the sequence,
    out[b, s, c] = bias[c] + sum_j w[j, c] * win[b, s + j, c], and the new
    history is the window's last k-1 positions."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    k = w.shape[0]
    B, S, C = x.shape
    hist = np.zeros((B, k - 1, C)) if history is None else np.asarray(history, np.float64)
    if FAULT == "conv_no_history":
        hist = np.zeros_like(hist)
    win = np.concatenate([hist, x], axis=1)
    taps = w[::-1] if FAULT == "conv_flip" else w
    out = np.zeros((B, S, C)) if bias is None else np.broadcast_to(
        np.asarray(bias, np.float64), (B, S, C)).copy()
    for j in range(k):
        out += taps[j] * win[:, j:j + S]
    new_history = win[:, :k - 1] if FAULT == "conv_history_head" else win[:, S:S + k - 1]
    return out, new_history.copy()


def widths(cfg):
    """(d_inner, bc_width, lambda_width, theta_width) of config.rs:165-200."""
    H, P, N, R, G = cfg["heads"], cfg["head_dim"], cfg["d_state"], cfg["rank"], cfg["groups"]
    lam_w = H if cfg["learned_lambda"] else 0
    th_w = H * N // 2 if cfg["rotational"] else 0
    return H * P * R, G * N * R, lam_w, th_w


def mixer_project(projected, cfg, p, rnd=False, batch=1, history=None):
    """projected [M, width] -> dict(z, x [M,H,P,R], b/c [M,H,N,R], dt, lam [M,H],
    theta [M,H,N/2] or None, conv_history [batch, k-1, channels] or None).
    With p["conv_w"] the M rows are `batch` sequences of M / batch positions,
    convolved from `history` (zeros when None)."""
    H, P, N, R, G = cfg["heads"], cfg["head_dim"], cfg["d_state"], cfg["rank"], cfg["groups"]
    din, bcw, lam_w, th_w = widths(cfg)
    pr = np.asarray(projected, np.float64)
    M = pr.shape[0]
    o = 0
    z = pr[:, o:o + din]; o += din
    xr = pr[:, o:o + din]; o += din
    br = pr[:, o:o + bcw]; o += bcw
    cr = pr[:, o:o + bcw]; o += bcw
    dtr = pr[:, o:o + H]; o += H
    lr = pr[:, o:o + lam_w]; o += lam_w
    thr = pr[:, o:o + th_w]; o += th_w
    new_history = None
    if p.get("conv_w") is not None:
        xbc = pr[:, din:2 * din + 2 * bcw].reshape(batch, M // batch, din + 2 * bcw)
        xbc, new_history = causal_conv1d(xbc, p["conv_w"], p.get("conv_b"), history)
        xbc = xbc.reshape(M, din + 2 * bcw)
        xr, br, cr = xbc[:, :din], xbc[:, din:din + bcw], xbc[:, din + bcw:]
    if FAULT == "bc_swap":
        br, cr = cr, br
    x = xr if FAULT == "no_silu_x" else silu(xr)
    x = _r(x, rnd).reshape(M, H, P, R)

    def bc(raw, bias):
        v = silu(raw).reshape(M, G, R, N)
        v = np.repeat(v, H // G, axis=1)                        # groups -> heads
        if bias is not None:
            v = v + np.asarray(bias, np.float64).reshape(1, H, 1, N)
        if p.get("bc_norm") is not None:
            if FAULT == "norm_axis":
                v = np.swapaxes(rms_norm(np.swapaxes(v, 1, 3), None, cfg["eps"]), 1, 3) * p["bc_norm"]
            else:
                v = rms_norm(v, p["bc_norm"], cfg["eps"])
        return _r(np.transpose(v, (0, 1, 3, 2)), rnd)           # [M, H, N, R]

    b = bc(br, p.get("b_bias"))
    c = bc(cr, p.get("c_bias"))
    sgn = -1.0 if FAULT == "dt_bias_sign" else 1.0
    dt = softplus(dtr + sgn * np.asarray(p["dt_bias"], np.float64)).astype(np.float32)
    lam = (sigmoid(lr) if lam_w else np.full((M, H), cfg["fixed_lambda"])).astype(np.float32)
    theta = thr.reshape(M, H, N // 2) if th_w else None
    return dict(z=z, x=x, b=b, c=c, dt=dt, lam=lam, theta=theta, conv_history=new_history)


def mixer_finish(y, z, p, cfg, rnd=False):
    """[post-gate norm](y) * silu(z) -> rows of d_inner (before out_proj)."""
    v = np.asarray(y, np.float64)
    if p.get("post_gate_norm") is not None:
        v = rms_norm(v, p["post_gate_norm"], cfg["eps"])
    zz = -z if FAULT == "gate_sign" else z
    return _r(v * silu(zz), rnd)


def mixer_apply(inp, p, cfg, state=None, rnd=False):
    """inp [B, T, D] (the normed rows) -> (out [B, T, D] = out_proj(gated),
    state' = (h, last_u, angle, conv history)).  `state` is such a tuple or
    None (zero state, zero convolution history)."""
    inp = np.asarray(inp, np.float64)
    B, T, D = inp.shape
    H, P, N, R = cfg["heads"], cfg["head_dim"], cfg["d_state"], cfg["rank"]
    projected = _r(inp.reshape(B * T, D) @ p["in_proj"], rnd)
    h0, lu0, an0, cv0 = state if state is not None else (None, None, None, None)
    pj = mixer_project(projected, cfg, p, rnd, batch=B, history=cv0)
    x = pj["x"].reshape(B, T, H, P, R)
    b = pj["b"].reshape(B, T, H, N, R)
    c = pj["c"].reshape(B, T, H, N, R)
    dt = pj["dt"].reshape(B, T, H)
    lam = pj["lam"].reshape(B, T, H)
    th = None if pj["theta"] is None else pj["theta"].reshape(B, T, H, N // 2)
    y, h, lu, an = _scan.scan_recurrence_f64(x, b, c, dt, p["a_log"], lam, th, p.get("d_skip"),
                                             h0, lu0, an0 if th is not None else None)
    y = _r(y, rnd).reshape(B * T, H * P * R)
    gated = mixer_finish(y, pj["z"], p, cfg, rnd)
    out = gated @ p["out_proj"]
    return out.reshape(B, T, D), (h, lu, an, pj["conv_history"])


def lm_forward(ids, model, rnd=False):
    """ids [B, T] -> logits [B, T, V] (all-Mamba stack, untied head)."""
    cfg = model["cfg"]
    x = np.asarray(model["embed"], np.float64)[np.asarray(ids)]
    for layer in model["layers"]:
        normed = _r(rms_norm(x, layer["norm"], cfg["eps"]), rnd)
        out, _ = mixer_apply(normed, layer, cfg, None, rnd)
        x = _r(x + out, rnd)
    h = _r(rms_norm(x, model["norm_f"], cfg["eps"]), rnd)
    return _r(h @ model["head"], rnd)


def lm_forward_stepwise(ids, model, split=0, rnd=False):
    """The cached path: the first `split` tokens as one window, then one token
    at a time, each layer's (h, last_u, angle, convolution history) carried
    forward."""
    cfg = model["cfg"]
    ids = np.asarray(ids)
    B, T = ids.shape
    H, P, N = cfg["heads"], cfg["head_dim"], cfg["d_state"]
    din, bcw, _, _ = widths(cfg)
    states = [(np.zeros((B, H, P, N)), np.zeros((B, H, P, N)),
               np.zeros((B, H, N // 2)) if cfg["rotational"] else None,
               None if layer.get("conv_w") is None
               else np.zeros((B, layer["conv_w"].shape[0] - 1, din + 2 * bcw)))
              for layer in model["layers"]]
    outs = []
    pieces = ([ids[:, :split]] if split else []) + [ids[:, t:t + 1] for t in range(split, T)]
    for piece in pieces:
        x = np.asarray(model["embed"], np.float64)[piece]
        for i, layer in enumerate(model["layers"]):
            normed = _r(rms_norm(x, layer["norm"], cfg["eps"]), rnd)
            out, st = mixer_apply(normed, layer, cfg, states[i], rnd)
            states[i] = st
            x = _r(x + out, rnd)
        h = _r(rms_norm(x, model["norm_f"], cfg["eps"]), rnd)
        outs.append(_r(h @ model["head"], rnd))
    return np.concatenate(outs, axis=1)


def random_model(rng, vocab=16, d_model=16, n_layers=2, heads=2, head_dim=4, d_state=4,
                 rank=1, groups=None, learned_lambda=True, fixed_lambda=float("nan"),
                 rotational=True, bc_bias=True, bc_norm=True, post_gate_norm=False,
                 skip=True, int8=False, bias_scale=0.0, conv_kernel=None):
    """A small all-Mamba model with the reference's initial distributions
    (normal 0.02 projections, residual-scaled out_proj, dt_bias inverse
    softplus of log-uniform [1e-3, 0.1], a_log = ln U(1, 16), convolution
    weights U(-sqrt(3/k), sqrt(3/k)) as KaimingUniform over [k, channels]
    draws them (nn/init.rs:82-93)); the projection scale is raised so the tiny
    model's activations are not all near zero, and the convolution bias (zero
    at the reference's init) is drawn with std bias_scale so that it shows."""
    groups = groups or heads
    cfg = dict(heads=heads, head_dim=head_dim, d_state=d_state, rank=rank, groups=groups,
               learned_lambda=learned_lambda, fixed_lambda=fixed_lambda, rotational=rotational,
               eps=1e-5)
    din, bcw, lam_w, th_w = widths(cfg)
    width = 2 * din + 2 * bcw + heads + lam_w + th_w
    layers = []
    for _ in range(n_layers):
        w_in = rng.normal(0, 0.3, (d_model, width)).astype(np.float32)
        w_out = rng.normal(0, 0.3 / np.sqrt(2 * n_layers), (din, d_model)).astype(np.float32)
        if int8:
            ci, si = quantize_int8_columns(w_in)
            co, so = quantize_int8_columns(w_out)
            w_in_eff, w_out_eff = ci.astype(np.float64) * si, co.astype(np.float64) * so
        else:
            w_in_eff, w_out_eff = bf16(w_in), bf16(w_out)
        dt = np.exp(rng.uniform(np.log(1e-3), np.log(0.1), heads)).clip(1e-4)
        conv = {}
        if conv_kernel is not None:
            bound = np.sqrt(3.0 / conv_kernel)
            conv = dict(conv_w=rng.uniform(-bound, bound, (conv_kernel, din + 2 * bcw)).astype(np.float32),
                        conv_b=rng.normal(0, bias_scale, din + 2 * bcw).astype(np.float32))
        layers.append(dict(**conv,
            norm=np.ones(d_model), in_proj_master=w_in, out_proj_master=w_out,
            in_proj=w_in_eff, out_proj=w_out_eff,
            dt_bias=(dt + np.log(-np.expm1(-dt))).astype(np.float32),
            a_log=np.log(rng.uniform(1, 16, heads)).astype(np.float32),
            d_skip=np.ones(heads, np.float32) if skip else None,
            b_bias=rng.normal(0, bias_scale, (heads, d_state)).astype(np.float32) if bc_bias else None,
            c_bias=rng.normal(0, bias_scale, (heads, d_state)).astype(np.float32) if bc_bias else None,
            bc_norm=np.ones(d_state) if bc_norm else None,
            post_gate_norm=np.ones(din) if post_gate_norm else None))
    return dict(cfg=cfg, layers=layers,
                embed=bf16(rng.normal(0, 1.0, (vocab, d_model))),
                norm_f=np.ones(d_model),
                head=bf16(rng.normal(0, 0.3, (d_model, vocab))))
