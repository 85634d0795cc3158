"""The Mamba-3 token mixer, bf16 activations, over libmamba3_hip.so.

Mirrors `Mamba3Mixer` (BectorVoom/mamba-trainer src/models/mamba3.rs):
init (168-266), project (350-466), finish (468-477), apply / apply_with_state
(479-567) and step (569-630).  The projections are hipBLASLt GEMMs with the
int8 per-output-channel weight grid applied in their epilogue; the prologue
(split, the causal convolution over [x | B | C] with its history, silu, B/C
bias + RMSNorm, softplus, sigmoid), the scan or the decode step, and the gate
are the library's own gfx950 kernels.

Not covered (raise UnsupportedError): the bidirectional form and LoRA adapters.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import math
from typing import Optional

import torch

from . import _lib
from .error import ShapeError, UnsupportedError
from .nn import Linear, RmsNorm, _bf16_dev, _stream, normal, residual_scaled, tensor_param
from .ssm import (ScanInputs, SsmConfig, SsmState, SsmStateFactored, StateDynamics, mamba3_scan,
                  mamba3_scan_gated,
                  mamba3_step_, mamba3_step_factored_)


@dataclasses.dataclass
class MixerCache:
    """mamba3.rs:35-70: the scan state and, for a mixer with a convolution,
    its history, the last conv_kernel-1 convolution inputs [B, k-1, channels]
    (bf16, copies of projection values).  `ssm` is an SsmState, or the
    factored form (SsmStateFactored: last_u carried as the previous token's
    x and b, no reference counterpart) when the cache was made with
    factored=True."""
    ssm: "SsmState | SsmStateFactored"
    conv: Optional[torch.Tensor] = None

    def clone(self) -> "MixerCache":
        return MixerCache(self.ssm.clone(), None if self.conv is None else self.conv.clone())


@dataclasses.dataclass
class Projected:
    """mamba3.rs:278-287, shaped for the scan."""
    z: torch.Tensor          # [B, T, d_inner] view into the projection (row stride width)
    projected: torch.Tensor  # [B, T, width] (keeps z's storage)
    x: torch.Tensor          # [B, T, H, P, R] bf16
    b: torch.Tensor          # [B, T, H, N, R] bf16
    c: torch.Tensor
    dt: torch.Tensor         # [B, T, H] f32
    lam: torch.Tensor
    theta: Optional[torch.Tensor]   # [B, T, H, N/2] bf16


class Mamba3Mixer:
    """A Mamba-3 mixer for `[batch, seq, d_model]` bf16 activations."""

    def __init__(self, cfg: SsmConfig, *, device, gen: torch.Generator, n_layers: int = 1,
                 int8_weights: bool = False):
        """Mamba3MixerConfig::init (mamba3.rs:168-266), parameters drawn as there
        from a torch generator (the reference's ChaCha stream is not reproduced)."""
        cfg.validate()
        if cfg.bias:
            raise UnsupportedError("unsupported: projection biases are not on the gfx950 path")
        self.cfg = cfg
        H, N = cfg.n_heads, cfg.d_state
        self.in_proj = Linear(normal((cfg.d_model, cfg.in_proj_width()), 0.02, device, gen),
                              int8_weights=int8_weights)
        self.out_proj = Linear(residual_scaled((cfg.d_inner(), cfg.d_model), 0.02, n_layers,
                                               device, gen), int8_weights=int8_weights)
        # CausalConv1dConfig::new(d_inner + 2 bc_width, k).init (mamba3.rs:205, 228-230;
        # nn/conv.rs:60-110): weight [k, channels] KaimingUniform with fan_in k
        # (bound sqrt(3 / k), nn/init.rs:82-93), bias zeros.
        self.conv_weight = self.conv_bias = None
        if cfg.conv_kernel is not None:
            k, ch = cfg.conv_kernel, self.conv_channels()
            bound = math.sqrt(3.0 / k)
            self.conv_weight = ((torch.rand((k, ch), generator=gen, device=device) * 2.0 - 1.0)
                                * bound).float().contiguous()
            self.conv_bias = torch.zeros(ch, device=device)
        # dt_bias: softplus(dt_bias) log-uniform over [dt_min, dt_max] (mamba3.rs:198-209)
        u = torch.rand(H, generator=gen, device=device)
        dt = torch.exp(math.log(cfg.dt_min) + u * (math.log(cfg.dt_max) - math.log(cfg.dt_min)))
        dt = dt.clamp_min(cfg.dt_init_floor)
        self.dt_bias = (dt + torch.log(-torch.expm1(-dt))).float()
        # a_log = ln(U(a_init_min, a_init_max)) (mamba3.rs:211-216)
        u = torch.rand(H, generator=gen, device=device)
        a = cfg.a_init_min + u * (cfg.a_init_max - cfg.a_init_min)
        self.a_log = torch.log(a.clamp_min(1e-4)).float()
        self.d_skip = torch.ones(H, device=device) if cfg.skip_connection else None
        self.b_bias = torch.zeros((H, N), device=device) if cfg.bc_bias else None
        self.c_bias = torch.zeros((H, N), device=device) if cfg.bc_bias else None
        self.bc_norm = RmsNorm(N, device) if cfg.bc_norm else None
        self.post_gate_norm = RmsNorm(cfg.d_inner(), device) if cfg.post_gate_norm else None

    def named_parameters(self):
        """mamba3.rs:634-656: the reference's visit order and paths."""
        out = [("in_proj.weight", self.in_proj.param()), ("out_proj.weight", self.out_proj.param())]
        if self.conv_weight is not None:     # nn/conv.rs visit: weight, then bias
            out += [("conv.weight", tensor_param(self, "conv_weight")),
                    ("conv.bias", tensor_param(self, "conv_bias"))]
        out += [("dt_bias", tensor_param(self, "dt_bias")), ("a_log", tensor_param(self, "a_log"))]
        if self.d_skip is not None:
            out.append(("d", tensor_param(self, "d_skip")))
        if self.b_bias is not None:
            out.append(("b_bias", tensor_param(self, "b_bias")))
        if self.c_bias is not None:
            out.append(("c_bias", tensor_param(self, "c_bias")))
        for name, norm in (("bc_norm", self.bc_norm), ("post_gate_norm", self.post_gate_norm)):
            if norm is not None and norm.weight is not None:
                out.append((f"{name}.weight", tensor_param(norm, "weight")))
        return out

    # ------------------------------------------------------------ pieces
    def conv_channels(self) -> int:
        """mamba3.rs:205: the convolution runs over [x | B | C]."""
        return self.cfg.d_inner() + 2 * self.cfg.bc_width()

    def _history(self, batch: int, device) -> torch.Tensor:
        """CausalConv1d::empty_history (nn/conv.rs:221-225)."""
        return torch.zeros((batch, self.cfg.conv_kernel - 1, self.conv_channels()),
                           dtype=torch.bfloat16, device=device)

    def _dims(self, tokens: int) -> _lib.MixerDimsC:
        c = self.cfg
        return _lib.MixerDimsC(tokens, c.n_heads, c.head_dim, c.d_state, c.mode.rank(),
                               c.n_groups, int(c.discretization), int(c.dynamics),
                               1e-5 if self.bc_norm is None else self.bc_norm.eps)

    def project(self, input: torch.Tensor, history: Optional[torch.Tensor] = None,
                new_history: Optional[torch.Tensor] = None,
                theta_in_place: bool = False) -> Projected:
        """mamba3.rs:350-466.  With a convolution, `history` [B, k-1, channels]
        (None: zeros, as CausalConv1d::apply) precedes the window, and the
        window's last k-1 convolution inputs go to `new_history` when given
        (which may be `history` itself for a one-position window).
        theta_in_place: theta is returned as a view of the projection's last
        H*N/2 columns instead of a copy (for the gated scan, which reads it
        at the projection's row stride)."""
        c = self.cfg
        input = _bf16_dev(input, "mixer input")
        if input.dim() != 3 or input.shape[2] != c.d_model:
            raise ShapeError(f"shape error: Mamba3Mixer expects d_model={c.d_model}, "
                             f"got {tuple(input.shape)}")
        B, T, _ = input.shape
        H, P, N, R = c.n_heads, c.head_dim, c.d_state, c.mode.rank()
        projected = self.in_proj.apply(input)
        dev = input.device
        x = torch.empty((B, T, H, P, R), dtype=torch.bfloat16, device=dev)
        b = torch.empty((B, T, H, N, R), dtype=torch.bfloat16, device=dev)
        cc = torch.empty_like(b)
        dt = torch.empty((B, T, H), dtype=torch.float32, device=dev)
        lam = torch.empty_like(dt)
        rot = c.dynamics == StateDynamics.Rotational
        theta = None
        if rot and theta_in_place:
            w = projected.shape[-1]
            theta = projected[..., w - H * (N // 2):].unflatten(-1, (H, N // 2))
        elif rot:
            theta = torch.empty((B, T, H, N // 2), dtype=torch.bfloat16, device=dev)
        dims = self._dims(B * T)
        ptr = lambda t: None if t is None else t.data_ptr()
        conv = None
        if self.conv_weight is not None:
            hshape = (B, c.conv_kernel - 1, self.conv_channels())
            for name, h in (("history", history), ("new history", new_history)):
                if h is not None and (tuple(h.shape) != hshape or h.dtype != torch.bfloat16
                                      or not h.is_contiguous() or h.device != dev):
                    raise ShapeError(f"shape error: the convolution {name} must be a contiguous "
                                     f"bf16 {hshape} tensor on {dev}, got {h.dtype} "
                                     f"{tuple(h.shape)} on {h.device}")
            conv = _lib.Conv1dC(c.conv_kernel, T, self.conv_weight.data_ptr(),
                                ptr(self.conv_bias), ptr(history), ptr(new_history))
        _lib.check(_lib.lib().m3_mixer_prologue_conv(
            C.byref(dims), None if conv is None else C.byref(conv), projected.data_ptr(),
            self.dt_bias.data_ptr(), ptr(self.b_bias),
            ptr(self.c_bias), None if self.bc_norm is None else self.bc_norm.weight.data_ptr(),
            x.data_ptr(), b.data_ptr(), cc.data_ptr(), dt.data_ptr(), lam.data_ptr(),
            None if theta_in_place else ptr(theta), _stream(input)))
        return Projected(projected[..., :c.d_inner()], projected, x, b, cc, dt, lam, theta)

    def finish(self, y: torch.Tensor, proj: Projected, residual: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """mamba3.rs:468-477: [post-gate norm] * silu(z), then out_proj; the
        stack's residual add rides on the projection's epilogue."""
        c = self.cfg
        d = c.d_inner()
        B, T = proj.x.shape[0], proj.x.shape[1]
        gated = torch.empty((B, T, d), dtype=torch.bfloat16, device=y.device)
        nw = None if self.post_gate_norm is None else self.post_gate_norm.weight.data_ptr()
        eps = 1e-5 if self.post_gate_norm is None else self.post_gate_norm.eps
        _lib.check(_lib.lib().m3_mixer_gate(B * T, d, y.data_ptr(), proj.projected.data_ptr(),
                                            proj.projected.shape[-1], nw, C.c_float(eps),
                                            gated.data_ptr(), _stream(y)))
        return self.out_proj.apply(gated, residual=residual, out=out)

    # ------------------------------------------------------------ entry points
    def empty_cache(self, batch: int, device, factored: bool = False) -> MixerCache:
        """mamba3.rs:303-316: a zero state and, with a convolution, a zero
        history.  factored: the state in the factored form (decode steps
        stream h only)."""
        c = self.cfg
        rot = c.dynamics == StateDynamics.Rotational
        ssm = (SsmStateFactored.zeros(batch, c.n_heads, c.head_dim, c.d_state, c.mode.rank(), rot,
                                      device, dtype=torch.bfloat16) if factored
               else SsmState.zeros(batch, c.n_heads, c.head_dim, c.d_state, rot, device))
        return MixerCache(ssm, None if self.conv_weight is None else self._history(batch, device))

    def apply(self, input: torch.Tensor, residual: Optional[torch.Tensor] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self.apply_with_state(input, None, residual=residual, out=out)[0]

    def apply_with_state(self, input: torch.Tensor, cache: Optional[MixerCache],
                         residual: Optional[torch.Tensor] = None,
                         out: Optional[torch.Tensor] = None):
        """mamba3.rs:498-567: the mixer over a window; with a cache the scan
        starts from its state (and the convolution from its history) and the
        boundary state is returned in a new cache."""
        hist = new_hist = None
        if cache is not None and self.conv_weight is not None:
            hist = cache.conv
            new_hist = self._history(input.shape[0], input.device) if input.dim() == 3 else None
        # the gated scan (below) reads theta in place from the projection
        gated = self.post_gate_norm is None and not (torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (self.a_log, self.d_skip)))
        proj = self.project(input, hist, new_hist, theta_in_place=gated)
        si = ScanInputs(proj.x, proj.b, proj.c, proj.dt, self.a_log, proj.lam)
        si = si.with_chunk_size(self.cfg.chunk_size).with_state_output(cache is not None)
        if proj.theta is not None:
            si = si.with_theta(proj.theta)
        if self.d_skip is not None:
            si = si.with_skip(self.d_skip)
        factored = cache is not None and isinstance(cache.ssm, SsmStateFactored)
        if cache is not None:
            si = si.with_state(cache.ssm.to_full() if factored else cache.ssm)
        grad = torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (proj.x, proj.b, proj.c, proj.dt, proj.lam,
                                                         proj.theta, self.a_log, self.d_skip))
        if self.post_gate_norm is None and not grad and proj.x.dtype == torch.bfloat16:
            # the gate on the scan's output (fused into its last kernel where
            # that form runs), then out_proj
            scan = mamba3_scan_gated(si, proj.projected)
            B, T = proj.x.shape[0], proj.x.shape[1]
            y = self.out_proj.apply(scan.y.view(B, T, self.cfg.d_inner()), residual=residual, out=out)
        else:
            scan = mamba3_scan(si)
            y = self.finish(scan.y, proj, residual=residual, out=out)
        new = None
        if cache is not None:
            st = scan.state
            if factored and proj.x.shape[1] > 0:
                # the window's last token carries last_u
                st = SsmStateFactored(st.h, proj.x[:, -1].contiguous(), proj.b[:, -1].contiguous(),
                                      st.angle)
            elif factored:
                st = cache.ssm
            new = MixerCache(st, new_hist)
        return y, new

    def step_(self, input: torch.Tensor, cache: MixerCache,
              residual: Optional[torch.Tensor] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """mamba3.rs:569-630 for [batch, 1, d_model], the cache's state updated
        in place (the reference returns a new cache)."""
        if input.dim() != 3 or input.shape[1] != 1:
            raise ShapeError("shape error: step() expects a single position; use "
                             "apply_with_state for a window")
        c = self.cfg
        B = input.shape[0]
        out_fused = self._step_fused(input, cache, residual, out)
        if out_fused is not None:
            return out_fused
        if self.conv_weight is not None and cache.conv is None:
            cache.conv = self._history(B, input.device)
        proj = self.project(input, cache.conv, cache.conv)
        sq = lambda t: None if t is None else t.reshape((B,) + tuple(t.shape[2:]))
        step = mamba3_step_factored_ if isinstance(cache.ssm, SsmStateFactored) else mamba3_step_
        y = step(sq(proj.x), sq(proj.b), sq(proj.c), sq(proj.dt), sq(proj.lam),
                 self.a_log, sq(proj.theta), self.d_skip, cache.ssm)
        return self.finish(y.reshape(proj.x.shape), proj, residual=residual, out=out)

    def _step_fused(self, input: torch.Tensor, cache: MixerCache, residual, out):
        """step_ through m3_mixer_step (prologue, state step and gate in one
        launch; the same results as the composed path bit for bit), or
        m3_mixer_step_conv with the convolution (its history updated in place
        by the same launch) or the post-gate norm (the gate after it, a second
        launch); None where it does not apply (its shapes, a cache it cannot
        take, or an in-place history shared by several heads of a group)."""
        c = self.cfg
        if input.dim() != 3 or input.shape[2] != c.d_model:
            return None
        B = input.shape[0]
        H, P, N, R = c.n_heads, c.head_dim, c.d_state, c.mode.rank()
        st = cache.ssm
        factored = isinstance(st, SsmStateFactored)
        rot = c.dynamics == StateDynamics.Rotational
        ok = st.h.shape == (B, H, P, N) and st.h.is_contiguous() and (not rot or st.angle is not None)
        if factored:
            ok = ok and st.x_prev.shape == (B, H, P, R) and st.b_prev.shape == (B, H, N, R) and \
                st.x_prev.dtype == torch.bfloat16 and st.b_prev.dtype == torch.bfloat16 and \
                st.x_prev.is_contiguous() and st.b_prev.is_contiguous()
        else:
            ok = ok and st.last_u.shape == (B, H, P, N) and st.last_u.is_contiguous()
        if not ok:
            return None
        hist = None
        if self.conv_weight is not None:
            # the fused step holds up to 4 taps, and updates the history in
            # place only where every channel belongs to one head
            if c.n_groups != c.n_heads or c.conv_kernel > 4:
                return None
            if cache.conv is None:
                cache.conv = self._history(B, input.device)
            hist = cache.conv
            if (tuple(hist.shape) != (B, c.conv_kernel - 1, self.conv_channels())
                    or hist.dtype != torch.bfloat16 or not hist.is_contiguous()
                    or hist.device != input.device):
                return None
        if getattr(self, "_fused_step_ok", None) is None:
            # an empty call reports whether the library covers these shapes
            probe = _lib.lib().m3_mixer_step(C.byref(self._dims(0)), None, None, None, None, None,
                                             None, None, C.byref(_lib.SsmStateC()), None, None, None)
            if probe not in (_lib.M3_OK, _lib.M3_ERR_UNSUPPORTED):
                _lib.check(probe)
            self._fused_step_ok = probe == _lib.M3_OK
        if not self._fused_step_ok:
            return None
        dims = self._dims(B)
        input = _bf16_dev(input, "mixer input")
        projected = self.in_proj.apply(input)
        gated = torch.empty((B, 1, c.d_inner()), dtype=torch.bfloat16, device=input.device)
        ptr = lambda t: None if t is None else t.data_ptr()
        ang = ptr(st.angle) if rot else None
        if factored:
            sc, fc = None, C.byref(_lib.SsmStateFactoredC(st.h.data_ptr(), st.x_prev.data_ptr(),
                                                          st.b_prev.data_ptr(), ang))
        else:
            sc, fc = C.byref(_lib.SsmStateC(st.h.data_ptr(), st.last_u.data_ptr(), ang)), None
        bcn = None if self.bc_norm is None else self.bc_norm.weight.data_ptr()
        pn = self.post_gate_norm
        if hist is None and pn is None:
            _lib.check(_lib.lib().m3_mixer_step(
                C.byref(dims), projected.data_ptr(), self.dt_bias.data_ptr(), ptr(self.b_bias),
                ptr(self.c_bias), bcn, self.a_log.data_ptr(), ptr(self.d_skip), sc, fc,
                gated.data_ptr(), _stream(input)))
        else:
            conv = None if hist is None else _lib.Conv1dC(
                c.conv_kernel, 1, self.conv_weight.data_ptr(), ptr(self.conv_bias),
                hist.data_ptr(), hist.data_ptr())
            _lib.check(_lib.lib().m3_mixer_step_conv(
                C.byref(dims), None if conv is None else C.byref(conv), projected.data_ptr(),
                self.dt_bias.data_ptr(), ptr(self.b_bias), ptr(self.c_bias), bcn,
                self.a_log.data_ptr(), ptr(self.d_skip), None if pn is None else pn.weight.data_ptr(),
                C.c_float(1e-5 if pn is None else pn.eps), sc, fc, gated.data_ptr(),
                _stream(input)))
        return self.out_proj.apply(gated, residual=residual, out=out)

    def step(self, input: torch.Tensor, cache: MixerCache):
        """mamba3.rs:569-630: returns (output, new cache) like the reference."""
        new = cache.clone()
        if new.ssm.angle is None and self.cfg.dynamics == StateDynamics.Rotational:
            B = input.shape[0]
            new.ssm.angle = torch.zeros((B, self.cfg.n_heads, self.cfg.d_state // 2),
                                        dtype=torch.float32, device=input.device)
        return self.step_(input, new), new
