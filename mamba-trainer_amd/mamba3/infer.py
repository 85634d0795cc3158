"""The decode-time state cache (src/infer/mod.rs:19-48) over the gfx950 step kernel.

One SsmState per Mamba layer, stored as views into a single allocation per
field ([layers, B, H, P, N] f32 for h and last_u, [layers, B, H, N/2] for the
angle), so the whole cache is two (three) contiguous HBM regions.  Steps run
in place through mamba3_step_, which is what keeps decode at the 16 bytes per
state element the recurrence needs.

With `factored=True` the cache holds the second format instead (no reference
counterpart): h plus the previous token's x [layers, B, H, P, R] and
unrotated b [layers, B, H, N, R], last_u being that token's outer product;
steps go through mamba3_step_factored_ and stream 8 bytes per state element.
"""
from __future__ import annotations

from typing import List, Optional, Union

import torch

from .error import ArgumentError
from .ssm.scan import SsmState, SsmStateFactored, mamba3_step_, mamba3_step_factored_


class StateCache:
    """infer/mod.rs:20-48: per-layer decoding state plus a position counter."""

    def __init__(self, n_layers: int, batch: int, heads: int, head_dim: int, d_state: int,
                 rotational: bool, device, init_std: Optional[float] = None,
                 generator: Optional[torch.Generator] = None, factored: bool = False,
                 rank: int = 1, dtype: torch.dtype = torch.bfloat16):
        shape = (n_layers, batch, heads, head_dim, d_state)
        self.factored = factored
        if init_std is None:
            self.h = torch.zeros(shape, dtype=torch.float32, device=device)
        else:
            self.h = torch.randn(shape, dtype=torch.float32, device=device,
                                 generator=generator) * init_std
        self.last_u = self.x_prev = self.b_prev = None
        if factored:
            # a zero previous token (zero last_u); with init_std, random x and b
            xs, bs = (n_layers, batch, heads, head_dim, rank), (n_layers, batch, heads, d_state, rank)
            if init_std is None:
                self.x_prev = torch.zeros(xs, dtype=dtype, device=device)
                self.b_prev = torch.zeros(bs, dtype=dtype, device=device)
            else:
                self.x_prev = torch.randn(xs, device=device, generator=generator).to(dtype)
                self.b_prev = (torch.randn(bs, device=device, generator=generator)
                               / d_state ** 0.5).to(dtype)
        elif init_std is None:
            self.last_u = torch.zeros(shape, dtype=torch.float32, device=device)
        else:
            self.last_u = torch.randn(shape, dtype=torch.float32, device=device,
                                      generator=generator) * init_std
        self.angle = (torch.zeros((n_layers, batch, heads, d_state // 2), dtype=torch.float32,
                                  device=device) if rotational else None)
        ang = lambda i: None if self.angle is None else self.angle[i]
        if factored:
            self._layers = [SsmStateFactored(self.h[i], self.x_prev[i], self.b_prev[i], ang(i))
                            for i in range(n_layers)]
        else:
            self._layers = [SsmState(self.h[i], self.last_u[i], ang(i)) for i in range(n_layers)]
        self._position = 0

    def position(self) -> int:
        """Number of tokens consumed so far."""
        return self._position

    def layers_mut(self) -> List[Union[SsmState, SsmStateFactored]]:
        return self._layers

    def advance(self, tokens: int) -> None:
        self._position += tokens

    def num_bytes(self) -> int:
        n = 4 * (self.h.numel() + (0 if self.angle is None else self.angle.numel()))
        if self.factored:
            return n + self.x_prev.numel() * self.x_prev.element_size() + \
                self.b_prev.numel() * self.b_prev.element_size()
        return n + 4 * self.last_u.numel()

    def step_all(self, inputs) -> List[torch.Tensor]:
        """One step of every layer in one launch (m3_step_layers), in place:
        inputs[l] = (x, b, c, dt, lam, a_log, theta, d_skip) of layer l, all
        of one shape.  Returns each layer's y; the same results as
        step_layer on each layer in turn."""
        import ctypes as C
        from . import _lib
        from .ssm.scan import _step_args, _stream, check_step_state
        if len(inputs) != len(self._layers):
            raise ArgumentError(f"step_all needs one input tuple per layer "
                                f"({len(self._layers)}), got {len(inputs)}")
        n = len(inputs)
        # every layer's inputs and state are checked before anything is
        # launched: the kernel steps each layer's cache slice in place at the
        # inputs' element size and shape
        checked = []
        for l, inp in enumerate(inputs):
            a, k = _step_args(*inp)
            check_step_state(k, inp[6] is not None, self._layers[l])
            checked.append((a, k))
        args = (_lib.StepInputsC * n)()
        keep, ys = [], []
        for l, (a, k) in enumerate(checked):
            args[l] = a
            keep.append(k)
            ys.append(torch.empty_like(k[0]))
        yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        st = self._layers
        if self.factored:
            fs = (_lib.SsmStateFactoredC * n)(*[_lib.SsmStateFactoredC(
                s.h.data_ptr(), s.x_prev.data_ptr(), s.b_prev.data_ptr(),
                None if s.angle is None else s.angle.data_ptr()) for s in st])
            _lib.check(_lib.lib().m3_step_layers(n, args, None, fs, yp, _stream(ys[0])))
        else:
            ss = (_lib.SsmStateC * n)(*[s._c() for s in st])
            _lib.check(_lib.lib().m3_step_layers(n, args, ss, None, yp, _stream(ys[0])))
        return ys

    def step_layer(self, layer: int, x, b, c, dt, lam, a_log, theta=None, d_skip=None):
        """mamba3_step on one layer's slot, in place; returns y [B, H, P, R]."""
        step = mamba3_step_factored_ if self.factored else mamba3_step_
        return step(x, b, c, dt, lam, a_log, theta, d_skip, self._layers[layer])
