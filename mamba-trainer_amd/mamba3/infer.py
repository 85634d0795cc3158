"""The decode-time state cache (src/infer/mod.rs:19-48) over the gfx950 step kernel.

One SsmState per Mamba layer, stored as views into a single allocation per
field ([layers, B, H, P, N] f32 for h and last_u, [layers, B, H, N/2] for the
angle), so the whole cache is two (three) contiguous HBM regions.  Steps run
in place through mamba3_step_, which is what keeps decode at the 16 bytes per
state element the recurrence needs.
"""
from __future__ import annotations

from typing import List, Optional

import torch

from .ssm.scan import SsmState, mamba3_step_


class StateCache:
    """infer/mod.rs:20-48: per-layer decoding state plus a position counter."""

    def __init__(self, n_layers: int, batch: int, heads: int, head_dim: int, d_state: int,
                 rotational: bool, device, init_std: Optional[float] = None,
                 generator: Optional[torch.Generator] = None):
        shape = (n_layers, batch, heads, head_dim, d_state)
        if init_std is None:
            self.h = torch.zeros(shape, dtype=torch.float32, device=device)
            self.last_u = torch.zeros(shape, dtype=torch.float32, device=device)
        else:
            self.h = torch.randn(shape, dtype=torch.float32, device=device,
                                 generator=generator) * init_std
            self.last_u = torch.randn(shape, dtype=torch.float32, device=device,
                                      generator=generator) * init_std
        self.angle = (torch.zeros((n_layers, batch, heads, d_state // 2), dtype=torch.float32,
                                  device=device) if rotational else None)
        self._layers: List[SsmState] = [
            SsmState(self.h[i], self.last_u[i], None if self.angle is None else self.angle[i])
            for i in range(n_layers)]
        self._position = 0

    def position(self) -> int:
        """Number of tokens consumed so far."""
        return self._position

    def layers_mut(self) -> List[SsmState]:
        return self._layers

    def advance(self, tokens: int) -> None:
        self._position += tokens

    def num_bytes(self) -> int:
        n = self.h.numel() + self.last_u.numel() + (0 if self.angle is None else self.angle.numel())
        return 4 * n

    def step_layer(self, layer: int, x, b, c, dt, lam, a_log, theta=None, d_skip=None):
        """mamba3_step on one layer's slot, in place; returns y [B, H, P, R]."""
        return mamba3_step_(x, b, c, dt, lam, a_log, theta, d_skip, self._layers[layer])
