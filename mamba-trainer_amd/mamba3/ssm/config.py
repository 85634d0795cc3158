"""SsmConfig and its enums (src/ssm/config.rs:5-347), validated through the C ABI."""
from __future__ import annotations

import ctypes as C
import dataclasses
import enum
import math
from typing import Optional

from .. import _lib


class Discretization(enum.IntEnum):
    """config.rs:19-26."""
    Euler = 0
    Trapezoid = 1
    LearnedTrapezoid = 2

    def fixed_lambda(self) -> Optional[float]:
        """config.rs:29-36: 1 for Euler, 1/2 for Trapezoid, None when learned."""
        v = float(_lib.lib().m3_discretization_fixed_lambda(int(self)))
        return None if math.isnan(v) else v

    def needs_lambda_projection(self) -> bool:
        return self is Discretization.LearnedTrapezoid


class StateDynamics(enum.IntEnum):
    """config.rs:46-55."""
    Real = 0
    Rotational = 1


@dataclasses.dataclass(frozen=True)
class SsmMode:
    """config.rs:59-80: Siso is rank 1, Mimo{rank} is rank R."""
    rank_: int = 1

    @staticmethod
    def siso() -> "SsmMode":
        return SsmMode(1)

    @staticmethod
    def mimo(rank: int) -> "SsmMode":
        return SsmMode(rank)

    def rank(self) -> int:
        return self.rank_


@dataclasses.dataclass
class SsmConfig:
    """config.rs:84-156 (fields and defaults)."""
    d_model: int = 768
    n_heads: int = 24
    head_dim: int = 64
    d_state: int = 64
    n_groups: int = 24
    discretization: Discretization = Discretization.LearnedTrapezoid
    dynamics: StateDynamics = StateDynamics.Rotational
    mode: SsmMode = dataclasses.field(default_factory=SsmMode.siso)
    chunk_size: int = 64
    conv_kernel: Optional[int] = 4
    bc_norm: bool = True
    bc_bias: bool = True
    post_gate_norm: bool = False
    skip_connection: bool = True
    dt_min: float = 0.001
    dt_max: float = 0.1
    dt_init_floor: float = 1e-4
    a_init_min: float = 1.0
    a_init_max: float = 16.0
    bias: bool = False

    def _c(self) -> _lib.SsmConfigC:
        return _lib.SsmConfigC(
            self.d_model, self.n_heads, self.head_dim, self.d_state, self.n_groups,
            int(self.discretization), int(self.dynamics), self.mode.rank(), self.chunk_size,
            0 if self.conv_kernel is None else self.conv_kernel,
            int(self.bc_norm), int(self.bc_bias), int(self.post_gate_norm),
            int(self.skip_connection), self.dt_min, self.dt_max, self.dt_init_floor,
            self.a_init_min, self.a_init_max, int(self.bias))

    @staticmethod
    def default_from_abi() -> "SsmConfig":
        """The ABI's own defaults (m3_config_default)."""
        c = _lib.SsmConfigC()
        _lib.check(_lib.lib().m3_config_default(C.byref(c)))
        return SsmConfig(
            c.d_model, c.n_heads, c.head_dim, c.d_state, c.n_groups,
            Discretization(c.discretization), StateDynamics(c.dynamics), SsmMode(c.rank),
            c.chunk_size, None if c.conv_kernel == 0 else c.conv_kernel, bool(c.bc_norm),
            bool(c.bc_bias), bool(c.post_gate_norm), bool(c.skip_connection), c.dt_min,
            c.dt_max, c.dt_init_floor, c.a_init_min, c.a_init_max, bool(c.bias))

    @staticmethod
    def builder() -> "SsmConfigBuilder":
        return SsmConfigBuilder()

    def validate(self) -> None:
        """config.rs:203-245 (raises ConfigError)."""
        if self.conv_kernel is not None and self.conv_kernel < 2:
            # a width of 0 or 1 cannot be told apart from None in the C struct
            from ..error import ConfigError
            raise ConfigError("invalid configuration: conv_kernel must be at least 2; "
                              "use None to disable")
        _lib.check(_lib.lib().m3_config_validate(C.byref(self._c())))

    def d_inner(self) -> int:
        return int(_lib.lib().m3_config_d_inner(C.byref(self._c())))

    def bc_width(self) -> int:
        return int(_lib.lib().m3_config_bc_width(C.byref(self._c())))

    def theta_width(self) -> int:
        return int(_lib.lib().m3_config_theta_width(C.byref(self._c())))

    def lambda_width(self) -> int:
        return int(_lib.lib().m3_config_lambda_width(C.byref(self._c())))

    def in_proj_width(self) -> int:
        return int(_lib.lib().m3_config_in_proj_width(C.byref(self._c())))


class SsmConfigBuilder:
    """config.rs:248-347."""

    def __init__(self):
        self._config = SsmConfig()

    def __getattr__(self, name):
        fields = {f.name for f in dataclasses.fields(SsmConfig)}
        if name in fields:
            def setter(value):
                setattr(self._config, name, value)
                return self
            return setter
        raise AttributeError(name)

    def dt_range(self, lo: float, hi: float):
        self._config.dt_min, self._config.dt_max = lo, hi
        return self

    def a_init_range(self, lo: float, hi: float):
        self._config.a_init_min, self._config.a_init_max = lo, hi
        return self

    def expand(self, expansion: float):
        c = self._config
        inner = int(c.d_model * expansion)
        per_head = c.head_dim * c.mode.rank()
        c.n_heads = max(inner // max(per_head, 1), 1)
        c.n_groups = c.n_heads
        return self

    def build(self) -> SsmConfig:
        self._config.validate()
        return self._config
