"""Layers around the scan, over the C ABI of mamba3_mixer.h (bf16 activations).

Mirrors the reference's `nn` items the Mamba-3 language model uses:
RmsNorm (src/nn/norm.rs:17-105), Linear with an optional int8 weight fake
quantizer (src/nn/linear.rs:40-185, src/nn/quant.rs:95-103, 231-330), Embedding
(src/nn/embedding.rs) and the initialisers (src/nn/init.rs:90-110).  Weights
are held on the device; every computation runs in libmamba3_hip.so.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional

import torch

from . import _lib
from .error import ArgumentError, ShapeError, UnsupportedError


def _stream(t: torch.Tensor):
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _bf16_dev(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ArgumentError(f"{what} must be a ROCm device tensor (there is no CPU path)")
    if t.dtype != torch.bfloat16:
        raise ArgumentError(f"{what} must be bfloat16, got {t.dtype}")
    return t.contiguous()


def normal(shape, std: float, device, gen: torch.Generator) -> torch.Tensor:
    """Initializer::Normal {mean 0, std} (init.rs:98-100)."""
    return torch.randn(shape, device=device, generator=gen, dtype=torch.float32) * std


def residual_scaled(shape, std: float, n_layers: int, device, gen: torch.Generator) -> torch.Tensor:
    """Initializer::ResidualScaled: std / sqrt(2 * n_layers) (init.rs:105-108)."""
    return normal(shape, std / math.sqrt(2.0 * max(n_layers, 1)), device, gen)


def tensor_param(owner, attr: str):
    """A checkpoint Param over an f32 device tensor held as `owner.<attr>`."""
    from .checkpoint import Param
    t = getattr(owner, attr)
    return Param(tuple(t.shape), lambda: getattr(owner, attr),
                 lambda v: getattr(owner, attr).copy_(v.to(torch.float32)))


_WS = {}


def linear_workspace(device) -> torch.Tensor:
    """The scratch m3_linear may use (one per device; stream-ordered use)."""
    key = (device.type, device.index)
    ws = _WS.get(key)
    if ws is None:
        ws = torch.empty(int(_lib.lib().m3_linear_workspace_bytes()), dtype=torch.uint8,
                         device=device)
        _WS[key] = ws
    return ws


class RmsNorm:
    """norm.rs:70-105: y = x * rsqrt(mean(x^2) + eps) * w over the last axis."""

    def __init__(self, dim: int, device, eps: float = 1e-5, weight: bool = True):
        self.dim, self.eps = dim, eps
        self.weight = torch.ones(dim, dtype=torch.float32, device=device) if weight else None

    def apply(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = _bf16_dev(x, "RmsNorm input")
        if x.shape[-1] != self.dim:
            raise ShapeError(f"shape error: RmsNorm expects a trailing dimension of {self.dim}, "
                             f"got {tuple(x.shape)}")
        y = torch.empty_like(x) if out is None else out
        rows = x.numel() // self.dim
        _lib.check(_lib.lib().m3_rms_norm(rows, self.dim, x.data_ptr(), self.dim,
                                          None if self.weight is None else self.weight.data_ptr(),
                                          C.c_float(self.eps), y.data_ptr(), self.dim, _stream(x)))
        return y


class Linear:
    """linear.rs:40-185 for bf16 activations: y = x @ w, w stored
    [in_features, out_features] as in the reference (no bias term).

    With `int8_weights` (QuantConfig::int8_weights, quant.rs:95-103) the weight
    used is the fake-quantized w' = code * scale (per output channel); the
    codes go to the GEMM as exact bf16 and the scales are applied in its
    epilogue, so w' is never rounded to bf16.  Without it the weight is used
    as bf16.  The GEMM operand is held transposed, codes_t [out, in]
    (m3_linear_nt); `codes` is its [in, out] view.
    """

    def __init__(self, weight: torch.Tensor, int8_weights: bool = False,
                 bias: Optional[torch.Tensor] = None):
        if weight.dim() != 2:
            raise ShapeError(f"shape error: a Linear weight is [in, out], got {tuple(weight.shape)}")
        if bias is not None:
            # SsmConfig::bias is false for the projections of every model here
            raise UnsupportedError("unsupported: Linear bias is not on the gfx950 path")
        self.weight = weight.float().contiguous()          # master copy, f32
        self.int8_weights = int8_weights
        self.codes: Optional[torch.Tensor] = None
        self.codes_t: Optional[torch.Tensor] = None
        self.scales: Optional[torch.Tensor] = None
        self.prepare()

    @property
    def in_features(self) -> int:
        return self.weight.shape[0]

    @property
    def out_features(self) -> int:
        return self.weight.shape[1]

    def prepare(self) -> None:
        """Derive the GEMM operands from the master weight (after any update)."""
        k, n = self.weight.shape
        if self.int8_weights:
            codes = torch.empty((k, n), dtype=torch.bfloat16, device=self.weight.device)
            self.scales = torch.empty(n, dtype=torch.float32, device=self.weight.device)
            _lib.check(_lib.lib().m3_quantize_int8_columns(
                k, n, self.weight.data_ptr(), codes.data_ptr(), self.scales.data_ptr(),
                _stream(self.weight)))
        else:
            codes = self.weight.to(torch.bfloat16)
            self.scales = None
        self.codes_t = codes.t().contiguous()
        self.codes = self.codes_t.t()

    def param(self):
        """The master weight [in, out] as a checkpoint Param; setting it
        re-derives the GEMM operands (codes and scales)."""
        from .checkpoint import Param

        def put(v):
            self.weight.copy_(v.to(torch.float32))
            self.prepare()
        return Param(tuple(self.weight.shape), lambda: self.weight, put)

    def effective_weight(self) -> torch.Tensor:
        """The weight the product uses, in f32 (w' for the quantized form)."""
        if self.scales is None:
            return self.codes.float()
        return self.codes.float() * self.scales

    def apply(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [..., in] -> [..., out]; `residual` [..., out] is added (it may be `out`)."""
        x = _bf16_dev(x, "Linear input")
        if x.shape[-1] != self.in_features:
            raise ShapeError(f"shape error: Linear expects a trailing dimension of "
                             f"{self.in_features}, got {tuple(x.shape)}")
        m = x.numel() // self.in_features
        shape = tuple(x.shape[:-1]) + (self.out_features,)
        y = torch.empty(shape, dtype=torch.bfloat16, device=x.device) if out is None else out
        if residual is not None:
            residual = _bf16_dev(residual, "Linear residual")
        ws = linear_workspace(x.device)
        _lib.check(_lib.lib().m3_linear_nt(
            m, self.in_features, self.out_features, x.data_ptr(), self.codes_t.data_ptr(),
            None if self.scales is None else self.scales.data_ptr(),
            None if residual is None else residual.data_ptr(), y.data_ptr(), ws.data_ptr(),
            ws.numel(), _stream(x)))
        return y


class Embedding:
    """embedding.rs: a [vocab, dim] table (Normal std 0.02), bf16 rows."""

    def __init__(self, table: torch.Tensor):
        self.table = table.to(torch.bfloat16).contiguous()

    @property
    def vocab(self) -> int:
        return self.table.shape[0]

    @property
    def dim(self) -> int:
        return self.table.shape[1]

    def param(self):
        """The table as a checkpoint Param: read as f32, stored back as bf16
        (round to nearest even, as the reference's from_f32 for bf16)."""
        from .checkpoint import Param
        return Param(tuple(self.table.shape), lambda: self.table.float(),
                     lambda v: self.table.copy_(v.to(torch.float32).to(torch.bfloat16)))

    def lookup(self, ids: torch.Tensor) -> torch.Tensor:
        if not ids.is_cuda:
            raise ArgumentError("ids must be a ROCm device tensor (there is no CPU path)")
        ids32 = ids.to(torch.int32).contiguous()
        out = torch.empty(tuple(ids.shape) + (self.dim,), dtype=torch.bfloat16, device=ids.device)
        _lib.check(_lib.lib().m3_embedding_lookup(ids32.numel(), self.dim, ids32.data_ptr(),
                                                  self.vocab, self.table.data_ptr(),
                                                  out.data_ptr(), _stream(ids32)))
        return out
