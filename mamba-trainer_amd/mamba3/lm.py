"""The Mamba-3 causal language model (all-Mamba stack), bf16 activations.

Mirrors `Mamba3Lm` (BectorVoom/mamba-trainer src/models/lm.rs:40-360) over the
`HybridStack` with `LayerPattern::AllMamba` and no feed-forward blocks
(src/models/hybrid.rs:142-157, 413-493): embedding, n_layers x
[RmsNorm -> Mamba3Mixer -> residual add], final RmsNorm, untied output head.
The residual add is the epilogue of each mixer's output projection.

Not covered (raise UnsupportedError): attention layers, MLP blocks, tied
embeddings, dropout, LoRA and activation quantization.
"""
from __future__ import annotations

import dataclasses
from typing import List, Optional

import torch

from .error import ShapeError, UnsupportedError
from .mixer import Mamba3Mixer, MixerCache
from .nn import Embedding, Linear, RmsNorm, normal, tensor_param
from .ssm import SsmConfig


@dataclasses.dataclass
class Mamba3LmConfig:
    """lm.rs:40-64 with the stack fields of hybrid.rs:142-157 that apply here."""
    vocab_size: int = 32_000
    d_model: int = 768
    n_layers: int = 12
    ssm: SsmConfig = dataclasses.field(default_factory=SsmConfig)
    int8_weights: bool = False       # QuantConfig::int8_weights on the mixer projections
    norm_eps: float = 1e-5
    tie_embeddings: bool = False
    seed: int = 0

    def validate(self) -> None:
        if self.vocab_size == 0 or self.d_model == 0 or self.n_layers == 0:
            from .error import ConfigError
            raise ConfigError("invalid configuration: d_model and n_layers must be positive")
        if self.tie_embeddings:
            raise UnsupportedError("unsupported: tied embeddings are not on the gfx950 path")
        ssm = dataclasses.replace(self.ssm, d_model=self.d_model)
        ssm.validate()


class Mamba3Lm:
    """lm.rs:248-360 for the all-Mamba stack."""

    def __init__(self, cfg: Mamba3LmConfig, device):
        cfg.validate()
        self.cfg = cfg
        gen = torch.Generator(device=device)
        gen.manual_seed(cfg.seed)
        ssm = dataclasses.replace(cfg.ssm, d_model=cfg.d_model)
        self.embed = Embedding(normal((cfg.vocab_size, cfg.d_model), 0.02, device, gen))
        self.layers: List[tuple] = []
        for _ in range(cfg.n_layers):
            norm = RmsNorm(cfg.d_model, device, eps=cfg.norm_eps)
            mixer = Mamba3Mixer(ssm, device=device, gen=gen, n_layers=cfg.n_layers,
                                int8_weights=cfg.int8_weights)
            self.layers.append((norm, mixer))
        self.norm_f = RmsNorm(cfg.d_model, device, eps=cfg.norm_eps)
        self.head = Linear(normal((cfg.d_model, cfg.vocab_size), 0.02, device, gen))

    # ------------------------------------------------------------ parameters
    def named_parameters(self):
        """lm.rs:355-362 over hybrid.rs:497-516: embed, stack.layers.{i}.{norm,
        mixer}, norm_f, head -- the paths of the reference's state dicts."""
        out = [("embed.weight", self.embed.param())]
        for i, (norm, mixer) in enumerate(self.layers):
            pre = f"stack.layers.{i}."
            if norm.weight is not None:
                out.append((pre + "norm.weight", tensor_param(norm, "weight")))
            out += [(pre + "mixer." + n, p) for n, p in mixer.named_parameters()]
        if self.norm_f.weight is not None:
            out.append(("norm_f.weight", tensor_param(self.norm_f, "weight")))
        out.append(("head.weight", self.head.param()))
        return out

    def num_parameters(self) -> int:
        return sum(p.numel() for _, p in self.named_parameters())

    def state_dict(self):
        from .checkpoint import state_dict
        return state_dict(self)

    def load_state_dict(self, state, strict: bool = True) -> None:
        from .checkpoint import load_state_dict
        load_state_dict(self, state, strict)

    # ------------------------------------------------------------ forward
    def hidden(self, ids: torch.Tensor) -> torch.Tensor:
        """lm.rs:295-303: the residual stream after the stack and the final norm."""
        if ids.dim() != 2:
            raise ShapeError(f"shape error: ids must be [batch, seq], got {tuple(ids.shape)}")
        x = self.embed.lookup(ids)
        normed = torch.empty_like(x)
        for norm, mixer in self.layers:
            norm.apply(x, out=normed)
            mixer.apply(normed, residual=x, out=x)      # x += mixer(norm(x))
        return self.norm_f.apply(x)

    def logits_from(self, hidden: torch.Tensor) -> torch.Tensor:
        """lm.rs:305-317 (untied head)."""
        return self.head.apply(hidden)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """lm.rs:319-327 (inference: no autodiff)."""
        return self.logits_from(self.hidden(ids))

    def empty_cache(self, batch: int, device, factored: bool = False) -> List[Optional[MixerCache]]:
        """lm.rs:330-335: one (zeroed) mixer cache per layer; factored=True
        keeps each layer's state in the factored form (decode steps stream h
        only; no reference counterpart)."""
        return [mixer.empty_cache(batch, device, factored) for _, mixer in self.layers]

    def forward_cached(self, ids: torch.Tensor, cache: List[MixerCache]) -> torch.Tensor:
        """lm.rs:337-353 / hybrid.rs:424-493: a window or one token through the
        stack, each layer's state carried in `cache` (updated in place)."""
        if len(cache) != len(self.layers):
            from .error import ConfigError
            raise ConfigError(f"invalid configuration: cache has {len(cache)} entries but the "
                              f"stack has {len(self.layers)} layers")
        x = self.embed.lookup(ids)
        normed = torch.empty_like(x)
        single = ids.shape[1] == 1
        for i, (norm, mixer) in enumerate(self.layers):
            norm.apply(x, out=normed)
            if single:
                mixer.step_(normed, cache[i], residual=x, out=x)
            else:
                _, cache[i] = mixer.apply_with_state(normed, cache[i], residual=x, out=x)
        return self.logits_from(self.norm_f.apply(x))

    def capture_decode(self, cache: List[MixerCache], batch: int) -> "DecodeGraph":
        """forward_cached for one token per sequence, captured once as a HIP
        graph over `cache` (whose states each replay updates in place).  No
        reference counterpart: the reference issues every op from the host."""
        return DecodeGraph(self, cache, batch)


class DecodeGraph:
    """One decode step of a Mamba3Lm (`forward_cached` over [batch, 1] ids,
    the cache's states updated in place) as a captured HIP graph: a replay
    sends the step's ~150 kernels to the GPU as one graph launch, with none of
    the host work of issuing them one by one.

    Capture records the cache's buffers (states and convolution histories):
    replays read and update those same tensors, so the cache must stay alive
    and keep its storage.  The warm-up before capture runs on copies of the
    cache (it settles the GEMM plans, whose first call times candidates and
    blocks, which capture forbids), so capturing does not advance the
    caller's states."""

    def __init__(self, lm: Mamba3Lm, cache: List[MixerCache], batch: int):
        dev = cache[0].ssm.h.device
        self.ids = torch.zeros((batch, 1), dtype=torch.int64, device=dev)
        scratch = [c.clone() for c in cache]
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            lm.forward_cached(self.ids, scratch)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = lm.forward_cached(self.ids, cache)
        self._captured = (lm, cache)

    def step(self, ids: torch.Tensor) -> torch.Tensor:
        """Replays the step for `ids` [batch, 1]; returns the logits buffer,
        which the next replay overwrites."""
        if tuple(ids.shape) != tuple(self.ids.shape):
            raise ShapeError(f"shape error: the captured step takes ids of shape "
                             f"{tuple(self.ids.shape)}, got {tuple(ids.shape)}")
        self.ids.copy_(ids)
        self.graph.replay()
        return self.logits
