"""Checkpoints and state dicts in the reference's JSON format.

Mirrors `TensorData` and `StateDict` (BectorVoom/mamba-trainer
src/nn/module.rs:297-345), `Checkpoint` (src/train/checkpoint.rs:16-83) and
`Module::state_dict` / `Module::load_state_dict` (module.rs:227-285).  Files are
parsed and written by libmamba3_hip.so on the host (include/mamba3_checkpoint.h),
several threads at a time, so a checkpoint of the config-4 model (about 163 M
values) loads in seconds; values are f32 in the file, as in the reference.

A model here exposes `named_parameters()`: (dotted path, Param) pairs in the
reference's visit order, with the reference's paths.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Tuple

import numpy as np

from . import _lib
from .error import ShapeError, StateDictError


@dataclass
class TensorData:
    """module.rs:297-304: dimensions and row-major f32 values."""
    shape: List[int]
    data: np.ndarray

    def __post_init__(self):
        self.shape = [int(d) for d in self.shape]
        self.data = np.ascontiguousarray(np.asarray(self.data, dtype=np.float32).reshape(-1))


@dataclass
class Param:
    """A parameter of a model here: its shape and how to read / replace its
    value as f32 (the reference's `Param::value().to_f32()` / `Param::set`)."""
    shape: Tuple[int, ...]
    get: Callable[[], "object"]          # -> torch float32 tensor of `shape`
    set: Callable[["object"], None]      # torch float32 tensor of `shape` on the model's device

    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n


def _read(path: str, checkpoint: bool):
    L = _lib.lib()
    h = C.c_void_p()
    fn = L.m3_checkpoint_load if checkpoint else L.m3_state_dict_load
    _lib.check(fn(str(path).encode(), C.byref(h)))
    try:
        entries: Dict[str, TensorData] = {}
        name = C.c_char_p()
        ndim = C.c_size_t()
        shape = C.POINTER(C.c_size_t)()
        data = C.POINTER(C.c_float)()
        numel = C.c_size_t()
        for i in range(int(L.m3_state_dict_len(h))):
            _lib.check(L.m3_state_dict_entry(h, i, C.byref(name), C.byref(ndim), C.byref(shape),
                                             C.byref(data), C.byref(numel)))
            dims = [int(shape[d]) for d in range(ndim.value)]
            n = int(numel.value)
            vals = (np.ctypeslib.as_array(data, shape=(n,)).copy() if n
                    else np.zeros(0, dtype=np.float32))
            entries[name.value.decode()] = TensorData(dims, vals)
        step = int(L.m3_checkpoint_step(h))
        meta = json.loads(L.m3_checkpoint_metadata(h).decode())
    finally:
        L.m3_state_dict_free(h)
    return StateDict(entries), step, meta


def _write(path: str, state: "StateDict", checkpoint: bool, step: int = 0, metadata: Any = None):
    keys = list(state.entries.keys())
    n = len(keys)
    tds = [state.entries[k] for k in keys]
    names = (C.c_char_p * max(n, 1))(*[k.encode() for k in keys])
    ndims = (C.c_size_t * max(n, 1))(*[len(t.shape) for t in tds])
    shape_arrs = [(C.c_size_t * max(len(t.shape), 1))(*t.shape) for t in tds]
    shapes = (C.POINTER(C.c_size_t) * max(n, 1))(
        *[C.cast(a, C.POINTER(C.c_size_t)) for a in shape_arrs])
    datas = (C.POINTER(C.c_float) * max(n, 1))(
        *[t.data.ctypes.data_as(C.POINTER(C.c_float)) for t in tds])
    numels = (C.c_size_t * max(n, 1))(*[int(t.data.size) for t in tds])
    meta = json.dumps(metadata).encode() if checkpoint else None
    _lib.check(_lib.lib().m3_state_dict_save(str(path).encode(), 1 if checkpoint else 0, int(step),
                                             meta, n, names, ndims, shapes, datas, numels))


class StateDict:
    """module.rs:306-345: parameter path -> TensorData, kept in key order."""

    def __init__(self, entries: Optional[Dict[str, TensorData]] = None):
        self.entries: Dict[str, TensorData] = dict(sorted((entries or {}).items()))

    def save(self, path) -> None:
        """module.rs:318-322."""
        _write(path, self, checkpoint=False)

    @staticmethod
    def load(path) -> "StateDict":
        """module.rs:325-329."""
        return _read(path, checkpoint=False)[0]

    def filter(self, pattern: str) -> "StateDict":
        """module.rs:333-343: entries whose key contains `pattern`."""
        return StateDict({k: v for k, v in self.entries.items() if pattern in k})

    def __len__(self) -> int:
        return len(self.entries)


def state_dict(model) -> StateDict:
    """module.rs:227-244: every parameter, as host f32, keyed by path."""
    out = {}
    for name, p in model.named_parameters():
        v = p.get().detach().float().cpu().numpy().reshape(-1)
        out[name] = TensorData(list(p.shape), v)
    return StateDict(out)


def load_state_dict(model, state: StateDict, strict: bool = True) -> None:
    """module.rs:249-285, rule for rule: with `strict` every parameter needs an
    entry and every entry a parameter; a shape mismatch is an error; entries are
    applied in parameter order (an error part way leaves the earlier ones set,
    as there)."""
    import torch
    params = model.named_parameters()
    if strict:
        names = {n for n, _ in params}
        for n, _ in params:
            if n not in state.entries:
                raise StateDictError(f"state dict error: missing entry for `{n}`")
        for n in state.entries:
            if n not in names:
                raise StateDictError(f"state dict error: unexpected entry `{n}`")
    for n, p in params:
        e = state.entries.get(n)
        if e is None:
            continue
        expected = list(p.shape)
        if list(e.shape) != expected:
            raise StateDictError(f"state dict error: `{n}`: checkpoint holds {list(e.shape)} but "
                                 f"the model expects {expected}")
        if e.data.size != p.numel():
            # Tensor::from_data (tensor/base.rs:74-81)
            raise ShapeError(f"shape error: data of length {e.data.size} does not fill shape "
                             f"{expected}")
        p.set(torch.from_numpy(e.data.reshape(expected)))


@dataclass
class Checkpoint:
    """checkpoint.rs:16-83: a state dict plus the step count and free-form JSON
    metadata (usually the model configuration)."""
    step: int = 0
    state: StateDict = field(default_factory=StateDict)
    metadata: Any = None

    @staticmethod
    def capture(model, step: int) -> "Checkpoint":
        return Checkpoint(step, state_dict(model), None)

    def with_metadata(self, metadata: Any) -> "Checkpoint":
        self.metadata = metadata
        return self

    def filtered(self, pattern: str) -> "Checkpoint":
        return Checkpoint(self.step, self.state.filter(pattern), self.metadata)

    def save(self, path) -> None:
        _write(path, self.state, checkpoint=True, step=self.step, metadata=self.metadata)

    @staticmethod
    def load(path) -> "Checkpoint":
        state, step, meta = _read(path, checkpoint=True)
        return Checkpoint(step, state, meta)

    def restore(self, model, strict: bool = True) -> None:
        load_state_dict(model, self.state, strict)

    def num_values(self) -> int:
        return sum(int(e.data.size) for e in self.state.entries.values())
