"""Weight ingestion on the gfx950 path: checkpoints in the reference's format
(src/train/checkpoint.rs, src/nn/module.rs) restored into Mamba3Lm and run.

The first two tests are the reference's own (tests/train.rs:241-275,
tests/model.rs:245-262).  The third writes the oracle model's weights under
the reference's parameter paths with Python's json module (not this library's
writer), loads them through the library's parser and requires the logits of
the oracle model (with and without the causal convolution); the same file
with B's and C's biases swapped, or with the convolution weight's B and C
channel blocks swapped, must not pass, so a misplaced tensor is visible.
"""
import dataclasses
import json

import numpy as np
import pytest
import torch

import mixer_oracle as mo
from cases import rel_l2

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _ssm(d_model=16, heads=2, head_dim=8, d_state=8, groups=None, rot=True, learned=True, rank=1,
         conv=None):
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    return SsmConfig(d_model=d_model, n_heads=heads, head_dim=head_dim, d_state=d_state,
                     n_groups=groups or heads,
                     discretization=Discretization.LearnedTrapezoid if learned else Discretization.Trapezoid,
                     dynamics=StateDynamics.Rotational if rot else StateDynamics.Real,
                     mode=SsmMode(rank), chunk_size=64, conv_kernel=conv)


def tiny_lm(seed, int8=True):
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    return Mamba3Lm(Mamba3LmConfig(vocab_size=8, d_model=16, n_layers=2, ssm=_ssm(),
                                   int8_weights=int8, seed=seed), DEV)


def max_abs_diff(a, b):
    return float(np.max(np.abs(a - b)))


def test_checkpoints_round_trip_and_can_be_filtered(tmp_path):
    """tests/train.rs:241-275."""
    from mamba3.checkpoint import Checkpoint
    path = tmp_path / "model.json"
    source = tiny_lm(12)
    checkpoint = Checkpoint.capture(source, 42).with_metadata({"note": "unit test"})
    checkpoint.save(path)

    loaded = Checkpoint.load(path)
    assert loaded.step == 42
    assert loaded.metadata["note"] == "unit test"

    target = tiny_lm(13)
    tokens = torch.tensor([[1, 2, 3, 4]], device=DEV)
    before = host(target.forward(tokens))
    loaded.restore(target, True)
    after = host(target.forward(tokens))
    expected = host(source.forward(tokens))
    assert max_abs_diff(before, expected) > 1e-5
    assert max_abs_diff(after, expected) < 1e-6

    filtered = checkpoint.filtered("in_proj")
    assert len(filtered.state.entries) > 0
    assert len(filtered.state.entries) < len(checkpoint.state.entries)
    assert all("in_proj" in k for k in filtered.state.entries)


def test_state_dict_round_trips():
    """tests/model.rs:245-262: a perturbed model takes another's state dict and
    then reproduces its output."""
    source, target = tiny_lm(1), tiny_lm(1)
    tokens = torch.tensor([[1, 2, 3, 4]], device=DEV)
    for _, p in target.named_parameters():
        p.set(p.get().float() + 0.1)
    before = host(target.forward(tokens))
    expected = host(source.forward(tokens))
    assert max_abs_diff(before, expected) > 1e-4
    target.load_state_dict(source.state_dict(), True)
    after = host(target.forward(tokens))
    assert max_abs_diff(after, expected) < 1e-6


def _reference_state_dict(model):
    """The oracle model's weights as the reference would save them: dotted paths
    of lm.rs:355-362 / hybrid.rs:497-516 / mamba3.rs:634-656, f32 values."""
    ent = {}

    def put(name, arr):
        a = np.asarray(arr, np.float32)
        ent[name] = {"shape": list(a.shape), "data": [float(v) for v in a.reshape(-1)]}

    put("embed.weight", model["embed"])
    for i, layer in enumerate(model["layers"]):
        pre = f"stack.layers.{i}."
        put(pre + "norm.weight", layer["norm"])
        put(pre + "mixer.in_proj.weight", layer["in_proj_master"])
        put(pre + "mixer.out_proj.weight", layer["out_proj_master"])
        if layer.get("conv_w") is not None:
            put(pre + "mixer.conv.weight", layer["conv_w"])
            put(pre + "mixer.conv.bias", layer["conv_b"])
        put(pre + "mixer.dt_bias", layer["dt_bias"])
        put(pre + "mixer.a_log", layer["a_log"])
        put(pre + "mixer.d", layer["d_skip"])
        put(pre + "mixer.b_bias", layer["b_bias"])
        put(pre + "mixer.c_bias", layer["c_bias"])
        put(pre + "mixer.bc_norm.weight", layer["bc_norm"])
    put("norm_f.weight", model["norm_f"])
    put("head.weight", model["head"])
    return ent


@pytest.mark.parametrize("rank,conv", [(1, None), (2, None), (1, 4), (2, 4)])
def test_ingested_weights_run_as_the_oracle_model(tmp_path, rank, conv):
    """With conv_kernel 4 the file carries each layer's mixer.conv.weight
    [4, channels] and mixer.conv.bias (nn/conv.rs visit order, after out_proj);
    a third file, with only the convolution weight's B and C channel blocks
    exchanged, must not pass either."""
    from mamba3.checkpoint import Checkpoint
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    rng = np.random.default_rng(70 + rank + (conv or 0))
    model = mo.random_model(rng, vocab=32, d_model=32, n_layers=2, heads=4, head_dim=8, d_state=16,
                            rank=rank, groups=2, int8=True, bias_scale=0.3, conv_kernel=conv)
    ent = _reference_state_dict(model)
    good = tmp_path / "good.json"
    good.write_text(json.dumps({"step": 1000, "state": {"entries": ent},
                                "metadata": {"d_model": 32}}))
    swapped, conv_swapped = dict(ent), dict(ent)
    din, bcw, _, _ = mo.widths(model["cfg"])
    for i in range(2):
        pre = f"stack.layers.{i}.mixer."
        swapped[pre + "b_bias"], swapped[pre + "c_bias"] = ent[pre + "c_bias"], ent[pre + "b_bias"]
        if conv is not None:
            cw = ent[pre + "conv.weight"]
            w = np.asarray(cw["data"]).reshape(cw["shape"])
            w = np.concatenate([w[:, :din], w[:, din + bcw:], w[:, din:din + bcw]], axis=1)
            conv_swapped[pre + "conv.weight"] = {"shape": cw["shape"],
                                                 "data": [float(v) for v in w.reshape(-1)]}
    files = {"good": good}
    for name, entries in (("swapped", swapped),) + ((("conv_swapped", conv_swapped),)
                                                    if conv is not None else ()):
        files[name] = tmp_path / f"{name}.json"
        files[name].write_text(json.dumps({"step": 1000, "state": {"entries": entries},
                                           "metadata": None}))

    cfg = Mamba3LmConfig(vocab_size=32, d_model=32, n_layers=2,
                         ssm=_ssm(d_model=32, heads=4, head_dim=8, d_state=16, groups=2, rank=rank,
                                  conv=conv),
                         int8_weights=True, seed=99)
    ids = rng.integers(0, 32, (2, 37))
    ref = mo.lm_forward(ids, model, rnd=True)
    errs = {}
    for name, path in files.items():
        lm = Mamba3Lm(cfg, DEV)
        ck = Checkpoint.load(path)
        assert ck.step == 1000
        ck.restore(lm, strict=True)
        got = host(lm.forward(torch.from_numpy(ids).to(DEV)))
        errs[name] = rel_l2(got, ref)
    assert errs["good"] <= 1e-2, errs
    assert errs["swapped"] > 5e-2, errs
    assert conv is None or errs["conv_swapped"] > 5e-2, errs
