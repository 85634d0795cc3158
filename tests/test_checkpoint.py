"""Weight ingestion on the host (no GPU): the reference's JSON checkpoint and
state-dict format (src/train/checkpoint.rs:16-83, src/nn/module.rs:297-345,
serde_json's encoding) read and written by libmamba3_hip.so.

Pinned by hand-written fixtures in that encoding (tests/golden/*.json), by
files written with Python's own json module, by bit-exact round trips of
awkward f32 values, by serde_json's number rule (the nearest double, then f32),
and by the reference's state-dict rules (module.rs:249-285) on a model built on
the CPU.
"""
import json
import math

from pathlib import Path

import numpy as np
import pytest

from mamba3 import checkpoint as ck
from mamba3.error import IoError, JsonError, ShapeError, StateDictError

GOLD = Path(__file__).resolve().parent / "golden"


def f32(*v):
    return np.array(v, dtype=np.float32)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_checkpoint_fixture():
    c = ck.Checkpoint.load(GOLD / "checkpoint_tiny.json")
    assert c.step == 7
    assert c.metadata == {"note": "unit test", "lr": 0.001}
    assert list(c.state.entries) == ["a.weight", "b", 'c"qé']
    a = c.state.entries["a.weight"]
    assert a.shape == [2, 3]
    want = f32(1.0, -0.0, 0.1, np.finfo(np.float32).max, 1e-45, -2.5)
    assert np.array_equal(bits(a.data), bits(want))          # -0.0 and the subnormal kept
    assert c.state.entries["b"].shape == []
    assert c.state.entries["b"].data.tolist() == [16777216.0]  # 2^24 + 1 rounds to even
    assert c.state.entries['c"qé'].shape == [0] and c.state.entries['c"qé'].data.size == 0
    assert c.num_values() == 7


def test_pretty_state_dict_fixture_with_unknown_fields():
    sd = ck.StateDict.load(GOLD / "state_dict_pretty.json")
    assert list(sd.entries) == ["embed.weight", "stack.layers.0.mixer.dt_bias"]
    assert np.array_equal(sd.entries["stack.layers.0.mixer.dt_bias"].data, f32(-4.5, 100.0, 2.0 ** -14))
    e = sd.entries["embed.weight"]
    assert e.shape == [1, 2]
    assert np.array_equal(bits(e.data), bits(f32(np.float32(1.0) / np.float32(3.0), -7.0)))


def test_numbers_go_through_the_nearest_double(tmp_path):
    """serde_json reads a number as f64 and then casts: a decimal just above the
    f32 midpoint 1 + 2^-24 rounds to that midpoint in f64, then ties to even
    (1.0); a direct f32 parse would give 1 + 2^-23."""
    path = tmp_path / "round.json"
    if True:
        path.write_text('{"entries":{"x":{"shape":[3],"data":['
                        '1.00000005960464477539062500000000001,'
                        '1.0000000596046448,-1e-50]}}}')
        x = ck.StateDict.load(path).entries["x"].data
        assert x[0] == 1.0
        assert x[1] == np.float32(1.0000000596046448)
        assert bits(x[2:]) == bits(f32(-0.0))             # underflow keeps the sign


def test_round_trip_is_bit_exact(tmp_path):
    rng = np.random.default_rng(0)
    awkward = f32(0.0, -0.0, 1e-45, -1e-45, 1.1754942e-38, 1.17549435e-38, 3.4028235e38,
                  -3.4028235e38, 0.1, 1 / 3, 16777216.0, 123456789.0, 1e-7, 5e-324)
    rand = (rng.standard_normal(5000) * 10.0 ** rng.integers(-30, 30, 5000)).astype(np.float32)
    sd = ck.StateDict({"z.last": ck.TensorData([awkward.size], awkward),
                       "a.first": ck.TensorData([50, 100], rand),
                       "m.empty": ck.TensorData([0, 3], np.zeros(0, np.float32))})
    p = tmp_path / "sd.json"
    sd.save(p)
    back = ck.StateDict.load(p)
    assert list(back.entries) == ["a.first", "m.empty", "z.last"]
    for k in sd.entries:
        assert back.entries[k].shape == sd.entries[k].shape
        assert np.array_equal(bits(back.entries[k].data), bits(sd.entries[k].data)), k
    # the writer's text is ordinary JSON with the same values
    doc = json.loads(p.read_text())
    assert list(doc) == ["entries"]
    assert np.array_equal(bits(np.array(doc["entries"]["a.first"]["data"], np.float64).astype(np.float32)),
                          bits(rand))


def test_checkpoint_round_trip_and_non_finite_values(tmp_path):
    sd = ck.StateDict({"w": ck.TensorData([2], f32(1.5, -2.0))})
    c = ck.Checkpoint(42, sd, {"note": "unit test", "cfg": [1, 2.5, None, True]})
    p = tmp_path / "ck.json"
    c.save(p)
    text = p.read_text()
    assert text.startswith('{"step":42,"state":{"entries":{"w":{"shape":[2],"data":[')
    back = ck.Checkpoint.load(p)
    assert back.step == 42 and back.metadata == c.metadata
    assert np.array_equal(back.state.entries["w"].data, f32(1.5, -2.0))
    # serde_json writes a non-finite f32 as null, and null then fails to load
    bad = ck.StateDict({"w": ck.TensorData([2], f32(1.0, np.inf))})
    bad.save(p)
    assert '"data":[1,null]' in p.read_text().replace("1.0", "1")
    with pytest.raises(JsonError, match="invalid type: null, expected f32"):
        ck.StateDict.load(p)


def test_files_written_by_pythons_json_module(tmp_path):
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(3000)                      # f64 values, not f32-exact
    doc = {"step": 3, "metadata": None, "junk": {"a": [1, {"b": "]"}]},
           "state": {"entries": {"p.q": {"data": vals.tolist(), "shape": [3000]}}}}
    for indent in (None, 2):
        p = tmp_path / f"py{indent}.json"
        p.write_text(json.dumps(doc, indent=indent))
        c = ck.Checkpoint.load(p)
        assert c.step == 3 and c.metadata is None
        assert np.array_equal(bits(c.state.entries["p.q"].data), bits(vals.astype(np.float32)))


def test_arrays_larger_than_one_parse_piece(tmp_path):
    """Several megabytes of numbers are split across threads at commas; the
    joined result is the sequential one."""
    rng = np.random.default_rng(2)
    vals = rng.standard_normal(1_200_003).astype(np.float32)
    text = ",".join(repr(float(v)) for v in vals)
    assert len(text) > 3 * (4 << 20)
    p = tmp_path / "big.json"
    p.write_text('{"entries":{"big":{"shape":[1200003],"data":[' + text + ']},'
                 '"small":{"shape":[1],"data":[2]}}}')
    sd = ck.StateDict.load(p)
    assert np.array_equal(bits(sd.entries["big"].data), bits(vals))
    assert sd.entries["small"].data.tolist() == [2.0]


@pytest.mark.parametrize("text,msg", [
    ('{"entries":{"x":{"shape":[2],"data":[1,2,]}}}', "trailing comma"),
    ('{"entries":{"x":{"shape":[2],"data":[1,,2]}}}', "expected value"),
    ('{"entries":{"x":{"data":[1]}}}', "missing field `shape`"),
    ('{"entries":{"x":{"shape":[1]}}}', "missing field `data`"),
    ('{"entries":{"x":{"shape":[1.5],"data":[1]}}}', "floating point"),
    ('{"entries":{"x":{"shape":[1],"data":[1]}}', "EOF"),
    ('{"entries":{}} x', "trailing characters"),
    ('{"other":{}}', "missing field `entries`"),
    ('', "EOF while parsing a value"),
])
def test_malformed_state_dicts(tmp_path, text, msg):
    p = tmp_path / "bad.json"
    p.write_text(text)
    with pytest.raises(JsonError, match=msg):
        ck.StateDict.load(p)


def test_checkpoint_needs_step_and_state(tmp_path):
    p = tmp_path / "c.json"
    p.write_text('{"state":{"entries":{}},"metadata":null}')
    with pytest.raises(JsonError, match="missing field `step`"):
        ck.Checkpoint.load(p)
    p.write_text('{"step":1,"metadata":null}')
    with pytest.raises(JsonError, match="missing field `state`"):
        ck.Checkpoint.load(p)
    with pytest.raises(IoError, match="No such file"):
        ck.Checkpoint.load(tmp_path / "missing.json")


def test_filter_and_repeated_keys(tmp_path):
    p = tmp_path / "r.json"
    p.write_text('{"entries":{"a.in_proj.weight":{"shape":[1],"data":[1]},'
                 '"b":{"shape":[1],"data":[2]},"a.in_proj.weight":{"shape":[1],"data":[3]}}}')
    sd = ck.StateDict.load(p)
    assert sd.entries["a.in_proj.weight"].data.tolist() == [3.0]   # the last value wins
    f = sd.filter("in_proj")
    assert list(f.entries) == ["a.in_proj.weight"] and len(sd) == 2


# ------------------------------------------------------------------ models on the CPU
def _cpu_lm(seed=0, layers=2, conv=None):
    from mamba3 import Discretization, SsmConfig, SsmMode, StateDynamics
    from mamba3.lm import Mamba3Lm, Mamba3LmConfig
    ssm = SsmConfig(d_model=16, n_heads=2, head_dim=8, d_state=8, n_groups=1,
                    discretization=Discretization.LearnedTrapezoid,
                    dynamics=StateDynamics.Rotational, mode=SsmMode(1), chunk_size=64,
                    conv_kernel=conv, bc_norm=True, post_gate_norm=True)
    return Mamba3Lm(Mamba3LmConfig(vocab_size=11, d_model=16, n_layers=layers, ssm=ssm, seed=seed),
                    "cpu")


def test_parameter_paths_are_the_references():
    """lm.rs:355-362, hybrid.rs:497-516, mamba3.rs:634-656, norm.rs:109-113,
    linear.rs:266-270, embedding.rs:106-108."""
    lm = _cpu_lm()
    names = [n for n, _ in lm.named_parameters()]
    per_layer = ["norm.weight", "mixer.in_proj.weight", "mixer.out_proj.weight", "mixer.dt_bias",
                 "mixer.a_log", "mixer.d", "mixer.b_bias", "mixer.c_bias", "mixer.bc_norm.weight",
                 "mixer.post_gate_norm.weight"]
    want = (["embed.weight"] + [f"stack.layers.{i}.{n}" for i in range(2) for n in per_layer]
            + ["norm_f.weight", "head.weight"])
    assert names == want
    shapes = dict((n, p.shape) for n, p in lm.named_parameters())
    width = 2 * 16 + 2 * 1 * 8 + 2 + 2 + 2 * 4
    assert shapes["stack.layers.1.mixer.in_proj.weight"] == (16, width)
    assert shapes["stack.layers.0.mixer.out_proj.weight"] == (16, 16)
    assert shapes["stack.layers.0.mixer.b_bias"] == (2, 8)
    assert shapes["embed.weight"] == (11, 16) and shapes["head.weight"] == (16, 11)


def test_convolution_parameters_follow_out_proj():
    """mamba3.rs:634-640 and nn/conv.rs: with conv_kernel k the mixer visits
    conv.weight [k, d_inner + 2 bc_width] and conv.bias right after out_proj;
    the weight starts in U(-sqrt(3/k), sqrt(3/k)) (KaimingUniform, fan_in k,
    nn/init.rs:82-93), the bias at zero."""
    lm = _cpu_lm(conv=4)
    names = [n for n, _ in lm.named_parameters()]
    i = names.index("stack.layers.0.mixer.out_proj.weight")
    assert names[i + 1:i + 4] == ["stack.layers.0.mixer.conv.weight",
                                  "stack.layers.0.mixer.conv.bias", "stack.layers.0.mixer.dt_bias"]
    params = dict(lm.named_parameters())
    ch = 16 + 2 * 8
    assert params["stack.layers.1.mixer.conv.weight"].shape == (4, ch)
    assert params["stack.layers.1.mixer.conv.bias"].shape == (ch,)
    w = params["stack.layers.1.mixer.conv.weight"].get().numpy()
    assert np.abs(w).max() <= math.sqrt(3.0 / 4) and np.abs(w).max() > 0.5 * math.sqrt(3.0 / 4)
    assert not params["stack.layers.1.mixer.conv.bias"].get().numpy().any()
    cache = lm.empty_cache(3, "cpu")
    assert tuple(cache[0].conv.shape) == (3, 3, ch) and not cache[0].conv.float().any()


def test_state_dict_rules(tmp_path):
    src, dst = _cpu_lm(1), _cpu_lm(2)
    sd = src.state_dict()
    p = tmp_path / "lm.json"
    ck.Checkpoint(5, sd, {"d_model": 16}).save(p)
    back = ck.Checkpoint.load(p)
    back.restore(dst, strict=True)
    for (n, a), (_, b) in zip(src.named_parameters(), dst.named_parameters()):
        assert np.array_equal(bits(a.get().float().numpy()), bits(b.get().float().numpy())), n
    # strict: every parameter needs an entry, every entry a parameter
    part = back.state.filter("mixer")
    with pytest.raises(StateDictError, match="missing entry for `embed.weight`"):
        dst.load_state_dict(part, strict=True)
    dst.load_state_dict(part, strict=False)
    extra = ck.StateDict(dict(back.state.entries, **{"stack.layers.9.norm.weight":
                                                     ck.TensorData([16], np.ones(16))}))
    with pytest.raises(StateDictError, match="unexpected entry `stack.layers.9.norm.weight`"):
        dst.load_state_dict(extra, strict=True)
    wrong = ck.StateDict({"norm_f.weight": ck.TensorData([8], np.ones(8))})
    with pytest.raises(StateDictError,
                       match=r"`norm_f.weight`: checkpoint holds \[8\] but the model expects \[16\]"):
        dst.load_state_dict(wrong, strict=False)
    short = ck.StateDict({"norm_f.weight": ck.TensorData([16], np.ones(15))})
    with pytest.raises(ShapeError, match="data of length 15 does not fill shape"):
        dst.load_state_dict(short, strict=False)
    assert math.isclose(float(back.num_values()), float(src.num_parameters()))
