"""The safetensors reader (crates/graph/src/checkpoint.rs) and config.json's schema
(crates/voxcpm/src/config.rs) on the CPU. The reader is libtgx's (tgx_checkpoint_*), which needs no
device; the checks follow the reference's own tests (checkpoint.rs:196-224,
crates/voxcpm/tests/config.rs) on its fixtures (tests/golden/voxcpm_config.json is its
fixtures/voxcpm.json; voxcpm_checkpoint.safetensors its fixture of the same name), with the
safetensors package as an independent reader of the same files."""

import json
import struct
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _write(path, header: dict, data: bytes, length=None):
    text = json.dumps(header).encode()
    n = len(text) if length is None else length
    path.write_bytes(struct.pack("<Q", n) + text + data)


def test_a_gather_reads_the_rows_the_whole_tensor_holds(tmp_path):
    """checkpoint.rs:196-224: quarters, which bfloat16 holds exactly."""
    from tgx import TgxError
    from tgx.checkpoint import Checkpoint

    rows = np.arange(12, dtype=np.float32) / 4.0 - 1.5
    bits = (rows.view(np.uint32) >> 16).astype("<u2").tobytes()
    p = tmp_path / "gather.safetensors"
    _write(p, {"table": {"dtype": "BF16", "shape": [3, 4], "data_offsets": [0, len(bits)]}}, bits)
    with Checkpoint(p) as ck:
        whole = ck.f32("table")
        assert np.array_equal(whole.ravel(), rows)
        got = ck.gather("table", [2, 0, 2])
        assert np.array_equal(got, np.stack([whole[2], whole[0], whole[2]]))
        with pytest.raises(TgxError) as e:
            ck.gather("table", [3])
        assert e.value.kind == "weights" and "row 3 of 3" in str(e.value)


def test_the_reference_fixture_reads_as_the_safetensors_package_reads_it():
    from safetensors.numpy import load_file

    from tgx.checkpoint import Checkpoint

    path = GOLDEN / "voxcpm_checkpoint.safetensors"
    want = load_file(str(path))
    with Checkpoint(path) as ck:
        assert ck.names() == sorted(want)  # __metadata__ is not a tensor
        for name, values in want.items():
            assert ck.shape(name) == values.shape
            assert ck.dtype(name) == "F32"
            assert np.array_equal(ck.f32(name), values)
        assert ck.shape("no.such.tensor") is None


def test_f16_and_f32_tensors_convert_exactly(tmp_path):
    from tgx.checkpoint import Checkpoint

    h = np.array([0.5, -2.0, 65504.0, 6.1e-5, 5.96e-8], dtype=np.float16)
    f = np.array([1.0, -0.1, 3.0e38], dtype=np.float32)
    data = h.tobytes() + f.tobytes()
    _write(tmp_path / "m.safetensors", {
        "__metadata__": {"format": "pt"},
        "h": {"dtype": "F16", "shape": [5], "data_offsets": [0, 10]},
        "f": {"dtype": "F32", "shape": [3], "data_offsets": [10, 22]},
    }, data)
    with Checkpoint(tmp_path / "m.safetensors") as ck:
        assert np.array_equal(ck.f32("h"), h.astype(np.float32))
        assert np.array_equal(ck.f32("f"), f)
        assert ck.names() == ["f", "h"]


@pytest.mark.parametrize("case,why", [
    ("dtype", "I64 weights"),
    ("size", "8 bytes for 2 BF16"),
    ("past", "data_offsets past the end of the file"),
    ("json", "the header"),
    ("long", "a header of"),
])
def test_a_bad_file_is_refused_with_the_reason(tmp_path, case, why):
    """checkpoint.rs:44-99: the header's length, its JSON, each entry's dtype and byte count."""
    from tgx import TgxError
    from tgx.checkpoint import Checkpoint

    p = tmp_path / f"{case}.safetensors"
    if case == "dtype":
        _write(p, {"t": {"dtype": "I64", "shape": [1], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "size":
        _write(p, {"t": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "past":
        _write(p, {"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, bytes(8))
    elif case == "json":
        p.write_bytes(struct.pack("<Q", 5) + b'{"t":')
    else:
        p.write_bytes(struct.pack("<Q", (100 << 20) + 1) + b"{}")
    with pytest.raises(TgxError) as e:
        Checkpoint(p)
    assert e.value.kind == "weights"
    assert why in str(e.value), str(e.value)


def _tiny():
    return json.loads((GOLDEN / "voxcpm_config.json").read_text())


def _parse(data):
    from tgx.config import Config

    return Config.from_json(json.dumps(data))


def test_stacks_are_derived_from_the_base_lm_as_upstream_derives_them():
    """crates/voxcpm/tests/config.rs:13-39."""
    config = _parse(_tiny())
    lm = config.lm_config
    residual = config.residual_lm()
    assert residual.num_hidden_layers == 1 and residual.no_rope and residual.vocab_size == 0
    assert residual.hidden_size == lm.hidden_size
    for stack, ffn in ((config.local_encoder(), 24), (config.local_dit(), 20)):
        assert stack.hidden_size == 16 and stack.intermediate_size == ffn
        assert stack.num_attention_heads == 4 and stack.num_hidden_layers == 2
        assert stack.kv_channels == 8 and stack.vocab_size == 0 and not stack.no_rope
        assert stack.rope_scaling == lm.rope_scaling
    vae = config.audio_vae()
    assert (vae.latent_dim, vae.decoder_dim) == (8, 16)


def test_missing_fields_take_upstreams_defaults():
    """crates/voxcpm/tests/config.rs:41-77."""
    from tgx.config import AudioVaeConfig, CfmConfig

    config = _parse({"lm_config": _tiny()["lm_config"], "encoder_config": {}, "dit_config": {"cfm_config": {}}})
    assert config.architecture is None
    assert (config.patch_size, config.feat_dim) == (4, 64)
    assert config.residual_lm_num_layers == 8 and not config.residual_lm_no_rope
    assert config.scalar_quantization_latent_dim == 512 and config.scalar_quantization_scale == 9
    assert config.max_length == 8192 and (config.device, config.dtype) == ("cuda", "bfloat16")
    assert config.audio_vae() == AudioVaeConfig()
    for stack in (config.encoder_config, config.dit_config):
        assert (stack.hidden_dim, stack.ffn_dim, stack.num_heads, stack.num_layers, stack.kv_channels) == (
            1024, 4096, 16, 4, None)
    assert not config.dit_config.dit_mean_mode and not config.dit_config.mean_mode
    cfm = config.dit_config.cfm_config
    assert cfm == CfmConfig() and (cfm.sigma_min, cfm.solver, cfm.inference_cfg_rate) == (1e-6, "euler", 1.0)


def test_null_audio_vae_config_is_upstreams_default():
    """crates/voxcpm/tests/config.rs:79-85."""
    from tgx.config import AudioVaeConfig

    data = _tiny()
    data["audio_vae_config"] = None
    data["feat_dim"] = 64
    assert _parse(data).audio_vae() == AudioVaeConfig()


@pytest.mark.parametrize("path,name", [
    ((), "dit_mean_mode"),
    (("encoder_config",), "num_kv_heads"),
    (("dit_config",), "concat_hidden"),
    (("dit_config", "cfm_config"), "sway_sampling_coef"),
])
def test_unknown_fields_are_refused(path, name):
    """crates/voxcpm/tests/config.rs:87-103."""
    from tgx.config import ConfigError

    data = _tiny()
    node = data
    for key in path:
        node = node[key]
    node[name] = True
    with pytest.raises(ConfigError) as e:
        _parse(data)
    assert f"unknown field `{name}`" in str(e.value)


@pytest.mark.parametrize("path,value,message", [
    (("architecture",), "voxcpm", 'architecture "voxcpm"'),
    (("dit_config", "dit_mean_mode"), True, "dit_config.dit_mean_mode: true"),
    (("dit_config", "mean_mode"), True, "dit_config.mean_mode: true"),
    (("dit_config", "cfm_config", "solver"), "heun", 'solver "heun"'),
    (("feat_dim",), 64, "feat_dim 64 where the audio VAE's latents have 8 channels"),
])
def test_unimplemented_values_are_refused(path, value, message):
    """crates/voxcpm/tests/config.rs:105-137, message for message."""
    from tgx.config import Unsupported

    data = _tiny()
    node = data
    for key in path[:-1]:
        node = node[key]
    node[path[-1]] = value
    with pytest.raises(Unsupported) as e:
        _parse(data)
    assert str(e.value) == message


def test_the_shape_of_a_stack_and_what_it_refuses():
    """decode::Shape::new (crates/graph/src/decode.rs:84-127): the fields it takes and its refusals."""
    import dataclasses

    from tgx.config import ShapeError, shape

    config = _parse(_tiny())
    s = shape(config.lm_config)
    assert (s.hidden, s.inner, s.heads, s.kv_heads, s.head_dim, s.layers, s.capacity) == (32, 48, 4, 2, 8, 2, 64)
    assert s.rope and s.eps == pytest.approx(1e-5) and s.rope_theta == 10000.0
    assert list(s.rope_factors) == [0.99, 1.6, 3.4, 8.9]  # the short factors, at the native length
    assert not shape(config.residual_lm()).rope
    lm = config.lm_config
    with pytest.raises(ShapeError, match="use_mup"):
        shape(dataclasses.replace(lm, use_mup=True))
    with pytest.raises(ShapeError, match="rope_scaling"):
        shape(dataclasses.replace(lm, rope_scaling=dataclasses.replace(lm.rope_scaling, kind="yarn")))
    with pytest.raises(ShapeError, match="3 of 2 layers"):
        shape(lm, layers=3)
    with pytest.raises(ShapeError, match="a cache of 65 past 64 positions"):
        shape(lm, capacity=65)
    # Without RoPE the scaling is not read (the residual LM's case).
    assert shape(dataclasses.replace(lm, no_rope=True, rope_scaling=dataclasses.replace(lm.rope_scaling, kind="x")))
