"""A VoxCPM2 checkpoint's config.json (crates/voxcpm/src/config.rs, crates/voxcpm/src/minicpm4.rs,
crates/voxcpm/src/audio_vae.rs) and the stack shapes the library is built at from it
(decode::Shape::new, crates/graph/src/decode.rs:84-127).

As the reference reads it: fields the JSON leaves out take upstream's defaults, a field the schema
does not have is refused (serde's deny_unknown_fields) as ConfigError, and values the build does
not implement are refused as Unsupported (another architecture, mean mode, a solver other than
Euler, latent frames other than the audio VAE's); Shape.new refusals are ShapeError."""

from __future__ import annotations

import json
from dataclasses import dataclass, field, fields, replace
from typing import Optional

from . import Shape


class ConfigError(ValueError):
    """voxcpm::Error::Config: not a config upstream would read."""


class Unsupported(ValueError):
    """voxcpm::Error::Unsupported: a config asking for what is not implemented."""


class ShapeError(ValueError):
    """graph::Error::Shape: a stack the kernels do not run."""


_REQUIRED = object()


def _read(cls, data, where: str):
    """A dataclass from a JSON object: unknown fields refused, missing ones defaulted or refused."""
    if not isinstance(data, dict):
        raise ConfigError(f"{where or 'config'}: expected an object")
    names = {f.name: f for f in fields(cls)}
    for key in data:
        if key not in names and key not in getattr(cls, "_ALIASES", {}):
            raise ConfigError(f"{where or 'config'}: unknown field `{key}`")
    kwargs = {}
    for f in fields(cls):
        key = getattr(cls, "_ALIASES_BACK", {}).get(f.name, f.name)
        if key in data:
            kwargs[f.name] = cls._convert(f.name, data[key], f"{where}/{key}")
        elif f.default is _REQUIRED:
            raise ConfigError(f"{where or 'config'}: missing field `{key}`")
    return cls(**kwargs)


def _int(v, where):
    if isinstance(v, bool) or not isinstance(v, int) or v < 0:
        raise ConfigError(f"{where}: expected a non-negative integer")
    return v


def _float(v, where):
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        raise ConfigError(f"{where}: expected a number")
    return float(v)


def _bool(v, where):
    if not isinstance(v, bool):
        raise ConfigError(f"{where}: expected a boolean")
    return v


def _str(v, where):
    if not isinstance(v, str):
        raise ConfigError(f"{where}: expected a string")
    return v


@dataclass
class RopeScaling:
    """minicpm4::RopeScaling (minicpm4.rs:57-69): LongRoPE's per-frequency factors."""

    kind: str = _REQUIRED
    long_factor: list = _REQUIRED
    short_factor: list = _REQUIRED
    original_max_position_embeddings: int = _REQUIRED
    _ALIASES = {"type": "kind"}
    _ALIASES_BACK = {"kind": "type"}

    @classmethod
    def _convert(cls, name, v, where):
        if name == "kind":
            return _str(v, where)
        if name in ("long_factor", "short_factor"):
            if not isinstance(v, list):
                raise ConfigError(f"{where}: expected a list")
            return [_float(x, where) for x in v]
        return _int(v, where)


@dataclass
class LmConfig:
    """minicpm4::Config (minicpm4.rs:12-49): a MiniCPM-4 stack's configuration."""

    bos_token_id: int = _REQUIRED
    eos_token_id: int = _REQUIRED
    hidden_size: int = _REQUIRED
    intermediate_size: int = _REQUIRED
    max_position_embeddings: int = _REQUIRED
    num_attention_heads: int = _REQUIRED
    num_hidden_layers: int = _REQUIRED
    num_key_value_heads: int = _REQUIRED
    rms_norm_eps: float = _REQUIRED
    rope_scaling: RopeScaling = _REQUIRED
    vocab_size: int = _REQUIRED
    use_mup: bool = True  # upstream assumes muP when the field is missing (minicpm4.rs:51-53)
    scale_emb: float = _REQUIRED
    dim_model_base: int = _REQUIRED
    scale_depth: float = _REQUIRED
    rope_theta: float = _REQUIRED
    kv_channels: Optional[int] = None
    no_rope: bool = False

    @classmethod
    def _convert(cls, name, v, where):
        if name == "rope_scaling":
            return _read(RopeScaling, v, where)
        if name in ("rms_norm_eps", "scale_emb", "scale_depth", "rope_theta"):
            return _float(v, where)
        if name in ("use_mup", "no_rope"):
            return _bool(v, where)
        if name == "kv_channels":
            return None if v is None else _int(v, where)
        return _int(v, where)

    def head_dim(self) -> int:
        """minicpm4.rs:84-88."""
        return self.kv_channels if self.kv_channels is not None else self.hidden_size // self.num_attention_heads

    def residual_lm(self, num_hidden_layers: int, no_rope: bool) -> "LmConfig":
        """minicpm4.rs:90-99."""
        return replace(self, num_hidden_layers=num_hidden_layers, vocab_size=0, no_rope=no_rope)

    def local(self, shape: "LocalShape") -> "LmConfig":
        """minicpm4.rs:101-111: head count and width are the shape's, whatever the hidden size."""
        return replace(self, hidden_size=shape.hidden_dim, intermediate_size=shape.ffn_dim,
                       num_attention_heads=shape.num_heads, num_hidden_layers=shape.num_layers,
                       kv_channels=shape.kv_channels, vocab_size=0)


@dataclass
class LocalShape:
    """`encoder_config` (config.rs:57-70): the shape of the local encoder's stack."""

    hidden_dim: int = 1024
    ffn_dim: int = 4096
    num_heads: int = 16
    num_layers: int = 4
    kv_channels: Optional[int] = None

    @classmethod
    def _convert(cls, name, v, where):
        if name == "kv_channels":
            return None if v is None else _int(v, where)
        return _int(v, where)


@dataclass
class CfmConfig:
    """`cfm_config` (config.rs:98-140): the flow matching the DiT was trained with."""

    sigma_min: float = 1e-6
    solver: str = "euler"
    t_scheduler: str = "log-norm"
    training_cfg_rate: float = 0.1
    inference_cfg_rate: float = 1.0
    reg_loss_type: str = "l1"
    ratio_r_neq_t_range: tuple = (0.25, 0.75)
    noise_cond_prob_range: tuple = (0.0, 0.0)
    noise_cond_scale: float = 0.0

    @classmethod
    def _convert(cls, name, v, where):
        if name in ("solver", "t_scheduler", "reg_loss_type"):
            return _str(v, where)
        if name in ("ratio_r_neq_t_range", "noise_cond_prob_range"):
            if not isinstance(v, list) or len(v) != 2:
                raise ConfigError(f"{where}: expected a pair")
            return (_float(v[0], where), _float(v[1], where))
        return _float(v, where)


@dataclass
class DitConfig:
    """`dit_config` (config.rs:72-95): the DiT's stack and how it is sampled."""

    hidden_dim: int = 1024
    ffn_dim: int = 4096
    num_heads: int = 16
    num_layers: int = 4
    kv_channels: Optional[int] = None
    dit_mean_mode: bool = False
    mean_mode: bool = False
    cfm_config: CfmConfig = _REQUIRED

    @classmethod
    def _convert(cls, name, v, where):
        if name == "cfm_config":
            return _read(CfmConfig, v, where)
        if name in ("dit_mean_mode", "mean_mode"):
            return _bool(v, where)
        if name == "kv_channels":
            return None if v is None else _int(v, where)
        return _int(v, where)

    def shape(self) -> LocalShape:
        return LocalShape(self.hidden_dim, self.ffn_dim, self.num_heads, self.num_layers, self.kv_channels)


@dataclass
class AudioVaeConfig:
    """audio_vae::AudioVaeConfig (audio_vae.rs:8-60); of it the path reads latent_dim alone."""

    encoder_dim: int = 128
    encoder_rates: list = field(default_factory=lambda: [2, 5, 8, 8])
    latent_dim: int = 64
    decoder_dim: int = 2048
    decoder_rates: list = field(default_factory=lambda: [8, 6, 5, 2, 2, 2])
    depthwise: bool = True
    sample_rate: int = 16000
    out_sample_rate: int = 48000
    use_noise_block: bool = False
    sr_bin_boundaries: Optional[list] = field(default_factory=lambda: [20000, 30000, 40000])
    cond_type: str = "scale_bias"
    cond_dim: int = 128
    cond_out_layer: bool = False

    @classmethod
    def _convert(cls, name, v, where):
        if name in ("encoder_rates", "decoder_rates"):
            if not isinstance(v, list):
                raise ConfigError(f"{where}: expected a list")
            return [_int(x, where) for x in v]
        if name == "sr_bin_boundaries":
            if v is None:
                return None
            if not isinstance(v, list):
                raise ConfigError(f"{where}: expected a list")
            return [_int(x, where) for x in v]
        if name in ("depthwise", "use_noise_block", "cond_out_layer"):
            return _bool(v, where)
        if name == "cond_type":
            return _str(v, where)
        return _int(v, where)


@dataclass
class Config:
    """voxcpm::Config (config.rs:14-55): upstream's VoxCPMConfig."""

    architecture: Optional[str] = None
    lm_config: LmConfig = _REQUIRED
    patch_size: int = 4
    feat_dim: int = 64
    residual_lm_num_layers: int = 8
    residual_lm_no_rope: bool = False
    scalar_quantization_latent_dim: int = 512
    scalar_quantization_scale: int = 9
    encoder_config: LocalShape = _REQUIRED
    dit_config: DitConfig = _REQUIRED
    audio_vae_config: Optional[AudioVaeConfig] = None
    max_length: int = 8192
    device: str = "cuda"
    dtype: str = "bfloat16"

    @classmethod
    def _convert(cls, name, v, where):
        if name == "architecture":
            return None if v is None else _str(v, where)
        if name == "lm_config":
            return _read(LmConfig, v, where)
        if name == "encoder_config":
            return _read(LocalShape, v, where)
        if name == "dit_config":
            return _read(DitConfig, v, where)
        if name == "audio_vae_config":
            return None if v is None else _read(AudioVaeConfig, v, where)
        if name == "residual_lm_no_rope":
            return _bool(v, where)
        if name in ("device", "dtype"):
            return _str(v, where)
        return _int(v, where)

    @classmethod
    def from_json(cls, text: str) -> "Config":
        """Config::from_json (config.rs:170-183): parsed, then checked."""
        try:
            data = json.loads(text)
        except json.JSONDecodeError as e:
            raise ConfigError(str(e)) from None
        config = _read(cls, data, "")
        config.check()
        return config

    def check(self) -> None:
        """Config::check (config.rs:185-214)."""
        if self.architecture is not None and self.architecture != "voxcpm2":
            raise Unsupported(f"architecture {json.dumps(self.architecture)}")
        dit = self.dit_config
        if dit.dit_mean_mode:
            raise Unsupported("dit_config.dit_mean_mode: true")
        if dit.mean_mode:
            raise Unsupported("dit_config.mean_mode: true")
        if dit.cfm_config.solver != "euler":
            raise Unsupported(f"solver {json.dumps(dit.cfm_config.solver)}")
        latent_dim = self.audio_vae().latent_dim
        if latent_dim != self.feat_dim:
            raise Unsupported(f"feat_dim {self.feat_dim} where the audio VAE's latents have {latent_dim} channels")

    def residual_lm(self) -> LmConfig:
        return self.lm_config.residual_lm(self.residual_lm_num_layers, self.residual_lm_no_rope)

    def local_encoder(self) -> LmConfig:
        return self.lm_config.local(self.encoder_config)

    def local_dit(self) -> LmConfig:
        return self.lm_config.local(self.dit_config.shape())

    def audio_vae(self) -> AudioVaeConfig:
        return self.audio_vae_config if self.audio_vae_config is not None else AudioVaeConfig()


def shape(config: LmConfig, layers: Optional[int] = None, capacity: Optional[int] = None) -> Shape:
    """decode::Shape::new (decode.rs:84-127): the stack `config` describes with its first `layers`
    layers and a cache of `capacity` positions; refuses muP, RoPE other than LongRoPE at its
    native length, more layers than the stack has and a cache past its positions."""
    layers = config.num_hidden_layers if layers is None else layers
    capacity = config.max_position_embeddings if capacity is None else capacity
    if config.use_mup:
        raise ShapeError("use_mup")
    rope = config.rope_scaling
    if not config.no_rope and (rope.kind != "longrope"
                               or config.max_position_embeddings != rope.original_max_position_embeddings):
        raise ShapeError(f"rope_scaling {json.dumps(rope.kind)} from {rope.original_max_position_embeddings} "
                         f"positions to {config.max_position_embeddings}")
    if layers > config.num_hidden_layers:
        raise ShapeError(f"{layers} of {config.num_hidden_layers} layers")
    if capacity > config.max_position_embeddings:
        raise ShapeError(f"a cache of {capacity} past {config.max_position_embeddings} positions")
    return Shape(hidden=config.hidden_size, inner=config.intermediate_size, heads=config.num_attention_heads,
                 kv_heads=config.num_key_value_heads, head_dim=config.head_dim(), layers=layers, capacity=capacity,
                 eps=float(config.rms_norm_eps), rope_theta=float(config.rope_theta), rope=not config.no_rope,
                 rope_factors=list(rope.short_factor))
