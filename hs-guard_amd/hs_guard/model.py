"""Backbone geometry and weights of the HS-Guard classifier (hybrid gated-delta / windowed attention).

``GuardConfig`` holds the geometry the streaming step needs (the fields of transformers'
Qwen3_5TextConfig the reference reads, plus the classifier heads of src/hs_guard/runtime.py:54-67).
``GuardModel`` holds bf16 weights under the reference checkpoint's parameter names
(``backbone.layers.{i}.linear_attn.in_proj_qkv.weight``, ``heads.{role}.projection.0.weight`` ...), so a
real bundle maps one-to-one. ``GuardModel.random(config, seed)`` draws the synthetic random-init weights
of the benchmark configurations.
"""
from __future__ import annotations

import dataclasses
from typing import Dict, List

import torch

ROLES = ("user", "assistant")


@dataclasses.dataclass
class GuardConfig:
    vocab_size: int = 151936
    hidden_size: int = 1024
    num_hidden_layers: int = 24
    full_attention_interval: int = 4
    layer_types: List[str] = None
    intermediate_size: int = 3584
    rms_norm_eps: float = 1e-6
    # gated delta net
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 16
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    # windowed attention
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int = 256
    partial_rotary_factor: float = 0.25
    rope_theta: float = 10000.0
    window_tokens: int = 512
    # classifier heads
    head_hidden: int = 512
    layer_norm_eps: float = 1e-5

    def __post_init__(self):
        if self.layer_types is None:
            # Qwen3.5 default pattern: every `full_attention_interval`-th layer is attention
            self.layer_types = ["linear_attention" if (i + 1) % self.full_attention_interval else "full_attention"
                                for i in range(self.num_hidden_layers)]

    @classmethod
    def from_hf(cls, d: dict, window_tokens: int = 512):
        """Geometry from a bundle's config.json (transformers' Qwen3_5TextConfig.to_dict(); rope settings under
        ``rope_parameters`` or, in older files, at top level) and the manifest's window."""
        rope = d.get("rope_parameters") or {}
        kw = {f.name: d[f.name] for f in dataclasses.fields(cls)
              if f.name in d and f.name not in ("window_tokens", "head_hidden", "layer_norm_eps")}
        kw["rope_theta"] = float(rope.get("rope_theta", d.get("rope_theta", 10000.0)))
        kw["partial_rotary_factor"] = float(rope.get("partial_rotary_factor", d.get("partial_rotary_factor", 0.25)))
        kw["window_tokens"] = int(window_tokens)
        return cls(**kw)

    @classmethod
    def baseline(cls, **kw):
        """The geometry BASELINE.json's configs state: vocab 151,936, 16q/4kv attention."""
        return cls(**kw)

    @classmethod
    def v10(cls, **kw):
        """The released v10 geometry: vocab 248,320, 8q/2kv attention (754,519,918 parameters)."""
        kw.setdefault("vocab_size", 248320)
        kw.setdefault("num_attention_heads", 8)
        kw.setdefault("num_key_value_heads", 2)
        return cls(**kw)

    @property
    def key_dim(self):
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def value_dim(self):
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def conv_dim(self):
        return 2 * self.key_dim + self.value_dim

    @property
    def rotary_dim(self):
        return int(self.head_dim * self.partial_rotary_factor)

    def parameter_shapes(self) -> Dict[str, tuple]:
        h, c = self.hidden_size, self
        shapes = {"backbone.embed_tokens.weight": (c.vocab_size, h), "backbone.norm.weight": (h,)}
        for i, kind in enumerate(self.layer_types):
            p = f"backbone.layers.{i}."
            shapes[p + "input_layernorm.weight"] = (h,)
            shapes[p + "post_attention_layernorm.weight"] = (h,)
            shapes[p + "mlp.gate_proj.weight"] = (c.intermediate_size, h)
            shapes[p + "mlp.up_proj.weight"] = (c.intermediate_size, h)
            shapes[p + "mlp.down_proj.weight"] = (h, c.intermediate_size)
            if kind == "linear_attention":
                a = p + "linear_attn."
                shapes[a + "in_proj_qkv.weight"] = (c.conv_dim, h)
                shapes[a + "in_proj_z.weight"] = (c.value_dim, h)
                shapes[a + "in_proj_b.weight"] = (c.linear_num_value_heads, h)
                shapes[a + "in_proj_a.weight"] = (c.linear_num_value_heads, h)
                shapes[a + "conv1d.weight"] = (c.conv_dim, 1, c.linear_conv_kernel_dim)
                shapes[a + "A_log"] = (c.linear_num_value_heads,)
                shapes[a + "dt_bias"] = (c.linear_num_value_heads,)
                shapes[a + "norm.weight"] = (c.linear_value_head_dim,)
                shapes[a + "out_proj.weight"] = (h, c.value_dim)
            else:
                a = p + "self_attn."
                shapes[a + "q_proj.weight"] = (c.num_attention_heads * c.head_dim * 2, h)
                shapes[a + "k_proj.weight"] = (c.num_key_value_heads * c.head_dim, h)
                shapes[a + "v_proj.weight"] = (c.num_key_value_heads * c.head_dim, h)
                shapes[a + "o_proj.weight"] = (h, c.num_attention_heads * c.head_dim)
                shapes[a + "q_norm.weight"] = (c.head_dim,)
                shapes[a + "k_norm.weight"] = (c.head_dim,)
        for role in ROLES:
            p = f"heads.{role}."
            shapes[p + "projection.0.weight"] = (c.head_hidden, h)
            shapes[p + "projection.0.bias"] = (c.head_hidden,)
            shapes[p + "projection.1.weight"] = (c.head_hidden,)
            shapes[p + "projection.1.bias"] = (c.head_hidden,)
            shapes[p + "risk.weight"] = (3, c.head_hidden)
            shapes[p + "risk.bias"] = (3,)
        return shapes


# Gains applied directly as multipliers (no 1 + w offset): drawn as 1 + N(0, std) so the random network
# passes signal. Every other tensor (including the RMSNorm (1 + w) deltas, A_log, dt_bias) is N(0, std).
_UNIT_GAINS = ("linear_attn.norm.weight", "projection.1.weight")


def head_dtype(name):
    """Storage dtype of a parameter. The classifier heads stay float32, as the reference keeps them: its
    backbone parameters are cast to bf16 and its heads are float32 modules the checkpoint is loaded into
    (src/hs_guard/runtime.py:108-113); the streaming readout casts the Linear weights to bf16 but applies the
    float32 LayerNorm (slot_engine_v7.py:44-61), and the complete-message readout runs entirely in float32
    (runtime.py:70-73,141). Everything else is bf16."""
    return torch.float32 if name.startswith("heads.") else torch.bfloat16


class _Backbone:
    def __init__(self, config):
        self.config = config


class GuardModel:
    """bf16 weights by reference parameter name, on one device."""

    def __init__(self, config: GuardConfig, weights: Dict[str, torch.Tensor]):
        self.config = config
        self.weights = weights
        self.backbone = _Backbone(config)   # `model.backbone.config.vocab_size`, as the reference reads it

    @property
    def device(self):
        return self.weights["backbone.norm.weight"].device

    def __getitem__(self, name):
        return self.weights[name]

    @classmethod
    def random(cls, config: GuardConfig = None, seed: int = 0, device="cuda", std=0.02, gen_device="cpu"):
        """Seeded random init, drawn in sorted-name order on ``gen_device`` (the CPU by default, so every
        device gets identical bytes) then moved to ``device``. Every value is rounded to bf16 (the heads are
        stored as float32 holding those values)."""
        config = config or GuardConfig.baseline()
        gen = torch.Generator(device=gen_device).manual_seed(seed)
        weights = {}
        for name, shape in sorted(config.parameter_shapes().items()):
            t = torch.randn(*shape, generator=gen, device=gen_device) * std
            if name.endswith(_UNIT_GAINS):
                t = t + 1.0
            weights[name] = t.to(torch.bfloat16).to(head_dtype(name)).to(device)
        return cls(config, weights)

    @classmethod
    def from_state_dict(cls, config: GuardConfig, state: Dict[str, torch.Tensor], head="redline", device="cuda"):
        """Weights of a classifier checkpoint (the state dict of src/hs_guard/runtime.py:54-74, loaded there with
        strict=True): every backbone and head tensor this build uses must be present with its shape, and any
        other key must be one of the checkpoint's classifier tensors this build does not use (category and
        general heads). head="general" reads the general projection and risk layers in place of the red-line
        ones (runtime.py:119-121). Backbone tensors are stored as bf16 and head tensors as float32 (head_dtype)
        on ``device``."""
        shapes = config.parameter_shapes()
        known_extra = ("category.", "general_projection.", "general.", "general_category.")
        unexpected = [k for k in state if k not in shapes and
                      not (k.startswith("heads.") and k.split(".", 2)[2].startswith(known_extra))]
        if unexpected:
            raise ValueError(f"Unexpected keys in checkpoint: {sorted(unexpected)[:5]}")
        weights = {}
        for name, shape in shapes.items():
            src = name
            if head == "general" and name.startswith("heads."):
                src = name.replace(".projection.", ".general_projection.").replace(".risk.", ".general.")
            if src not in state:
                raise ValueError(f"Missing key in checkpoint: {src}")
            t = state[src]
            if tuple(t.shape) != tuple(shape):
                raise ValueError(f"Shape mismatch for {src}: {tuple(t.shape)} != {tuple(shape)}")
            weights[name] = t.to(head_dtype(name)).to(device).contiguous()
        return cls(config, weights)

    def to(self, device):
        return GuardModel(self.config, {k: v.to(device) for k, v in self.weights.items()})

    def num_parameters(self):
        return sum(v.numel() for v in self.weights.values())
