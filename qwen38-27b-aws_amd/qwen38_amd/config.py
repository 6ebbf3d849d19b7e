"""Model shapes for the verify path, mirroring the reference's `TextConfig` (qwen38_inf2/config.py:11-130).

Differences from the reference, all because this build runs one GPU holding the whole model:
* no `validate_tp` and no `tp_degree`: nothing is split across devices;
* `weight_format` and `kv_cache_format` here are the reference's field values and only describe the reference's
  numerics ("fp8": e5m2 activations into FP8 projections); the engine's own storage formats are chosen when it is built
  (`steps.Engine(weight_format="e4m3" | "mxfp4", kv_cache_format="bf16" | "fp8")`);
* `recurrent_state_format` is always "bf16".

`verify_configs()` gives BASELINE's five workloads: the parity tests run configs 0, 1, 3 and 4 one block deep
(tests/test_gpu_layers.py) and `bench.py` measures config 2.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, replace
from pathlib import Path

LINEAR = "linear_attention"
FULL = "full_attention"


@dataclass(frozen=True)
class TextConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    layer_types: tuple[str, ...]
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    linear_num_key_heads: int
    linear_num_value_heads: int
    linear_key_head_dim: int
    linear_value_head_dim: int
    linear_conv_kernel_dim: int
    rms_norm_eps: float
    rope_theta: float
    partial_rotary_factor: float
    weight_format: str = "fp8"
    recurrent_state_format: str = "bf16"
    kv_cache_format: str = "bf16"

    @property
    def num_hidden_layers(self) -> int:
        return len(self.layer_types)

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def linear_key_dim(self) -> int:
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def linear_value_dim(self) -> int:
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def linear_conv_dim(self) -> int:
        return 2 * self.linear_key_dim + self.linear_value_dim

    @property
    def num_key_value_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def linear_key_repeat(self) -> int:
        return self.linear_num_value_heads // self.linear_num_key_heads

    @classmethod
    def from_model_config(cls, config: dict) -> "TextConfig":
        """Same fields as the reference reads from a Hugging Face config (config.py:85-105)."""
        text = config.get("text_config", config)
        rope = text["rope_parameters"]
        return cls(
            vocab_size=text["vocab_size"],
            hidden_size=text["hidden_size"],
            intermediate_size=text["intermediate_size"],
            layer_types=tuple(text["layer_types"]),
            num_attention_heads=text["num_attention_heads"],
            num_key_value_heads=text["num_key_value_heads"],
            head_dim=text["head_dim"],
            linear_num_key_heads=text["linear_num_key_heads"],
            linear_num_value_heads=text["linear_num_value_heads"],
            linear_key_head_dim=text["linear_key_head_dim"],
            linear_value_head_dim=text["linear_value_head_dim"],
            linear_conv_kernel_dim=text["linear_conv_kernel_dim"],
            rms_norm_eps=text["rms_norm_eps"],
            rope_theta=rope["rope_theta"],
            partial_rotary_factor=rope["partial_rotary_factor"],
        )

    @classmethod
    def from_file(cls, path: str | Path) -> "TextConfig":
        return cls.from_model_config(json.loads(Path(path).read_text()))

    def check(self) -> None:
        """Shape rules the HIP kernels rely on; a config breaking one is refused here, on the host."""
        problems = []
        if self.linear_key_head_dim != 128 or self.linear_value_head_dim != 128:
            problems.append("gated-delta head dims must be 128")
        if self.head_dim != 256:
            problems.append("attention head_dim must be 256")
        if self.rotary_dim != 64:
            problems.append("rotary_dim must be 64")
        if self.linear_conv_kernel_dim != 4:
            problems.append("conv width must be 4")
        if self.linear_num_value_heads % self.linear_num_key_heads:
            problems.append("value heads must be a multiple of key heads")
        if self.num_attention_heads % self.num_key_value_heads:
            problems.append("query heads must be a multiple of KV heads")
        for name, width in (
            ("hidden_size", self.hidden_size),
            ("intermediate_size", self.intermediate_size),
            ("linear_value_dim", self.linear_value_dim),
            ("attention width", self.num_attention_heads * self.head_dim),
        ):
            if width % 512:
                problems.append(f"{name}={width} must be a multiple of 512 (FP8 GEMM K-steps of 4x128)")
        for name, width in (
            ("intermediate_size", self.intermediate_size),
            ("vocab_size", self.vocab_size),
            ("linear_conv_dim", self.linear_conv_dim),
        ):
            if width % 64:
                problems.append(f"{name}={width} must be a multiple of 64 (GEMM column tiles)")
        if problems:
            raise ValueError("; ".join(problems))


def tiny_config(num_blocks: int = 1) -> TextConfig:
    """the tiny hybrid block, small enough for the CPU oracle to run in seconds."""
    return TextConfig(
        vocab_size=32768,
        hidden_size=1024,
        intermediate_size=3072,
        layer_types=(LINEAR, LINEAR, LINEAR, FULL) * num_blocks,
        num_attention_heads=8,
        num_key_value_heads=2,
        head_dim=256,
        linear_num_key_heads=4,
        linear_num_value_heads=8,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        rms_norm_eps=1e-6,
        rope_theta=10000000.0,
        partial_rotary_factor=0.25,
    )


def qwen38_27b_config(num_blocks: int = 16) -> TextConfig:
    """The 27B shapes (reference tests/fixtures/config.json text_config); `num_blocks` repeats of 3 GDN + 1 attention."""
    return TextConfig(
        vocab_size=248320,
        hidden_size=5120,
        intermediate_size=17408,
        layer_types=(LINEAR, LINEAR, LINEAR, FULL) * num_blocks,
        num_attention_heads=24,
        num_key_value_heads=4,
        head_dim=256,
        linear_num_key_heads=16,
        linear_num_value_heads=48,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        rms_norm_eps=1e-6,
        rope_theta=10000000.0,
        partial_rotary_factor=0.25,
    )


@dataclass(frozen=True)
class Workload:
    """One BASELINE workload: model shapes plus rows, tokens per row and context per row."""

    name: str
    cfg: TextConfig
    batch: int
    tokens: int
    context: int
    max_seq_len: int
    mtp: bool
    head: bool


def verify_configs() -> list[Workload]:
    """BASELINE.json configs 0-4, in order."""
    big = qwen38_27b_config
    return [
        Workload("tiny-block-b4", tiny_config(1), 4, 4, 512, 1024, True, True),
        Workload("27b-block-b64-k4-ctx512", big(1), 64, 4, 512, 1024, False, False),
        Workload("27b-64L-b64-k4-ctx512-mtp-head", big(16), 64, 4, 512, 1024, True, True),
        Workload("27b-block-b16-k4-ctx32k", big(1), 16, 4, 32768, 32768 + 64, False, False),
        Workload("27b-block-b256-k8-ctx4k", big(1), 256, 8, 4096, 4096 + 64, False, False),
    ]


def with_layers(cfg: TextConfig, layer_types) -> TextConfig:
    return replace(cfg, layer_types=tuple(layer_types))
