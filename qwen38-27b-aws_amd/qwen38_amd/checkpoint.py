"""Reading a Qwen3.8 MXFP4 checkpoint (Hugging Face safetensors files) into the (name, value) pairs `steps.Engine.load`
takes, for one GPU holding the whole model: the reference's weight cutting (qwen38_inf2/checkpoint.py:177-224 decoder
layers, 227-233 KV scales, 324-342 head, 363-392 MTP layer) without its per-rank slices.

* Decoder-layer projections are the checkpoint's own MXFP4 bytes (``weight_packed`` uint8 ``[N, K/2]``,
  ``weight_scale`` E8M0 uint8 ``[N, K/32]``): passed through for an ``"mxfp4"`` engine, or converted exactly to e4m3 +
  the same E8M0 scales for an ``"e4m3"`` one.
* lm_head and the MTP layer's matrices are bf16 in the checkpoint; they become e4m3 + E8M0 here (`quantize_e4m3`, in
  row slices), where the reference makes e5m2 bytes of them (checkpoint.py:332, 368).
* KV-cache scales (kv_cache_format "fp8") are stretched by 448 / 240 as the reference does (checkpoint.py:32, 227-233)
  and go to `Engine.set_kv_scales`; the MTP file has none (the reference takes measured ones, checkpoint.py:363-392).

Only safetensors loaders are used: nothing in a checkpoint file is executed.
"""

from __future__ import annotations

from collections.abc import Iterator
from pathlib import Path

import torch

from .config import FULL, LINEAR, TextConfig
from .quant import mxfp4_to_e4m3, quantize_e4m3

TEXT_PREFIX = "model.language_model."
LM_HEAD = "lm_head.weight"
EMBED_TOKENS = TEXT_PREFIX + "embed_tokens.weight"
FINAL_NORM = TEXT_PREFIX + "norm.weight"
MTP_FILE = "model_mtp.safetensors"
KV_SCALE_STRETCH = 448.0 / 240.0
ROWS_PER_SLICE = 16384  # rows of a bf16 matrix quantized at once (bounds the float32 temporaries)


class Checkpoint:
    """The tensors of a directory's safetensors files (or of one file), read on demand."""

    def __init__(self, path: str | Path, exclude: tuple[str, ...] = (MTP_FILE,)):
        from safetensors import safe_open

        path = Path(path)
        files = [path] if path.is_file() else sorted(p for p in path.glob("*.safetensors") if p.name not in exclude)
        if not files:
            raise FileNotFoundError(f"no safetensors files in {path}")
        self._handles = [safe_open(str(f), framework="pt") for f in files]
        self._where = {name: h for h in self._handles for name in h.keys()}

    def __contains__(self, name: str) -> bool:
        return name in self._where

    def get(self, name: str) -> torch.Tensor:
        if name not in self._where:
            raise KeyError(f"checkpoint has no tensor {name}")
        return self._where[name].get_tensor(name)


def e4m3_from_bf16(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """A bf16 ``[N, K]`` matrix as e4m3 bytes + E8M0 scales, quantized in row slices."""
    n, k = weight.shape
    coded = torch.empty(n, k, dtype=torch.uint8)
    scales = torch.empty(n, k // 32, dtype=torch.uint8)
    for first in range(0, n, ROWS_PER_SLICE):
        rows = slice(first, min(n, first + ROWS_PER_SLICE))
        coded[rows], scales[rows] = quantize_e4m3(weight[rows].float())
    return coded, scales


def _fp4_matrix(ck: Checkpoint, hf_name: str, weight_format: str):
    packed, scale = ck.get(f"{hf_name}.weight_packed"), ck.get(f"{hf_name}.weight_scale")
    if packed.dtype != torch.uint8 or scale.dtype != torch.uint8 or packed.shape[1] * 2 != scale.shape[1] * 32:
        raise ValueError(f"{hf_name}: expected MXFP4 weight_packed uint8 [N, K/2] and weight_scale uint8 [N, K/32]")
    return (packed, scale) if weight_format == "mxfp4" else mxfp4_to_e4m3(packed, scale)


def layer_weights(ck: Checkpoint, cfg: TextConfig, index: int, weight_format: str = "mxfp4") -> list[tuple[str, object]]:
    """Decoder layer ``index`` (reference checkpoint.py:185-224, one rank holding everything)."""
    hf, ours = f"{TEXT_PREFIX}layers.{index}", f"layers.{index}"
    bf16 = lambda name: ck.get(name).to(torch.bfloat16)  # noqa: E731
    out = [
        (f"{ours}.input_layernorm_weight", bf16(f"{hf}.input_layernorm.weight")),
        (f"{ours}.post_attention_layernorm_weight", bf16(f"{hf}.post_attention_layernorm.weight")),
    ]
    out += [(f"{ours}.mlp.{m}", _fp4_matrix(ck, f"{hf}.mlp.{m}", weight_format)) for m in ("gate_proj", "up_proj", "down_proj")]
    if cfg.layer_types[index] == LINEAR:
        hl, la = f"{hf}.linear_attn", f"{ours}.linear_attn"
        out += [(f"{la}.{m}", _fp4_matrix(ck, f"{hl}.{m}", weight_format)) for m in ("in_proj_qkv", "in_proj_z", "out_proj")]
        out += [
            (f"{la}.in_proj_b", bf16(f"{hl}.in_proj_b.weight")),
            (f"{la}.in_proj_a", bf16(f"{hl}.in_proj_a.weight")),
            (f"{la}.conv_weight", bf16(f"{hl}.conv1d.weight").squeeze(1)),
            (f"{la}.A_log", bf16(f"{hl}.A_log")),
            (f"{la}.dt_bias", bf16(f"{hl}.dt_bias")),
            (f"{la}.norm_weight", bf16(f"{hl}.norm.weight")),
        ]
    elif cfg.layer_types[index] == FULL:
        hs, sa = f"{hf}.self_attn", f"{ours}.self_attn"
        out += [(f"{sa}.{m}", _fp4_matrix(ck, f"{hs}.{m}", weight_format)) for m in ("q_proj", "k_proj", "v_proj", "o_proj")]
        out += [(f"{sa}.q_norm_weight", bf16(f"{hs}.q_norm.weight")), (f"{sa}.k_norm_weight", bf16(f"{hs}.k_norm.weight"))]
    else:
        raise ValueError(f"unknown layer type {cfg.layer_types[index]}")
    return out


def head_weights(ck: Checkpoint) -> list[tuple[str, object]]:
    """Final norm, lm_head (e4m3 + E8M0 for the group maxima, and its bf16 rows for the exact recheck, which the
    reference reads from the checkpoint: generate.py:196-206) and the embedding table (reference checkpoint.py:324-342)."""
    lm_head = ck.get(LM_HEAD).to(torch.bfloat16)
    return [
        ("head.norm_weight", ck.get(FINAL_NORM).to(torch.bfloat16)),
        ("head.lm_head", e4m3_from_bf16(lm_head)),
        ("head.lm_head_rows", lm_head),
        ("embed_tokens", ck.get(EMBED_TOKENS).to(torch.bfloat16)),
    ]


def mtp_weights(mtp: Checkpoint) -> list[tuple[str, object]]:
    """The MTP layer from its own file, bf16 matrices as e4m3 + E8M0 (reference checkpoint.py:363-392)."""
    vec = lambda name: mtp.get(f"mtp.{name}.weight").to(torch.bfloat16)  # noqa: E731
    mat = lambda name: e4m3_from_bf16(mtp.get(f"mtp.{name}.weight"))  # noqa: E731
    out = [
        ("mtp.fc", mat("fc")),
        ("mtp.embedding_norm_weight", vec("pre_fc_norm_embedding")),
        ("mtp.hidden_norm_weight", vec("pre_fc_norm_hidden")),
        ("mtp.norm_weight", vec("norm")),
        ("mtp.layer.input_layernorm_weight", vec("layers.0.input_layernorm")),
        ("mtp.layer.post_attention_layernorm_weight", vec("layers.0.post_attention_layernorm")),
        ("mtp.layer.self_attn.q_norm_weight", vec("layers.0.self_attn.q_norm")),
        ("mtp.layer.self_attn.k_norm_weight", vec("layers.0.self_attn.k_norm")),
    ]
    out += [(f"mtp.layer.self_attn.{m}", mat(f"layers.0.self_attn.{m}")) for m in ("q_proj", "k_proj", "v_proj", "o_proj")]
    out += [(f"mtp.layer.mlp.{m}", mat(f"layers.0.mlp.{m}")) for m in ("gate_proj", "up_proj", "down_proj")]
    return out


def model_weights(directory: str | Path, cfg: TextConfig, weight_format: str = "mxfp4", mtp: bool = True) -> Iterator[tuple[str, object]]:
    """Every weight `Engine.load` takes, layer by layer (so host memory holds about one layer at a time)."""
    if weight_format not in ("mxfp4", "e4m3"):
        raise ValueError(f"weight_format {weight_format!r}")
    ck = Checkpoint(directory)
    for i in range(cfg.num_hidden_layers):
        yield from layer_weights(ck, cfg, i, weight_format)
    yield from head_weights(ck)
    if mtp:
        yield from mtp_weights(Checkpoint(Path(directory) / MTP_FILE, exclude=()))


def kv_scales(directory, cfg: TextConfig) -> dict[int, tuple[torch.Tensor, torch.Tensor]]:
    """Each attention layer's (k_scale, v_scale), bf16 ``[1]``, stretched for the cache's 240 limit (reference
    checkpoint.py:227-233). ``directory`` may also be an open `Checkpoint` (anything with ``get(name)``)."""
    ck = directory if hasattr(directory, "get") else Checkpoint(directory)
    out = {}
    for i, kind in enumerate(cfg.layer_types):
        if kind == FULL:
            hs = f"{TEXT_PREFIX}layers.{i}.self_attn"
            out[i] = tuple((ck.get(f"{hs}.{n}").float() * KV_SCALE_STRETCH).reshape(1).to(torch.bfloat16) for n in ("k_scale", "v_scale"))
    return out
