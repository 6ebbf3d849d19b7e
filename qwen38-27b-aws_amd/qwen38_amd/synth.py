"""Seeded synthetic weights, states and drafts for the verify-path workloads.

There are no real weights: every workload runs on random-init weights of the right architecture. Each tensor gets
its own generator, seeded from (seed, tensor name), so a tensor does not depend on which others were made first.
The same code runs on CPU (tests, oracle) or on the GPU (the 27B configs, 25 GB of FP8 weights); the two devices'
generators give different values, so a GPU-side test copies what it made back for the oracle.

Distributions (plus the builder's choices where it says nothing, marked *):
* FP8 projections: N(0, 0.02), quantized to e4m3 with an E8M0 scale per 32 (`quant.quantize_e4m3`).
* in_proj_a / in_proj_b (bf16 in the checkpoint, reference model.py:294-296): N(0, 0.02).
* embeddings: N(0, 0.02), bf16.
* (1 + w) norm weights*: N(0, 0.1), so a kernel that drops the weight or the 1 is caught.
* gated-norm weight*: 1 + N(0, 0.1).
* conv weights*: N(0, 0.3), so conv outputs are not negligible next to the state.
* A_log = log U(1, 16) (Hugging Face Qwen3.5 init); dt_bias* = -4, so per-token decays exp(g) spread over (0, 1)
  instead of collapsing to 0, and the state commit and cross-token terms matter.
* states: gated-delta state, conv state and prefix KV are N(0, 1) in bf16 (unit RMS); snapshots start at zero.
"""

from __future__ import annotations

import zlib
from collections.abc import Iterable, Iterator
from dataclasses import dataclass

import torch

from .config import FULL, LINEAR, TextConfig
from .quant import dequantize_e4m3, mxfp4_to_e4m3, quantize_e4m3, quantize_mxfp4


@dataclass(frozen=True)
class Spec:
    name: str
    kind: str  # "fp8", "normal", "norm", "gated_norm", "a_log", "const"
    shape: tuple
    std: float = 0.0
    value: float = 0.0


def _gen(seed: int, name: str, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed((seed * 1000003 + zlib.crc32(name.encode())) & 0x7FFFFFFFFFFF)
    return g


def _randn(shape, seed: int, name: str, device) -> torch.Tensor:
    return torch.randn(*shape, generator=_gen(seed, name, device), device=device, dtype=torch.float32)


def layer_specs(cfg: TextConfig, index: int, prefix: str | None = None) -> list[Spec]:
    """Weights of decoder layer ``index`` with the reference's `Qwen38Step` names (checkpoint.py:185-224)."""
    p = prefix if prefix is not None else f"layers.{index}."
    h, inter = cfg.hidden_size, cfg.intermediate_size
    out = [
        Spec(p + "input_layernorm_weight", "norm", (h,)),
        Spec(p + "post_attention_layernorm_weight", "norm", (h,)),
        Spec(p + "mlp.gate_proj", "fp8", (inter, h)),
        Spec(p + "mlp.up_proj", "fp8", (inter, h)),
        Spec(p + "mlp.down_proj", "fp8", (h, inter)),
    ]
    layer_type = cfg.layer_types[index] if prefix is None else FULL
    if layer_type == LINEAR:
        la = p + "linear_attn."
        hv = cfg.linear_num_value_heads
        out += [
            Spec(la + "in_proj_qkv", "fp8", (cfg.linear_conv_dim, h)),
            Spec(la + "in_proj_z", "fp8", (cfg.linear_value_dim, h)),
            Spec(la + "out_proj", "fp8", (h, cfg.linear_value_dim)),
            Spec(la + "in_proj_b", "normal", (hv, h), std=0.02),
            Spec(la + "in_proj_a", "normal", (hv, h), std=0.02),
            Spec(la + "conv_weight", "normal", (cfg.linear_conv_dim, cfg.linear_conv_kernel_dim), std=0.3),
            Spec(la + "A_log", "a_log", (hv,)),
            Spec(la + "dt_bias", "const", (hv,), value=-4.0),
            Spec(la + "norm_weight", "gated_norm", (cfg.linear_value_head_dim,)),
        ]
    else:
        sa = p + "self_attn."
        hd = cfg.head_dim
        out += [
            Spec(sa + "q_proj", "fp8", (cfg.num_attention_heads * hd * 2, h)),
            Spec(sa + "k_proj", "fp8", (cfg.num_key_value_heads * hd, h)),
            Spec(sa + "v_proj", "fp8", (cfg.num_key_value_heads * hd, h)),
            Spec(sa + "o_proj", "fp8", (h, cfg.num_attention_heads * hd)),
            Spec(sa + "q_norm_weight", "norm", (hd,)),
            Spec(sa + "k_norm_weight", "norm", (hd,)),
        ]
    return out


def mtp_specs(cfg: TextConfig) -> list[Spec]:
    """The MTP layer with `model.MTPStep` names (checkpoint.py:363-392), prefixed ``mtp.``. Its final norm weight is
    the head's (``head.norm_weight``), as in the reference."""
    h = cfg.hidden_size
    return [
        Spec("mtp.fc", "fp8", (h, 2 * h)),
        Spec("mtp.embedding_norm_weight", "norm", (h,)),
        Spec("mtp.hidden_norm_weight", "norm", (h,)),
        Spec("mtp.norm_weight", "norm", (h,)),
    ] + layer_specs(cfg, 0, prefix="mtp.layer.")


def head_specs(cfg: TextConfig) -> list[Spec]:
    h = cfg.hidden_size
    return [
        Spec("head.norm_weight", "norm", (h,)),
        Spec("head.lm_head", "fp8", (cfg.vocab_size, h)),
        Spec("embed_tokens", "normal", (cfg.vocab_size, h), std=0.02),
    ]


def model_specs(cfg: TextConfig, mtp: bool = True, head: bool = True) -> list[Spec]:
    specs = [s for i in range(cfg.num_hidden_layers) for s in layer_specs(cfg, i)]
    if head or mtp:
        specs += head_specs(cfg)
    if mtp:
        specs += mtp_specs(cfg)
    return specs


def make(spec: Spec, seed: int, device="cpu"):
    """One weight: (e4m3 bytes, E8M0 bytes) for "fp8", else a bf16 tensor."""
    if spec.kind == "fp8":
        n, k = spec.shape
        # Rows in slices bound the float32 temporary for lm_head and the MLP matrices.
        coded = torch.empty(n, k, dtype=torch.uint8, device=device)
        scales = torch.empty(n, k // 32, dtype=torch.uint8, device=device)
        g = _gen(seed, spec.name, device)
        step = max(1, (1 << 26) // k)
        for first in range(0, n, step):
            rows = min(step, n - first)
            w = torch.randn(rows, k, generator=g, device=device, dtype=torch.float32) * 0.02
            coded[first : first + rows], scales[first : first + rows] = quantize_e4m3(w)
        return coded, scales
    if spec.kind == "normal":
        if spec.shape[0] * (spec.shape[1] if len(spec.shape) > 1 else 1) > (1 << 26):
            out = torch.empty(*spec.shape, dtype=torch.bfloat16, device=device)
            g = _gen(seed, spec.name, device)
            step = max(1, (1 << 26) // spec.shape[1])
            for first in range(0, spec.shape[0], step):
                rows = min(step, spec.shape[0] - first)
                out[first : first + rows] = (torch.randn(rows, spec.shape[1], generator=g, device=device) * spec.std).to(torch.bfloat16)
            return out
        return (_randn(spec.shape, seed, spec.name, device) * spec.std).to(torch.bfloat16)
    if spec.kind == "norm":
        return (_randn(spec.shape, seed, spec.name, device) * 0.1).to(torch.bfloat16)
    if spec.kind == "gated_norm":
        return (1.0 + _randn(spec.shape, seed, spec.name, device) * 0.1).to(torch.bfloat16)
    if spec.kind == "a_log":
        u = torch.rand(*spec.shape, generator=_gen(seed, spec.name, device), device=device) * 15.0 + 1.0
        return torch.log(u).to(torch.bfloat16)
    if spec.kind == "const":
        return torch.full(spec.shape, spec.value, dtype=torch.bfloat16, device=device)
    raise ValueError(spec.kind)


def make_all(specs: list[Spec], seed: int, device="cpu") -> Iterator[tuple[Spec, object]]:
    for spec in specs:
        yield spec, make(spec, seed, device)


def to_mxfp4(weights: Iterable[tuple[str, object]]) -> Iterator[tuple[str, object]]:
    """The same model as an MXFP4 checkpoint holds it: each decoder layer's projection requantized from its e4m3 values
    to (packed E2M1 [N, K/2], E8M0 [N, K/32]); the MTP layer and the head, bf16 in such a checkpoint, stay e4m3."""
    for name, value in weights:
        if name.startswith("layers.") and isinstance(value, tuple):
            coded, scales = value
            n, k = coded.shape
            packed = torch.empty(n, k // 2, dtype=torch.uint8, device=coded.device)
            e8m0 = torch.empty_like(scales)
            step = max(32, (1 << 24) // k)  # rows per slice: bounds the quantizer's [rows, K, 8] temporary
            for first in range(0, n, step):
                rows = slice(first, min(n, first + step))
                packed[rows], e8m0[rows] = quantize_mxfp4(dequantize_e4m3(coded[rows], scales[rows]))
            value = (packed, e8m0)
        yield name, value


def mxfp4_as_e4m3(weights: Iterable[tuple[str, object]]) -> Iterator[tuple[str, object]]:
    """`to_mxfp4`'s model with its decoder-layer projections written back as e4m3 + E8M0, value for value (exact)."""
    for name, value in weights:
        if name.startswith("layers.") and isinstance(value, tuple):
            value = mxfp4_to_e4m3(*value)
        yield name, value


# ----------------------------------------------------------------------------------------------- states


def gdn_state_shapes(cfg: TextConfig, batch: int, tokens: int) -> dict:
    hv, d, c = cfg.linear_num_value_heads, cfg.linear_key_head_dim, cfg.linear_conv_dim
    return {
        "recurrent_state": ((batch, hv, d, d), torch.bfloat16),
        "conv_state": ((batch, c, cfg.linear_conv_kernel_dim - 1), torch.bfloat16),
        "pending_key_state": ((batch, tokens, hv, d), torch.float32),
        "pending_delta_state": ((batch, tokens, hv, d), torch.float32),
        "pending_decay_state": ((batch, tokens, hv), torch.float32),
        "pending_input_state": ((batch, tokens, c), torch.bfloat16),
    }


def gdn_states(cfg: TextConfig, batch: int, tokens: int, seed: int, name: str, device="cpu") -> dict:
    """Unit-RMS bf16 recurrent and conv states; zero snapshots (the first verify step after them commits none)."""
    out = {}
    for key, (shape, dtype) in gdn_state_shapes(cfg, batch, tokens).items():
        if key in ("recurrent_state", "conv_state"):
            out[key] = _randn(shape, seed, f"{name}.{key}", device).to(dtype)
        else:
            out[key] = torch.zeros(shape, dtype=dtype, device=device)
    return out


def kv_states(cfg: TextConfig, batch: int, max_seq_len: int, context, seed: int, name: str, device="cpu") -> dict:
    """bf16 K/V caches ``[B, Hkv, S, hd]``: N(0, 1) at each row's first ``context[b]`` positions, zero after."""
    shape = (batch, cfg.num_key_value_heads, max_seq_len, cfg.head_dim)
    out = {}
    for key in ("k_cache", "v_cache"):
        cache = torch.zeros(shape, dtype=torch.bfloat16, device=device)
        g = _gen(seed, f"{name}.{key}", device)
        for b in range(batch):
            n = int(context[b])
            if n:
                cache[b, :, :n] = torch.randn(cfg.num_key_value_heads, n, cfg.head_dim, generator=g, device=device).to(torch.bfloat16)
        out[key] = cache
    return out


def kv_scales(cfg: TextConfig, seed: int, name: str, device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """One attention layer's FP8 KV-cache scales (k_scale, v_scale), bf16 ``[1]`` each, as a checkpoint's calibrated
    static scales (reference checkpoint.py:227-233): about 3 / 240, so unit-RMS keys and values use e4m3's range and the
    largest few clamp."""
    u = torch.rand(2, generator=_gen(seed, f"{name}.kv_scales", device), device=device)
    s = (0.0125 * (1.0 + 0.5 * u)).to(torch.bfloat16)
    return s[0:1].clone(), s[1:2].clone()


def hidden_states(shape, seed: int, name: str, device="cpu") -> torch.Tensor:
    """Unit-RMS bf16 activations (e.g. a step's input embeddings or an MTP seed's hidden states)."""
    return _randn(shape, seed, name, device).to(torch.bfloat16)


def corrupt_drafts(greedy: list[list[int]], vocab: int, seed: int, p: float = 0.3) -> list[list[int]]:
    """Each greedy draft replaced with probability ``p`` by a uniform random token (1, 3)."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for row in greedy:
        draws = torch.rand(len(row), generator=g).tolist()
        tokens = torch.randint(0, vocab, (len(row),), generator=g).tolist()
        out.append([t if d >= p else r for t, d, r in zip(row, draws, tokens)])
    return out


def prefix_drafts(greedy: list[list[int]], vocab: int, seed: int) -> list[list[int]]:
    """Config 4: each row keeps a uniform number L in 0..K-1 of greedy drafts and has draft L+1 replaced by a token
    that differs from the greedy one, so exactly L drafts are accepted."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for row in greedy:
        keep = int(torch.randint(0, len(row) + 1, (1,), generator=g))
        row = list(row)
        if keep < len(row):
            row[keep] = (row[keep] + 1 + int(torch.randint(0, vocab - 1, (1,), generator=g))) % vocab
        out.append(row)
    return out
