"""Write golden vectors at the 27B widths from the reference's own CPU path: one gated-delta layer and one attention
layer, each with its MLP, at H = 5120 (16 key heads and 48 value heads, a three-fold value-head repeat; 24 query heads
over 4 KV heads, six-fold GQA; SwiGLU 17408), B = 2 rows of K = 4 tokens.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden_27b_slice.py /root/reference

It imports the reference's CPU modules (qwen38_inf2.model, generate) and runs two consecutive verify steps of a
two-layer `Qwen38Step` (layer types [linear_attention, full_attention], the 27B config otherwise) with this build's
seeded weights (qwen38_amd.synth on the CPU, seed 7) and seeded states and caches: step 1 commits nothing, step 2
commits 3 and 2 tokens. The inputs are seeded embeddings (no vocabulary table at this width). As in make_golden.py, the
reference's e5m2 weight decoder is swapped for a lookup returning each weight's exact dequantized e4m3 + E8M0 values;
every other op is the reference's own. The fixture holds the two steps' hidden states and cos/sin, and SHA-256
digests of every state buffer after step 2 (the weights and states are regenerated from the seed by the test).
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "qwen38-27b-aws_amd"))

from qwen38_amd import synth  # noqa: E402
from qwen38_amd.config import qwen38_27b_config, with_layers  # noqa: E402
from qwen38_amd.quant import dequantize_e4m3  # noqa: E402

OUT = Path(__file__).resolve().parent
SLICE = {"seed": 7, "batch": 2, "tokens": 4, "max_seq_len": 128, "context": [40, 64], "accepted_2": [3, 2],
         "layer_types": ["linear_attention", "full_attention"]}


def slice_config():
    return with_layers(qwen38_27b_config(1), tuple(SLICE["layer_types"]))


def slice_states(cfg):
    """Seeded unit-RMS gated-delta and conv states (empty snapshots) and caches filled below each row's context."""
    b, k, s, seed = SLICE["batch"], SLICE["tokens"], SLICE["max_seq_len"], SLICE["seed"]
    states = []
    for i, kind in enumerate(cfg.layer_types):
        one = with_layers(cfg, (kind,))
        if kind == "linear_attention":
            states.append(synth.gdn_states(one, b, k, seed, f"slice.{i}"))
        else:
            states.append(synth.kv_states(one, b, s, SLICE["context"], seed, f"slice.{i}"))
    return states


def slice_inputs(cfg):
    """The two steps' input embeddings [2, B, K, H] (bf16, RMS 0.02 like the embedding table's rows)."""
    x = synth.hidden_states((2, SLICE["batch"], SLICE["tokens"], cfg.hidden_size), SLICE["seed"], "slice.x")
    return (x.float() * 0.02).to(torch.bfloat16)


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from qwen38_inf2 import model as ref_model
    from qwen38_inf2.config import TextConfig as RefConfig
    from qwen38_inf2.generate import verify_inputs
    from qwen38_inf2.model import Qwen38Step

    cfg = slice_config()
    ref_cfg = RefConfig(**{f: getattr(cfg, f) for f in RefConfig.__dataclass_fields__})
    dtype = torch.bfloat16
    b, k, s = SLICE["batch"], SLICE["tokens"], SLICE["max_seq_len"]
    weights = dict((spec.name, value) for spec, value in synth.make_all(synth.model_specs(cfg, mtp=False, head=False), SLICE["seed"]))

    dense = {}
    original = ref_model.fp4.fp8_to_float
    ref_model.fp4.fp8_to_float = lambda byte: dense[byte.data_ptr()] if byte.data_ptr() in dense else original(byte)
    step = Qwen38Step(ref_cfg, s, 1, dtype, batch_size=b, verify_tokens=k).eval()
    for name, param in step.named_parameters():
        if name.endswith("weight_fp8"):
            coded, scales = weights[name.removesuffix(".weight_fp8")]
            holder = torch.zeros(coded.shape[1], coded.shape[0], dtype=torch.uint8)
            dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
            param.data = holder
        else:
            param.data = weights[name].to(param.dtype)
    for i, (layer, st) in enumerate(zip(step.layers, slice_states(cfg))):
        target = layer.linear_attn if cfg.layer_types[i] == "linear_attention" else layer.self_attn
        for key, value in st.items():
            setattr(target, key, value)
    x = slice_inputs(cfg)
    positions = SLICE["context"]
    out = {}
    with torch.no_grad():
        inputs1 = verify_inputs(ref_cfg, positions, k, s, dtype, [True] * b, [0] * b)
        out["hidden1"] = step(inputs_embeds=x[0], **inputs1)
        positions2 = [p + a for p, a in zip(positions, SLICE["accepted_2"])]
        inputs2 = verify_inputs(ref_cfg, positions2, k, s, dtype, [True] * b, SLICE["accepted_2"])
        out["hidden2"] = step(inputs_embeds=x[1], **inputs2)
        states = {name: digest(buf) for name, buf in step.named_buffers()}
    out.update(cos1=inputs1["cos"], sin1=inputs1["sin"], cos2=inputs2["cos"], sin2=inputs2["sin"])
    from safetensors.torch import save_file

    save_file({key: v.contiguous() for key, v in out.items()}, OUT / "slice_27b.safetensors")
    meta = {**SLICE, "positions_2": positions2, "state_sha256": states, "torch": torch.__version__}
    (OUT / "slice_27b.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", OUT / "slice_27b.safetensors", {key: float(v.float().norm()) for key, v in out.items() if key.startswith("hidden")})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
