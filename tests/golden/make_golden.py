"""Write golden vectors for the verify path from the reference's own CPU path.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports the reference's CPU modules (qwen38_inf2.model, generate, checkpoint) and runs, on config 0 shapes with
this build's seeded weights (qwen38_amd.synth, seed 0):
* two consecutive verify steps of the 4-layer block (accepted 0, then forced counts 4/2/3/0), B=4 rows with one fresh
  row (position 0) and one inactive row;
* `HeadStep` group maxima and `ChipHead.next_tokens` (4 groups and 1 group) on the second step's hidden states;
* one `MTPStep` step on them.

The reference decodes FP8 weights as e5m2 bytes ``[in, out]`` (fp4.fp8_to_float). This build's weights are e4m3 with
E8M0 scales, so the script swaps that one helper for a lookup returning each weight's exact dequantized values. Every
other op is the reference's own. The fixture holds inputs, outputs and SHA-256 digests of every state buffer after
step 2; tests/test_oracle.py checks the oracle against it bit for bit.
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
from qwen38_amd.config import tiny_config  # noqa: E402
from qwen38_amd.quant import dequantize_e4m3  # noqa: E402

OUT = Path(__file__).resolve().parent
SEED = 0
BATCH, K, MAX_SEQ_LEN = 4, 4, 128
POSITIONS_1 = [40, 64, 0, 17]
ACTIVE = [True, True, True, False]
ACCEPTED_2 = [4, 2, 3, 0]
CONTEXT = [40, 64, 0, 17]


def scenario_ids(vocab: int):
    g = torch.Generator().manual_seed(1234)
    return torch.randint(0, vocab, (2, BATCH, K), generator=g)


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from qwen38_inf2 import checkpoint
    from qwen38_inf2 import model as ref_model
    from qwen38_inf2.config import TextConfig as RefConfig
    from qwen38_inf2.generate import ChipHead, mtp_step_inputs, verify_inputs
    from qwen38_inf2.model import HeadStep, MTPStep, Qwen38Step

    cfg = tiny_config(1)
    ref_cfg = RefConfig(**{f: getattr(cfg, f) for f in RefConfig.__dataclass_fields__})
    dtype = torch.bfloat16
    weights = dict((spec.name, value) for spec, value in synth.make_all(synth.model_specs(cfg), SEED))

    dense = {}
    original = ref_model.fp4.fp8_to_float

    def fp8_lookup(byte: torch.Tensor) -> torch.Tensor:
        return dense[byte.data_ptr()] if byte.data_ptr() in dense else original(byte)

    ref_model.fp4.fp8_to_float = fp8_lookup

    def fill(module, prefix: str):
        for name, param in module.named_parameters():
            key = prefix + name
            if name.endswith("weight_fp8"):
                coded, scales = weights[key.removesuffix(".weight_fp8")]
                holder = torch.zeros(coded.shape[1], coded.shape[0], dtype=torch.uint8)
                dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
                param.data = holder
            else:
                param.data = weights[key].to(param.dtype)

    step = Qwen38Step(ref_cfg, MAX_SEQ_LEN, 1, dtype, batch_size=BATCH, verify_tokens=K).eval()
    fill(step, "")
    for i, layer in enumerate(step.layers):
        if cfg.layer_types[i] == "linear_attention":
            st = synth.gdn_states(cfg, BATCH, K, SEED, f"layers.{i}")
            for key, value in st.items():
                setattr(layer.linear_attn, key, value)
        else:
            kv = synth.kv_states(cfg, BATCH, MAX_SEQ_LEN, CONTEXT, SEED, f"layers.{i}")
            layer.self_attn.k_cache, layer.self_attn.v_cache = kv["k_cache"], kv["v_cache"]

    ids = scenario_ids(cfg.vocab_size)
    embed = weights["embed_tokens"]
    out = {"ids": ids.to(torch.int32)}
    with torch.no_grad():
        inputs1 = verify_inputs(ref_cfg, POSITIONS_1, K, MAX_SEQ_LEN, dtype, ACTIVE, [0] * BATCH)
        hidden1 = step(inputs_embeds=embed[ids[0]].reshape(BATCH, K, -1), **inputs1)
        positions2 = [p + (a if on else 0) for p, a, on in zip(POSITIONS_1, ACCEPTED_2, ACTIVE)]
        inputs2 = verify_inputs(ref_cfg, positions2, K, MAX_SEQ_LEN, dtype, ACTIVE, ACCEPTED_2)
        hidden2 = step(inputs_embeds=embed[ids[1]].reshape(BATCH, K, -1), **inputs2)
        states = {name: digest(buf) for name, buf in step.named_buffers()}

        head = HeadStep(ref_cfg, 1, batch_size=BATCH * K, group_rows=32, head_format="fp8").eval()
        coded, scales = weights["head.lm_head"]
        holder = torch.zeros(cfg.hidden_size, cfg.vocab_size, dtype=torch.uint8)
        dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
        head.lm_head.data = holder
        head.norm_weight.data = weights["head.norm_weight"]
        head.rank_gate.data = torch.ones(1)
        rows = hidden2.reshape(BATCH * K, 1, -1)
        maxima = head(rows)
        source = checkpoint.DictSource(
            {
                checkpoint.FINAL_NORM: weights["head.norm_weight"],
                checkpoint.LM_HEAD: dequantize_e4m3(coded, scales).to(torch.bfloat16),
                checkpoint.EMBED_TOKENS: embed,
            }
        )
        chip = ChipHead(source, cfg.rms_norm_eps, lambda hidden: head(hidden), BATCH * K)
        picks4 = chip.next_tokens(rows)
        picks1 = chip.next_tokens(rows, recheck_groups=1)

        mtp = MTPStep(ref_cfg, 1, MAX_SEQ_LEN, dtype, ref_model.identity_all_reduce, BATCH).eval()
        for name, param in mtp.named_parameters():
            key = "mtp." + name
            if name == "final_norm_weight":
                param.data = weights["head.norm_weight"]
            elif name.endswith("weight_fp8"):
                coded, scales = weights[key.removesuffix(".weight_fp8")]
                holder = torch.zeros(coded.shape[1], coded.shape[0], dtype=torch.uint8)
                dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
                param.data = holder
            else:
                param.data = weights[key].to(param.dtype)
        mkv = synth.kv_states(cfg, BATCH, MAX_SEQ_LEN, CONTEXT, SEED, "mtp")
        mtp.layer.self_attn.k_cache, mtp.layer.self_attn.v_cache = mkv["k_cache"], mkv["v_cache"]
        pick_ids = torch.tensor(picks4).reshape(BATCH, K)
        mtp_out = mtp(hidden=hidden2, inputs_embeds=embed[pick_ids], **mtp_step_inputs(ref_cfg, positions2, K, MAX_SEQ_LEN, dtype, ACTIVE))
        states_mtp = {name: digest(buf) for name, buf in mtp.named_buffers()}

    out.update(
        {
            "cos1": inputs1["cos"], "sin1": inputs1["sin"], "cos2": inputs2["cos"], "sin2": inputs2["sin"],
            "hidden1": hidden1, "hidden2": hidden2, "maxima": maxima,
            "picks4": torch.tensor(picks4, dtype=torch.int32), "picks1": torch.tensor(picks1, dtype=torch.int32),
            "mtp_out": mtp_out,
        }
    )
    from safetensors.torch import save_file

    save_file({k: v.contiguous() for k, v in out.items()}, OUT / "verify_tiny.safetensors")
    meta = {
        "seed": SEED, "batch": BATCH, "tokens": K, "max_seq_len": MAX_SEQ_LEN, "positions_1": POSITIONS_1,
        "positions_2": positions2, "active": ACTIVE, "accepted_2": ACCEPTED_2, "context": CONTEXT,
        "state_sha256": states, "mtp_state_sha256": states_mtp,
        "weights_sha256": {name: digest(v if isinstance(v, torch.Tensor) else torch.cat([v[0].flatten(), v[1].flatten()])) for name, v in sorted(weights.items())},
        "torch": torch.__version__,
    }
    (OUT / "verify_tiny.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", OUT / "verify_tiny.safetensors")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
