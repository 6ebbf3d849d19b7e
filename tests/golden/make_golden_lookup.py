"""Write golden vectors for the verify step with prompt-lookup drafts from the reference's own Scheduler.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden_lookup.py /root/reference

It imports the reference's CPU modules (qwen38_inf2.scheduler, drafting, model, generate, checkpoint) and runs five
calls of `Scheduler._verify_step` with no MTP drafter, so every row's drafts come from its own `Drafter`
(scheduler.py:276-282), as `Scheduler.run_sessions` does between prefills, on config 0 shapes in bf16 with this
build's seeded weights (qwen38_amd.synth, seed 0) and the steered head of tests/scenario.py. Four slots: three running
rows seeded as a prefill leaves them (tests/scenario.py `lookup_start`: prompts of 40, 64 and 1 tokens ending in runs
of the steered tokens, plus the first new token) over the speculative scenario's seeded states and caches, and one
empty slot.

As in make_golden.py, the reference's e5m2 weight decoder is swapped for a lookup returning each weight's exact
dequantized e4m3 + E8M0 values; every other op is the reference's own. The fixture holds per step the positions, the
accepted counts the verify commits, the padded drafts, the head's picks, the matches and the verify hidden states;
plus SHA-256 digests of every decoder state buffer after the last step.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (ROOT, ROOT / "qwen38-27b-aws_amd", HERE.parent):
    sys.path.insert(0, str(p))

from qwen38_amd import synth  # noqa: E402
from qwen38_amd.config import tiny_config  # noqa: E402
from qwen38_amd.quant import dequantize_e4m3  # noqa: E402
from scenario import LOOKUP, lookup_start, spec_states, steer_head  # noqa: E402

SEED = LOOKUP["seed"]
BATCH, K, MAX_SEQ_LEN, CHUNK = LOOKUP["batch"], LOOKUP["tokens"], LOOKUP["max_seq_len"], LOOKUP["chunk"]
STEPS = LOOKUP["steps"]


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from qwen38_inf2 import checkpoint
    from qwen38_inf2 import model as ref_model
    from qwen38_inf2.config import TextConfig as RefConfig
    from qwen38_inf2.generate import ChipHead
    from qwen38_inf2.model import HeadStep, Qwen38Step
    from qwen38_inf2.scheduler import Scheduler, _Row

    cfg = tiny_config(1)
    ref_cfg = RefConfig(**{f: getattr(cfg, f) for f in RefConfig.__dataclass_fields__})
    dtype = torch.bfloat16
    weights = steer_head(dict((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg), SEED)), cfg, SEED)

    dense = {}
    original = ref_model.fp4.fp8_to_float
    ref_model.fp4.fp8_to_float = lambda byte: dense[byte.data_ptr()] if byte.data_ptr() in dense else original(byte)

    def fp8_holder(name):
        coded, scales = weights[name]
        holder = torch.zeros(coded.shape[1], coded.shape[0], dtype=torch.uint8)
        dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
        return holder

    step = Qwen38Step(ref_cfg, MAX_SEQ_LEN, 1, dtype, batch_size=BATCH, verify_tokens=K).eval()
    for name, param in step.named_parameters():
        param.data = fp8_holder(name.removesuffix(".weight_fp8")) if name.endswith("weight_fp8") else weights[name].to(param.dtype)
    states, _ = spec_states(cfg, LOOKUP)
    for i, layer in enumerate(step.layers):
        target = layer.linear_attn if cfg.layer_types[i] == "linear_attention" else layer.self_attn
        for key, value in states[i].items():
            setattr(target, key, value.clone())

    head = HeadStep(ref_cfg, 1, batch_size=BATCH * K, group_rows=32, head_format="fp8").eval()
    head.lm_head.data = fp8_holder("head.lm_head")
    head.norm_weight.data = weights["head.norm_weight"]
    head.rank_gate.data = torch.ones(1)
    coded, scales = weights["head.lm_head"]
    source = checkpoint.DictSource({
        checkpoint.FINAL_NORM: weights["head.norm_weight"],
        checkpoint.LM_HEAD: dequantize_e4m3(coded, scales).to(torch.bfloat16),
        checkpoint.EMBED_TOKENS: weights["embed_tokens"],
    })
    chip = ChipHead(source, cfg.rms_norm_eps, lambda hidden: head(hidden), BATCH * K)

    sched = Scheduler(None, None, chip, ref_cfg, BATCH, MAX_SEQ_LEN, CHUNK, (), dtype, verify=lambda **inputs: step(**inputs),
                      verify_tokens=K)
    start = lookup_start(cfg)
    slots = []
    for slot, row in enumerate(start):
        if row is None:
            slots.append(None)
            continue
        r = _Row((slot, 0), list(row["ids"]), row["prompt_len"])
        r.written = row["prompt_len"]
        slots.append(r)

    seen = {}
    real_verify = sched.verify

    def verify_recording(**inputs):
        seen["accepted"] = inputs["accepted"].clone()
        seen["embeds"] = inputs["inputs_embeds"].clone()
        seen["hidden"] = real_verify(**inputs)
        return seen["hidden"]

    sched.verify = verify_recording
    real_next = chip.next_tokens

    def next_recording(hidden, recheck_groups=None):
        seen["chosen"] = real_next(hidden, recheck_groups)
        return seen["chosen"]

    chip.next_tokens = next_recording
    embed_rows = weights["embed_tokens"]
    out = {}
    counts = set()
    with torch.no_grad():
        for n in range(STEPS):
            positions = [row.written if row else 0 for row in slots]
            active = [row is not None for row in slots]
            ready = [slot for slot, row in enumerate(slots) if row]
            emitted = sched._verify_step(slots, positions, active, ready)
            drafts = torch.full((BATCH, K - 1), -1, dtype=torch.int32)
            picks = torch.full((BATCH, K), -1, dtype=torch.int32)
            match = torch.full((BATCH,), -1, dtype=torch.int32)
            chosen = iter(emitted)
            for slot in ready:
                # The verify's tokens are [last, drafts]; recover the drafts from the embedded rows the step verified.
                rows = seen["embeds"][slot, 1:].reshape(K - 1, -1)
                for j in range(K - 1):
                    hit = (embed_rows == rows[j]).all(dim=-1).nonzero().flatten().tolist()
                    drafts[slot, j] = hit[0]
                tokens = next(chosen)
                match[slot] = len(tokens) - 1
                counts.add(len(tokens))
            for i, slot in enumerate(ready):
                picks[slot] = torch.tensor(seen["chosen"][i * K : (i + 1) * K], dtype=torch.int32)
            for slot, tokens in zip(ready, emitted):
                assert tokens == picks[slot, : match[slot] + 1].tolist()
                slots[slot].ids += tokens
                slots[slot].written += len(tokens)
            out.update({f"step{n}.positions": torch.tensor(positions, dtype=torch.int32), f"step{n}.drafts": drafts,
                        f"step{n}.picks": picks, f"step{n}.match": match, f"step{n}.accepted_in": seen["accepted"].to(torch.int32),
                        f"step{n}.hidden": seen["hidden"]})
            print(f"step {n}: positions {positions} drafts {drafts.tolist()} picks {picks.tolist()} match {match.tolist()}")
        state_digests = {name: digest(buf) for name, buf in step.named_buffers()}
    print("accepted counts seen:", sorted(counts))

    for slot, row in enumerate(start):
        if row is not None:
            out[f"start.ids.{slot}"] = torch.tensor(row["ids"], dtype=torch.int32)
    from safetensors.torch import save_file

    save_file({k: v.contiguous() for k, v in out.items()}, HERE / "lookup_tiny.safetensors")
    meta = {**LOOKUP, "state_sha256": state_digests, "torch": torch.__version__, "accepted_counts": sorted(counts)}
    (HERE / "lookup_tiny.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", HERE / "lookup_tiny.safetensors")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
