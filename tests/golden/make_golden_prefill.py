"""Write golden vectors for the prefill form from the reference's own CPU path.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden_prefill.py /root/reference

On config 0 shapes with this build's seeded weights (seed 0) and the verify scenario's starting states (B=4 rows,
max_seq_len 128; tests/golden/make_golden.py), it runs the reference's `Qwen38Step` prefill form twice on row 1: a
full chunk of 64 tokens from position 0 (which restarts the row), then 40 real tokens of the next chunk of 64 from
position 64 (the rest padding); then `MTPStep`'s prefill form (cache only) on the first chunk's hidden states. The
e5m2 weight decode is swapped for this build's exact e4m3 + E8M0 values, as in make_golden.py; every other op is the
reference's. The fixture holds the prompt ids, both chunks' hidden states, the MTP call's output and SHA-256 digests
of every state buffer afterwards; tests/test_oracle.py checks the oracle's prefill against it bit for bit.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parents[1] / "qwen38-27b-aws_amd"))

from make_golden import BATCH, CONTEXT, MAX_SEQ_LEN, SEED, digest  # noqa: E402
from qwen38_amd import synth  # noqa: E402
from qwen38_amd.config import tiny_config  # noqa: E402
from qwen38_amd.quant import dequantize_e4m3  # noqa: E402

SLOT, CHUNK = 1, 64
CHUNKS = [(0, 64), (64, 40)]  # (start, n_valid)


def prompt_ids(vocab: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(4321)
    return torch.randint(0, vocab, (2 * CHUNK,), generator=g)


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from qwen38_inf2 import model as ref_model
    from qwen38_inf2.config import TextConfig as RefConfig
    from qwen38_inf2.generate import mtp_prefill_inputs, prefill_inputs
    from qwen38_inf2.model import MTPStep, Qwen38Step

    cfg = tiny_config(1)
    ref_cfg = RefConfig(**{f: getattr(cfg, f) for f in RefConfig.__dataclass_fields__})
    dtype = torch.bfloat16
    weights = dict((spec.name, value) for spec, value in synth.make_all(synth.model_specs(cfg), SEED))

    dense = {}
    original = ref_model.fp4.fp8_to_float
    ref_model.fp4.fp8_to_float = lambda byte: dense[byte.data_ptr()] if byte.data_ptr() in dense else original(byte)

    def fill(module, prefix: str):
        for name, param in module.named_parameters():
            key = prefix + name
            if name == "final_norm_weight":
                param.data = weights["head.norm_weight"]
            elif name.endswith("weight_fp8"):
                coded, scales = weights[key.removesuffix(".weight_fp8")]
                holder = torch.zeros(coded.shape[1], coded.shape[0], dtype=torch.uint8)
                dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
                param.data = holder
            else:
                param.data = weights[key].to(param.dtype)

    step = Qwen38Step(ref_cfg, MAX_SEQ_LEN, 1, dtype, batch_size=BATCH).eval()
    fill(step, "")
    for i, layer in enumerate(step.layers):
        if cfg.layer_types[i] == "linear_attention":
            st = synth.gdn_states(cfg, BATCH, 4, SEED, f"layers.{i}")
            layer.linear_attn.recurrent_state = st["recurrent_state"]
            layer.linear_attn.conv_state = st["conv_state"]
        else:
            kv = synth.kv_states(cfg, BATCH, MAX_SEQ_LEN, CONTEXT, SEED, f"layers.{i}")
            layer.self_attn.k_cache, layer.self_attn.v_cache = kv["k_cache"], kv["v_cache"]

    ids = prompt_ids(cfg.vocab_size)
    embed = weights["embed_tokens"]
    out = {"ids": ids.to(torch.int32)}
    with torch.no_grad():
        for n, (start, n_valid) in enumerate(CHUNKS):
            chunk_ids = ids[start : start + CHUNK].clone()
            chunk_ids[n_valid:] = 0  # padding, as the scheduler pads
            inputs = prefill_inputs(ref_cfg, SLOT, start, n_valid, CHUNK, dtype)
            out[f"hidden_p{n + 1}"] = step(inputs_embeds=embed[chunk_ids].reshape(1, CHUNK, -1), **inputs)
        states = {name: digest(buf) for name, buf in step.named_buffers() if "recurrent_state" in name or "conv_state" in name or "cache" in name}

        mtp = MTPStep(ref_cfg, 1, MAX_SEQ_LEN, dtype, ref_model.identity_all_reduce, BATCH).eval()
        fill(mtp, "mtp.")
        mkv = synth.kv_states(cfg, BATCH, MAX_SEQ_LEN, CONTEXT, SEED, "mtp")
        mtp.layer.self_attn.k_cache, mtp.layer.self_attn.v_cache = mkv["k_cache"], mkv["v_cache"]
        shifted = torch.cat((ids[1:CHUNK + 1], ids[:0]))
        out["mtp_x"] = mtp(hidden=out["hidden_p1"], inputs_embeds=embed[shifted].reshape(1, CHUNK, -1),
                           **mtp_prefill_inputs(ref_cfg, SLOT, 0, CHUNK, CHUNK, dtype))
        states_mtp = {name: digest(buf) for name, buf in mtp.named_buffers() if "cache" in name}

    from safetensors.torch import save_file

    save_file({k: v.contiguous() for k, v in out.items()}, HERE / "prefill_tiny.safetensors")
    meta = {"seed": SEED, "batch": BATCH, "max_seq_len": MAX_SEQ_LEN, "context": CONTEXT, "slot": SLOT, "chunk": CHUNK,
            "chunks": CHUNKS, "state_sha256": states, "mtp_state_sha256": states_mtp, "torch": torch.__version__}
    (HERE / "prefill_tiny.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", HERE / "prefill_tiny.safetensors")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
