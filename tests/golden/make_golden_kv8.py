"""Write golden vectors for the FP8 KV cache from the reference's own CPU path.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden_kv8.py /root/reference

One attention decoder layer of config 0 shapes (this build's seeded weights, seed 0) with kv_cache_format "fp8":
the layer's k_scale / v_scale from `synth.kv_scales`, its cache the verify scenario's K/V (tests/golden/make_golden.py)
stored as e4m3 bytes. Through the reference's `Qwen38Step` it runs two verify steps (accepted 0, then 4/2/3/0), one
decode step, and one prefill chunk of 64 tokens (40 real) on row 2 from position 16. The e5m2 weight decode is swapped
for this build's exact e4m3 + E8M0 values, as in make_golden.py; every other op, the cache's _store / _load /
_round_trip included, is the reference's. The fixture holds the hidden states of each call and SHA-256 digests of the
cache bytes after each; tests/test_oracle.py checks the oracle's FP8 KV path against it bit for bit.
"""

from __future__ import annotations

import dataclasses
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parents[1] / "qwen38-27b-aws_amd"))

from make_golden import ACCEPTED_2, ACTIVE, BATCH, CONTEXT, K, MAX_SEQ_LEN, POSITIONS_1, SEED, digest  # noqa: E402
from qwen38_amd import synth  # noqa: E402
from qwen38_amd.config import tiny_config, with_layers  # noqa: E402
from qwen38_amd.quant import dequantize_e4m3, encode_kv  # noqa: E402

PREFILL = {"slot": 2, "start": 16, "n_valid": 40, "chunk": 64}


def scenario(cfg):
    """Token ids of the calls and the decode positions (each row's position after step 2's accepted tokens)."""
    g = torch.Generator().manual_seed(777)
    verify_ids = torch.randint(0, cfg.vocab_size, (2, BATCH, K), generator=g)
    decode_ids = torch.randint(0, cfg.vocab_size, (BATCH,), generator=g)
    prefill_ids = torch.randint(0, cfg.vocab_size, (PREFILL["chunk"],), generator=g)
    prefill_ids[PREFILL["n_valid"]:] = 0
    positions_2 = [p + (K if a else 0) for p, a in zip(POSITIONS_1, ACTIVE)]
    decode_positions = [p + (n if a else 0) for p, n, a in zip(positions_2, ACCEPTED_2, ACTIVE)]
    return verify_ids, decode_ids, prefill_ids, positions_2, decode_positions


def layer_config():
    return with_layers(tiny_config(1), ("full_attention",))


def initial_cache(cfg):
    """(k_scale, v_scale, k bytes, v bytes) of the layer before the first call."""
    ks, vs = synth.kv_scales(cfg, SEED, "layers.0")
    kv = synth.kv_states(cfg, BATCH, MAX_SEQ_LEN, CONTEXT, SEED, "layers.0")
    return ks, vs, encode_kv(kv["k_cache"], ks), encode_kv(kv["v_cache"], vs)


def main(reference: str) -> None:
    sys.path.insert(0, reference)
    from qwen38_inf2 import model as ref_model
    from qwen38_inf2.config import TextConfig as RefConfig
    from qwen38_inf2.generate import batch_step_inputs, prefill_inputs, verify_inputs
    from qwen38_inf2.model import Qwen38Step

    cfg = layer_config()
    ref_cfg = RefConfig(**{f: getattr(cfg, f) for f in RefConfig.__dataclass_fields__ if hasattr(cfg, f)})
    ref_cfg = dataclasses.replace(ref_cfg, kv_cache_format="fp8")
    dtype = torch.bfloat16
    weights = dict((spec.name, value) for spec, value in synth.make_all(synth.model_specs(cfg), SEED))
    ks, vs, kc, vc = initial_cache(cfg)

    dense = {}
    original = ref_model.fp4.fp8_to_float
    ref_model.fp4.fp8_to_float = lambda byte: dense[byte.data_ptr()] if byte.data_ptr() in dense else original(byte)

    step = Qwen38Step(ref_cfg, MAX_SEQ_LEN, 1, dtype, batch_size=BATCH, verify_tokens=K).eval()
    for name, param in step.named_parameters():
        if name.endswith("weight_fp8"):
            coded, scales = weights[name.removesuffix(".weight_fp8")]
            holder = torch.zeros(coded.shape[1], coded.shape[0], dtype=torch.uint8)
            dense[holder.data_ptr()] = dequantize_e4m3(coded, scales).T.contiguous()
            param.data = holder
        elif name.endswith("k_scale"):
            param.data = ks.clone()
        elif name.endswith("v_scale"):
            param.data = vs.clone()
        else:
            param.data = weights[name].to(param.dtype)
    attn = step.layers[0].self_attn
    assert attn.fp8_cache
    attn.k_cache, attn.v_cache = kc.clone(), vc.clone()

    verify_ids, decode_ids, prefill_ids, positions_2, decode_positions = scenario(cfg)
    embed = weights["embed_tokens"]
    out, digests = {}, {}

    def record(name, hidden):
        out[name] = hidden
        digests[name] = {"k_cache": digest(attn.k_cache), "v_cache": digest(attn.v_cache)}

    with torch.no_grad():
        in1 = verify_inputs(ref_cfg, POSITIONS_1, K, MAX_SEQ_LEN, dtype, ACTIVE, [0] * BATCH)
        record("verify1", step(inputs_embeds=embed[verify_ids[0]], **in1))
        in2 = verify_inputs(ref_cfg, positions_2, K, MAX_SEQ_LEN, dtype, ACTIVE, ACCEPTED_2)
        record("verify2", step(inputs_embeds=embed[verify_ids[1]], **in2))
        di = batch_step_inputs(ref_cfg, decode_positions, MAX_SEQ_LEN, dtype, ACTIVE)
        record("decode", step(inputs_embeds=embed[decode_ids].unsqueeze(1), **di))
        pi = prefill_inputs(ref_cfg, PREFILL["slot"], PREFILL["start"], PREFILL["n_valid"], PREFILL["chunk"], dtype)
        record("prefill", step(inputs_embeds=embed[prefill_ids].unsqueeze(0), **pi))

    from safetensors.torch import save_file

    save_file({k: v.contiguous() for k, v in out.items()}, HERE / "kv8_tiny.safetensors")
    meta = {"seed": SEED, "batch": BATCH, "tokens": K, "max_seq_len": MAX_SEQ_LEN, "context": CONTEXT,
            "positions_1": POSITIONS_1, "positions_2": positions_2, "decode_positions": decode_positions,
            "active": ACTIVE, "accepted_2": ACCEPTED_2, "prefill": PREFILL, "cache_sha256": digests,
            "torch": torch.__version__}
    (HERE / "kv8_tiny.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", HERE / "kv8_tiny.safetensors")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
