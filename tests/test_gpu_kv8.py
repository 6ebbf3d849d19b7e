"""The FP8 KV cache on the GPU (e4m3 bytes of value / scale with per-layer bf16 scales; the reference's kv_cache_format
"fp8", model.py:557-601) against the reference and the oracle, on the FP8 KV golden scenario: one attention decoder
layer through two verify steps, a decode step and a prefill chunk (tests/golden/kv8_tiny.*, written from the
reference's own CPU path; the oracle is pinned to it bit for bit on the CPU).

* Hidden states after each call against the reference's, per token (test_gpu_prefill.check_tokens): the bulk at the
  float32 level, every token within 0.15, at most one in sixteen above the north-star 2e-2. A token above it has an
  e5m2 tie at an activation, or one of its own key or value bytes on the neighbouring e4m3 code, decided the other
  way by a float32-ulp difference upstream; the step grows to a few percent of that token's row through the MLP.
* Cache bytes after each call against the oracle's: the GPU's keys and values come out of its own GEMM and norm, a
  float32 ulp or so from the oracle's, and e4m3 rounds them to 1/16 of a value: so a few bytes may land on the
  neighbouring code. Held to: at most 1% of the bytes differ, each by one code step, and positions no call writes
  keep their bytes.
"""

from __future__ import annotations

import json
import sys

import pytest
import torch

from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.generate import batch_step_inputs, prefill_inputs, verify_inputs
from qwen38_amd.steps import Engine, StepGraph, VerifyStep
from safetensors.torch import load_file
from scenario import GOLDEN, oracle_weights
from test_gpu_prefill import check_tokens


def row_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu().reshape(want.shape[0], -1), want.float().cpu().reshape(want.shape[0], -1)
    return max(float((g - w).norm() / w.norm().clamp_min(1e-30)) for g, w in zip(got, want))


def check_codes(got: torch.Tensor, want: torch.Tensor, name: str) -> None:
    got, want = got.cpu().to(torch.int32), want.to(torch.int32)
    diff = got != want
    frac = float(diff.float().mean())
    # e4m3 codes of one sign are ordered by magnitude: a neighbouring value is one code away
    step = ((got - want).abs() == 1) & ((got ^ want) & 0x80 == 0)
    print(f"{name}: {int(diff.sum())} of {diff.numel()} bytes differ ({frac:.2%})", flush=True)
    assert frac <= 0.01 and bool(step[diff].all()), name


@pytest.mark.gpu
def test_fp8_kv_cache_steps_like_the_reference(gpu):
    sys.path.insert(0, str(GOLDEN))
    import make_golden_kv8 as g8

    cfg = g8.layer_config()
    meta = json.loads((GOLDEN / "kv8_tiny.json").read_text())
    gold = load_file(GOLDEN / "kv8_tiny.safetensors")
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), g8.SEED))
    layers, _, _ = oracle_weights(values, cfg)
    ks, vs, kc, vc = g8.initial_cache(cfg)
    st = {"k_cache": kc.clone(), "v_cache": vc.clone(), "k_scale": ks, "v_scale": vs}

    engine = Engine(cfg, b, k, s, mtp=False, prefill_chunk=meta["prefill"]["chunk"], kv_cache_format="fp8")
    engine.load((n, v) for n, v in values.items() if not n.startswith("mtp."))
    engine.set_kv_scales(0, ks, vs)
    engine.set_kv(0, kc, vc)
    verify, step = VerifyStep(engine), StepGraph(engine)
    verify_ids, decode_ids, prefill_ids, positions_2, decode_positions = g8.scenario(cfg)
    embed, kind = values["embed_tokens"], "full_attention"

    def check(name, got, want):
        torch.cuda.synchronize()
        gk, gv = engine.get_kv(0)
        check_codes(gk, st["k_cache"], f"{name} k_cache")
        check_codes(gv, st["v_cache"], f"{name} v_cache")
        h = gold[name].shape[-1]
        rows = [r for r in range(b) if meta["active"][r]]  # an inactive row's output is not used
        print(f"{name}: CPU builds apart {row_rel(want, gold[name]):.3g}", flush=True)
        check_tokens(got[rows].reshape(-1, h), gold[name][rows].reshape(-1, h))

    for n, (pos, acc) in enumerate(((meta["positions_1"], [0] * b), (positions_2, meta["accepted_2"]))):
        print(f"verify {n + 1}", flush=True)
        vi = verify_inputs(cfg, pos, k, s, torch.bfloat16, meta["active"], acc)
        got = verify(inputs_embeds=embed[verify_ids[n]], **vi)
        want = om.decoder_layer(cfg, kind, layers[0], st, embed[verify_ids[n]], vi["cos"], vi["sin"], vi["position"],
                                vi["active"], accepted=vi["accepted"])
        check(f"verify{n + 1}", got, want)
    print("decode", flush=True)
    di = batch_step_inputs(cfg, decode_positions, s, torch.bfloat16, meta["active"])
    got = step(inputs_embeds=embed[decode_ids].unsqueeze(1), **di)
    want = om.decoder_layer(cfg, kind, layers[0], st, embed[decode_ids].unsqueeze(1), di["cos"], di["sin"], di["position"],
                            di["active"])
    check("decode", got, want)
    print("prefill", flush=True)
    p = meta["prefill"]
    pi = prefill_inputs(cfg, p["slot"], p["start"], p["n_valid"], p["chunk"], torch.bfloat16)
    x = embed[prefill_ids].unsqueeze(0)
    got = step(inputs_embeds=x, **pi)
    want = om.decoder_layer(cfg, kind, layers[0], st, x, pi["cos"], pi["sin"], None, None, slot=pi["slot"],
                            start=pi["start"], n_valid=pi["n_valid"])
    # Only row `slot`'s prefill positions are compared: the reference also writes junk at every other row's last
    # positions, which this build leaves alone (nothing reads them before a later step overwrites them).
    torch.cuda.synchronize()
    n = p["n_valid"]
    check_tokens(got[0, :n], gold["prefill"][0, :n])
    gk, gv = engine.get_kv(0)
    span = slice(p["start"], p["start"] + p["chunk"])
    check_codes(gk[p["slot"], :, span], st["k_cache"][p["slot"], :, span], "prefill k_cache")
    check_codes(gv[p["slot"], :, span], st["v_cache"][p["slot"], :, span], "prefill v_cache")
