"""The whole verify path on the GPU against the CPU oracle on the golden scenario (config 0 shapes, seed 0): two
consecutive verify steps (the second commits 4/2/3/0 tokens), the committed states, the head's group maxima and picks,
and one MTP step. Tolerances: hidden states and logits 2e-2 relative, committed bf16 state
1e-2 relative, picks exact except at rows whose top-2 logit gap is below 1e-3."""

from __future__ import annotations

import pytest
import torch

from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import mtp_step_inputs, verify_inputs
from qwen38_amd.steps import Engine, HeadGraph, MTPStep, VerifyStep
from scenario import clone_states, golden_meta, golden_tensors, oracle_weights, tiny_states


def rel(got: torch.Tensor, want: torch.Tensor) -> float:
    """Largest absolute difference relative to the reference tensor's largest magnitude."""
    got, want = got.float().cpu(), want.float().cpu()
    return float((got - want).abs().max() / want.abs().max().clamp_min(1e-30))


@pytest.fixture(scope="module")
def scenario(gpu):
    cfg = tiny_config(1)
    meta = golden_meta()
    values = dict((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    engine = Engine(cfg, meta["batch"], meta["tokens"], meta["max_seq_len"], mtp=True)
    engine.load(values.items())
    states = tiny_states(cfg, meta, meta["seed"])
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, states[i])
        else:
            engine.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])
    mkv = synth.kv_states(cfg, meta["batch"], meta["max_seq_len"], meta["context"], meta["seed"], "mtp")
    engine.set_kv(engine.mtp_layer, mkv["k_cache"], mkv["v_cache"])
    return cfg, meta, values, engine, states


@pytest.mark.gpu
def test_verify_head_and_mtp_match_the_oracle(scenario):
    cfg, meta, values, engine, states = scenario
    gold = golden_tensors()
    layers, mtp_w, head_w = oracle_weights(values, cfg)
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    embed = values["embed_tokens"]
    ids = gold["ids"].long()
    verify = VerifyStep(engine)
    ref_states = clone_states(states)

    print("verify step 1", flush=True)
    in1 = verify_inputs(cfg, meta["positions_1"], k, s, torch.bfloat16, meta["active"], [0] * b)
    h1 = verify(inputs_embeds=embed[ids[0]], **in1)
    torch.cuda.synchronize()
    assert rel(h1, gold["hidden1"]) < 2e-2
    om.step_verify(cfg, layers, ref_states, embed[ids[0]], in1["cos"], in1["sin"], in1["position"], in1["active"], in1["accepted"])

    print("verify step 2", flush=True)
    in2 = verify_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"], meta["accepted_2"])
    h2 = verify(inputs_embeds=embed[ids[1]], **in2)
    torch.cuda.synchronize()
    assert rel(h2, gold["hidden2"]) < 2e-2
    om.step_verify(cfg, layers, ref_states, embed[ids[1]], in2["cos"], in2["sin"], in2["position"], in2["active"], in2["accepted"])

    # Committed and snapshot state after step 2.
    rep = cfg.linear_key_repeat
    for i, kind in enumerate(cfg.layer_types):
        want = ref_states[i]
        if kind == "linear_attention":
            got = engine.gdn_state(i)
            assert rel(got["recurrent_state"], want["recurrent_state"]) < 1e-2, i
            assert rel(got["conv_state"], want["conv_state"]) < 1e-2, i
            assert rel(got["pending_input_state"], want["pending_input_state"]) < 2e-2, i
            assert rel(got["pending_key_state"], want["pending_key_state"][:, :, ::rep]) < 2e-2, i
            assert rel(got["pending_delta_state"], want["pending_delta_state"]) < 2e-2, i
            assert rel(got["pending_decay_state"], want["pending_decay_state"]) < 2e-2, i
        else:
            kc, vc = engine.get_kv(i)
            for row, p in enumerate(meta["positions_2"]):
                if meta["active"][row]:
                    # Positions before the step's own writes are committed; the last step's writes sit there too.
                    assert rel(kc[row, :, : p + k], want["k_cache"][row, :, : p + k]) < 1e-2, (i, row)
                    assert rel(vc[row, :, : p + k], want["v_cache"][row, :, : p + k]) < 1e-2, (i, row)

    print("head", flush=True)
    head = HeadGraph(engine)
    rows = h2.reshape(b * k, 1, -1)
    maxima = head(hidden=rows)
    assert rel(maxima, gold["maxima"]) < 2e-2
    gaps = om.top2_gap(cfg, head_w["norm_weight"], head_w["lm_head"], gold["hidden2"].reshape(b * k, 1, -1))
    picks4 = head.pick(rows, 4).tolist()
    picks1 = head.pick(rows, 1).tolist()
    for got, want, gap in zip(picks4, gold["picks4"].tolist(), gaps.tolist()):
        assert got == want or gap < 1e-3
    for got, want, gap in zip(picks1, gold["picks1"].tolist(), gaps.tolist()):
        assert got == want or gap < 1e-3

    print("mtp", flush=True)
    mtp = MTPStep(engine)
    picks = gold["picks4"].long().reshape(b, k)
    mi = mtp_step_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"])
    out = mtp(hidden=gold["hidden2"], inputs_embeds=embed[picks], **mi)
    torch.cuda.synchronize()
    assert rel(out, gold["mtp_out"]) < 2e-2


@pytest.mark.gpu
def test_embedding_rows_and_acceptance_on_the_gpu(scenario):
    cfg, meta, values, engine, _ = scenario
    head = HeadGraph(engine)
    ids = [0, 5, cfg.vocab_size - 1, 77]
    assert torch.equal(head.embed(ids).cpu(), values["embed_tokens"][ids])
    with pytest.raises(ValueError):
        head.embed([cfg.vocab_size])
    b, k = meta["batch"], meta["tokens"]
    picks = torch.tensor([[5, 6, 7, 8], [5, 6, 7, 8], [1, 2, 3, 4], [9, 9, 9, 9]], dtype=torch.int32).cuda()
    drafts = torch.tensor([[5, 6, 9], [5, 6, 7], [2, 2, 3], [9, 9, 9]], dtype=torch.int32).cuda()
    active = torch.tensor([1.0, 1.0, 1.0, 0.0]).cuda()
    match = torch.empty(b, dtype=torch.int32).cuda()
    accepted = torch.empty(b, dtype=torch.int32).cuda()
    engine.handle.accept(picks, drafts, active, match, accepted)
    assert match.tolist() == [2, 3, 0, 3]
    assert accepted.tolist() == [3, 4, 1, 0]
    for row in range(b):
        assert om.accept(picks[row].tolist(), drafts[row].tolist(), k)[0] == match[row]
