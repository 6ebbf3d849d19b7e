"""The whole verify path on the GPU against the CPU oracle on the golden scenario (config 0 shapes, seed 0): two
consecutive verify steps (the second commits 4/2/3/0 tokens), the committed state, the head's group maxima and picks,
and one MTP step.

Two kinds of check:
* quantities computed from identical inputs (the head on the reference's hidden states, the MTP step on them): tight
  tolerances, picks exact except at rows whose top-2 logit gap is below 1e-3;
* end-to-end quantities (hidden states after 4 layers, state after two steps): within twice the distance between the
  oracle and the reference's own CPU path built with scalar kernels (tests/floor.py; one sample of a stochastic
  floor, hence the factor), or within the north-star tolerances (2e-2 hidden, 1e-2 committed state) where that floor
  is below them.
"""

from __future__ import annotations

import pytest
import torch

import floor
from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import mtp_step_inputs, verify_inputs
from qwen38_amd.steps import Engine, HeadGraph, MTPStep, VerifyStep
from scenario import golden_meta, golden_tensors, oracle_weights, tiny_states

FLOOR_FACTOR = 2.0


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
    return cfg, meta, values, engine


@pytest.mark.gpu
def test_head_picks_and_maxima_from_the_references_hidden_states(scenario):
    cfg, meta, values, engine = scenario
    gold = golden_tensors()
    _, _, head_w = oracle_weights(values, cfg)
    b, k = meta["batch"], meta["tokens"]
    rows = gold["hidden2"].reshape(b * k, 1, -1)
    head = HeadGraph(engine)
    maxima = head(hidden=rows)
    assert rel(maxima, gold["maxima"]) < 1e-4
    gaps = om.top2_gap(cfg, head_w["norm_weight"], head_w["lm_head"], rows)
    for groups, want in ((4, gold["picks4"]), (1, gold["picks1"])):
        picks = head.pick(rows, groups).tolist()
        for got, ref, gap in zip(picks, want.tolist(), gaps.tolist()):
            assert got == ref or gap < 1e-3, (groups, got, ref, gap)


@pytest.mark.gpu
def test_mtp_step_on_the_references_inputs(scenario, references):
    cfg, meta, values, engine = scenario
    gold = golden_tensors()
    ref, scalar = references
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    picks = gold["picks4"].long().reshape(b, k)
    mi = mtp_step_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"])
    out = MTPStep(engine)(hidden=gold["hidden2"], inputs_embeds=values["embed_tokens"][picks], **mi)
    torch.cuda.synchronize()
    assert torch.equal(ref["mtp_out"], gold["mtp_out"]) or floor.row_rel(ref["mtp_out"], gold["mtp_out"]) < 2e-2
    bound = max(2e-2, FLOOR_FACTOR * floor.row_rel(scalar["mtp_out"], gold["mtp_out"]))
    assert floor.row_rel(out, gold["mtp_out"]) <= bound


@pytest.mark.gpu
def test_two_verify_steps_stay_within_the_references_own_floor(scenario, references):
    cfg, meta, values, engine = scenario
    gold = golden_tensors()
    ref, scalar = references
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    embed = values["embed_tokens"]
    ids = gold["ids"].long()
    verify = VerifyStep(engine)

    def check(name, got, tol):
        floor_err = floor.row_rel(scalar[name], ref[name])
        err = floor.row_rel(got, ref[name])
        print(f"{name}: gpu {err:.3g}, scalar-build floor {floor_err:.3g}", flush=True)
        assert err <= max(tol, FLOOR_FACTOR * floor_err), name

    print("verify step 1", flush=True)
    in1 = verify_inputs(cfg, meta["positions_1"], k, s, torch.bfloat16, meta["active"], [0] * b)
    h1 = verify(inputs_embeds=embed[ids[0]], **in1)
    check("hidden1", h1, 2e-2)
    print("verify step 2", flush=True)
    in2 = verify_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"], meta["accepted_2"])
    h2 = verify(inputs_embeds=embed[ids[1]], **in2)
    torch.cuda.synchronize()
    check("hidden2", h2, 2e-2)

    rep = cfg.linear_key_repeat
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            got = engine.gdn_state(i)
            check(f"state.{i}.recurrent_state", got["recurrent_state"], 1e-2)
            check(f"state.{i}.conv_state", got["conv_state"], 1e-2)
            for key in ("pending_input_state", "pending_delta_state", "pending_decay_state"):
                check(f"state.{i}.{key}", got[key], 2e-2)
            ref[f"state.{i}.pending_key_state"] = ref[f"state.{i}.pending_key_state"][:, :, ::rep]
            scalar[f"state.{i}.pending_key_state"] = scalar[f"state.{i}.pending_key_state"][:, :, ::rep]
            check(f"state.{i}.pending_key_state", got["pending_key_state"], 2e-2)
        else:
            kc, vc = engine.get_kv(i)
            for name, cache in (("k_cache", kc), ("v_cache", vc)):
                # Committed positions and the last step's own writes; the inactive row writes only the tail.
                for row, p in enumerate(meta["positions_2"]):
                    if meta["active"][row]:
                        key = f"state.{i}.{name}"
                        err = floor.row_rel(cache[row : row + 1, :, : p + k], ref[key][row : row + 1, :, : p + k])
                        floor_err = floor.row_rel(scalar[key][row : row + 1, :, : p + k], ref[key][row : row + 1, :, : p + k])
                        assert err <= max(1e-2, FLOOR_FACTOR * floor_err), (name, row)


@pytest.mark.gpu
def test_embedding_rows_and_acceptance_on_the_gpu(scenario):
    cfg, meta, values, engine = scenario
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
