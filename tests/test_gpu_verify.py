"""The verify path on the GPU against the CPU oracle on the golden scenario (config 0 shapes, seed 0; one fresh row at
position 0 and one inactive row): the head's group maxima and picks and one MTP step on the reference's own hidden
states, two consecutive verify steps layer by layer (the second commits 4/2/3/0 tokens), embeddings and acceptance.

* The head and the MTP step take the reference's hidden states, so they are compared directly: maxima within 1e-4,
  picks exact except at rows whose top-2 logit gap is below 1e-3, the MTP output within 2e-2 per token.
* The verify steps are teacher-forced per layer (tests/layerwise.py): each layer from the GPU's own input and state,
  its output within 2e-2 per token and every state vector within 1e-2.
"""

from __future__ import annotations

import pytest
import torch

from layerwise import HIDDEN_TOL, STATE_NAMES, STATE_TOL, LayerStack, rel_rows
from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import mtp_step_inputs, verify_inputs
from qwen38_amd.steps import Engine, HeadGraph, MTPStep
from scenario import golden_meta, golden_tensors, oracle_weights, tiny_states


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
def test_mtp_step_on_the_references_inputs(scenario):
    cfg, meta, values, engine = scenario
    gold = golden_tensors()
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    picks = gold["picks4"].long().reshape(b, k)
    mi = mtp_step_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"])
    out = MTPStep(engine)(hidden=gold["hidden2"], inputs_embeds=values["embed_tokens"][picks], **mi)
    torch.cuda.synchronize()
    err = rel_rows(out, gold["mtp_out"], cfg.hidden_size)
    print(f"mtp out per token: max {float(err.max()):.3g}, median {float(err.median()):.3g}", flush=True)
    assert float(err.max()) <= HIDDEN_TOL


@pytest.mark.gpu
def test_two_verify_steps_layer_by_layer(scenario):
    cfg, meta, values, _ = scenario
    gold = golden_tensors()
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    stack = LayerStack(cfg, values, b, k, s, tiny_states(cfg, meta, meta["seed"]))
    embed, ids = values["embed_tokens"], gold["ids"].long()
    worst = {}
    steps = ((meta["positions_1"], [0] * b, ids[0]), (meta["positions_2"], meta["accepted_2"], ids[1]))
    for n, (positions, accepted, step_ids) in enumerate(steps):
        print(f"verify step {n + 1}", flush=True)
        inputs = verify_inputs(cfg, positions, k, s, torch.bfloat16, meta["active"], accepted)
        out = stack.verify_step(embed[step_ids].cuda(), {name: t.cuda() for name, t in inputs.items()},
                                log=lambda m: print(m, flush=True))
        for key, value in out["worst"].items():
            worst[key] = max(worst.get(key, 0.0), value)
    assert worst["hidden"] <= HIDDEN_TOL
    for key, value in worst.items():
        if key in STATE_NAMES:
            assert value <= STATE_TOL, key


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
