"""The one-token decode graph and the saved-state copies on the GPU against the CPU oracle (config 0 shapes, seed 0).

* One layer of each kind, three decode steps from positions 40/64/0/17 (row 2 starts a sequence at position 0, so its
  gated-delta states restart from zero; row 3 is inactive), each step started from the oracle's own state: the output
  within the north-star 2e-2 per row, the state after the step within 1e-2, the inactive row's state and cache bit for
  bit. One layer keeps the e5m2 roundings that amplify last-bit differences to a few, so these bounds are tight.
* The whole 4-layer graph on the golden scenario's weights and states: the same three steps, then a verify step with
  accepted = 0, as the reference's scheduler runs one after a decode or prefill step. After four layers a single
  flipped rounding (a gate's bf16 linear output one ulp apart, say) grows to percents, as it does between the oracle
  and its own scalar-kernel build, so the hidden states are held to that floor (tests/floor.py: twice the distance
  between the two builds) or to 2e-2 where the floor is below it; the inactive row must come back bit for bit.
* `copy_states`: save a row, let decode change it, restore it: the row bit for bit, the other rows untouched.
"""

from __future__ import annotations

import pytest
import torch

import floor
from qwen38_amd import synth
from oracle import model as om
from qwen38_amd.config import tiny_config, with_layers
from qwen38_amd.generate import batch_step_inputs, verify_inputs
from qwen38_amd.steps import Engine, StepGraph
from scenario import clone_states, golden_meta, golden_tensors, oracle_weights, tiny_states

FLOOR_FACTOR = 2.0


def set_states(engine, cfg, states):
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, states[i])
        else:
            engine.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])


def load_engine(cfg, meta, values):
    engine = Engine(cfg, meta["batch"], meta["tokens"], meta["max_seq_len"], mtp=False, saved_states=True)
    engine.load((n, v) for n, v in values.items() if not n.startswith("mtp."))
    states = tiny_states(cfg, meta, meta["seed"])
    set_states(engine, cfg, states)
    return engine, states


@pytest.fixture(scope="module")
def scenario(gpu):
    cfg = tiny_config(1)
    meta = golden_meta()
    values = dict((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    return cfg, meta, values


def check(ref, scalar, name, got, tol):
    floor_err = floor.row_rel(scalar[name], ref[name])
    err = floor.row_rel(got, ref[name])
    print(f"{name}: gpu {err:.3g}, scalar-build floor {floor_err:.3g}", flush=True)
    assert err <= max(tol, FLOOR_FACTOR * floor_err), name


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["linear_attention", "full_attention"])
def test_one_layer_decodes_like_the_oracle_step_by_step(gpu, kind):
    cfg = with_layers(tiny_config(1), (kind,))
    meta = golden_meta()
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    layers, _, _ = oracle_weights(values, cfg)
    engine, states = load_engine(cfg, meta, values)
    step = StepGraph(engine)
    s, active, embed = meta["max_seq_len"], meta["active"], values["embed_tokens"]
    ids = golden_tensors()["ids"].long()
    pos = list(meta["positions_1"])
    for t in range(3):
        print(f"{kind} step {t}", flush=True)
        set_states(engine, cfg, states)  # this step starts from the oracle's state
        inputs = batch_step_inputs(cfg, pos, s, torch.bfloat16, active)
        x = embed[ids[0][:, t]].unsqueeze(1)
        got = step(inputs_embeds=x, **inputs)
        torch.cuda.synchronize()
        before = clone_states(states)
        want = om.step_decode(cfg, layers, states, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"])
        err = floor.row_rel(got, want)
        print(f"  hidden {err:.3g}", flush=True)
        assert err <= 2e-2
        if kind == "linear_attention":
            mine = engine.gdn_state(0)
            for key in ("recurrent_state", "conv_state"):
                err = floor.row_rel(mine[key], states[0][key])
                print(f"  {key} {err:.3g}", flush=True)
                assert err <= 1e-2, key
                assert torch.equal(mine[key][3].cpu(), before[0][key][3]), key
        else:
            kc, vc = engine.get_kv(0)
            for name, cache in (("k_cache", kc), ("v_cache", vc)):
                for row in range(meta["batch"]):
                    at = pos[row] if active[row] else s - 1
                    assert floor.row_rel(cache[row, :, at], states[0][name][row, :, at]) <= 1e-2, (name, row)
                    keep = torch.ones(s, dtype=torch.bool)
                    keep[at] = False
                    assert torch.equal(cache[row, :, keep].cpu(), before[0][name][row, :, keep]), (name, row)
        pos = [p + 1 if a else p for p, a in zip(pos, active)]


@pytest.mark.gpu
def test_decode_steps_then_verify_stay_within_the_references_own_floor(scenario, references):
    cfg, meta, values = scenario
    ref, scalar = references
    engine, start = load_engine(cfg, meta, values)
    step = StepGraph(engine)
    gold = golden_tensors()
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    embed, ids, active = values["embed_tokens"], gold["ids"].long(), meta["active"]
    pos = list(meta["positions_1"])
    for t in range(floor.DECODE_STEPS):
        print(f"decode step {t}", flush=True)
        inputs = batch_step_inputs(cfg, pos, s, torch.bfloat16, active)
        hidden = step(inputs_embeds=embed[ids[0][:, t]].unsqueeze(1), **inputs)
        torch.cuda.synchronize()
        check(ref, scalar, f"decode.hidden{t}", hidden, 2e-2)
        pos = [p + 1 if a else p for p, a in zip(pos, active)]

    # The inactive row keeps its states exactly and writes only the cache's last position.
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            got = engine.gdn_state(i)
            for key in ("recurrent_state", "conv_state"):
                assert torch.equal(got[key][3].cpu(), start[i][key][3]), (i, key)
        else:
            kc, vc = engine.get_kv(i)
            for name, cache in (("k_cache", kc), ("v_cache", vc)):
                assert torch.equal(cache[3, :, : s - 1].cpu(), start[i][name][3, :, : s - 1]), (i, name)

    print("verify after decode", flush=True)
    vi = verify_inputs(cfg, pos, k, s, torch.bfloat16, active, [0] * b)
    hidden = step(inputs_embeds=embed[ids[1]], accepted=vi.pop("accepted"), **vi)
    torch.cuda.synchronize()
    check(ref, scalar, "decode.verify", hidden, 2e-2)


@pytest.mark.gpu
def test_copy_states_saves_and_restores_one_row_exactly(scenario):
    cfg, meta, values = scenario
    engine, _ = load_engine(cfg, meta, values)
    step = StepGraph(engine)
    s, active = meta["max_seq_len"], meta["active"]
    embed = values["embed_tokens"]
    linear = [i for i, kind in enumerate(cfg.layer_types) if kind == "linear_attention"]
    zeros = torch.zeros(1, 1, cfg.hidden_size, dtype=torch.bfloat16)

    def snapshot():
        return {(i, key): engine.gdn_state(i)[key].clone() for i in linear for key in ("recurrent_state", "conv_state")}

    before = snapshot()
    assert step(inputs_embeds=zeros, save_slot=torch.tensor([1], dtype=torch.int32)) is zeros
    pos = list(meta["positions_1"])
    for t in range(2):
        inputs = batch_step_inputs(cfg, pos, s, torch.bfloat16, active)
        step(inputs_embeds=embed[torch.tensor([3, 4, 5, 6]) + t].unsqueeze(1), **inputs)
        pos = [p + 1 if a else p for p, a in zip(pos, active)]
    moved = snapshot()
    assert not torch.equal(moved[(linear[0], "recurrent_state")][1], before[(linear[0], "recurrent_state")][1])
    step(inputs_embeds=zeros, restore_slot=torch.tensor([1], dtype=torch.int32))
    torch.cuda.synchronize()
    after = snapshot()
    for (i, key), value in after.items():
        assert torch.equal(value[1], before[(i, key)][1]), (i, key)          # row 1 restored bit for bit
        assert torch.equal(value[0], moved[(i, key)][0]), (i, key)           # other rows untouched by the copy
        assert torch.equal(value[2], moved[(i, key)][2]), (i, key)

    # An engine built without saved states refuses the copy, as the reference's layer does.
    plain = Engine(cfg, meta["batch"], meta["tokens"], s, mtp=False)
    with pytest.raises(ValueError):
        StepGraph(plain)(inputs_embeds=zeros, save_slot=torch.tensor([0], dtype=torch.int32))
