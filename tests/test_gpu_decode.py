"""The one-token decode graph and the saved-state copies on the GPU against the CPU oracle (config 0 shapes, seed 0).

* One layer of each kind, three decode steps from positions 40/64/0/17 (row 2 starts a sequence at position 0, so its
  gated-delta states restart from zero; row 3 is inactive), each step started from the oracle's own state: the output
  within the north-star 2e-2 per row, the state after the step within 1e-2, the inactive row's state and cache bit for
  bit. One layer keeps the e5m2 roundings that amplify last-bit differences to a few, so these bounds are tight.
* The whole 4-layer graph on the golden scenario's weights and states: the same three steps, then a verify step with
  accepted = 0, as the reference's scheduler runs one after a decode or prefill step, checked one layer at a time
  (teacher-forced): beside the graph runs a chain of one-layer engines, each fed the hidden states the GPU's layer
  before it produced, from the states the GPU left in it. The same kernels run the same inputs, so the chain's last
  output and every layer's states equal the graph's bit for bit; and each layer's output is held to the north-star
  2e-2 per token (a token above it explained by one e5m2 rounding tie after its mixer, `ties.check_tokens`), its
  states to 1e-2, against the oracle run on that layer's GPU input from its GPU state. The inactive row must come
  back bit for bit.
* `copy_states`: save a row, let decode change it, restore it: the row bit for bit, the other rows untouched.
"""

from __future__ import annotations

import pytest
import torch

import layerwise
import ties
from qwen38_amd import synth
from oracle import model as om
from qwen38_amd.config import tiny_config, with_layers
from qwen38_amd.generate import batch_step_inputs, verify_inputs
from qwen38_amd.steps import Engine, StepGraph
from scenario import clone_states, golden_meta, golden_tensors, oracle_weights, row_rel, tiny_states

DECODE_STEPS = 3


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


def state_of(engine: Engine, cfg, kind: str) -> dict:
    """Layer 0's current state on the host, in the oracle's shapes."""
    return layerwise.gdn_state_from(engine, cfg) if kind == "linear_attention" else layerwise.kv_state_from(engine)


def check_layer_state(kind: str, got: dict, want: dict, what: str) -> None:
    """A layer's state after a step against the oracle's from the same start: every gated-delta state vector within
    1e-2 (per row of conv state, per (row, head) matrix and snapshot vector); the caches within 1e-2 per (row, head,
    position) vector, which covers the positions written and the bit-equal rest alike."""
    for key, w in want.items():
        width = {"recurrent_state": w.shape[-1] * w.shape[-2], "conv_state": w.shape[-2] * w.shape[-1]}.get(key, w.shape[-1])
        if kind != "linear_attention":
            width = w.shape[-1]
        err = float(layerwise.rel_rows(got[key], w, width).max())
        print(f"    {what} {key} {err:.3g}", flush=True)
        assert err <= 1e-2, (what, key)


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
        err = row_rel(got, want)
        print(f"  hidden {err:.3g}", flush=True)
        assert err <= 2e-2
        if kind == "linear_attention":
            mine = engine.gdn_state(0)
            for key in ("recurrent_state", "conv_state"):
                err = row_rel(mine[key], states[0][key])
                print(f"  {key} {err:.3g}", flush=True)
                assert err <= 1e-2, key
                assert torch.equal(mine[key][3].cpu(), before[0][key][3]), key
        else:
            kc, vc = engine.get_kv(0)
            for name, cache in (("k_cache", kc), ("v_cache", vc)):
                for row in range(meta["batch"]):
                    at = pos[row] if active[row] else s - 1
                    assert row_rel(cache[row, :, at], states[0][name][row, :, at]) <= 1e-2, (name, row)
                    keep = torch.ones(s, dtype=torch.bool)
                    keep[at] = False
                    assert torch.equal(cache[row, :, keep].cpu(), before[0][name][row, :, keep]), (name, row)
        pos = [p + 1 if a else p for p, a in zip(pos, active)]


@pytest.mark.gpu
def test_decode_steps_then_verify_layer_by_layer(scenario):
    cfg, meta, values = scenario
    engine, start = load_engine(cfg, meta, values)
    step = StepGraph(engine)
    layers, _, _ = oracle_weights(values, cfg)
    chain = []
    for i, kind in enumerate(cfg.layer_types):
        one = with_layers(cfg, (kind,))
        e = Engine(one, meta["batch"], meta["tokens"], meta["max_seq_len"], mtp=False, saved_states=True)
        e.load(layerwise.layer_values(values, i).items())
        set_states(e, one, [start[i]])
        chain.append((e, StepGraph(e), one, kind, layers[i]))
    gold = golden_tensors()
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    embed, ids, active = values["embed_tokens"], gold["ids"].long(), meta["active"]

    def run(x, oracle_step, **inputs):
        """The graph and the chain on x; every layer of the chain against the oracle from its own GPU input and state."""
        hidden = step(inputs_embeds=x, **inputs)
        h = x
        for i, (e, st, one, kind, w) in enumerate(chain):
            before = state_of(e, one, kind)
            out = st(inputs_embeds=h, **inputs)
            torch.cuda.synchronize()
            with ties.Recorder() as rec:
                want = oracle_step(one, [w], [before], h.cpu())
            o_in = rec.inputs[id(w.get("self_attn.o_proj", w.get("linear_attn.out_proj")))]
            print(f"  layer {i} ({kind})", flush=True)
            hs = cfg.hidden_size
            ties.check_tokens(out.reshape(-1, hs), want.reshape(-1, hs), w, cfg.rms_norm_eps, h.cpu().reshape(-1, hs),
                              o_in.reshape(want.reshape(-1, hs).shape[0], -1))
            check_layer_state(kind, state_of(e, one, kind), before, f"layer {i}")
            h = out
        torch.cuda.synchronize()
        assert torch.equal(h.cpu(), hidden.cpu())  # the chain is the graph, layer by layer
        for i, (e, _, one, kind, _) in enumerate(chain):
            mine, full = state_of(e, one, kind), state_of_layer(engine, cfg, i, kind)
            for key in mine:
                assert torch.equal(mine[key], full[key]), (i, key)

    pos = list(meta["positions_1"])
    for t in range(DECODE_STEPS):
        print(f"decode step {t}", flush=True)
        inputs = batch_step_inputs(cfg, pos, s, torch.bfloat16, active)
        run(embed[ids[0][:, t]].unsqueeze(1),
            lambda one, w, st, h: om.step_decode(one, w, st, h, inputs["cos"], inputs["sin"], inputs["position"],
                                                 inputs["active"]), **inputs)
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
    accepted = vi.pop("accepted")
    run(embed[ids[1]],
        lambda one, w, st, h: om.step_verify(one, w, st, h, vi["cos"], vi["sin"], vi["position"], vi["active"], accepted),
        accepted=accepted, **vi)


def state_of_layer(engine: Engine, cfg, i: int, kind: str) -> dict:
    """Layer i's current state of a multi-layer engine on the host, in the oracle's shapes."""
    if kind == "linear_attention":
        st = {key: v.cpu().clone() for key, v in engine.gdn_state(i).items()}
        st["pending_key_state"] = om.repeat_interleave(st["pending_key_state"], cfg.linear_key_repeat, dim=2).contiguous()
        return st
    kc, vc = engine.get_kv(i)
    return {"k_cache": kc.cpu(), "v_cache": vc.cpu()}


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
