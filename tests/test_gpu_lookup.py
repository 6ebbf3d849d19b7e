"""The verify step with prompt-lookup drafts (the reference's `Scheduler._verify_step` without an MTP drafter,
scheduler.py:269-301 with drafting.py:27-51) on the GPU, at config 0 shapes.

* Plumbing, bit for bit: five `steps.LookupStep` steps (the product's `drafting.Drafter` on the host, one
  `q38_verify_step` per step on the device) equal the oracle's restated scheduler (pinned to the reference's own on
  this scenario, tests/golden/lookup_tiny.*) driving this build's `VerifyStep` and `ChipHead` over `HeadGraph` on a
  second engine: emitted tokens, drafts, picks, matches, accepted counts, positions, verify hidden states and every
  state buffer; accepted counts 1 to 4 all occur.
* Every decision proven (tests/spec_check.py): each step's verify layer by layer, its head picks and its acceptance.
"""

from __future__ import annotations

import pytest
import torch

from oracle import scheduler as osch
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import ChipHead
from qwen38_amd.steps import Engine, LookupStep
from scenario import LOOKUP, lookup_start, spec_states, steer_head
from spec_check import OracleWeights, Recorder, host_slots, prove_step, run_host_step

B, K, S = LOOKUP["batch"], LOOKUP["tokens"], LOOKUP["max_seq_len"]


@pytest.fixture(scope="module")
def lookup_run(gpu):
    cfg = tiny_config(1)
    values = steer_head(dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg, mtp=False), LOOKUP["seed"])), cfg,
                        LOOKUP["seed"])
    states, _ = spec_states(cfg, LOOKUP)

    def engine():
        e = Engine(cfg, B, K, S, mtp=False)
        e.load(values.items())
        for i, kind in enumerate(cfg.layer_types):
            if kind == "linear_attention":
                e.set_gdn(i, states[i])
            else:
                e.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])
        return e

    dev_engine, host_engine = engine(), engine()
    start = lookup_start(cfg)
    device = LookupStep(dev_engine, [row["ids"] if row else None for row in start], [row["prompt_len"] if row else 0 for row in start])
    rec = Recorder(host_engine)
    sched = osch.Scheduler(None, None, ChipHead(None, cfg.rms_norm_eps, rec.head, B * K), cfg, B, S, LOOKUP["chunk"],
                           verify=rec.verify, verify_tokens=K)
    slots = host_slots(start, mtp=False)
    steps = []
    for n in range(LOOKUP["steps"]):
        print(f"step {n}", flush=True)
        emitted_dev = device()
        positions, ready, emitted = run_host_step(sched, slots)
        steps.append({"emitted_dev": emitted_dev, "emitted": dict(zip(ready, emitted)), "last": dict(sched.last), "ready": ready,
                      "device": {n_: getattr(device, n_).clone() for n_ in ("drafts", "picks", "match", "accepted", "position", "hidden")},
                      "written": [row.written if row else 0 for row in slots]})
    return cfg, values, dev_engine, host_engine, rec, steps


@pytest.mark.gpu
def test_lookup_steps_equal_the_restated_scheduler(lookup_run):
    cfg, _, dev_engine, host_engine, _, steps = lookup_run
    counts = set()
    for n, step in enumerate(steps):
        dev, last = step["device"], step["last"]
        for b in step["ready"]:
            assert step["emitted_dev"][b] == step["emitted"][b], (n, b)
            assert dev["drafts"][b].tolist() == last["drafts"][b], (n, b)
            assert dev["picks"][b].tolist() == last["picks"][b], (n, b)
            assert int(dev["match"][b]) == last["match"][b] and int(dev["accepted"][b]) == last["match"][b] + 1, (n, b)
            assert int(dev["position"][b]) == step["written"][b], (n, b)
            assert torch.equal(dev["hidden"][b], last["hidden"][b]), (n, b)
            counts.add(last["match"][b] + 1)
        assert step["emitted_dev"][3] is None
    assert counts == {1, 2, 3, 4}, counts
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            got, want = dev_engine.gdn_state(i), host_engine.gdn_state(i)
            for key in got:
                assert torch.equal(got[key][:3], want[key][:3]), (i, key)
        else:
            for a, bb in zip(dev_engine.get_kv(i), host_engine.get_kv(i)):
                assert torch.equal(a[:3], bb[:3]), i


@pytest.mark.gpu
def test_every_lookup_pick_and_accepted_count_is_the_oracles_decision(lookup_run):
    cfg, values, _, host_engine, rec, steps = lookup_run
    weights = OracleWeights(cfg, values)
    log = lambda m: print(m, flush=True)
    for n, step in enumerate(steps):
        worst = prove_step(host_engine, weights, rec, step["last"], first_head=n, first_mtp=0, verify_call=n, log=log)
        log(f"step {n}: worst {{{', '.join(f'{key}: {v:.3g}' for key, v in worst.items() if key != 'head')}}}, "
            f"picks differing (near-ties) {worst['head']['differ']} of {worst['head']['rows']}")
