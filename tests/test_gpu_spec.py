"""`q38_spec_step`, the whole speculative step bench.py times (three MTP drafts with the one-group head, the K-token
verify, the head over every row's K tokens with the top-4 recheck, acceptance, position advance), on the GPU, at
config 0 shapes (tests/test_gpu_config2.py runs the benched configuration itself).

* Plumbing, bit for bit: five device-side steps equal the oracle's restatement of the reference's
  `Scheduler._verify_step` / `_mtp_drafts` (oracle/scheduler.py, pinned to the reference's own scheduler) driving this
  build's step objects (`VerifyStep`, `MTPStep`, `ChipHead` over `HeadGraph`) from the same state: drafts, picks,
  matches, accepted counts, positions, MTP indices, verify hidden states and every state buffer of the running rows;
  the empty slot's decoder state is untouched.
* Every decision proven (tests/spec_check.py): each step's MTP calls, its verify (every layer teacher-forced, stage by
  stage), its head calls (each pick the oracle's from the same hidden row, or a proven near-tie) and its acceptance
  (the oracle's acceptance of those picks and drafts). So every pick, draft and accepted count is explained.
* The un-forced drift: the all-CPU oracle from each step's starting state over the same inputs, its hidden states and
  picks against the device's, reported.

The steered head of tests/scenario.py makes drafts agree with the model's picks about half the time, so accepted
counts 1 to 4 all occur.
"""

from __future__ import annotations

import pytest
import torch

from layerwise import rel_rows
from oracle import model as om
from oracle import scheduler as osch
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import ChipHead
from qwen38_amd.steps import Engine, HeadGraph
from scenario import SPEC, spec_start, spec_states, steer_head
from spec_check import DeviceStep, OracleWeights, Recorder, head_logits, host_slots, oracle_chain, prove_step, run_host_step

B, K, S = SPEC["batch"], SPEC["tokens"], SPEC["max_seq_len"]


@pytest.fixture(scope="module")
def spec(gpu):
    cfg = tiny_config(1)
    values = steer_head(dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), SPEC["seed"])), cfg, SPEC["seed"])
    return cfg, values


def load_engine(cfg, values):
    engine = Engine(cfg, B, K, S, mtp=True)
    engine.load(values.items())
    states, mtp_kv = spec_states(cfg)
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, states[i])
        else:
            engine.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])
    engine.set_kv(engine.mtp_layer, mtp_kv["k_cache"], mtp_kv["v_cache"])
    return engine, states


@pytest.fixture(scope="module")
def spec_run(spec):
    """Five device steps on one engine and five restated-scheduler steps over recorded step objects on another."""
    cfg, values = spec
    dev_engine, start_states = load_engine(cfg, values)
    host_engine, _ = load_engine(cfg, values)
    start = spec_start(cfg)
    device = DeviceStep(dev_engine, start)
    rec = Recorder(host_engine)
    head = ChipHead(None, cfg.rms_norm_eps, rec.head, B * K)
    sched = osch.Scheduler(None, None, head, cfg, B, S, SPEC["chunk"], verify=rec.verify, verify_tokens=K, mtp=rec.mtp)
    slots = host_slots(start)
    steps = []
    for n in range(SPEC["steps"]):
        print(f"step {n}", flush=True)
        device()
        positions, ready, _ = run_host_step(sched, slots)
        steps.append({"device": {name: getattr(device, name).clone() for name in
                                 ("drafts", "picks", "match", "accepted", "index", "position", "hidden")},
                      "last": dict(sched.last), "positions": positions, "ready": ready,
                      "written": [row.written if row else 0 for row in slots]})
    return cfg, values, dev_engine, host_engine, start_states, rec, steps


@pytest.mark.gpu
def test_device_step_equals_the_restated_scheduler_on_this_builds_step_objects(spec_run):
    cfg, _, dev_engine, host_engine, start_states, _, steps = spec_run
    counts = set()
    for n, step in enumerate(steps):
        dev, last = step["device"], step["last"]
        for b in step["ready"]:
            assert dev["drafts"][b].tolist() == last["drafts"][b], (n, b)
            assert dev["picks"][b].tolist() == last["picks"][b], (n, b)
            assert int(dev["match"][b]) == last["match"][b], (n, b)
            assert int(dev["accepted"][b]) == last["match"][b] + 1, (n, b)
            assert int(dev["index"][b]) == step["positions"][b] and int(dev["position"][b]) == step["written"][b], (n, b)
            assert torch.equal(dev["hidden"][b], last["hidden"][b]), (n, b)
            counts.add(last["match"][b] + 1)
        assert int(dev["accepted"][3]) == 0
    assert counts == {1, 2, 3, 4}, counts
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            got, want = dev_engine.gdn_state(i), host_engine.gdn_state(i)
            for key in got:
                assert torch.equal(got[key][:3], want[key][:3]), (i, key)
            for key in ("recurrent_state", "conv_state"):
                assert torch.equal(got[key][3].cpu(), start_states[i][key][3]), (i, key)
        else:
            for a, bb in zip(dev_engine.get_kv(i), host_engine.get_kv(i)):
                assert torch.equal(a[:3], bb[:3]), i
    for a, bb in zip(dev_engine.get_kv(dev_engine.mtp_layer), host_engine.get_kv(host_engine.mtp_layer)):
        assert torch.equal(a[:3], bb[:3])


@pytest.mark.gpu
def test_every_pick_draft_and_accepted_count_is_the_oracles_decision(spec_run):
    """Each step's MTP calls, verify layers, head calls and acceptance against the oracle (tests/spec_check.py): the
    continuous stages equal the oracle's up to proven rounding ties, and every discrete decision is the oracle's on the
    GPU's own numbers, or a proven near-tie."""
    cfg, values, _, host_engine, _, rec, steps = spec_run
    weights = OracleWeights(cfg, values)
    log = lambda m: print(m, flush=True)
    differ = rows = 0
    for n, step in enumerate(steps):
        log(f"step {n}")
        worst = prove_step(host_engine, weights, rec, step["last"], first_head=n * K, first_mtp=n * (K - 1), verify_call=n, log=log)
        differ, rows = differ + worst["head"]["differ"], rows + worst["head"]["rows"]
        log(f"step {n}: worst {{{', '.join(f'{key}: {v:.3g}' for key, v in worst.items() if key != 'head')}}}, "
            f"head rows {worst['head']['rows']}, picks differing (near-ties) {worst['head']['differ']}")
    log(f"head picks differing from the oracle's on the same hidden rows: {differ} of {rows}, each a proven near-tie")


@pytest.mark.gpu
def test_unforced_drift_from_the_all_cpu_oracle_is_reported(spec_run):
    """The all-CPU oracle over each recorded verify call, from the call's starting state and inputs: the per-token
    distance of its hidden states from the device's and whether its picks (the oracle head on its own hidden states)
    are the device's. A measurement: the per-stage proofs above are the parity bound."""
    cfg, values, _, host_engine, _, rec, steps = spec_run
    weights = OracleWeights(cfg, values)
    head = weights.head()
    same = total = 0
    for n, step in enumerate(steps):
        call = rec.verify_calls[n]
        with torch.no_grad():
            hidden = oracle_chain(host_engine, weights, call)
        ready = step["ready"]
        err = rel_rows(call["out"][ready], hidden[ready], cfg.hidden_size)
        rows = hidden[ready].reshape(-1, 1, cfg.hidden_size)
        maxima = torch.stack([g.amax(dim=-1) for g in head_logits(cfg, head, rows).split(32, dim=-1)], dim=-1)
        picks = om.chip_next_tokens(cfg, head.norm_weight, head.lm_head, rows, maxima, 4, rows_bf16=head.rows)
        got = [t for b in ready for t in step["last"]["picks"][b]]
        same += sum(int(a == c) for a, c in zip(picks, got))
        total += len(got)
        print(f"step {n}: un-forced hidden distance per token median {float(err.median()):.3g} max {float(err.max()):.3g}; "
              f"picks equal {sum(int(a == c) for a, c in zip(picks, got))}/{len(got)}", flush=True)
    print(f"un-forced picks equal to the device's: {same}/{total}", flush=True)


@pytest.mark.gpu
def test_graph_replays_of_the_step_equal_its_launches(spec):
    """`q38_spec_step_graph` (the step captured once per gated-delta parity, then replayed) against `q38_spec_step`
    on a second engine from the same state: after every one of five steps, with eager work and synchronisations between
    the replays, the drafts, picks, matches, accepted counts, positions, indices and verify hidden states are equal bit
    for bit, and so is every state buffer at the end."""
    cfg, values = spec
    eager_engine, _ = load_engine(cfg, values)
    graph_engine, _ = load_engine(cfg, values)
    start = spec_start(cfg)
    eager, graph = DeviceStep(eager_engine, start), DeviceStep(graph_engine, start)
    for n in range(SPEC["steps"]):
        print(f"step {n}", flush=True)
        eager()
        graph(graph=True)
        _ = torch.ones(1024, device="cuda").sum().item()  # eager work between replays
        for name in ("drafts", "picks", "match", "accepted", "position", "index", "hidden"):
            assert torch.equal(getattr(eager, name), getattr(graph, name)), (n, name)
        assert eager_engine.handle.parity == graph_engine.handle.parity
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            got, want = graph_engine.gdn_state(i), eager_engine.gdn_state(i)
            for key in got:
                assert torch.equal(got[key], want[key]), (i, key)
        else:
            for a, b in zip(graph_engine.get_kv(i), eager_engine.get_kv(i)):
                assert torch.equal(a, b), i


@pytest.mark.gpu
def test_step_errors_are_recorded_on_the_device_and_raised_as_the_references(spec):
    """A row whose tokens would pass the last usable position, and a head row with no finite logit, are recorded in
    the device's status word and raised as the reference raises them on the host (ValueError, FloatingPointError);
    a clean step leaves the word at zero."""
    cfg, values = spec
    engine, _ = load_engine(cfg, values)
    device = DeviceStep(engine, spec_start(cfg))
    device()
    assert engine.handle.step_status() == 0
    device.position[0] = S - K  # position + K > max_seq_len - 1 for an active row
    device()
    with pytest.raises(ValueError, match="max_seq_len"):
        engine.handle.raise_step_errors()
    assert engine.handle.step_status() == 0  # cleared by the read
    hidden = torch.full((4, 1, cfg.hidden_size), float("nan"), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(FloatingPointError):
        HeadGraph(engine).pick(hidden, 4)
    with pytest.raises(FloatingPointError):
        engine.handle.raise_step_errors()
