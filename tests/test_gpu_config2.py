"""BASELINE config 2, the configuration bench.py times, on the GPU: the whole speculative step of the 64-layer 27B
model (48 gated-delta + 16 attention layers, H = 5120), the MTP layer (fc 10240 -> 5120) drafting 3 tokens per row,
the 248,320-token head (256 verify rows with the top-4 recheck, 64 rows per draft with the one-group recheck) and
acceptance, at B = 64, K = 4, 512-token contexts, over two consecutive steps (the first commits nothing, the second
commits the first's accepted prefixes).

The head is steered (tests/scenario.py): two lm_head rows along one direction, so the model's picks and the MTP
drafts mostly land on those two tokens and every accepted count 1..4 occurs; with independent random rows a
random-init model accepts no draft.

* Plumbing, bit for bit: two device steps (`q38_spec_step` on one engine) equal the oracle's restated scheduler
  (pinned to the reference's own) driving this build's `VerifyStep`, `MTPStep` and `ChipHead` over `HeadGraph` on a
  second engine: drafts, picks, matches, accepted counts, positions, indices, verify hidden states, every state buffer.
* Every decision proven (tests/spec_check.py), on the recorded host-driven run: all 64 layers of both verify calls
  teacher-forced stage by stage (every differing rounding a tie, every layer output within 2e-2 per token, every
  committed state vector within 1e-2), the six MTP calls (fc, the attention layer, the output tail), the eight head
  calls (maxima within 1e-4 on every row, the 256-row head GEMM included; each pick the oracle's from the same hidden
  row or a proven near-tie) and acceptance (the oracle's on the GPU's picks and drafts, exactly).
* Measured, not bounded: the all-CPU oracle from the second step's starting state over the same inputs, its hidden
  states, logits and picks against the device's.

Weights are regenerated on the GPU per layer for the oracle, so the host holds one layer's weights at a time (plus the
head's).
"""

from __future__ import annotations

import os
import time

import pytest
import torch

from layerwise import rel_rows
from oracle import model as om
from oracle import scheduler as osch
from qwen38_amd import synth
from qwen38_amd.config import verify_configs
from qwen38_amd.generate import ChipHead
from qwen38_amd.steps import Engine
from scenario import steer_head
from spec_check import (DeviceStep, OracleWeights, Recorder, check_acceptance, check_head, check_mtp, check_verify, head_logits,
                        host_slots, oracle_chain, reordered_sums, run_host_step)

WORKLOAD = verify_configs()[2]
CFG, B, K, CTX, S = WORKLOAD.cfg, WORKLOAD.batch, WORKLOAD.tokens, WORKLOAD.context, WORKLOAD.max_seq_len
SEED, STEPS, CHUNK = 29, 2, 256
LAYER_GROUPS = 4  # each verify call's 64 layers are checked in four tests of 16
# The projections' MFMA (the engine's default unless Q38_TEST_MFMA names one: "bf16" or "fp8").
MFMA = {"projection_mfma": os.environ["Q38_TEST_MFMA"]} if os.environ.get("Q38_TEST_MFMA") else {}


def log(msg: str) -> None:
    print(msg, flush=True)


def head_values() -> dict:
    """The head's weights as loaded: the final norm, the steered lm_head (e4m3 + E8M0) and the embeddings, on the GPU."""
    made = {s.name: synth.make(s, SEED, "cuda") for s in synth.head_specs(CFG)}
    return steer_head(made, CFG, SEED)


def weights(head: dict):
    for spec in synth.model_specs(CFG, mtp=True, head=True):
        yield spec.name, head[spec.name] if spec.name in head else synth.make(spec, SEED, "cuda")


def load_engine(head: dict) -> Engine:
    engine = Engine(CFG, B, K, S, mtp=True, **MFMA)
    engine.load(weights(head))
    for i, kind in enumerate(CFG.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, synth.gdn_states(CFG, B, K, SEED, f"c2.state.{i}", "cuda"))
        else:
            kv = synth.kv_states(CFG, B, S, [CTX] * B, SEED, f"c2.kv.{i}", "cuda")
            engine.set_kv(i, kv["k_cache"], kv["v_cache"])
    kv = synth.kv_states(CFG, B, S, [CTX - 1] * B, SEED, "c2.kv.mtp", "cuda")
    engine.set_kv(engine.mtp_layer, kv["k_cache"], kv["v_cache"])
    return engine


def start_rows() -> list:
    """Every row as a prefill of a CTX-token prompt leaves it: its first new token and the prompt's last hidden state."""
    g = torch.Generator().manual_seed(SEED)
    ids = torch.randint(0, CFG.vocab_size, (B,), generator=g).tolist()
    return [{"ids": [t], "prompt_len": CTX, "hidden": synth.hidden_states((1, CFG.hidden_size), SEED, f"c2.seed.{b}")}
            for b, t in enumerate(ids)]


@pytest.fixture(scope="module")
def run(gpu):
    started = time.time()
    head = head_values()
    dev_engine, host_engine = load_engine(head), load_engine(head)
    torch.cuda.synchronize()
    log(f"two 27B engines loaded in {time.time() - started:.0f}s")
    start = start_rows()
    device = DeviceStep(dev_engine, start)
    rec = Recorder(host_engine)
    sched = osch.Scheduler(None, None, ChipHead(None, CFG.rms_norm_eps, rec.head, B * K), CFG, B, S, CHUNK, verify=rec.verify,
                           verify_tokens=K, mtp=rec.mtp)
    slots = host_slots(start)
    steps = []
    for n in range(STEPS):
        device()
        positions, ready, _ = run_host_step(sched, slots)
        torch.cuda.synchronize()
        steps.append({"device": {name: getattr(device, name).clone() for name in
                                 ("drafts", "picks", "match", "accepted", "index", "position", "hidden")},
                      "last": dict(sched.last), "positions": positions, "ready": ready,
                      "written": [row.written if row else 0 for row in slots]})
        counts = sorted({m + 1 for m in sched.last["match"].values()})
        log(f"step {n} done at {time.time() - started:.0f}s: accepted counts {counts}")
    return {"dev": dev_engine, "host": host_engine, "rec": rec, "steps": steps,
            "weights": OracleWeights(CFG, seed=SEED, head=head)}


@pytest.mark.gpu
def test_config2_device_steps_equal_the_restated_scheduler(run):
    dev_engine, host_engine, steps = run["dev"], run["host"], run["steps"]
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
    log(f"accepted counts over both steps: {sorted(counts)}")
    assert counts == {1, 2, 3, 4}, counts
    for i, kind in enumerate(CFG.layer_types):
        if kind == "linear_attention":
            got, want = dev_engine.gdn_state(i), host_engine.gdn_state(i)
            for key in got:
                assert torch.equal(got[key], want[key]), (i, key)
        else:
            for a, bb in zip(dev_engine.kv_cache(i), host_engine.kv_cache(i)):
                assert torch.equal(a, bb), i
    for a, bb in zip(dev_engine.kv_cache(dev_engine.mtp_layer), host_engine.kv_cache(host_engine.mtp_layer)):
        assert torch.equal(a, bb)


@pytest.mark.gpu
@pytest.mark.parametrize("group", range(LAYER_GROUPS))
@pytest.mark.parametrize("step", range(STEPS))
def test_config2_verify_layers_match_the_oracle_teacher_forced(run, step, group):
    per = CFG.num_hidden_layers // LAYER_GROUPS
    layers = range(group * per, (group + 1) * per)
    started = time.time()
    worst = check_verify(run["host"], run["weights"], run["rec"].verify_calls[step], layers, log=log)
    log(f"step {step} layers {layers.start}-{layers.stop - 1} in {time.time() - started:.0f}s: worst "
        f"{{{', '.join(f'{k}: {v:.3g}' for k, v in worst.items())}}}")


@pytest.mark.gpu
def test_config2_mtp_calls_match_the_oracle(run):
    rec = run["rec"]
    assert len(rec.mtp_calls) == STEPS * (K - 1)
    for n, call in enumerate(rec.mtp_calls):
        worst = check_mtp(run["host"], run["weights"], call, log=log)
        log(f"MTP call {n}: worst {{{', '.join(f'{k}: {v:.3g}' for k, v in worst.items())}}}")


@pytest.mark.gpu
def test_config2_head_picks_drafts_and_acceptance_are_the_oracles(run):
    """The eight head calls (per step: three 64-row draft picks with one rechecked group, then the 256-row verify picks
    with four) and each step's acceptance."""
    rec, steps = run["rec"], run["steps"]
    head = run["weights"].head()
    assert len(rec.head_calls) == STEPS * K
    differ = rows = 0
    for n, call in enumerate(rec.head_calls):
        got = check_head(CFG, head, call, log)
        differ, rows = differ + got["differ"], rows + got["rows"]
        log(f"head call {n} ({got['rows']} rows, {call['groups']} groups): normed rows differing {got['norm_ties']} (ties), "
            f"maxima within {got['maxima_off']:.2g}, {got['differ']} picks differ (near-ties)")
    for step in steps:
        last = step["last"]
        for slot in last["picks"]:
            check_acceptance(last["picks"][slot], last["drafts"][slot], last["match"][slot], K)
    log(f"picks differing from the oracle's on the same hidden rows: {differ} of {rows}, each a proven near-tie")


@pytest.mark.gpu
def test_config2_unforced_drift_from_the_all_cpu_oracle_is_reported(run):
    """The all-CPU oracle over the second step's verify from that step's starting state and inputs (its own roundings
    through all 64 layers): the per-token distance of its hidden states and logits from the device's, and how many of
    its picks are the device's. Reported: the bound is the per-stage proof above."""
    host_engine, rec, steps = run["host"], run["rec"], run["steps"]
    weights = run["weights"]
    call = rec.verify_calls[STEPS - 1]
    started = time.time()
    with torch.no_grad():
        hidden = oracle_chain(host_engine, weights, call)
    gpu = call["out"].cpu()
    err = rel_rows(gpu, hidden, CFG.hidden_size)
    head = weights.head()
    rows_cpu, rows_gpu = hidden.reshape(-1, 1, CFG.hidden_size), gpu.reshape(-1, 1, CFG.hidden_size)
    logits_cpu, logits_gpu = head_logits(CFG, head, rows_cpu), head_logits(CFG, head, rows_gpu)
    lerr = rel_rows(logits_gpu, logits_cpu, CFG.vocab_size)
    maxima = torch.stack([g.amax(dim=-1) for g in logits_cpu.split(32, dim=-1)], dim=-1)
    picks = om.chip_next_tokens(CFG, head.norm_weight, head.lm_head, rows_cpu, maxima, 4, rows_bf16=head.rows)
    got = [t for b in range(B) for t in steps[STEPS - 1]["last"]["picks"][b]]
    same = sum(int(a == c) for a, c in zip(picks, got))
    top = logits_cpu.topk(2, dim=-1).values
    near = int(((top[:, 0] - top[:, 1]) < 1e-3).sum())
    log(f"un-forced 64-layer oracle ({time.time() - started:.0f}s): hidden distance per token median {float(err.median()):.3g} "
        f"max {float(err.max()):.3g}; logits median {float(lerr.median()):.3g} max {float(lerr.max()):.3g}; picks equal "
        f"{same}/{len(got)} ({near} rows with a top-2 gap under 1e-3)")
    run["unforced"] = (hidden, logits_cpu, picks)


@pytest.mark.gpu
def test_config2_control_two_cpu_evaluations_drift_alike(run):
    """The control for the drift above: a second CPU evaluation of the same 64-layer chain whose float32 sums run in
    another order (`reordered_sums`), against the first. Reported."""
    if "unforced" not in run:
        pytest.skip("needs the un-forced oracle run of the test before")
    hidden, logits_cpu, picks = run["unforced"]
    weights, head = run["weights"], run["weights"].head()
    call = run["rec"].verify_calls[STEPS - 1]
    started = time.time()
    with torch.no_grad(), reordered_sums():
        other = oracle_chain(run["host"], weights, call)
    rows_other = other.reshape(-1, 1, CFG.hidden_size)
    logits_other = head_logits(CFG, head, rows_other)
    maxima_other = torch.stack([g.amax(dim=-1) for g in logits_other.split(32, dim=-1)], dim=-1)
    picks_other = om.chip_next_tokens(CFG, head.norm_weight, head.lm_head, rows_other, maxima_other, 4, rows_bf16=head.rows)
    cerr, clerr = rel_rows(other, hidden, CFG.hidden_size), rel_rows(logits_other, logits_cpu, CFG.vocab_size)
    log(f"control ({time.time() - started:.0f}s), two CPU evaluations of the oracle differing only in float32 summation "
        f"order: hidden distance per token median {float(cerr.median()):.3g} max {float(cerr.max()):.3g}; logits median "
        f"{float(clerr.median()):.3g} max {float(clerr.max()):.3g}; picks equal "
        f"{sum(int(a == c) for a, c in zip(picks, picks_other))}/{len(picks)}")
