"""Pin the oracle's speculative scheduler (oracle/scheduler.py): bit for bit against the reference's own
`Scheduler._verify_step` / `_mtp_drafts` (tests/golden/spec_tiny.*), by the reference's speculation invariants
(tests/test_prefill.py:267-289, 380-448) and by a fake-device contract in the style of reference
tests/test_scheduler.py:13-80 that fixes every index of the draft loop by closed form."""

from __future__ import annotations

import hashlib
import json

import pytest
import torch

from oracle import model as om
from oracle import scheduler as osch
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from scenario import GOLDEN, SPEC, oracle_weights, spec_start, spec_states, steer_head


def _digest(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def build_oracle(cfg, values, states, mtp_kv, batch, tokens, dtype=torch.bfloat16):
    """The oracle's graphs over ``values``: step (verify/decode/prefill), MTP and the chip head for B*K rows."""
    layers, mtp_w, head_w = oracle_weights(values, cfg)
    step = osch.Step(cfg, layers, states)
    mtp = osch.MTP(cfg, mtp_w, mtp_kv)
    head = osch.ChipHead(cfg, head_w["norm_weight"], head_w["lm_head"], values["embed_tokens"].to(dtype), batch * tokens)
    return step, mtp, head


def spec_slots(cfg):
    slots = []
    for row in spec_start(cfg):
        if row is None:
            slots.append(None)
            continue
        r = osch.Row(0, list(row["ids"]), row["prompt_len"], written=row["prompt_len"])
        r.seed = (row["hidden"], [row["ids"][-1]], row["prompt_len"] - 1, 0)
        slots.append(r)
    return slots


def test_oracle_speculative_steps_match_the_references_scheduler_bit_for_bit():
    from safetensors.torch import load_file

    cfg = tiny_config(1)
    meta = json.loads((GOLDEN / "spec_tiny.json").read_text())
    gold = load_file(GOLDEN / "spec_tiny.safetensors")
    assert {k: meta[k] for k in SPEC} == SPEC
    b, k, s = SPEC["batch"], SPEC["tokens"], SPEC["max_seq_len"]
    values = steer_head(dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), SPEC["seed"])), cfg, SPEC["seed"])
    states, mtp_kv = spec_states(cfg)
    step, mtp, head = build_oracle(cfg, values, states, mtp_kv, b, k)
    sched = osch.Scheduler(None, None, head, cfg, b, s, SPEC["chunk"], verify=step, verify_tokens=k, mtp=mtp)
    slots = spec_slots(cfg)
    for slot, row in enumerate(slots):
        if row is not None:
            assert gold[f"start.ids.{slot}"].tolist() == row.ids
    accepted_counts = set()
    with torch.no_grad():
        for n in range(SPEC["steps"]):
            positions = [row.written if row else 0 for row in slots]
            active = [row is not None for row in slots]
            ready = [slot for slot, row in enumerate(slots) if row]
            assert positions == gold[f"step{n}.positions"].tolist()
            assert [sched.accepted[i] if slots[i] else 0 for i in range(b)] == gold[f"step{n}.accepted_in"].tolist()
            emitted = sched.verify_step(slots, positions, active, ready)
            for slot in ready:
                assert sched.last["drafts"][slot] == gold[f"step{n}.drafts"][slot].tolist(), (n, slot)
                assert slots[slot].seed[1] == gold[f"step{n}.picks"][slot].tolist(), (n, slot)
                assert slots[slot].seed[3] == int(gold[f"step{n}.match"][slot]), (n, slot)
                accepted_counts.add(slots[slot].seed[3] + 1)
            assert torch.equal(sched.last["hidden"], gold[f"step{n}.hidden"]), n
            for slot, tokens in zip(ready, emitted):
                slots[slot].ids += tokens
                slots[slot].written += len(tokens)
    assert accepted_counts == {1, 2, 3, 4}
    for i, st in enumerate(states):
        for key, value in st.items():
            assert _digest(value) == meta["state_sha256"][f"layers.{i}.{'linear_attn' if 'k_cache' not in st else 'self_attn'}.{key}"], (i, key)
    for key in ("k_cache", "v_cache"):
        assert _digest(mtp_kv[key]) == meta["state_sha256"][f"mtp.layer.self_attn.{key}"], key


def test_oracle_lookup_steps_match_the_references_scheduler_bit_for_bit():
    """The prompt-lookup branch of `Scheduler._verify_step` (scheduler.py:276-282, no MTP drafter): five steps of the
    restated scheduler over the oracle equal the reference's own (tests/golden/lookup_tiny.*, every accepted count 1..4
    among them): positions, committed counts, padded drafts, picks, matches, verify hidden states, final state digests."""
    from safetensors.torch import load_file

    from scenario import LOOKUP, lookup_start

    cfg = tiny_config(1)
    meta = json.loads((GOLDEN / "lookup_tiny.json").read_text())
    gold = load_file(GOLDEN / "lookup_tiny.safetensors")
    assert {k: meta[k] for k in LOOKUP} == LOOKUP
    b, k, s = LOOKUP["batch"], LOOKUP["tokens"], LOOKUP["max_seq_len"]
    values = steer_head(dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), LOOKUP["seed"])), cfg, LOOKUP["seed"])
    states, mtp_kv = spec_states(cfg, LOOKUP)
    step, _, head = build_oracle(cfg, values, states, mtp_kv, b, k)
    sched = osch.Scheduler(None, None, head, cfg, b, s, LOOKUP["chunk"], verify=step, verify_tokens=k)
    slots = []
    for slot, row in enumerate(lookup_start(cfg)):
        slots.append(None if row is None else osch.Row(0, list(row["ids"]), row["prompt_len"], written=row["prompt_len"]))
        if row is not None:
            assert gold[f"start.ids.{slot}"].tolist() == row["ids"]
    counts = set()
    with torch.no_grad():
        for n in range(LOOKUP["steps"]):
            positions = [row.written if row else 0 for row in slots]
            active = [row is not None for row in slots]
            ready = [slot for slot, row in enumerate(slots) if row]
            assert positions == gold[f"step{n}.positions"].tolist()
            assert [sched.accepted[i] if slots[i] else 0 for i in range(b)] == gold[f"step{n}.accepted_in"].tolist()
            emitted = sched.verify_step(slots, positions, active, ready)
            for slot, tokens in zip(ready, emitted):
                assert sched.last["drafts"][slot] == gold[f"step{n}.drafts"][slot].tolist(), (n, slot)
                assert sched.last["picks"][slot] == gold[f"step{n}.picks"][slot].tolist(), (n, slot)
                assert sched.last["match"][slot] == int(gold[f"step{n}.match"][slot]), (n, slot)
                counts.add(len(tokens))
                slots[slot].ids += tokens
                slots[slot].written += len(tokens)
            assert torch.equal(sched.last["hidden"], gold[f"step{n}.hidden"]), n
    assert counts == {1, 2, 3, 4} == set(meta["accepted_counts"])
    for i, st in enumerate(states):
        for key, value in st.items():
            assert _digest(value) == meta["state_sha256"][f"layers.{i}.{'linear_attn' if 'k_cache' not in st else 'self_attn'}.{key}"], (i, key)


def test_the_drafter_drafts_what_a_scan_of_the_history_drafts():
    """The reference's own check of its `Drafter` (tests/test_scheduler.py:177-185), on this build's
    `drafting.Drafter` against the oracle's restated scan and the build's own `lookup_draft`, over histories of 3 and 6
    symbols, with max_match 4 and 2; plus closed cases: nothing to match, a draft running into the history's end, the
    longest match winning over a later shorter one, and `padded_draft`'s padding."""
    from qwen38_amd import drafting

    for seed, symbols, max_match in ((0, 6, 4), (1, 3, 4), (2, 6, 2)):
        rng = torch.Generator().manual_seed(seed)
        history = torch.randint(0, symbols, (400,), generator=rng).tolist()
        drafter = drafting.Drafter(history[:50], max_match=max_match)
        for end in range(50, 400):
            want = osch.lookup_draft(history[:end], 3, max_match=max_match)
            assert drafter.draft(3) == want == drafting.lookup_draft(history[:end], 3, max_match=max_match), (seed, end)
            drafter.extend([history[end]])
    assert drafting.Drafter([1, 2, 3]).draft(3) == [] == osch.lookup_draft([1, 2, 3], 3)
    assert drafting.Drafter([5, 6, 7, 5]).draft(3) == [6, 7, 5]
    assert drafting.Drafter([5, 6, 5]).draft(3) == [6, 5]  # runs into the end of the history
    # [1, 2] occurred followed by 9; the later [2] alone was followed by 8: the longer match wins.
    assert drafting.Drafter([1, 2, 9, 2, 8, 1, 2]).draft(2) == [9, 2]
    assert drafting.padded_draft(drafting.Drafter([4, 4]), 4, 3) == [4, 4, 4]
    assert drafting.padded_draft(drafting.Drafter([1, 2, 3]), 3, 3) == [3, 3, 3]


def test_accepted_per_step_counts_what_each_lookup_step_emits():
    """`drafting.accepted_per_step` (reference drafting.py:54-74) against the restated verify loop driven by a fake
    model that emits ``output``: the same per-step counts, and they sum to the output's length."""
    from qwen38_amd import drafting

    rng = torch.Generator().manual_seed(5)
    for trial in range(20):
        history = torch.randint(0, 4, (30,), generator=rng).tolist()
        output = torch.randint(0, 4, (25,), generator=rng).tolist()
        steps, seen, done = [], list(history), 0
        while done < len(output):
            draft = osch.lookup_draft(seen, 3)
            match = 0
            while match < len(draft) and done + match < len(output) and draft[match] == output[done + match]:
                match += 1
            take = min(match + 1, len(output) - done)
            steps.append(take)
            seen += output[done : done + take]
            done += take
        got = drafting.accepted_per_step(history, output, 3)
        assert got == steps and sum(got) == len(output), trial


def test_input_builders_keep_the_references_bounds():
    cfg = tiny_config(1)
    with pytest.raises(ValueError):
        osch.verify_inputs(cfg, [124], 4, 128, torch.bfloat16, [True], [0])
    osch.verify_inputs(cfg, [123, 125], 4, 128, torch.bfloat16, [True, False], [0, 0])  # the last fit; inactive rows unchecked
    with pytest.raises(ValueError):
        osch.mtp_step_inputs(cfg, [124], 4, 128, torch.bfloat16, [True])
    with pytest.raises(ValueError):
        osch.batch_step_inputs(cfg, [127], 128, torch.bfloat16)
    with pytest.raises(ValueError):
        osch.prefill_inputs(cfg, 0, 0, 0, 16, torch.bfloat16)
    cos, _ = osch.rotary(cfg, torch.tensor([0, 5]), torch.float32)
    mi = osch.mtp_step_inputs(cfg, [4], 2, 128, torch.float32, [True])
    assert torch.equal(mi["cos"][0, 0], cos[1]) and int(mi["position"][0]) == 4  # cached at the index, rotated one on


# ----------------------------------------------------------------------------------------------- invariants


INV_CHUNK, INV_MAX_SEQ_LEN = 16, 64
INV_PROMPTS = [[3, 17, 42, 99, 5, 8, 120, 7, 64, 33, 2, 91, 14, 77, 50, 6, 23, 88, 1, 45, 12, 3, 17],
               [9, 9, 4, 1] * 5, [8, 120, 7, 64, 33, 2, 91, 14, 77, 50, 6, 23, 88, 1, 45, 12, 3, 3, 3]]


def float32_model(cfg, values, batch, tokens):
    """The oracle in float32, without the e5m2 input rounding (the reference's float32 tests run its bf16-weight
    linears), with fresh states for ``batch`` rows of ``tokens`` verify tokens."""
    fvalues = {n: (v.float() if isinstance(v, torch.Tensor) else v) for n, v in values.items()}
    states = []
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            st = synth.gdn_states(cfg, batch, max(tokens, 1), 0, f"inv.{i}")
            st = {key: torch.zeros_like(v, dtype=torch.float32) for key, v in st.items()}
        else:
            st = {key: torch.zeros(batch, cfg.num_key_value_heads, INV_MAX_SEQ_LEN, cfg.head_dim) for key in ("k_cache", "v_cache")}
        states.append(st)
    mtp_kv = {key: torch.zeros(batch, cfg.num_key_value_heads, INV_MAX_SEQ_LEN, cfg.head_dim) for key in ("k_cache", "v_cache")}
    layers, mtp_w, head_w = oracle_weights(fvalues, cfg)
    head = osch.HostHead(cfg, head_w["norm_weight"], head_w["lm_head"], fvalues["embed_tokens"], batch * max(tokens, 1))
    return osch.Step(cfg, layers, states), osch.MTP(cfg, mtp_w, mtp_kv), head, mtp_w


@pytest.fixture(scope="module")
def invariant_runs():
    """Plain greedy decoding and speculation with MTP drafts (K = 4) over the same prompts, two slots, float32."""
    cfg = tiny_config(1)
    values = steer_head(dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), 3)), cfg, 3)
    runs = {}
    old = om.ROUND_E5M2
    om.ROUND_E5M2 = False
    try:
        with torch.no_grad():
            for k in (1, 4):
                step, mtp, head, mtp_w = float32_model(cfg, values, 2, k)
                sched = osch.Scheduler(step, step, head, cfg, 2, INV_MAX_SEQ_LEN, INV_CHUNK, (), torch.float32,
                                       verify=step if k > 1 else None, verify_tokens=k, mtp=mtp if k > 1 else None)
                seen = []
                if k > 1:
                    real = sched.mtp_drafts

                    def recording(slots, real=real, sched=sched, seen=seen):
                        drafts = real(slots)
                        for slot, row in enumerate(slots):
                            if row is not None and row.seed is not None:
                                seen.append((row.index, row.seed[2] + row.seed[3], drafts[slot][0]))
                        return drafts

                    sched.mtp_drafts = recording
                out = [[] for _ in INV_PROMPTS]
                for index, token in sched.run(INV_PROMPTS, 12):
                    out[index].append(token)
                runs[k] = (out, sched.decode_calls, sched.drafted_tokens, seen)
    finally:
        om.ROUND_E5M2 = old
    return cfg, values, runs


def test_speculation_with_lookup_drafts_gives_the_tokens_plain_greedy_decoding_gives(invariant_runs):
    """The reference's invariant (tests/test_prefill.py:267-289) for the prompt-lookup branch: speculation with
    drafts from each row's history (K = 4, no MTP drafter) emits exactly plain greedy decoding's tokens, some drafts
    match, and it never takes more steps."""
    cfg, values, runs = invariant_runs
    old = om.ROUND_E5M2
    om.ROUND_E5M2 = False
    try:
        with torch.no_grad():
            step, _, head, _ = float32_model(cfg, values, 2, 4)
            sched = osch.Scheduler(step, step, head, cfg, 2, INV_MAX_SEQ_LEN, INV_CHUNK, (), torch.float32, verify=step,
                                   verify_tokens=4)
            out = [[] for _ in INV_PROMPTS]
            for index, token in sched.run(INV_PROMPTS, 12):
                out[index].append(token)
    finally:
        om.ROUND_E5M2 = old
    assert out == runs[1][0]
    assert sched.drafted_tokens > 0 and sched.decode_calls <= runs[1][1]


def test_speculation_with_mtp_drafts_gives_the_tokens_plain_greedy_decoding_gives(invariant_runs):
    _, _, runs = invariant_runs
    assert runs[4][0] == runs[1][0]
    # Drafts from the steered head match often; they must never cost steps.
    assert runs[4][2] > 0 and runs[4][1] < runs[1][1]


def test_each_steps_first_draft_is_the_mtp_layer_over_the_true_history(invariant_runs):
    """The reference's check (tests/test_prefill.py:422-448): the MTP layer run in steps of 4 over each finished
    sequence, from the main model's hidden states of a plain prefill, gives at each index the first draft the
    speculative run drafted there."""
    cfg, values, runs = invariant_runs
    plain_out = runs[1][0]
    old = om.ROUND_E5M2
    om.ROUND_E5M2 = False
    reference = {}
    try:
        with torch.no_grad():
            for p, prompt in enumerate(INV_PROMPTS):
                ids = prompt + plain_out[p]
                step, mtp, head, _ = float32_model(cfg, values, 1, 1)
                hidden = []
                for start in range(0, len(ids), INV_CHUNK):
                    chunk = ids[start : start + INV_CHUNK]
                    embeds = head.embed_batch(chunk + [0] * (INV_CHUNK - len(chunk)), torch.float32).reshape(1, INV_CHUNK, -1)
                    out = step(inputs_embeds=embeds, **osch.prefill_inputs(cfg, 0, start, len(chunk), INV_CHUNK, torch.float32))
                    hidden.append(out[0, : len(chunk)])
                hidden = torch.cat(hidden)
                _, mtp, _, _ = float32_model(cfg, values, 2, 4)
                picks = []
                for start in range(0, len(ids) - 1, 4):
                    n = min(4, len(ids) - 1 - start)

                    def pad(t, n=n):
                        return torch.stack((torch.cat((t, torch.zeros(4 - n, t.shape[-1]))), torch.zeros(4, t.shape[-1])))

                    embeds = head.embed_batch(ids[start + 1 : start + 1 + n], torch.float32)[:, 0]
                    y = mtp(hidden=pad(hidden[start : start + n]), inputs_embeds=pad(embeds),
                            **osch.mtp_step_inputs(cfg, [start, 0], 4, INV_MAX_SEQ_LEN, torch.float32, [True, False]))
                    picks += head.next_tokens(y[0, :n].unsqueeze(1))
                reference[p] = picks
    finally:
        om.ROUND_E5M2 = old
    checked = [(p, t, d, reference[p][t]) for p, t, d in runs[4][3] if t < len(reference[p])]
    assert len(checked) > 10 and all(d == r for _, _, d, r in checked), [c for c in checked if c[2] != c[3]][:5]


# ----------------------------------------------------------------------------------------------- fake-device contract


def next_token(history) -> int:
    """A deterministic stand-in for the model (as reference tests/test_scheduler.py:13-18): depends on every token so
    far and their order."""
    value = len(history)
    for token in history:
        value = (value * 31 + token) % 1009
    return value % 50


def draft_token(history) -> int:
    """The fake drafter: the model's choice, except after histories whose length is a multiple of 3."""
    token = next_token(history)
    return token if len(history) % 3 else (token + 1) % 50


class FakeDevice:
    """Per slot, the tokens in the main model's cache (by position) and in the MTP layer's cache (by MTP index, which
    holds the token one position on). Hidden rows carry (kind, slot, position) in their first three dims: kind 0 for
    the main model's hidden at a position, kind 1 for the MTP layer's output at an index. Every call checks the
    indices the scheduler passes against what the caches hold."""

    def __init__(self, cfg, batch, k, max_seq_len):
        self.cfg, self.k, self.max_seq_len = cfg, k, max_seq_len
        self.cache = [[] for _ in range(batch)]
        self.mtp_cache = [[] for _ in range(batch)]
        self.last_verify = [None] * batch

    def _hidden(self, shape, kind, slot, positions):
        h = torch.zeros(*shape, self.cfg.hidden_size)
        for i, p in enumerate(positions):
            h[i, :3] = torch.tensor([kind, slot, p], dtype=torch.float32)
        return h

    def prefill(self, inputs_embeds, cos, sin, slot, start, n_valid):
        slot, start, n_valid = int(slot[0]), int(start[0]), int(n_valid[0])
        assert len(self.cache[slot]) >= start or start == 0
        self.cache[slot] = self.cache[slot][:start] + [int(t) for t in inputs_embeds[0, :n_valid, 0]]
        chunk = inputs_embeds.shape[1]
        return self._hidden((chunk,), 0, slot, range(start, start + chunk)).unsqueeze(0)

    def verify(self, inputs_embeds, cos, sin, position, active, accepted):
        b, k = inputs_embeds.shape[:2]
        out = torch.zeros(b, k, self.cfg.hidden_size)
        for slot in range(b):
            if not active[slot]:
                continue
            p, a = int(position[slot]), int(accepted[slot])
            last = self.last_verify[slot]
            # The previous verify of this row wrote K tokens from its position; exactly `accepted` of them are kept,
            # so this step starts right after them (a prefill in between starts the row anew with accepted 0).
            if last is not None and a:
                assert p == last + a, (slot, p, last, a)
            assert len(self.cache[slot]) >= p
            self.cache[slot] = self.cache[slot][:p] + [int(t) for t in inputs_embeds[slot, :, 0]]
            out[slot] = self._hidden((k,), 0, slot, range(p, p + k))
            self.last_verify[slot] = p
        return out

    def mtp(self, hidden, inputs_embeds, cos, sin, position=None, active=None, slot=None, start=None, n_valid=None):
        if slot is not None:  # prefill form: index start + i takes hidden at start + i and the token one on
            s, first, n = int(slot[0]), int(start[0]), int(n_valid[0])
            for i in range(n):
                assert hidden[0, i, :3].tolist() == [0, s, first + i], (s, first, i)
            self.mtp_cache[s] = self.mtp_cache[s][:first] + [int(t) for t in inputs_embeds[0, :n, 0]]
            return hidden[:, :1]
        b, k = inputs_embeds.shape[:2]
        out = torch.zeros(b, k, self.cfg.hidden_size)
        for s in range(b):
            if not active[s]:
                continue
            index = int(position[s])
            kind, row, at = hidden[s, 0, :3].tolist()
            assert row == s and (kind, at) in ((0, index), (1, index - 1)), (s, index, hidden[s, 0, :3].tolist())
            assert len(self.mtp_cache[s]) >= index, (s, index, len(self.mtp_cache[s]))
            self.mtp_cache[s] = self.mtp_cache[s][:index] + [int(t) for t in inputs_embeds[s, :, 0]]
            out[s] = self._hidden((k,), 1, s, range(index, index + k))
        return out


class FakeHead:
    def __init__(self, device: FakeDevice):
        self.device = device

    def embed_batch(self, ids, dtype):
        out = torch.zeros(len(ids), 1, self.device.cfg.hidden_size, dtype=dtype)
        out[:, 0, 0] = torch.tensor(ids, dtype=dtype)
        return out

    def next_tokens(self, hidden, recheck_groups=None):
        out = []
        for kind, slot, p in hidden.reshape(-1, hidden.shape[-1])[:, :3].tolist():
            slot, p = int(slot), int(p)
            if kind == 0:  # the main model at position p: the token at p + 1
                out.append(next_token(self.device.cache[slot][: p + 1]))
            else:  # the MTP layer at index p: holds tokens up to position p + 1; drafts the token at p + 2
                out.append(draft_token(self.device.cache[slot][:1] + self.device.mtp_cache[slot][: p + 1]))
        return out


def alone(prompt, max_new_tokens, max_seq_len, chunk, k):
    ids, out = list(prompt), []
    while True:
        token = next_token(ids)
        out.append(token)
        ids.append(token)
        # The scheduler's stop (scheduler.py:195-197): the next step would write K positions from len(ids) - 1.
        if len(out) >= max_new_tokens or len(ids) - 1 + k > max_seq_len - chunk:
            return out


@pytest.mark.parametrize("batch", [1, 3])
def test_fake_device_speculation_accepts_exactly_the_drafts_that_agree(batch):
    cfg = tiny_config(1)
    k, max_seq_len, chunk = 4, 96, 8
    torch.manual_seed(0)
    prompts = [torch.randint(1, 50, (n,)).tolist() for n in (1, 7, 8, 9, 16, 17, 30, 3)]
    device = FakeDevice(cfg, batch, k, max_seq_len)
    head = FakeHead(device)
    sched = osch.Scheduler(None, device.prefill, head, cfg, batch, max_seq_len, chunk, (), torch.float32, verify=device.verify,
                           verify_tokens=k, mtp=device.mtp)
    want_drafted = 0
    real = sched.verify_step

    def counting(slots, positions, active, ready):
        nonlocal want_drafted
        # Closed form: a row's drafts are the fake drafter's continuation of its true tokens, each drafted from the
        # history including the drafts before it, and the leading ones equal to the model's own choices are kept.
        expect = {}
        for slot in ready:
            hist = list(slots[slot].ids)
            drafts = []
            for _ in range(k - 1):
                drafts.append(draft_token(hist))
                hist = hist + [drafts[-1]]
            expect[slot] = drafts
        emitted = real(slots, positions, active, ready)
        for slot, tokens in zip(ready, emitted):
            assert sched.last["drafts"][slot] == expect[slot], (slot, sched.last["drafts"][slot], expect[slot])
            hist, agree = list(slots[slot].ids), 0
            while agree < k - 1 and expect[slot][agree] == next_token(hist):
                hist.append(expect[slot][agree])
                agree += 1
            assert len(tokens) == agree + 1
            want_drafted += agree
        return emitted

    sched.verify_step = counting
    got = {i: [] for i in range(len(prompts))}
    for index, token in sched.run(prompts, max_new_tokens=12):
        got[index].append(token)
    assert got == {i: alone(p, 12, max_seq_len, chunk, k) for i, p in enumerate(prompts)}
    assert sched.drafted_tokens == want_drafted > 0
