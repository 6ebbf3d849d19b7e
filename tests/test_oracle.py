"""Pin the CPU oracle: against golden vectors from the reference's own CPU path, and against invariants and closed
forms that a plausible mistake (a dropped term, a wrong index or sign, a transposed operand) breaks."""

from __future__ import annotations

import hashlib
import sys
import json
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config, with_layers
from qwen38_amd.generate import batch_step_inputs, mtp_prefill_inputs, mtp_step_inputs, prefill_inputs, verify_inputs
from qwen38_amd.quant import dequantize_e4m3, quantize_e4m3
from safetensors.torch import load_file
from scenario import GOLDEN, clone_states, golden_meta, golden_tensors, oracle_weights, tiny_states


def _digest(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


@pytest.fixture(scope="module")
def tiny():
    cfg = tiny_config(1)
    meta = golden_meta()
    values = dict((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    return cfg, meta, values


def test_synthetic_weights_are_the_ones_the_golden_vectors_were_made_with(tiny):
    cfg, meta, values = tiny
    for name, v in values.items():
        t = v if isinstance(v, torch.Tensor) else torch.cat([v[0].flatten(), v[1].flatten()])
        assert _digest(t) == meta["weights_sha256"][name], name


def test_oracle_verify_head_and_mtp_match_the_reference_bit_for_bit(tiny):
    cfg, meta, values = tiny
    gold = golden_tensors()
    layers, mtp_w, head_w = oracle_weights(values, cfg)
    states = tiny_states(cfg, meta, meta["seed"])
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    embed = values["embed_tokens"]
    ids = gold["ids"].long()
    active = torch.tensor(meta["active"]).float()

    in1 = verify_inputs(cfg, meta["positions_1"], k, s, torch.bfloat16, meta["active"], [0] * b)
    assert torch.equal(in1["cos"], gold["cos1"]) and torch.equal(in1["sin"], gold["sin1"])
    h1 = om.step_verify(cfg, layers, states, embed[ids[0]], in1["cos"], in1["sin"], in1["position"], in1["active"], in1["accepted"])
    assert torch.equal(h1, gold["hidden1"])
    in2 = verify_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"], meta["accepted_2"])
    h2 = om.step_verify(cfg, layers, states, embed[ids[1]], in2["cos"], in2["sin"], in2["position"], in2["active"], in2["accepted"])
    assert torch.equal(h2, gold["hidden2"])
    for i, (kind, st) in enumerate(zip(cfg.layer_types, states)):
        owner = "linear_attn" if kind == "linear_attention" else "self_attn"
        for key, value in st.items():
            assert _digest(value) == meta["state_sha256"][f"layers.{i}.{owner}.{key}"], (i, key)

    rows = h2.reshape(b * k, 1, -1)
    maxima = om.head_group_maxima(cfg, head_w["norm_weight"], head_w["lm_head"], rows)
    assert torch.equal(maxima, gold["maxima"])
    assert om.chip_next_tokens(cfg, head_w["norm_weight"], head_w["lm_head"], rows, maxima) == gold["picks4"].tolist()
    assert om.chip_next_tokens(cfg, head_w["norm_weight"], head_w["lm_head"], rows, maxima, 1) == gold["picks1"].tolist()

    mst = synth.kv_states(cfg, b, s, meta["context"], meta["seed"], "mtp")
    picks = gold["picks4"].long().reshape(b, k)
    mi = mtp_step_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"])
    out = om.mtp_forward(cfg, mtp_w, mst, h2, embed[picks], mi["cos"], mi["sin"], mi["position"], mi["active"])
    assert torch.equal(out, gold["mtp_out"])
    for key, value in mst.items():
        assert _digest(value) == meta["mtp_state_sha256"][f"layer.self_attn.{key}"], key


# ------------------------------------------------------------------------------------------- invariants


def _float32_tiny(num_layers_types, seed=3):
    cfg = with_layers(tiny_config(1), num_layers_types)
    values = dict((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg, mtp=False, head=False), seed))
    layers, _, _ = oracle_weights(values, cfg)
    for w in layers:
        for key, v in list(w.items()):
            if isinstance(v, torch.Tensor):
                w[key] = v.float()
    return cfg, layers


@pytest.mark.parametrize("kind", ["linear_attention", "full_attention"])
def test_verify_steps_equal_decoding_the_accepted_tokens_one_by_one(monkeypatch, kind):
    """Reference tests/test_prefill.py:235-263, on one layer of each kind in float32: after steps that commit
    2, 4, 1, 3, 1 of the last step's tokens, every accepted position's output equals one-token decode."""
    monkeypatch.setattr(om, "ROUND_E5M2", False)
    cfg, layers = _float32_tiny((kind,))
    k, batch, s = 4, 2, 64
    g = torch.Generator().manual_seed(5)
    tokens = torch.randn(16, cfg.hidden_size, generator=g)

    def fresh():
        if kind == "linear_attention":
            st = synth.gdn_states(cfg, batch, k, 7, "x")
            return [{key: v.float() if key != "pending_input_state" and key != "conv_state" else v.float() for key, v in st.items()}]
        st = synth.kv_states(cfg, batch, s, [20, 0], 7, "x")
        return [{key: v.float() for key, v in st.items()}]

    plain = fresh()
    start = 20
    want = []
    for i in range(14):
        inputs = batch_step_inputs(cfg, [start + i, 0], s, torch.float32, [True, False])
        x = torch.stack([tokens[i], torch.zeros(cfg.hidden_size)]).reshape(2, 1, -1)
        want.append(om.step_decode(cfg, layers, plain, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"])[0, 0])

    spec = fresh()
    done, accepted = 0, 0
    for take in [2, 4, 1, 3, 1]:
        x = torch.zeros(2, k, cfg.hidden_size)
        x[0, :take] = tokens[done : done + take]
        x[0, take:] = tokens[15]
        inputs = verify_inputs(cfg, [start + done, 0], k, s, torch.float32, [True, False], [accepted, 0])
        out = om.step_verify(cfg, layers, spec, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"], inputs["accepted"])
        for j in range(take):
            assert torch.allclose(out[0, j], want[done + j], atol=1e-4, rtol=1e-4), (done, j, (out[0, j] - want[done + j]).abs().max())
        done, accepted = done + take, take


def test_gated_delta_verify_equals_the_textbook_recurrence_in_float64():
    """Reference tests/test_prefill.py:18-26's recurrence: S_t = e^{g_t} S_{t-1} + k_t d_t^T,
    d_t = b_t (v_t - S_{t-1}^T k_t e^{g_t}), o_t = S_t^T q_t, checked against the verify form's commit (pending
    snapshots from a previous step, any accepted count) and its in-step K x K solve."""
    torch.manual_seed(0)
    pairs, k, d = 3, 4, 16
    q = torch.nn.functional.normalize(torch.randn(pairs, 2 * k, d, dtype=torch.float64), dim=-1) / d**0.5
    key = torch.nn.functional.normalize(torch.randn(pairs, 2 * k, d, dtype=torch.float64), dim=-1)
    v = torch.randn(pairs, 2 * k, d, dtype=torch.float64)
    g = -torch.rand(pairs, 2 * k, dtype=torch.float64)
    beta = torch.rand(pairs, 2 * k, dtype=torch.float64)
    s0 = torch.randn(pairs, d, d, dtype=torch.float64)

    def textbook(state, first, n):
        outs, deltas = [], []
        for t in range(first, first + n):
            state_dec = state * g[:, t].exp().reshape(-1, 1, 1)
            delta = beta[:, t].unsqueeze(-1) * (v[:, t] - (state_dec * key[:, t].unsqueeze(-1)).sum(-2))
            state = state_dec + key[:, t].unsqueeze(-1) * delta.unsqueeze(-2)
            outs.append((state * q[:, t].unsqueeze(-1)).sum(-2))
            deltas.append(delta)
        if not outs:
            return state, None, None
        return state, torch.stack(outs, 1), torch.stack(deltas, 1)

    for accepted in range(k + 1):
        # Step A runs tokens 0..k-1 from s0; its snapshots are (key, delta, g). Step B commits `accepted` of them
        # and runs tokens `accepted`..`accepted+k-1` (the rejected ones re-sent).
        _, _, deltas_a = textbook(s0, 0, k)
        taken = [float(accepted > s) for s in range(k)]
        decays = [g[:, s] * taken[s] for s in range(k)]
        remaining = sum(decays)
        scale = remaining.exp()
        weighted = []
        for s in range(k):
            remaining = remaining - decays[s]
            weighted.append(key[:, s] * (remaining.exp() * taken[s]).unsqueeze(-1))
        committed, products = om.commit_and_read(
            s0.float(), scale.reshape(pairs, 1, 1).float(), torch.stack(weighted, 1).float(), deltas_a.float(),
            torch.cat((key[:, accepted : accepted + k], q[:, accepted : accepted + k]), 1).transpose(1, 2).float(),
        )
        committed, products = committed.double(), products.double()
        want_state, want_out, _ = textbook(s0, 0, accepted)
        assert torch.allclose(committed, want_state, atol=1e-5)
        # In-step solve of step B, written as gdn_verify runs it.
        gb, bb = g[:, accepted : accepted + k], beta[:, accepted : accepted + k]
        kb, qb, vb = key[:, accepted : accepted + k], q[:, accepted : accepted + k], v[:, accepted : accepted + k]
        key_state, query_state = products[:, :k], products[:, k:]
        cum = gb.cumsum(-1)
        ds, outs = [], []
        for t in range(k):
            delta = vb[:, t] - cum[:, t].exp().unsqueeze(-1) * key_state[:, t]
            for s in range(t):
                delta = delta - ((cum[:, t] - cum[:, s]).exp() * (kb[:, t] * kb[:, s]).sum(-1)).unsqueeze(-1) * ds[s]
            ds.append(delta * bb[:, t].unsqueeze(-1))
            out = cum[:, t].exp().unsqueeze(-1) * query_state[:, t]
            for s in range(t + 1):
                out = out + ((cum[:, t] - cum[:, s]).exp() * (qb[:, t] * kb[:, s]).sum(-1)).unsqueeze(-1) * ds[s]
            outs.append(out)
        _, want_b, want_db = textbook(want_state, accepted, k)
        assert torch.allclose(torch.stack(outs, 1), want_b, atol=1e-5)
        assert torch.allclose(torch.stack(ds, 1), want_db, atol=1e-5)


def test_verify_attention_equals_full_softmax_over_the_visible_keys(monkeypatch):
    """Each verify token attends to cached positions before `position` and to its own step's tokens up to itself:
    brute force in float64 over exactly those keys."""
    monkeypatch.setattr(om, "ROUND_E5M2", False)
    cfg, layers = _float32_tiny(("full_attention",))
    w = layers[0]
    k, batch, s = 4, 3, 48
    positions = [10, 0, 30]
    st = {key: v.float() for key, v in synth.kv_states(cfg, batch, s, [10, 0, 30], 9, "y").items()}
    cache_k, cache_v = st["k_cache"].clone(), st["v_cache"].clone()
    x = torch.randn(batch, k, cfg.hidden_size, generator=torch.Generator().manual_seed(2))
    inputs = verify_inputs(cfg, positions, k, s, torch.float32, [True] * batch, [0] * batch)
    query, key, value, gate = om._attention_project(cfg, w, x, inputs["cos"], inputs["sin"])
    got_o = om.attention_verify(cfg, w, st, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"])
    groups = cfg.num_key_value_groups
    out = torch.zeros(batch, k, cfg.num_attention_heads, cfg.head_dim, dtype=torch.float64)
    for b in range(batch):
        for h in range(cfg.num_attention_heads):
            kv = h // groups
            for t in range(k):
                keys = torch.cat((cache_k[b, kv, : positions[b]], key[b, kv, : t + 1])).double()
                vals = torch.cat((cache_v[b, kv, : positions[b]], value[b, kv, : t + 1])).double()
                p = torch.softmax(keys @ query[b, h, t].double() / math.sqrt(cfg.head_dim), 0)
                out[b, t, h] = p @ vals
    want = om.linear_fp8((out.reshape(batch, k, -1).float() * torch.sigmoid(gate)), w["self_attn.o_proj"])
    assert torch.allclose(got_o, want, atol=1e-4, rtol=1e-4)
    # Writes land at position..position+K-1 and nowhere else.
    for b in range(batch):
        assert torch.equal(st["k_cache"][b, :, positions[b] : positions[b] + k], key[b])
        assert torch.equal(st["k_cache"][b, :, : positions[b]], cache_k[b, :, : positions[b]])


def test_chip_head_picks_what_the_host_head_picks():
    """Reference tests/test_model_parity.py:280-309: group maxima plus the exact recheck pick the full argmax."""
    cfg = tiny_config(1)
    specs = [sp for sp in synth.head_specs(cfg) if sp.name != "embed_tokens"]
    values = dict((sp.name, v) for sp, v in synth.make_all(specs, 11))
    _, _, head = oracle_weights(values, cfg)
    hidden = torch.randn(24, 1, cfg.hidden_size, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    maxima = om.head_group_maxima(cfg, head["norm_weight"], head["lm_head"], hidden)
    got = om.chip_next_tokens(cfg, head["norm_weight"], head["lm_head"], hidden, maxima)
    want = om.host_next_tokens(cfg, head["norm_weight"], head["lm_head"], hidden)
    gaps = om.top2_gap(cfg, head["norm_weight"], head["lm_head"], hidden)
    assert all(g == w or gap < 1e-3 for g, w, gap in zip(got, want, gaps.tolist()))
    # Group maxima are the largest logits of their groups: their argmax group holds the argmax token (ties aside).
    assert sum(int(maxima[r].argmax()) == want[r] // 32 for r in range(24)) >= 22


def test_acceptance_is_the_longest_matching_draft_prefix():
    assert om.accept([5, 6, 7, 8], [5, 6, 9], 4) == (2, [5, 6, 7])
    assert om.accept([5, 6, 7, 8], [5, 6, 7], 4) == (3, [5, 6, 7, 8])
    assert om.accept([5, 6, 7, 8], [1, 6, 7], 4) == (0, [5])
    assert om.accept([5], [], 1) == (0, [5])


# ------------------------------------------------------------------------------------------- formats


def test_e4m3_bit_field_decode_equals_torchs_cast_for_every_byte():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float()
    got = om.e4m3_to_float(codes)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(got[~torch.isnan(got)], want[~torch.isnan(want)])


def test_quantizer_keeps_groups_in_range_and_dequantizes_exactly_in_bf16():
    w = torch.randn(64, 512, generator=torch.Generator().manual_seed(0)) * 0.02
    w[3, :32] = 0.0
    w[5, 64:96] *= 1e3
    coded, scales = quantize_e4m3(w)
    d = dequantize_e4m3(coded, scales)
    assert torch.equal(d, om.FP8Weight(coded, scales).dense())
    assert torch.equal(d.to(torch.bfloat16).float(), d)
    groups = (d.reshape(64, 16, 32).abs().amax(-1) / torch.pow(2.0, scales.float() - 127))
    nonzero = groups > 0
    assert (groups[nonzero] >= 256).all() and (groups[nonzero] <= 448).all()
    # Rounding error per element is at most half an e4m3 step (2**-4 relative for normals) or saturation.
    rel = ((d - w).abs() / w.abs().clamp_min(1e-30))[w.abs() > 1e-3]
    assert rel.max() <= 0.0625 + 1e-6 or ((d - w).abs().max() <= 64 * torch.pow(2.0, scales.float().max() - 127))


def test_e5m2_rounding_of_every_bf16_value_is_round_to_nearest_even():
    """The activation rounding the kernels must reproduce: e5m2 is bf16's sign and exponent range with 2 mantissa
    bits, so rounding a bf16 to it is round-half-even on the low 5 mantissa bits, with overflow to infinity only past
    the largest finite e5m2 (57344) after rounding, and subnormals below 2**-14."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    got = bits.to(torch.float8_e5m2).float()
    x = bits.double()
    finite = torch.isfinite(x)
    mag = x.abs()
    exponent = torch.floor(torch.log2(mag.clamp_min(2.0**-40))).clamp(min=-14)
    step = torch.pow(2.0, exponent - 2)
    q = mag / step
    r = torch.floor(q)
    frac = q - r
    up = (frac > 0.5) | ((frac == 0.5) & (torch.remainder(r, 2) == 1))
    want = torch.where(up, r + 1, r) * step * torch.sign(x)
    want = torch.where(want.abs() > 57344, torch.sign(x) * math.inf, want)
    sel = finite & (mag < 2.0**17)
    assert torch.equal(got[sel].double(), want[sel])


def test_oracle_prefill_matches_the_reference_bit_for_bit(tiny):
    """tests/golden/prefill_tiny.*: two prefill chunks of row 1 (a full one from position 0, then 40 real tokens of
    the next from position 64) and the MTP layer's prefill form, from the reference's own CPU path."""
    cfg, meta, values = tiny
    gold = load_file(GOLDEN / "prefill_tiny.safetensors")
    pmeta = json.loads((GOLDEN / "prefill_tiny.json").read_text())
    layers, mtp_w, _ = oracle_weights(values, cfg)
    states = tiny_states(cfg, meta, meta["seed"])
    s, chunk, slot = pmeta["max_seq_len"], pmeta["chunk"], pmeta["slot"]
    embed = values["embed_tokens"]
    ids = gold["ids"].long()
    for n, (start, n_valid) in enumerate(pmeta["chunks"]):
        chunk_ids = ids[start : start + chunk].clone()
        chunk_ids[n_valid:] = 0
        pi = prefill_inputs(cfg, slot, start, n_valid, chunk, torch.bfloat16)
        h = om.step_prefill(cfg, layers, states, embed[chunk_ids].reshape(1, chunk, -1), pi["cos"], pi["sin"], pi["slot"],
                            pi["start"], pi["n_valid"])
        assert torch.equal(h, gold[f"hidden_p{n + 1}"]), n
    for i, (kind, st) in enumerate(zip(cfg.layer_types, states)):
        owner = "linear_attn" if kind == "linear_attention" else "self_attn"
        for key in ("recurrent_state", "conv_state", "k_cache", "v_cache"):
            if key in st:
                assert _digest(st[key]) == pmeta["state_sha256"][f"layers.{i}.{owner}.{key}"], (i, key)

    mst = synth.kv_states(cfg, meta["batch"], s, meta["context"], meta["seed"], "mtp")
    mi = mtp_prefill_inputs(cfg, slot, 0, chunk, chunk, torch.bfloat16)
    x = om.mtp_prefill(cfg, mtp_w, mst, gold["hidden_p1"], embed[ids[1 : chunk + 1]].reshape(1, chunk, -1), mi["cos"], mi["sin"],
                       mi["slot"], mi["start"], mi["n_valid"])
    assert torch.equal(x, gold["mtp_x"])
    for key, value in mst.items():
        assert _digest(value) == pmeta["mtp_state_sha256"][f"layer.self_attn.{key}"], key


def test_unit_lower_inverse_is_the_inverse_and_the_chunked_rule_is_the_recurrence():
    """`unit_lower_inverse` against a dense inverse; `chunked_gated_delta` against the rule one token at a time in
    float64, with pieces of 64 and 128, strongly correlated keys, and padding tokens (no decay, no write) that leave
    the state alone (reference tests/test_prefill.py:18-71)."""
    g = torch.Generator().manual_seed(0)
    lower = torch.tril(torch.randn(3, 128, 128, generator=g, dtype=torch.float64) * 0.2, -1)
    dense = torch.linalg.inv(torch.eye(128, dtype=torch.float64) - lower)
    assert (om.unit_lower_inverse(lower) - dense).abs().max() < 1e-10

    def recurrent(query, key, value, log_decay, beta, state):
        outs = []
        for t in range(key.shape[1]):
            state = state * log_decay[:, t].exp().reshape(-1, 1, 1)
            delta = (value[:, t] - (state * key[:, t].unsqueeze(-1)).sum(-2)) * beta[:, t].unsqueeze(-1)
            state = state + key[:, t].unsqueeze(-1) * delta.unsqueeze(-2)
            outs.append((state * query[:, t].unsqueeze(-1)).sum(-2))
        return torch.stack(outs, dim=1), state

    heads, tokens, dim = 2, 256, 64
    shared = torch.randn(heads, 1, dim, generator=g)
    for mix in (1.0, 0.01):  # independent keys, then keys within 1% of a shared direction
        key = F.normalize((1 - mix) * shared + mix * torch.randn(heads, tokens, dim, generator=g), dim=-1)
        query = F.normalize(torch.randn(heads, tokens, dim, generator=g), dim=-1) / dim**0.5
        value = torch.randn(heads, tokens, dim, generator=g)
        log_decay, beta = -torch.rand(heads, tokens, generator=g) * 0.3, torch.rand(heads, tokens, generator=g)
        state = torch.randn(heads, dim, dim, generator=g) * 0.1
        want_out, want_state = recurrent(*(t.double() for t in (query, key, value, log_decay, beta, state)))
        for chunk in (64, 128):
            out, got_state = om.chunked_gated_delta(query, key, value, log_decay, beta, state, chunk)
            assert (out - want_out).abs().max() < 1e-4, (mix, chunk)
            assert (got_state - want_state).abs().max() < 1e-4, (mix, chunk)
        real = 200
        log_decay[:, real:], beta[:, real:] = 0, 0
        _, want_state = recurrent(*(t[:, :real].double() for t in (query, key, value, log_decay, beta)), state.double())
        _, got_state = om.chunked_gated_delta(query, key, value, log_decay, beta, state, 128)
        assert (got_state - want_state).abs().max() < 1e-4, mix


def test_blocked_attention_equals_full_softmax():
    """`blocked_attention` with blocks smaller than the positions against one softmax over every visible position."""
    g = torch.Generator().manual_seed(1)
    q = (torch.randn(2, 24, 32, generator=g) / 32**0.5).to(torch.bfloat16)
    k = torch.randn(2, 100, 32, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 100, 32, generator=g).to(torch.bfloat16)
    visible = torch.rand(24, 100, generator=g) < 0.6
    visible[:, 0] = True
    scores = (q.float() @ k.float().transpose(-1, -2)).masked_fill(~visible, float("-inf"))
    want = torch.softmax(scores, dim=-1) @ v.float()
    got = om.blocked_attention(q, k, v, visible, 32)
    assert (got - want).abs().max() < 3e-2 * want.abs().max()


def test_prefill_then_decode_equals_decoding_every_token(monkeypatch):
    """A row prefilled in two chunks (the second part padding) and then decoded gives, in float32 without the e5m2
    rounding, what feeding every token through decode gives: outputs at every real position and the final states
    (reference tests/test_prefill.py:143-166)."""
    monkeypatch.setattr(om, "ROUND_E5M2", False)
    cfg, layers = _float32_tiny(("linear_attention", "full_attention"))
    batch, s, chunk, slot = 2, 64, 16, 1
    g = torch.Generator().manual_seed(9)
    tokens = torch.randn(24, cfg.hidden_size, generator=g)

    def fresh():
        out = []
        for i, kind in enumerate(cfg.layer_types):
            if kind == "linear_attention":
                st = synth.gdn_states(cfg, batch, 1, 7, f"x{i}")
                out.append({"recurrent_state": st["recurrent_state"].float(), "conv_state": st["conv_state"].float()})
            else:
                st = synth.kv_states(cfg, batch, s, [0, 0], 7, f"x{i}")
                out.append({key: v.float() for key, v in st.items()})
        return out

    plain = fresh()
    want = []
    for t in range(24):
        inputs = batch_step_inputs(cfg, [0, t], s, torch.float32, [False, True])
        x = torch.stack([torch.zeros(cfg.hidden_size), tokens[t]]).reshape(2, 1, -1)
        want.append(om.step_decode(cfg, layers, plain, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"])[1, 0])

    pre = fresh()
    got = []
    for start, n_valid in ((0, 16), (16, 4)):
        x = torch.zeros(1, chunk, cfg.hidden_size)
        x[0, :n_valid] = tokens[start : start + n_valid]
        pi = prefill_inputs(cfg, slot, start, n_valid, chunk, torch.float32)
        h = om.step_prefill(cfg, layers, pre, x, pi["cos"], pi["sin"], pi["slot"], pi["start"], pi["n_valid"])
        got += list(h[0, :n_valid])
    for t in range(20, 24):
        inputs = batch_step_inputs(cfg, [0, t], s, torch.float32, [False, True])
        x = torch.stack([torch.zeros(cfg.hidden_size), tokens[t]]).reshape(2, 1, -1)
        got.append(om.step_decode(cfg, layers, pre, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"])[1, 0])
    for t in range(24):
        assert torch.allclose(got[t], want[t], atol=2e-4, rtol=2e-4), (t, (got[t] - want[t]).abs().max())
    for i, kind in enumerate(cfg.layer_types):
        keys = ("recurrent_state", "conv_state") if kind == "linear_attention" else ("k_cache", "v_cache")
        for key in keys:
            a, b = pre[i][key][slot], plain[i][key][slot]
            if key.endswith("cache"):
                a, b = a[:, :24], b[:, :24]
            assert torch.allclose(a, b, atol=2e-4, rtol=2e-4), (i, key)


def test_mxfp4_codec_matches_the_references_decode_kat_and_converts_exactly_to_e4m3():
    """The checkpoint's MXFP4 decode against the reference's own known-answer file (tests/golden/fp4_decode_kat,
    the reference's tests/golden/decode.safetensors: every byte value, scales as bf16 powers of two); quantization
    round trips every E2M1 value; the e4m3 form of the same weights dequantizes to the same values."""
    from safetensors.torch import load_file as load

    from qwen38_amd.quant import dequantize_e4m3, dequantize_mxfp4, mxfp4_to_e4m3, quantize_mxfp4

    kat = load(GOLDEN / "fp4_decode_kat.safetensors")
    mant, exp = torch.frexp(kat["weight_scale"].float())
    assert bool((mant == 0.5).all())
    scale_bytes = (exp - 1 + 127).to(torch.uint8)
    assert torch.equal(dequantize_mxfp4(kat["weight_packed"], scale_bytes).to(torch.bfloat16), kat["expected"])

    codes = torch.arange(256, dtype=torch.uint8).reshape(8, 32)  # every byte: both nibbles of every code
    scales = torch.tensor([[100 + r] for r in range(8)], dtype=torch.uint8)
    values = dequantize_mxfp4(codes, scales)
    packed, back = quantize_mxfp4(values)
    assert torch.equal(dequantize_mxfp4(packed, back), values)
    coded, s8 = mxfp4_to_e4m3(codes, scales)
    assert torch.equal(dequantize_e4m3(coded, s8), values)


def bf16_spacing(x: torch.Tensor) -> torch.Tensor:
    """The distance between the two bf16 values around each of x (float64)."""
    return torch.pow(2.0, torch.floor(torch.log2(x.abs().clamp_min(2.0**-126))) - 7)


def test_fp4_planes_match_the_decode_kat_and_fp4_linear_sums_its_planes_apart():
    """`decode_planes` against the reference's FP4 decode known-answer file (its even and odd columns); `linear_fp4`
    (FP4Linear.forward, model.py:205-208): each plane's bf16 product within one bf16 spacing of its float64 sum (a
    plane with the other parity's inputs, a plausible slip, misses it by far), and the output the two planes' bf16 sum."""
    kat = load_file(GOLDEN / "fp4_decode_kat.safetensors")
    _, exp = torch.frexp(kat["weight_scale"].float())
    even, odd = om.decode_planes(kat["weight_packed"], (exp - 1 + 127).to(torch.uint8))
    assert torch.equal(even, kat["expected"][:, ::2]) and torch.equal(odd, kat["expected"][:, 1::2])
    assert not bool((even.view(torch.int16) == -32768).any())  # no negative zeros (sign-free codes)

    g = torch.Generator().manual_seed(7)
    n, k, rows = 64, 512, 16
    packed = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    scale_bytes = torch.randint(118, 128, (n, k // 32), generator=g, dtype=torch.uint8)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    even, odd = om.decode_planes(packed, scale_bytes)
    planes = [F.linear(x[:, p::2], w) for p, w in ((0, even), (1, odd))]
    for p, w in ((0, even), (1, odd)):
        exact = x[:, p::2].double() @ w.double().T
        assert bool(((planes[p].double() - exact).abs() <= bf16_spacing(exact)).all())
        wrong = x[:, 1 - p :: 2].double() @ w.double().T
        assert not bool(((wrong - exact).abs() <= bf16_spacing(exact)).all())
    assert torch.equal(om.linear_fp4(x, packed, scale_bytes), (planes[0].float() + planes[1].float()).to(torch.bfloat16))


def _kv8_layer():
    """The FP8 KV golden scenario's single attention layer: config, weights, oracle state (cache bytes + scales)."""
    import make_golden_kv8 as g8

    cfg = g8.layer_config()
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), g8.SEED))
    layers, _, _ = oracle_weights(values, cfg)
    ks, vs, kc, vc = g8.initial_cache(cfg)
    return g8, cfg, values, layers[0], {"k_cache": kc, "v_cache": vc, "k_scale": ks, "v_scale": vs}


def test_oracle_fp8_kv_cache_matches_the_reference_bit_for_bit():
    """tests/golden/kv8_tiny.*: one attention layer with an FP8 e4m3 cache and per-layer scales through two verify
    steps, a decode step and a prefill chunk, from the reference's own CPU path: hidden states and cache bytes."""
    sys.path.insert(0, str(GOLDEN))
    g8, cfg, values, w, st = _kv8_layer()
    gold = load_file(GOLDEN / "kv8_tiny.safetensors")
    meta = json.loads((GOLDEN / "kv8_tiny.json").read_text())
    verify_ids, decode_ids, prefill_ids, positions_2, decode_positions = g8.scenario(cfg)
    assert positions_2 == meta["positions_2"] and decode_positions == meta["decode_positions"]
    embed, b, k, s = values["embed_tokens"], meta["batch"], meta["tokens"], meta["max_seq_len"]
    kind = "full_attention"

    def check(name, h):
        assert torch.equal(h, gold[name]), name
        assert _digest(st["k_cache"]) == meta["cache_sha256"][name]["k_cache"], name
        assert _digest(st["v_cache"]) == meta["cache_sha256"][name]["v_cache"], name

    for n, (pos, acc) in enumerate(((meta["positions_1"], [0] * b), (positions_2, meta["accepted_2"]))):
        vi = verify_inputs(cfg, pos, k, s, torch.bfloat16, meta["active"], acc)
        h = om.decoder_layer(cfg, kind, w, st, embed[verify_ids[n]], vi["cos"], vi["sin"], vi["position"], vi["active"],
                             accepted=vi["accepted"])
        check(f"verify{n + 1}", h)
    di = batch_step_inputs(cfg, decode_positions, s, torch.bfloat16, meta["active"])
    h = om.decoder_layer(cfg, kind, w, st, embed[decode_ids].unsqueeze(1), di["cos"], di["sin"], di["position"], di["active"])
    check("decode", h)
    p = meta["prefill"]
    pi = prefill_inputs(cfg, p["slot"], p["start"], p["n_valid"], p["chunk"], torch.bfloat16)
    h = om.decoder_layer(cfg, kind, w, st, embed[prefill_ids].unsqueeze(0), pi["cos"], pi["sin"], None, None,
                         slot=pi["slot"], start=pi["start"], n_valid=pi["n_valid"])
    check("prefill", h)


def test_fp8_kv_round_trip_reencodes_to_the_same_bytes():
    """A cached value read back (bf16 of e4m3 x scale) encodes to the bytes it came from, for every bf16 value and
    several scales: so a kernel may keep only the read-back value of a step's own key or value and encode that into
    the cache. (The bf16 rounding moves a value by at most 2^-9 relative; e4m3's rounding boundaries are at least
    2^-5 relative away from its values.)"""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits[torch.isfinite(bits.float())]
    for scale in (0.0125, 0.0173, 0.5, 3.0, 1e-3):
        s = torch.tensor([scale], dtype=torch.bfloat16)
        coded = om.kv_store(x, s)
        back = om.kv_load(coded, s, torch.bfloat16)
        assert torch.equal(om.kv_store(back, s), coded), scale
        # and the codec is the bit-field definition: clamp to +-240, round to nearest even e4m3
        ref = om.e4m3_to_float(coded)
        want = (x.float() / s.float()).clamp(-240, 240)
        assert bool(((ref - want).abs() <= _e4m3_half_step(want) + 1e-30).all()), scale


def _e4m3_half_step(v: torch.Tensor) -> torch.Tensor:
    """Half the spacing of e4m3 values around |v| (subnormal spacing 2^-9)."""
    e = torch.floor(torch.log2(v.abs().clamp_min(2.0**-6)))
    return torch.pow(2.0, e - 3) / 2


def test_oracle_matches_the_reference_at_the_27b_widths_bit_for_bit():
    """tests/golden/slice_27b.*: two verify steps of one gated-delta and one attention layer (each with its MLP) at the
    27B widths (H 5120; 16 key heads repeated three-fold over 48 value heads; 24 query heads over 4 KV heads, six-fold
    GQA; SwiGLU 17408), B = 2, from the reference's own CPU path: the hidden states of both steps and every state buffer
    after the second, bit for bit. Pins the value-head repeat and the GQA grouping at their 27B factors, which the
    config 0 goldens (two-fold and four-fold) do not."""
    import sys

    sys.path.insert(0, str(GOLDEN))
    import make_golden_27b_slice as gs

    meta = json.loads((GOLDEN / "slice_27b.json").read_text())
    gold = load_file(GOLDEN / "slice_27b.safetensors")
    assert {k: meta[k] for k in gs.SLICE} == gs.SLICE
    cfg = gs.slice_config()
    assert (cfg.linear_key_repeat, cfg.num_attention_heads // cfg.num_key_value_heads) == (3, 6)
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg, mtp=False, head=False), gs.SLICE["seed"]))
    layers, _, _ = oracle_weights(values, cfg)
    states = gs.slice_states(cfg)
    x = gs.slice_inputs(cfg)
    b, k, s = gs.SLICE["batch"], gs.SLICE["tokens"], gs.SLICE["max_seq_len"]
    in1 = verify_inputs(cfg, gs.SLICE["context"], k, s, torch.bfloat16, [True] * b, [0] * b)
    assert torch.equal(in1["cos"], gold["cos1"]) and torch.equal(in1["sin"], gold["sin1"])
    h1 = om.step_verify(cfg, layers, states, x[0], in1["cos"], in1["sin"], in1["position"], in1["active"], in1["accepted"])
    assert torch.equal(h1, gold["hidden1"])
    in2 = verify_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, [True] * b, gs.SLICE["accepted_2"])
    h2 = om.step_verify(cfg, layers, states, x[1], in2["cos"], in2["sin"], in2["position"], in2["active"], in2["accepted"])
    assert torch.equal(h2, gold["hidden2"])
    for i, (kind, st) in enumerate(zip(cfg.layer_types, states)):
        owner = "linear_attn" if kind == "linear_attention" else "self_attn"
        for key, value in st.items():
            assert _digest(value) == meta["state_sha256"][f"layers.{i}.{owner}.{key}"], (i, key)
