"""The prefill form on the GPU against the CPU oracle (config 0 shapes, seed 0): chunks of 64 tokens of row 1, a full
one from position 0 (which restarts the row), then 40 real tokens of the next from position 64 (the rest padding),
as tests/golden/prefill_tiny.json has them; and the MTP layer's prefill form.

* One layer of each kind, each chunk started from the oracle's own state: the real tokens' outputs (padding tokens'
  are never read) within the north-star 2e-2, each token above it explained by one e5m2 rounding tie after its mixer
  (`ties.check_tokens`), row 1's states and the cache positions it writes within 1e-2, everything else bit for bit
  (the reference also writes junk at the other rows' last cache positions, which nothing reads; this build leaves
  them alone).
* The 4-layer graph on the same scenario, one layer at a time (teacher-forced): beside the graph runs a chain of
  one-layer engines, each fed the hidden states the GPU's layer before it produced, from the states the GPU left in
  it. The same kernels run the same inputs, so the chain's last output and every layer's states equal the graph's
  bit for bit; each layer's output is held as above, its states to 1e-2, against the oracle from that layer's GPU
  input and GPU state.
* The MTP prefill on the oracle's first-chunk hidden states: the cache positions written within 1e-2, the rest
  unchanged, and the fc output row the reference returns within 2e-2.
"""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import load_file

import layerwise
import ties
from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config, with_layers
from qwen38_amd.generate import mtp_prefill_inputs, prefill_inputs
from qwen38_amd.steps import Engine, MTPStep, StepGraph
from scenario import GOLDEN, clone_states, golden_meta, oracle_weights, row_rel, tiny_states


def prefill_meta():
    return json.loads((GOLDEN / "prefill_tiny.json").read_text()), load_file(GOLDEN / "prefill_tiny.safetensors")["ids"].long()


def rel_all(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu(), want.float().cpu()
    return float((got - want).norm() / want.norm().clamp_min(1e-30))


def oracle_layer(cfg, w: dict, st: dict, x, pi):
    """The oracle's one-layer prefill of chunk ``x``, with the out projection's input it rounded (for `ties`)."""
    with ties.Recorder() as rec:
        want = om.step_prefill(cfg, [w], [st], x, pi["cos"], pi["sin"], pi["slot"], pi["start"], pi["n_valid"])
    o_w = w.get("self_attn.o_proj", w.get("linear_attn.out_proj"))
    return want, rec.inputs[id(o_w)]


def check_layer(got, want, w: dict, cfg, x, o_in, n_valid: int) -> None:
    """The chunk's real tokens (padding tokens' outputs are never read) within 2e-2, or explained by a rounding tie."""
    h = cfg.hidden_size
    ties.check_tokens(got.reshape(-1, h)[:n_valid], want.reshape(-1, h)[:n_valid], w, cfg.rms_norm_eps,
                      x.reshape(-1, h)[:n_valid], o_in.reshape(want.reshape(-1, h).shape[0], -1)[:n_valid])


def set_states(engine, cfg, states):
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            engine.set_gdn(i, states[i])
        else:
            engine.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])


def chunk_embeds(values, ids, start, n_valid, chunk):
    chunk_ids = ids[start : start + chunk].clone()
    chunk_ids[n_valid:] = 0
    return values["embed_tokens"][chunk_ids].reshape(1, chunk, -1)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["linear_attention", "full_attention"])
def test_one_layer_prefills_like_the_oracle_chunk_by_chunk(gpu, kind):
    cfg = with_layers(tiny_config(1), (kind,))
    meta = golden_meta()
    pmeta, ids = prefill_meta()
    chunk, slot, s = pmeta["chunk"], pmeta["slot"], pmeta["max_seq_len"]
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    layers, _, _ = oracle_weights(values, cfg)
    engine = Engine(cfg, meta["batch"], meta["tokens"], s, mtp=False, prefill_chunk=chunk)
    engine.load((n, v) for n, v in values.items() if not n.startswith("mtp."))
    step = StepGraph(engine)
    states = tiny_states(cfg, meta, meta["seed"])
    for start, n_valid in pmeta["chunks"]:
        print(f"{kind} chunk at {start}, {n_valid} real tokens", flush=True)
        set_states(engine, cfg, states)  # this chunk starts from the oracle's state
        before = clone_states(states)
        x = chunk_embeds(values, ids, start, n_valid, chunk)
        pi = prefill_inputs(cfg, slot, start, n_valid, chunk, torch.bfloat16)
        got = step(inputs_embeds=x, **pi)
        torch.cuda.synchronize()
        want, o_in = oracle_layer(cfg, layers[0], states[0], x, pi)
        check_layer(got, want, layers[0], cfg, x, o_in, n_valid)
        others = [r for r in range(meta["batch"]) if r != slot]
        if kind == "linear_attention":
            mine = engine.gdn_state(0)
            for key in ("recurrent_state", "conv_state"):
                err = rel_all(mine[key][slot], states[0][key][slot])
                print(f"  {key} {err:.3g}", flush=True)
                assert err <= 1e-2, key
                assert torch.equal(mine[key][others].cpu(), before[0][key][others]), key
        else:
            kc, vc = engine.get_kv(0)
            for name, cache in (("k_cache", kc), ("v_cache", vc)):
                cache = cache.cpu()
                written = slice(start, start + chunk)
                assert row_rel(cache[slot, :, written].transpose(0, 1), states[0][name][slot, :, written].transpose(0, 1)) <= 1e-2, name
                keep = torch.ones(s, dtype=torch.bool)
                keep[written] = False
                assert torch.equal(cache[slot, :, keep], before[0][name][slot, :, keep]), name
                assert torch.equal(cache[others], before[0][name][others]), name


@pytest.mark.gpu
def test_two_prefill_chunks_layer_by_layer(gpu):
    cfg = tiny_config(1)
    meta = golden_meta()
    pmeta, ids = prefill_meta()
    chunk, slot, s = pmeta["chunk"], pmeta["slot"], pmeta["max_seq_len"]
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    layers, _, _ = oracle_weights(values, cfg)
    start_states = tiny_states(cfg, meta, meta["seed"])
    engine = Engine(cfg, meta["batch"], meta["tokens"], s, mtp=False, prefill_chunk=chunk)
    engine.load((n, v) for n, v in values.items() if not n.startswith("mtp."))
    set_states(engine, cfg, start_states)
    step = StepGraph(engine)
    chain = []
    for i, kind in enumerate(cfg.layer_types):
        one = with_layers(cfg, (kind,))
        e = Engine(one, meta["batch"], meta["tokens"], s, mtp=False, prefill_chunk=chunk)
        e.load(layerwise.layer_values(values, i).items())
        set_states(e, one, [start_states[i]])
        chain.append((e, StepGraph(e), one, kind, layers[i]))
    for n, (start, n_valid) in enumerate(pmeta["chunks"]):
        print(f"chunk {n + 1} at {start}, {n_valid} real tokens", flush=True)
        pi = prefill_inputs(cfg, slot, start, n_valid, chunk, torch.bfloat16)
        x = chunk_embeds(values, ids, start, n_valid, chunk)
        hidden = step(inputs_embeds=x, **pi)
        h = x
        for i, (e, st, one, kind, w) in enumerate(chain):
            before = layer_state(e, one, kind, 0)
            got = st(inputs_embeds=h, **pi)
            torch.cuda.synchronize()
            print(f"  layer {i} ({kind})", flush=True)
            want, o_in = oracle_layer(one, w, before, h.cpu(), pi)
            check_layer(got, want, w, one, h.cpu(), o_in, n_valid)
            mine = layer_state(e, one, kind, 0)
            for key, value in before.items():  # the oracle's state after the chunk
                if key in ("k_cache", "v_cache"):
                    written = slice(start, start + chunk)
                    err = row_rel(mine[key][slot, :, written].transpose(0, 1), value[slot, :, written].transpose(0, 1))
                else:
                    err = rel_all(mine[key][slot], value[slot])
                print(f"    {key} {err:.3g}", flush=True)
                assert err <= 1e-2, (i, key)
            h = got
        torch.cuda.synchronize()
        assert torch.equal(h.cpu(), hidden.cpu())  # the chain is the graph, layer by layer
        for i, (e, _, one, kind, _) in enumerate(chain):
            mine, full = layer_state(e, one, kind, 0), layer_state(engine, cfg, kind, i)
            for key in mine:
                assert torch.equal(mine[key], full[key]), (i, key)


def layer_state(engine: Engine, cfg, kind: str, i: int) -> dict:
    """Layer i's current state on the host, in the oracle's shapes."""
    if kind == "linear_attention":
        st = {key: v.cpu().clone() for key, v in engine.gdn_state(i).items()}
        st["pending_key_state"] = om.repeat_interleave(st["pending_key_state"], cfg.linear_key_repeat, dim=2).contiguous()
        return st
    kc, vc = engine.get_kv(i)
    return {"k_cache": kc.cpu(), "v_cache": vc.cpu()}


@pytest.mark.gpu
def test_mtp_prefill_writes_the_layers_cache_like_the_oracle(gpu):
    cfg = tiny_config(1)
    meta = golden_meta()
    pmeta, ids = prefill_meta()
    chunk, slot, s = pmeta["chunk"], pmeta["slot"], pmeta["max_seq_len"]
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    _, mtp_w, _ = oracle_weights(values, cfg)
    engine = Engine(cfg, meta["batch"], meta["tokens"], s, mtp=True, prefill_chunk=chunk)
    engine.load(values.items())
    mst = synth.kv_states(cfg, meta["batch"], s, meta["context"], meta["seed"], "mtp")
    engine.set_kv(engine.mtp_layer, mst["k_cache"], mst["v_cache"])
    before = {k: v.clone() for k, v in mst.items()}
    hidden = synth.hidden_states((1, chunk, cfg.hidden_size), meta["seed"], "prefill.hidden")
    embeds = values["embed_tokens"][ids[1 : chunk + 1]].reshape(1, chunk, -1)
    mi = mtp_prefill_inputs(cfg, slot, 0, chunk, chunk, torch.bfloat16)
    got = MTPStep(engine)(hidden=hidden, inputs_embeds=embeds, **mi)
    torch.cuda.synchronize()
    want = om.mtp_prefill(cfg, mtp_w, mst, hidden, embeds, mi["cos"], mi["sin"], mi["slot"], mi["start"], mi["n_valid"])
    assert row_rel(got[0], want[0]) <= 2e-2
    kc, vc = engine.get_kv(engine.mtp_layer)
    others = [r for r in range(meta["batch"]) if r != slot]
    for name, cache in (("k_cache", kc.cpu()), ("v_cache", vc.cpu())):
        assert row_rel(cache[slot, :, :chunk].transpose(0, 1), mst[name][slot, :, :chunk].transpose(0, 1)) <= 1e-2, name
        assert torch.equal(cache[slot, :, chunk:], before[name][slot, :, chunk:]), name
        assert torch.equal(cache[others], before[name][others]), name


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("heads", [8, 16])
def test_prefill_attention_over_several_tiles_and_blocks(gpu, heads, kv):
    """One attention layer, one chunk of 288 tokens (270 real) of row 1 from position 1601 of a 1984-position cache:
    three 128-token tiles (the last one partly live, part of it padding), the chunk's tokens 64 and on in the second
    2048-position block of [cache, chunk] (the reference's blocked softmax, model.py:760-781), so a block boundary cuts
    the chunk and some waves of a tile hold no token of a block; 8 and 16 query heads over 2 KV heads (4 and 8 query
    heads per KV head on an XCD). The real tokens within 2e-2 of the oracle or explained by a rounding tie
    (`ties.check_tokens`); the written cache positions within 1e-2 (bf16) or at most 1% of the bytes one e4m3 code
    apart (FP8, the oracle then forced onto the GPU's bytes for the chunk's own keys and values, as
    tests/test_gpu_kv8.py does); every other position unchanged."""
    from dataclasses import replace

    from qwen38_amd.quant import encode_kv

    cfg = replace(with_layers(tiny_config(1), ("full_attention",)), num_attention_heads=heads)
    rows, s, chunk, slot, start, n_valid, seed = 2, 1984, 288, 1, 1601, 270, 41
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg, mtp=False, head=False), seed))
    layers, _, _ = oracle_weights(values, cfg)
    w = layers[0]
    st = synth.kv_states(cfg, rows, s, [700, start], seed, "pf.kv")
    engine = Engine(cfg, rows, 4, s, mtp=False, prefill_chunk=chunk, kv_cache_format=kv)
    engine.load(values.items())
    if kv == "fp8":
        ks, vs = synth.kv_scales(cfg, seed, "pf.kv")
        st = {"k_cache": encode_kv(st["k_cache"], ks), "v_cache": encode_kv(st["v_cache"], vs), "k_scale": ks, "v_scale": vs}
        engine.set_kv_scales(0, ks, vs)
    engine.set_kv(0, st["k_cache"], st["v_cache"])
    before = {k: v.clone() for k, v in st.items()}
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, cfg.vocab_size, (chunk,), generator=g)
    ids[n_valid:] = 0
    x = synth.hidden_states((1, chunk, cfg.hidden_size), seed, "pf.x")
    pi = prefill_inputs(cfg, slot, start, n_valid, chunk, torch.bfloat16)
    got = StepGraph(engine)(inputs_embeds=x, **pi)
    torch.cuda.synchronize()
    kc, vc = (t.cpu() for t in engine.get_kv(0))
    written = slice(start, start + chunk)
    plain = om.kv_store
    oracle_bytes = None
    if kv == "fp8":
        # The oracle's own bytes for the chunk, from an unforced run on a copy of the cache.
        unforced = {k: v.clone() for k, v in st.items()}
        oracle_layer(cfg, w, unforced, x, pi)
        oracle_bytes = unforced
        own = (kc[slot, :, written], vc[slot, :, written])
        calls = []

        def forced(t, scale):
            calls.append(t)
            return own[(len(calls) - 1) % 2].reshape(t.shape)

        om.kv_store = forced
    try:
        want, o_in = oracle_layer(cfg, w, st, x, pi)
    finally:
        om.kv_store = plain
    check_layer(got, want, w, cfg, x, o_in, n_valid)
    keep = torch.ones(s, dtype=torch.bool)
    keep[written] = False
    for name, cache in (("k_cache", kc), ("v_cache", vc)):
        if kv == "fp8":
            want_bytes = oracle_bytes[name][slot, :, written]
            diff = cache[slot, :, written].int() != want_bytes.int()
            print(f"  {name}: {int(diff.sum())} of {diff.numel()} written bytes differ", flush=True)
            assert float(diff.float().mean()) <= 0.01, name
            assert bool((((cache[slot, :, written].int() - want_bytes.int()).abs() == 1))[diff].all()), name
        else:
            err = row_rel(cache[slot, :, written].transpose(0, 1), st[name][slot, :, written].transpose(0, 1))
            print(f"  {name}: written positions within {err:.3g}", flush=True)
            assert err <= 1e-2, name
        assert torch.equal(cache[slot, :, keep], before[name][slot, :, keep]), name
        assert torch.equal(cache[0], before[name][0]), name
