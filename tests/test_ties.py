"""The rounding-tie prover (tests/ties.py) on the CPU: its tail recomputation is the oracle's layer, it finds a tie
planted in the oracle's own computation, and it explains neither a generic error nor a flip at a value far from a
tie."""

from __future__ import annotations

import torch

import ties
from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config, with_layers
from qwen38_amd.generate import batch_step_inputs
from scenario import golden_meta, oracle_weights, tiny_states


def one_layer(kind: str):
    cfg = with_layers(tiny_config(1), (kind,))
    meta = golden_meta()
    values = dict((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    layers, _, _ = oracle_weights(values, cfg)
    states = tiny_states(cfg, meta, meta["seed"])
    x = synth.hidden_states((meta["batch"], 1, cfg.hidden_size), meta["seed"], "ties.x")
    inputs = batch_step_inputs(cfg, meta["positions_1"], meta["max_seq_len"], torch.bfloat16, meta["active"])
    with ties.Recorder() as rec:
        want = om.step_decode(cfg, layers, states, x, inputs["cos"], inputs["sin"], inputs["position"], inputs["active"])
    w = layers[0]
    o_in = rec.inputs[id(w.get("self_attn.o_proj", w.get("linear_attn.out_proj")))]
    return cfg, w, x.reshape(-1, cfg.hidden_size), o_in.reshape(x.shape[0], -1), want.reshape(-1, cfg.hidden_size)


def test_e5m2_ties_are_the_values_next_to_a_midpoint():
    # Between 1.0 and 1.25 (e5m2 neighbours) the midpoint is 1.125; bf16 steps there are 2^-7.
    vec = torch.tensor([1.125, 1.125 - 2**-7, 1.125 + 2**-7, 1.125 - 2**-6, 1.0, -1.125, 0.0], dtype=torch.bfloat16)
    idx, other = ties.e5m2_ties(vec)
    assert idx.tolist() == [0, 1, 2, 5]
    assert other[0] == 1.25 and other[1] == 1.25 and other[2] == 1.0 and other[5] == -1.25


def test_layer_tail_is_the_oracles_layer_and_a_planted_tie_is_found():
    for kind in ("full_attention", "linear_attention"):
        cfg, w, x, o_in, want = one_layer(kind)
        eps = cfg.rms_norm_eps
        for t in range(x.shape[0]):
            out, _ = ties.layer_tail(w, eps, x[t], o_in[t])
            assert ties.rel(out, want[t]) < 1e-2, (kind, t)  # the same arithmetic on one token (float32 sums aside)
        t = 1
        base, sites = ties.layer_tail(w, eps, x[t], o_in[t])
        for site in ("o", "mlp", "down"):
            idx, other = ties.e5m2_ties(sites[site])
            assert len(idx), (kind, site)
            # The candidate whose flip moves the token most: a "GPU" that rounded it the other way.
            moved = [(ties.rel(ties.layer_tail(w, eps, x[t], o_in[t], (site, j, float(other[j])))[0], base), j)
                     for j in idx.tolist()[:64]]
            _, j = max(moved)
            gpu, _ = ties.layer_tail(w, eps, x[t], o_in[t], (site, j, float(other[j])))
            assert ties.explain(w, eps, x[t], o_in[t], gpu) is not None, (kind, site)


def test_generic_errors_and_far_flips_are_not_explained():
    cfg, w, x, o_in, want = one_layer("full_attention")
    eps = cfg.rms_norm_eps
    t = 2
    base, sites = ties.layer_tail(w, eps, x[t], o_in[t])
    noisy = base.float() * (1 + 0.05 * torch.randn(base.shape, generator=torch.Generator().manual_seed(0)))
    assert ties.explain(w, eps, x[t], o_in[t], noisy.to(base.dtype)) is None
    # A flip of a value exactly on an e5m2 value (no tie): its other neighbour is a whole e5m2 step away.
    vec = sites["o"].flatten()
    exact = ((vec.float() == om.fp8_round(vec).float()) & (vec != 0)).nonzero().flatten()
    big = max(exact.tolist(), key=lambda j: abs(float(vec[j])))
    far = float(vec[big]) * 2  # two e5m2 steps away and more
    gpu, _ = ties.layer_tail(w, eps, x[t], o_in[t], ("o", big, far))
    assert ties.rel(gpu, base) > ties.TOL  # large enough to need explaining
    assert ties.explain(w, eps, x[t], o_in[t], gpu) is None


def test_swiglu_enumeration_finds_planted_ties_and_rejects_other_values():
    """`layerwise.swiglu_ties` (the down-projection input's exact tie enumeration): with a gate sum planted exactly on a
    bf16 rounding boundary, the e5m2 input computed from either rounding of it is explained, and so is every value the
    oracle's own SwiGLU gives; a value an e5m2 step or more from every candidate is not."""
    from layerwise import swiglu_ties

    g = torch.Generator().manual_seed(3)
    k = 256
    x = om.fp8_round(torch.randn(2, k, generator=g).to(torch.bfloat16))
    wg = quant_pair(torch.randn(4, k, generator=g) * 0.05)
    wu = quant_pair(torch.randn(4, k, generator=g) * 0.05)
    gate, up = om.FP8Weight(*wg), om.FP8Weight(*wu)
    rows, cols = torch.tensor([0, 0, 1, 1]), torch.tensor([0, 1, 2, 3])
    pre = om.silu(om.linear_fp8(x, gate)) * om.linear_fp8(x, up)
    own = om.fp8_round(pre).float()[rows, cols]
    assert bool(swiglu_ties(x, gate, up, rows, cols, own, 8.0).all())
    # Plant a tie: move one weight so that the gate sum of (0, 0) is a bf16 midpoint (exactly representable).
    exact = float((x[0].double() * gate.dense()[0].double()).sum())
    step = 2.0 ** (float(torch.floor(torch.log2(torch.tensor(abs(exact))))) - 7)
    midpoint = (float(torch.floor(torch.tensor(exact / step))) + 0.5) * step
    need = midpoint - exact
    j = int(x[0].abs().argmax())
    dense = gate.dense().clone()
    dense[0, j] += need / float(x[0, j])
    # The moved weight need not be e4m3; the enumeration only reads the dense values.
    planted = om.FP8Weight(gate.coded, gate.scales, dense.T.contiguous())
    total = float((x[0].double() * planted.dense()[0].double()).sum())
    for rounded in (torch.tensor(total - step / 4).to(torch.bfloat16), torch.tensor(total + step / 4).to(torch.bfloat16)):
        s = torch.sigmoid(rounded.float()).to(torch.bfloat16)
        act = (rounded.float() * s.float()).to(torch.bfloat16)
        u = om.linear_fp8(x[:1], up)[0, 0]
        h = om.fp8_round((act.float() * u.float()).to(torch.bfloat16))
        assert bool(swiglu_ties(x, planted, up, rows[:1], cols[:1], h.float().reshape(1), 8.0)[0])
    far = own.clone()
    far[0] = own[0] * 4 + torch.sign(own[0]) * 0.5
    assert not bool(swiglu_ties(x, gate, up, rows[:1], cols[:1], far[:1], 8.0)[0])


def quant_pair(w):
    from qwen38_amd.quant import quantize_e4m3

    return quantize_e4m3(w)
