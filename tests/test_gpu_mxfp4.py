"""MXFP4 weights read natively: the checkpoint's E2M1 nibbles and E8M0 scales packed into 1 KiB tiles and widened in
registers by the GEMM (v_cvt_scalef32_pk_bf16_fp4), against the e4m3 path on the same values.

Every E2M1 value times its E8M0 scale is an e4m3 value times the same scale (quant.mxfp4_to_e4m3, pinned on the CPU
against the reference's FP4 decode known-answer vectors), and both paths widen to the same bf16 operands before the
same MFMAs in the same order, so the bar is bit-for-bit equality: for the standalone projection at every token-tile
shape, and for a whole engine (verify, MTP, decode and prefill steps, every state) whose decoder layers are bound as
MXFP4. An fp32 product of the dequantized weights checks the nibble order independently of the e4m3 path.
"""

from __future__ import annotations

import pytest
import torch

from qwen38_amd import ext, synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import batch_step_inputs, mtp_step_inputs, prefill_inputs, verify_inputs
from qwen38_amd.quant import dequantize_mxfp4, mxfp4_to_e4m3, quantize_mxfp4, round_e5m2
from qwen38_amd.steps import Engine, MTPStep, StepGraph, VerifyStep
from scenario import golden_meta, golden_tensors, tiny_states


def same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.gpu
@pytest.mark.parametrize("rows,k,n", [(256, 5120, 1024), (64, 2048, 512), (3, 1024, 256), (300, 768, 512)])
def test_fp4_linear_matches_the_references_fp4_numerics(gpu, rows, k, n):
    """`q38_fp4_linear` (FP4Linear.forward, model.py:205-208: bf16 inputs, even and odd inputs through their weight
    planes apart, each product rounded to bf16, then added) against the oracle's `linear_fp4`: equal, except at an
    output where a plane's float64 sum lies within 2^-20 of its sum |x w| of a point halfway between two bf16 values
    (there the GPU's and torch's float32 sums, in different orders, may round to different neighbours); at most 1% of
    the outputs are such."""
    from oracle import model as om

    print(f"fp4 linear rows={rows} k={k} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows + k + n)
    w = torch.randn(n, k, generator=g) * 0.02
    w[:, 64:96] *= 1e-6  # a group whose scale is far below the others
    packed, scales = quantize_mxfp4(w)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    tiles, words = ext.pack_weight_fp4(packed.cuda(), scales.cuda())
    got = ext.fp4_linear(x.cuda(), tiles, words, n).cpu()
    again = ext.fp4_linear(x.cuda(), tiles, words, n).cpu()
    want = om.linear_fp4(x, packed, scales)
    assert same(got, again)
    differ = got != want
    print(f"  outputs differing from the oracle: {int(differ.sum())} of {differ.numel()}", flush=True)
    assert float(differ.float().mean()) <= 0.01
    if differ.any():
        even, odd = om.decode_planes(packed, scales)
        near = torch.zeros_like(differ)
        for p, wp in ((0, even), (1, odd)):
            xp, wd = x[:, p::2].double(), wp.double()
            exact, abs_sum = xp @ wd.T, xp.abs() @ wd.abs().T
            step = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0**-126))) - 7)
            mid = torch.floor(exact / step) * step + step / 2  # the halfway point inside exact's bf16 interval
            near |= (exact - mid).abs() <= 2.0**-20 * abs_sum
        assert bool(near[differ].all())


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [3, 64, 128, 256, 300])
def test_mxfp4_projection_equals_the_e4m3_projection_of_the_same_values(gpu, rows):
    print(f"mxfp4 linear rows={rows}", flush=True)
    g = torch.Generator().manual_seed(rows)
    n, k = 1024, 2048
    w = torch.randn(n, k, generator=g) * 0.02
    w[:, 64:96] *= 1e-6  # a group whose scale is far below the others
    packed, scales = quantize_mxfp4(w)
    coded, scales8 = mxfp4_to_e4m3(packed, scales)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    t4, s4 = ext.pack_weight_fp4(packed.cuda(), scales.cuda())
    t8, s8 = ext.pack_weight(coded.cuda(), scales8.cuda())
    assert t4.numel() * 2 == t8.numel()
    got = ext.mxfp4_linear(x.cuda(), t4, s4, n)
    ref = ext.fp8_linear(x.cuda(), t8, s8, n)
    torch.cuda.synchronize()
    assert same(got, ref)
    want = round_e5m2(x).float() @ dequantize_mxfp4(packed, scales).T
    err = float((got.cpu().float() - want).abs().max() / want.abs().max())
    assert err < 1e-2, err


@pytest.mark.gpu
def test_an_mxfp4_engine_steps_bit_for_bit_like_the_e4m3_engine(gpu):
    cfg = tiny_config(1)
    meta = golden_meta()
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), meta["seed"]))
    fp4 = dict(synth.to_mxfp4(values.items()))
    e4m3 = dict(synth.mxfp4_as_e4m3(fp4.items()))
    states = tiny_states(cfg, meta, meta["seed"])
    mkv = synth.kv_states(cfg, b, s, meta["context"], meta["seed"], "mtp")
    engines = []
    for fmt, weights in (("mxfp4", fp4), ("e4m3", e4m3)):
        e = Engine(cfg, b, k, s, mtp=True, prefill_chunk=64, weight_format=fmt)
        e.load(weights.items())
        for i, kind in enumerate(cfg.layer_types):
            if kind == "linear_attention":
                e.set_gdn(i, states[i])
            else:
                e.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])
        e.set_kv(e.mtp_layer, mkv["k_cache"], mkv["v_cache"])
        engines.append(e)
    f4, f8 = engines
    assert f4.buffer("mlp.gate_up.tiles", 0).numel() * 2 == f8.buffer("mlp.gate_up.tiles", 0).numel()
    assert same(f4.buffer("mtp.fc.tiles", f4.mtp_layer), f8.buffer("mtp.fc.tiles", f8.mtp_layer))

    embed = values["embed_tokens"]
    ids = golden_tensors()["ids"].long()

    def both(run):
        return [run(e) for e in engines]

    print("verify steps", flush=True)
    in1 = verify_inputs(cfg, meta["positions_1"], k, s, torch.bfloat16, meta["active"], [0] * b)
    out = both(lambda e: VerifyStep(e)(inputs_embeds=embed[ids[0]], **in1))
    assert same(*out)
    in2 = verify_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"], meta["accepted_2"])
    out = both(lambda e: VerifyStep(e)(inputs_embeds=embed[ids[1]], **in2))
    assert same(*out)
    print("mtp step", flush=True)
    mi = mtp_step_inputs(cfg, meta["positions_2"], k, s, torch.bfloat16, meta["active"])
    hidden = out[1]
    out = both(lambda e: MTPStep(e)(hidden=hidden, inputs_embeds=embed[ids[1]], **mi))
    assert same(*out)
    print("decode step", flush=True)
    di = batch_step_inputs(cfg, [p + k for p in meta["positions_2"]], s, torch.bfloat16, meta["active"])
    out = both(lambda e: StepGraph(e)(inputs_embeds=embed[ids[0][:, :1]], **di))
    assert same(*out)
    print("prefill chunk", flush=True)
    pi = prefill_inputs(cfg, 1, 0, 50, 64, torch.bfloat16)
    x = embed[torch.arange(64) * 7 % embed.shape[0]].unsqueeze(0)
    out = both(lambda e: StepGraph(e)(inputs_embeds=x, **pi))
    assert same(*out)
    torch.cuda.synchronize()
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            a, c = f4.gdn_state(i), f8.gdn_state(i)
            for key in a:
                assert same(a[key], c[key]), (i, key)
        else:
            for a, c in zip(f4.get_kv(i), f8.get_kv(i)):
                assert same(a, c), i
    for a, c in zip(f4.get_kv(f4.mtp_layer), f8.get_kv(f8.mtp_layer)):
        assert same(a, c)


@pytest.mark.gpu
def test_engines_loaded_from_an_mxfp4_checkpoint_agree_bit_for_bit(gpu, tmp_path):
    """A Hugging Face layout checkpoint (tests/test_checkpoint.py) read by qwen38_amd.checkpoint into an "mxfp4" engine
    (the checkpoint's bytes) and an "e4m3" engine (converted on the host): the same verify and MTP outputs."""
    from qwen38_amd import checkpoint as ckpt
    from test_checkpoint import fake_model

    cfg, _, _ = fake_model(tmp_path)
    meta = golden_meta()
    b, k, s = meta["batch"], meta["tokens"], meta["max_seq_len"]
    states = tiny_states(cfg, meta, meta["seed"])
    outs = []
    for fmt in ("mxfp4", "e4m3"):
        print(f"engine {fmt}", flush=True)
        e = Engine(cfg, b, k, s, mtp=True, weight_format=fmt)
        e.load(ckpt.model_weights(tmp_path, cfg, fmt))
        for i, kind in enumerate(cfg.layer_types):
            if kind == "linear_attention":
                e.set_gdn(i, states[i])
            else:
                e.set_kv(i, states[i]["k_cache"], states[i]["v_cache"])
        embed = e.buffer("embed_tokens", -1).view(cfg.vocab_size, cfg.hidden_size).cpu()
        ids = golden_tensors()["ids"].long()
        vi = verify_inputs(cfg, meta["positions_1"], k, s, torch.bfloat16, meta["active"], [0] * b)
        h = VerifyStep(e)(inputs_embeds=embed[ids[0]], **vi)
        mi = mtp_step_inputs(cfg, meta["positions_1"], k, s, torch.bfloat16, meta["active"])
        m = MTPStep(e)(hidden=h, inputs_embeds=embed[ids[1]], **mi)
        torch.cuda.synchronize()
        outs.append((h.clone(), m.clone()))
    assert same(outs[0][0], outs[1][0]) and same(outs[0][1], outs[1][1])
    assert torch.isfinite(outs[0][0].float()).all()
