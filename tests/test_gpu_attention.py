"""Full attention at long contexts, through the MTP step (one fc + full-attention layer + norm) against the oracle.

The golden scenario's contexts are short; these cases spread each (row, KV head) over many chunks (the tiny block at
2048 positions, with 4 tokens per row and with 1 as in decode), take the one-launch path with one and with two blocks
of 512 positions per wave, take the 64-query-row path (16 query heads over 2 KV heads, 8 tokens), run 512 (row, KV
head) pairs (each row's weights x V in one workgroup, at 32 and 64 query rows), run a cache whose length is not a
whole number of 64-position groups (contexts ending at its edge), and include an empty cache and
inactive rows (which write the cache tail), each with a bf16 cache and with an FP8 one (e4m3 bytes with the layer's
scales). Checked: the
MTP output (one layer, held to the north-star 2e-2 per row), the positions the step writes in
both caches (1e-2 on the values they read back: the keys are normed and rotated in bf16 by both sides), and every
other cache position unchanged.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.generate import mtp_step_inputs
from qwen38_amd.quant import decode_kv, encode_kv
from qwen38_amd.steps import Engine, MTPStep
from scenario import oracle_weights

CASES = {
    # name: (query heads, batch, tokens, max_seq_len, contexts, active)
    "tiny-2048-16chunks": (8, 4, 4, 2048, [1900, 700, 0, 1500], [True, True, True, False]),
    "64rows-1024": (16, 2, 8, 1024, [1000, 333], [True, True]),
    "tail-edge": (8, 2, 4, 512, [507, 511], [True, False]),
    # contexts between one and two blocks of 512 positions per wave (the one-launch path up to 1024)
    "fused-two-blocks": (8, 4, 4, 1024, [1019, 513, 767, 1000], [True, True, True, False]),
    # one token per row, as the decode step runs it, over many chunks
    "one-token-2048": (8, 4, 1, 2048, [2000, 1025, 0, 600], [True, True, True, False]),
    # a cache of 49 blocks of 32 positions (not whole groups of 64): the last group's second block lies past the
    # cache, rows' contexts end inside and at the edge of it
    "ragged-1568": (8, 4, 4, 1568, [1563, 1100, 1539, 1201], [True, True, True, False]),
    # 512 (row, KV head) pairs: the weights x V pass takes each row's positions in one workgroup, which then finishes
    # the row itself (fewer pairs split the positions and finish in a second kernel), with 32 and with 64 query rows
    "512-pairs-1536": (8, 256, 4, 1536, [1025 + (37 * r) % 507 for r in range(256)], [r % 17 != 5 for r in range(256)]),
    "512-pairs-64rows": (16, 256, 8, 1024, [513 + (29 * r) % 503 for r in range(256)], [r % 13 != 3 for r in range(256)]),
}


def row_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu(), want.float().cpu()
    worst = 0.0
    for r in range(want.shape[0]):
        n = float(want[r].norm())
        worst = max(worst, float((got[r] - want[r]).norm()) / max(n, 1e-30))
    return worst


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("case", list(CASES))
def test_mtp_attention_at_long_context_matches_the_oracle(gpu, case, kv):
    hq, b, k, s, context, active = CASES[case]
    print(f"case {case} kv {kv}", flush=True)
    cfg = dataclasses.replace(tiny_config(1), num_attention_heads=hq)
    seed = 11
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), seed))
    _, mtp_w, _ = oracle_weights(values, cfg)
    engine = Engine(cfg, b, k, s, mtp=True, kv_cache_format=kv)
    engine.load(values.items())
    mst = synth.kv_states(cfg, b, s, context, seed, "mtp")
    if kv == "fp8":
        ks, vs = synth.kv_scales(cfg, seed, "mtp")
        mst = {"k_cache": encode_kv(mst["k_cache"], ks), "v_cache": encode_kv(mst["v_cache"], vs), "k_scale": ks, "v_scale": vs}
        engine.set_kv_scales(engine.mtp_layer, ks, vs)
    engine.set_kv(engine.mtp_layer, mst["k_cache"], mst["v_cache"])
    before = {key: v.clone() for key, v in mst.items()}

    # Positions: each row's context (the step's own tokens go right after it; an inactive row's go to the tail).
    mi = mtp_step_inputs(cfg, context, k, s, torch.bfloat16, active)
    mi["position"] = torch.as_tensor(context, dtype=torch.int32)
    hidden = synth.hidden_states((b, k, cfg.hidden_size), seed, "attn.hidden")
    ids = torch.randint(0, cfg.vocab_size, (b, k), generator=torch.Generator().manual_seed(seed))
    embeds = values["embed_tokens"][ids]

    out = MTPStep(engine)(hidden=hidden, inputs_embeds=embeds, **mi)
    torch.cuda.synchronize()
    want = om.mtp_forward(cfg, mtp_w, mst, hidden, embeds, mi["cos"], mi["sin"], mi["position"], mi["active"])
    err = row_rel(out, want)
    print(f"mtp_out row_rel {err:.3g}", flush=True)
    assert err <= 2e-2

    # The step's own keys and values come from the fc and q/k/v projections of e5m2-rounded inputs, which the
    # un-forced oracle rounds on its own: a near-tie e5m2 input rounded the other way moves a row's keys and values by
    # about 0.8% each here (hidden 1024), and an FP8 cache rounds such a value a step further. Up to 64 rows every row
    # is held to 1e-2. Over 256 rows a few rows take such flips (measured: 3 of 256, the same rows in the keys and in
    # the values, which the attention kernels store as the projection made them, 1.7% and up to 3.3% with an FP8
    # cache; every other row bit for bit), so there the median row is held to 1e-2, at most 2% of the rows may exceed
    # it and none 5e-2 (a wrong token or position would). Every position the step does not write stays bit for bit.
    kc, vc = engine.get_kv(engine.mtp_layer)
    for name, got in (("k_cache", kc.cpu()), ("v_cache", vc.cpu())):
        read = (lambda t: decode_kv(t, mst[name[0] + "_scale"])) if kv == "fp8" else (lambda t: t)
        rels = []
        for row in range(b):
            start = context[row] if active[row] else s - k
            own = slice(start, start + k)
            rels.append(row_rel(read(got[row, :, own]).transpose(0, 1), read(mst[name][row, :, own]).transpose(0, 1)))
            keep = torch.ones(s, dtype=torch.bool)
            keep[own] = False
            assert torch.equal(got[row, :, keep], before[name][row, :, keep]), (name, row)
        worst = sorted(range(b), key=lambda r: -rels[r])[:3]
        med = float(torch.tensor(rels).median())
        print(f"{name} own writes: median row_rel {med:.3g}, worst rows {[(r, round(rels[r], 4)) for r in worst]}", flush=True)
        assert med <= 1e-2, name
        if b <= 64:
            assert max(rels) <= 1e-2, (name, worst[0])
        else:
            assert sum(r > 1e-2 for r in rels) <= 0.02 * b and max(rels) <= 5e-2, (name, worst)
