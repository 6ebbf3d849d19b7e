"""The head's exact recheck against lm_head's bf16 rows (`head.lm_head.rows`): the reference's ChipHead rechecks its
best groups against the checkpoint's bf16 lm_head (generate.py:196-206), while the group maxima come from its head
graph's lower-precision weights. With an lm_head that e4m3 cannot represent (random bf16 rows), the GPU's picks must
be the oracle's recheck over those bf16 rows (`om.chip_next_tokens` with ``rows_bf16``), except at a top-2 logit gap
under 1e-3; and the check must tell the two apart: rechecking against the e4m3 values instead picks differently on
some rows."""

from __future__ import annotations

import pytest
import torch

from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.quant import quantize_e4m3
from qwen38_amd.steps import Engine, HeadGraph


@pytest.mark.gpu
def test_recheck_reads_lm_heads_bf16_rows(gpu):
    cfg, b, k, s = tiny_config(1), 16, 4, 128
    rows = b * k
    g = torch.Generator().manual_seed(5)
    lm = (torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g) * 0.02).to(torch.bfloat16)
    coded, scales = quantize_e4m3(lm.float())
    norm_w = (torch.randn(cfg.hidden_size, generator=g) * 0.1).to(torch.bfloat16)
    engine = Engine(cfg, b, k, s, mtp=False)
    engine.load([("head.norm_weight", norm_w), ("head.lm_head", (coded, scales)), ("head.lm_head_rows", lm)])
    hidden = synth.hidden_states((rows, 1, cfg.hidden_size), 5, "head.x")
    got = HeadGraph(engine).pick(hidden.cuda(), 4).tolist()
    w8 = om.FP8Weight(coded, scales)
    maxima = om.head_group_maxima(cfg, norm_w, w8, hidden)
    want = om.chip_next_tokens(cfg, norm_w, w8, hidden, maxima, 4, rows_bf16=lm)
    from_e4m3 = om.chip_next_tokens(cfg, norm_w, w8, hidden, maxima, 4)
    norm = om.rms_norm(hidden.float(), norm_w, cfg.rms_norm_eps).squeeze(1)
    top = (norm @ lm.float().T).topk(2, dim=-1).values
    gaps = top[:, 0] - top[:, 1]
    differ = [r for r in range(rows) if got[r] != want[r]]
    print(f"picks differing from the bf16-row recheck: {differ}; e4m3 recheck differs on "
          f"{sum(a != c for a, c in zip(want, from_e4m3))} of {rows} rows", flush=True)
    assert all(float(gaps[r]) < 1e-3 for r in differ), [(r, float(gaps[r])) for r in differ]
    assert any(a != c for a, c in zip(want, from_e4m3)), "this lm_head does not tell the two rechecks apart"
