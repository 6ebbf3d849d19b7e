"""The loader (`qwen38_amd.runner`, the reference's runner.load / Loaded, qwen38_inf2/runner.py:21-90): its load-time
checks raise the reference's errors before anything touches the GPU, and on the GPU a loaded model's verify graph
and head give the same result as an engine built by hand."""

from __future__ import annotations

import pytest
import torch

from qwen38_amd import runner, synth
from qwen38_amd.config import tiny_config


def test_a_verify_graph_needs_a_head_for_rows_times_tokens():
    with pytest.raises(ValueError, match="a verify graph of 4 tokens for 8 rows needs a head for 32 rows"):
        runner.check_build(8, 4, None, 31, None)
    runner.check_build(8, 4, None, 32, None)
    runner.check_build(8, 0, None, 1, None)


def test_the_mtp_build_must_match_the_blocks():
    with pytest.raises(ValueError, match="the MTP build's rows, tokens and chunk"):
        runner.check_build(8, 4, 256, None, {"batch_size": 8, "mtp_tokens": 3, "chunk": 256})
    with pytest.raises(ValueError, match="don't match the blocks'"):
        runner.check_build(8, 4, 256, None, {"batch_size": 4, "mtp_tokens": 4, "chunk": 256})
    runner.check_build(8, 4, 256, None, {"batch_size": 8, "mtp_tokens": 4, "chunk": 256})


def test_load_refuses_before_building_an_engine():
    with pytest.raises(ValueError, match="needs a head for"):
        runner.load(cfg=tiny_config(1), weights=[], batch_size=4, verify_tokens=4, head_batch=8)


@pytest.mark.gpu
def test_loaded_verify_and_head_equal_a_hand_built_engine(gpu):
    from qwen38_amd.generate import verify_inputs
    from qwen38_amd.steps import Engine, HeadGraph, VerifyStep

    cfg, b, k, s = tiny_config(1), 4, 4, 128
    weights = lambda: ((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), 3))  # noqa: E731
    loaded = runner.load(cfg=cfg, weights=weights(), batch_size=b, max_seq_len=s, verify_tokens=k, mtp=True,
                         weight_format="e4m3", log=lambda m: None)
    assert (loaded.batch_size, loaded.verify_tokens, loaded.max_seq_len, loaded.chunk) == (b, k, s, None)
    assert loaded.verify is not None and loaded.mtp is not None and loaded.prefill is None
    assert loaded.head.batch_size == b * k
    engine = Engine(cfg, b, k, s, mtp=True)
    engine.load(weights())
    inputs = verify_inputs(cfg, [5, 9, 0, 17], k, s, torch.bfloat16, [True, True, False, True], [0] * b)
    x = (synth.hidden_states((b, k, cfg.hidden_size), 3, "x").float() * 0.02).to(torch.bfloat16)
    got = loaded.verify(x.cuda(), **{n: t.cuda() for n, t in inputs.items()})
    want = VerifyStep(engine)(x.cuda(), **{n: t.cuda() for n, t in inputs.items()})
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert loaded.head.next_tokens(got.reshape(b * k, 1, -1)) == HeadGraph(engine).pick(want.reshape(b * k, 1, -1), 4).tolist()
