"""q38_fp8_linear_noalloc, the standalone FP8 projection whose scratch is the library's static device array: through
the C ABI it gives the same bits as q38_fp8_linear with a caller's scratch, on two calls in a row (the second with a
smaller input, so the array keeps the first call's contents), and refuses sizes beyond its array."""

from __future__ import annotations

import pytest
import torch

from qwen38_amd import ext
from qwen38_amd.quant import quantize_e4m3


def packed(n: int, k: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    coded, scales = quantize_e4m3(torch.randn(n, k, generator=g) * 0.02)
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    x = torch.randn(64, k, generator=g).to(torch.bfloat16).cuda()
    return tiles, words, x


@pytest.mark.gpu
def test_noalloc_projection_equals_the_scratch_argument_one_on_two_calls(gpu):
    for rows, k, n, seed in [(64, 5120, 16384, 1), (9, 1024, 768, 2)]:
        print(f"rows {rows} k {k} n {n}", flush=True)
        tiles, words, x = packed(n, k, seed)
        x = x[:rows].contiguous()
        want = ext.fp8_linear(x, tiles, words, n)
        got = ext.fp8_linear_noalloc(x, tiles, words, n)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (rows, k, n)


@pytest.mark.gpu
def test_noalloc_projection_refuses_sizes_beyond_its_array(gpu):
    tiles, words, x = packed(256, 1024, 3)
    with pytest.raises(RuntimeError, match="1 to 64 rows"):
        ext.fp8_linear_noalloc(torch.zeros(65, 1024, dtype=torch.bfloat16, device="cuda"), tiles, words, 256)
    with pytest.raises(RuntimeError, match="K <= 32768"):
        ext.fp8_linear_noalloc(torch.zeros(64, 33024, dtype=torch.bfloat16, device="cuda"), tiles, words, 256)


@pytest.mark.gpu
def test_noalloc_projection_captured_in_a_graph_replays_like_the_scratch_argument_one(gpu):
    """The callers this entry point is for capture it: two calls of different shapes captured into one
    torch.cuda.CUDAGraph (no allocation and no memset inside: its counters are cleared by a kernel), replayed twice
    with eager work between the replays, each replay's outputs equal to q38_fp8_linear's bit for bit."""
    calls = []
    for rows, k, n, seed in [(64, 5120, 16384, 4), (9, 1024, 768, 5)]:
        tiles, words, x = packed(n, k, seed)
        x = x[:rows].contiguous()
        calls.append((x, tiles, words, n, torch.empty(rows, n, dtype=torch.bfloat16, device="cuda"),
                      ext.fp8_linear(x, tiles, words, n)))
    for x, tiles, words, n, out, _ in calls:  # eager first calls: the array's address is resolved before capture
        ext.fp8_linear_noalloc(x, tiles, words, n, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for x, tiles, words, n, out, _ in calls:
            ext.fp8_linear_noalloc(x, tiles, words, n, out=out)
    for replay in range(2):
        for call in calls:
            call[4].zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _ = torch.ones(1024, device="cuda").sum().item()  # eager work between replays
        for x, tiles, words, n, out, want in calls:
            assert torch.equal(out.view(torch.int16), want.view(torch.int16)), (replay, x.shape[0], n)
