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
