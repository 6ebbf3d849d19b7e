"""FP8 projection kernel (packed e4m3 + E8M0 weights widened to bf16 in registers, bf16 MFMA, e5m2-rounded activation
tiles) against the CPU oracle's `linear_fp8` (reference FP8Linear.forward, qwen38_inf2/model.py:221-225)."""

from __future__ import annotations

import pytest
import torch

from oracle import model as om
from qwen38_amd import ext
from qwen38_amd.quant import dequantize_e4m3, quantize_e4m3, round_e5m2


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    mag = x.float().abs().clamp_min(2.0**-126)
    return torch.pow(2.0, torch.floor(torch.log2(mag)) - 7)


@pytest.mark.gpu
def test_activation_rounding_to_e5m2_matches_torch_for_every_bf16_value(gpu):
    """Identity weights (e4m3 1.0, scale 2^0) make the projection return its e5m2-rounded input: every finite bf16 value
    whose e5m2 rounding is finite, against torch's cast (the reference's fp8_round)."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.clone()
    bad = ~torch.isfinite(x.float()) | (x.float().abs() >= 61440)
    x[bad] = 0
    x = x.reshape(256, 256)
    coded = torch.zeros(256, 256, dtype=torch.uint8)
    coded[torch.arange(256), torch.arange(256)] = 0x38
    scales = torch.full((256, 8), 127, dtype=torch.uint8)
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    got = ext.fp8_linear(x.cuda(), tiles, words, 256).cpu()
    want = x.to(torch.float8_e5m2).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)) or torch.equal(got.float(), want.float())


@pytest.mark.gpu
def test_each_mx_block_is_scaled_by_its_own_e8m0_scale(gpu):
    """All-ones weights whose block b (of 32 inputs) has scale 2^b, against one-hot activations: the output for
    input k must be 2^(k // 32), so every input sits in the MX block whose scale the hardware applies to it."""
    n, k = 256, 256
    coded = torch.full((n, k), 0x38, dtype=torch.uint8)
    scales = (127 + torch.arange(k // 32)).to(torch.uint8).repeat(n, 1)
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    x = torch.eye(k, dtype=torch.bfloat16)
    got = ext.fp8_linear(x.cuda(), tiles, words, n).cpu().float()
    want = torch.pow(2.0, (torch.arange(k) // 32).float()).unsqueeze(1).expand(k, n)
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,k,n", [(16, 1024, 512), (64, 5120, 256), (128, 2048, 768), (256, 1024, 1024), (300, 512, 256)])
def test_fp8_linear_matches_the_oracle_within_rounding_and_accumulation_error(gpu, rows, k, n):
    print(f"fp8_linear rows={rows} k={k} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + k + n)
    w = torch.randn(n, k, generator=g) * 0.02
    w[:, :32] *= 50.0  # groups with different scales
    coded, scales = quantize_e4m3(w)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    want = om.linear_fp8(x, om.FP8Weight(coded, scales))
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    got = ext.fp8_linear(x.cuda(), tiles, words, n).cpu()
    # Error bound: bf16 rounding of the result plus float32 accumulation error (the bf16 MFMA's sums are float32-grade:
    # about 1e-8 of the sum of |x * w|, measured); the bound allows 2^-20. Outputs then differ from the CPU oracle only
    # where one of the two float32 sums lands across a bf16 rounding midpoint.
    xq, wd = round_e5m2(x).double(), dequantize_e4m3(coded, scales).double()
    exact = xq @ wd.T
    abs_sum = xq.abs() @ wd.abs().T
    err = (got.double() - exact).abs()
    assert (err <= 0.5 * bf16_ulp(exact) + 2.0**-20 * abs_sum).all(), float((err / abs_sum).max())
    assert (got.float() == want.float()).float().mean() > 0.999


@pytest.mark.gpu
def test_bf16_outputs_round_to_nearest_even_like_torch(gpu):
    """Only the first 64 inputs nonzero (one MFMA block: every split of the sum adds exact zeros, so the bf16 and
    float32 outputs come from the same float32 sums): the bf16 output must be torch's round-to-nearest-even of the
    float32 output. Products of e5m2 and e4m3 values have at most 7 significant bits, so many sums fall exactly halfway
    between two bf16 values and the ties are exercised."""
    g = torch.Generator().manual_seed(3)
    n, k, rows = 512, 256, 256
    coded, scales = quantize_e4m3(torch.randn(n, k, generator=g))
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    x[:, 64:] = 0
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    f32 = ext.fp8_linear_f32(x.cuda(), tiles, words, n).cpu()
    bf = ext.fp8_linear(x.cuda(), tiles, words, n).cpu()
    ties = (f32.view(torch.int32) & 0xFFFF) == 0x8000
    assert int(ties.sum()) > 100
    assert torch.equal(bf.view(torch.int16), f32.to(torch.bfloat16).view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("rows,k,n", [(256, 5120, 512), (64, 17408, 256), (256, 256, 256)])
def test_fp8_mfma_projection_sums_within_its_accumulation_bound(gpu, rows, k, n):
    """The projection on the scaled FP8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4 reading the e4m3 weight and e5m2
    activation tiles as they are, the weight's E8M0 bytes as the block scales): float32 outputs within 2^-14 of
    sum |x w| of the exact float64 sum (its measured internal accumulation is about 2^-15.5 of a 64-input block's
    sum |x w|), against the bf16 MFMA path's float32-grade sums on the same inputs; the bf16 outputs of the two paths equal except
    where the exact sum lies within that bound of a bf16 rounding boundary; and the same identity and one-hot checks as
    the bf16 path (every MX block scaled by its own scale)."""
    g = torch.Generator().manual_seed(rows + k)
    coded, scales = quantize_e4m3(torch.randn(n, k, generator=g) * 0.02)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    xq = round_e5m2(x).double()
    wd = dequantize_e4m3(coded, scales).double()
    exact, abs_sum = xq @ wd.T, xq.abs() @ wd.abs().T
    f8 = ext.fp8_linear_mfma(x.cuda(), tiles, words, n, "fp8", f32_out=True).cpu().double()
    bf = ext.fp8_linear_mfma(x.cuda(), tiles, words, n, "bf16", f32_out=True).cpu().double()
    e8, eb = float(((f8 - exact).abs() / abs_sum).max()), float(((bf - exact).abs() / abs_sum).max())
    print(f"rows {rows} k {k}: fp8 MFMA max err / sum|xw| {e8:.3g} (2^{torch.log2(torch.tensor(e8)):.1f}), bf16 MFMA {eb:.3g}")
    assert e8 <= 2.0**-14 and eb <= 2.0**-22
    o8 = ext.fp8_linear_mfma(x.cuda(), tiles, words, n, "fp8").cpu()
    ob = ext.fp8_linear_mfma(x.cuda(), tiles, words, n, "bf16").cpu()
    assert torch.equal(ob, ext.fp8_linear(x.cuda(), tiles, words, n).cpu())
    differ = o8 != ob
    if differ.any():
        ulp = bf16_ulp(exact[differ])
        lo = torch.floor(exact[differ] / ulp) * ulp  # the two bf16 neighbours of the exact sum (within a binade)
        boundary = torch.minimum((exact[differ] - lo - ulp / 2).abs(), (exact[differ] - lo + ulp / 2).abs())
        assert bool((boundary <= 2.0**-14 * abs_sum[differ]).all())
    print(f"  bf16 outputs differing between the MFMAs: {int(differ.sum())} of {differ.numel()}")


@pytest.mark.gpu
@pytest.mark.parametrize("mfma", ["bf16", "fp8"])
@pytest.mark.parametrize("rows,k,n", [(256, 5120, 16384), (256, 2048, 768), (128, 5120, 4096), (64, 17408, 5120), (32, 1024, 2560)])
def test_split_tiles_finished_by_recomputation_equal_the_l2_partials(gpu, rows, k, n, mfma):
    """The stream-K GEMM finishes a tile split between workgroups from their float32 partials in the XCD's L2; if the
    contributors ever ran on different XCDs it recomputes every contributor's partial itself. Forced on every split
    tile, that path gives the same bits as the partials (the same MFMAs from zero sums, added in the same order), at
    each workgroup tile shape (128 x 256 and 256 x 256 features x tokens at 256 rows, 512 x 128 at 128, 128 x 64 at 64,
    512 x 32 at 32) and on both MFMAs; two calls in a row leave the arrival counters at zero."""
    g = torch.Generator().manual_seed(rows + k + n)
    coded, scales = quantize_e4m3(torch.randn(n, k, generator=g) * 0.02)
    tiles, words = ext.pack_weight(coded.cuda(), scales.cuda())
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16).cuda()
    scratch = ext.linear_scratch(rows, k, x.device)
    plain = ext.fp8_linear_mfma(x, tiles, words, n, mfma, scratch=scratch)
    redo = ext.fp8_linear_mfma(x, tiles, words, n, mfma, scratch=scratch, recompute=True)
    again = ext.fp8_linear_mfma(x, tiles, words, n, mfma, scratch=scratch)
    torch.cuda.synchronize()
    assert torch.equal(plain.view(torch.int16), redo.view(torch.int16))
    assert torch.equal(plain.view(torch.int16), again.view(torch.int16))
