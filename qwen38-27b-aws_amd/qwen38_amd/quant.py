"""Weight formats of this build: FP8 e4m3 bytes with one E8M0 power-of-two scale per 32 input elements, and the
checkpoint's MXFP4 (E2M1 nibbles with the same E8M0 scales), which the GEMMs also read directly.

The reference stores FP8 e5m2 weights ``[in, out]`` with the FP4 checkpoint's scale folded in
(qwen38_inf2/fp4.py:118-140, checkpoint.py:177-182). BASELINE's weights are FP8 e4m3 with per-32 power-of-two
scales, which gfx950's scaled MFMA (`v_mfma_scale_f32_*_f8f6f4`) applies in hardware. Canonical host layout here is
``[out, in]`` (row per output column, like a torch Linear weight): ``weight_fp8`` uint8 ``[N, K]`` and
``scale_e8m0`` uint8 ``[N, K/32]``. A dequantized weight ``e4m3 * 2**(scale-127)`` is exact in bf16.

Activations are rounded to FP8 e5m2 at every projection input, as the reference does (model.py:85-87, 222-225).

These are torch ops and run on whichever device the tensor is on; the results are bit-identical on CPU and GPU
because every step is exact or a correctly rounded cast.
"""

from __future__ import annotations

import torch

GROUP = 32
E8M0_BIAS = 127
E4M3_MAX = 448.0


def quantize_e4m3(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a float ``[N, K]`` matrix to (e4m3 bytes ``[N, K]``, E8M0 bytes ``[N, K/32]``).

    OCP MX recipe: a group's scale is ``2**(floor(log2(amax)) - 8)``, 8 being e4m3's largest exponent, so the group's
    largest element lands in [256, 512) and saturates at 448.
    """
    n, k = weight.shape
    if k % GROUP:
        raise ValueError(f"K={k} is not a multiple of {GROUP}")
    groups = weight.float().reshape(n, k // GROUP, GROUP)
    amax = groups.abs().amax(dim=-1)
    _, exponent = torch.frexp(amax)  # amax = m * 2**exponent with m in [0.5, 1), so floor(log2(amax)) = exponent - 1
    scale_exp = torch.where(amax > 0, exponent - 1 - 8, torch.zeros_like(exponent)).clamp(-126, 126)
    scaled = groups * pow2(-scale_exp).unsqueeze(-1)
    coded = scaled.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
    return coded.reshape(n, k), (scale_exp + E8M0_BIAS).to(torch.uint8)


def pow2(exponent: torch.Tensor) -> torch.Tensor:
    """Exactly ``2**exponent`` as float32 for integer exponents in [-126, 127], built from the bit fields."""
    return ((exponent.to(torch.int32) + 127) << 23).view(torch.float32)


def dequantize_e4m3(coded: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """float32 ``[N, K]`` from e4m3 bytes and E8M0 scale bytes."""
    n, k = coded.shape
    values = coded.view(torch.float8_e4m3fn).float().reshape(n, k // GROUP, GROUP)
    return (values * pow2(scales.to(torch.int32) - E8M0_BIAS).unsqueeze(-1)).reshape(n, k)


E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def quantize_mxfp4(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a float ``[N, K]`` matrix to the checkpoint's MXFP4 (OCP microscaling E2M1 + E8M0, the format the
    reference loads, fp4.py:1-13): (packed bytes ``[N, K/2]``, the even element in the low nibble, a nibble being sign
    (bit 3) and a magnitude index into 0, 0.5, 1, 1.5, 2, 3, 4, 6; E8M0 bytes ``[N, K/32]``). A group's scale is
    ``2**(floor(log2(amax)) - 2)``, 2 being E2M1's largest exponent; values round to the nearest magnitude (ties to
    the even index) and saturate at 6."""
    n, k = weight.shape
    if k % GROUP:
        raise ValueError(f"K={k} is not a multiple of {GROUP}")
    groups = weight.float().reshape(n, k // GROUP, GROUP)
    amax = groups.abs().amax(dim=-1)
    _, exponent = torch.frexp(amax)
    scale_exp = torch.where(amax > 0, exponent - 1 - 2, torch.zeros_like(exponent)).clamp(-126, 126)
    scaled = groups * pow2(-scale_exp).unsqueeze(-1)
    mags = torch.tensor(E2M1_MAGNITUDES, device=weight.device)
    # Nearest magnitude; at a midpoint the even index (a zero mantissa bit) wins, as round-to-nearest-even does.
    dist = (scaled.abs().clamp(max=6.0).unsqueeze(-1) - mags).abs()
    best = dist.min(dim=-1, keepdim=True).values
    cand = (dist == best) & (torch.arange(8, device=weight.device) % 2 == 0)
    index = torch.where(cand.any(dim=-1), cand.int().argmax(dim=-1), dist.argmin(dim=-1))
    nibble = (index | torch.where(scaled < 0, 8, 0)).to(torch.uint8).reshape(n, k)
    packed = nibble[:, 0::2] | (nibble[:, 1::2] << 4)
    return packed, (scale_exp + E8M0_BIAS).to(torch.uint8)


def dequantize_mxfp4(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """float32 ``[N, K]`` from MXFP4 bytes and E8M0 scale bytes (the reference's `fp4.decode_host`, fp4.py:36-42)."""
    n, half = packed.shape
    lut = torch.tensor(E2M1_MAGNITUDES, device=packed.device)
    lut = torch.cat((lut, -lut))
    nibbles = torch.stack((packed & 0x0F, packed >> 4), dim=-1).reshape(n, 2 * half)
    values = lut[nibbles.long()].reshape(n, half * 2 // GROUP, GROUP)
    return (values * pow2(scales.to(torch.int32) - E8M0_BIAS).unsqueeze(-1)).reshape(n, 2 * half)


def mxfp4_to_e4m3(packed: torch.Tensor, scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The same weights in this build's FP8 format, exactly: every E2M1 magnitude is an e4m3 value, so the e4m3 bytes
    keep the group's E8M0 scale."""
    n, half = packed.shape
    lut = torch.tensor(E2M1_MAGNITUDES, device=packed.device)
    lut = torch.cat((lut, -lut)).to(torch.float8_e4m3fn).view(torch.uint8)
    nibbles = torch.stack((packed & 0x0F, packed >> 4), dim=-1).reshape(n, 2 * half)
    return lut[nibbles.long()], scales.clone()


# The FP8 KV cache's largest value (the reference clamps to NeuronCore-v2's finite e4m3 range, model.py:41).
FP8_KV_MAX = 240.0


def encode_kv(t: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """KV-cache bytes of ``t`` with the layer's bf16 scale: e4m3 of ``float32(t) / float32(scale)`` clamped to +-240
    (the reference's `FullAttentionStep._store`, model.py:579-585), for preparing synthetic caches on the host."""
    return (t.float() / scale.float()).clamp(-FP8_KV_MAX, FP8_KV_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def decode_kv(coded: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Cached values back: ``dtype(e4m3 value * scale)`` (model.py:587-589)."""
    return (coded.view(torch.float8_e4m3fn).to(dtype) * scale.to(dtype)).to(dtype)


def round_e5m2(x: torch.Tensor) -> torch.Tensor:
    """Round to FP8 e5m2 and back, as `model.fp8_round` does (model.py:85-87)."""
    return x.to(torch.float8_e5m2).to(x.dtype)
