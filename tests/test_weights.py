"""Host-side weight preparation for MXFP4 engines (CPU): the requantized model and its e4m3 twin hold the same values."""

from __future__ import annotations

import torch

from qwen38_amd import synth
from qwen38_amd.config import tiny_config
from qwen38_amd.quant import dequantize_e4m3, dequantize_mxfp4


def test_mxfp4_model_and_its_e4m3_twin_hold_the_same_values():
    cfg = tiny_config(1)
    values = dict((sp.name, v) for sp, v in synth.make_all(synth.model_specs(cfg), 0))
    fp4 = dict(synth.to_mxfp4(values.items()))
    twin = dict(synth.mxfp4_as_e4m3(fp4.items()))
    converted = 0
    for name, value in fp4.items():
        if not isinstance(value, tuple):
            assert value is values[name]
            continue
        n, k = values[name][0].shape
        if name.startswith("layers."):
            converted += 1
            assert value[0].shape == (n, k // 2) and value[1].shape == (n, k // 32)
            w4 = dequantize_mxfp4(*value)
            assert torch.equal(w4, dequantize_e4m3(*twin[name]))
            w = dequantize_e4m3(*values[name])
            # Requantization keeps each group's largest magnitude within E2M1's relative step (1/4 at worst).
            assert float((w4 - w).norm() / w.norm()) < 0.2
        else:  # the MTP layer and the head stay e4m3
            assert value is values[name] and twin[name] is values[name]
    assert converted == sum(len([1 for s in synth.layer_specs(cfg, i) if s.kind == "fp8"]) for i in range(cfg.num_hidden_layers))
