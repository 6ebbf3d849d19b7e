"""The checkpoint reader against the real 27B checkpoint's header (the reference's tests/fixtures: config.json and the
dtype and shape of each of its 1,616 tensors, copied by tests/golden/copy_checkpoint_header.py), as the reference's
tests/test_real_checkpoint.py:38-80 checks its own reader. No weights are read: the source serves meta tensors of the
header's dtypes and shapes.

* The real config parses to this build's 27B preset, field for field, and passes the kernels' shape checks.
* Every decoder layer's weights come out under the names and shapes `steps.Engine.load` takes (the specs the GPU tests
  load, `synth.layer_specs`): each projection as the checkpoint's MXFP4 bytes [N, K/2] with E8M0 scales [N, K/32].
* The head's and embeddings' names and shapes match too, and the KV scales of every attention layer are found.
* Only the vision tower goes unread (the MTP layer lives in its own file).
"""

from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import pytest
import torch

from qwen38_amd import checkpoint, synth
from qwen38_amd.config import FULL, TextConfig, qwen38_27b_config

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = {"BF16": torch.bfloat16, "U8": torch.uint8, "F32": torch.float32}


class HeaderSource:
    """`checkpoint.Checkpoint`'s interface over the header: meta tensors, and a record of the names read."""

    def __init__(self, header: dict):
        self.header, self.read = header, set()

    def __contains__(self, name: str) -> bool:
        return name in self.header

    def get(self, name: str) -> torch.Tensor:
        if name not in self.header:
            raise KeyError(f"checkpoint has no tensor {name}")
        self.read.add(name)
        entry = self.header[name]
        return torch.empty(entry["shape"], dtype=DTYPES[entry["dtype"]], device="meta")


@pytest.fixture(scope="module")
def cfg():
    return TextConfig.from_file(GOLDEN / "ref_27b_config.json")


@pytest.fixture(scope="module")
def header():
    return json.loads((GOLDEN / "ref_27b_model.header.json").read_text())


def test_real_config_is_the_27b_preset(cfg):
    assert cfg.num_hidden_layers == 64 and cfg.layer_types.count(FULL) == 16 and cfg.rotary_dim == 64
    preset = qwen38_27b_config(16)
    for field in dataclasses.fields(TextConfig):
        assert getattr(cfg, field.name) == getattr(preset, field.name), field.name
    cfg.check()


def test_every_decoder_layer_loads_under_the_engines_names_and_shapes(cfg, header):
    source = HeaderSource(header)
    for i in range(cfg.num_hidden_layers):
        got = dict(checkpoint.layer_weights(source, cfg, i, "mxfp4"))
        specs = {s.name: s for s in synth.layer_specs(cfg, i)}
        assert set(got) == set(specs), i
        for name, spec in specs.items():
            value = got[name]
            if spec.kind == "fp8":
                packed, scales = value
                n, k = spec.shape
                assert packed.dtype == torch.uint8 and tuple(packed.shape) == (n, k // 2), name
                assert scales.dtype == torch.uint8 and tuple(scales.shape) == (n, k // 32), name
            else:
                assert value.dtype == torch.bfloat16 and tuple(value.shape) == tuple(spec.shape), name


def test_head_embeddings_and_kv_scales(cfg, header, monkeypatch):
    source = HeaderSource(header)
    # Shapes only: the e4m3 quantization of lm_head is the codec tests' business, not this header's.
    monkeypatch.setattr(checkpoint, "e4m3_from_bf16",
                        lambda w: (torch.empty(w.shape, dtype=torch.uint8, device="meta"),
                                   torch.empty(w.shape[0], w.shape[1] // 32, dtype=torch.uint8, device="meta")))
    got = dict(checkpoint.head_weights(source))
    specs = {s.name: s for s in synth.head_specs(cfg)}
    # Besides the engine's head weights, lm_head's bf16 rows for the exact recheck.
    assert set(got) == set(specs) | {"head.lm_head_rows"}
    for name, spec in specs.items():
        value = got[name][0] if spec.kind == "fp8" else got[name]
        assert tuple(value.shape) == tuple(spec.shape), name
    assert got["head.lm_head_rows"].dtype == torch.bfloat16
    assert tuple(got["head.lm_head_rows"].shape) == (cfg.vocab_size, cfg.hidden_size)
    scales = checkpoint.kv_scales(source, cfg)
    assert sorted(scales) == [i for i, kind in enumerate(cfg.layer_types) if kind == FULL]
    assert all(tuple(k.shape) == (1,) and tuple(v.shape) == (1,) for k, v in scales.values())


def test_only_the_vision_tower_goes_unread(cfg, header, monkeypatch):
    source = HeaderSource(header)
    monkeypatch.setattr(checkpoint, "e4m3_from_bf16", lambda w: (w, w))
    for i in range(cfg.num_hidden_layers):
        checkpoint.layer_weights(source, cfg, i, "mxfp4")
    checkpoint.head_weights(source)
    checkpoint.kv_scales(source, cfg)
    unread = set(header) - source.read
    assert unread and all(n.startswith("model.visual.") for n in unread), sorted(n for n in unread if "visual" not in n)[:5]
    assert not [n for n in source.read if "visual" in n or "mtp" in n]
