"""The C ABI: the built library loads without a GPU and exports every function include/q38.h declares; shape checks
at handle creation refuse what the kernels do not support (no GPU work is done here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from qwen38_amd import ext
from qwen38_amd.config import qwen38_27b_config, tiny_config, with_layers

HEADER = Path(__file__).resolve().parents[1] / "include" / "q38.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(q38_\w+)\s*\(", text)))


def test_every_declared_function_is_exported():
    lib = ext.library()
    names = declared_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(ext.EXPORTS)


def test_handles_are_created_for_every_workload_shape_and_buffers_are_sized():
    for cfg, b, k, s in [(tiny_config(1), 4, 4, 128), (qwen38_27b_config(16), 64, 4, 1024), (qwen38_27b_config(1), 256, 8, 4160)]:
        h = ext.Handle(cfg, b, k, s, True)
        assert h.buffer_size("linear_attn.recurrent_state", 0) == b * cfg.linear_num_value_heads * 128 * 128 * 2
        assert h.buffer_size("self_attn.k_cache", 3) == b * cfg.num_key_value_heads * s * 256 * 2
        assert h.buffer_size("mtp.fc.tiles", cfg.num_hidden_layers) == cfg.hidden_size * 2 * cfg.hidden_size
        assert h.buffer_size("head.lm_head.scales", -1) == cfg.vocab_size * cfg.hidden_size // 32
        assert h.buffer_size("workspace", -1) > 0
        assert h.parity == 0


def test_unsupported_shapes_and_names_are_refused():
    with pytest.raises(RuntimeError, match="verify_tokens"):
        ext.Handle(tiny_config(1), 4, 9, 128, True)
    with pytest.raises(RuntimeError, match="max_seq_len"):
        ext.Handle(tiny_config(1), 4, 4, 100, True)
    h = ext.Handle(with_layers(tiny_config(1), ("linear_attention",)), 2, 4, 128, False)
    with pytest.raises(RuntimeError, match="no buffer"):
        h.buffer_size("self_attn.k_cache", 0)
    with pytest.raises(RuntimeError, match="no buffer"):
        h.buffer_size("mtp.fc.tiles", 1)
    lib = ext.library()
    assert lib.q38_bind(h.h, b"linear_attn.recurrent_state", 0, ctypes.c_void_p(4096), 3) != 0
    assert b"needs" in lib.q38_last_error()
