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
    # The FP4Linear operator checks its shapes before any device work; its scratch holds bf16 input tiles (twice the
    # e5m2 tiles of the FP8 projection's scratch) before the same GEMM counters and partial slots.
    p = ctypes.c_void_p(4096)
    assert lib.q38_fp4_linear(p, 4, 256, p, p, 100, p, p, None) != 0
    assert b"N % 256" in lib.q38_last_error()
    assert lib.q38_fp4_linear(None, 4, 256, p, p, 256, p, p, None) != 0
    assert b"null" in lib.q38_last_error()
    for rows, k in ((3, 256), (64, 5120), (256, 17408)):
        extra = lib.q38_fp4_linear_scratch(rows, k) - lib.q38_fp8_linear_scratch(rows, k)
        assert extra == lib.q38_tiles_size(rows, k)


def test_weight_and_kv_cache_formats_size_their_buffers():
    cfg = tiny_config(1)  # layers 0-2 gated delta, 3 attention; MTP layer 4
    e4, f4 = ext.Handle(cfg, 4, 4, 128, True), ext.Handle(cfg, 4, 4, 128, True, weight_format="mxfp4")
    h, i = cfg.hidden_size, cfg.intermediate_size
    assert e4.buffer_size("mlp.gate_up.tiles", 0) == 2 * i * h
    assert f4.buffer_size("mlp.gate_up.tiles", 0) == i * h  # E2M1: half a byte per weight
    assert f4.buffer_size("mlp.gate_up.scales", 0) == e4.buffer_size("mlp.gate_up.scales", 0)
    assert f4.buffer_size("self_attn.o_proj.tiles", 3) * 2 == e4.buffer_size("self_attn.o_proj.tiles", 3)
    # the MTP layer and the head stay e4m3 in an MXFP4 engine
    assert f4.buffer_size("mtp.fc.tiles", 4) == e4.buffer_size("mtp.fc.tiles", 4)
    assert f4.buffer_size("mlp.down.tiles", 4) == e4.buffer_size("mlp.down.tiles", 4)
    assert f4.buffer_size("head.lm_head.tiles", -1) == e4.buffer_size("head.lm_head.tiles", -1)

    kv8 = ext.Handle(cfg, 4, 4, 128, True, kv_cache_format="fp8")
    assert kv8.buffer_size("self_attn.k_cache", 3) * 2 == e4.buffer_size("self_attn.k_cache", 3)
    assert kv8.buffer_size("self_attn.v_cache", 4) * 2 == e4.buffer_size("self_attn.v_cache", 4)
    assert kv8.buffer_size("self_attn.k_scale", 3) == 2 and kv8.buffer_size("self_attn.v_scale", 4) == 2
    with pytest.raises(RuntimeError, match="no buffer"):
        e4.buffer_size("self_attn.k_scale", 3)  # a bf16 cache has no scales

    c = ext.make_config(cfg, 4, 4, 128, True)
    lib, out = ext.library(), ctypes.c_void_p()
    for field in ("weight_format", "kv_cache_format"):
        bad = ext.make_config(cfg, 4, 4, 128, True)
        setattr(bad, field, 2)
        assert lib.q38_create(ctypes.byref(bad), ctypes.byref(out)) != 0
        assert b"unknown " + field.encode() in lib.q38_last_error()
    assert lib.q38_create(ctypes.byref(c), ctypes.byref(out)) == 0
    lib.q38_destroy(out)


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
