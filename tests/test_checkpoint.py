"""The checkpoint reader (qwen38_amd.checkpoint) on a small checkpoint written here in the Hugging Face layout the
reference reads (qwen38_inf2/checkpoint.py:24-32, 177-233, 324-392): MXFP4 decoder projections, bf16 everything else,
the MTP layer in its own file, KV-cache scales per attention layer. CPU only; the GPU test loads the same files."""

from __future__ import annotations

import torch
from safetensors.torch import save_file

from qwen38_amd import checkpoint as ckpt
from qwen38_amd import synth
from qwen38_amd.config import FULL, LINEAR, tiny_config
from qwen38_amd.quant import dequantize_e4m3, mxfp4_to_e4m3

P = ckpt.TEXT_PREFIX


def write_checkpoint(cfg, values: dict, directory) -> dict:
    """`values` (synth names, decoder projections already MXFP4) as a Hugging Face checkpoint in `directory`;
    returns the raw KV scales written."""
    bf = lambda t: t.to(torch.bfloat16).contiguous()  # noqa: E731
    dense = lambda v: dequantize_e4m3(*v).to(torch.bfloat16)  # noqa: E731
    main, mtp, scales = {}, {}, {}
    for i, kind in enumerate(cfg.layer_types):
        o, h = f"layers.{i}.", f"{P}layers.{i}."
        main[h + "input_layernorm.weight"] = bf(values[o + "input_layernorm_weight"])
        main[h + "post_attention_layernorm.weight"] = bf(values[o + "post_attention_layernorm_weight"])
        mats = ["mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
        if kind == LINEAR:
            mats += ["linear_attn.in_proj_qkv", "linear_attn.in_proj_z", "linear_attn.out_proj"]
            for k in ("in_proj_a", "in_proj_b"):
                main[h + f"linear_attn.{k}.weight"] = bf(values[o + f"linear_attn.{k}"])
            main[h + "linear_attn.conv1d.weight"] = bf(values[o + "linear_attn.conv_weight"]).unsqueeze(1).contiguous()
            main[h + "linear_attn.A_log"] = bf(values[o + "linear_attn.A_log"])
            main[h + "linear_attn.dt_bias"] = bf(values[o + "linear_attn.dt_bias"])
            main[h + "linear_attn.norm.weight"] = bf(values[o + "linear_attn.norm_weight"])
        else:
            mats += ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj"]
            main[h + "self_attn.q_norm.weight"] = bf(values[o + "self_attn.q_norm_weight"])
            main[h + "self_attn.k_norm.weight"] = bf(values[o + "self_attn.k_norm_weight"])
            scales[i] = torch.tensor([0.02 + 0.001 * i, 0.03 + 0.001 * i])
            main[h + "self_attn.k_scale"] = scales[i][0].clone()
            main[h + "self_attn.v_scale"] = scales[i][1].clone()
        for m in mats:
            packed, e8m0 = values[o + m]
            main[h + m + ".weight_packed"] = packed.contiguous()
            main[h + m + ".weight_scale"] = e8m0.contiguous()
    main[ckpt.FINAL_NORM] = bf(values["head.norm_weight"])
    main[ckpt.LM_HEAD] = dense(values["head.lm_head"])
    main[ckpt.EMBED_TOKENS] = bf(values["embed_tokens"])
    mtp["mtp.fc.weight"] = dense(values["mtp.fc"])
    for ours, theirs in (("embedding_norm_weight", "pre_fc_norm_embedding"), ("hidden_norm_weight", "pre_fc_norm_hidden"),
                         ("norm_weight", "norm")):
        mtp[f"mtp.{theirs}.weight"] = bf(values[f"mtp.{ours}"])
    for name, value in values.items():
        if name.startswith("mtp.layer."):
            short = name[len("mtp.layer."):]
            key = "mtp.layers.0." + short.replace("_weight", ".weight") if short.endswith("_weight") else f"mtp.layers.0.{short}.weight"
            mtp[key] = dense(value) if isinstance(value, tuple) else bf(value)
    half = len(main) // 2  # two shards, as a real checkpoint has several files
    names = sorted(main)
    save_file({k: main[k] for k in names[:half]}, str(directory / "model-00001-of-00002.safetensors"))
    save_file({k: main[k] for k in names[half:]}, str(directory / "model-00002-of-00002.safetensors"))
    save_file(mtp, str(directory / ckpt.MTP_FILE))
    return scales


def fake_model(tmp_path):
    cfg = tiny_config(1)
    values = dict(synth.to_mxfp4((s.name, v) for s, v in synth.make_all(synth.model_specs(cfg), 3)))
    scales = write_checkpoint(cfg, values, tmp_path)
    return cfg, values, scales


def test_checkpoint_reader_yields_the_engine_names_and_the_checkpoints_own_bytes(tmp_path):
    cfg, values, scales = fake_model(tmp_path)
    got = dict(ckpt.model_weights(tmp_path, cfg, "mxfp4"))
    # lm_head also comes as the file's own bf16 rows, which the head's exact recheck reads.
    assert set(got) == set(values) | {"head.lm_head_rows"}
    assert torch.equal(got["head.lm_head_rows"], dequantize_e4m3(*values["head.lm_head"]).to(torch.bfloat16))
    for name, want in values.items():
        value = got[name]
        if name.startswith("layers.") and isinstance(want, tuple):
            assert torch.equal(value[0], want[0]) and torch.equal(value[1], want[1]), name  # passed through
        elif isinstance(want, tuple):  # head and MTP matrices: bf16 in the file, e4m3 + E8M0 here
            w = dequantize_e4m3(*want)
            err = float((dequantize_e4m3(*value) - w).abs().max() / w.abs().max())
            assert err < 2.0**-4, (name, err)
        else:
            assert torch.equal(value, want.to(torch.bfloat16)), name
    e4 = dict(ckpt.model_weights(tmp_path, cfg, "e4m3", mtp=False))
    for name, want in values.items():
        if name.startswith("layers.") and isinstance(want, tuple):
            c, s = mxfp4_to_e4m3(*want)
            assert torch.equal(e4[name][0], c) and torch.equal(e4[name][1], s), name
    ks = ckpt.kv_scales(tmp_path, cfg)
    assert sorted(ks) == [i for i, k in enumerate(cfg.layer_types) if k == FULL]
    for i, (k, v) in ks.items():
        want = (scales[i] * (448.0 / 240.0)).to(torch.bfloat16)
        assert torch.equal(k, want[0:1]) and torch.equal(v, want[1:2])
