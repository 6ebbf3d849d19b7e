"""Shared test scenarios: seeded weights and states turned into oracle inputs, and the same inputs for the GPU."""

from __future__ import annotations

import json
from pathlib import Path

import torch

from oracle import model as om
from qwen38_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def oracle_weights(specs_values: dict, cfg):
    """Per-layer oracle weight dicts (short names) plus the MTP and head pieces, from ``{name: value}``."""
    def conv(v):
        return om.FP8Weight(*v) if isinstance(v, tuple) else v

    layers = []
    for i in range(cfg.num_hidden_layers):
        prefix = f"layers.{i}."
        layers.append({n[len(prefix):]: conv(v) for n, v in specs_values.items() if n.startswith(prefix)})
    mtp = {n[len("mtp."):]: conv(v) for n, v in specs_values.items() if n.startswith("mtp.")}
    if "head.norm_weight" in specs_values:
        mtp["final_norm_weight"] = specs_values["head.norm_weight"]
    head = {n[len("head."):]: conv(v) for n, v in specs_values.items() if n.startswith("head.")}
    return layers, mtp, head


def golden_meta() -> dict:
    return json.loads((GOLDEN / "verify_tiny.json").read_text())


def golden_tensors() -> dict:
    from safetensors.torch import load_file

    return load_file(GOLDEN / "verify_tiny.safetensors")


def tiny_states(cfg, meta, seed):
    """Oracle states for the golden scenario: per-layer dicts, same generator names as make_golden.py."""
    states = []
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            states.append(synth.gdn_states(cfg, meta["batch"], meta["tokens"], seed, f"layers.{i}"))
        else:
            states.append(synth.kv_states(cfg, meta["batch"], meta["max_seq_len"], meta["context"], seed, f"layers.{i}"))
    return states


def clone_states(states):
    return [{k: v.clone() for k, v in st.items()} for st in states]
