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


# Two tokens whose lm_head rows are +c*u and -c*u for one unit direction u: the model's picks and the MTP drafts then
# mostly land on these two, so drafts match the model's picks about half the time and a speculative step accepts
# 1..K tokens per row. With independent random rows a random-init model accepts no draft at all.
STEER_TOKENS = (1000, 2000)
STEER_SCALE = 50.0


def steer_head(values: dict, cfg, seed: int) -> dict:
    """``values`` with ``head.lm_head`` rows STEER_TOKENS replaced by +-STEER_SCALE * u (e4m3 + E8M0)."""
    from qwen38_amd.quant import quantize_e4m3

    g = torch.Generator().manual_seed(seed * 7919 + 17)
    u = torch.randn(cfg.hidden_size, generator=g)
    u = u / u.norm()
    coded, scales = (t.clone() for t in values["head.lm_head"])
    rc, rs = (t.to(coded.device) for t in quantize_e4m3(torch.stack((STEER_SCALE * u, -STEER_SCALE * u))))
    for i, token in enumerate(STEER_TOKENS):
        coded[token], scales[token] = rc[i], rs[i]
    out = dict(values)
    out["head.lm_head"] = (coded, scales)
    return out


# The speculative-step scenario (tests/golden/make_golden_spec.py, tests/test_oracle_spec.py, tests/test_gpu_spec.py):
# config 0 shapes, four slots of which three run, seeded as a prefill of prompts of 40, 64 and 1 tokens leaves them.
SPEC = {"seed": 0, "batch": 4, "tokens": 4, "max_seq_len": 128, "chunk": 16, "prompt_lens": [40, 64, 1, None], "steps": 5}


def spec_start(cfg, spec=SPEC):
    """The starting rows: prompt ids plus the first new token, and the prompt's last hidden state, per running slot
    (None for an empty slot)."""
    g = torch.Generator().manual_seed(4321)
    rows = []
    for slot, n in enumerate(spec["prompt_lens"]):
        if n is None:
            rows.append(None)
            continue
        ids = torch.randint(0, cfg.vocab_size, (n + 1,), generator=g).tolist()
        hidden = synth.hidden_states((1, cfg.hidden_size), spec["seed"], f"spec.seed.{slot}")
        rows.append({"ids": ids, "prompt_len": n, "hidden": hidden})
    return rows


def spec_states(cfg, spec=SPEC):
    """Decoder-layer states and the MTP layer's cache as a prefill of each prompt leaves them in shape: caches filled
    below the prompt length (the MTP cache below the last MTP index), seeded gated-delta and conv states, empty
    snapshots (the first verify step commits none of them)."""
    b, k, s, seed = spec["batch"], spec["tokens"], spec["max_seq_len"], spec["seed"]
    context = [n or 0 for n in spec["prompt_lens"]]
    states = []
    for i, kind in enumerate(cfg.layer_types):
        if kind == "linear_attention":
            states.append(synth.gdn_states(cfg, b, k, seed, f"spec.layers.{i}"))
        else:
            states.append(synth.kv_states(cfg, b, s, context, seed, f"spec.layers.{i}"))
    mtp = synth.kv_states(cfg, b, s, [max(n - 1, 0) for n in context], seed, "spec.mtp")
    return states, mtp


def row_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    """Largest per-row relative distance ||got - want|| / ||want|| over the leading dimension."""
    got, want = got.float().cpu(), want.float().cpu()
    worst = 0.0
    for r in range(want.shape[0]):
        n = float(want[r].norm())
        if n > 0:
            worst = max(worst, float((got[r] - want[r]).norm()) / n)
    return worst


# The prompt-lookup scenario (tests/golden/make_golden_lookup.py, tests/test_oracle_spec.py, tests/test_gpu_lookup.py):
# the speculative scenario's shapes, slots and states with no MTP drafter, so drafts come from each row's own history.
# Each prompt ends in a run of the two steered tokens, which the steered head mostly picks, so prompt lookup finds
# drafts that the model's picks match about half the time.
LOOKUP = dict(SPEC)


def lookup_start(cfg, spec=LOOKUP):
    """The starting rows: prompt ids (a random prefix, then a seeded run of the steered tokens) plus the first new
    token, per running slot (None for an empty slot)."""
    g = torch.Generator().manual_seed(8765)
    rows = []
    for n in spec["prompt_lens"]:
        if n is None:
            rows.append(None)
            continue
        tail = (n + 1) // 2
        prefix = torch.randint(0, cfg.vocab_size, (n + 1 - tail,), generator=g).tolist()
        run = [STEER_TOKENS[int(c)] for c in torch.randint(0, 2, (tail,), generator=g)]
        rows.append({"ids": prefix + run, "prompt_len": n})
    return rows
