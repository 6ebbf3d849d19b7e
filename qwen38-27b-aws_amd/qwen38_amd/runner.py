"""Load the model once onto the GPU and hand the scheduler its graphs: the counterpart of the reference's
`runner.load` / `Loaded` (qwen38_inf2/runner.py:21-90) for one MI355X.

The reference reads a compiled Neuron build's facts (rows, context, prefill chunk, verify tokens) from its build
info and loads the head and the MTP drafter from their own builds; here nothing is compiled ahead, so those facts are
arguments, and the head and the MTP layer live in the same `steps.Engine` as the blocks. The reference's two checks
on what it loads stay, with its messages: a verify graph needs a head for rows x tokens rows (runner.py:76-77), and
an MTP build must match the blocks' rows, tokens and chunk (runner.py:80-84).
"""

from __future__ import annotations

import time
from collections.abc import Callable, Iterable
from dataclasses import dataclass
from pathlib import Path

import torch

from .config import TextConfig


def _log(message: str) -> None:
    print(message, flush=True)


@dataclass
class Loaded:
    """The fields of the reference's `Loaded` (runner.py:21-37)."""

    cfg: TextConfig
    tokenizer: object
    head: object
    step: Callable[..., torch.Tensor]
    batch_size: int
    max_seq_len: int
    load_seconds: float
    # The prefill graph, called as `generate.prefill_prompt` does, and its tokens per call. None without one.
    prefill: Callable[..., torch.Tensor] | None = None
    chunk: int | None = None
    # The verify graph for speculative decoding and its tokens per row, with a head for that many rows each.
    verify: Callable[..., torch.Tensor] | None = None
    verify_tokens: int = 0
    # The MTP drafter, if loaded; the blocks' last hidden state goes to it.
    mtp: Callable[..., torch.Tensor] | None = None
    engine: object = None


def check_build(batch_size: int, verify_tokens: int, chunk: int | None, head_batch: int | None,
                mtp_build: dict | None) -> None:
    """The reference's load-time checks (runner.py:76-77, 83-84), with its messages."""
    if verify_tokens and head_batch is not None and head_batch < batch_size * verify_tokens:
        raise ValueError(f"a verify graph of {verify_tokens} tokens for {batch_size} rows needs a head for "
                         f"{batch_size * verify_tokens} rows")
    if mtp_build is not None:
        if (mtp_build["batch_size"], mtp_build["mtp_tokens"], mtp_build["chunk"]) != (batch_size, verify_tokens, chunk):
            raise ValueError(f"the MTP build's rows, tokens and chunk {mtp_build} don't match the blocks'")


def load(model_dir: str | Path | None = None, *, cfg: TextConfig | None = None,
         weights: Iterable[tuple[str, object]] | None = None, batch_size: int = 1, max_seq_len: int = 4096,
         verify_tokens: int = 0, chunk: int | None = None, mtp: bool = False, head_batch: int | None = None,
         mtp_build: dict | None = None, weight_format: str = "mxfp4", kv_cache_format: str = "bf16",
         saved_states: bool = False, log: Callable[[str], None] = _log) -> Loaded:
    """The model of ``model_dir`` (its config.json, its safetensors files through `checkpoint.model_weights`, its
    tokenizer.json if present), or ``cfg`` with ``weights`` as (name, value) pairs (`synth.model_specs` names), on the
    GPU. ``head_batch`` is the head's rows (default rows x tokens); ``mtp_build`` ({"batch_size", "mtp_tokens",
    "chunk"}) describes a separately built drafter to check against the blocks, as the reference checks its MTP
    build's info."""
    from . import checkpoint
    from .generate import ChipHead
    from .steps import Engine, HeadGraph, MTPStep, StepGraph, VerifyStep

    if cfg is None:
        if model_dir is None:
            raise ValueError("load needs a model directory or a config")
        cfg = TextConfig.from_file(Path(model_dir) / "config.json")
    check_build(batch_size, verify_tokens, chunk, head_batch, mtp_build)
    if weights is None:
        if model_dir is None:
            raise ValueError("load needs a model directory or weights")
        weights = checkpoint.model_weights(model_dir, cfg, weight_format, mtp)
    tokenizer = None
    if model_dir is not None and (Path(model_dir) / "tokenizer.json").exists():
        from tokenizers import Tokenizer

        tokenizer = Tokenizer.from_file(str(Path(model_dir) / "tokenizer.json"))

    started = time.perf_counter()
    engine = Engine(cfg, batch_size, max(verify_tokens, 1), max_seq_len, mtp=mtp, saved_states=saved_states,
                    prefill_chunk=chunk or 0, weight_format="mxfp4" if weight_format == "mxfp4" else "e4m3",
                    kv_cache_format=kv_cache_format)
    engine.load(weights)
    if kv_cache_format == "fp8" and model_dir is not None:
        for i, (k, v) in checkpoint.kv_scales(model_dir, cfg).items():
            engine.set_kv_scales(i, k, v)
    torch.cuda.synchronize()
    load_seconds = time.perf_counter() - started
    log(f"loaded {batch_size}-row engine in {load_seconds:.1f}s")
    head = ChipHead(None, cfg.rms_norm_eps, HeadGraph(engine), head_batch or batch_size * max(verify_tokens, 1))
    step = StepGraph(engine)
    return Loaded(cfg, tokenizer, head, step, batch_size, max_seq_len, load_seconds, step if chunk else None, chunk,
                  VerifyStep(engine) if verify_tokens else None, verify_tokens, MTPStep(engine) if mtp else None, engine)
