"""Host side of the verify path, mirroring the reference's generate.py: RoPE tables, the verify/MTP input dicts,
embedding gathers and the head that turns hidden states into token ids.

The input builders keep the reference's names, arguments, dtypes and errors exactly (generate.py:25-116), so a
caller written for the reference builds the same dicts. `ChipHead` keeps its signature (generate.py:162-208); its
`run_graph` is this package's `steps.HeadGraph`, so the group max *and* the exact top-group recheck run on the GPU and
only token ids come back to the host.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch

from .config import TextConfig

# From the checkpoint's generation_config.json: <|im_end|> and <|endoftext|> (reference generate.py:15-16).
EOS_TOKEN_IDS = (248046, 248044)


def rotary(cfg: TextConfig, positions: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """cos and sin for each position, ``[len(positions), rotary_dim]`` (reference generate.py:25-31): float32
    inverse frequencies ``theta^(-2i/d)``, repeated twice, rounded to ``dtype``."""
    dim = cfg.rotary_dim
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    freqs = positions.float().unsqueeze(-1) * inv_freq
    return freqs.cos().repeat(1, 2).to(dtype), freqs.sin().repeat(1, 2).to(dtype)


def rope_table(cfg: TextConfig, max_seq_len: int, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``[max_seq_len, 2, rotary_dim]``: `rotary` for every position, so the device can gather a row's cos/sin by
    position when it produces positions itself (the on-device speculative step)."""
    cos, sin = rotary(cfg, torch.arange(max_seq_len), dtype)
    return torch.stack((cos, sin), dim=1).contiguous()


def step_inputs(cfg: TextConfig, position: int, max_seq_len: int, dtype: torch.dtype) -> dict[str, torch.Tensor]:
    return batch_step_inputs(cfg, [position], max_seq_len, dtype)


def batch_step_inputs(
    cfg: TextConfig, positions: Sequence[int], max_seq_len: int, dtype: torch.dtype, active: Sequence[bool] | None = None
) -> dict[str, torch.Tensor]:
    """Decode inputs, one row per sequence (reference generate.py:38-55)."""
    position = torch.as_tensor(positions, dtype=torch.int32)
    on = torch.ones(len(positions), dtype=torch.bool) if active is None else torch.as_tensor(active, dtype=torch.bool)
    if bool((position[on] >= max_seq_len - 1).any()):
        raise ValueError(f"position {int(position[on].max())} is past the last usable one of max_seq_len {max_seq_len}")
    cos, sin = rotary(cfg, position, dtype)
    return {"cos": cos.unsqueeze(1), "sin": sin.unsqueeze(1), "position": position, "active": on.float()}


def verify_inputs(
    cfg: TextConfig, positions: Sequence[int], tokens: int, max_seq_len: int, dtype: torch.dtype, active: Sequence[bool], accepted: Sequence[int]
) -> dict[str, torch.Tensor]:
    """Verify inputs for `tokens` tokens per row from each row's position (reference generate.py:72-87)."""
    position = torch.as_tensor(positions, dtype=torch.int32)
    on = torch.as_tensor(active, dtype=torch.bool)
    if bool((position[on] + tokens > max_seq_len - 1).any()):
        raise ValueError(f"a row's {tokens} tokens from position {int(position[on].max())} pass max_seq_len {max_seq_len}")
    cos, sin = rotary(cfg, (position.unsqueeze(-1) + torch.arange(tokens)).reshape(-1), dtype)
    return {
        "cos": cos.reshape(len(positions), tokens, -1),
        "sin": sin.reshape(len(positions), tokens, -1),
        "position": position,
        "active": on.float(),
        "accepted": torch.as_tensor(accepted, dtype=torch.int32),
    }


def mtp_step_inputs(
    cfg: TextConfig, indices: Sequence[int], tokens: int, max_seq_len: int, dtype: torch.dtype, active: Sequence[bool]
) -> dict[str, torch.Tensor]:
    """Inputs for MTP steps: `tokens` per row from each row's MTP index, at positions one on (generate.py:90-99)."""
    inputs = verify_inputs(cfg, indices, tokens, max_seq_len, dtype, active, [0] * len(indices))
    del inputs["accepted"]
    at = (torch.as_tensor(indices, dtype=torch.int32).unsqueeze(-1) + 1 + torch.arange(tokens)).reshape(-1)
    cos, sin = rotary(cfg, at, dtype)
    inputs["cos"], inputs["sin"] = cos.reshape(len(indices), tokens, -1), sin.reshape(len(indices), tokens, -1)
    return inputs


def prefill_inputs(cfg: TextConfig, slot: int, start: int, n_valid: int, chunk: int, dtype: torch.dtype) -> dict[str, torch.Tensor]:
    """Prefill inputs for `n_valid` tokens of one row from position `start`, padded to a full chunk (reference
    generate.py:58-69)."""
    if start < 0 or not 0 < n_valid <= chunk:
        raise ValueError(f"a chunk must start at a position and hold 1 to {chunk} tokens")
    cos, sin = rotary(cfg, start + torch.arange(chunk), dtype)
    return {
        "cos": cos.unsqueeze(0),
        "sin": sin.unsqueeze(0),
        "slot": torch.tensor([slot], dtype=torch.int32),
        "start": torch.tensor([start], dtype=torch.int32),
        "n_valid": torch.tensor([n_valid], dtype=torch.int32),
    }


def mtp_prefill_inputs(cfg: TextConfig, slot: int, start: int, n_valid: int, chunk: int, dtype: torch.dtype) -> dict[str, torch.Tensor]:
    """Inputs for an MTP prefill chunk of one row from MTP index `start`, at positions one on (reference
    generate.py:102-107)."""
    inputs = prefill_inputs(cfg, slot, start, n_valid, chunk, dtype)
    cos, sin = rotary(cfg, start + 1 + torch.arange(chunk), dtype)
    inputs["cos"], inputs["sin"] = cos.unsqueeze(0), sin.unsqueeze(0)
    return inputs


def state_copy_inputs(cfg: TextConfig, slot: int, save: bool, dtype: torch.dtype) -> dict[str, torch.Tensor]:
    """Inputs that save one row's recurrent states, or restore them (reference generate.py:110-116)."""
    return {
        "inputs_embeds": torch.zeros(1, 1, cfg.hidden_size, dtype=dtype),
        ("save_slot" if save else "restore_slot"): torch.tensor([slot], dtype=torch.int32),
    }


class BlockChain:
    """Run blocks of layers in sequence as one step (reference generate.py:211-221)."""

    def __init__(self, blocks: Sequence[Callable[..., torch.Tensor]]):
        self.blocks = blocks

    def __call__(self, inputs_embeds: torch.Tensor, **inputs: torch.Tensor) -> torch.Tensor:
        hidden = inputs_embeds
        for block in self.blocks:
            hidden = block(inputs_embeds=hidden, **inputs)
        return hidden


class ChipHead:
    """lm_head as group maxima plus an exact recheck of the best groups (reference generate.py:162-208).

    ``source`` has ``get(name)``, ``get_rows(name, ids)`` and ``matrix_view(name)`` for the final norm, the embedding
    table and lm_head (as the reference's checkpoint sources do); it may be None, since ``run_graph`` (a
    `steps.HeadGraph`) holds the final norm, lm_head and embeddings on the GPU and runs the maxima and the recheck there.
    """

    FINAL_NORM = "model.language_model.norm.weight"
    LM_HEAD = "lm_head.weight"
    EMBED_TOKENS = "model.language_model.embed_tokens.weight"

    def __init__(self, source, eps: float, run_graph: Callable[..., torch.Tensor], batch_size: int, group_rows: int = 32, recheck_groups: int = 4):
        self.source = source
        self.eps = eps
        self.run_graph = run_graph
        self.batch_size = batch_size
        self.group_rows = group_rows
        self.recheck_groups = recheck_groups

    def embed_batch(self, token_ids: Sequence[int], dtype: torch.dtype) -> torch.Tensor:
        embed = getattr(self.run_graph, "embed", None)
        if embed is not None:
            return embed(token_ids).unsqueeze(1).to(dtype)
        return self.source.get_rows(self.EMBED_TOKENS, list(token_ids)).unsqueeze(1).to(dtype)

    def next_tokens(self, hidden: torch.Tensor, recheck_groups: int | None = None) -> list[int]:
        """Greedy next token for each row of ``[rows, 1, hidden]``."""
        groups = recheck_groups or self.recheck_groups
        pick = getattr(self.run_graph, "pick", None)
        if pick is None:
            raise TypeError("run_graph must be a steps.HeadGraph: the group max and its recheck run on the GPU")
        return pick(hidden, groups).tolist()
