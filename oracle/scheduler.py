"""CPU restatement of the reference's speculative scheduler. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

What it restates, from /root/reference/qwen38_inf2:
* the step input builders `rotary`, `batch_step_inputs`, `prefill_inputs`, `verify_inputs`, `mtp_step_inputs`,
  `mtp_prefill_inputs` (generate.py:25-107);
* `Scheduler._mtp_drafts` (scheduler.py:160-193): K - 1 drafts per running row from the MTP layer, the first call over
  the row's last K positions, each later one on the previous call's output and the token it drafted;
* `Scheduler._verify_step` (scheduler.py:269-301): ``[last token] + drafts`` per row, one verify call, the head over
  every row's K tokens, longest-prefix acceptance, the next step's MTP seed; without an MTP drafter the drafts come
  from the row's own history by prompt lookup, padded with the row's last token (scheduler.py:276-282);
* `lookup_draft` (drafting.py:11-24), the history scan that `Drafter.draft` (drafting.py:44-51) equals (reference
  tests/test_scheduler.py:177-185), which the restated step calls on the row's tokens;
* the parts of `Scheduler.run_sessions`, `_prefill` and `_mtp_prefill` (scheduler.py:110-158, 201-267) a speculative
  run needs, for single-turn prompts without prefix reuse, so the reference's invariants can run on it;
* graph adapters with the reference's call forms over `oracle.model`: `Step` (`Qwen38Step.forward`, model.py:983-995),
  `MTP` (`MTPStep.forward`, model.py:843-860), `ChipHead` (generate.py:162-208 over `HeadStep`'s CPU branch,
  model.py:890-900) and `HostHead` (generate.py:156-159).

The loop takes its graphs as callables with the reference's keyword forms, as the reference's `Scheduler` does, so the
same restated loop drives the CPU oracle's graphs, fakes, or the GPU build's step objects.

Pinning:
* tests/golden/spec_tiny.safetensors, written by tests/golden/make_golden_spec.py from the reference's own
  `Scheduler._verify_step` (which calls `_mtp_drafts`) over three speculative steps on config 0 shapes in bf16: drafts,
  picks, matches, emitted tokens, hidden states and state digests bit for bit;
* tests/golden/lookup_tiny.safetensors, written by tests/golden/make_golden_lookup.py from the reference's own
  `Scheduler._verify_step` with no MTP drafter (its `Drafter` drafts) over five steps on config 0 shapes: drafts,
  picks, matches, hidden states and state digests bit for bit;
* tests/test_oracle_spec.py holds the reference's invariants on it: speculation with MTP drafts gives the tokens plain
  greedy decoding gives, and each step's first draft is what the MTP layer gives over the sequence's true history
  (reference tests/test_prefill.py:267-289, 380-448); and a fake-device contract in the style of reference
  tests/test_scheduler.py:13-80 fixing every index the draft loop computes by closed form;
* the input builders: cos/sin bit-equal to the golden vectors' (reference verify_inputs) and the ValueError bounds.
"""

from __future__ import annotations

from collections.abc import Callable, Iterator, Sequence
from dataclasses import dataclass

import torch

from . import model as om


# ----------------------------------------------------------------------------------------------- input builders


def rotary(cfg, positions: torch.Tensor, dtype: torch.dtype):
    """generate.py:25-31: float32 inverse frequencies theta^(-2i/d), angles per position, cos/sin repeated twice along
    the rotary dims, rounded to ``dtype``."""
    dim = cfg.rotary_dim
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    angles = positions.float().unsqueeze(-1) * inv_freq
    return angles.cos().repeat(1, 2).to(dtype), angles.sin().repeat(1, 2).to(dtype)


def batch_step_inputs(cfg, positions, max_seq_len: int, dtype, active=None) -> dict:
    """generate.py:38-55: one-token decode inputs; ValueError for an active row at or past max_seq_len - 1."""
    position = torch.as_tensor(positions, dtype=torch.int32)
    on = torch.ones(len(positions), dtype=torch.bool) if active is None else torch.as_tensor(active, dtype=torch.bool)
    if bool((position[on] >= max_seq_len - 1).any()):
        raise ValueError(f"position {int(position[on].max())} is past the last usable one of max_seq_len {max_seq_len}")
    cos, sin = rotary(cfg, position, dtype)
    return {"cos": cos.unsqueeze(1), "sin": sin.unsqueeze(1), "position": position, "active": on.float()}


def prefill_inputs(cfg, slot: int, start: int, n_valid: int, chunk: int, dtype) -> dict:
    """generate.py:58-69: a chunk of one row from ``start``, padded to ``chunk`` tokens."""
    if start < 0 or not 0 < n_valid <= chunk:
        raise ValueError(f"a chunk must start at a position and hold 1 to {chunk} tokens")
    cos, sin = rotary(cfg, start + torch.arange(chunk), dtype)
    return {"cos": cos.unsqueeze(0), "sin": sin.unsqueeze(0), "slot": torch.tensor([slot], dtype=torch.int32),
            "start": torch.tensor([start], dtype=torch.int32), "n_valid": torch.tensor([n_valid], dtype=torch.int32)}


def verify_inputs(cfg, positions, tokens: int, max_seq_len: int, dtype, active, accepted) -> dict:
    """generate.py:72-87: ``tokens`` per row from each row's position; ValueError when an active row's last one passes
    max_seq_len - 1."""
    position = torch.as_tensor(positions, dtype=torch.int32)
    on = torch.as_tensor(active, dtype=torch.bool)
    if bool((position[on] + tokens > max_seq_len - 1).any()):
        raise ValueError(f"a row's {tokens} tokens from position {int(position[on].max())} pass max_seq_len {max_seq_len}")
    cos, sin = rotary(cfg, (position.unsqueeze(-1) + torch.arange(tokens)).reshape(-1), dtype)
    return {"cos": cos.reshape(len(positions), tokens, -1), "sin": sin.reshape(len(positions), tokens, -1),
            "position": position, "active": on.float(), "accepted": torch.as_tensor(accepted, dtype=torch.int32)}


def mtp_step_inputs(cfg, indices, tokens: int, max_seq_len: int, dtype, active) -> dict:
    """generate.py:90-99: verify inputs at the MTP indices (same bounds), with cos/sin one position on."""
    out = verify_inputs(cfg, indices, tokens, max_seq_len, dtype, active, [0] * len(indices))
    del out["accepted"]
    at = (torch.as_tensor(indices, dtype=torch.int32).unsqueeze(-1) + 1 + torch.arange(tokens)).reshape(-1)
    cos, sin = rotary(cfg, at, dtype)
    out["cos"], out["sin"] = cos.reshape(len(indices), tokens, -1), sin.reshape(len(indices), tokens, -1)
    return out


def mtp_prefill_inputs(cfg, slot: int, start: int, n_valid: int, chunk: int, dtype) -> dict:
    """generate.py:102-107: prefill inputs from MTP index ``start``, with cos/sin one position on."""
    out = prefill_inputs(cfg, slot, start, n_valid, chunk, dtype)
    cos, sin = rotary(cfg, start + 1 + torch.arange(chunk), dtype)
    out["cos"], out["sin"] = cos.unsqueeze(0), sin.unsqueeze(0)
    return out


# ----------------------------------------------------------------------------------------------- prompt lookup


def lookup_draft(history: Sequence[int], count: int, max_match: int = 4, min_match: int = 1) -> list[int]:
    """drafting.py:11-24: for n from ``max_match`` (at most len - 1) down to ``min_match``, the latest earlier start
    of the history's last n tokens; the first n with such a start drafts the up to ``count`` tokens after it. Empty
    when no length matches."""
    tokens = list(history)
    size = len(tokens)
    for n in range(min(max_match, size - 1), min_match - 1, -1):
        tail = tokens[size - n :]
        for start in range(size - n - 1, -1, -1):
            if tokens[start : start + n] == tail:
                return tokens[start + n : start + n + count]
    return []


# ----------------------------------------------------------------------------------------------- graph adapters


class Step:
    """`Qwen38Step.forward` (model.py:983-995) over the oracle: verify with ``accepted``, prefill with ``slot``, else
    decode. ``states`` are the per-layer dicts `oracle.model` updates in place."""

    def __init__(self, cfg, layers: list, states: list):
        self.cfg, self.layers, self.states = cfg, layers, states

    def __call__(self, inputs_embeds, cos=None, sin=None, position=None, active=None, accepted=None, slot=None, start=None,
                 n_valid=None):
        if slot is not None:
            return om.step_prefill(self.cfg, self.layers, self.states, inputs_embeds, cos, sin, slot, start, n_valid)
        if accepted is not None:
            return om.step_verify(self.cfg, self.layers, self.states, inputs_embeds, cos, sin, position, active, accepted)
        return om.step_decode(self.cfg, self.layers, self.states, inputs_embeds, cos, sin, position, active)


class MTP:
    """`MTPStep.forward` (model.py:843-860) over the oracle: the step form, or the prefill form with ``slot``."""

    def __init__(self, cfg, weights: dict, state: dict):
        self.cfg, self.weights, self.state = cfg, weights, state

    def __call__(self, hidden, inputs_embeds, cos, sin, position=None, active=None, slot=None, start=None, n_valid=None):
        if slot is not None:
            return om.mtp_prefill(self.cfg, self.weights, self.state, hidden, inputs_embeds, cos, sin, slot, start, n_valid)
        return om.mtp_forward(self.cfg, self.weights, self.state, hidden, inputs_embeds, cos, sin, position, active)


class ChipHead:
    """`ChipHead` (generate.py:162-208) with `HeadStep`'s CPU branch as its graph: rows padded to ``batch_size`` for the
    graph (the padding can change float32 sums, so it is kept), group maxima, then the exact recheck."""

    def __init__(self, cfg, norm_weight, lm_head: om.FP8Weight, embed: torch.Tensor, batch_size: int, recheck_groups: int = 4):
        self.cfg, self.norm_weight, self.lm_head, self.embed = cfg, norm_weight, lm_head, embed
        self.batch_size, self.recheck_groups = batch_size, recheck_groups

    def embed_batch(self, token_ids: Sequence[int], dtype) -> torch.Tensor:
        return self.embed[torch.as_tensor(list(token_ids), dtype=torch.long)].unsqueeze(1).to(dtype)

    def next_tokens(self, hidden: torch.Tensor, recheck_groups: int | None = None) -> list[int]:
        rows = hidden.shape[0]
        full = torch.zeros(self.batch_size, 1, hidden.shape[-1], dtype=hidden.dtype)
        full[:rows] = hidden
        maxima = om.head_group_maxima(self.cfg, self.norm_weight, self.lm_head, full)
        return om.chip_next_tokens(self.cfg, self.norm_weight, self.lm_head, hidden, maxima, recheck_groups or self.recheck_groups)


class HostHead(ChipHead):
    """`HostHead.next_tokens` (generate.py:156-159): argmax over the whole vocabulary; ``recheck_groups`` is ignored."""

    def next_tokens(self, hidden: torch.Tensor, recheck_groups: int | None = None) -> list[int]:
        return om.host_next_tokens(self.cfg, self.norm_weight, self.lm_head, hidden)


# ----------------------------------------------------------------------------------------------- the scheduler


@dataclass
class Row:
    """One running sequence in a slot (scheduler.py:30-43): its tokens so far, how many are in the cache, and, with
    MTP drafts, its seed ``(hidden [n, H], tokens [n], first index, take)`` for the next step's drafts."""

    index: int
    ids: list
    prompt_len: int
    new: int = 0
    written: int = 0
    seed: tuple | None = None


class Scheduler:
    """The reference's `Scheduler` with a verify graph (scheduler.py:45-301), single-turn prompts, no prefix reuse.

    ``decode``/``prefill``/``verify``/``mtp`` are callables with the reference's keyword forms; ``head`` has
    ``embed_batch`` and ``next_tokens``. Without ``verify`` every step is a one-token decode step."""

    def __init__(self, decode: Callable | None, prefill: Callable | None, head, cfg, batch_size: int, max_seq_len: int,
                 chunk: int, eos_token_ids=(), dtype=torch.bfloat16, verify: Callable | None = None, verify_tokens: int = 1,
                 mtp: Callable | None = None):
        self.decode, self.prefill, self.head, self.cfg = decode, prefill, head, cfg
        self.batch_size, self.max_seq_len, self.chunk, self.dtype = batch_size, max_seq_len, chunk, dtype
        self.eos = set(eos_token_ids)
        self.verify = verify
        self.k = verify_tokens if verify else 1
        self.mtp = mtp if verify else None
        # The accepted count each slot's next verify step commits, and counters (scheduler.py:97-103).
        self.accepted = [0] * batch_size
        self.drafted_tokens = 0
        self.decode_calls = 0

    # -------------------------------------------------------------------------------------- speculative step

    def mtp_drafts(self, slots: Sequence[Row | None]) -> dict[int, list[int]]:
        """scheduler.py:160-193. Rows with a seed are active: their seed's hidden states and tokens fill the first rows
        of a [K]-token call at their seed index; the output at ``take`` drafts the first token. Each later draft comes
        from a call at index ``first + take + 1 + j`` on ``[previous output, 0...]`` with ``[previous draft, 0...]``.
        The head rechecks one group per draft."""
        k, batch, size = self.k, self.batch_size, self.cfg.hidden_size
        hidden = torch.zeros(batch, k, size, dtype=self.dtype)
        ids = [[0] * k for _ in range(batch)]
        first, take, on = [0] * batch, [0] * batch, [False] * batch
        for slot, row in enumerate(slots):
            if row is not None and row.seed is not None:
                seed_hidden, seed_ids, first[slot], take[slot] = row.seed
                hidden[slot, : seed_hidden.shape[0]] = seed_hidden
                ids[slot][: len(seed_ids)] = seed_ids
                on[slot] = True
        running = [slot for slot in range(batch) if on[slot]]
        drafts: dict[int, list[int]] = {slot: [] for slot in running}
        embeds = self.head.embed_batch([t for row in ids for t in row], self.dtype).reshape(batch, k, -1)
        out = self.mtp(hidden=hidden, inputs_embeds=embeds, **mtp_step_inputs(self.cfg, first, k, self.max_seq_len, self.dtype, on))
        current = out[torch.arange(batch), torch.tensor(take)]
        for j in range(k - 1):
            picked = self.head.next_tokens(current[running].unsqueeze(1), recheck_groups=1)
            for slot, token in zip(running, picked):
                drafts[slot].append(token)
            if j == k - 2:
                break
            hidden = torch.zeros(batch, k, size, dtype=self.dtype)
            hidden[:, 0] = current
            ids = [[drafts[slot][-1] if on[slot] else 0] + [0] * (k - 1) for slot in range(batch)]
            embeds = self.head.embed_batch([t for row in ids for t in row], self.dtype).reshape(batch, k, -1)
            at = [first[slot] + take[slot] + 1 + j for slot in range(batch)]
            current = self.mtp(hidden=hidden, inputs_embeds=embeds,
                               **mtp_step_inputs(self.cfg, at, k, self.max_seq_len, self.dtype, on))[:, 0]
        return drafts

    def verify_step(self, slots: Sequence[Row | None], positions, active, ready) -> list[list[int]]:
        """scheduler.py:269-301. Drafts from the MTP layer when there is one, else from each row's own history
        (`lookup_draft`, padded to K - 1 with the row's last token). Returns each ready slot's new tokens (the matching
        drafts, then the model's own next pick); with MTP it leaves each ready row's next seed ``(hidden [K, H], picks,
        position, match)``. ``last`` keeps the step's drafts, hidden states, picks and matches."""
        k = self.k
        if self.mtp:
            drafts = self.mtp_drafts(slots)
        else:
            drafts = {}
            for slot, row in enumerate(slots):
                if row is not None:
                    found = lookup_draft(row.ids, k - 1)
                    drafts[slot] = found + [row.ids[-1]] * (k - 1 - len(found))
        tokens = []
        for slot, row in enumerate(slots):
            tokens += [row.ids[-1]] + drafts[slot] if row is not None else [0] * k
        accepted = [self.accepted[slot] if slots[slot] is not None else 0 for slot in range(self.batch_size)]
        embeds = self.head.embed_batch(tokens, self.dtype).reshape(self.batch_size, k, -1)
        hidden = self.verify(inputs_embeds=embeds,
                             **verify_inputs(self.cfg, positions, k, self.max_seq_len, self.dtype, active, accepted))
        chosen = self.head.next_tokens(hidden[ready].reshape(len(ready) * k, 1, -1))
        emitted, picked, matched = [], {}, {}
        for i, slot in enumerate(ready):
            picks, draft = chosen[i * k : (i + 1) * k], drafts[slot]
            match = 0
            while match < k - 1 and draft[match] == picks[match]:
                match += 1
            self.accepted[slot] = match + 1
            self.drafted_tokens += match
            emitted.append(picks[: match + 1])
            picked[slot], matched[slot] = picks, match
            if self.mtp:
                slots[slot].seed = (hidden[slot], picks, positions[slot], match)
        self.last = {"drafts": drafts, "hidden": hidden, "chosen": chosen, "picks": picked, "match": matched}
        return emitted

    # -------------------------------------------------------------------------------------- prompts and the run loop

    def _prefill(self, slot: int, row: Row) -> int:
        """scheduler.py:110-141 without prefix reuse: the prompt in chunks (and through the MTP layer's prefill form),
        then the first new token from the last real position."""
        hidden, last, n_valid = None, None, 0
        for start in range(0, row.prompt_len, self.chunk):
            ids = row.ids[start : start + self.chunk]
            n_valid = len(ids)
            embeds = self.head.embed_batch(ids + [0] * (self.chunk - n_valid), self.dtype).reshape(1, self.chunk, -1)
            hidden = self.prefill(inputs_embeds=embeds, **prefill_inputs(self.cfg, slot, start, n_valid, self.chunk, self.dtype))
            if self.mtp:
                last = self._mtp_prefill(slot, start, n_valid, embeds, hidden, last)
        self.accepted[slot] = 0
        row.written = row.prompt_len
        token = self.head.next_tokens(hidden[:, n_valid - 1 : n_valid])[0]
        if self.mtp:
            row.seed = (last[0], [token], row.prompt_len - 1, 0)
        return token

    def _mtp_prefill(self, slot: int, start: int, n_valid: int, embeds, hidden, last):
        """scheduler.py:143-158: MTP index t pairs hidden t with token t + 1, so a chunk at ``start`` covers indices
        from ``start - 1`` (from the last chunk's final hidden ``last``); the first chunk covers one index fewer."""
        if start == 0 or last is None:
            first, states = start, hidden[:, : n_valid - 1]
            embeds = torch.cat((embeds[:, 1:], embeds[:, :1]), dim=1)
        else:
            first, states = start - 1, torch.cat((last, hidden[:, : n_valid - 1]), dim=1)
        if states.shape[1]:
            pad = torch.zeros(1, self.chunk - states.shape[1], states.shape[-1], dtype=states.dtype)
            self.mtp(hidden=torch.cat((states, pad), dim=1), inputs_embeds=embeds,
                     **mtp_prefill_inputs(self.cfg, slot, first, n_valid - (first == start), self.chunk, self.dtype))
        return hidden[:, n_valid - 1 : n_valid]

    def _finished(self, row: Row, token: int, max_new_tokens: int) -> bool:
        """scheduler.py:195-197."""
        return token in self.eos or row.new >= max_new_tokens or row.written + self.k > self.max_seq_len - self.chunk

    def run(self, prompts: Sequence[Sequence[int]], max_new_tokens: int) -> Iterator[tuple[int, int]]:
        """scheduler.py:199-267 for single-turn prompts: fill free slots by prefill, then one decode or verify step over
        every running slot; yields (prompt index, token) in the order the reference yields them."""
        for prompt in prompts:
            if not prompt:
                raise ValueError("a prompt is empty")
            if len(prompt) >= self.max_seq_len - self.chunk:
                raise ValueError(f"a prompt of {len(prompt)} tokens leaves no room in max_seq_len {self.max_seq_len}")
        waiting = list(range(len(prompts)))[::-1]
        slots: list[Row | None] = [None] * self.batch_size
        while waiting or any(slots):
            for slot in range(self.batch_size):
                while slots[slot] is None and waiting:
                    p = waiting.pop()
                    row = Row(p, list(prompts[p]), len(prompts[p]))
                    token = self._prefill(slot, row)
                    row.new = 1
                    row.ids.append(token)
                    yield p, token
                    if not self._finished(row, token, max_new_tokens):
                        slots[slot] = row
            if not any(slots):
                continue
            positions = [row.written if row else 0 for row in slots]
            active = [row is not None for row in slots]
            ready = [slot for slot, row in enumerate(slots) if row]
            if self.verify:
                emitted = self.verify_step(slots, positions, active, ready)
            else:
                last = [row.ids[-1] if row else 0 for row in slots]
                hidden = self.decode(inputs_embeds=self.head.embed_batch(last, self.dtype),
                                     **batch_step_inputs(self.cfg, positions, self.max_seq_len, self.dtype, active))
                emitted = [[token] for token in self.head.next_tokens(hidden[ready])]
            self.decode_calls += 1
            for slot, tokens in zip(ready, emitted):
                row = slots[slot]
                for token in tokens:
                    row.written += 1
                    row.new += 1
                    row.ids.append(token)
                    yield row.index, token
                    if self._finished(row, token, max_new_tokens):
                        slots[slot] = None
                        break
