"""Prompt-lookup drafts for the verify step when no MTP drafter is loaded: the reference's drafting.py API
(qwen38_inf2/drafting.py:11-74) for the host side of this build.

A row's next tokens are guessed from its own history: the tokens that followed the latest earlier occurrence of the
history's last n tokens, for the longest n from ``max_match`` down to ``min_match`` that occurred before. The
reference's `Scheduler._verify_step` (scheduler.py:276-282) keeps one `Drafter` per row, pads its draft to K - 1
tokens with the row's last token and hands them to the verify graph; here `steps.LookupStep` does the same around
`q38_verify_step`.

`Drafter` keeps one map from every n-gram (n <= max_match) that has been followed by a token to the index just past
its latest such occurrence, updated as tokens arrive, so a draft is at most ``max_match`` lookups; `lookup_draft`
is the plain scan it must agree with (the reference's own test, tests/test_scheduler.py:177-185, checks the same
equality for its class).
"""

from __future__ import annotations

from collections.abc import Sequence


def lookup_draft(history: Sequence[int], count: int, max_match: int = 4, min_match: int = 1) -> list[int]:
    """Up to ``count`` tokens that followed the latest earlier occurrence of the history's last n tokens, trying n from
    ``max_match`` (at most ``len(history) - 1``) down to ``min_match``; empty when none occurred (drafting.py:11-24)."""
    seq = list(history)
    end = len(seq)
    for n in range(min(max_match, end - 1), min_match - 1, -1):
        key = seq[end - n :]
        # An occurrence must end before the tail starts to be followed by something inside the history.
        for first in range(end - n - 1, -1, -1):
            if seq[first : first + n] == key:
                return seq[first + n : first + n + count]
    return []


class Drafter:
    """`lookup_draft` over a growing sequence (drafting.py:27-51): ``extend`` appends tokens, ``draft`` looks the tail
    up in the successor map instead of scanning."""

    def __init__(self, history: Sequence[int], max_match: int = 4, min_match: int = 1):
        self.tokens: list[int] = []
        self.max_match, self.min_match = max_match, min_match
        # n-gram (as a tuple, so its length is its n) -> index of the token that followed its latest occurrence.
        self._follower: dict[tuple, int] = {}
        self.extend(history)

    def extend(self, tokens: Sequence[int]) -> None:
        seq, follower = self.tokens, self._follower
        for token in tokens:
            at = len(seq)
            # Every n-gram ending here is now followed by `token`, at index `at`.
            for n in range(1, min(self.max_match, at) + 1):
                follower[tuple(seq[at - n :])] = at
            seq.append(token)

    def draft(self, count: int) -> list[int]:
        seq = self.tokens
        end = len(seq)
        for n in range(min(self.max_match, end - 1), self.min_match - 1, -1):
            at = self._follower.get(tuple(seq[end - n :]))
            if at is not None:
                return seq[at : at + count]
        return []


def padded_draft(drafter: Drafter, last: int, count: int) -> list[int]:
    """``count`` drafts for the verify step: the drafter's, then the row's last token repeated (scheduler.py:280-281)."""
    found = drafter.draft(count)
    return found + [last] * (count - len(found))


def accepted_per_step(history: Sequence[int], output: Sequence[int], draft_len: int) -> list[int]:
    """Tokens each verify step would emit if greedy decoding produced ``output`` after ``history`` with prompt-lookup
    drafts of ``draft_len``: the leading drafts that match, plus the model's own pick, capped by what is left
    (drafting.py:54-74)."""
    seen, out, done = list(history), list(output), 0
    steps = []
    while done < len(out):
        guess = lookup_draft(seen, draft_len)
        match = 0
        while match < len(guess) and done + match < len(out) and guess[match] == out[done + match]:
            match += 1
        take = min(match + 1, len(out) - done)
        steps.append(take)
        seen.extend(out[done : done + take])
        done += take
    return steps
