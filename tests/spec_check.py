"""Speculative steps driven from the host and recorded, and the proofs that tie every number and every decision of
such a step to the oracle (oracle/model.py, oracle/scheduler.py).

The restated scheduler (`oracle.scheduler.Scheduler`, pinned to the reference's own) drives this build's step objects
on one engine through recording wrappers: `RecordingVerify` (around `VerifyStep`), `RecordingMTP` (around `MTPStep`)
and `RecordingHead` (a `HeadGraph` whose picks are kept). Each recorded call keeps its inputs, the engine's state
before and after it, every layer's probe and its output. The device's own step (`q38_spec_step`, `q38_verify_step`)
is then held equal to that run bit for bit, so what is proven about the recorded calls holds for the device's step.

The proofs, per call:
* verify (`check_verify`): every decoder layer against the oracle from the GPU's own input to it and its own state
  before the call, stage by stage (tests/layerwise.py): every differing rounding a tie, each layer's output within
  2e-2 per token, every committed state vector within 1e-2;
* MTP (`check_mtp`): the fc output from the GPU's inputs within 2e-2 per token, the attention layer teacher-forced as a
  verify layer, and the output tail (final norm over 1 + the head's norm weight) from the GPU's own layer stages;
* head (`check_head`): the normed rows equal the oracle's up to proven rounding ties, the group maxima from them within
  1e-4 of the largest, and every pick equal to the oracle's pick from the same hidden row, or else explained: the two picks' exact logits within 1e-3 (a top-2 near-tie), or the selection of
  rechecked groups tied at its boundary (the last rechecked and the next group maxima within the maxima's tolerance)
  with the GPU's group at that boundary;
* acceptance (`check_acceptance`): the matches and accepted counts are the oracle's acceptance of the GPU's picks and
  drafts, exactly.
Together: each pick, draft and accepted count is the oracle's decision on numbers that are themselves proven equal to
the oracle's up to rounding ties, so no difference from the all-CPU oracle is left unexplained. `oracle_chain` runs
the all-CPU oracle over a recorded verify call from its starting state, for the un-forced drift, which is reported.

Weights: `OracleWeights` gives each layer's oracle weights on demand, from a dict of CPU values or by regenerating the
layer's seeded weights on the GPU (exact dequantization there, spot-checked against the oracle's own decoding), so a
27B model needs one layer's weights on the host at a time.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

from layerwise import HIDDEN_TOL, MODE_TOL, STATE_NAMES, STATE_TOL, attention_layer_errors, gdn_layer_errors, rel_rows
from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import FULL, LINEAR, with_layers
from qwen38_amd.quant import dequantize_e4m3
from qwen38_amd.steps import DTYPE, Engine, HeadGraph, MTPStep, VerifyStep

MAXIMA_TOL, GAP_TOL = 1e-4, 1e-3


# ----------------------------------------------------------------------------------------------- oracle weights


def oracle_fp8(value) -> om.FP8Weight:
    """An (e4m3, E8M0) pair as the oracle's weight; a GPU pair is dequantized there (exact) and the first rows checked
    against the oracle's own decoding of the bytes."""
    coded, scales = value
    if not coded.is_cuda:
        return om.FP8Weight(coded, scales)
    dense_t = dequantize_e4m3(coded, scales).T.contiguous().cpu()
    w = om.FP8Weight(coded.cpu(), scales.cpu(), dense_t)
    rows = slice(0, min(64, coded.shape[0]))
    assert torch.equal(w.decoded_t(rows), dense_t[:, rows]), "GPU dequantization differs from the oracle's"
    return w


def _oracle_value(v):
    return oracle_fp8(v) if isinstance(v, tuple) else v.cpu()


class OracleWeights:
    """Oracle weights of a model, layer by layer. ``values`` (name -> value, e.g. `synth.make_all` on the CPU) or, for
    models too large to hold, ``seed`` to regenerate each layer's seeded weights on the GPU (`synth.make`) with the
    head replaced by ``head`` (name -> value for ``head.*`` and ``embed_tokens``, as loaded)."""

    def __init__(self, cfg, values: dict | None = None, seed: int | None = None, head: dict | None = None):
        self.cfg, self.values, self.seed = cfg, values, seed
        self._head_values = head if head is not None else {n: v for n, v in (values or {}).items() if n.startswith("head.") or n == "embed_tokens"}
        self._head = None
        self._mtp = None

    def _made(self, specs) -> dict:
        if self.values is not None:
            return {s.name: self.values[s.name] for s in specs}
        return {s.name: synth.make(s, self.seed, "cuda") for s in specs}

    def layer(self, i: int) -> dict:
        prefix = f"layers.{i}."
        made = self._made(synth.layer_specs(self.cfg, i))
        return {n[len(prefix):]: _oracle_value(v) for n, v in made.items()}

    def mtp(self) -> dict:
        """The MTP layer's weights with `oracle.model.mtp_forward`'s names."""
        if self._mtp is None:
            made = self._made(synth.mtp_specs(self.cfg))
            w = {n[len("mtp."):]: _oracle_value(v) for n, v in made.items()}
            w["final_norm_weight"] = self._head_values["head.norm_weight"].cpu()
            self._mtp = w
        return self._mtp

    def head(self) -> SimpleNamespace:
        """norm_weight, lm_head (FP8Weight), rows (the bf16 rows the recheck reads: the e4m3 values, exact in bf16)."""
        if self._head is None:
            lm = oracle_fp8(self._head_values["head.lm_head"])
            self._head = SimpleNamespace(norm_weight=self._head_values["head.norm_weight"].cpu(), lm_head=lm,
                                         rows=lm.dense_t().T.contiguous().to(torch.bfloat16))
        return self._head


# ----------------------------------------------------------------------------------------------- recording


def _gdn_reference(engine: Engine, i: int) -> dict:
    """Layer i's current gated-delta state, cloned, in the reference's shapes (pending keys per value head)."""
    st = {k: v.clone() for k, v in engine.gdn_state(i).items()}
    st["pending_key_state"] = om.repeat_interleave(st["pending_key_state"], engine.cfg.linear_key_repeat, dim=2).contiguous()
    return st


def _kv_reference(engine: Engine, i: int) -> dict:
    kc, vc = engine.get_kv(i)
    return {"k_cache": kc, "v_cache": vc}


def snapshot(engine: Engine, layers) -> dict:
    """Clones (on the GPU) of the given layers' states in the reference's shapes."""
    return {i: (_gdn_reference(engine, i) if i < engine.cfg.num_hidden_layers and engine.cfg.layer_types[i] == LINEAR
                else _kv_reference(engine, i)) for i in layers}


def _cpu(t):
    return t.detach().cpu() if isinstance(t, torch.Tensor) else t


class Recorder:
    """Recording wrappers around one engine's verify, MTP and head calls. ``keep_verify(n)`` / ``keep_mtp(n)`` say
    which calls (0-based, in call order) keep their states and probes (the heavy parts); head calls are always kept."""

    def __init__(self, engine: Engine, keep_verify=lambda n: True, keep_mtp=lambda n: True):
        self.engine = engine
        self.verify_calls, self.mtp_calls, self.head_calls = [], [], []
        self.keep_verify, self.keep_mtp = keep_verify, keep_mtp
        cfg = engine.cfg
        for i in range(cfg.num_hidden_layers):
            engine.enable_probe(i)
        if engine.mtp:
            engine.enable_probe(engine.mtp_layer)
        engine.enable_head_probe()
        self.verify = RecordingVerify(self)
        self.mtp = RecordingMTP(self) if engine.mtp else None
        self.head = RecordingHead(self)


class RecordingVerify:
    def __init__(self, rec: Recorder):
        self.rec, self.step = rec, VerifyStep(rec.engine)

    def __call__(self, inputs_embeds, **inputs):
        e, n = self.rec.engine, len(self.rec.verify_calls)
        layers = range(e.cfg.num_hidden_layers)
        keep = self.rec.keep_verify(n)
        before = snapshot(e, layers) if keep else None
        out = self.step(inputs_embeds=inputs_embeds, **inputs)
        call = {"inputs": {k: _cpu(v) for k, v in inputs.items()}, "embeds": _cpu(inputs_embeds), "out": out.clone()}
        if keep:
            call.update(before=before, after=snapshot(e, layers),
                        probes={i: e.buffer("probe", i).clone() for i in layers})
        self.rec.verify_calls.append(call)
        return out


class RecordingMTP:
    def __init__(self, rec: Recorder):
        self.rec, self.step = rec, MTPStep(rec.engine)

    def __call__(self, hidden, inputs_embeds, **inputs):
        e, n = self.rec.engine, len(self.rec.mtp_calls)
        keep = self.rec.keep_mtp(n)
        m = e.mtp_layer
        before = snapshot(e, [m])[m] if keep else None
        out = self.step(hidden=hidden, inputs_embeds=inputs_embeds, **inputs)
        call = {"inputs": {k: _cpu(v) for k, v in inputs.items()}, "hidden": _cpu(hidden), "embeds": _cpu(inputs_embeds),
                "out": out.clone()}
        if keep:
            call.update(before=before, after=snapshot(e, [m])[m], probe=e.buffer("probe", m).clone())
        self.rec.mtp_calls.append(call)
        return out


class RecordingHead(HeadGraph):
    def __init__(self, rec: Recorder):
        super().__init__(rec.engine)
        self.rec = rec

    def pick(self, hidden: torch.Tensor, groups: int) -> torch.Tensor:
        ids = super().pick(hidden, groups)
        maxima = self(hidden)
        rows = hidden.reshape(-1, self.engine.cfg.hidden_size).shape[0]
        self.rec.head_calls.append({"hidden": _cpu(hidden).reshape(-1, 1, self.engine.cfg.hidden_size), "groups": groups,
                                    "ids": ids.tolist(), "maxima": maxima.cpu(), "normed": self.engine.head_probe(rows).cpu()})
        return ids


# ----------------------------------------------------------------------------------------------- proofs


def _args(inputs: dict):
    return inputs["cos"], inputs["sin"], inputs["position"], inputs["active"], inputs["accepted"]


def _log_errors(log, label: str, errs: dict, worst: dict) -> None:
    for name, e in errs.items():
        if name.startswith("_"):
            continue
        top = float(e.max())
        worst[name] = max(worst.get(name, 0.0), top)
        tol = STATE_TOL if name in STATE_NAMES else HIDDEN_TOL
        if name in STATE_NAMES or top > tol / 4:
            log(f"  {label} {name}: max {top:.3g} median {float(e.median()):.3g} above {tol:g}: {int((e > tol).sum())}/{e.numel()}")
    for note in errs.get("_notes", []):
        if "differing 0 " not in note:
            log(f"  {label} {note}")


def _cpu_state(st: dict) -> dict:
    return {k: v.cpu() for k, v in st.items()}


def check_verify(engine: Engine, weights: OracleWeights, call: dict, layers=None, own: bool = False, log=print) -> dict:
    """Every layer in ``layers`` (default all) of a recorded verify call against the oracle from the GPU's own input
    and state (tests/layerwise.py); asserts the stage checks and returns the worst error per quantity."""
    cfg = engine.cfg
    b, k, h = engine.batch_size, engine.verify_tokens, cfg.hidden_size
    inputs = call["inputs"]
    args = _args(inputs)
    tol = MODE_TOL[engine.projection_mfma]
    stack = SimpleNamespace(cfg=cfg, batch=b, tokens=k, max_seq_len=engine.max_seq_len)
    probes = {i: {n: t.cpu() for n, t in engine.probe(i, call["probes"][i]).items()} for i in (layers or range(cfg.num_hidden_layers))}
    worst: dict[str, float] = {}
    last = cfg.num_hidden_layers - 1
    for i in sorted(probes):
        kind = cfg.layer_types[i]
        one = with_layers(cfg, (kind,))
        w = weights.layer(i)
        probe = probes[i]
        x = probe["input"].reshape(b, k, h)
        y = (call["out"].cpu() if i == last else engine.probe(i + 1, call["probes"][i + 1])["input"].cpu()).reshape(b, k, h)
        if i == 0:
            assert torch.equal(x, call["embeds"].reshape(b, k, h).to(DTYPE)), "layer 0's input is not the step's embeddings"
        before, after = _cpu_state(call["before"][i]), _cpu_state(call["after"][i])
        if kind == LINEAR:
            errs = gdn_layer_errors(one, w, x, y, probe, after, before, args, tol, own=own)
        else:
            errs = attention_layer_errors(stack, one, w, x, y, probe, after, before, args, inputs, i, tol, own=own)
        _log_errors(log, f"layer {i} {kind[:6]}", errs, worst)
        for name, e in errs.items():
            if name.startswith("_") or name == "hidden_own":
                continue
            limit = STATE_TOL if name in STATE_NAMES else HIDDEN_TOL
            assert float(e.max()) <= limit, f"layer {i} {name}: {float(e.max()):.3g} above {limit:g}"
    return worst


def mtp_tail(cfg, w: dict, y: torch.Tensor) -> torch.Tensor:
    """`MTPStep.forward`'s output from the layer output (model.py:858-860): rms norm, then divided by 1 + the final
    norm's weight in float32, rounded to bf16."""
    out = om.rms_norm(y, w["norm_weight"], cfg.rms_norm_eps)
    return (out.float() / (1.0 + w["final_norm_weight"].float())).to(y.dtype)


def check_mtp(engine: Engine, weights: OracleWeights, call: dict, log=print) -> dict:
    """A recorded MTP call: the fc output (the layer's probed input) against the oracle's from the GPU's inputs, within
    2e-2 per token; the full-attention layer teacher-forced like a verify layer (its cache writes included); the output
    against the oracle's tail from the GPU's own mixer output and down-projection input, within 2e-2 per token."""
    cfg = engine.cfg
    b, k, h = engine.batch_size, engine.verify_tokens, cfg.hidden_size
    w = weights.mtp()
    eps = cfg.rms_norm_eps
    inputs = dict(call["inputs"])
    inputs["accepted"] = inputs["active"]  # mtp_forward runs its layer with accepted=active (model.py:857)
    probe = {n: t.cpu() for n, t in engine.probe(engine.mtp_layer, call["probe"]).items()}
    hidden, embeds = call["hidden"].to(DTYPE), call["embeds"].to(DTYPE)
    joined = torch.cat((om.rms_norm(embeds, w["embedding_norm_weight"], eps),
                        om.rms_norm(om.rms_norm(hidden, w["final_norm_weight"], eps), w["hidden_norm_weight"], eps)), dim=-1)
    x_gpu = probe["input"].reshape(b, k, h)
    fc = rel_rows(x_gpu, om.linear_fp8(joined, w["fc"]), h)
    layer_w = {n[len("layer."):]: t for n, t in w.items() if n.startswith("layer.")}
    one = with_layers(cfg, (FULL,))
    stack = SimpleNamespace(cfg=cfg, batch=b, tokens=k, max_seq_len=engine.max_seq_len)
    tol = MODE_TOL[engine.projection_mfma]
    # The layer output is not probed (the MTP output is its tail); stand in the oracle's output from the GPU's own
    # stages, which the tail check below then holds the GPU's output to.
    y_forced = (probe["mixed"] + om.linear_fp8(probe["ffn"], layer_w["mlp.down_proj"])).reshape(b, k, h)
    errs = attention_layer_errors(stack, one, layer_w, x_gpu, y_forced, probe, _cpu_state(call["after"]),
                                  _cpu_state(call["before"]), _args(inputs), inputs, engine.mtp_layer, tol, own=False)
    errs["fc"] = fc
    errs["tail"] = rel_rows(call["out"], mtp_tail(cfg, w, y_forced), h)
    worst: dict[str, float] = {}
    _log_errors(log, "MTP", errs, worst)
    for name, e in errs.items():
        if name.startswith("_"):
            continue
        limit = STATE_TOL if name in STATE_NAMES else HIDDEN_TOL
        assert float(e.max()) <= limit, f"MTP {name}: {float(e.max()):.3g} above {limit:g}"
    return worst


def head_logits(cfg, head: SimpleNamespace, hidden: torch.Tensor) -> torch.Tensor:
    """`HeadStep.forward`'s CPU logits (model.py:890-895): float32 ``[R, V]``."""
    x = om.rms_norm(hidden, head.norm_weight, cfg.rms_norm_eps).reshape(hidden.shape[0], -1)
    return x.float() @ head.lm_head.dense_t()


def check_head(cfg, head: SimpleNamespace, call: dict, log=print) -> dict:
    """A recorded head call, teacher-forced at the final norm: the GPU's normed rows equal the oracle's norm of the
    same hidden rows except at proven rounding ties (`layerwise.norm_ties`); the group maxima within 1e-4 of the row's
    largest magnitude of the oracle's maxima from the GPU's normed rows; each pick the oracle's (`chip_next_tokens`
    from the same hidden rows, with those maxima choosing the groups), or explained as a near-tie of the two picks'
    exact logits (under 1e-3) or of the group ranking (the GPU's group's maximum within the maxima tolerance of the
    oracle's last rechecked group). Returns counts."""
    from layerwise import norm_ties

    hidden, groups, got = call["hidden"].to(DTYPE), call["groups"], call["ids"]
    normed = call["normed"]
    ties = norm_ties(hidden, head.norm_weight, cfg.rms_norm_eps, normed, om.rms_norm(hidden, head.norm_weight, cfg.rms_norm_eps))
    logits = normed.float() @ head.lm_head.dense_t()
    maxima = torch.stack([g.amax(dim=-1) for g in logits.split(32, dim=-1)], dim=-1)
    scale = maxima.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    off = float(((call["maxima"] - maxima).abs() / scale).max())
    assert off <= MAXIMA_TOL, f"head maxima off by {off:.3g} of the row's largest"
    want = om.chip_next_tokens(cfg, head.norm_weight, head.lm_head, hidden, maxima, groups, rows_bf16=head.rows)
    norm = om.rms_norm(hidden.float(), head.norm_weight, cfg.rms_norm_eps).squeeze(1)
    explained = []
    for r, (g, o) in enumerate(zip(got, want)):
        if g == o:
            continue
        exact = head.rows[[g, o]].float() @ norm[r]
        gap = float((exact[1] - exact[0]).abs())
        # The groups rechecked are the top `groups` maxima; where the last of them and the next are within the maxima's
        # tolerance, the GPU may recheck either, so its pick may come from any group that close to the boundary.
        ranked = maxima[r].sort(descending=True).values
        slack = MAXIMA_TOL * float(scale[r])
        boundary = float(ranked[groups - 1])
        ambiguous = groups < len(ranked) and float(ranked[groups]) >= boundary - slack
        group_tie = ambiguous and float(maxima[r, g // 32]) >= boundary - slack
        assert gap < GAP_TOL or group_tie, (f"row {r}: GPU pick {g}, oracle pick {o}, exact logits {exact.tolist()}, "
                                            f"group maxima {float(maxima[r, g // 32]):.6g} vs rechecked boundary {boundary:.6g}")
        explained.append((r, g, o, gap, group_tie))
    if explained:
        log(f"  head ({len(got)} rows, {groups} groups): {len(explained)} picks differ, each a near-tie: {explained}")
    return {"rows": len(got), "differ": len(explained), "maxima_off": off, "norm_ties": ties}


def check_acceptance(picks: list, drafts: list, match: int, k: int) -> None:
    """The oracle's greedy acceptance (scheduler.py:291-298) of the GPU's picks and drafts gives the GPU's match."""
    want, _ = om.accept(list(picks), list(drafts), k)
    assert want == match, (picks, drafts, match, want)


class reordered_sums:
    """Within this context the oracle's FP8 projections take their float32 sums over the inputs in reverse order
    (a float32 matmul of the reversed inputs, then the bf16 rounding): a second correct evaluation of the reference's
    semantics, which differs from the first only where a sum's float32 rounding differs. Run against the plain oracle,
    it shows how far two correct evaluations of the 64-layer chain drift apart through the reference's e5m2 input
    roundings."""

    def __enter__(self):
        self.original = om.linear_fp8

        def linear(x, weight):
            x = om.fp8_round(x)
            return (x.flip(-1).float() @ weight.dense_t().flip(0)).to(x.dtype)

        om.linear_fp8 = linear
        return self

    def __exit__(self, *exc):
        om.linear_fp8 = self.original
        return False


def oracle_chain(engine: Engine, weights: OracleWeights, call: dict) -> torch.Tensor:
    """The all-CPU oracle's verify over a recorded call from the call's starting state: its hidden states [B, K, H]."""
    cfg = engine.cfg
    inputs = call["inputs"]
    x = call["embeds"].to(DTYPE)
    for i, kind in enumerate(cfg.layer_types):
        st = _cpu_state(call["before"][i])
        x = om.decoder_layer(cfg, kind, weights.layer(i), st, x, *_args(inputs))
    return x


# ----------------------------------------------------------------------------------------------- driving the steps


class DeviceStep:
    """The device state `q38_spec_step` carries from step to step, started as a prefill of each prompt leaves a row
    (``start[b]``: {"ids", "prompt_len", "hidden"} or None): the prompt's last hidden state and first new token as the
    MTP seed at index prompt_len - 1, position prompt_len, nothing to commit."""

    def __init__(self, engine: Engine, start: list):
        self.engine = engine
        b, k, h = engine.batch_size, engine.verify_tokens, engine.cfg.hidden_size
        position, index = torch.zeros(b, dtype=torch.int32), torch.zeros(b, dtype=torch.int32)
        active, hidden, picks = torch.zeros(b), torch.zeros(b, k, h, dtype=DTYPE), torch.zeros(b, k, dtype=torch.int32)
        for slot, row in enumerate(start):
            if row is not None:
                position[slot], index[slot], active[slot] = row["prompt_len"], row["prompt_len"] - 1, 1.0
                hidden[slot, 0] = row["hidden"].reshape(-1)
                picks[slot, 0] = row["ids"][-1]
        dev = engine.device
        self.position, self.index, self.active = position.to(dev), index.to(dev), active.to(dev)
        self.hidden, self.picks = hidden.to(dev), picks.to(dev)
        self.match = torch.zeros(b, dtype=torch.int32, device=dev)
        self.accepted = torch.zeros(b, dtype=torch.int32, device=dev)
        self.drafts = torch.zeros(b, k - 1, dtype=torch.int32, device=dev)

    def __call__(self, graph: bool = False):
        self.engine.handle.spec_step(self.position, self.index, self.match, self.accepted, self.active, self.hidden, self.picks,
                                     self.drafts, graph=graph)
        torch.cuda.synchronize()


def host_slots(start: list, mtp: bool = True) -> list:
    """The restated scheduler's rows for the same starting point (with the MTP seed when ``mtp``)."""
    from oracle import scheduler as osch

    slots = []
    for row in start:
        if row is None:
            slots.append(None)
            continue
        r = osch.Row(0, list(row["ids"]), row["prompt_len"], written=row["prompt_len"])
        if mtp:
            r.seed = (row["hidden"].reshape(1, -1), [row["ids"][-1]], row["prompt_len"] - 1, 0)
        slots.append(r)
    return slots


def run_host_step(sched, slots) -> tuple[list, list, list]:
    """One `Scheduler.verify_step` over the running slots; appends the emitted tokens. Returns (positions, ready,
    emitted)."""
    positions = [row.written if row else 0 for row in slots]
    active = [row is not None for row in slots]
    ready = [slot for slot, row in enumerate(slots) if row]
    with torch.no_grad():
        emitted = sched.verify_step(slots, positions, active, ready)
    for slot, tokens in zip(ready, emitted):
        slots[slot].ids += tokens
        slots[slot].written += len(tokens)
    return positions, ready, emitted


def prove_step(engine: Engine, weights: OracleWeights, rec: Recorder, last: dict, first_head: int, first_mtp: int,
               verify_call: int, log=print, layers=None) -> dict:
    """Every decision of one recorded speculative step: its MTP calls from ``first_mtp`` and head calls from
    ``first_head`` (K - 1 draft picks, then the verify's picks), its verify call (every layer in ``layers``), and its
    acceptance (``last``: the scheduler's record of the step). Returns the worst errors and head counts."""
    cfg = engine.cfg
    k = engine.verify_tokens
    worst: dict = {}
    if engine.mtp:
        for call in rec.mtp_calls[first_mtp : first_mtp + k - 2 + 1]:
            for key, v in check_mtp(engine, weights, call, log).items():
                worst["mtp " + key] = max(worst.get("mtp " + key, 0.0), v)
    for key, v in check_verify(engine, weights, rec.verify_calls[verify_call], layers, log=log).items():
        worst[key] = max(worst.get(key, 0.0), v)
    head = weights.head()
    counts = {"rows": 0, "differ": 0}
    n_heads = k if engine.mtp else 1
    for call in rec.head_calls[first_head : first_head + n_heads]:
        got = check_head(cfg, head, call, log)
        counts["rows"] += got["rows"]
        counts["differ"] += got["differ"]
    drafts, picks, match = last["drafts"], last["picks"], last["match"]
    for slot in picks:
        check_acceptance(picks[slot], drafts[slot], match[slot], k)
    worst["head"] = counts
    return worst
