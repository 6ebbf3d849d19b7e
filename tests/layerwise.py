"""Per-layer teacher-forced parity: every decoder layer of a verify step runs on the GPU in a one-layer engine, and the
oracle recomputes that layer from the GPU's own input to it and the GPU's own state before the step, stage by stage at
the reference's rounding boundaries, each stage fed the GPU's own results of the stages before it (the engine's state
snapshots, and its per-layer probe: the normed input, the mixer's projection output, the residual after the mixer and
the three e5m2 GEMM inputs).

Why stages: the reference rounds every projection input to e5m2 (four values per octave). Two correct
implementations whose float32 sums run in different orders round a few values that sit exactly on a bf16 rounding tie
to opposite sides (0.005% of the GEMM outputs at the 27B shapes); the next e5m2 rounding turns that last-bit
difference into a difference of an e5m2 step, and a few such steps can move a token's layer output by several percent.
So each rounding stage is held to "equal, or a rounding tie":
* a bf16 GEMM output or norm output that differs must be, in both results, a correct bf16 rounding of a float32 value
  within eight float32 ulps of the exact (float64) value;
* an e5m2 GEMM input that differs must lie within the e5m2 roundings of the oracle's value moved by two bf16 steps of
  the token's typical element (what a tie in a bf16 term upstream can move it by), and at most one in a thousand may
  differ (for attention's output only the count: its bf16-rounded scores move a softmax weight by up to 1.6% at a tie,
  so the attention stage is held by its output per token);
* a decay or delta vector above 1e-2 must come from a gate projection a rounding tie apart (its bf16 value one step
  from the oracle's).
Every other stage, given identical inputs, is held to the north-star tolerances: 2e-2 per token of hidden state, 1e-2
per state vector. The plain distance of the layer output from the oracle with its own roundings throughout
(``hidden_own``) is reported alongside.

Error measures: relative 2-norm distance per token (a row of hidden state), per (row, value head) recurrent-state
matrix, per row of conv state, per (row, token) snapshot vector and per (row, head, position) KV vector.
"""

from __future__ import annotations

import torch

from oracle import model as om
from qwen38_amd import synth
from qwen38_amd.config import LINEAR, with_layers
from qwen38_amd.quant import decode_kv, encode_kv
from qwen38_amd.steps import Engine, VerifyStep

HIDDEN_TOL, STATE_TOL = 2e-2, 1e-2
STATE_NAMES = {"recurrent_state", "conv_state", "pending_key", "pending_delta", "pending_decay", "pending_input", "k_cache",
               "v_cache"}


def rel_rows(got: torch.Tensor, want: torch.Tensor, width: int) -> torch.Tensor:
    """Relative distance of each ``width``-long vector."""
    g = got.float().cpu().reshape(-1, width)
    w = want.float().cpu().reshape(-1, width)
    return (g - w).norm(dim=-1) / w.norm(dim=-1).clamp_min(1e-30)


def layer_values(values: dict, i: int) -> dict:
    """Layer ``i``'s weights renamed as layer 0 (for a one-layer engine)."""
    prefix = f"layers.{i}."
    return {"layers.0." + n[len(prefix):]: v for n, v in values.items() if n.startswith(prefix)}


def oracle_layer_weights(values: dict, i: int) -> dict:
    prefix = f"layers.{i}."
    return {n[len(prefix):]: (om.FP8Weight(v[0].cpu(), v[1].cpu()) if isinstance(v, tuple) else v.cpu())
            for n, v in values.items() if n.startswith(prefix)}


def gdn_state_from(engine: Engine, cfg) -> dict:
    """The engine's current gated-delta state in the reference's shapes (pending keys repeated per value head)."""
    st = {k: v.cpu().clone() for k, v in engine.gdn_state(0).items()}
    st["pending_key_state"] = om.repeat_interleave(st["pending_key_state"], cfg.linear_key_repeat, dim=2).contiguous()
    return st


def kv_state_from(engine: Engine, scales=None) -> dict:
    """The layer's caches on the host; with an FP8 cache (``scales`` = (k_scale, v_scale)) the bytes and the scales, as
    the oracle's attention takes them."""
    kc, vc = engine.get_kv(0)
    st = {"k_cache": kc.cpu(), "v_cache": vc.cpu()}
    if scales is not None:
        st["k_scale"], st["v_scale"] = scales
    return st


def seeded_states(cfg, batch: int, tokens: int, max_seq_len: int, context, seed: int, device="cuda", kv: str = "bf16"):
    """Per-layer starting states: unit-RMS gated-delta and conv states with empty snapshots, caches filled below each
    row's context (synth.gdn_states / synth.kv_states), made one layer at a time; with ``kv`` "fp8" the caches as
    e4m3 bytes of the layer's scales (synth.kv_scales), with the scales."""
    for i, kind in enumerate(cfg.layer_types):
        one = with_layers(cfg, (kind,))
        if kind == LINEAR:
            yield synth.gdn_states(one, batch, tokens, seed, f"layers.{i}", device=device)
        else:
            st = synth.kv_states(one, batch, max_seq_len, context, seed, f"layers.{i}", device=device)
            if kv == "fp8":
                ks, vs = synth.kv_scales(one, seed, f"layers.{i}")
                st = {"k_cache": encode_kv(st["k_cache"], ks.to(device)), "v_cache": encode_kv(st["v_cache"], vs.to(device)),
                      "k_scale": ks, "v_scale": vs}
            yield st


class LayerStack:
    """One one-layer engine per decoder layer of ``cfg``, loaded with ``values`` and the per-layer ``states``
    (reference shapes; consumed layer by layer so a caller can pass a generator), each with its probe bound."""

    def __init__(self, cfg, values: dict, batch: int, tokens: int, max_seq_len: int, states, projection_mfma: str = "bf16",
                 kv_cache_format: str = "bf16"):
        self.cfg, self.batch, self.tokens, self.max_seq_len = cfg, batch, tokens, max_seq_len
        self.engines, self.weights, self.kv_scales = [], [], {}
        for i, (kind, st) in enumerate(zip(cfg.layer_types, states)):
            engine = Engine(with_layers(cfg, (kind,)), batch, tokens, max_seq_len, mtp=False, projection_mfma=projection_mfma,
                            kv_cache_format=kv_cache_format)
            engine.load(layer_values(values, i).items())
            engine.enable_probe(0)
            if kind == LINEAR:
                engine.set_gdn(0, st)
            else:
                if "k_scale" in st:
                    self.kv_scales[i] = (st["k_scale"].cpu(), st["v_scale"].cpu())
                    engine.set_kv_scales(0, st["k_scale"].cuda(), st["v_scale"].cuda())
                engine.set_kv(0, st["k_cache"], st["v_cache"])
            del st
            self.engines.append(engine)
            self.weights.append(oracle_layer_weights(values, i))

    def verify_step(self, x: torch.Tensor, inputs: dict, log=print) -> dict:
        """One verify step through every layer, each against the oracle from the GPU's own input and state. Returns the
        worst errors per quantity and the GPU's final hidden states; raises AssertionError on a failed check."""
        cfg = self.cfg
        worst: dict[str, float] = {}
        cpu_inputs = {k: v.cpu() for k, v in inputs.items()}
        args = (cpu_inputs["cos"], cpu_inputs["sin"], cpu_inputs["position"], cpu_inputs["active"], cpu_inputs["accepted"])
        for i, (kind, engine, w) in enumerate(zip(cfg.layer_types, self.engines, self.weights)):
            one = with_layers(cfg, (kind,))
            before = gdn_state_from(engine, one) if kind == LINEAR else kv_state_from(engine, self.kv_scales.get(i))
            y = VerifyStep(engine)(inputs_embeds=x, **inputs)
            torch.cuda.synchronize()
            probe = {name: t.cpu().clone() for name, t in engine.probe(0).items()}
            if kind == LINEAR:
                errs = gdn_layer_errors(one, w, x.cpu(), y.cpu(), probe, gdn_state_from(engine, one), before, args,
                                        MODE_TOL[engine.projection_mfma])
            else:
                errs = attention_layer_errors(self, one, w, x.cpu(), y.cpu(), probe, kv_state_from(engine, self.kv_scales.get(i)), before, args,
                                              cpu_inputs, i, MODE_TOL[engine.projection_mfma])
            for name, e in errs.items():
                if name.startswith("_"):
                    continue
                top = float(e.max())
                worst[name] = max(worst.get(name, 0.0), top)
                tol = STATE_TOL if name in STATE_NAMES else HIDDEN_TOL
                log(f"  layer {i} {kind[:6]} {name}: max {top:.3g} median {float(e.median()):.3g} "
                    f"above {tol:g}: {int((e > tol).sum())}/{e.numel()}")
            for note in errs.get("_notes", []):
                log(f"  layer {i} {kind[:6]} {note}")
            x = y
        return {"worst": worst, "hidden": x}


# ----------------------------------------------------------------------------------------------- rounding stages


def bf16_half_step(v: torch.Tensor) -> torch.Tensor:
    """Half the spacing of bf16 values around ``v`` (float64)."""
    return torch.pow(2.0, torch.floor(torch.log2(v.abs().clamp_min(1e-38))) - 8)


# Per projection MFMA (the engine's projection_mfma): how far a projection's float32 sum may lie from the exact sum, in
# float32 ulps of sum |x*w| (eight for the bf16 MFMA's float32-grade sums; 2^9 for the scaled FP8 MFMA, which sums each
# 64-input block to about 2^-15.5 of its sum |x*w|: tests/test_gpu_linear.py measures both); how many bf16 steps an
# upstream difference may move a value before its e5m2 rounding; and which fraction of an e5m2 GEMM input may differ.
# The FP8 MFMA rounds about 1% of projection outputs to the other bf16 neighbour (the bf16 MFMA 0.005%), so more of
# them reach an e5m2 rounding boundary downstream.
MODE_TOL = {"bf16": {"sum_ulps": 8.0, "steps": 2, "flips": 1e-3}, "fp8": {"sum_ulps": 512.0, "steps": 4, "flips": 3e-2}}


def gemm_ties(x_e5m2: torch.Tensor, weight: om.FP8Weight, got: torch.Tensor, want: torch.Tensor, ulps: float = 8.0) -> tuple[int, float]:
    """A bf16 GEMM output against the oracle's, from the same e5m2 input ``[T, K]``: every element that differs must be,
    in both results, a correct bf16 rounding of a float32 value within ``ulps`` float32 ulps of sum|x*w| of the exact
    float64 sum (the oracle's is always within eight). Returns (number of differing elements, their largest distance in
    float32 ulps of sum|x*w|)."""
    got, want = got.reshape(x_e5m2.shape[0], -1), want.reshape(x_e5m2.shape[0], -1)
    idx = (got != want).nonzero()
    if not len(idx):
        return 0, 0.0
    rows, cols = idx[:, 0], idx[:, 1]
    products = x_e5m2[rows].double() * weight.dense()[cols].double()
    exact, scale = products.sum(-1), products.abs().sum(-1)
    worst = 0.0
    for v in (got[rows, cols].double(), want[rows, cols].double()):
        dist = ((v - exact).abs() - bf16_half_step(v)).clamp_min(0) / (scale * 2.0**-24)
        worst = max(worst, float(dist.max()))
    assert worst <= ulps, f"{len(idx)} differing GEMM outputs are not rounding ties (off by {worst:.3g} float32 ulps of sum|x*w|)"
    return len(idx), worst


def norm_ties(x: torch.Tensor, weight: torch.Tensor, eps: float, got: torch.Tensor, want: torch.Tensor) -> int:
    """The input RMS norm's bf16 output against the oracle's: every element that differs must be, in both results, a
    correct bf16 rounding of a float32 value within eight float32 ulps of the exact float64 x * rsqrt(mean(x^2) + eps) *
    (1 + w). Returns the number of differing elements."""
    got, want = got.reshape(-1, x.shape[-1]), want.reshape(-1, x.shape[-1])
    idx = (got != want).nonzero()
    if not len(idx):
        return 0
    xd = x.reshape(-1, x.shape[-1]).double()
    exact = (xd * torch.rsqrt((xd * xd).mean(-1, keepdim=True) + eps) * (1.0 + weight.double()))[idx[:, 0], idx[:, 1]]
    for v in (got[idx[:, 0], idx[:, 1]].double(), want[idx[:, 0], idx[:, 1]].double()):
        off = ((v - exact).abs() - bf16_half_step(v)).clamp_min(0) / (exact.abs() * 2.0**-24)
        assert float(off.max()) <= 8.0, f"{len(idx)} differing norm outputs are not rounding ties (off {float(off.max()):.3g} ulps)"
    return len(idx)


def bf16_steps(v: torch.Tensor, steps: int) -> list[torch.Tensor]:
    """``v`` (bf16) and its neighbours up to ``steps`` bf16 steps away in magnitude, same sign."""
    bits = v.contiguous().view(torch.int16).int()
    sign, mag = bits & 0x8000, bits & 0x7FFF
    out = []
    for d in range(-steps, steps + 1):
        m = (mag + d).clamp(0, 0x7F7F)
        out.append((sign | m).to(torch.int16).view(torch.bfloat16))
    return out


def e5m2_stage(pre: torch.Tensor, got: torch.Tensor, name: str, reach: bool = True, tol: dict = MODE_TOL["bf16"],
               explain=None) -> str:
    """An e5m2 GEMM input of the GPU (``got``, as bf16 values) against the oracle's bf16 value before that rounding
    (``pre``), computed from the GPU's own inputs to the stage. An element may differ from the oracle's e5m2 rounding
    only as far as a rounding tie upstream can move it: ``got`` must lie between the e5m2 roundings of pre -/+ slack,
    slack being ``tol["steps"]`` bf16 steps of the larger of the element and its token's RMS (a tie in a bf16 term of a
    sum moves the sum by a step of that term, however small the sum), and at most ``tol["flips"]`` of the elements may
    differ. With
    ``reach`` False only the count is held (attention's output, whose bf16-rounded scores move a softmax weight by a
    step of the score, up to 1.6%, at a rounding tie). ``explain(rows, cols, got)``, when given, proves elements beyond
    that reach another way (returns a bool per element)."""
    pre, got = pre.reshape(got.shape).float(), got.float()
    own = om.fp8_round(pre.to(torch.bfloat16)).float()
    diff = own != got
    n = int(diff.sum())
    explained = 0
    if n:
        rms = pre.pow(2).mean(-1, keepdim=True).sqrt().expand_as(pre)
        slack = 2 * tol["steps"] * bf16_half_step(torch.maximum(pre.abs(), rms).double()).float()
        lo = om.fp8_round((pre - slack).to(torch.bfloat16)).float()
        hi = om.fp8_round((pre + slack).to(torch.bfloat16)).float()
        inside = (got >= lo) & (got <= hi) | (not reach)
        if explain is not None and not bool(inside[diff].all()):
            where = (diff & ~inside).nonzero()
            ok = explain(where[:, 0], where[:, 1], got[where[:, 0], where[:, 1]])
            inside[where[ok, 0], where[ok, 1]] = True
            explained = int(ok.sum())
        if not bool(inside[diff].all()):
            where = (diff & ~inside).nonzero()[:8].tolist()
            print(f"{name}: outside (row, col, oracle pre, gpu e5m2, token rms) "
                  f"{[(r, c, float(pre[r, c]), float(got[r, c]), float(rms[r, c])) for r, c in where]}", flush=True)
        assert bool(inside[diff].all()), f"{name}: {int((diff & ~inside).sum())} e5m2 inputs beyond a rounding tie's reach"
        assert n <= max(1, int(got.numel() * tol["flips"])), f"{name}: {n} of {got.numel()} e5m2 inputs differ"
    where = "each within a rounding tie's reach of the oracle's value" if reach else "(count bound only)"
    if explained:
        where += f" ({explained} by an exact enumeration of the ties upstream)"
    return f"{name} e5m2 inputs differing {n} of {got.numel()}, {where}"


def mlp_stage(cfg, w: dict, probe: dict, y: torch.Tensor, notes: list, tol: dict) -> torch.Tensor:
    """The MLP from the GPU's residual after the mixer: its input norm and its SwiGLU product (e5m2 stages), then the
    layer output from the GPU's own down-projection input."""
    mixed, mlp_in, ffn = probe["mixed"], probe["mlp_in"], probe["ffn"]
    notes.append(e5m2_stage(om.rms_norm(mixed, w["post_attention_layernorm_weight"], cfg.rms_norm_eps), mlp_in, "MLP input", tol=tol))
    pre = om.silu(om.linear_fp8(mlp_in, w["mlp.gate_proj"])) * om.linear_fp8(mlp_in, w["mlp.up_proj"])
    explain = lambda rows, cols, got: swiglu_ties(mlp_in, w["mlp.gate_proj"], w["mlp.up_proj"], rows, cols, got, tol["sum_ulps"])
    notes.append(e5m2_stage(pre, ffn, "down input", tol=tol, explain=explain))
    return rel_rows(y, mixed + om.linear_fp8(ffn, w["mlp.down_proj"]), cfg.hidden_size)


def bf16_candidates(exact: torch.Tensor, spread: torch.Tensor) -> list[torch.Tensor]:
    """The bf16 values a correct rounding of any value within ``spread`` of ``exact`` (float64) can give: the
    roundings of the interval's two ends (monotone rounding reaches nothing else between them, at most two values for a
    spread under half a bf16 step)."""
    return [(exact - spread).float().to(torch.bfloat16), (exact + spread).float().to(torch.bfloat16)]


def swiglu_ties(x_e5m2: torch.Tensor, gate: om.FP8Weight, up: om.FP8Weight, rows, cols, got, ulps: float) -> torch.Tensor:
    """Whether each down-projection input ``got[i]`` (an e5m2 value of token ``rows[i]``, feature ``cols[i]``) is
    e5m2(bf16(bf16(g * bf16(sigmoid(g))) * u)) for some bf16 gate sum g and up sum u that are correct roundings of a
    float32 value within ``ulps`` float32 ulps of sum |x*w| of the exact (float64) sums, and a sigmoid rounded either
    way where sigmoid(g) lies within 2^-20 (relative) of a bf16 rounding boundary (a float32 exp and reciprocal are
    within a few ulps). The two products are exact in float32, so they round one way only. This is every value the
    reference's SwiGLU (model.py:48-51, 258-259) can give when the GPU's float32 sums and transcendental differ from
    the CPU's only by rounding."""
    x = x_e5m2[rows].double()
    out = torch.zeros(len(rows), dtype=torch.bool)
    pg, pu = x * gate.dense()[cols].double(), x * up.dense()[cols].double()
    gs, us = pg.sum(-1), pu.sum(-1)
    gspread, uspread = pg.abs().sum(-1) * ulps * 2.0**-24, pu.abs().sum(-1) * ulps * 2.0**-24
    for i in range(len(rows)):
        want = float(got[i])
        for g in {float(v[i]) for v in bf16_candidates(gs, gspread)}:
            sig = 1.0 / (1.0 + torch.exp(torch.tensor(-g, dtype=torch.float64)))
            for s in {float(v) for v in bf16_candidates(sig, sig * 2.0**-20)}:
                act = torch.tensor(g * s, dtype=torch.float32).to(torch.bfloat16).float()
                for u in {float(v[i]) for v in bf16_candidates(us, uspread)}:
                    h = (act * u).to(torch.bfloat16)
                    if float(om.fp8_round(h).float()) == want:
                        out[i] = True
        if not out[i]:
            print(f"SwiGLU input of token {int(rows[i])} feature {int(cols[i])}: GPU {want}; exact gate {float(gs[i]):.9g} "
                  f"(spread {float(gspread[i]):.3g}), up {float(us[i]):.9g} (spread {float(uspread[i]):.3g})", flush=True)
    return out


def mixer_output_stage(cfg, x, probe: dict, pre_mid, out_weight, notes: list, tol: dict, reach: bool = True) -> torch.Tensor:
    """The mixer's out_proj/o_proj input (an e5m2 stage from the oracle's value given the GPU's earlier stages), then the
    residual after the mixer from the GPU's own out_proj input."""
    notes.append(e5m2_stage(pre_mid, probe["mid"], "out_proj input", reach, tol))
    want = x.reshape(-1, cfg.hidden_size) + om.linear_fp8(probe["mid"], out_weight)
    return rel_rows(probe["mixed"], want, cfg.hidden_size)


# ----------------------------------------------------------------------------------------------- layers


def kv_errors(stack, got: dict, before: dict, want: dict, cpu_inputs: dict, layer: int) -> dict:
    """The step's own cache positions against the oracle; every other position must be untouched. A bf16 cache: the
    relative error of each written (head, token) row. An FP8 cache: the share of written bytes that differ from the
    oracle's per batch row (``k_cache``, ``v_cache``) and the relative error of each written row decoded
    (``k_cache_decoded``, ``v_cache_decoded``). The layer's keys and values come from the oracle's own projection of the
    GPU's input, so a near-tie e5m2 input rounded the other way moves a row by a little; its bytes then differ now and
    then, and a value near zero can move by several of e4m3's fine codes, so single bytes are not held to one code."""
    pos, k, s = cpu_inputs["position"].long(), stack.tokens, stack.max_seq_len
    on = cpu_inputs["active"] > 0.5
    fp8 = "k_scale" in want
    out = {}
    for name in ("k_cache", "v_cache"):
        written, decoded = [], []
        for b in range(stack.batch):
            at = slice(int(pos[b]), int(pos[b]) + k) if on[b] else slice(s - k, s)
            if fp8:
                g, w = got[name][b, :, at], want[name][b, :, at]
                written.append((g != w).float().mean().reshape(1))
                sc = want["k_scale" if name == "k_cache" else "v_scale"]
                decoded.append(rel_rows(decode_kv(g, sc), decode_kv(w, sc), stack.cfg.head_dim))
            else:
                written.append(rel_rows(got[name][b, :, at], want[name][b, :, at], stack.cfg.head_dim))
            keep = torch.ones(s, dtype=torch.bool)
            keep[at] = False
            assert torch.equal(got[name][b][:, keep], before[name][b][:, keep]), f"layer {layer}: {name} row {b} changed elsewhere"
        out[name] = torch.cat(written)
        if fp8:
            out[name + "_decoded"] = torch.cat(decoded)
    return out


def attention_layer_errors(stack, cfg, w: dict, x, y, probe: dict, got: dict, before: dict, args, cpu_inputs: dict,
                           layer: int, tol: dict = MODE_TOL["bf16"], own: bool = True) -> dict:
    """An attention layer: the residual after attention from the GPU's input (the oracle's own attention) and from the
    GPU's own o_proj input, the MLP stages and the written cache positions; ``hidden_own`` (with ``own``) is the whole
    layer from the GPU's input with the oracle's own roundings throughout."""
    st, trace, notes = {k: v.clone() for k, v in before.items()}, {}, []
    h = om.rms_norm(x, w["input_layernorm_weight"], cfg.rms_norm_eps)
    want_mixed = x + om.attention_verify(cfg, w, st, h, *args[:4], trace=trace)
    attention = rel_rows(probe["mixed"], want_mixed, cfg.hidden_size)
    o_proj = mixer_output_stage(cfg, x, probe, trace["finish"], w["self_attn.o_proj"], notes, tol, reach=False)
    errs = {
        "hidden": torch.maximum(torch.maximum(attention, o_proj), mlp_stage(cfg, w, probe, y, notes, tol)),
        "_notes": notes,
    }
    if own:
        want = want_mixed + om.mlp(w, om.rms_norm(want_mixed, w["post_attention_layernorm_weight"], cfg.rms_norm_eps))
        errs["hidden_own"] = rel_rows(y, want, cfg.hidden_size)
    errs.update(kv_errors(stack, got, before, st, cpu_inputs, layer))
    return errs


def beta_explains(w: dict, h, trace: dict, delta_gpu: torch.Tensor, active, bad: torch.Tensor) -> float:
    """For the delta vectors ``bad`` (flat over [B, K, Hv]): the GPU's delta must be beta' times the step's other terms
    (v - e^G k.S' - the earlier tokens' coupling terms, from the oracle's trace with the GPU's own earlier deltas) for
    beta' = bf16(sigmoid(b')), b' the oracle's bf16 gate projection or one bf16 step from it. Returns the largest
    relative distance between the GPU's delta and the best such beta' times the terms."""
    b, k, hv, _ = delta_gpu.shape
    key, v, g, ks = trace["key"], trace["value"], trace["cumulative"], trace["key_state"]
    gate = torch.nn.functional.linear(h.reshape(b * k, -1), w["linear_attn.in_proj_b"]).reshape(b, k, hv)
    worst = 0.0
    for flat in bad.nonzero().flatten().tolist():
        row, rest = divmod(flat, k * hv)
        t, head = divmod(rest, hv)
        terms = v[row, t, head] - g[row, t, head].exp() * ks[row, t, head]
        for s in range(t):
            coupling = (g[row, t, head] - g[row, s, head]).exp() * (key[row, t, head] * key[row, s, head]).sum()
            terms = terms - coupling * delta_gpu[row, s, head]
        target = delta_gpu[row, t, head]
        best = min(float((target - torch.sigmoid(c).float() * float(active[row]) * terms).norm() / target.norm())
                   for c in bf16_steps(gate[row, t, head].reshape(1), 1))
        assert best <= 1e-3, f"delta of row {row} token {t} head {head} is not a bf16 gate step from the oracle's ({best:.3g})"
        worst = max(worst, best)
    return worst


def gdn_layer_errors(cfg, w: dict, x, y, probe: dict, got: dict, before: dict, args, tol: dict = MODE_TOL["bf16"],
                     own: bool = True) -> dict:
    """A gated-delta layer stage by stage, each against the oracle fed the GPU's own results of the stages before it
    (`gdn_verify`'s ``force``):
    * the input norm's bf16 output: equal or rounding ties;
    * from the GPU's normed input, the in_proj_qkv and in_proj_z outputs (the pending input snapshot and the probe):
      equal or rounding ties;
    * the committed bf16 state, the conv state and the decays against the oracle's; a decay vector above 1e-2 only
      where the GPU's gate input, recovered from its stored decay, is one bf16 step from the oracle's;
    * keys and in-step deltas from the GPU's qkv, committed state and decays; a delta vector above 1e-2 only where the
      GPU's beta is the sigmoid of a gate input one bf16 step from the oracle's;
    * out_proj's e5m2 input from all of those, the GPU's z and its deltas; the residual after the mixer from the GPU's
      out_proj input; the MLP stages; 2e-2 per token for the two hidden-state stages (``hidden``).
    ``hidden_own`` (with ``own``) is the layer output against the oracle's own roundings throughout, reported."""
    d, hv, eps = cfg.linear_key_head_dim, cfg.linear_num_value_heads, cfg.rms_norm_eps
    b, k = got["pending_input_state"].shape[:2]
    position, active, accepted = args[2:]
    h_own = om.rms_norm(x, w["input_layernorm_weight"], eps)
    n_norm = norm_ties(x, w["input_layernorm_weight"], eps, probe["normed"], h_own)
    h, z_gpu = probe["normed"].reshape(b, k, -1), probe["projection"]
    st, trace_a = {key: v.clone() for key, v in before.items()}, {}
    om.gdn_verify(cfg, w, st, h, position, active, accepted, trace=trace_a)
    forced = {"qkv": got["pending_input_state"], "committed": got["recurrent_state"], "log_decay": got["pending_decay_state"]}
    st_b, trace_b = {key: v.clone() for key, v in before.items()}, {}
    # z only reaches the gated norm, which this run's checks do not read; the GPU's z saves the projection.
    om.gdn_verify(cfg, w, st_b, h, position, active, accepted, force={**forced, "z": z_gpu.reshape(b, k, -1)}, trace=trace_b)
    full, trace_c = {**forced, "z": z_gpu.reshape(b, k, -1), "delta": got["pending_delta_state"]}, {}
    om.gdn_verify(cfg, w, {key: v.clone() for key, v in before.items()}, h, position, active, accepted, force=full, trace=trace_c)
    xq = om.fp8_round(h).reshape(b * k, -1)
    n_qkv, t_qkv = gemm_ties(xq, w["linear_attn.in_proj_qkv"], got["pending_input_state"], st["pending_input_state"], tol["sum_ulps"])
    n_z, t_z = gemm_ties(xq, w["linear_attn.in_proj_z"], z_gpu, trace_a["z"], tol["sum_ulps"])
    notes = [f"input norm outputs differing {n_norm}, qkv {n_qkv}, z {n_z}: all rounding ties "
             f"(GEMM sums within {max(t_qkv, t_z):.2g} float32 ulps of sum|x*w|)"]
    # The gated norm from the GPU's own in-step output o (model.py:339-345).
    o_gpu = probe["inner"].reshape(b * k, hv, d)
    finish = {}
    om._gdn_finish(cfg, w, o_gpu, z_gpu.reshape(b * k, hv, d), torch.bfloat16, trace=finish)
    errs = {
        "hidden": torch.maximum(mixer_output_stage(cfg, x, probe, finish["finish"], w["linear_attn.out_proj"], notes, tol),
                                mlp_stage(cfg, w, probe, y, notes, tol)),
        "inner": rel_rows(o_gpu, trace_c["out"].to(torch.bfloat16), d),
        "pending_input": rel_rows(got["pending_input_state"], st["pending_input_state"], cfg.linear_conv_dim),
        "recurrent_state": rel_rows(got["recurrent_state"], st["recurrent_state"], d * d),
        "conv_state": rel_rows(got["conv_state"], st["conv_state"], got["conv_state"][0].numel()),
        "pending_decay": rel_rows(got["pending_decay_state"], st["pending_decay_state"], hv),
        "pending_key": rel_rows(got["pending_key_state"], st_b["pending_key_state"], d),
        "pending_delta": rel_rows(got["pending_delta_state"], st_b["pending_delta_state"], d),
        "_notes": notes,
    }
    if own:
        mixed_own = x + om.gdn_verify(cfg, w, {key: v.clone() for key, v in before.items()}, h_own, position, active, accepted)
        want_own = mixed_own + om.mlp(w, om.rms_norm(mixed_own, w["post_attention_layernorm_weight"], eps))
        errs["hidden_own"] = rel_rows(y, want_own, cfg.hidden_size)
    # Decays: recover the GPU's bf16 gate input a from g = -exp(A_log) * softplus(a + dt_bias).
    bad = (errs["pending_decay"] > STATE_TOL) & (active.repeat_interleave(k) > 0.5)
    if bad.any():
        g = got["pending_decay_state"].double().reshape(-1, hv)[bad]
        a_log, dt_bias = w["linear_attn.A_log"].double(), w["linear_attn.dt_bias"].double()
        a_gpu = torch.log(torch.expm1(-g / a_log.exp())) - dt_bias
        a_ref = torch.nn.functional.linear(h.reshape(b * k, -1), w["linear_attn.in_proj_a"]).double()[bad]
        off = (a_gpu - a_ref).abs() / (2 * bf16_half_step(a_ref))
        assert float(off.max()) <= 1.01, f"decay gate input off by {float(off.max()):.3g} bf16 steps"
        notes.append(f"decay vectors above 1e-2: {int(bad.sum())}, gate input within {float(off.max()):.3g} bf16 step")
        errs["pending_decay"] = errs["pending_decay"][~bad] if (~bad).any() else torch.zeros(1)
    bad = errs["pending_delta"] > STATE_TOL
    if bad.any():
        off = beta_explains(w, h, trace_b, got["pending_delta_state"], active, bad)
        notes.append(f"delta vectors above 1e-2: {int(bad.sum())}, each from a beta gate input one bf16 step from the "
                     f"oracle's (delta reproduced within {off:.2g})")
        errs["pending_delta"] = errs["pending_delta"][~bad] if (~bad).any() else torch.zeros(1)
    return errs


# ----------------------------------------------------------------------------------------------- accepted counts


def accepted_like_corrupted_drafts(batch: int, tokens: int, seed: int, p: float = 0.3) -> list[int]:
    """Accepted counts as greedy drafts corrupted with probability ``p`` give them (1, 3): one plus
    the number of leading drafts kept."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(batch):
        keep = (torch.rand(tokens - 1, generator=g) >= p).tolist()
        n = 0
        while n < tokens - 1 and keep[n]:
            n += 1
        out.append(n + 1)
    return out


def accepted_uniform(batch: int, tokens: int, seed: int) -> list[int]:
    """L ~ U{0..K-1} drafts accepted per row."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(0, tokens, (batch,), generator=g) + 1).tolist()
