"""CPU restatement of the reference's verify, decode and prefill semantics. TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Every function follows the reference CPU path op for op, in torch CPU, at the same rounding points (dtype bf16 in
production; float32 for the invariant tests, as the reference's own tests do). The one deliberate difference is the
weight format: FP8 e4m3 bytes ``[out, in]`` with an E8M0 scale per 32 inputs, dequantized exactly, where the
reference decodes e5m2 bytes ``[in, out]`` (qwen38_inf2/model.py:221-225, fp4.py:157-166).

Pinning of each function (what fixes it besides this text):
* tests/golden/verify_tiny.safetensors, written by tests/golden/make_golden.py from the reference's own CPU path
  (imported in the build container): pins `gdn_verify`, `attention_verify`, `mlp`, `decoder_layer`, `step_verify`,
  `mtp_forward`, `head_group_maxima`, `chip_next_tokens`, `accept` bit for bit on config 0 shapes.
* tests/golden/prefill_tiny.safetensors, written by tests/golden/make_golden_prefill.py from the reference's CPU path:
  pins `gdn_prefill`, `chunked_gated_delta`, `unit_lower_inverse`, `attention_prefill`, `blocked_attention`,
  `_write_chunk`, `attention_cache_chunk`, `step_prefill` and `mtp_prefill` bit for bit (two chunks of one row, the
  second padded, and the MTP layer's prefill form).
* tests/golden/kv8_tiny.safetensors, written by tests/golden/make_golden_kv8.py from the reference's CPU path with
  kv_cache_format "fp8": pins `kv_store`, `kv_load`, `kv_round_trip` and the FP8-cache branches of
  `attention_verify`, `attention_decode` and `attention_prefill` bit for bit (hidden states and cache bytes after two
  verify steps, a decode step and a prefill chunk of one attention layer); tests/test_oracle.py also holds the e4m3
  codec against its bit fields over every bf16 value.
* `decode_planes` and `linear_fp4` (the weight_format "fp4" numerics): the planes against the reference's FP4 decode
  known-answer file (tests/golden/fp4_decode_kat), each plane's product against its float64 sum (one of the two bf16
  neighbours) and the sum of the planes in bf16, in tests/test_oracle.py.
* invariants in tests/test_oracle.py: prefill then decode equals decoding every token (float32, reference
  tests/test_prefill.py:143-166); the chunked rule equals the recurrence in float64 with correlated keys and padding;
  `unit_lower_inverse` equals a dense inverse; blocked attention equals one softmax;
  verify with every token accepted equals sequential `gdn_decode`/`attention_decode`
  steps (reference tests/test_prefill.py:235-263); the textbook recurrence in float64; full-softmax attention by brute
  force; ChipHead equals HostHead (reference tests/test_model_parity.py:280-309); e4m3 dequantization against its bit
  fields; e5m2 rounding against an exhaustive bf16 table.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

# Added to the scores of unfilled cache slots (model.py:30-32).
MASKED_SCORE = -1e4
# Tokens per piece of the chunked gated delta rule (model.py:34) and cache positions per block of prefill attention
# (model.py:36).
DELTA_CHUNK = 128
ATTENTION_BLOCK = 2048
# The FP8 KV cache's largest value: the reference clamps to NeuronCore-v2's finite e4m3 range before the cast to
# e4m3fn (model.py:41, 581-585).
FP8_KV_MAX = 240.0
# The reference rounds every FP8 projection's input to e5m2 (model.py:85-87, 222-225). Tests that compare two float32
# forms of the same computation switch it off, as reference tests/test_model_parity.py:255-260 does.
ROUND_E5M2 = True


# ----------------------------------------------------------------------------------------------- elementwise pieces


def silu(x: torch.Tensor) -> torch.Tensor:
    """model.py:48-51."""
    return x * torch.sigmoid(x)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """model.py:54-57: float32 inside, ``(1 + weight)``, result in x's dtype."""
    h = x.float()
    h = h * torch.rsqrt((h * h).mean(-1, keepdim=True) + eps)
    return (h * (1.0 + weight.float())).type_as(x)


def l2_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """model.py:60-61."""
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def repeat_interleave(x: torch.Tensor, repeats: int, dim: int) -> torch.Tensor:
    """model.py:64-67."""
    expanded = x.unsqueeze(dim + 1).expand(*x.shape[: dim + 1], repeats, *x.shape[dim + 1 :])
    return expanded.reshape(*x.shape[:dim], x.shape[dim] * repeats, *x.shape[dim + 1 :])


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """model.py:70-72."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """model.py:75-82: partial RoPE on the first ``cos.shape[-1]`` dims."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    rot = cos.shape[-1]
    q_rot, q_pass = q[..., :rot], q[..., rot:]
    k_rot, k_pass = k[..., :rot], k[..., rot:]
    q_out = q_rot * cos + rotate_half(q_rot) * sin
    k_out = k_rot * cos + rotate_half(k_rot) * sin
    return torch.cat((q_out, q_pass), dim=-1), torch.cat((k_out, k_pass), dim=-1)


def fp8_round(x: torch.Tensor) -> torch.Tensor:
    """model.py:85-87: round to e5m2 and back."""
    return x.to(torch.float8_e5m2).to(x.dtype) if ROUND_E5M2 else x


def e4m3_to_float(coded: torch.Tensor) -> torch.Tensor:
    """OCP e4m3fn bytes to float32 from the bit fields: sign, 4 exponent bits (bias 7), 3 mantissa bits, subnormals
    at exponent 0, and 0x7F/0xFF NaN. Written from the format definition rather than torch's cast, so tests can hold
    the two against each other."""
    b = coded.to(torch.int32)
    exponent, mantissa = (b >> 3) & 15, b & 7
    magnitude = torch.where(
        exponent == 0, mantissa.float() * 2.0**-9, (1.0 + mantissa.float() / 8.0) * torch.pow(2.0, exponent.float() - 7.0)
    )
    magnitude = torch.where((b & 127) == 127, torch.full_like(magnitude, float("nan")), magnitude)
    return torch.where(b >= 128, -magnitude, magnitude)


class FP8Weight:
    """One projection's weight: e4m3 bytes ``[out, in]`` and E8M0 bytes ``[out, in/32]``. ``dense_t`` may be given
    when the caller already holds the exact float32 values ``[in, out]`` (tests dequantize large weights on the GPU,
    where the same exact arithmetic is faster, and spot-check them against `dense_t`'s own decoding)."""

    def __init__(self, coded: torch.Tensor, scales: torch.Tensor, dense_t: torch.Tensor | None = None):
        self.coded, self.scales = coded, scales
        self._dense_t = dense_t
        self._cast: dict = {}

    def decoded_t(self, rows: slice) -> torch.Tensor:
        """float32 ``[in, rows]`` of the given output rows, decoded from the bytes (never from a given ``dense_t``)."""
        coded, scales = self.coded[rows], self.scales[rows]
        n, k = coded.shape
        values = e4m3_to_float(coded).reshape(n, k // 32, 32)
        return (values * torch.pow(2.0, scales.float() - 127.0).unsqueeze(-1)).reshape(n, k).T

    def dense_t_as(self, dtype: torch.dtype) -> torch.Tensor:
        """`dense_t` converted to ``dtype`` (exact for bf16 and wider), kept for later calls."""
        if dtype == torch.float32:
            return self.dense_t()
        if dtype not in self._cast:
            self._cast[dtype] = self.dense_t().to(dtype)
        return self._cast[dtype]

    def dense_t(self) -> torch.Tensor:
        """float32 ``[in, out]``, contiguous, the layout the reference's weights have (``weight_fp8`` is
        ``[in, out]``, model.py:214-219), so torch's CPU matmuls see the same strides and sum in the same order.
        Exact, and exact again in bf16."""
        if self._dense_t is None:
            n, k = self.coded.shape
            values = e4m3_to_float(self.coded).reshape(n, k // 32, 32)
            scale = torch.pow(2.0, self.scales.float() - 127.0).unsqueeze(-1)
            self._dense_t = (values * scale).reshape(n, k).T.contiguous()
        return self._dense_t

    def dense(self) -> torch.Tensor:
        """float32 ``[out, in]`` (a transposed view)."""
        return self.dense_t().T


def linear_fp8(x: torch.Tensor, weight: FP8Weight) -> torch.Tensor:
    """`FP8Linear.forward` on CPU (model.py:221-225): e5m2 input, weights in x's dtype, x's dtype out."""
    x = fp8_round(x)
    return F.linear(x, weight.dense_t_as(x.dtype).T)


# E2M1 magnitudes of nibble codes 0-7 (codes 8-15 are their negatives), fp4.py:31.
E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def decode_planes(packed: torch.Tensor, scale_bytes: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The checkpoint's MXFP4 weight (``packed`` uint8 ``[out, in / 2]``, the even input in the low nibble; E8M0
    ``scale_bytes`` ``[out, in / 32]``) as its even and odd input columns in bf16 (fp4.py:93-100 on the sign-free form,
    which `to_sign_free` makes from these bytes, fp4.py:75-84; every value exact in bf16, fp4.py:20-22)."""
    lut = torch.tensor(E2M1_MAGNITUDES, dtype=torch.float32)
    lut = torch.cat((lut, -lut))
    scale = torch.pow(2.0, scale_bytes.float() - 127.0).repeat_interleave(16, dim=-1)  # 16 of each plane per group
    even = lut[(packed & 15).long()] * scale
    odd = lut[(packed >> 4).long()] * scale
    # The sign-free codes have one zero: a negative zero decodes as +0 (fp4.py:78).
    return (torch.where(even == 0, 0.0, even).to(torch.bfloat16), torch.where(odd == 0, 0.0, odd).to(torch.bfloat16))


def linear_fp4(x: torch.Tensor, packed: torch.Tensor, scale_bytes: torch.Tensor) -> torch.Tensor:
    """`FP4Linear.forward` (model.py:205-208): x's even and odd inputs through the two planes, each a matmul in x's
    dtype, the results added in x's dtype."""
    even, odd = decode_planes(packed, scale_bytes)
    return F.linear(x[..., ::2], even.to(x.dtype)) + F.linear(x[..., 1::2], odd.to(x.dtype))


def mlp(w: dict, x: torch.Tensor) -> torch.Tensor:
    """`MLP.forward` on CPU (model.py:250-259), tp 1."""
    return linear_fp8(silu(linear_fp8(x, w["mlp.gate_proj"])) * linear_fp8(x, w["mlp.up_proj"]), w["mlp.down_proj"])


# ----------------------------------------------------------------------------------------------- gated delta net


def _gdn_split(cfg, mixed: torch.Tensor):
    """`GatedDeltaNetStep._split` (model.py:322-331): q, k per value head and v, float32; q scaled by d^-1/2."""
    tokens = mixed.shape[0]
    k_head, v_head = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    key_dim = cfg.linear_key_dim
    query = mixed[:, :key_dim].reshape(tokens, cfg.linear_num_key_heads, k_head)
    key = mixed[:, key_dim : 2 * key_dim].reshape(tokens, cfg.linear_num_key_heads, k_head)
    value = mixed[:, 2 * key_dim :].reshape(tokens, cfg.linear_num_value_heads, v_head)
    query = repeat_interleave(query, cfg.linear_key_repeat, dim=1)
    key = repeat_interleave(key, cfg.linear_key_repeat, dim=1)
    return l2_norm(query.float()) / math.sqrt(k_head), l2_norm(key.float()), value.float()


def _gdn_gates(w: dict, x: torch.Tensor):
    """`GatedDeltaNetStep._gates` (model.py:333-337): beta and log decay, float32 ``[tokens, v_heads]``."""
    beta = F.linear(x, w["linear_attn.in_proj_b"]).sigmoid().float()
    a = F.linear(x, w["linear_attn.in_proj_a"]).float()
    return beta, -w["linear_attn.A_log"].float().exp() * F.softplus(a + w["linear_attn.dt_bias"].float())


def _gdn_finish(cfg, w: dict, out: torch.Tensor, z: torch.Tensor, dtype: torch.dtype, trace=None) -> torch.Tensor:
    """`GatedDeltaNetStep._finish` (model.py:339-345): gated RMS norm per value head (weight without 1+), then
    out_proj. ``out``, ``z`` ``[tokens, v_heads, v_head]``. ``trace`` (tests only) receives ``finish``, out_proj's input
    before its e5m2 rounding."""
    h = out.float()
    h = h * torch.rsqrt((h * h).mean(-1, keepdim=True) + cfg.rms_norm_eps)
    h = w["linear_attn.norm_weight"] * h.to(dtype)
    h = (h * silu(z.float())).to(dtype)
    if trace is not None:
        trace["finish"] = h.reshape(out.shape[0], cfg.linear_value_dim)
    return linear_fp8(h.reshape(out.shape[0], 1, cfg.linear_value_dim), w["linear_attn.out_proj"])


def commit_and_read(state, scale, weighted, deltas, reads):
    """`_commit_and_read` CPU branch (model.py:262-266): ``S' = (S*scale + W^T D)`` rounded to the state's dtype, and
    ``R^T float(S')``."""
    committed = (state.float() * scale + weighted.transpose(1, 2) @ deltas).to(state.dtype)
    return committed, reads.transpose(1, 2) @ committed.float()


def gdn_verify(cfg, w: dict, st: dict, x, position, active, accepted, force=None, trace=None):
    """`GatedDeltaNetStep.verify` (model.py:376-454), tp 1. ``x`` ``[B, K, H]`` (the input norm's output).

    ``st`` holds ``recurrent_state [B,Hv,d,d]``, ``conv_state [B,C,3]``, ``pending_key_state [B,K,Hv,d]`` (f32),
    ``pending_delta_state [B,K,Hv,d]`` (f32), ``pending_decay_state [B,K,Hv]`` (f32), ``pending_input_state [B,K,C]``;
    the entries are replaced by their new values. Returns ``[B, K, H]``.

    ``force`` and ``trace`` serve tests that compare another implementation stage by stage. ``force`` may hold that
    implementation's ``qkv`` (the in_proj_qkv output ``[B, K, C]``), ``z`` (the in_proj_z output ``[B, K, Hv*d]``),
    ``committed`` (the committed state
    ``[B, Hv, d, d]``), ``log_decay`` (``[B, K, Hv]``) or ``delta`` (``[B, K, Hv, d]``), used in place of this function's
    own values from that point on. ``trace``, a dict, receives the in-step quantities (``query``, ``key``, ``value``,
    ``cumulative`` ``[B, K, Hv]``, ``query_state`` = q·S', ``key_state`` = k·S', ``beta``, ``delta``, ``out``) and the
    in_proj_z output ``z`` ``[B*K, Hv, d]``.
    """
    force = force or {}
    dtype = x.dtype
    batch, tokens = x.shape[:2]
    kernel = cfg.linear_conv_kernel_dim
    on = (active > 0.5).reshape(batch, 1)
    keep = torch.where((position.reshape(batch, 1) == 0) & on, 0.0, 1.0)
    taken = [(accepted.reshape(batch, 1) > s).float() for s in range(st["pending_key_state"].shape[1])]
    decays = [st["pending_decay_state"][:, s] * taken[s] for s in range(len(taken))]
    remaining, weighted = sum(decays), []
    scale = torch.where(on, remaining.exp() * keep, 1.0)
    for s in range(len(taken)):
        remaining = remaining - decays[s]
        weighted.append(st["pending_key_state"][:, s] * (remaining.exp() * taken[s] * keep * on).unsqueeze(-1))
    window = torch.cat((st["conv_state"], st["pending_input_state"].transpose(1, 2)), dim=-1)
    index = (accepted.long().reshape(batch, 1, 1) + torch.arange(kernel - 1)).expand(-1, window.shape[1], -1)
    history = window.gather(2, index) * keep.reshape(batch, 1, 1).to(dtype)
    history = torch.where(on.reshape(batch, 1, 1), history, st["conv_state"])
    st["conv_state"] = history

    qkv = force["qkv"].to(dtype) if "qkv" in force else linear_fp8(x, w["linear_attn.in_proj_qkv"])
    window = torch.cat((history, qkv.transpose(1, 2)), dim=-1)
    conv_weight = w["linear_attn.conv_weight"]
    mixed = torch.stack([(window[:, :, t : t + kernel] * conv_weight).sum(dim=-1) for t in range(tokens)], dim=1)
    query, key, value = (
        part.reshape(batch, tokens, *part.shape[1:]) for part in _gdn_split(cfg, silu(mixed).reshape(batch * tokens, -1))
    )
    heads = cfg.linear_num_value_heads
    z = force["z"].to(dtype) if "z" in force else linear_fp8(x, w["linear_attn.in_proj_z"])
    z = z.reshape(batch * tokens, heads, -1)
    beta, log_decay = _gdn_gates(w, x.reshape(batch * tokens, -1))
    beta = beta.reshape(batch, tokens, -1) * active.reshape(batch, 1, 1)
    log_decay = log_decay.reshape(batch, tokens, -1) * active.reshape(batch, 1, 1)
    if "log_decay" in force:
        log_decay = force["log_decay"].float()

    state = st["recurrent_state"]
    k_head, v_head = state.shape[2:]
    pairs = batch * heads
    reads = torch.cat((key, query), dim=1).permute(0, 2, 3, 1).reshape(pairs, k_head, 2 * tokens)
    committed, products = commit_and_read(
        state.reshape(pairs, k_head, v_head),
        scale.reshape(pairs, 1, 1).expand(-1, k_head, -1),
        torch.stack(weighted, dim=2).reshape(pairs, -1, k_head),
        st["pending_delta_state"].transpose(1, 2).reshape(pairs, -1, v_head),
        reads,
    )
    if "committed" in force:
        committed = force["committed"].to(state.dtype).reshape(pairs, k_head, v_head)
        products = reads.transpose(1, 2) @ committed.float()
    st["recurrent_state"] = committed.reshape(batch, heads, k_head, v_head)
    products = products.reshape(batch, heads, 2 * tokens, v_head).transpose(1, 2)
    key_state, query_state = products[:, :tokens], products[:, tokens:]

    cumulative = [log_decay[:, 0]]
    for t in range(1, tokens):
        cumulative.append(cumulative[-1] + log_decay[:, t])
    deltas, outs = [], []
    for t in range(tokens):
        delta = value[:, t] - cumulative[t].exp().unsqueeze(-1) * key_state[:, t]
        for s in range(t):
            coupling = (cumulative[t] - cumulative[s]).exp() * (key[:, t] * key[:, s]).sum(dim=-1)
            delta = delta - coupling.unsqueeze(-1) * deltas[s]
        deltas.append(force["delta"][:, t].float() if "delta" in force else delta * beta[:, t].unsqueeze(-1))
        out = cumulative[t].exp().unsqueeze(-1) * query_state[:, t]
        for s in range(t + 1):
            attend = (cumulative[t] - cumulative[s]).exp() * (query[:, t] * key[:, s]).sum(dim=-1)
            out = out + attend.unsqueeze(-1) * deltas[s]
        outs.append(out)
    delta, out = torch.stack(deltas, dim=1), torch.stack(outs, dim=1)
    if trace is not None:
        trace.update(query=query, key=key, value=value, cumulative=torch.stack(cumulative, dim=1), query_state=query_state,
                     key_state=key_state, beta=beta, delta=delta, out=out, z=z)
    # The reference adds the commit kernel's zero output to order these writes after its reads (model.py:449-452);
    # adding 0.0 also turns -0.0 into +0.0, which the stored bits show.
    st["pending_key_state"] = key.float() + 0.0
    st["pending_delta_state"] = delta
    st["pending_decay_state"] = log_decay.float() + 0.0
    st["pending_input_state"] = qkv + torch.zeros((), dtype=qkv.dtype)
    out = out.reshape(batch * tokens, heads, -1).to(dtype)
    return _gdn_finish(cfg, w, out, z, dtype, trace).reshape(batch, tokens, -1)


def gdn_decode(cfg, w: dict, st: dict, x, position, active):
    """`GatedDeltaNetStep.forward` (model.py:347-374): one token per row, ``x`` ``[B, 1, H]``. Used only to check the
    verify form against (reference tests/test_prefill.py:235-263)."""
    dtype = x.dtype
    batch = x.shape[0]
    on = active.reshape(batch, 1, 1) > 0.5
    keep = torch.where((position == 0) & (active > 0.5), 0.0, 1.0)
    qkv = linear_fp8(x, w["linear_attn.in_proj_qkv"]).transpose(1, 2)
    conv_state = st["conv_state"]
    window = torch.cat((conv_state * keep.reshape(batch, 1, 1).to(dtype), qkv), dim=-1)
    st["conv_state"] = torch.where(on, window[:, :, 1:], conv_state)
    query, key, value = _gdn_split(cfg, silu((window * w["linear_attn.conv_weight"]).sum(dim=-1)))
    heads = cfg.linear_num_value_heads
    z = linear_fp8(x, w["linear_attn.in_proj_z"]).reshape(batch, heads, -1)
    beta, log_decay = _gdn_gates(w, x.reshape(batch, -1))
    beta = (beta * active.unsqueeze(-1)).unsqueeze(-1)
    log_decay = log_decay * active.unsqueeze(-1)
    state = st["recurrent_state"].float() * keep.reshape(batch, 1, 1, 1) * log_decay.exp()[..., None, None]
    delta = (value - (state * key.unsqueeze(-1)).sum(dim=-2)) * beta
    state = state + key.unsqueeze(-1) * delta.unsqueeze(-2)
    st["recurrent_state"] = state.to(st["recurrent_state"].dtype)
    out = (state * query.unsqueeze(-1)).sum(dim=-2).to(dtype)
    return _gdn_finish(cfg, w, out, z, dtype)


# ----------------------------------------------------------------------------------------------- full attention


def _attention_project(cfg, w: dict, x, cos, sin):
    """`FullAttentionStep._project` (model.py:565-577)."""
    head = cfg.head_dim
    rows, tokens = x.shape[:2]
    q_and_gate = linear_fp8(x, w["self_attn.q_proj"]).reshape(rows, tokens, cfg.num_attention_heads, head * 2)
    query, gate = q_and_gate[..., :head], q_and_gate[..., head:]
    query = rms_norm(query, w["self_attn.q_norm_weight"], cfg.rms_norm_eps).transpose(1, 2)
    key = linear_fp8(x, w["self_attn.k_proj"]).reshape(rows, tokens, cfg.num_key_value_heads, head)
    key = rms_norm(key, w["self_attn.k_norm_weight"], cfg.rms_norm_eps).transpose(1, 2)
    value = linear_fp8(x, w["self_attn.v_proj"]).reshape(rows, tokens, cfg.num_key_value_heads, head).transpose(1, 2)
    query, key = apply_rotary(query, key, cos, sin)
    return query, key, value, gate.reshape(rows, tokens, cfg.num_attention_heads * head)


def kv_store(t: torch.Tensor, scale) -> torch.Tensor:
    """`FullAttentionStep._store` (model.py:579-585), CPU branch: what the cache holds for ``t``: itself (a bf16 cache,
    ``scale`` None), or the e4m3 bytes of ``float32(t) / float32(scale)`` clamped to +-240."""
    if scale is None:
        return t
    return (t.float() / scale.float()).clamp(-FP8_KV_MAX, FP8_KV_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def kv_load(t: torch.Tensor, scale, dtype: torch.dtype) -> torch.Tensor:
    """`FullAttentionStep._load` (model.py:587-589): cached values back, ``dtype(e4m3 value * scale)`` for bytes."""
    if scale is None:
        return t
    return (t.view(torch.float8_e4m3fn).to(dtype) * scale).to(dtype)


def kv_round_trip(t: torch.Tensor, scale, dtype: torch.dtype) -> torch.Tensor:
    """`FullAttentionStep._round_trip` (model.py:591-593): a step's own key or value as later steps will read it."""
    return kv_load(kv_store(t, scale), scale, dtype)


def kv_scales(st: dict):
    """The layer's (k_scale, v_scale) for an FP8 cache (``st`` holding them), else (None, None)."""
    return st.get("k_scale"), st.get("v_scale")


def _write_both(st: dict, key, value, positions):
    """`FullAttentionStep._write_both` (model.py:603-608): ``key``/``value`` already in the cache's format."""
    rows, kv_heads, n, head = key.shape
    at = positions.reshape(rows, 1, n, 1).expand(-1, kv_heads, -1, head)
    st["k_cache"] = st["k_cache"].scatter(2, at, key)
    st["v_cache"] = st["v_cache"].scatter(2, at, value)


def attention_verify(cfg, w: dict, st: dict, x, cos, sin, position, active, trace=None):
    """`FullAttentionStep.verify` CPU branch (model.py:641-672), tp 1. ``st`` holds ``k_cache``/``v_cache``
    ``[B, Hkv, S, hd]`` (bf16, or e4m3 bytes with ``k_scale``/``v_scale``), replaced by the written caches. ``trace``
    (tests only) receives ``finish``, o_proj's input before its e5m2 rounding."""
    head = cfg.head_dim
    batch, tokens = x.shape[:2]
    max_seq_len = st["k_cache"].shape[2]
    query, key, value, gate = _attention_project(cfg, w, x, cos, sin)
    groups = cfg.num_key_value_groups
    steps = torch.arange(tokens)
    where = torch.where(active.unsqueeze(-1) > 0.5, position.long().unsqueeze(-1) + steps, max_seq_len - tokens + steps)
    grouped = query.reshape(batch, cfg.num_key_value_heads, groups, tokens, head)
    ks, vs = kv_scales(st)
    keys = kv_load(st["k_cache"], ks, x.dtype).unsqueeze(2)
    values = kv_load(st["v_cache"], vs, x.dtype).unsqueeze(2)
    earlier = torch.arange(max_seq_len) < position.unsqueeze(-1)
    cached = torch.matmul(grouped, keys.transpose(-1, -2)).float() + torch.where(earlier, 0.0, MASKED_SCORE).reshape(batch, 1, 1, 1, -1)
    own_key = kv_round_trip(key, ks, x.dtype).unsqueeze(2)
    own_value = kv_round_trip(value, vs, x.dtype).unsqueeze(2)
    causal = steps.unsqueeze(0) <= steps.unsqueeze(-1)
    own = torch.matmul(grouped, own_key.transpose(-1, -2)).float() + torch.where(causal, 0.0, MASKED_SCORE)
    weights = torch.softmax(torch.cat((cached, own), dim=-1) * head**-0.5, dim=-1).to(x.dtype)
    out = torch.matmul(weights[..., :max_seq_len], values) + torch.matmul(weights[..., max_seq_len:], own_value)
    out = out.permute(0, 3, 1, 2, 4).reshape(batch, tokens, cfg.num_attention_heads * head)
    _write_both(st, kv_store(key, ks), kv_store(value, vs), where)
    gated = out * torch.sigmoid(gate)
    if trace is not None:
        trace["finish"] = gated.reshape(batch * tokens, -1)
    return linear_fp8(gated, w["self_attn.o_proj"])


def attention_decode(cfg, w: dict, st: dict, x, cos, sin, position, active):
    """`FullAttentionStep.forward` CPU branch (model.py:610-639): one token per row."""
    head = cfg.head_dim
    batch = x.shape[0]
    max_seq_len = st["k_cache"].shape[2]
    query, key, value, gate = _attention_project(cfg, w, x, cos, sin)
    grouped = query.reshape(batch, cfg.num_key_value_heads, cfg.num_key_value_groups, head)
    where = torch.where(active > 0.5, position.long(), max_seq_len - 1).unsqueeze(-1)
    ks, vs = kv_scales(st)
    keys, values = kv_load(st["k_cache"], ks, x.dtype), kv_load(st["v_cache"], vs, x.dtype)
    earlier = torch.arange(max_seq_len) < position.unsqueeze(-1)
    cached = torch.matmul(grouped, keys.transpose(2, 3)).float() + torch.where(earlier, 0.0, MASKED_SCORE).reshape(batch, 1, 1, -1)
    own = torch.matmul(grouped, kv_round_trip(key, ks, x.dtype).transpose(2, 3)).float()
    weights = torch.softmax(torch.cat((cached, own), dim=-1) * head**-0.5, dim=-1).to(x.dtype)
    out = torch.matmul(weights[..., :-1], values) + weights[..., -1:] * kv_round_trip(value, vs, x.dtype)
    out = out.reshape(batch, 1, cfg.num_attention_heads * head)
    _write_both(st, kv_store(key, ks), kv_store(value, vs), where)
    return linear_fp8(out * torch.sigmoid(gate), w["self_attn.o_proj"])


# ----------------------------------------------------------------------------------------------- layers and step


def decoder_layer(cfg, layer_type: str, w: dict, st: dict, x, cos, sin, position, active, accepted=None, slot=None,
                  start=None, n_valid=None, gdn_force=None, gdn_trace=None):
    """`DecoderLayer.forward` (model.py:918-930): verify when ``accepted`` is given, prefill when ``slot`` is, else
    decode. ``gdn_force`` / ``gdn_trace`` (tests only) go to `gdn_verify` as ``force`` / ``trace``."""
    eps = cfg.rms_norm_eps
    h = rms_norm(x, w["input_layernorm_weight"], eps)
    if slot is not None and accepted is None:
        if layer_type == "linear_attention":
            mixer = gdn_prefill(cfg, w, st, h, slot, start, n_valid)
        else:
            mixer = attention_prefill(cfg, w, st, h, cos, sin, slot, start, n_valid)
    elif layer_type == "linear_attention":
        if accepted is not None:
            mixer = gdn_verify(cfg, w, st, h, position, active, accepted, gdn_force, gdn_trace)
        else:
            mixer = gdn_decode(cfg, w, st, h, position, active)
    else:
        if accepted is not None:
            mixer = attention_verify(cfg, w, st, h, cos, sin, position, active)
        else:
            mixer = attention_decode(cfg, w, st, h, cos, sin, position, active)
    x = x + mixer
    return x + mlp(w, rms_norm(x, w["post_attention_layernorm_weight"], eps))


def step_verify(cfg, layers: list, states: list, inputs_embeds, cos, sin, position, active, accepted):
    """`Qwen38Step.forward` with ``accepted`` (model.py:983-995): all layers, hidden before the final norm."""
    x = inputs_embeds
    for layer_type, w, st in zip(cfg.layer_types, layers, states):
        x = decoder_layer(cfg, layer_type, w, st, x, cos, sin, position, active, accepted)
    return x


def step_prefill(cfg, layers: list, states: list, inputs_embeds, cos, sin, slot, start, n_valid):
    """`Qwen38Step.forward` prefill form (model.py:983-995): one chunk ``[1, L, H]`` of row ``slot`` from ``start``."""
    x = inputs_embeds
    for layer_type, w, st in zip(cfg.layer_types, layers, states):
        x = decoder_layer(cfg, layer_type, w, st, x, cos, sin, None, None, slot=slot, start=start, n_valid=n_valid)
    return x


def step_decode(cfg, layers: list, states: list, inputs_embeds, cos, sin, position, active):
    """`Qwen38Step.forward` decode form (model.py:983-995)."""
    x = inputs_embeds
    for layer_type, w, st in zip(cfg.layer_types, layers, states):
        x = decoder_layer(cfg, layer_type, w, st, x, cos, sin, position, active)
    return x


def mtp_forward(cfg, w: dict, st: dict, hidden, inputs_embeds, cos, sin, position, active):
    """`MTPStep.forward` step form (model.py:843-860), tp 1. ``w`` uses the MTP names (``fc``,
    ``embedding_norm_weight``, ``hidden_norm_weight``, ``norm_weight``, ``final_norm_weight`` and ``layer.*``)."""
    eps = cfg.rms_norm_eps
    embedded = rms_norm(inputs_embeds, w["embedding_norm_weight"], eps)
    state = rms_norm(rms_norm(hidden, w["final_norm_weight"], eps), w["hidden_norm_weight"], eps)
    joined = torch.cat((embedded, state), dim=-1)
    x = linear_fp8(joined, w["fc"])
    layer_w = {name[len("layer.") :]: t for name, t in w.items() if name.startswith("layer.")}
    x = decoder_layer(cfg, "full_attention", layer_w, st, x, cos, sin, position, active, accepted=active)
    out = rms_norm(x, w["norm_weight"], eps)
    return (out.float() / (1.0 + w["final_norm_weight"].float())).to(x.dtype)


def mtp_prefill(cfg, w: dict, st: dict, hidden, inputs_embeds, cos, sin, slot, start, n_valid):
    """`MTPStep.forward` prefill form (model.py:843-855): only the layer's cache for the chunk is written
    (`cache_chunk`); returns ``x[:, :1]`` as the reference does."""
    eps = cfg.rms_norm_eps
    embedded = rms_norm(inputs_embeds, w["embedding_norm_weight"], eps)
    state = rms_norm(rms_norm(hidden, w["final_norm_weight"], eps), w["hidden_norm_weight"], eps)
    x = linear_fp8(torch.cat((embedded, state), dim=-1), w["fc"])
    layer_w = {name[len("layer.") :]: t for name, t in w.items() if name.startswith("layer.")}
    attention_cache_chunk(cfg, layer_w, st, rms_norm(x, layer_w["input_layernorm_weight"], eps), cos, sin, slot, start)
    return x[:, :1]


# ----------------------------------------------------------------------------------------------- prefill


def unit_lower_inverse(lower: torch.Tensor, base: int = 8) -> torch.Tensor:
    """`unit_lower_inverse` (model.py:127-153): ``(I - lower)^-1`` for strictly lower triangular ``lower``
    ``[..., n, n]``. Diagonal blocks of ``base`` as ``(I + L)(I + L^2)(I + L^4)`` (exact: ``L^base = 0`` there), then
    neighbouring blocks merged, the merged inverse's lower block being ``B^-1 C A^-1`` for ``[[A, 0], [C, B]]``."""
    n = lower.shape[-1]
    block_of = torch.arange(n) // base
    local = lower * (block_of.unsqueeze(-1) == block_of)
    inverse = torch.eye(n, dtype=lower.dtype) + local
    power = local
    for _ in range(int(math.log2(base)) - 1):
        power = power @ power
        inverse = inverse + inverse @ power
    size = base
    while size < n:
        merged = inverse.clone()
        for first in range(0, n, 2 * size):
            top, bottom = slice(first, first + size), slice(first + size, first + 2 * size)
            merged[..., bottom, top] = inverse[..., bottom, bottom] @ lower[..., bottom, top] @ inverse[..., top, top]
        inverse, size = merged, 2 * size
    return inverse


def chunked_gated_delta(query, key, value, log_decay, beta, state, chunk: int = DELTA_CHUNK):
    """`chunked_gated_delta` (model.py:88-124): the gated delta rule over ``tokens`` in pieces of ``chunk``.
    ``query``, ``key`` ``[heads, tokens, dk]`` (normed, query scaled), ``value`` ``[heads, tokens, dv]``,
    ``log_decay``, ``beta`` ``[heads, tokens]``, ``state`` ``[heads, dk, dv]``, all float32. Within a piece the
    cumulative log decay g, the decay matrix e^(g_i - g_j) (i >= j), the unit-lower solve of the in-piece coupling
    and its products; across pieces the state recurrence. Returns (outputs ``[heads, tokens, dv]``, final state)."""
    heads, tokens, dk = key.shape
    pieces = tokens // chunk
    q = query.reshape(heads, pieces, chunk, dk)
    k = key.reshape(heads, pieces, chunk, dk)
    v = value.reshape(heads, pieces, chunk, -1)
    g = log_decay.reshape(heads, pieces, chunk).cumsum(-1)
    b = beta.reshape(heads, pieces, chunk, 1)
    i = torch.arange(chunk)
    causal = (i.unsqueeze(-1) >= i.unsqueeze(0)).float()
    below = (i.unsqueeze(-1) > i.unsqueeze(0)).float()
    decay = ((g.unsqueeze(-1) - g.unsqueeze(-2)) * causal).exp() * causal
    k_beta = k * b
    inverse = unit_lower_inverse(-(k_beta @ k.transpose(-1, -2)) * decay * below)
    new_values = inverse @ (v * b)
    cumulative_keys = inverse @ (k_beta * g.exp().unsqueeze(-1))
    outputs = []
    for p in range(pieces):
        attn = (q[:, p] @ k[:, p].transpose(-1, -2)) * decay[:, p]
        v_new = new_values[:, p] - cumulative_keys[:, p] @ state
        outputs.append((q[:, p] * g[:, p].exp().unsqueeze(-1)) @ state + attn @ v_new)
        last = g[:, p, -1]
        carried = (k[:, p] * (last.unsqueeze(-1) - g[:, p]).exp().unsqueeze(-1)).transpose(-1, -2) @ v_new
        state = state * last.exp().reshape(heads, 1, 1) + carried
    return torch.cat(outputs, dim=1), state


def gdn_prefill(cfg, w: dict, st: dict, x, slot, start, n_valid):
    """`GatedDeltaNetStep.prefill` CPU branch (model.py:476-521): a chunk ``x`` ``[1, L, H]`` of row ``slot`` from
    ``start`` (0 restarts the row's states), tokens from ``n_valid`` on padding. Conv taps are bf16 products summed by
    bf16 additions; the chunked rule runs in float32 from the row's state; the new conv state is the last three real
    inputs. ``st`` entries of row ``slot`` are replaced."""
    dtype = x.dtype
    tokens = x.shape[1]
    kernel = cfg.linear_conv_kernel_dim
    slot, keep = slot.long(), (start > 0).to(dtype)
    valid = (torch.arange(tokens) < n_valid).float()
    qkv = linear_fp8(x, w["linear_attn.in_proj_qkv"])[0]
    history = st["conv_state"].index_select(0, slot)[0] * keep
    window = torch.cat((history.transpose(0, 1), qkv))
    carried = window.index_select(0, n_valid.long() + torch.arange(kernel - 1)).transpose(0, 1)
    st["conv_state"] = st["conv_state"].index_copy(0, slot, carried.unsqueeze(0))
    z = linear_fp8(x, w["linear_attn.in_proj_z"])[0]
    beta, log_decay = _gdn_gates(w, x[0])
    beta, log_decay = beta * valid.unsqueeze(-1), log_decay * valid.unsqueeze(-1)
    state = st["recurrent_state"].index_select(0, slot)[0].float() * keep.float()
    taps = window.transpose(0, 1)
    conv_weight = w["linear_attn.conv_weight"]
    conv = sum(taps[:, j : j + tokens] * conv_weight[:, j : j + 1] for j in range(kernel))
    query, key, value = _gdn_split(cfg, silu(conv).transpose(0, 1))
    out, state = chunked_gated_delta(
        query.transpose(0, 1), key.transpose(0, 1), value.transpose(0, 1), log_decay.transpose(0, 1), beta.transpose(0, 1),
        state, min(DELTA_CHUNK, tokens),
    )
    st["recurrent_state"] = st["recurrent_state"].index_copy(0, slot, state.unsqueeze(0).to(st["recurrent_state"].dtype))
    z = z.reshape(tokens, cfg.linear_num_value_heads, -1)
    return _gdn_finish(cfg, w, out.transpose(0, 1).to(dtype), z, dtype).reshape(1, tokens, -1)


def blocked_attention(query, keys, values, visible, block: int):
    """`blocked_attention` (model.py:170-191): softmax attention over positions in blocks of ``block`` with a running
    maximum and sum. ``query`` ``[kv_heads, queries, head]`` (scaled), ``keys``/``values`` ``[kv_heads, positions,
    head]``, ``visible`` bool ``[queries, positions]``. Scores are a bf16 matmul; each block's unnormalised weights
    go to bf16 for their matmul with the values, whose bf16 result is added in float32."""
    best = torch.full((*query.shape[:2], 1), 2 * MASKED_SCORE)
    total = torch.zeros(*query.shape[:2], 1)
    out = torch.zeros(*query.shape[:2], values.shape[-1])
    for first in range(0, keys.shape[1], block):
        scores = (query @ keys[:, first : first + block].transpose(-1, -2)).float()
        scores = scores + torch.where(visible[:, first : first + block], 0.0, MASKED_SCORE)
        new_best = torch.maximum(best, scores.amax(dim=-1, keepdim=True))
        weights = (scores - new_best).exp()
        rescale = (best - new_best).exp()
        total = total * rescale + weights.sum(dim=-1, keepdim=True)
        out = out * rescale + (weights.to(values.dtype) @ values[:, first : first + block]).float()
        best = new_best
    return out / total


def _write_chunk(st: dict, key, value, slot, start):
    """`FullAttentionStep._write_chunk` (model.py:791-799), ``key``/``value`` in the cache's format: row ``slot`` at
    ``start`` onward, every other row at the cache's last ``L`` positions (junk, never read before overwritten)."""
    rows, max_seq_len = st["k_cache"].shape[0], st["k_cache"].shape[2]
    tokens = key.shape[2]
    positions = start.long() + torch.arange(tokens)
    junk = max_seq_len - tokens + torch.arange(tokens)
    others = torch.arange(rows) != slot.long()
    where = torch.where(others.unsqueeze(-1), junk.unsqueeze(0), positions.unsqueeze(0))
    _write_both(st, key.expand(rows, -1, -1, -1), value.expand(rows, -1, -1, -1), where)


def attention_prefill(cfg, w: dict, st: dict, x, cos, sin, slot, start, n_valid):
    """`FullAttentionStep.prefill` CPU branch (model.py:704-783): the chunk's queries against row
    ``slot``'s cached positions before ``start`` and the chunk's own tokens causally, by `blocked_attention`; then the
    chunk's keys and values written (`_write_chunk`)."""
    head = cfg.head_dim
    tokens = x.shape[1]
    max_seq_len = st["k_cache"].shape[2]
    query, key, value, gate = _attention_project(cfg, w, x, cos, sin)
    groups = cfg.num_key_value_groups
    grouped = (query[0] * head**-0.5).reshape(cfg.num_key_value_heads, groups * tokens, head)
    ks, vs = kv_scales(st)
    cache_keys = kv_load(st["k_cache"].index_select(0, slot.long())[0], ks, x.dtype)
    cache_values = kv_load(st["v_cache"].index_select(0, slot.long())[0], vs, x.dtype)
    index = torch.arange(groups * tokens) % tokens
    visible = torch.cat(
        ((torch.arange(max_seq_len) < start).expand(groups * tokens, -1), torch.arange(tokens).unsqueeze(0) <= index.unsqueeze(-1)),
        dim=-1,
    )
    own_keys, own_values = kv_round_trip(key[0], ks, x.dtype), kv_round_trip(value[0], vs, x.dtype)
    out = blocked_attention(grouped, torch.cat((cache_keys, own_keys), dim=1), torch.cat((cache_values, own_values), dim=1),
                            visible, ATTENTION_BLOCK)
    out = out.to(x.dtype).reshape(cfg.num_attention_heads, tokens, head).transpose(0, 1).reshape(1, tokens, -1)
    _write_chunk(st, kv_store(key, ks), kv_store(value, vs), slot, start)
    return linear_fp8(out * torch.sigmoid(gate), w["self_attn.o_proj"])


def attention_cache_chunk(cfg, w: dict, st: dict, x, cos, sin, slot, start):
    """`FullAttentionStep.cache_chunk` (model.py:784-790): only the chunk's keys and values, written as prefill does."""
    _, key, value, _ = _attention_project(cfg, w, x, cos, sin)
    ks, vs = kv_scales(st)
    _write_chunk(st, kv_store(key, ks), kv_store(value, vs), slot, start)


# ----------------------------------------------------------------------------------------------- head and acceptance


def head_group_maxima(cfg, norm_weight, lm_head: FP8Weight, hidden, group_rows: int = 32):
    """`HeadStep.forward` CPU branch (model.py:890-895), tp 1: final norm in hidden's dtype, float32 logits, the
    largest in each group of ``group_rows`` tokens. ``hidden`` ``[R, 1, H]`` -> ``[R, V / group_rows]``."""
    x = rms_norm(hidden, norm_weight, cfg.rms_norm_eps).reshape(hidden.shape[0], -1)
    logits = x.float() @ lm_head.dense_t()
    return torch.stack([g.amax(dim=-1) for g in logits.split(group_rows, dim=-1)], dim=-1)


def chip_next_tokens(cfg, norm_weight, lm_head: FP8Weight, hidden, maxima, recheck_groups: int = 4, group_rows: int = 32,
                     rows_bf16: torch.Tensor | None = None):
    """`ChipHead.next_tokens` after the graph (generate.py:194-208): the best ``recheck_groups`` groups by maxima,
    exact float32 logits inside them from float32-normed hidden, the first strictly larger in top-k order wins. The
    reference rechecks against the checkpoint's bf16 lm_head (its ``self.lm_head``); ``rows_bf16`` is that matrix
    [V, H], else the FP8 weight's values stand in for it (a synthetic lm_head that is e4m3 to begin with)."""
    rows = hidden.shape[0]
    maxima = maxima[:rows].float()
    best_groups = maxima.topk(min(recheck_groups, maxima.shape[-1]), dim=-1).indices.tolist()
    norm = rms_norm(hidden.float(), norm_weight, cfg.rms_norm_eps).squeeze(1)
    dense = lm_head.dense().contiguous().to(torch.bfloat16) if rows_bf16 is None else rows_bf16
    tokens = []
    for row, groups in enumerate(best_groups):
        best_token, best_logit = -1, -torch.inf
        for group in groups:
            first = group * group_rows
            logit, index = (dense[first : first + group_rows].float() @ norm[row]).max(dim=0)
            if logit > best_logit:
                best_token, best_logit = first + int(index), logit
        if best_token < 0:
            raise FloatingPointError(f"row {row}'s logits are not finite, so the graph produced NaN or infinity")
        tokens.append(best_token)
    return tokens


def host_next_tokens(cfg, norm_weight, lm_head: FP8Weight, hidden):
    """`HostHead.next_tokens` (generate.py:156-159): argmax over the whole vocabulary in float32."""
    norm = rms_norm(hidden.float(), norm_weight, cfg.rms_norm_eps).squeeze(1)
    return torch.argmax(norm @ lm_head.dense_t(), dim=-1).tolist()


def accept(picks: list, drafts: list, k: int):
    """Greedy longest-prefix acceptance (scheduler.py:291-298): leading drafts equal to the model's picks are kept,
    then the model's own next pick. Returns (match, emitted)."""
    match = 0
    while match < k - 1 and drafts[match] == picks[match]:
        match += 1
    return match, picks[: match + 1]


def top2_gap(cfg, norm_weight, lm_head: FP8Weight, hidden) -> torch.Tensor:
    """Per row, the gap between the two largest float32 logits: rows under 1e-3 are near-ties, where a pick may
    legitimately differ between two correct implementations."""
    norm = rms_norm(hidden.float(), norm_weight, cfg.rms_norm_eps).squeeze(1)
    top = (norm @ lm_head.dense_t()).topk(2, dim=-1).values
    return top[:, 0] - top[:, 1]
