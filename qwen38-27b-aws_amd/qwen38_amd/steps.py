"""Step objects with the reference's call contracts, running on libq38 (the HIP library) on one GPU.

* `VerifyStep.__call__(inputs_embeds, cos, sin, position, active, accepted)` -> hidden ``[B, K, H]``: the reference's
  verify graph, `Qwen38Step.forward` with `accepted` (qwen38_inf2/model.py:933-995, called at scheduler.py:288).
* `StepGraph.__call__(inputs_embeds, cos, sin, position, active)` -> hidden ``[B, 1, H]``: the one-token decode graph
  (`Qwen38Step.forward`'s decode form, called at generate.py:251,258,290); with ``save_slot`` or ``restore_slot``
  instead, it saves or restores one row's gated-delta states and returns ``inputs_embeds`` (model.py:988-992, called
  at scheduler.py:119,133); with ``accepted`` it is the verify graph.
* `MTPStep.__call__(hidden, inputs_embeds, cos, sin, position, active)` -> ``[B, K, H]``: `MTPStep.forward`
  (model.py:843-860, called at scheduler.py:179,192).
* `HeadGraph.__call__(hidden=[R, 1, H])` -> group maxima ``[R, V/32]`` float32: the head graph `run_graph`
  (`HeadStep.forward`, model.py:890-900, called at generate.py:195); `pick` runs `ChipHead.next_tokens`'s recheck on the
  GPU too, and `embed` gathers embedding rows.

`Engine` owns every device buffer the library uses (weights packed once, recurrent/conv/snapshot states, KV caches, the
workspace) and binds them to one handle. Inputs may be host or device tensors; outputs are device tensors.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence

import torch

from . import ext
from .config import FULL, LINEAR, TextConfig

DTYPE = torch.bfloat16


def _interleave32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Rows of a and b alternating in blocks of 32: the gate/up tile pairs the SwiGLU epilogue reads."""
    n = a.shape[0]
    return torch.stack((a.reshape(n // 32, 32, -1), b.reshape(n // 32, 32, -1)), dim=1).reshape(2 * n, -1)


def _cat_fp8(parts: Sequence[tuple[torch.Tensor, torch.Tensor]]):
    return torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])


class Engine:
    """Device state of one loaded model: a q38 handle plus the tensors bound to it."""

    def __init__(self, cfg: TextConfig, batch_size: int, verify_tokens: int, max_seq_len: int, mtp: bool = True, device="cuda",
                 saved_states: bool = False, prefill_chunk: int = 0, weight_format: str = "e4m3", kv_cache_format: str = "bf16",
                 projection_mfma: str = "bf16"):
        if not torch.cuda.is_available():
            raise RuntimeError("the verify path runs on the GPU only")
        self.cfg, self.batch_size, self.verify_tokens, self.max_seq_len, self.mtp = cfg, batch_size, verify_tokens, max_seq_len, mtp
        self.saved_states, self.prefill_chunk, self.weight_format = saved_states, prefill_chunk, weight_format
        self.kv_cache_format = kv_cache_format
        self.device = torch.device(device)
        self.projection_mfma = projection_mfma
        self.handle = ext.Handle(cfg, batch_size, verify_tokens, max_seq_len, mtp, saved_states, prefill_chunk, weight_format,
                                 kv_cache_format, projection_mfma)
        kv_dtype = torch.uint8 if kv_cache_format == "fp8" else DTYPE
        self.buffers: dict[tuple[str, int], torch.Tensor] = {}
        self.mtp_layer = cfg.num_hidden_layers
        self._bind_zeros("workspace", -1, torch.uint8)
        for i, kind in enumerate(cfg.layer_types):
            if kind == LINEAR:
                self._bind_zeros("linear_attn.recurrent_state", i, DTYPE)
                self._bind_zeros("linear_attn.conv_state", i, DTYPE)
                self._bind_zeros("linear_attn.pending_key", i, torch.float32)
                self._bind_zeros("linear_attn.pending_delta", i, torch.float32)
                self._bind_zeros("linear_attn.pending_decay", i, torch.float32)
                self._bind_zeros("linear_attn.pending_input", i, DTYPE)
                if saved_states:
                    self._bind_zeros("linear_attn.saved_state", i, DTYPE)
                    self._bind_zeros("linear_attn.saved_conv", i, DTYPE)
            else:
                self._bind_zeros("self_attn.k_cache", i, kv_dtype)
                self._bind_zeros("self_attn.v_cache", i, kv_dtype)
        if mtp:
            self._bind_zeros("self_attn.k_cache", self.mtp_layer, kv_dtype)
            self._bind_zeros("self_attn.v_cache", self.mtp_layer, kv_dtype)
        if verify_tokens >= 2:
            # cos/sin of every position, which the on-device speculative steps gather by the positions they compute.
            from .generate import rope_table

            self.bind("rope_table", -1, rope_table(cfg, max_seq_len))

    # ------------------------------------------------------------------------------------------------ buffers

    def _bind_zeros(self, name: str, layer: int, dtype: torch.dtype) -> torch.Tensor:
        nbytes = self.handle.buffer_size(name, layer)
        size = torch.empty((), dtype=dtype).element_size()
        t = torch.zeros(nbytes // size, dtype=dtype, device=self.device)
        return self.bind(name, layer, t)

    def bind(self, name: str, layer: int, t: torch.Tensor) -> torch.Tensor:
        t = t.to(self.device).contiguous()
        self.handle.bind(name, layer, t)
        self.buffers[(name, layer)] = t
        return t

    def buffer(self, name: str, layer: int) -> torch.Tensor:
        return self.buffers[(name, layer)]

    # ------------------------------------------------------------------------------------------------ weights

    def _fp8(self, name: str, layer: int, coded: torch.Tensor, scales: torch.Tensor) -> None:
        """A projection: (e4m3 bytes [N, K], E8M0 [N, K/32]); for a decoder layer of an "mxfp4" engine the checkpoint's
        (packed E2M1 [N, K/2], E8M0 [N, K/32]) instead."""
        if self.weight_format == "mxfp4" and 0 <= layer < self.cfg.num_hidden_layers:
            if coded.shape[1] * 2 != scales.shape[1] * 32:
                raise ValueError(f"{name} of layer {layer}: an mxfp4 engine takes packed E2M1 weights [N, K/2]")
            tiles, scales_t = ext.pack_weight_fp4(coded.to(self.device), scales.to(self.device))
        else:
            tiles, scales_t = ext.pack_weight(coded.to(self.device), scales.to(self.device))
        self.bind(name + ".tiles", layer, tiles)
        self.bind(name + ".scales", layer, scales_t)

    def load_layer(self, layer: int, w: dict, kind: str) -> None:
        """One decoder layer's weights by the reference's short names (synth.layer_specs without the prefix)."""
        self.bind("input_layernorm", layer, w["input_layernorm_weight"])
        self.bind("post_attention_layernorm", layer, w["post_attention_layernorm_weight"])
        g, u = w["mlp.gate_proj"], w["mlp.up_proj"]
        self._fp8("mlp.gate_up", layer, _interleave32(g[0], u[0]), _interleave32(g[1], u[1]))
        self._fp8("mlp.down", layer, *w["mlp.down_proj"])
        if kind == LINEAR:
            la = "linear_attn."
            self._fp8(la + "in_proj_qkvz", layer, *_cat_fp8([w[la + "in_proj_qkv"], w[la + "in_proj_z"]]))
            self._fp8(la + "out_proj", layer, *w[la + "out_proj"])
            for key in ("in_proj_a", "in_proj_b", "conv_weight", "A_log", "dt_bias", "norm_weight"):
                self.bind(la + key, layer, w[la + key].to(DTYPE))
        else:
            sa = "self_attn."
            self._fp8(sa + "qkv", layer, *_cat_fp8([w[sa + "q_proj"], w[sa + "k_proj"], w[sa + "v_proj"]]))
            self._fp8(sa + "o_proj", layer, *w[sa + "o_proj"])
            self.bind(sa + "q_norm", layer, w[sa + "q_norm_weight"])
            self.bind(sa + "k_norm", layer, w[sa + "k_norm_weight"])

    def load(self, weights: Iterable[tuple[str, object]]) -> None:
        """Weights by their full names (`synth.model_specs`): ``layers.{i}.*``, ``mtp.*``, ``head.*``, ``embed_tokens``.
        Consumed layer by layer, so a generator keeps host and device peaks to one layer."""
        pending: dict[int, dict] = {}
        need = {}
        for name, value in weights:
            if name.startswith("layers."):
                i = int(name.split(".")[1])
                short = name[len(f"layers.{i}.") :]
                pending.setdefault(i, {})[short] = value
                kind = self.cfg.layer_types[i]
                if i not in need:
                    need[i] = self._layer_names(kind)
                if need[i] <= set(pending[i]):
                    self.load_layer(i, pending.pop(i), kind)
            elif name.startswith("mtp.layer."):
                pending.setdefault(self.mtp_layer, {})[name[len("mtp.layer.") :]] = value
                if self._layer_names(FULL) <= set(pending[self.mtp_layer]):
                    self.load_layer(self.mtp_layer, pending.pop(self.mtp_layer), FULL)
            elif name == "mtp.fc":
                self._fp8("mtp.fc", self.mtp_layer, *value)
            elif name in ("mtp.embedding_norm_weight", "mtp.hidden_norm_weight", "mtp.norm_weight"):
                self.bind(name[: -len("_weight")], self.mtp_layer, value)
            elif name == "head.norm_weight":
                self.bind("head.norm", -1, value)
            elif name == "head.lm_head":
                self._fp8("head.lm_head", -1, *value)
            elif name == "head.lm_head_rows":
                # The checkpoint's bf16 lm_head: the head's exact recheck reads these rows (the maxima use the tiles).
                self.bind("head.lm_head.rows", -1, value)
            elif name == "embed_tokens":
                self.bind("embed_tokens", -1, value)
            else:
                raise KeyError(f"unknown weight {name}")
        if pending:
            raise ValueError(f"incomplete layers {sorted(pending)}")

    @staticmethod
    def _layer_names(kind: str) -> set:
        from .config import tiny_config, with_layers
        from .synth import layer_specs

        return {s.name[len("layers.0.") :] for s in layer_specs(with_layers(tiny_config(1), (kind,)), 0)}

    # ------------------------------------------------------------------------------------------------ state views

    @property
    def parity(self) -> int:
        return self.handle.parity

    def gdn_state(self, layer: int, current: bool = True) -> dict:
        """Views of a gated-delta layer's state in the reference's buffer shapes where they agree: recurrent_state
        [B,Hv,d,d], conv_state [B,C,3], pending_key [B,K,Hk,d] (one per key head; the reference repeats it per value
        head), pending_delta [B,K,Hv,d], pending_decay [B,K,Hv], pending_input [B,K,C]. ``current`` picks the half the
        next verify step reads."""
        cfg, b, k = self.cfg, self.batch_size, self.verify_tokens
        half = self.parity if current else 1 - self.parity
        hv, hk, d, c = cfg.linear_num_value_heads, cfg.linear_num_key_heads, cfg.linear_key_head_dim, cfg.linear_conv_dim
        get = lambda n: self.buffer("linear_attn." + n, layer)
        return {
            "recurrent_state": get("recurrent_state").view(b, hv, d, d),
            "conv_state": get("conv_state").view(2, b, c, 3)[half],
            "pending_key_state": get("pending_key").view(2, b, k, hk, d)[half],
            "pending_delta_state": get("pending_delta").view(2, b, k, hv, d)[half],
            "pending_decay_state": get("pending_decay").view(2, b, k, hv)[half],
            "pending_input_state": get("pending_input").view(2, b, k, c)[half],
        }

    def enable_probe(self, layer: int) -> None:
        """Bind layer ``layer``'s optional probe: later verify calls copy the layer's intermediate activations into it
        (include/q38.h), read back with `probe`."""
        self._bind_zeros("probe", layer, torch.uint8)

    def probe(self, layer: int, flat: torch.Tensor | None = None) -> dict:
        """The last verify call's intermediates of layer ``layer`` (or the last MTP call's, for ``mtp_layer``), for
        ``T = B*K`` tokens: ``normed`` [T, H] (gated-delta layers), ``projection`` [T, P] (in_proj_z, or the attention
        q|gate|k|v projection), ``inner`` [T, Hv*128] (the gated-delta in-step output before its gated norm; empty for
        attention), ``mixed`` [T, H] (the residual after the mixer), all bf16; the e5m2 GEMM inputs as bf16 values:
        ``mid`` (out_proj/o_proj input), ``mlp_in`` [T, H], ``ffn`` [T, I]; and ``input`` [T, H] bf16, the residual
        stream entering the layer (for the MTP layer, its fc output). ``flat`` parses a saved copy of the probe buffer
        instead of the bound one."""
        cfg = self.cfg
        t, hsz = self.batch_size * self.verify_tokens, cfg.hidden_size
        linear = layer < cfg.num_hidden_layers and cfg.layer_types[layer] == LINEAR
        width = cfg.linear_value_dim if linear else cfg.num_attention_heads * cfg.head_dim * 2 + 2 * cfg.num_key_value_heads * cfg.head_dim
        mid = cfg.linear_value_dim if linear else cfg.num_attention_heads * cfg.head_dim
        inner = cfg.linear_value_dim if linear else 0
        flat = self.buffer("probe", layer) if flat is None else flat
        bf = flat[: t * (2 * hsz + width + inner) * 2].view(DTYPE)
        out = {"normed": bf[: t * hsz].view(t, hsz), "projection": bf[t * hsz : t * (hsz + width)].view(t, width),
               "inner": bf[t * (hsz + width) : t * (hsz + width + inner)].view(t, inner),
               "mixed": bf[t * (hsz + width + inner) :].view(t, hsz)}
        at, t32 = t * (2 * hsz + width + inner) * 2, (t + 31) // 32 * 32
        for name, k in (("mid", mid), ("mlp_in", hsz), ("ffn", cfg.intermediate_size)):
            out[name] = act_tiles_to_rows(flat[at : at + t32 * k], t32, k)[:t]
            at += t32 * k
        out["input"] = flat[at : at + t * hsz * 2].view(DTYPE).view(t, hsz)
        return out

    def enable_head_probe(self) -> None:
        """Bind the head's optional probe: later head calls copy their normed rows into it, read back with
        `head_probe`."""
        self._bind_zeros("head.probe", -1, DTYPE)

    def head_probe(self, rows: int) -> torch.Tensor:
        """The last head call's normed rows ``[rows, H]`` bf16 (the final norm's output the group-max GEMM reads)."""
        h = self.cfg.hidden_size
        t32 = (rows + 31) // 32 * 32
        tiles = self.buffer("head.probe", -1)[: t32 * h]
        return tiles[tile_offsets(t32, h, tiles.device)].reshape(t32, h)[:rows]

    def kv_cache(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(k_cache [B,Hkv,S,hd], v_cache stored transposed [B,Hkv,S/32,hd,32])."""
        cfg, b, s = self.cfg, self.batch_size, self.max_seq_len
        kc = self.buffer("self_attn.k_cache", layer).view(b, cfg.num_key_value_heads, s, cfg.head_dim)
        vc = self.buffer("self_attn.v_cache", layer).view(b, cfg.num_key_value_heads, s // 32, cfg.head_dim, 32)
        return kc, vc

    def set_kv_scales(self, layer: int, k_scale: torch.Tensor, v_scale: torch.Tensor) -> None:
        """An FP8 cache's static scales for one attention layer (the MTP layer included): bf16 ``[1]`` each, the
        reference's ``self_attn.k_scale`` / ``v_scale`` (model.py:559-561, checkpoint.py:227-233)."""
        self.bind("self_attn.k_scale", layer, k_scale.reshape(1).to(DTYPE))
        self.bind("self_attn.v_scale", layer, v_scale.reshape(1).to(DTYPE))

    def set_kv(self, layer: int, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
        """Write reference-layout caches [B,Hkv,S,hd] (bf16, or e4m3 bytes for an FP8 cache)."""
        kc, vc = self.kv_cache(layer)
        kc.copy_(k_cache)
        b, h, s, d = v_cache.shape
        vc.copy_(v_cache.reshape(b, h, s // 32, 32, d).transpose(-1, -2))

    def get_kv(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Caches in the reference layout [B,Hkv,S,hd]."""
        kc, vc = self.kv_cache(layer)
        b, h, n, d, _ = vc.shape
        return kc.clone(), vc.transpose(-1, -2).reshape(b, h, n * 32, d)

    def set_gdn(self, layer: int, st: dict) -> None:
        """Load reference-shaped gated-delta state (pending_key_state per value head) into the current half."""
        mine = self.gdn_state(layer)
        rep = self.cfg.linear_key_repeat
        for key, value in st.items():
            value = value.to(self.device)
            if key == "pending_key_state":
                value = value[:, :, ::rep]
            mine[key].copy_(value)


def tile_offsets(tokens: int, k: int, device) -> torch.Tensor:
    """Element index of each (token, input) in the GEMMs' activation tile layout (tiles of 32 tokens x 64 inputs,
    token-block major; inside a tile ``[m][lane][8]`` with lane = t % 32 + 32 * ((k % 32) // 16) and element
    e = 16 * ((k % 64) // 32) + k % 16, m = e // 8), flat over ``[tokens, k]``."""
    t = torch.arange(tokens, device=device).unsqueeze(1)
    c = torch.arange(k, device=device).unsqueeze(0)
    e = ((c % 64) // 32) * 16 + (c % 16)
    lane = t % 32 + 32 * ((c % 32) // 16)
    return (((t // 32) * (k // 64) + c // 64) * 2048 + (e // 8) * 512 + lane * 8 + e % 8).reshape(-1)


def act_tiles_to_rows(tiles: torch.Tensor, tokens: int, k: int) -> torch.Tensor:
    """e5m2 activation tiles (`tile_offsets`' layout, one byte per element) as bf16 values ``[tokens, k]``."""
    return tiles[tile_offsets(tokens, k, tiles.device)].view(torch.float8_e5m2).to(DTYPE).reshape(tokens, k)


def _dev(t: torch.Tensor, dtype: torch.dtype, device) -> torch.Tensor:
    return t.to(device=device, dtype=dtype, non_blocking=True).contiguous()


class VerifyStep:
    """The verify graph over the engine's B rows and K tokens per row."""

    def __init__(self, engine: Engine):
        self.engine = engine

    def __call__(self, inputs_embeds: torch.Tensor, **inputs: torch.Tensor) -> torch.Tensor:
        e = self.engine
        if "accepted" not in inputs:
            raise NotImplementedError("only the verify form (inputs with `accepted`) runs on this build")
        b, k, h = e.batch_size, e.verify_tokens, e.cfg.hidden_size
        if tuple(inputs_embeds.shape) != (b, k, h):
            raise ValueError(f"inputs_embeds must be [{b}, {k}, {h}], got {list(inputs_embeds.shape)}")
        dev = e.device
        out = torch.empty(b, k, h, dtype=DTYPE, device=dev)
        e.handle.verify(
            _dev(inputs_embeds, DTYPE, dev), _dev(inputs["cos"], DTYPE, dev), _dev(inputs["sin"], DTYPE, dev),
            _dev(inputs["position"], torch.int32, dev), _dev(inputs["active"], torch.float32, dev),
            _dev(inputs["accepted"], torch.int32, dev), out,
        )
        return out


class StepGraph:
    """The step graph's other calls over the engine's B rows (the reference's `Qwen38Step.forward`, model.py:983-995):
    one-token decode, saving or restoring one row's gated-delta states, and (with ``accepted``) verify."""

    def __init__(self, engine: Engine):
        self.engine = engine
        self.verify = VerifyStep(engine)

    def __call__(self, inputs_embeds: torch.Tensor, cos=None, sin=None, position=None, active=None, slot=None, start=None,
                 n_valid=None, save_slot=None, restore_slot=None, accepted=None) -> torch.Tensor:
        e = self.engine
        if save_slot is not None or restore_slot is not None:
            if not e.saved_states:
                raise ValueError("this layer keeps no saved states")
            which = save_slot if save_slot is not None else restore_slot
            e.handle.copy_states(_dev(torch.as_tensor(which).reshape(1), torch.int32, e.device), save_slot is not None)
            return inputs_embeds
        if slot is not None:
            return self._prefill(inputs_embeds, cos, sin, slot, start, n_valid)
        if accepted is not None:
            return self.verify(inputs_embeds, cos=cos, sin=sin, position=position, active=active, accepted=accepted)
        b, h = e.batch_size, e.cfg.hidden_size
        if tuple(inputs_embeds.shape) != (b, 1, h):
            raise ValueError(f"inputs_embeds must be [{b}, 1, {h}], got {list(inputs_embeds.shape)}")
        dev = e.device
        out = torch.empty(b, 1, h, dtype=DTYPE, device=dev)
        e.handle.decode(
            _dev(inputs_embeds, DTYPE, dev), _dev(cos, DTYPE, dev), _dev(sin, DTYPE, dev), _dev(position, torch.int32, dev),
            _dev(active, torch.float32, dev), out,
        )
        return out


    def _prefill(self, inputs_embeds, cos, sin, slot, start, n_valid) -> torch.Tensor:
        """One chunk ``[1, L, H]`` of row ``slot`` from ``start`` (model.py:476-521, 704-783); returns ``[1, L, H]``."""
        e = self.engine
        chunk = _check_chunk(e, inputs_embeds, slot, start, n_valid)
        dev, h = e.device, e.cfg.hidden_size
        out = torch.empty(1, chunk, h, dtype=DTYPE, device=dev)
        e.handle.prefill(
            _dev(inputs_embeds.reshape(chunk, h), DTYPE, dev), _dev(cos.reshape(chunk, -1), DTYPE, dev),
            _dev(sin.reshape(chunk, -1), DTYPE, dev), _dev(slot.reshape(1), torch.int32, dev),
            _dev(start.reshape(1), torch.int32, dev), _dev(n_valid.reshape(1), torch.int32, dev), chunk, out,
        )
        return out


def _check_chunk(e, inputs_embeds, slot, start, n_valid) -> int:
    """The host-side checks of a prefill chunk's inputs (the device reads slot, start and n_valid itself)."""
    if not e.prefill_chunk:
        raise ValueError("the engine was built without a prefill chunk (prefill_chunk=0)")
    if inputs_embeds.dim() != 3 or inputs_embeds.shape[0] != 1 or inputs_embeds.shape[2] != e.cfg.hidden_size:
        raise ValueError(f"inputs_embeds must be [1, chunk, {e.cfg.hidden_size}], got {list(inputs_embeds.shape)}")
    chunk = inputs_embeds.shape[1]
    if chunk % 32 or chunk > e.prefill_chunk:
        raise ValueError(f"a chunk holds a multiple of 32 tokens up to {e.prefill_chunk}, got {chunk}")
    s, st, n = int(torch.as_tensor(slot).reshape(-1)[0]), int(torch.as_tensor(start).reshape(-1)[0]), int(torch.as_tensor(n_valid).reshape(-1)[0])
    if not 0 <= s < e.batch_size or st < 0 or st + chunk > e.max_seq_len or not 0 < n <= chunk:
        raise ValueError(f"slot {s}, start {st}, n_valid {n} do not fit a chunk of {chunk} in {e.batch_size} rows of {e.max_seq_len}")
    return chunk


class MTPStep:
    """The MTP drafter's step form over [B, K] rows and tokens."""

    def __init__(self, engine: Engine):
        if not engine.mtp:
            raise ValueError("the engine was built without the MTP layer")
        self.engine = engine

    def __call__(self, hidden: torch.Tensor, inputs_embeds: torch.Tensor, **inputs: torch.Tensor) -> torch.Tensor:
        e = self.engine
        if inputs.get("slot") is not None:
            return self._prefill(hidden, inputs_embeds, **inputs)
        b, k, h = e.batch_size, e.verify_tokens, e.cfg.hidden_size
        for name, t in (("hidden", hidden), ("inputs_embeds", inputs_embeds)):
            if tuple(t.shape) != (b, k, h):
                raise ValueError(f"{name} must be [{b}, {k}, {h}], got {list(t.shape)}")
        dev = e.device
        out = torch.empty(b, k, h, dtype=DTYPE, device=dev)
        e.handle.mtp_step(
            _dev(hidden, DTYPE, dev), _dev(inputs_embeds, DTYPE, dev), _dev(inputs["cos"], DTYPE, dev),
            _dev(inputs["sin"], DTYPE, dev), _dev(inputs["position"], torch.int32, dev),
            _dev(inputs["active"], torch.float32, dev), out,
        )
        return out


    def _prefill(self, hidden, inputs_embeds, cos, sin, slot, start, n_valid, **_) -> torch.Tensor:
        """The prefill form (model.py:843-855): only the layer's cache for the chunk; returns the fc output's first
        row ``[1, 1, H]`` as the reference does."""
        e = self.engine
        chunk = _check_chunk(e, inputs_embeds, slot, start, n_valid)
        if tuple(hidden.shape) != tuple(inputs_embeds.shape):
            raise ValueError(f"hidden must be {list(inputs_embeds.shape)}, got {list(hidden.shape)}")
        dev, h = e.device, e.cfg.hidden_size
        out = torch.empty(1, 1, h, dtype=DTYPE, device=dev)
        e.handle.mtp_prefill(
            _dev(hidden.reshape(chunk, h), DTYPE, dev), _dev(inputs_embeds.reshape(chunk, h), DTYPE, dev),
            _dev(cos.reshape(chunk, -1), DTYPE, dev), _dev(sin.reshape(chunk, -1), DTYPE, dev),
            _dev(slot.reshape(1), torch.int32, dev), _dev(start.reshape(1), torch.int32, dev), chunk, out,
        )
        return out


class HeadGraph:
    """The head: group maxima, the exact top-group recheck and embedding rows, all on the GPU."""

    def __init__(self, engine: Engine, group_rows: int = 32):
        if group_rows != 32:
            raise ValueError("the head's groups are 32 rows (one weight tile)")
        self.engine = engine
        self.batch_size = engine.batch_size * engine.verify_tokens

    def _rows(self, hidden: torch.Tensor) -> torch.Tensor:
        e = self.engine
        rows = hidden.reshape(-1, e.cfg.hidden_size)
        if rows.shape[0] > self.batch_size:
            raise ValueError(f"the head takes at most {self.batch_size} rows, got {rows.shape[0]}")
        return _dev(rows, DTYPE, e.device)

    def __call__(self, hidden: torch.Tensor) -> torch.Tensor:
        rows = self._rows(hidden)
        maxima = torch.empty(rows.shape[0], self.engine.cfg.vocab_size // 32, dtype=torch.float32, device=rows.device)
        self.engine.handle.head_groupmax(rows, rows.shape[0], maxima)
        return maxima

    def pick(self, hidden: torch.Tensor, groups: int) -> torch.Tensor:
        """Greedy token per row (`ChipHead.next_tokens`); raises FloatingPointError for a row with no finite logit."""
        rows = self._rows(hidden)
        ids = torch.empty(rows.shape[0], dtype=torch.int32, device=rows.device)
        self.engine.handle.head_pick(rows, rows.shape[0], groups, ids)
        ids = ids.cpu()
        bad = (ids < 0).nonzero()
        if len(bad):
            raise FloatingPointError(f"row {int(bad[0])}'s logits are not finite, so the graph produced NaN or infinity")
        return ids

    def embed(self, token_ids) -> torch.Tensor:
        e = self.engine
        ids = torch.as_tensor(list(token_ids), dtype=torch.int32)
        if len(ids) and (int(ids.min()) < 0 or int(ids.max()) >= e.cfg.vocab_size):
            raise ValueError(f"token ids must be in [0, {e.cfg.vocab_size})")
        out = torch.empty(len(ids), e.cfg.hidden_size, dtype=DTYPE, device=e.device)
        if len(ids):
            e.handle.embed(ids.to(e.device), len(ids), out)
        return out


class LookupStep:
    """Speculative verify steps with prompt-lookup drafts: the reference's `Scheduler._verify_step` without an MTP
    drafter (scheduler.py:269-301) for the engine's B slots. Each slot's `drafting.Drafter` runs on the host over the
    row's tokens; the step itself (embedding of ``[last token] + drafts``, the K-token verify with the accepted-prefix
    commit, the head's picks over every row's K tokens, acceptance, position advance) is one `q38_verify_step` call
    on the device. The picks and matches come back to the host once per step, as the drafter needs them.

    ``rows[b]`` is slot b's token ids so far (prompt and the tokens chosen after it), or None for an empty slot;
    ``written[b]`` how many of them are in the slot's cache and states (after a prefill: the prompt length)."""

    def __init__(self, engine: Engine, rows: Sequence[Sequence[int] | None], written: Sequence[int]):
        from .drafting import Drafter

        e = self.engine = engine
        b, k = e.batch_size, e.verify_tokens
        if len(rows) != b or len(written) != b:
            raise ValueError(f"LookupStep needs one row and one written count per slot ({b})")
        if k < 2:
            raise ValueError("speculative steps need at least 2 verify tokens")
        dev = e.device
        self.drafters = [Drafter(ids) if ids is not None else None for ids in rows]
        picks = torch.zeros(b, k, dtype=torch.int32)
        for slot, ids in enumerate(rows):
            if ids is not None:
                picks[slot, 0] = ids[-1]
        self.position = torch.tensor(list(written), dtype=torch.int32, device=dev)
        self.index = torch.zeros(b, dtype=torch.int32, device=dev)
        self.match = torch.zeros(b, dtype=torch.int32, device=dev)
        self.accepted = torch.zeros(b, dtype=torch.int32, device=dev)
        self.active = torch.tensor([float(ids is not None) for ids in rows], device=dev)
        self.hidden = torch.zeros(b, k, e.cfg.hidden_size, dtype=DTYPE, device=dev)
        self.picks = picks.to(dev)
        self.drafts = torch.zeros(b, k - 1, dtype=torch.int32, device=dev)

    def __call__(self) -> list[list[int] | None]:
        """One step for every running slot; returns each slot's new tokens (the drafts the model chose too, then its
        own next pick), or None for an empty slot."""
        from .drafting import padded_draft

        e = self.engine
        k = e.verify_tokens
        host = torch.zeros(e.batch_size, k - 1, dtype=torch.int32)
        for slot, drafter in enumerate(self.drafters):
            if drafter is not None:
                host[slot] = torch.tensor(padded_draft(drafter, drafter.tokens[-1], k - 1), dtype=torch.int32)
        self.drafts.copy_(host)
        e.handle.verify_step(self.position, self.index, self.match, self.accepted, self.active, self.hidden, self.picks,
                             self.drafts)
        picks, match = self.picks.cpu(), self.match.cpu()
        e.handle.raise_step_errors()
        out: list[list[int] | None] = []
        for slot, drafter in enumerate(self.drafters):
            if drafter is None:
                out.append(None)
                continue
            tokens = picks[slot, : int(match[slot]) + 1].tolist()
            drafter.extend(tokens)
            out.append(tokens)
        return out
