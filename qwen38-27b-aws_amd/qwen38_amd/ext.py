"""ctypes binding of libq38.so (include/q38.h). Device tensors are passed as raw pointers on torch's current HIP stream.

There is no fallback: if the library is missing or was built for another architecture, `library()` raises, and every
step object fails with it. Build it with `python -m qwen38_amd.build` (or `__graft_entry__.build()`).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from .config import FULL, LINEAR, TextConfig

LIB_PATH = Path(__file__).resolve().parent / "libq38.so"
MAX_LAYERS = 128

EXPORTS = (
    "q38_last_error", "q38_create", "q38_destroy", "q38_buffer_size", "q38_bind", "q38_parity", "q38_set_parity",
    "q38_pack_weight", "q38_pack_weight_fp4", "q38_mxfp4_linear", "q38_fp4_linear", "q38_fp4_linear_scratch", "q38_fp8_linear", "q38_fp8_linear_scratch", "q38_fp8_linear_f32", "q38_fp8_linear_mfma", "q38_fp8_linear_noalloc", "q38_mlp_up", "q38_tiles_size", "q38_verify", "q38_decode", "q38_copy_states", "q38_prefill", "q38_mtp_prefill", "q38_mtp_step", "q38_head_groupmax", "q38_head_pick", "q38_embed", "q38_accept", "q38_spec_step", "q38_spec_step_graph", "q38_verify_step", "q38_step_status",
    "q38_kernel_timer",
)


class Q38Config(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int), ("intermediate_size", ctypes.c_int), ("vocab_size", ctypes.c_int),
        ("num_layers", ctypes.c_int), ("layer_types", ctypes.c_int * MAX_LAYERS),
        ("num_attention_heads", ctypes.c_int), ("num_key_value_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
        ("rotary_dim", ctypes.c_int),
        ("linear_num_key_heads", ctypes.c_int), ("linear_num_value_heads", ctypes.c_int),
        ("linear_key_head_dim", ctypes.c_int), ("linear_value_head_dim", ctypes.c_int),
        ("linear_conv_kernel_dim", ctypes.c_int), ("rms_norm_eps", ctypes.c_float),
        ("batch_size", ctypes.c_int), ("verify_tokens", ctypes.c_int), ("max_seq_len", ctypes.c_int), ("mtp", ctypes.c_int),
        ("saved_states", ctypes.c_int), ("prefill_chunk", ctypes.c_int), ("weight_format", ctypes.c_int),
        ("kv_cache_format", ctypes.c_int), ("projection_mfma", ctypes.c_int),
    ]


_lib = None


WEIGHT_FORMATS = {"e4m3": 0, "mxfp4": 1}
KV_CACHE_FORMATS = {"bf16": 0, "fp8": 1}
PROJECTION_MFMA = {"bf16": 0, "fp8": 1}


def library() -> ctypes.CDLL:
    """The loaded libq38.so with argument types set. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m qwen38_amd.build` (the verify path has no fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    p, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.q38_last_error.restype = ctypes.c_char_p
    lib.q38_last_error.argtypes = []
    lib.q38_create.argtypes = [ctypes.POINTER(Q38Config), ctypes.POINTER(p)]
    lib.q38_destroy.argtypes = [p]
    lib.q38_destroy.restype = None
    lib.q38_buffer_size.argtypes = [p, ctypes.c_char_p, i, ctypes.POINTER(sz)]
    lib.q38_bind.argtypes = [p, ctypes.c_char_p, i, p, sz]
    lib.q38_parity.argtypes = [p, ctypes.POINTER(i)]
    lib.q38_set_parity.argtypes = [p, i]
    lib.q38_pack_weight.argtypes = [p, p, i, i, p, p, p]
    lib.q38_pack_weight_fp4.argtypes = [p, p, i, i, p, p, p]
    lib.q38_fp8_linear.argtypes = [p, i, i, p, p, i, p, p, p]
    lib.q38_mxfp4_linear.argtypes = [p, i, i, p, p, i, p, p, p]
    lib.q38_fp4_linear.argtypes = [p, i, i, p, p, i, p, p, p]
    lib.q38_fp4_linear_scratch.argtypes = [i, i]
    lib.q38_fp8_linear_scratch.argtypes = [i, i]
    lib.q38_fp8_linear_f32.argtypes = [p, i, i, p, p, i, p, p, p]
    lib.q38_fp8_linear_mfma.argtypes = [p, i, i, p, p, i, i, i, p, p, p]
    lib.q38_fp8_linear_noalloc.argtypes = [p, i, i, p, p, i, p, p]
    lib.q38_mlp_up.argtypes = [p, i, i, p, p, i, p, p, p]
    lib.q38_tiles_size.argtypes = [i, i]
    lib.q38_kernel_timer.argtypes = [p, i, ctypes.POINTER(i), ctypes.POINTER(ctypes.c_float)]
    lib.q38_verify.argtypes = [p] * 8 + [p]
    lib.q38_decode.argtypes = [p] * 8
    lib.q38_copy_states.argtypes = [p, p, i, p]
    lib.q38_prefill.argtypes = [p, p, p, p, p, p, p, i, p, p]
    lib.q38_mtp_prefill.argtypes = [p, p, p, p, p, p, p, i, p, p]
    lib.q38_mtp_step.argtypes = [p] * 8 + [p]
    lib.q38_head_groupmax.argtypes = [p, p, i, p, p]
    lib.q38_head_pick.argtypes = [p, p, i, i, p, p]
    lib.q38_embed.argtypes = [p, p, i, p, p]
    lib.q38_accept.argtypes = [p, p, p, p, p, p, p]
    lib.q38_spec_step.argtypes = [p] * 10
    lib.q38_spec_step_graph.argtypes = [p] * 10
    lib.q38_verify_step.argtypes = [p] * 10
    lib.q38_step_status.argtypes = [p, ctypes.POINTER(i), i, p]
    for name in EXPORTS:
        if name not in ("q38_last_error", "q38_destroy"):
            getattr(lib, name).restype = ctypes.c_size_t if name in ("q38_fp8_linear_scratch", "q38_fp4_linear_scratch", "q38_tiles_size") else ctypes.c_int
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc:
        raise RuntimeError("libq38: " + library().q38_last_error().decode())


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("libq38 takes device tensors")
    if not t.is_contiguous():
        raise ValueError("libq38 takes contiguous tensors")
    return t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def make_config(cfg: TextConfig, batch: int, tokens: int, max_seq_len: int, mtp: bool, saved_states: bool = False,
                prefill_chunk: int = 0, weight_format: str = "e4m3", kv_cache_format: str = "bf16",
                projection_mfma: str = "bf16") -> Q38Config:
    c = Q38Config()
    c.hidden_size, c.intermediate_size, c.vocab_size = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    if cfg.num_hidden_layers > MAX_LAYERS:
        raise ValueError(f"at most {MAX_LAYERS} layers")
    c.num_layers = cfg.num_hidden_layers
    for i, kind in enumerate(cfg.layer_types):
        c.layer_types[i] = {LINEAR: 0, FULL: 1}[kind]
    c.num_attention_heads, c.num_key_value_heads, c.head_dim = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    c.rotary_dim = cfg.rotary_dim
    c.linear_num_key_heads, c.linear_num_value_heads = cfg.linear_num_key_heads, cfg.linear_num_value_heads
    c.linear_key_head_dim, c.linear_value_head_dim = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    c.linear_conv_kernel_dim = cfg.linear_conv_kernel_dim
    c.rms_norm_eps = cfg.rms_norm_eps
    c.batch_size, c.verify_tokens, c.max_seq_len, c.mtp = batch, tokens, max_seq_len, int(mtp)
    c.saved_states = int(saved_states)
    c.prefill_chunk = prefill_chunk
    c.weight_format = WEIGHT_FORMATS[weight_format]
    c.kv_cache_format = KV_CACHE_FORMATS[kv_cache_format]
    c.projection_mfma = PROJECTION_MFMA[projection_mfma]
    return c


class Handle:
    """One q38_handle: shapes fixed at creation, every buffer bound by the owner."""

    def __init__(self, cfg: TextConfig, batch: int, tokens: int, max_seq_len: int, mtp: bool, saved_states: bool = False,
                 prefill_chunk: int = 0, weight_format: str = "e4m3", kv_cache_format: str = "bf16", projection_mfma: str = "bf16"):
        self.lib = library()
        self.c = make_config(cfg, batch, tokens, max_seq_len, mtp, saved_states, prefill_chunk, weight_format, kv_cache_format,
                             projection_mfma)
        h = ctypes.c_void_p()
        check(self.lib.q38_create(ctypes.byref(self.c), ctypes.byref(h)))
        self.h = h

    def __del__(self):
        if getattr(self, "h", None) and self.h.value:
            self.lib.q38_destroy(self.h)
            self.h = None

    def buffer_size(self, name: str, layer: int) -> int:
        n = ctypes.c_size_t()
        check(self.lib.q38_buffer_size(self.h, name.encode(), layer, ctypes.byref(n)))
        return n.value

    def bind(self, name: str, layer: int, t: torch.Tensor) -> None:
        check(self.lib.q38_bind(self.h, name.encode(), layer, ptr(t), t.numel() * t.element_size()))

    @property
    def parity(self) -> int:
        p = ctypes.c_int()
        check(self.lib.q38_parity(self.h, ctypes.byref(p)))
        return p.value

    @parity.setter
    def parity(self, value: int) -> None:
        check(self.lib.q38_set_parity(self.h, value))

    def verify(self, embeds, cos, sin, position, active, accepted, out) -> None:
        check(self.lib.q38_verify(self.h, *map(ptr, (embeds, cos, sin, position, active, accepted, out)), stream()))

    def decode(self, embeds, cos, sin, position, active, out) -> None:
        check(self.lib.q38_decode(self.h, *map(ptr, (embeds, cos, sin, position, active, out)), stream()))

    def prefill(self, embeds, cos, sin, slot, start, n_valid, tokens: int, out) -> None:
        check(self.lib.q38_prefill(self.h, *map(ptr, (embeds, cos, sin, slot, start, n_valid)), tokens, ptr(out), stream()))

    def mtp_prefill(self, hidden, embeds, cos, sin, slot, start, tokens: int, out) -> None:
        check(self.lib.q38_mtp_prefill(self.h, *map(ptr, (hidden, embeds, cos, sin, slot, start)), tokens, ptr(out), stream()))

    def copy_states(self, slot, to_saved: bool) -> None:
        check(self.lib.q38_copy_states(self.h, ptr(slot), int(to_saved), stream()))

    def mtp_step(self, hidden, embeds, cos, sin, position, active, out) -> None:
        check(self.lib.q38_mtp_step(self.h, *map(ptr, (hidden, embeds, cos, sin, position, active, out)), stream()))

    def head_groupmax(self, hidden, rows: int, maxima) -> None:
        check(self.lib.q38_head_groupmax(self.h, ptr(hidden), rows, ptr(maxima), stream()))

    def head_pick(self, hidden, rows: int, groups: int, ids) -> None:
        check(self.lib.q38_head_pick(self.h, ptr(hidden), rows, groups, ptr(ids), stream()))

    def embed(self, ids, n: int, out) -> None:
        check(self.lib.q38_embed(self.h, ptr(ids), n, ptr(out), stream()))

    def accept(self, picks, drafts, active, match, accepted) -> None:
        check(self.lib.q38_accept(self.h, *map(ptr, (picks, drafts, active, match, accepted)), stream()))

    def spec_step(self, position, index, match, accepted, active, hidden, picks, drafts, graph: bool = False) -> None:
        """One speculative step on the device (`q38_spec_step`), or its captured HIP graph (`q38_spec_step_graph`)."""
        fn = self.lib.q38_spec_step_graph if graph else self.lib.q38_spec_step
        check(fn(self.h, *map(ptr, (position, index, match, accepted, active, hidden, picks, drafts)), stream()))

    def verify_step(self, position, index, match, accepted, active, hidden, picks, drafts) -> None:
        """The verify half of the speculative step for host-made drafts (`q38_verify_step`): the prompt-lookup
        branch of the reference's `Scheduler._verify_step` (scheduler.py:269-301)."""
        check(self.lib.q38_verify_step(self.h, *map(ptr, (position, index, match, accepted, active, hidden, picks, drafts)),
                                       stream()))

    def step_status(self, clear: bool = True) -> int:
        """The device's step status word (`q38_step_status`: STATUS_NONFINITE, STATUS_POSITION), then reset."""
        v = ctypes.c_int(0)
        check(self.lib.q38_step_status(self.h, ctypes.byref(v), int(clear), stream()))
        return v.value

    def raise_step_errors(self) -> None:
        """The reference's host-side errors for what the last steps recorded on the device: FloatingPointError for a
        row with no finite logit (generate.py:206-207), ValueError for tokens past the last usable position
        (generate.py:78-79)."""
        status = self.step_status()
        if status & STATUS_NONFINITE:
            raise FloatingPointError("a row's logits are not finite, so the step produced NaN or infinity")
        if status & STATUS_POSITION:
            raise ValueError("a row's tokens pass max_seq_len")

    def kernel_timer(self, on: bool) -> tuple[int, float]:
        """Start (on) or stop bracketing the gate/up GEMM launches with HIP events; stopping returns (launches, total
        milliseconds)."""
        n, ms = ctypes.c_int(0), ctypes.c_float(0.0)
        check(self.lib.q38_kernel_timer(self.h, int(on), ctypes.byref(n), ctypes.byref(ms)))
        return n.value, ms.value


def pack_weight(coded: torch.Tensor, scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(e4m3 bytes [N, K], E8M0 bytes [N, K/32]) on the GPU -> (tiles, tile scales) in the GEMM layout."""
    n, k = coded.shape
    tiles = torch.empty(n * k, dtype=torch.uint8, device=coded.device)
    tile_scales = torch.empty(n * k // 32, dtype=torch.uint8, device=coded.device)
    check(library().q38_pack_weight(ptr(coded.contiguous()), ptr(scales.contiguous()), n, k, ptr(tiles), ptr(tile_scales), stream()))
    return tiles, tile_scales


def pack_weight_fp4(packed: torch.Tensor, scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The checkpoint's MXFP4 (packed bytes [N, K/2], E8M0 bytes [N, K/32]) on the GPU -> (tiles, tile scales)."""
    n, half = packed.shape
    k = 2 * half
    tiles = torch.empty(n * half, dtype=torch.uint8, device=packed.device)
    tile_scales = torch.empty(n * k // 32, dtype=torch.uint8, device=packed.device)
    check(library().q38_pack_weight_fp4(ptr(packed.contiguous()), ptr(scales.contiguous()), n, k, ptr(tiles), ptr(tile_scales),
                                        stream()))
    return tiles, tile_scales


def linear_scratch(rows: int, k: int, device="cuda") -> torch.Tensor:
    """Zero-filled scratch for the standalone projections (input tiles, then the GEMM's counters and partials)."""
    return torch.zeros(library().q38_fp8_linear_scratch(rows, k), dtype=torch.uint8, device=device)


def fp8_linear(x: torch.Tensor, tiles: torch.Tensor, scales: torch.Tensor, n: int, scratch=None) -> torch.Tensor:
    """`FP8Linear.forward` on the GPU: bf16 x [rows, k] -> bf16 [rows, n] through a packed FP8 weight."""
    rows, k = x.shape
    scratch = linear_scratch(rows, k, x.device) if scratch is None else scratch
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=x.device)
    check(library().q38_fp8_linear(ptr(x.contiguous()), rows, k, ptr(tiles), ptr(scales), n, ptr(scratch), ptr(out), stream()))
    return out


def fp8_linear_noalloc(x: torch.Tensor, tiles: torch.Tensor, scales: torch.Tensor, n: int, out=None) -> torch.Tensor:
    """`fp8_linear` with the library's static scratch (no device allocation by the library): 1 to 64 rows."""
    rows, k = x.shape
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=x.device) if out is None else out
    check(library().q38_fp8_linear_noalloc(ptr(x.contiguous()), rows, k, ptr(tiles), ptr(scales), n, ptr(out), stream()))
    return out


GEMM_RECOMPUTE = 4  # Q38_GEMM_RECOMPUTE
STATUS_NONFINITE, STATUS_POSITION = 1, 2  # Q38_STATUS_*


def fp8_linear_mfma(x: torch.Tensor, tiles: torch.Tensor, scales: torch.Tensor, n: int, mfma: str, f32_out: bool = False,
                    scratch=None, recompute: bool = False) -> torch.Tensor:
    """The FP8 projection with its products on the named MFMA ("fp8" or "bf16"), bf16 or float32 output; with
    ``recompute`` every tile split between workgroups is finished by recomputing its partials (the GEMM's path for
    contributors on different XCDs)."""
    rows, k = x.shape
    scratch = linear_scratch(rows, k, x.device) if scratch is None else scratch
    out = torch.empty(rows, n, dtype=torch.float32 if f32_out else torch.bfloat16, device=x.device)
    flags = PROJECTION_MFMA[mfma] | (GEMM_RECOMPUTE if recompute else 0)
    check(library().q38_fp8_linear_mfma(ptr(x.contiguous()), rows, k, ptr(tiles), ptr(scales), n, flags,
                                        int(f32_out), ptr(scratch), ptr(out), stream()))
    return out


def mxfp4_linear(x: torch.Tensor, tiles: torch.Tensor, scales: torch.Tensor, n: int, scratch=None) -> torch.Tensor:
    """The projection through a packed MXFP4 weight (`pack_weight_fp4`): bf16 x [rows, k] -> bf16 [rows, n]."""
    rows, k = x.shape
    scratch = linear_scratch(rows, k, x.device) if scratch is None else scratch
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=x.device)
    check(library().q38_mxfp4_linear(ptr(x.contiguous()), rows, k, ptr(tiles), ptr(scales), n, ptr(scratch), ptr(out), stream()))
    return out


def fp4_linear(x: torch.Tensor, tiles: torch.Tensor, scales: torch.Tensor, n: int, scratch=None) -> torch.Tensor:
    """`FP4Linear.forward` on the GPU (the weight_format "fp4" numerics): bf16 x [rows, k] -> bf16 [rows, n] through a
    packed MXFP4 weight (`pack_weight_fp4`), the even and odd inputs summed apart and their bf16 results added."""
    rows, k = x.shape
    if scratch is None:
        scratch = torch.zeros(library().q38_fp4_linear_scratch(rows, k), dtype=torch.uint8, device=x.device)
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=x.device)
    check(library().q38_fp4_linear(ptr(x.contiguous()), rows, k, ptr(tiles), ptr(scales), n, ptr(scratch), ptr(out), stream()))
    return out


def fp8_linear_f32(x: torch.Tensor, tiles: torch.Tensor, scales: torch.Tensor, n: int, scratch=None) -> torch.Tensor:
    """The FP8 projection with float32 output (no bf16 rounding): rows in {32, 64, 128} or a multiple of 256."""
    rows, k = x.shape
    scratch = linear_scratch(rows, k, x.device) if scratch is None else scratch
    out = torch.empty(rows, n, dtype=torch.float32, device=x.device)
    check(library().q38_fp8_linear_f32(ptr(x.contiguous()), rows, k, ptr(tiles), ptr(scales), n, ptr(scratch), ptr(out), stream()))
    return out


def mlp_up(x: torch.Tensor | None, rows: int, k: int, tiles: torch.Tensor, scales: torch.Tensor, inter: int, scratch=None,
           out=None) -> torch.Tensor:
    """The fused gate/up projection with SwiGLU (`mlp_up`): bf16 x [rows, k] -> the down projection's e5m2 input tiles.
    With x None the scratch already holds the input tiles of an earlier call."""
    lib = library()
    if scratch is None:
        scratch = linear_scratch(rows, k)
    if out is None:
        out = torch.empty(lib.q38_tiles_size(rows, inter), dtype=torch.uint8, device=scratch.device)
    xp = None if x is None else ptr(x.contiguous())
    check(lib.q38_mlp_up(xp, rows, k, ptr(tiles), ptr(scales), inter, ptr(scratch), ptr(out), stream()))
    return out
