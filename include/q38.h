/* C ABI of the MI355X verify-step library (libq38.so), built from qwen38-27b-aws_amd/qwen38_amd/csrc.
 *
 * It replaces, for the MTP speculative-decoding verify step of the Qwen3.8 hybrid model, the reference's compiled
 * Neuron graphs and the CPU path that stands in for them:
 *   q38_verify       <- `verify(**verify_inputs(...))`, the K-token graph: Qwen38Step.forward with `accepted`
 *                       (reference qwen38_inf2/model.py:933-995; call site scheduler.py:288; inputs generate.py:72-87)
 *   q38_decode       <- `step(**batch_step_inputs(...))`, the one-token graph: Qwen38Step.forward's decode form
 *                       (model.py:983-995; call sites generate.py:251,258,290; inputs generate.py:34-60)
 *   q38_prefill      <- `prefill(**prefill_inputs(...))`, the step graph's prefill form (model.py:983-995 with
 *                       GatedDeltaNetStep.prefill model.py:476-521 and FullAttentionStep.prefill model.py:704-783;
 *                       call site scheduler.py:125; inputs generate.py:58-69)
 *   q38_mtp_prefill  <- `mtp(hidden=..., inputs_embeds=..., **mtp_prefill_inputs(...))`, MTPStep.forward's prefill form
 *                       (model.py:843-855; call site scheduler.py:157; inputs generate.py:102-107)
 *   q38_copy_states  <- the same graph with save_slot / restore_slot (model.py:988-992, GatedDeltaNetStep.copy_states
 *                       model.py:456-464; call sites scheduler.py:119,133; inputs generate.py:110-116)
 *   q38_mtp_step     <- `mtp(hidden=..., inputs_embeds=..., **mtp_step_inputs(...))`, MTPStep.forward
 *                       (model.py:843-860; call sites scheduler.py:179,192)
 *   q38_head_groupmax<- the head graph `run_graph(hidden=...)`, HeadStep.forward (model.py:890-900;
 *                       generate.py:195)
 *   q38_head_pick    <- ChipHead.next_tokens' top-group recheck (generate.py:196-208), on the GPU
 *   q38_accept       <- the greedy acceptance loop (scheduler.py:291-300), for the on-device step
 *   q38_embed        <- ChipHead.embed_batch (generate.py:183-184)
 *
 * Conventions. Every function returns 0 on success or a nonzero code; q38_last_error() then describes the failure
 * (thread-local). All tensor arguments are device pointers; `stream` is a hipStream_t (0 for the null stream). The
 * library allocates no device memory: the caller binds every weight, state and workspace buffer with q38_bind, after
 * asking q38_buffer_size for its size. A handle is not re-entrant: one call at a time per handle; different handles
 * are independent. bf16 is passed as uint16_t bits.
 */
#ifndef Q38_H
#define Q38_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q38_handle q38_handle;

#define Q38_MAX_LAYERS 128
#define Q38_LINEAR 0
#define Q38_FULL 1
#define Q38_WEIGHTS_E4M3 0  /* projections bound as q38_pack_weight tiles */
#define Q38_WEIGHTS_MXFP4 1 /* decoder-layer projections bound as q38_pack_weight_fp4 tiles (MTP layer, head: e4m3) */
#define Q38_KV_BF16 0
#define Q38_KV_FP8 1 /* KV caches of e4m3 bytes of value / scale, clamped to +-240, with bf16 scales per layer */
#define Q38_MFMA_BF16 0
#define Q38_MFMA_FP8 1
/* Or'ed into q38_fp8_linear_mfma's `mfma`: finish every stream-K tile by recomputing its contributors' partials, the
 * path the GEMM takes when a tile's contributors run on different XCDs (so do not share an L2). */
#define Q38_GEMM_RECOMPUTE 4

/* Bits of the step status word (q38_step_status). */
#define Q38_STATUS_NONFINITE 1 /* a head row had no finite logit (the reference raises FloatingPointError) */
#define Q38_STATUS_POSITION 2  /* an active row's tokens passed the last usable position (the reference: ValueError) */

/* Model shapes (reference TextConfig, qwen38_inf2/config.py:11-62) plus the build's batch (rows), verify tokens per
 * row, cache length and whether the MTP layer is present (reference build_info keys batch_size, verify_tokens,
 * max_seq_len, mtp_tokens; neuron.py:128-140,182-185). */
typedef struct q38_config {
    int hidden_size, intermediate_size, vocab_size;
    int num_layers;
    int layer_types[Q38_MAX_LAYERS]; /* Q38_LINEAR (gated delta) or Q38_FULL (attention) */
    int num_attention_heads, num_key_value_heads, head_dim, rotary_dim;
    int linear_num_key_heads, linear_num_value_heads, linear_key_head_dim, linear_value_head_dim;
    int linear_conv_kernel_dim;
    float rms_norm_eps;
    int batch_size, verify_tokens, max_seq_len, mtp;
    int saved_states; /* a saved recurrent and conv state per row, for q38_copy_states (reference saved_states) */
    int prefill_chunk; /* most tokens of one q38_prefill call (a multiple of 32; 0: no prefill workspace) */
    int weight_format; /* Q38_WEIGHTS_E4M3 or Q38_WEIGHTS_MXFP4 (the reference's weight_format, config.py:28-30) */
    int kv_cache_format; /* Q38_KV_BF16 or Q38_KV_FP8 (the reference's kv_cache_format, config.py:33-34, model.py:557-601) */
    int projection_mfma; /* Q38_MFMA_FP8: decoder and MTP projections (e4m3 weights x e5m2 activations) on the scaled FP8
                            MFMA, each 64-input block summed to about 2^-15.5 of its sum |x w|; Q38_MFMA_BF16: both widened
                            exactly to bf16 for the bf16 MFMA (float32-grade sums, twice the MFMA time). The head's
                            group maxima always run on the bf16 MFMA (bf16 activations). */
} q38_config;

const char* q38_last_error(void);

/* Validates the shapes the kernels support and creates a handle with nothing bound. */
int q38_create(const q38_config* cfg, q38_handle** out);
void q38_destroy(q38_handle* h);

/* Buffers, by name and layer (layer -1 for model-wide buffers; layer num_layers is the MTP layer). Sizes in bytes.
 * Weights (projections bound as packed tiles + tile scales from q38_pack_weight; with weight_format MXFP4 the decoder
 * layers' projections from q38_pack_weight_fp4, half the tile bytes):
 *   per layer: input_layernorm, post_attention_layernorm (bf16 [H]), mlp.gate_up.{tiles,scales} (gate and up rows
 *     interleaved by 32), mlp.down.{tiles,scales}
 *   gated-delta layers: linear_attn.in_proj_qkvz.{tiles,scales} (in_proj_qkv rows then in_proj_z rows),
 *     linear_attn.out_proj.{tiles,scales}, linear_attn.in_proj_a, linear_attn.in_proj_b (bf16 [Hv][H]),
 *     linear_attn.conv_weight (bf16 [C][4]), linear_attn.A_log, linear_attn.dt_bias (bf16 [Hv]),
 *     linear_attn.norm_weight (bf16 [128])
 *   attention layers and the MTP layer: self_attn.qkv.{tiles,scales} (q_proj, k_proj, v_proj rows),
 *     self_attn.o_proj.{tiles,scales}, self_attn.q_norm, self_attn.k_norm (bf16 [head_dim])
 *   MTP layer only: mtp.fc.{tiles,scales}, mtp.embedding_norm, mtp.hidden_norm, mtp.norm (bf16 [H])
 *   model-wide: head.norm (bf16 [H], also the MTP's final norm), head.lm_head.{tiles,scales}, embed_tokens (bf16 [V][H]),
 *     rope_table (bf16 [max_seq_len][2][rotary_dim], for q38_spec_step)
 * State (per layer):
 *   linear_attn.recurrent_state bf16 [B][Hv][128][128]
 *   linear_attn.conv_state bf16 [2][B][C][3], linear_attn.pending_key f32 [2][B][K][Hk][128],
 *   linear_attn.pending_delta f32 [2][B][K][Hv][128], linear_attn.pending_decay f32 [2][B][K][Hv],
 *   linear_attn.pending_input bf16 [2][B][K][C]: two halves, the current one given by q38_parity
 *   self_attn.k_cache bf16 [B][Hkv][S][hd]; self_attn.v_cache bf16 [B][Hkv][S/32][hd][32] (transposed per 32 positions);
 *   with kv_cache_format FP8 the same layouts of e4m3 bytes, and self_attn.k_scale, self_attn.v_scale (bf16 [1], the
 *   checkpoint's static scales, reference checkpoint.py:227-233) among the layer's weights
 *   with saved_states: linear_attn.saved_state bf16 [B][Hv][128][128], linear_attn.saved_conv bf16 [B][C][3]
 * Scratch: workspace (model-wide; its GEMM counters are zeroed when it is bound).
 * Optional, per decoder layer: probe, which a q38_verify call fills when it is bound (size from q38_buffer_size): as
 *   bf16 [B*K][.], the layer's normed input (gated-delta layers), the mixer's projection output (the gated-delta
 *   in_proj_z part, Hv*128 wide; or the attention q|gate|k|v projection) and the residual stream after the mixer; then
 *   the e5m2 activation tiles of the out_proj/o_proj input, the MLP input and the down projection's input, for the
 *   first B*K tokens rounded up to 32; last, bf16 [B*K][H], the residual stream entering the layer. For
 *   stage-by-stage comparison with another implementation; unbound, nothing is copied. The MTP layer (index
 *   num_layers) takes one too, filled by q38_mtp_step (its layer input is the fc output).
 * Optional, model-wide: head.probe, which q38_head_groupmax (and q38_head_pick) fills when bound: the head's normed
 *   rows as bf16 activation tiles (the e5m2 tiles' element order, two bytes each) of whole 32-row blocks. */
int q38_buffer_size(q38_handle* h, const char* name, int layer, size_t* nbytes);
int q38_bind(q38_handle* h, const char* name, int layer, void* dev_ptr, size_t nbytes);

/* Which half of the double-buffered gated-delta state is current (read by the next q38_verify), and setting it. */
int q38_parity(q38_handle* h, int* parity);
int q38_set_parity(q38_handle* h, int parity);

/* Pack an FP8 projection: e4m3 bytes [N][K] and E8M0 scale bytes [N][K/32] (row-major, a torch Linear weight's
 * layout) into tiles [N/32][K/64][64][32] and tile scales [N/32][K/64][32][2] (N * K / 32 bytes). N % 32 == 0,
 * K % 256 == 0. */
int q38_pack_weight(const uint8_t* coded, const uint8_t* scales, int n, int k, uint8_t* tiles, uint8_t* tile_scales,
                    void* stream);

/* Pack an MXFP4 projection as the checkpoint stores it (weight_packed uint8 [N][K/2], the even input in the low
 * nibble; weight_scale E8M0 bytes [N][K/32]; reference fp4.py:1-13, checkpoint.py:177-182) into tiles
 * [N/32][K/64][4][64][4] (N * K / 2 bytes: the same element order as q38_pack_weight's, two inputs per byte) and the
 * same tile scales. N % 32 == 0, K % 256 == 0. The checkpoint's bytes are read as they are: no e5m2 re-encoding
 * (fp4.to_fp8, fp4.py:118-140) and so none of its rounding of groups with tiny scales. */
int q38_pack_weight_fp4(const uint8_t* packed, const uint8_t* scales, int n, int k, uint8_t* tiles, uint8_t* tile_scales,
                        void* stream);

/* A standalone FP8 projection, `FP8Linear.forward` (reference model.py:211-229): x bf16 [rows][k] rounded to e5m2,
 * times the packed weight ([n][k] e4m3 + E8M0), float32 sums, bf16 out [rows][n]. n % 256 == 0, k % 256 == 0.
 * scratch holds q38_fp8_linear_scratch(rows, k) bytes: the e5m2 input tiles (q38_tiles_size(rows, k) bytes), then the
 * GEMM's arrival counters and partial sums. It must be zero-filled before its first use; every call leaves the
 * counters at zero again. Calls that share a scratch must not overlap. With x null the scratch already holds the input
 * tiles (of an earlier call with the same rows and k). */
int q38_fp8_linear(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                   uint8_t* scratch, uint16_t* out, void* stream);
size_t q38_fp8_linear_scratch(int rows, int k);
/* q38_fp8_linear (f32_out 0: bf16 [rows][n]) or q38_fp8_linear_f32 (f32_out 1: float32 [rows][n], rows as there) with
 * the products on the MFMA `mfma` names (Q38_MFMA_FP8 or Q38_MFMA_BF16, optionally | Q38_GEMM_RECOMPUTE);
 * q38_fp8_linear itself is Q38_MFMA_BF16. Same scratch. No counterpart in the reference: for measuring the two MFMAs'
 * sums on the same projection, and the GEMM's two ways of finishing a tile split between workgroups. */
int q38_fp8_linear_mfma(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n, int mfma,
                        int f32_out, uint8_t* scratch, void* out, void* stream);
/* q38_fp8_linear with an MXFP4 weight from q38_pack_weight_fp4: e5m2(x) times the exact E2M1 x E8M0 values, which is
 * `FP8Linear.forward` on the weights `fp4.to_fp8` makes from the checkpoint (model.py:211-229) wherever that conversion
 * is exact. Same scratch. */
int q38_mxfp4_linear(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                     uint8_t* scratch, uint16_t* out, void* stream);
/* The reference's `FP4Linear.forward` (model.py:198-208, the weight_format "fp4" numerics): bf16 x [rows][k] against an
 * MXFP4 weight from q38_pack_weight_fp4, out = bf16(bf16(x_even . W_even) + bf16(x_odd . W_odd)) [rows][n] with the
 * inputs split by parity (fp4.decode_planes, fp4.py:93-100) and float32 sums. scratch holds q38_fp4_linear_scratch(rows,
 * k) bytes, zero-filled before its first use (bf16 input tiles, then the GEMM's counters and partial sums); calls that
 * share it must not overlap. */
int q38_fp4_linear(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                   uint8_t* scratch, uint16_t* out, void* stream);
size_t q38_fp4_linear_scratch(int rows, int k);
/* q38_fp8_linear for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops):
 * the same outputs, with the scratch in the library's own static device array (66.5 MiB in the library's code object:
 * resident on every GPU where any libq38 kernel is loaded, from then until the process ends, whether or not this entry
 * point is called) instead of an argument. 1 to 64 rows, K <= 32768, n % 256 == 0; other sizes are
 * refused. Calls share their GPU's array, so calls that overlap on one GPU race. No counterpart in the reference. */
int q38_fp8_linear_noalloc(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                           uint16_t* out, void* stream);
/* The same with float32 output [rows][n] (no bf16 rounding); rows in {32, 64, 128} or a multiple of 256. */
int q38_fp8_linear_f32(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                       uint8_t* scratch, float* out, void* stream);

/* The MLP's fused gate/up projection, the chip's `mlp_up` (reference kernels.py:74-118, model.py:250-259):
 * x bf16 [rows][k] rounded to e5m2, times the gate/up weight packed with gate and up rows interleaved by 32
 * ([2*inter][k]), then bf16(silu(gate)) * up rounded to e5m2, written as the down projection's input tiles
 * (e5m2 bytes [pad(rows)/32][inter/64][4][64][8], q38_tiles_size(rows, inter) bytes). scratch as for
 * q38_fp8_linear. */
int q38_mlp_up(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int inter,
               uint8_t* scratch, uint8_t* out_tiles, void* stream);
/* Bytes of e5m2 activation tiles for rows x k (rows padded to 32, 64, 128 or a multiple of 256). */
size_t q38_tiles_size(int rows, int k);

/* One verify step over all B rows: embeds bf16 [B][K][H]; cos, sin bf16 [B][K][rotary_dim]; position int32 [B];
 * active f32 [B]; accepted int32 [B]. Writes the last layer's hidden state bf16 [B][K][H] (before the final norm),
 * commits each row's `accepted` tokens of the previous step, and flips the parity. */
int q38_verify(q38_handle* h, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin, const int32_t* position,
               const float* active, const int32_t* accepted, uint16_t* out_hidden, void* stream);

/* One decode step over all B rows, one token each: embeds bf16 [B][1][H]; cos, sin bf16 [B][1][rotary_dim];
 * position int32 [B] (0 starts a new sequence: the row's gated-delta states restart from zero); active f32 [B] (0 keeps
 * the row's states and cache exactly). Writes the last layer's hidden state bf16 [B][1][H] and flips the parity (the
 * conv states go to the other half). The gated-delta layers run the recurrent form (GatedDeltaNetStep.forward,
 * model.py:347-374), the attention layers FullAttentionStep.forward (model.py:610-639). A verify step after it takes
 * accepted = 0, as in the reference. */
int q38_decode(q38_handle* h, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin, const int32_t* position,
               const float* active, uint16_t* out_hidden, void* stream);

/* One prefill chunk of one row: embeds bf16 [tokens][H]; cos, sin bf16 [tokens][rotary_dim] for positions start ..;
 * slot, start, n_valid int32 [1] on the device (start 0 restarts the row's gated-delta states; tokens from n_valid on
 * are padding, which leaves the states alone). tokens is a multiple of 32 up to the config's prefill_chunk, and
 * start + tokens <= max_seq_len. Writes the last layer's hidden states bf16 [tokens][H] and updates row slot's
 * gated-delta states (the current half) and its KV caches at start .. start + tokens - 1 in place; the other rows are
 * untouched (the reference also writes junk at their cache's last positions, which nothing reads). */
int q38_prefill(q38_handle* h, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin, const int32_t* slot,
                const int32_t* start, const int32_t* n_valid, int tokens, uint16_t* out_hidden, void* stream);

/* The MTP layer's prefill form: hidden, embeds bf16 [tokens][H]; cos, sin for positions start + 1 ..; slot, start int32
 * [1] on the device. Writes only the MTP layer's KV cache for row slot at start .. start + tokens - 1, and, when out_x
 * is not null, the fc output's first row bf16 [H] (the reference returns x[:, :1]). */
int q38_mtp_prefill(q38_handle* h, const uint16_t* hidden, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin,
                    const int32_t* slot, const int32_t* start, int tokens, uint16_t* out_x, void* stream);

/* Save (to_saved != 0) or restore one row's gated-delta recurrent and conv states in every gated-delta layer; slot is
 * int32 [1] on the device (a slot outside [0, B) copies nothing). Needs saved_states in the config and the saved
 * buffers bound. */
int q38_copy_states(q38_handle* h, const int32_t* slot, int to_saved, void* stream);

/* One MTP step: hidden, embeds bf16 [B][K][H]; cos, sin [B][K][rotary_dim]; position, active [B]. Writes bf16
 * [B][K][H]. */
int q38_mtp_step(q38_handle* h, const uint16_t* hidden, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin,
                 const int32_t* position, const float* active, uint16_t* out, void* stream);

/* Head: rows bf16 [R][H] (R <= B*K). q38_head_groupmax writes the group maxima f32 [R][V/32]; q38_head_pick computes
 * them itself and writes ids int32 [R] (-1: no finite logit) after rechecking the best `groups` (1..4) groups. */
int q38_head_groupmax(q38_handle* h, const uint16_t* hidden, int rows, float* maxima, void* stream);
int q38_head_pick(q38_handle* h, const uint16_t* hidden, int rows, int groups, int32_t* ids, void* stream);
/* (q38_head_pick rechecks the best groups against lm_head's bf16 rows when the optional global buffer
 * "head.lm_head.rows" (bf16 [V][H], the checkpoint's lm_head) is bound, as the reference's ChipHead rechecks against
 * the checkpoint's rows (generate.py:196-206); without it, against the e4m3 tiles dequantized exactly.) */

/* Embedding rows for ids int32 [n] into bf16 [n][H]. */
int q38_embed(q38_handle* h, const int32_t* ids, int n, uint16_t* out, void* stream);

/* Greedy acceptance: picks int32 [B][K], drafts int32 [B][K-1], active f32 [B] -> match, accepted int32 [B]. */
int q38_accept(q38_handle* h, const int32_t* picks, const int32_t* drafts, const float* active, int32_t* match,
               int32_t* accepted, void* stream);

/* One whole speculative step on the device (the reference's Scheduler._verify_step with MTP drafts,
 * scheduler.py:160-193,269-301), for all B rows, with no host round trip. Device state, read and updated:
 *   position int32 [B]  the verify step's first position (row.written); advanced by the accepted count
 *   index    int32 [B]  the last step's position (the MTP drafter's index); set to the old position
 *   match    int32 [B]  the last step's matched drafts (the MTP's `take`); replaced by this step's
 *   accepted int32 [B]  tokens the verify commits from the last step (match + 1); replaced by this step's
 *   hidden   bf16 [B][K][H], picks int32 [B][K]: the last step's verify output and picks; replaced by this step's
 * active f32 [B] is read; drafts int32 [B][K-1] receives this step's drafts. Needs the MTP layer, the head, the
 * embeddings and a bound "rope_table" (bf16 [max_seq_len][2][rotary_dim]: cos then sin of each position). */
int q38_spec_step(q38_handle* h, int32_t* position, int32_t* index, int32_t* match, int32_t* accepted, const float* active,
                  uint16_t* hidden, int32_t* picks, int32_t* drafts, void* stream);
/* The verify half of q38_spec_step for drafts the host made: the reference's Scheduler._verify_step without an MTP
 * drafter (scheduler.py:269-301), whose drafts come from the row's own history (`Drafter.draft`, drafting.py:44-51,
 * padded with the row's last token, scheduler.py:276-282). drafts int32 [B][K-1] is read; position, index, match,
 * accepted, hidden and picks are read and updated as by q38_spec_step: [picks[match], drafts] per row is embedded and
 * verified, the head picks K tokens per row over all B*K rows (top-4 recheck) and acceptance sets match and accepted.
 * The emitted tokens of row b are picks[b][0..match[b]]. Needs the head, the embeddings and the bound "rope_table". */
int q38_verify_step(q38_handle* h, int32_t* position, int32_t* index, int32_t* match, int32_t* accepted, const float* active,
                    uint16_t* hidden, int32_t* picks, const int32_t* drafts, void* stream);
/* q38_spec_step as one HIP graph: the step is captured on first use for the current gated-delta parity and these
 * argument pointers (at most one graph per parity is kept; other pointers, or any q38_bind, capture again) and
 * replayed with hipGraphLaunch on `stream`, the host's parity flipping as after q38_spec_step. The same kernels with
 * the same arguments, so the same results. While the kernel timer is on or a probe is bound it runs q38_spec_step.
 * No counterpart in the reference (its step is one compiled Neuron graph per shape). */
int q38_spec_step_graph(q38_handle* h, int32_t* position, int32_t* index, int32_t* match, int32_t* accepted,
                        const float* active, uint16_t* hidden, int32_t* picks, int32_t* drafts, void* stream);
/* The step status word and, with clear != 0, its reset: the errors the reference raises on the host
 * (FloatingPointError for a row with no finite logit, generate.py:206-207; ValueError for tokens past the last usable
 * position, generate.py:78-79), which q38_spec_step (and q38_head_pick) record on the device instead of producing
 * silently wrong ids or positions. Reads back one int: a synchronisation of `stream`. */
int q38_step_status(q38_handle* h, int* status, int clear, void* stream);

/* Measurement hook, with no counterpart in the reference (for benchmarks that time one kernel inside the step):
 * on != 0 starts bracketing every gate/up projection GEMM launched by q38_verify, q38_mtp_step and q38_spec_step with
 * HIP events on the launch's stream (at most 4096 launches); on == 0 stops, waits for the last event and reports the
 * number of bracketed launches and the sum of their durations in milliseconds. */
int q38_kernel_timer(q38_handle* h, int on, int* launches, float* total_ms);

#ifdef __cplusplus
}
#endif

#endif
