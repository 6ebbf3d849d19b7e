// Kernel argument blocks and launchers of the verify path; the host engine (engine.cpp) fills these.
#pragma once

#include "common.h"

enum { EPI_BF16 = 0, EPI_SWIGLU = 1, EPI_PARTIAL = 2, EPI_GROUPMAX = 3 };

constexpr int GEMM_SPLIT_MAX = 8;      // split-K partial buffers (EPI_PARTIAL)
constexpr int GEMM_COUNTERS = 65536;   // stream-K arrival counters (8 bytes each)
constexpr int GEMM_SLOT_FLOATS = 65536;  // floats of one stream-K partial (largest workgroup tile)

struct GemmArgs {
    const uint8_t* w;    // weight tiles [N/32][K/64][64][32] (e4m3), or with w4 [N/32][K/64][4][64][4] (E2M1 pairs)
    const uint8_t* ws;   // scales [N/32][K/64][32][2] (E8M0): row r's bytes for the K-step's two MX blocks
    const void* act;     // activation tiles [Tpad/32][K/64][4][64][8]: e5m2 bytes, or bf16 for EPI_GROUPMAX
    int K, N, T, Tpad;
    void* out0;
    int ld0, n0;
    void* out1;
    int ld1;
    float* part;         // EPI_PARTIAL: [split][Tpad][N]; EPI_GROUPMAX: maxima [T][N/32]
    float* fix;          // stream-K partial slots: 2 per workgroup of GEMM_SLOT_FLOATS
    size_t fix_floats;
    unsigned long long* counters;  // stream-K arrivals per tile, one byte per XCD; zero between launches (each
                                   // launch leaves them zero)
    int counters_n;
    int cus;             // compute units: one persistent workgroup each
    int splits_max;      // EPI_PARTIAL: at most this many splits (0: as many as fill the CUs)
    int recompute;       // finish every split tile by recomputing its partials (as when contributors share no L2)
    int splits;          // EPI_PARTIAL split count (set by the launcher)
    int w4;              // weight tiles hold MXFP4 (q38_pack_fp4) rather than e4m3
    int f8;              // e4m3 weights x e5m2 activations on the FP8 MFMA (else widened to bf16 for the bf16 MFMA)
    int bf16_act;        // with w4 and EPI_BF16: bf16 activation tiles (q38_act_tiles_bf16) instead of e5m2 ones
    int accumulate;      // EPI_BF16: out = bf16(out + bf16(sum)) instead of bf16(sum)
};

struct NormArgs {
    const float* part;     // split-K partials [splits][Tpad][H], or null
    int splits, Tpad;
    const bf16_t* xin;     // without partials: the rows to normalize
    const bf16_t* resid;   // with partials: x_new = bf16(resid + bf16(sum)); null: x_new = bf16(sum)
    bf16_t* xout;          // x_new (may alias resid), or null
    const bf16_t* w;       // norm weight, used as (1 + w)
    float eps;
    uint8_t* act;          // e5m2 activation tiles of width Kact at column act_col0, or null
    int Kact, act_col0;
    bf16_t* hout;          // bf16 normed rows [T][H], or null
    const bf16_t* div_w;   // MTP tail: hout = bf16(normed / (1 + div_w))
    int H, T;
};

struct GatesArgs {
    const bf16_t* x;       // [T][H] bf16 (the input norm's output)
    const bf16_t* wb;      // in_proj_b [Hv][H]
    const bf16_t* wa;      // in_proj_a [Hv][H]
    int T, H, Hv;
    int groups;            // K ranges (H % (64 * groups) == 0, at most 16 MFMA steps per wave)
    float* part;           // [groups][T][2 Hv]: x . in_proj_b rows, then x . in_proj_a rows
};

struct GdnArgs {
    int B, K, Hk, Hv, C;
    const bf16_t* qkv_new;   // [B*K][C]: this step's in_proj_qkv output, also the new pending input snapshot
    const bf16_t* qkv_old;   // [B*K][C]: the last step's (pending_input_state)
    const bf16_t* z;         // [B*K][Hv*128]
    const float* gate_part;  // [gate_groups][B*K][2 Hv]: partial x . in_proj_b, x . in_proj_a (gates kernel)
    int gate_groups;
    const bf16_t* a_log;     // [Hv]
    const bf16_t* dt_bias;   // [Hv]
    const bf16_t* conv_w;    // [C][4]
    const bf16_t* norm_w;    // [128]
    const int* position;
    const float* active;
    const int* accepted;
    bf16_t* state;           // [B][Hv][128][128]
    const bf16_t* conv_old;  // [B][C][3]
    bf16_t* conv_new;
    const float* key_old;    // [B][K][Hk][128]
    float* key_new;
    const float* delta_old;  // [B][K][Hv][128]
    float* delta_new;
    const float* decay_old;  // [B][K][Hv]
    float* decay_new;
    uint8_t* act;            // e5m2 activation tiles of width Hv*128 for out_proj
    float eps;
    bf16_t* out_probe;       // optional [B*K][Hv*128]: the in-step output o (bf16) before the gated norm
};

// Gated delta net over one prefill chunk of one row (prefill.hip).
struct PrefillGdnArgs {
    int L, Hk, Hv, C;
    int rows;                // rows of the state buffers: a slot outside [0, rows) makes every kernel return
    const int* slot;         // int32 [1] on the device: the row
    const int* start;        // int32 [1]: the chunk's first position (0 restarts the row's states)
    const int* n_valid;      // int32 [1]: real tokens; the rest are padding
    const bf16_t* qkv;       // [L][C]: the chunk's in_proj_qkv output
    const bf16_t* z;         // [L][Hv*128]
    const float* gate_part;  // [gate_groups][L][2 Hv] (gates kernel)
    int gate_groups;
    const bf16_t* a_log;
    const bf16_t* dt_bias;
    const bf16_t* conv_w;    // [C][4]
    const bf16_t* norm_w;    // [128]
    bf16_t* state;           // [B][Hv][128][128]: row slot read and replaced
    bf16_t* conv;            // [B][C][3], the current half: row slot read and replaced
    float* qn;               // scratch [L][Hk][128]: normed q times d^-1/2
    float* kn;               // scratch [L][Hk][128]
    float* v;                // scratch [L][Hv][128]
    float* beta;             // scratch [L][Hv]
    float* g;                // scratch [L][Hv]
    float* o;                // scratch [L][Hv][128]
    uint8_t* act;            // e5m2 activation tiles of width Hv*128 for out_proj
    float eps;
};

// Attention over one prefill chunk of one row (prefill.hip); with keys_only, only the keys and values are written
// (the MTP layer's cache_chunk).
struct PrefillAttnArgs {
    int L, Hq, Hkv, S;
    int rows;                // rows of the caches: a slot outside [0, rows) makes every kernel return
    const int* slot;
    const int* start;
    const bf16_t* qkv;       // [L][ld]: per query head [q 256 | gate 256], keys and values from column kv_col
    int ld, kv_col;
    const bf16_t* q_norm;
    const bf16_t* k_norm;
    const bf16_t* cos;       // [L][64]
    const bf16_t* sin;
    bf16_t* k_cache;         // [B][Hkv][S][256]
    bf16_t* v_cache;         // [B][Hkv][S/32][256][32]
    bf16_t* qs;              // scratch [Hq][L][256]: normed, rotated queries times 1/16
    uint8_t* act;            // e5m2 activation tiles of width Hq*256 for o_proj
    float eps;
    int keys_only;
    int kv8;                 // e4m3 caches with the layer's scales, as AttnArgs
    const bf16_t* k_scale;
    const bf16_t* v_scale;
};

#define ATTN_KMAX 8   // verify tokens
#define ATTN_QMAX 64  // query rows per KV head
#define ATTN_CHUNK 512  // cached positions per attn_scores workgroup (32 per wave)

struct AttnArgs {
    int B, K, Hq, Hkv, S;
    const bf16_t* qkv;      // [B*K][ld]: per query head [q 256 | gate 256], then k [Hkv][256], then v [Hkv][256]
    int ld;
    const bf16_t* q_norm;   // [256]
    const bf16_t* k_norm;   // [256]
    const bf16_t* cos;      // [B*K][64]
    const bf16_t* sin;
    const int* position;
    const float* active;
    bf16_t* k_cache;
    bf16_t* v_cache;
    int nchunks;            // chunks of ATTN_CHUNK cached positions over S
    bf16_t* scores;         // [B*Hkv][ATTN_QMAX][S]: the scores times 16 (bf16-exact); attn_pv forms exp(s - chunk max)
    float* stats;           // [B*Hkv][nchunks][ATTN_QMAX][2]: per chunk, max and sum of exp(score - max)
    float* own;             // [B*Hkv][ATTN_QMAX][ATTN_KMAX]: scores of the step's own keys (-inf where masked)
    float* kv_own;          // [B*Hkv][2][ATTN_KMAX][256]: the step's keys (normed, rotated) and values
    bf16_t* qprep;          // [B*Hkv][ATTN_QMAX][256]: query rows normed and rotated, for the rows attn_scores takes
    float* pv_part;         // attn_pv's split sums, [B*Hkv][pv_splits][query tiles][8192]
    size_t pv_part_floats;  // its capacity (splits are capped to fit)
    float* pv_rows;         // [B*Hkv][ATTN_QMAX][2 + ATTN_KMAX]: per query row M, 1 / S and the own weights, for attn_pv_finish
    int pv_splits;          // set by the launcher
    int cus;                // compute units of the device
    uint8_t* act;           // e5m2 activation tiles of width Hq*256 for o_proj
    float eps;
    int fused_max;          // set by the launcher: rows with at most this many visible positions take attn_fused
    int kv8;                // the caches hold e4m3 bytes of value / scale (same layouts, one byte per element)
    const bf16_t* k_scale;  // kv8: the layer's scales, bf16 [1] each
    const bf16_t* v_scale;
};

struct PickArgs {
    const float* maxima;   // [R][ngroups]
    int ngroups;
    const float* x32;      // [R][H]
    const uint8_t* w;      // lm_head tiles [V/32][H/64][64][32]
    const uint8_t* ws;     // lm_head scales [V/32][H/64][32][2]
    const bf16_t* rows;    // lm_head's bf16 rows [V][H] for the recheck, or null (then the tiles, dequantized)
    int* status;           // or null: Q38_STATUS_NONFINITE is or'ed in for a row with no finite logit
    int H, R, groups;
    int* ids;              // [R]
};

hipError_t q38_gemm(const GemmArgs& a, int epi, int* splits_out, hipStream_t stream);
hipError_t q38_residual_norm(const NormArgs& a, hipStream_t stream);
hipError_t q38_head_norm(const bf16_t* hidden, const bf16_t* w, float eps, int H, int rows, bf16_t* tiles, float* x32,
                         hipStream_t stream);
hipError_t q38_embed(const int* ids, int n, const bf16_t* table, int V, int H, bf16_t* out, hipStream_t stream);
hipError_t q38_gdn_gates(const GatesArgs& a, hipStream_t stream);
hipError_t q38_gdn_verify(const GdnArgs& a, hipStream_t stream);
// One decode token per row (a.K == 1): reads qkv_new, z, the gate partials, conv_old and the state; writes conv_new,
// the state in place and act. The snapshot fields are unused.
hipError_t q38_gdn_decode(const GdnArgs& a, hipStream_t stream);
// Copy one row of every listed gated-delta layer's recurrent state ([rows][Hv][128][128] bf16) and conv state
// ([rows][C][3] bf16) between the live buffers and the saved ones; the row is read from `slot` on the device.
#define COPY_STATES_MAX 64  // layers per launch (the pointer tables keep the arguments at 2 KiB)
struct CopyStatesArgs {
    int n;                       // layers
    bf16_t* state[COPY_STATES_MAX];
    bf16_t* saved_state[COPY_STATES_MAX];
    bf16_t* conv[COPY_STATES_MAX];
    bf16_t* saved_conv[COPY_STATES_MAX];
    size_t state_row, conv_row;  // bf16 elements per row
    const int* slot;
    int rows;                    // live rows (slot must be below)
    int to_saved;
};
hipError_t q38_copy_states(const CopyStatesArgs& a, hipStream_t stream);
hipError_t q38_gdn_prefill(const PrefillGdnArgs& a, hipStream_t stream);
hipError_t q38_attn_prefill(const PrefillAttnArgs& a, hipStream_t stream);
hipError_t q38_attn_verify(const AttnArgs& a, hipStream_t stream);
hipError_t q38_head_pick(const PickArgs& a, hipStream_t stream);
hipError_t q38_accept(const int* picks, const int* drafts, const float* active, int B, int K, int* match, int* accepted,
                      hipStream_t stream);
hipError_t q38_pack(const uint8_t* coded, const uint8_t* scales, int N, int K, uint8_t* tiles, uint8_t* tile_scales,
                    hipStream_t stream);
hipError_t q38_pack_fp4(const uint8_t* packed, const uint8_t* scales, int N, int K, uint8_t* tiles, uint8_t* tile_scales,
                        hipStream_t stream);
hipError_t q38_act_tiles(const bf16_t* x, int T, int K, uint8_t* act, hipStream_t stream);
// bf16 activation tiles (the same element order) of x's inputs k with k % 2 == plane; the other inputs zero.
hipError_t q38_act_tiles_bf16(const bf16_t* x, int T, int K, int plane, bf16_t* act, hipStream_t stream);

// Host helpers of the C ABI (engine.cpp): the thread's q38_last_error message (returns 1), the device's CUs, and one
// projection outside a handle (input tiles into act, GEMM counters then fix_floats floats of partial slots at gemm).
int q38_report(const char* msg);
int q38_device_cus();
int q38_projection(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n, int epi,
                   uint8_t* act, uint8_t* gemm, size_t fix_floats, void* out, int splits_max, hipStream_t stream, int w4,
                   int f8, int recompute);
// Step status bits (include/q38.h): a row with no finite logit, a row whose tokens pass the last usable position.
#ifndef Q38_STATUS_NONFINITE
#define Q38_STATUS_NONFINITE 1
#define Q38_STATUS_POSITION 2
#endif
hipError_t q38_rope_gather(const int* base, int offset, int B, int K, int S, const bf16_t* table, bf16_t* cos, bf16_t* sin,
                           hipStream_t s, const float* active = nullptr, int* status = nullptr);
hipError_t q38_select_rows(const bf16_t* rows, const int* idx, int B, int K, int H, bf16_t* out, hipStream_t s);
hipError_t q38_mtp_followup(const bf16_t* current, const int* draft, int B, int K, int H, bf16_t* states, int* ids,
                            hipStream_t s);
hipError_t q38_verify_tokens(const int* picks, const int* match, const int* drafts, int B, int K, int* ids, hipStream_t s);
hipError_t q38_offset_positions(const int* index, const int* match, int add, int B, int* at, hipStream_t s);
hipError_t q38_advance(int* position, int* index, const int* accepted, int B, hipStream_t s);
hipError_t q38_draft_column(const int* ids, int K, int B, int j, int* drafts, hipStream_t s);
