// Full attention, multi-token verify form: `FullAttentionStep.verify` with a bf16 cache (reference
// qwen38_inf2/model.py:641-672, projections and norms model.py:565-577, RoPE model.py:70-82). The query rows of one
// (row, KV head) are its G query heads x K verify tokens.
//
// Reference arithmetic, kept here: q and k RMS-normed (1 + w) in float32 then bf16; RoPE on the first 64 dims in bf16
// ops; scores are a bf16 matmul (float32 sums rounded to bf16); cache positions before `position` are visible and the
// step's own tokens causally; softmax of scores / 16 in float32, weights rounded to bf16; cache part and own part are
// separate bf16 matmuls added in bf16; times bf16 sigmoid(gate). The masked entries of the reference's full-length
// softmax contribute exact zeros (exp of about -600 underflows), so only visible positions are read.
//
// Rows whose visible context is at most NB * 512 positions take one launch, attn_fused (KV head, row): sixteen
// waves score NB blocks of 32 positions each, the softmax completes in the workgroup, and each wave then multiplies
// the weights with 16 dims of V (NB = 2 for up to 32 query rows per KV head, else 1). Longer contexts take two or
// three more launches, so that every (row, KV head) spreads over several workgroups (each kernel skips the rows the
// other path takes); for them attn_fused only prepares the row once: its query rows normed and rotated (qprep) and
// the step's own keys, normed and rotated, and values (kv_own).
//   attn_scores (chunk of 512 cached positions, KV head, row): the prepared query rows, the chunk's scores by MFMA
//       (sixteen waves, one block of 32 positions each), the chunk's per-row max m_c, the sum s_c of e = exp(s - m_c),
//       and the scores s themselves (stored as bf16: each is bf16 / 16, so two bytes hold it exactly; rows past the
//       real query rows are not stored). Chunk 0 also scores the step's own keys.
//   attn_pv (split of the row's positions, KV head, row; eight waves, all 256 dims): the row's max M and sum
//       S = sum_c s_c e^(m_c - M) + own terms; per group of 64 positions, each bf16 weight bf16(e * (e^(m_c - M) / S))
//       formed once from the stored scores (e = exp(s - m_c), the same float32 values attn_scores summed) into LDS,
//       and multiplied with V by MFMA, each wave 32 dims, groups added in position order. With one split per row it
//       finishes the row (below); with more, it stores its sums.
//   attn_pv_finish (quarter of the dims, KV head, row; only with several splits): the splits' sums added in split
//       order, then the row finished: the own part, the gate, e5m2 activation tiles for o_proj, the step's keys and
//       values into the cache.
//   The weights differ from the reference's bf16(e^(s - M) / S) by a few float32 ulps before the bf16 rounding (the
//   product of two exponentials).
//
// FP8 KV cache (KV8; the reference's kv_cache_format "fp8", model.py:557-601 with its CPU path's _store / _load /
// _round_trip): the same layouts with one e4m3 byte of value / scale per element. Cached keys and values widen to
// bf16(e4m3 x scale) in registers as they load; the step's own keys and values are used as they read back
// (kv_round_trip) and written as bytes.
//
// Cache layout (this build's): K row-major [B][Hkv][S][256]; V transposed per block of 32 positions,
// [B][Hkv][S/32][256][32], so both MFMA operands read 16 contiguous bytes per lane (8 with KV8):
//   scores  v_mfma_f32_32x32x16_bf16, A = 32 keys x 16 dims, B = 16 dims x 32 query rows
//   output  v_mfma_f32_32x32x16_bf16, A = 32 query rows x 16 positions (weights), B = 16 positions x 32 dims (V)
// The cache loads of a workgroup are issued first, so their latency overlaps the row-statistics work; loads are issued
// before global stores (the pointers may alias as far as the compiler knows, and a load issued after a store waits
// for it).
#include <algorithm>
#include <type_traits>

#include "kernels.h"

#define QPITCH 264  // bf16 elements per query row in LDS (256 + 8: rows start 4 banks apart)

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t u4t __attribute__((ext_vector_type(4)));
typedef uint32_t u2t __attribute__((ext_vector_type(2)));

namespace {

__device__ __forceinline__ v8bf load8(const bf16_t* p) { return *(const v8bf*)p; }

__device__ __forceinline__ int visible(const AttnArgs& a, int b) { return min(max(a.position[b], 0), a.S); }

__device__ __forceinline__ void unpack4(uint2 r, float* v) {
    v[0] = bf2f(r.x & 0xffff);
    v[1] = bf2f(r.x >> 16);
    v[2] = bf2f(r.y & 0xffff);
    v[3] = bf2f(r.y >> 16);
}

__device__ __forceinline__ uint2 pack4(const float* v) { return make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3])); }

// Row of a 32x32 MFMA accumulator held in element i by `lane` (columns are lane % 32).
__device__ __forceinline__ int acc_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

constexpr int SW = ATTN_CHUNK / 32;  // waves of the 1024-thread kernels: one block of 32 positions each

// This wave's 32 keys of the cache, positions p0 .. p0 + 31: lane l holds key l % 32, dims 128 (l / 32) + 8m .. + 7
// in kf[m].
template <bool KV8>
__device__ __forceinline__ void load_keys(const AttnArgs& a, size_t head, int p0, int lane, v8bf (&kf)[16]) {
    const size_t off = (head * a.S + p0 + (lane & 31)) * 256 + (lane >> 5) * 128;
    if constexpr (KV8) {
        const uint8_t* kp = (const uint8_t*)a.k_cache + off;
        uint2 r[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) r[m] = *(const uint2*)(kp + m * 8);
        const float sc = bf2f(*a.k_scale);
#pragma unroll
        for (int m = 0; m < 16; ++m) kf[m] = __builtin_bit_cast(v8bf, kv_widen8(r[m].x, r[m].y, sc));
    } else {
#pragma unroll
        for (int m = 0; m < 16; ++m) kf[m] = load8(a.k_cache + off + m * 8);
    }
}

// q rows normed and rotated (bf16, qb; rows NQ .. QT*32 - 1 zero) and, with `own`, the step's keys normed and rotated
// (bf16, kb) and values: to kv_own (float32, global) and/or vown (float32, LDS), where given; with KV8 the own keys
// and values as they read back from the cache. NWV waves; wave w takes rows w, w + NWV, ...; lane l holds dims
// 4l .. 4l + 3. load() issues every load, unconditionally (rows past the real ones read row 0, cos/sin past dim 64
// read dims 0-63), so that a kernel can issue its cache loads behind them and wait for these alone in finish().
template <int QT, int NWV, bool KV8>
struct RowLoads {
    static constexpr int RPW = (QT * 32 + 2 * ATTN_KMAX + NWV - 1) / NWV;
    uint2 raw[RPW], rc[RPW], rs_[RPW], qn, kn;
    bf16_t ksc_b, vsc_b;

    __device__ __forceinline__ void load(const AttnArgs& a, int b, int kvh, int wave, int lane, bool own) {
        const int K = a.K, G = a.Hq / a.Hkv, NQ = G * K;
        const int nrows = QT * 32 + (own ? 2 * K : 0), d0 = lane * 4;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            int r = wave + NWV * i;
            if (r >= nrows || (r >= NQ && r < QT * 32)) r = 0;
            const bf16_t* src;
            int t;
            if (r < NQ) {
                t = r % K;
                src = a.qkv + ((size_t)b * K + t) * a.ld + (size_t)(kvh * G + r / K) * 512;
            } else if (r < QT * 32 + K) {
                t = r - QT * 32;
                src = a.qkv + ((size_t)b * K + t) * a.ld + (size_t)a.Hq * 512 + kvh * 256;
            } else {
                t = r - QT * 32 - K;
                src = a.qkv + ((size_t)b * K + t) * a.ld + (size_t)a.Hq * 512 + (size_t)a.Hkv * 256 + kvh * 256;
            }
            raw[i] = *(const uint2*)(src + d0);
            rc[i] = *(const uint2*)(a.cos + ((size_t)b * K + t) * 64 + (d0 & 63));
            rs_[i] = *(const uint2*)(a.sin + ((size_t)b * K + t) * 64 + (d0 & 63));
        }
        qn = *(const uint2*)(a.q_norm + d0);
        kn = *(const uint2*)(a.k_norm + d0);
        if constexpr (KV8) ksc_b = *a.k_scale, vsc_b = *a.v_scale;
    }

    __device__ __forceinline__ void finish(const AttnArgs& a, int wave, int lane, bool own, bf16_t* qb, bf16_t* kb,
                                           float* kv_own, float (*vown)[256]) {
        const int K = a.K, G = a.Hq / a.Hkv, NQ = G * K;
        const int nrows = QT * 32 + (own ? 2 * K : 0), d0 = lane * 4;
        float qn_w[4], kn_w[4], ksc = 0.0f, vsc = 0.0f;
        if constexpr (KV8) ksc = bf2f(ksc_b), vsc = bf2f(vsc_b);
        unpack4(qn, qn_w);
        unpack4(kn, kn_w);

        // All rows' sums of squares reduced together (independent shuffle chains), then norm, RoPE and stores.
        float v[RPW][4], ss[RPW];
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            unpack4(raw[i], v[i]);
            ss[i] = v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
            for (int i = 0; i < RPW; ++i) ss[i] += __shfl_xor(ss[i], o);
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int r = wave + NWV * i;
            const float* nw = r < QT * 32 ? qn_w : kn_w;
            const float rsq = 1.0f / sqrtf(ss[i] / 256.0f + a.eps);
            float hn[4], part[4], cs[4], sn[4], out[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) hn[e] = rbf(v[i][e] * rsq * (1.0f + nw[e]));
#pragma unroll
            for (int e = 0; e < 4; ++e) part[e] = __shfl_xor(hn[e], 8);
            unpack4(rc[i], cs);
            unpack4(rs_[i], sn);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = d0 + e;
                const float rot = d < 32 ? -part[e] : part[e];
                out[e] = d < 64 ? rbf(rbf(hn[e] * cs[e]) + rbf(rot * sn[e])) : hn[e];
            }
            if (r < QT * 32) {
                *(uint2*)(qb + r * QPITCH + d0) = r < NQ ? pack4(out) : make_uint2(0, 0);
            } else if (r >= nrows) {
                // rows of own keys and values exist only with `own`
            } else if (r < QT * 32 + K) {
                const int t = r - QT * 32;
                if constexpr (KV8)
#pragma unroll
                    for (int e = 0; e < 4; ++e) out[e] = kv_round_trip(out[e], ksc);
                *(uint2*)(kb + t * QPITCH + d0) = pack4(out);
                if (kv_own) *(v4f*)(kv_own + t * 256 + d0) = (v4f){out[0], out[1], out[2], out[3]};
            } else {
                const int t = r - QT * 32 - K;
                if constexpr (KV8)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[i][e] = kv_round_trip(v[i][e], vsc);
                if (kv_own) *(v4f*)(kv_own + (ATTN_KMAX + t) * 256 + d0) = (v4f){v[i][0], v[i][1], v[i][2], v[i][3]};
                if (vown) *(v4f*)&vown[t][d0] = (v4f){v[i][0], v[i][1], v[i][2], v[i][3]};
            }
        }
    }
};

// Scores of 32 keys against the query tiles (lane l: query row l % 32 of each 32-row tile, positions p0 +
// acc_row(i, l)), as rbf(q.k) / 16, -inf at positions p_hi and beyond; lmax takes their maximum.
template <int QT>
__device__ __forceinline__ void score_block(const v8bf (&kf)[16], const bf16_t* qb, int lane, int p0, int p_hi,
                                            v16f (&sacc)[QT], float (&lmax)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const bf16_t* qp = qb + (qt * 32 + (lane & 31)) * QPITCH + (lane >> 5) * 128;
        v16f acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[m], load8(qp + m * 8), acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[i] = p0 + acc_row(i, lane) < p_hi ? rbf(acc[i]) * 0.0625f : -INFINITY;
            lmax[qt] = fmaxf(lmax[qt], acc[i]);
        }
        sacc[qt] = acc;
    }
}

// Scores of the step's own keys (kb rows 0..K-1; rows past K read as zero): query row q = g*K + t sees own tokens
// t' <= t. Calls f(q, t', score) for q < NQ, t' < K.
template <int QT, typename F>
__device__ __forceinline__ void own_scores(const bf16_t* qb, const bf16_t* kb, int lane, int K, int NQ, F f) {
    const bool key_row = (lane & 31) < K;
    v8bf zero;
#pragma unroll
    for (int e = 0; e < 8; ++e) zero[e] = (__bf16)0.0f;
    const bf16_t* kp = kb + min(lane & 31, ATTN_KMAX - 1) * QPITCH + (lane >> 5) * 128;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const bf16_t* qp = qb + (qt * 32 + (lane & 31)) * QPITCH + (lane >> 5) * 128;
        v16f acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(key_row ? load8(kp + m * 8) : zero, load8(qp + m * 8), acc, 0, 0, 0);
        const int q = qt * 32 + (lane & 31);
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // key rows 0..7
            const int tp = acc_row(i, lane);
            if (tp < K && q < NQ) f(q, tp, tp <= q % K ? rbf(acc[i]) * 0.0625f : -INFINITY);
        }
    }
}

// Whole verify attention of one (row, KV head) whose visible context is at most NB * ATTN_CHUNK positions: 16 waves;
// wave w scores the blocks of positions 32 (16 nb + w) + [0, 32), nb < NB, then takes dims 16w .. 16w + 15 of the
// output. The softmax is complete inside the workgroup, so the weights are the reference's bf16(e^(s - M) / S) exactly;
// they go through LDS to the weights x V product (v_mfma_f32_16x16x32_bf16: A = 16 query rows x 32 positions, B = 32
// positions x 16 dims), one pass of 16 position blocks per nb.
template <int QT, int NB, bool KV8>
__global__ __launch_bounds__(SW * 64) void attn_fused_kernel(const AttnArgs a) {
    constexpr int RT = QT * 2;                   // 16-row tiles of query rows
    constexpr int WPITCH = NB * ATTN_CHUNK + 8;  // bf16 per weight row in LDS (rows start 4 banks apart)
    __shared__ __attribute__((aligned(16))) bf16_t qb[QT * 32 * QPITCH];
    __shared__ __attribute__((aligned(16))) bf16_t kb[ATTN_KMAX * QPITCH];
    __shared__ __attribute__((aligned(16))) float vown[ATTN_KMAX][256];
    __shared__ float sown[QT * 32][ATTN_KMAX], wown[QT * 32][ATTN_KMAX];
    __shared__ float wred[SW][QT * 32], mrow[QT * 32], irow[QT * 32];
    __shared__ __attribute__((aligned(16))) bf16_t wts[QT * 32 * WPITCH];

    const int kvh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K, G = a.Hq / a.Hkv, NQ = G * K, S = a.S;
    const int npos = visible(a, b);
    const size_t head = (size_t)b * a.Hkv + kvh;
    if (npos > NB * ATTN_CHUNK) {
        // The chunked kernels take this row: here only its rows, once for all of its chunks — the query rows normed
        // and rotated into qprep, the step's own keys (normed, rotated) and values into kv_own.
        RowLoads<QT, SW, KV8> rows;
        rows.load(a, b, kvh, wave, lane, true);
        rows.finish(a, wave, lane, true, qb, kb, a.kv_own + head * 2 * ATTN_KMAX * 256, nullptr);
        __syncthreads();
        bf16_t* dst = a.qprep + head * ATTN_QMAX * 256;
        for (int i = tid; i < QT * 32 * 32; i += SW * 64) {  // 16-byte pieces: row i / 32, dims 8 (i % 32) + [0, 8)
            const int r = i >> 5, d = (i & 31) * 8;
            *(uint4*)(dst + r * 256 + d) = *(const uint4*)(qb + r * QPITCH + d);
        }
        return;
    }
    auto scored = [&](int nb) { return (nb * SW + wave) * 32 < npos; };
    const int dcol = wave * 16 + (lane & 15);  // output dim of this lane

    // The step's rows first, then this wave's cache keys (the first block also for waves past the visible positions,
    // whose scores are never formed): the row work waits for its own loads only. The compiler barriers keep that
    // order.
    RowLoads<QT, SW, KV8> rows;
    rows.load(a, b, kvh, wave, lane, true);
    asm volatile("" ::: "memory");
    v8bf kf[16];
    load_keys<KV8>(a, head, min(wave * 32, S - 32), lane, kf);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);  // nor may the row arithmetic (and its waits) be scheduled above the key loads
    rows.finish(a, wave, lane, true, qb, kb, nullptr, vown);
    __syncthreads();

    v16f sacc[NB][QT];
    float lmax[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) lmax[qt] = -INFINITY;
    if (scored(0)) score_block<QT>(kf, qb, lane, wave * 32, npos, sacc[0], lmax);
#pragma unroll
    for (int nb = 1; nb < NB; ++nb)
        if (scored(nb)) {
            load_keys<KV8>(a, head, (nb * SW + wave) * 32, lane, kf);
            score_block<QT>(kf, qb, lane, (nb * SW + wave) * 32, npos, sacc[nb], lmax);
        }
    if (wave == SW - 1) own_scores<QT>(qb, kb, lane, K, NQ, [&](int q, int tp, float v) { sown[q][tp] = v; });

    // This wave's V columns over the first 16 position blocks: lane l holds dim dcol, positions 32j + 8 (l / 16) ..
    // + 7. Issued only once the keys are consumed (the compiler barrier keeps both out of registers at once).
    asm volatile("" ::: "memory");
    const int nblk = (npos + 31) >> 5;
    v8bf vf[SW];
    uint2 vr[SW];  // KV8: the raw bytes, widened at their MFMA
    const size_t voff = head * S * 256 + dcol * 32 + 8 * (lane >> 4);
    const float vsc = KV8 ? bf2f(*a.v_scale) : 0.0f;
    auto load_v = [&](int nb) {
#pragma unroll
        for (int j = 0; j < SW; ++j) {
            const size_t off = voff + (size_t)max(min(nb * SW + j, nblk - 1), 0) * 8192;  // past nblk: unused
            if constexpr (KV8)
                vr[j] = *(const uint2*)((const uint8_t*)a.v_cache + off);
            else
                vf[j] = load8(a.v_cache + off);
        }
    };
    load_v(0);

#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float m = fmaxf(lmax[qt], __shfl_xor(lmax[qt], 32));
        if (lane < 32) wred[wave][qt * 32 + lane] = m;
    }
    __syncthreads();
    if (tid < QT * 32) {
        float m = wred[0][tid];
#pragma unroll
        for (int w = 1; w < SW; ++w) m = fmaxf(m, wred[w][tid]);
        if (tid < NQ)
            for (int tp = 0; tp < K; ++tp) m = fmaxf(m, sown[tid][tp]);
        mrow[tid] = m;
    }
    __syncthreads();

    // e = exp(s - M); the row sums over the cache positions, then the own terms.
    float lsum[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        lsum[qt] = 0.0f;
        const float m = mrow[qt * 32 + (lane & 31)];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (!scored(nb)) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sacc[nb][qt][i] = expf(sacc[nb][qt][i] - m);
                lsum[qt] += sacc[nb][qt][i];
            }
        }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float s = lsum[qt] + __shfl_xor(lsum[qt], 32);
        if (lane < 32) wred[wave][qt * 32 + lane] = s;
    }
    __syncthreads();
    if (tid < QT * 32) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < SW; ++w) s += wred[w][tid];
        const float m = mrow[tid];
        for (int tp = 0; tp < K; ++tp)
            if (tid < NQ && sown[tid][tp] > -INFINITY) s += expf(sown[tid][tp] - m);
        const float iv = s > 0.0f ? 1.0f / s : 0.0f;
        irow[tid] = iv;
        for (int tp = 0; tp < ATTN_KMAX; ++tp)
            wown[tid][tp] = tid < NQ && tp < K && sown[tid][tp] > -INFINITY ? rbf(expf(sown[tid][tp] - m) * iv) : 0.0f;
    }
    __syncthreads();

    // bf16 weights of this wave's positions into LDS (rows of WPITCH), four consecutive positions per store.
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            if (!scored(nb)) continue;
            const int q = qt * 32 + (lane & 31);
            const float iv = irow[q];
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *(uint2*)(wts + q * WPITCH + (nb * SW + wave) * 32 + g * 8 + (lane >> 5) * 4) =
                    make_uint2(pk_bf16(sacc[nb][qt][4 * g] * iv, sacc[nb][qt][4 * g + 1] * iv),
                               pk_bf16(sacc[nb][qt][4 * g + 2] * iv, sacc[nb][qt][4 * g + 3] * iv));
        }
    __syncthreads();

    // Weights x V for this wave's 16 dims; then the own part, the gate and the e5m2 activation bytes. The gates load
    // here, where the scores' registers are free, behind the V loads and ahead of the MFMAs that hide them.
    uint32_t gate[RT][4];  // gates of this lane's output rows rt*16 + 4 (l / 16) + i, dim dcol
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = min(rt * 16 + 4 * (lane >> 4) + i, NQ - 1);
            gate[rt][i] = a.qkv[(size_t)(b * K + q % K) * a.ld + (size_t)(kvh * G + q / K) * 512 + 256 + dcol];
        }
    v4f acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (nb > 0) {
            if (nb * SW >= nblk) break;
            load_v(nb);
        }
#pragma unroll
        for (int j = 0; j < SW; ++j)
            if (nb * SW + j < nblk) {
                v8bf vj;
                if constexpr (KV8)
                    vj = __builtin_bit_cast(v8bf, kv_widen8(vr[j].x, vr[j].y, vsc));
                else
                    vj = vf[j];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        load8(wts + (rt * 16 + (lane & 15)) * WPITCH + (nb * SW + j) * 32 + 8 * (lane >> 4)), vj, acc[rt], 0, 0, 0);
            }
    }
    const int act_k = a.Hq * 256;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = rt * 16 + 4 * (lane >> 4) + i;
            if (q >= NQ) continue;
            float own = 0.0f;
            for (int tp = 0; tp < K; ++tp) own += wown[q][tp] * vown[tp][dcol];
            float o = rbf(rbf(acc[rt][i]) + rbf(own));
            o = rbf(o * rbf(sigmoidf_(bf2f((bf16_t)gate[rt][i]))));
            a.act[act_offset(b * K + q % K, (kvh * G + q / K) * 256 + dcol, act_k)] = (uint8_t)e5m2_byte(o);
        }

    // The step's own keys and values into the cache (model.py:603-608, 653-654) once every wave has read its V;
    // inactive rows write the tail.
    __syncthreads();
    const int base = a.active[b] > 0.5f ? a.position[b] : S - K;
    const float ksc = KV8 ? bf2f(*a.k_scale) : 0.0f;
    for (int i = tid; i < K * 256; i += SW * 64) {
        const int t = i >> 8, d = i & 255, p = base + t;
        if (p < 0 || p >= S) continue;
        const size_t ko = (head * S + p) * 256 + d, vo = head * S * 256 + (size_t)(p >> 5) * 8192 + d * 32 + (p & 31);
        if constexpr (KV8) {
            ((uint8_t*)a.k_cache)[ko] = (uint8_t)kv_code(bf2f(kb[t * QPITCH + d]), ksc);
            ((uint8_t*)a.v_cache)[vo] = (uint8_t)kv_code(vown[t][d], vsc);
        } else {
            a.k_cache[ko] = kb[t * QPITCH + d];
            a.v_cache[vo] = f2bf(vown[t][d]);
        }
    }
}

template <int QT, bool KV8>
__global__ __launch_bounds__(SW * 64) void attn_scores_kernel(const AttnArgs a) {
    __shared__ __attribute__((aligned(16))) bf16_t qb[QT * 32 * QPITCH];
    __shared__ __attribute__((aligned(16))) bf16_t kb[ATTN_KMAX * QPITCH];  // own keys (chunk 0)
    __shared__ float wred[SW][QT * 32], mrow[QT * 32];

    const int c = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K, G = a.Hq / a.Hkv, NQ = G * K, S = a.S;
    const int npos = visible(a, b);
    if (npos <= a.fused_max) return;  // attn_fused takes this row
    const int p_lo = c * ATTN_CHUNK, p_hi = min(p_lo + ATTN_CHUNK, npos);
    const bool first = c == 0;  // also does the step's own keys
    if (!first && p_lo >= p_hi) return;
    const size_t head = (size_t)b * a.Hkv + kvh;
    const int blk = (p_lo >> 5) + wave;  // this wave's 32 positions
    const bool scored = blk * 32 < p_hi;

    // The query rows as attn_fused prepared them (normed, rotated; chunk 0 also the step's own keys) first, then the
    // cache keys (clamped into the cache for waves past the chunk's positions, whose scores are never formed), so that
    // the copy into LDS waits for its own loads only.
    constexpr int QP = QT * 32 * 32 / (SW * 64);  // 16-byte pieces of the query rows per thread
    const bf16_t* qsrc = a.qprep + head * ATTN_QMAX * 256;
    uint4 qv[QP];
#pragma unroll
    for (int u = 0; u < QP; ++u) qv[u] = *(const uint4*)(qsrc + (tid + u * SW * 64) * 8);
    const float* ksrc = a.kv_own + head * 2 * ATTN_KMAX * 256;
    float4 kv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // own keys: 4 of K x 256 per thread (chunk 0)
    if (first && tid * 4 < K * 256) kv = *(const float4*)(ksrc + tid * 4);
    asm volatile("" ::: "memory");
    v8bf kf[16];
    load_keys<KV8>(a, head, min(blk * 32, S - 32), lane, kf);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);  // nor may the copies (and their waits) be scheduled above the key loads
#pragma unroll
    for (int u = 0; u < QP; ++u) {
        const int i = tid + u * SW * 64, r = i >> 5, d = (i & 31) * 8;
        *(uint4*)(qb + r * QPITCH + d) = qv[u];
    }
    if (first && tid * 4 < K * 256) {
        const int t = (tid * 4) >> 8, d = (tid * 4) & 255;
        *(uint2*)(kb + t * QPITCH + d) = make_uint2(pk_bf16(kv.x, kv.y), pk_bf16(kv.z, kv.w));
    }
    __syncthreads();

    // The wave's block of scores, kept in registers; chunk 0's last wave also scores the own keys.
    v16f sacc[QT];
    float lmax[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) lmax[qt] = -INFINITY;
    if (scored) score_block<QT>(kf, qb, lane, blk * 32, p_hi, sacc, lmax);
    if (first && wave == SW - 1)
        own_scores<QT>(qb, kb, lane, K, NQ,
                       [&](int q, int tp, float v) { a.own[(head * ATTN_QMAX + q) * ATTN_KMAX + tp] = v; });

#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float m = fmaxf(lmax[qt], __shfl_xor(lmax[qt], 32));
        if (lane < 32) wred[wave][qt * 32 + lane] = m;
    }
    __syncthreads();
    if (tid < QT * 32) {
        float m = wred[0][tid];
#pragma unroll
        for (int w = 1; w < SW; ++w) m = fmaxf(m, wred[w][tid]);
        mrow[tid] = m;
    }
    __syncthreads();

    // Phase C: the sums of the chunk's e = exp(s - m_c), and the scores themselves for attn_out, which forms the same
    // e from them. A score is bf16(acc) / 16 (score_block), so 16 s is a bf16 value and its upper half keeps it whole:
    // two bytes a score instead of the four of e.
    float lsum[QT];
    bf16_t* sr = a.scores + head * ATTN_QMAX * S;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        lsum[qt] = 0.0f;
        if (!scored) continue;
        const int q = qt * 32 + (lane & 31);
        const float m = mrow[q];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float s[4] = {sacc[qt][g * 4], sacc[qt][g * 4 + 1], sacc[qt][g * 4 + 2], sacc[qt][g * 4 + 3]};
            lsum[qt] += (expf(s[0] - m) + expf(s[1] - m)) + (expf(s[2] - m) + expf(s[3] - m));
            uint32_t hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) hi[i] = __float_as_uint(s[i] * 16.0f) >> 16;
            if (q < NQ)  // rows past NQ are never read
                *(uint2*)(sr + (size_t)q * S + blk * 32 + g * 8 + (lane >> 5) * 4) =
                    make_uint2(hi[0] | hi[1] << 16, hi[2] | hi[3] << 16);
        }
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float s = lsum[qt] + __shfl_xor(lsum[qt], 32);
        if (lane < 32) wred[wave][qt * 32 + lane] = s;
    }
    __syncthreads();
    if (tid < QT * 32) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < SW; ++w) s += wred[w][tid];
        float* st = a.stats + ((head * a.nchunks + c) * ATTN_QMAX + tid) * 2;
        st[0] = mrow[tid];
        st[1] = mrow[tid] == -INFINITY ? 0.0f : s;
    }
}

constexpr int PV_GP = 64;          // positions per group of attn_pv: one LDS weight tile and one barrier
constexpr int PV_WP = PV_GP + 8;    // bf16 per weight row in LDS (rows start 4 banks apart)
constexpr int PV_RP = 256 + 4;      // floats per row of the output tile in LDS
constexpr int PV_SPLIT_MAX = 16;

// The row statistics of the chunked path, by all 512 threads (a barrier inside): the row's max M over its chunks'
// maxima and own scores, 1 / S with S = sum_c s_c e^(m_c - M) + its own terms e^(s - M), and its own weights
// bf16(e^(s - M) / S). Each row's chunks are split in P contiguous parts, one thread each; the parts' sums are added
// in part order, so the result is fixed. red holds 512 floats.
template <int QT>
__device__ __forceinline__ void pv_row_stats(const AttnArgs& a, size_t head, int npos, int tid, float* mx, float* inv,
                                             float (*wown)[ATTN_KMAX], float* red) {
    constexpr int R = QT * 32, P = 512 / R;
    const int K = a.K, NQ = a.Hq / a.Hkv * K;
    const int r = tid % R, p = tid / R;
    const int nch = (npos + ATTN_CHUNK - 1) / ATTN_CHUNK, c0 = p * nch / P, c1 = (p + 1) * nch / P;
    const float* st = a.stats + head * a.nchunks * ATTN_QMAX * 2 + r * 2;
    float m = -INFINITY;
    for (int c = c0; c < c1; ++c) m = fmaxf(m, st[c * ATTN_QMAX * 2]);
    red[tid] = m;
    __syncthreads();
    float so[ATTN_KMAX];
    if (tid < R) {
        const float* own = a.own + (head * ATTN_QMAX + tid) * ATTN_KMAX;
#pragma unroll
        for (int tp = 0; tp < ATTN_KMAX; ++tp) so[tp] = tp < K && tid < NQ ? own[tp] : -INFINITY;
        float mm = red[tid];
#pragma unroll
        for (int q = 1; q < P; ++q) mm = fmaxf(mm, red[q * R + tid]);
#pragma unroll
        for (int tp = 0; tp < ATTN_KMAX; ++tp) mm = fmaxf(mm, so[tp]);
        mx[tid] = mm;
    }
    __syncthreads();
    const float M = mx[r];
    float s = 0.0f;
    for (int c = c0; c < c1; ++c) {
        const float sc_ = st[c * ATTN_QMAX * 2 + 1];
        if (sc_ > 0.0f) s += sc_ * expf(st[c * ATTN_QMAX * 2] - M);
    }
    red[tid] = s;
    __syncthreads();
    if (tid < R) {
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < P; ++q) ss += red[q * R + tid];
#pragma unroll
        for (int tp = 0; tp < ATTN_KMAX; ++tp)
            if (so[tp] > -INFINITY) ss += expf(so[tp] - M);
        const float iv = ss > 0.0f ? 1.0f / ss : 0.0f;
        inv[tid] = iv;
#pragma unroll
        for (int tp = 0; tp < ATTN_KMAX; ++tp) wown[tid][tp] = so[tp] > -INFINITY ? rbf(expf(so[tp] - M) * iv) : 0.0f;
    }
}

// The step's own values (float32), dims dbase .. dbase + 32 NW - 1, into LDS ([K][32 NW]), for the own part of the
// output; NW * 64 threads.
template <int NW>
__device__ __forceinline__ void pv_own_values(const AttnArgs& a, size_t head, int dbase, int tid, float* vown) {
    constexpr int D = 32 * NW;
    const float* src = a.kv_own + (head * 2 + 1) * ATTN_KMAX * 256 + dbase;
    for (int i = tid * 4; i < a.K * D; i += NW * 64 * 4) *(v4f*)&vown[i] = *(const v4f*)(src + (i / D) * 256 + i % D);
}

// The output of one (row, KV head) from the weights x V sums in acc (NW waves; wave w: dims dbase + 32w + l % 32 of
// its lane l, query rows acc_row(i, l) of each 32-row tile): own part, gate and e5m2 activation bytes, as the
// reference adds them (cache part and own part as separate bf16 matmuls added in bf16, then times bf16
// sigmoid(gate)); then the step's own keys and values of these dims into the cache (model.py:603-608, 653-654;
// inactive rows write the tail). Every wave has consumed its V loads before the first barrier here, so the cache
// writes come after every read of this row's V in the workgroup. red holds 32 x (32 NW + 4) floats, vown the own
// values of these dims ([K][32 NW]).
template <int QT, bool KV8, int NW>
__device__ __forceinline__ void pv_finish(const AttnArgs& a, int b, int kvh, size_t head, int dbase, v16f (&acc)[QT],
                                          float* red, const float (*wown)[ATTN_KMAX], const float* vown, int tid, int lane,
                                          int wave) {
    constexpr int D = 32 * NW, RP = D + 4, TPR = 2 * NW;  // dims, LDS row pitch, threads per row
    const int K = a.K, G = a.Hq / a.Hkv, NQ = G * K, S = a.S, act_k = a.Hq * 256;
    const int fr = tid / TPR, dl = (tid % TPR) * 16;  // this thread: row fr of each tile, dims dbase + dl .. + 15
    u4t gate[QT][2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int q = min(qt * 32 + fr, NQ - 1);
        const bf16_t* gp = a.qkv + (size_t)(b * K + q % K) * a.ld + (size_t)(kvh * G + q / K) * 512 + 256 + dbase + dl;
        gate[qt][0] = *(const u4t*)gp;
        gate[qt][1] = *(const u4t*)(gp + 8);
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        __syncthreads();  // the weight tiles' last reads (or the previous tile's) are done
#pragma unroll
        for (int i = 0; i < 16; ++i) red[acc_row(i, lane) * RP + wave * 32 + (lane & 31)] = acc[qt][i];
        __syncthreads();
        const int q = qt * 32 + fr;
        if (q < NQ) {
            uint32_t bytes[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const v4f cache = *(const v4f*)&red[fr * RP + dl + 4 * h];
                const u4t gw = gate[qt][h >> 1];
                float gt[4], o[4];
                unpack4(make_uint2(gw[(h & 1) * 2], gw[(h & 1) * 2 + 1]), gt);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float own = 0.0f;
                    for (int tp = 0; tp < K; ++tp) own += wown[q][tp] * vown[tp * D + dl + 4 * h + e];
                    o[e] = rbf(rbf(cache[e]) + rbf(own));
                    o[e] = rbf(o[e] * rbf(sigmoidf_(gt[e])));
                }
                bytes[h] = pk_e5m2(o[0], o[1], o[2], o[3]);
            }
            const int t = q % K, col = (kvh * G + q / K) * 256 + dbase + dl;
            *(uint2*)(a.act + act_offset(b * K + t, col, act_k)) = make_uint2(bytes[0], bytes[1]);
            *(uint2*)(a.act + act_offset(b * K + t, col + 8, act_k)) = make_uint2(bytes[2], bytes[3]);
        }
    }

    const int base = a.active[b] > 0.5f ? a.position[b] : S - K;
    const float* kown = a.kv_own + head * 2 * ATTN_KMAX * 256 + dbase;
    const float ksc = KV8 ? bf2f(*a.k_scale) : 0.0f, vsc = KV8 ? bf2f(*a.v_scale) : 0.0f;
    for (int i = tid; i < K * D; i += NW * 64) {
        const int t = i / D, d = i % D, p = base + t;
        if (p < 0 || p >= S) continue;
        const size_t ko = (head * S + p) * 256 + dbase + d,
                     vo = head * S * 256 + (size_t)(p >> 5) * 8192 + (dbase + d) * 32 + (p & 31);
        if constexpr (KV8) {
            ((uint8_t*)a.k_cache)[ko] = (uint8_t)kv_code(kown[t * 256 + d], ksc);
            ((uint8_t*)a.v_cache)[vo] = (uint8_t)kv_code(vown[t * D + d], vsc);
        } else {
            a.k_cache[ko] = f2bf(kown[t * 256 + d]);
            a.v_cache[vo] = f2bf(vown[t * D + d]);
        }
    }
}

// Weights x V of the chunked path over one split of a (row, KV head)'s positions (blockIdx.x of pv_splits, whole
// groups of 64 positions), eight waves, all 256 dims: per group, the 512 threads form the group's bf16 weights
// bf16(e^(s - m_c) * (e^(m_c - M) / S)) once each, from the scores and chunk maxima attn_scores stored (the float32
// values it summed), into an LDS tile; wave w multiplies the tile with dims 32w .. 32w + 31 of V by MFMA
// (A = 32 query rows x 16 positions from LDS, B = 16 positions x 32 dims from registers), adding the groups in
// position order. Loads run PF groups ahead (slot j of each round of PF; past the range they load the last
// group again, never used, so that every load is unconditional). With one split the workgroup finishes the row;
// with more, each stores its sums and attn_pv_finish adds them in split order.
template <int QT, bool KV8>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void attn_pv_kernel(const AttnArgs a) {
    constexpr int WPT = QT * 32 * PV_GP / 512;  // weights formed per thread per group (4 or 8)
    // Groups whose loads a wave keeps in flight: four, or three where two query tiles of bf16 V would not fit
    // 128 VGPRs (two workgroups per CU) with four.
    constexpr int PF = QT == 2 && !KV8 ? 3 : 4;
    constexpr int NT = PF % 2 == 0 ? 2 : PF;    // LDS weight tiles (slot j writes tile j % NT)
    constexpr int TILE = QT * 32 * PV_WP;       // bf16 per LDS weight tile
    constexpr int SMEM = NT * TILE * 2 > 32 * PV_RP * 4 ? NT * TILE * 2 : 32 * PV_RP * 4;
    __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];  // the weight tiles; after the loop, red
    __shared__ float mx[QT * 32], inv[QT * 32], wown[QT * 32][ATTN_KMAX], sred[512];
    __shared__ __attribute__((aligned(16))) float vown[ATTN_KMAX][256];
    bf16_t* wt = (bf16_t*)smem;

    const int z = blockIdx.x, hh = blockIdx.y, b = hh / a.Hkv, kvh = hh % a.Hkv;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int npos = visible(a, b), S = a.S, ns = a.pv_splits;
    if (npos <= a.fused_max) return;  // attn_fused takes this row
    const size_t head = (size_t)hh;
    const int ngrp = (npos + PV_GP - 1) / PV_GP, g_lo = z * ngrp / ns, g_hi = (z + 1) * ngrp / ns;
    const bf16_t* sr = a.scores + head * ATTN_QMAX * S;
    const float* cst = a.stats + head * a.nchunks * ATTN_QMAX * 2;
    const size_t vc = head * S * 256 + (size_t)(wave * 32 + (lane & 31)) * 32 + (lane >> 5) * 8;
    const float vsc = KV8 ? bf2f(*a.v_scale) : 0.0f;
    const int fr = tid / (PV_GP / WPT), fc = tid % (PV_GP / WPT) * WPT;  // weights formed: row fr, positions + fc
    const int NQ = a.Hq / a.Hkv * a.K, lr = min(fr, NQ - 1);              // rows past NQ load a real row, weigh 0

    // Slot loads: V of this wave's dims over the group's 64 positions (lane half h: positions 16 kk + 8 h .. + 7 of
    // MFMA step kk), the scores of the weights this thread forms and their chunk's max.
    typedef typename std::conditional<KV8, uint2, v8bf>::type VSlot;
    typedef typename std::conditional<WPT == 8, u4t, u2t>::type SSlot;
    VSlot vs[PF][4];
    SSlot ss[PF];
    float mc[PF];
    auto issue = [&](int j, int g) {
        g = min(g, max(g_hi - 1, g_lo));
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const size_t vo = vc + (size_t)min(2 * g + (kk >> 1), S / 32 - 1) * 8192 + (kk & 1) * 16;
            if constexpr (KV8)
                vs[j][kk] = *(const uint2*)((const uint8_t*)a.v_cache + vo);
            else
                vs[j][kk] = load8(a.v_cache + vo);
        }
        ss[j] = *(const SSlot*)(sr + (size_t)lr * S + min(g * PV_GP + fc, S - WPT));
        mc[j] = cst[((g * PV_GP / ATTN_CHUNK) * ATTN_QMAX + lr) * 2];
    };
#pragma unroll
    for (int j = 0; j < PF; ++j) issue(j, g_lo + j);

    pv_row_stats<QT>(a, head, npos, tid, mx, inv, wown, sred);
    if (ns == 1) pv_own_values<8>(a, head, 0, tid, &vown[0][0]);
    __syncthreads();

    v16f acc[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[qt][i] = 0.0f;
    const float fm = mx[lr], fi = inv[lr];
    // Group g from slot j: its weights into tile w (positions at or past npos, and rows past NQ, weigh zero).
    const int nlim = fr < NQ ? npos : 0;
    auto form = [&](int j, int g, bf16_t* w) {
        const float m = mc[j], f = expf(m - fm) * fi;
        const int p0 = g * PV_GP + fc;
        uint32_t words[WPT / 2];
#pragma unroll
        for (int e = 0; e < WPT / 2; ++e) {
            const uint32_t pair = ss[j][e];
            const float s0 = bf2f(pair & 0xffff) * 0.0625f, s1 = bf2f(pair >> 16) * 0.0625f;
            words[e] = pk_bf16(p0 + 2 * e < nlim ? expf(s0 - m) * f : 0.0f, p0 + 2 * e + 1 < nlim ? expf(s1 - m) * f : 0.0f);
        }
        if constexpr (WPT == 8)
            *(uint4*)(w + fr * PV_WP + fc) = make_uint4(words[0], words[1], words[2], words[3]);
        else
            *(uint2*)(w + fr * PV_WP + fc) = make_uint2(words[0], words[1]);
    };
    auto mfma = [&](int j, const bf16_t* w) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            v8bf vb;
            if constexpr (KV8)
                vb = __builtin_bit_cast(v8bf, kv_widen8(vs[j][kk].x, vs[j][kk].y, vsc));
            else
                vb = vs[j][kk];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
                acc[qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    load8(w + (qt * 32 + (lane & 31)) * PV_WP + kk * 16 + (lane >> 5) * 8), vb, acc[qt], 0, 0, 0);
        }
    };
    // Whole rounds of PF groups, each slot refilled after its MFMAs (the loop has no other exit, so the waits at
    // its top count only the oldest slot's loads), then the last, partial round. Tile j % NT was last read NT
    // groups earlier, before the barrier of the group after it.
    int g = g_lo;
    for (; g + PF <= g_hi; g += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            bf16_t* w = wt + (j % NT) * TILE;
            form(j, g + j, w);
            __syncthreads();
            mfma(j, w);
            issue(j, g + j + PF);
        }
    }
#pragma unroll
    for (int j = 0; j < PF - 1; ++j)
        if (g + j < g_hi) {
            bf16_t* w = wt + (j % NT) * TILE;
            form(j, g + j, w);
            __syncthreads();
            mfma(j, w);
        }

    if (ns == 1) {
        pv_finish<QT, KV8, 8>(a, b, kvh, head, 0, acc, (float*)smem, wown, &vown[0][0], tid, lane, wave);
        return;
    }
    if (z == 0 && tid < QT * 32) {  // the row statistics attn_pv_finish needs
        float* rs = a.pv_rows + (head * ATTN_QMAX + tid) * (2 + ATTN_KMAX);
        rs[0] = mx[tid];
        rs[1] = inv[tid];
#pragma unroll
        for (int tp = 0; tp < ATTN_KMAX; ++tp) rs[2 + tp] = wown[tid][tp];
    }
    // This split's sums, [pair][split][tile][wave][i][lane] (each store 256 contiguous bytes).
    float* part = a.pv_part + ((size_t)hh * ns + z) * QT * 8192 + wave * 1024 + lane;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int i = 0; i < 16; ++i) part[qt * 8192 + i * 64] = acc[qt][i];
}

// The splits' sums of one (row, KV head) added in split order, then the row finished as attn_pv finishes it; one
// workgroup of two waves per quarter of the 256 dims (blockIdx.x), with the row statistics split 0 stored.
template <int QT, bool KV8>
__global__ __launch_bounds__(128) void attn_pv_finish_kernel(const AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float red[32 * 68];
    __shared__ float wown[QT * 32][ATTN_KMAX];
    __shared__ __attribute__((aligned(16))) float vown[ATTN_KMAX * 64];
    const int quarter = blockIdx.x, hh = blockIdx.y, b = hh / a.Hkv, kvh = hh % a.Hkv;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int npos = visible(a, b), ns = a.pv_splits;
    if (npos <= a.fused_max) return;
    const size_t head = (size_t)hh;
    const float* part = a.pv_part + (size_t)hh * ns * QT * 8192 + (quarter * 2 + wave) * 1024 + lane;
    v16f acc[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[qt][i] = part[qt * 8192 + i * 64];
#pragma unroll 4
    for (int z = 1; z < ns; ++z)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[qt][i] += part[((size_t)z * QT + qt) * 8192 + i * 64];
    for (int i = tid; i < QT * 32 * ATTN_KMAX; i += 128)
        wown[i / ATTN_KMAX][i % ATTN_KMAX] = a.pv_rows[(head * ATTN_QMAX + i / ATTN_KMAX) * (2 + ATTN_KMAX) + 2 + i % ATTN_KMAX];
    pv_own_values<2>(a, head, quarter * 64, tid, vown);
    pv_finish<QT, KV8, 2>(a, b, kvh, head, quarter * 64, acc, red, wown, vown, tid, lane, wave);
}

template <int QT, int NB, bool KV8>
hipError_t launch_attn(AttnArgs a, hipStream_t stream) {
    a.fused_max = NB * ATTN_CHUNK;
    hipLaunchKernelGGL((attn_fused_kernel<QT, NB, KV8>), dim3(a.Hkv, a.B), dim3(SW * 64), 0, stream, a);
    if (a.S > a.fused_max) {
        // Splits of each (row, KV head)'s positions for attn_pv: about two workgroups per CU in all, as many as the
        // partial buffer holds.
        const long pairs = (long)a.B * a.Hkv;
        int ns = pairs >= 2L * a.cus ? 1 : (int)std::min<long>(PV_SPLIT_MAX, std::max<long>(1, 2L * a.cus / pairs));
        while (ns > 1 && (size_t)pairs * ns * QT * 8192 > a.pv_part_floats) --ns;
        a.pv_splits = ns;
        hipLaunchKernelGGL((attn_scores_kernel<QT, KV8>), dim3(a.nchunks, a.Hkv, a.B), dim3(SW * 64), 0, stream, a);
        hipLaunchKernelGGL((attn_pv_kernel<QT, KV8>), dim3(ns, pairs), dim3(512), 0, stream, a);
        if (ns > 1) hipLaunchKernelGGL((attn_pv_finish_kernel<QT, KV8>), dim3(4, pairs), dim3(128), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t q38_attn_verify(const AttnArgs& a, hipStream_t stream) {
    const int NQ = a.Hq / a.Hkv * a.K;
    if (NQ > ATTN_QMAX || a.K > ATTN_KMAX || (long)a.nchunks * ATTN_CHUNK < a.S) return hipErrorInvalidValue;
    if (a.S < 32 || a.S % 32) return hipErrorInvalidValue;  // whole blocks of 32 positions (every wave loads one)
    // Two position blocks per wave need 66 KB of bf16 weights in LDS at 32 query rows; 64 rows keep one.
    if (a.kv8) {
        if (!a.k_scale || !a.v_scale) return hipErrorInvalidValue;
        return NQ <= 32 ? launch_attn<1, 2, true>(a, stream) : launch_attn<2, 1, true>(a, stream);
    }
    return NQ <= 32 ? launch_attn<1, 2, false>(a, stream) : launch_attn<2, 1, false>(a, stream);
}
