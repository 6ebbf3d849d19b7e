// Full attention, multi-token verify form: `FullAttentionStep.verify` with a bf16 cache (reference
// qwen38_inf2/model.py:641-672, projections and norms model.py:565-577, RoPE model.py:70-82). One workgroup per
// (row, KV head) holds that head's G query heads x K verify tokens as query rows.
//
// Reference arithmetic, kept here: q and k RMS-normed (1 + w) in float32 then bf16; RoPE on the first 64 dims in bf16
// ops; scores are a bf16 matmul (float32 sums rounded to bf16); cache positions before `position` are visible and the
// step's own tokens causally; softmax of scores / 16 in float32, weights rounded to bf16; cache part and own part are
// separate bf16 matmuls added in bf16; times bf16 sigmoid(gate). The masked entries of the reference's full-length
// softmax contribute exact zeros (exp of about -600 underflows), so only visible positions are read.
//
// Cache layout (this build's): K row-major [B][Hkv][S][256]; V transposed per block of 32 positions,
// [B][Hkv][S/32][256][32], so both MFMA operands read 16 contiguous bytes per lane:
//   scores  v_mfma_f32_32x32x16_bf16, A = 32 cached keys x 16 dims, B = 16 dims x 32 query rows
//   output  v_mfma_f32_32x32x16_bf16, A = 32 query rows x 16 positions (weights), B = 16 positions x 32 dims (V)
// Scores of a workgroup go through a global scratch (L2-resident at short context) because the bf16 weights need the
// softmax's final max and sum before any V product; the weights themselves are formed in registers. Loads that feed a
// phase are issued before that phase's global stores (the pointers may alias as far as the compiler knows).
#include "kernels.h"

#define ATTN_KMAX 8
#define ATTN_QMAX 64
#define QPITCH 264  // bf16 elements per query row in LDS (256 + 8: rows start 4 banks apart)

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v8bf load8(const bf16_t* p) { return *(const v8bf*)p; }

template <int QT>
__global__ __launch_bounds__(256) void attn_verify_kernel(const AttnArgs a) {
    __shared__ __attribute__((aligned(16))) bf16_t qb[ATTN_QMAX * QPITCH];
    __shared__ float kown[ATTN_KMAX][256], vown[ATTN_KMAX][256];
    __shared__ float sown[ATTN_QMAX][ATTN_KMAX];
    __shared__ float wmax[4][ATTN_QMAX], wsum[4][ATTN_QMAX];
    __shared__ float mx[ATTN_QMAX], inv[ATTN_QMAX];

    const int kvh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K, G = a.Hq / a.Hkv, NQ = G * K, S = a.S;
    const int npos = min(max(a.position[b], 0), S);
    const int nblk = (npos + 31) >> 5;
    const size_t head = (size_t)b * a.Hkv + kvh;
    float* sc = a.scores + head * ATTN_QMAX * S;
    const bf16_t* kc = a.k_cache + head * S * 256;
    const bf16_t* vc = a.v_cache + head * S * 256;

    // Phase A: normed and rotated q rows (bf16, LDS), own k (normed, rotated) and v. Wave w takes rows w, w + 4, ...;
    // all its global loads are issued first.
    constexpr int RPW = (QT * 32 + 2 * ATTN_KMAX + 3) / 4;
    const int nrows = QT * 32 + 2 * K, d0 = lane * 4;
    uint2 raw[RPW], rc[RPW], rs_[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int r = wave + 4 * i;
        raw[i] = rc[i] = rs_[i] = make_uint2(0, 0);
        if (r >= nrows || (r >= NQ && r < QT * 32)) continue;
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
        if (d0 < 64) {
            rc[i] = *(const uint2*)(a.cos + ((size_t)b * K + t) * 64 + d0);
            rs_[i] = *(const uint2*)(a.sin + ((size_t)b * K + t) * 64 + d0);
        }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int r = wave + 4 * i;
        if (r >= nrows) break;
        if (r >= NQ && r < QT * 32) {
            *(uint2*)(qb + r * QPITCH + d0) = make_uint2(0, 0);
            continue;
        }
        const int kind = r < NQ ? 0 : r < QT * 32 + K ? 1 : 2;
        const int t = kind == 0 ? r % K : kind == 1 ? r - QT * 32 : r - QT * 32 - K;
        float v[4] = {bf2f(raw[i].x & 0xffff), bf2f(raw[i].x >> 16), bf2f(raw[i].y & 0xffff), bf2f(raw[i].y >> 16)};
        if (kind == 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e) vown[t][d0 + e] = v[e];
            continue;
        }
        const bf16_t* nw = kind == 0 ? a.q_norm : a.k_norm;
        float ss = warp_sum(v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3]);
        const float rsq = 1.0f / sqrtf(ss / 256.0f + a.eps);
        float hn[4], part[4], out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) hn[e] = rbf(v[e] * rsq * (1.0f + bf2f(nw[d0 + e])));
#pragma unroll
        for (int e = 0; e < 4; ++e) part[e] = __shfl_xor(hn[e], 8);
        const float cs[4] = {bf2f(rc[i].x & 0xffff), bf2f(rc[i].x >> 16), bf2f(rc[i].y & 0xffff), bf2f(rc[i].y >> 16)};
        const float sn[4] = {bf2f(rs_[i].x & 0xffff), bf2f(rs_[i].x >> 16), bf2f(rs_[i].y & 0xffff), bf2f(rs_[i].y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = d0 + e;
            if (d < 64) {
                float rot = d < 32 ? -part[e] : part[e];
                out[e] = rbf(rbf(hn[e] * cs[e]) + rbf(rot * sn[e]));
            } else {
                out[e] = hn[e];
            }
        }
        if (kind == 0) {
            *(uint2*)(qb + r * QPITCH + d0) = make_uint2((uint32_t)f2bf(out[0]) | ((uint32_t)f2bf(out[1]) << 16),
                                                        (uint32_t)f2bf(out[2]) | ((uint32_t)f2bf(out[3]) << 16));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) kown[t][d0 + e] = out[e];
        }
    }
    __syncthreads();

    // Own scores: query row q = g*K + t sees own tokens t' <= t.
    for (int p = wave; p < NQ * K; p += 4) {
        const int q = p / K, tp = p % K, t = q % K;
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += bf2f(qb[q * QPITCH + lane * 4 + e]) * kown[tp][lane * 4 + e];
        acc = warp_sum(acc);
        if (lane == 0) sown[q][tp] = tp <= t ? rbf(acc) * 0.0625f : -INFINITY;
    }

    // Phase B: cached scores by MFMA, blocks of 32 positions spread over the waves.
    float lmax[2] = {-INFINITY, -INFINITY};
    {
        v8bf qf[2][16];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
            if (qt < QT)
#pragma unroll
                for (int m = 0; m < 16; ++m) qf[qt][m] = load8(qb + (qt * 32 + (lane & 31)) * QPITCH + (lane >> 5) * 128 + m * 8);
        for (int blk = wave; blk < nblk; blk += 4) {
            const int p0 = blk * 32;
            const bf16_t* kp = kc + (size_t)(p0 + (lane & 31)) * 256 + (lane >> 5) * 128;
            v8bf kf[16];
#pragma unroll
            for (int m = 0; m < 16; ++m) kf[m] = load8(kp + m * 8);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                if (qt >= QT) break;
                v16f acc;
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
                for (int m = 0; m < 16; ++m) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[m], qf[qt][m], acc, 0, 0, 0);
                const int q = qt * 32 + (lane & 31);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int p = p0 + g * 8 + (lane >> 5) * 4;
                    v4f s;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s[e] = p + e < npos ? rbf(acc[g * 4 + e]) * 0.0625f : -INFINITY;
                        lmax[qt] = fmaxf(lmax[qt], s[e]);
                    }
                    *(v4f*)(sc + (size_t)q * S + p) = s;
                }
            }
        }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float m = fmaxf(lmax[qt], __shfl_xor(lmax[qt], 32));
        if (lane < 32) wmax[wave][qt * 32 + lane] = m;
    }
    __syncthreads();
    if (tid < ATTN_QMAX) {
        float m = fmaxf(fmaxf(wmax[0][tid], wmax[1][tid]), fmaxf(wmax[2][tid], wmax[3][tid]));
        if (tid < NQ)
            for (int tp = 0; tp < K; ++tp) m = fmaxf(m, sown[tid][tp]);
        mx[tid] = m;
    }
    __syncthreads();

    // Phase C: partial sums of exp(s - max), each wave over the blocks it scored (loads only).
    float lsum[2] = {0.0f, 0.0f};
    for (int blk = wave; blk < nblk; blk += 4) {
        const int p0 = blk * 32;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int q = qt * 32 + (lane & 31);
            const float m = mx[q];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const v4f sv = *(const v4f*)(sc + (size_t)q * S + p0 + g * 8 + (lane >> 5) * 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) lsum[qt] += expf(sv[e] - m);
            }
        }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float sm = lsum[qt] + __shfl_xor(lsum[qt], 32);
        if (lane < 32) wsum[wave][qt * 32 + lane] = sm;
    }
    __syncthreads();
    if (tid < ATTN_QMAX) {
        float sm = (wsum[0][tid] + wsum[1][tid]) + (wsum[2][tid] + wsum[3][tid]);
        if (tid < NQ)
            for (int tp = 0; tp < K; ++tp) sm += expf(sown[tid][tp] - mx[tid]);
        inv[tid] = 1.0f / sm;
    }
    __syncthreads();

    // Phase D: weights x V by MFMA; wave w owns dims [64w, 64w + 64). The bf16 weights, bf16(exp(s - max) / sum), are
    // formed from the scores as each MFMA needs them; two position blocks' loads are in flight at a time.
    v16f acc[QT][2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[qt][dt][i] = 0.0f;
    float qm[QT], qi[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        qm[qt] = mx[qt * 32 + (lane & 31)];
        qi[qt] = inv[qt * 32 + (lane & 31)];
    }
    constexpr int PF = 2;
    for (int blk0 = 0; blk0 < nblk; blk0 += PF) {
        v8bf vf[PF][2][2];
        v4f sf[PF][QT][4];
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            if (blk0 + j >= nblk) break;
            const int p0 = (blk0 + j) * 32;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                const int d = (wave * 2 + dt) * 32 + (lane & 31);
                const bf16_t* vp = vc + (size_t)(blk0 + j) * 8192 + d * 32 + (lane >> 5) * 16;
                vf[j][dt][0] = load8(vp);
                vf[j][dt][1] = load8(vp + 8);
            }
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const float* sp = sc + (size_t)(qt * 32 + (lane & 31)) * S + p0 + (lane >> 5) * 16;
#pragma unroll
                for (int g = 0; g < 4; ++g) sf[j][qt][g] = *(const v4f*)(sp + g * 4);
            }
        }
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            if (blk0 + j >= nblk) break;
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                uint32_t wbits[8];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    wbits[2 * g] = (uint32_t)f2bf(expf(sf[j][qt][g][0] - qm[qt]) * qi[qt]) |
                                   ((uint32_t)f2bf(expf(sf[j][qt][g][1] - qm[qt]) * qi[qt]) << 16);
                    wbits[2 * g + 1] = (uint32_t)f2bf(expf(sf[j][qt][g][2] - qm[qt]) * qi[qt]) |
                                       ((uint32_t)f2bf(expf(sf[j][qt][g][3] - qm[qt]) * qi[qt]) << 16);
                }
                typedef uint32_t u4t __attribute__((ext_vector_type(4)));
                const v8bf w0 = __builtin_bit_cast(v8bf, (u4t){wbits[0], wbits[1], wbits[2], wbits[3]});
                const v8bf w1 = __builtin_bit_cast(v8bf, (u4t){wbits[4], wbits[5], wbits[6], wbits[7]});
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    acc[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, vf[j][dt][0], acc[qt][dt], 0, 0, 0);
                    acc[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, vf[j][dt][1], acc[qt][dt], 0, 0, 0);
                }
            }
        }
    }

    // Phase E: own part, sum, gate, e5m2 for o_proj. Gate values are loaded before the first store.
    const int act_k = a.Hq * 256;
    float gate[QT][2][16];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            const int d = (wave * 2 + dt) * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int q = min(qt * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3), NQ - 1);
                const int tok = b * K + q % K, hq = kvh * G + q / K;
                gate[qt][dt][i] = bf2f(a.qkv[(size_t)tok * a.ld + (size_t)hq * 512 + 256 + d]);
            }
        }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            const int d = (wave * 2 + dt) * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int q = qt * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (q >= NQ) continue;
                const int g = q / K, t = q % K;
                float own = 0.0f;
                for (int tp = 0; tp < K; ++tp) own += rbf(expf(sown[q][tp] - mx[q]) * inv[q]) * vown[tp][d];
                float o = rbf(rbf(acc[qt][dt][i]) + rbf(own));
                const int hq = kvh * G + g, tok = b * K + t;
                o = rbf(o * rbf(sigmoidf_(gate[qt][dt][i])));
                a.act[act_offset(tok, hq * 256 + d, act_k)] = (uint8_t)e5m2_byte(o);
            }
        }
    }
    __syncthreads();

    // Phase F: the step's own keys and values into the cache (model.py:603-608, 653-654).
    for (int i = tid; i < K * 256; i += 256) {
        const int t = i >> 8, d = i & 255;
        const int p = a.active[b] > 0.5f ? a.position[b] + t : S - K + t;
        if (p < 0 || p >= S) continue;
        a.k_cache[(head * S + p) * 256 + d] = f2bf(kown[t][d]);
        a.v_cache[head * S * 256 + (size_t)(p >> 5) * 8192 + d * 32 + (p & 31)] = f2bf(vown[t][d]);
    }
}

hipError_t q38_attn_verify(const AttnArgs& a, hipStream_t stream) {
    if (a.Hq / a.Hkv * a.K <= 32)
        hipLaunchKernelGGL(attn_verify_kernel<1>, dim3(a.Hkv, a.B), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(attn_verify_kernel<2>, dim3(a.Hkv, a.B), dim3(256), 0, stream, a);
    return hipGetLastError();
}
