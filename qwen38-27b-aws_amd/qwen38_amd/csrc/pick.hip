// Token choice from the head's group maxima: `ChipHead.next_tokens` after its graph (reference
// qwen38_inf2/generate.py:186-208), on the GPU so only ids go back to the host.
//   1. the `groups` best groups of 32 vocabulary rows by group maximum (torch.topk order: largest first);
//   2. exact float32 logits of their rows against the float32-normed hidden state: lm_head's bf16 rows when they are
//      bound (the checkpoint's own rows, which the reference rechecks against), else the e4m3 tiles dequantized;
//   3. the best row of each group, and across groups the first strictly larger in top-k order.
// A row with no finite logit gets id -1, which the host turns into the reference's FloatingPointError.
// Greedy acceptance (scheduler.py:291-300) is here too, for the on-device speculative step.
#include "kernels.h"

#define PICK_GMAX 4

typedef float v2f __attribute__((ext_vector_type(2)));

// torch.topk order: NaN first, then larger values; equal values by lower index.
__device__ __forceinline__ bool ranks_before(float a, int ia, float b, int ib) {
    bool na = a != a, nb = b != b;
    if (na != nb) return na;
    if (na) return ia < ib;
    return a > b || (a == b && ia < ib);
}

constexpr int PICK_THREADS = 1024;  // 16 waves: the recheck splits each group's K range over 16 / G waves

__global__ __launch_bounds__(PICK_THREADS) void head_pick_kernel(const PickArgs a) {
    constexpr int NWAVE = PICK_THREADS / 64;
    __shared__ float lv[PICK_THREADS][PICK_GMAX];
    __shared__ int li[PICK_THREADS][PICK_GMAX];
    __shared__ float xrow[8192];
    __shared__ float part[NWAVE][32];
    __shared__ float glogit[PICK_GMAX];
    __shared__ int gtoken[PICK_GMAX];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.groups;

    // 1. The G best groups: each thread's share of the group maxima (eight loads in flight at a time; the ranking does
    //    not depend on the order candidates are seen in), then a merge tree over the threads.
    float bv[PICK_GMAX];
    int bi[PICK_GMAX];
#pragma unroll
    for (int k = 0; k < PICK_GMAX; ++k) {
        bv[k] = -INFINITY;
        bi[k] = 0x7fffffff;
    }
    const float* mrow = a.maxima + (size_t)r * a.ngroups;
    constexpr int CH = 8;
    for (int i0 = tid; i0 < a.ngroups; i0 += PICK_THREADS * CH) {
        float vv[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) vv[c] = i0 + c * PICK_THREADS < a.ngroups ? mrow[i0 + c * PICK_THREADS] : 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i = i0 + c * PICK_THREADS;
            const float v = vv[c];
            if (i >= a.ngroups || !ranks_before(v, i, bv[G - 1], bi[G - 1])) continue;
            int k = G - 1;
            while (k > 0 && ranks_before(v, i, bv[k - 1], bi[k - 1])) {
                bv[k] = bv[k - 1];
                bi[k] = bi[k - 1];
                --k;
            }
            bv[k] = v;
            bi[k] = i;
        }
    }
#pragma unroll
    for (int k = 0; k < PICK_GMAX; ++k) {
        lv[tid][k] = bv[k];
        li[tid][k] = bi[k];
    }
    for (int c = tid; c < a.H; c += PICK_THREADS) xrow[c] = a.x32[(size_t)r * a.H + c];
    __syncthreads();
    for (int stride = PICK_THREADS / 2; stride > 0; stride >>= 1) {
        if (tid < stride) {
            float mv[PICK_GMAX];
            int mi[PICK_GMAX];
            int x = 0, y = 0;
            for (int k = 0; k < G; ++k) {
                bool takex = ranks_before(lv[tid][x], li[tid][x], lv[tid + stride][y], li[tid + stride][y]);
                mv[k] = takex ? lv[tid][x] : lv[tid + stride][y];
                mi[k] = takex ? li[tid][x] : li[tid + stride][y];
                if (takex) ++x; else ++y;
            }
            for (int k = 0; k < G; ++k) {
                lv[tid][k] = mv[k];
                li[tid][k] = mi[k];
            }
        }
        __syncthreads();
    }

    // 2. Exact float32 logits of the G groups' rows: group k's K-steps split into SPL ranges, one wave each; lane l
    //    accumulates row l % 32 over its half of each K-step's inputs. Lane half h holds inputs [16h, 16h + 16) of the
    //    K-step in bytes 0-15 (first MX block) and [32 + 16h, 48 + 16h) in bytes 16-31 (second block).
    const int KS = a.H >> 6, SPL = NWAVE / G;
    const int gk = wave / SPL, sp = wave % SPL;
    if (gk < G) {
        const int grp = li[0][gk];
        float acc = 0.0f;
        if (grp >= 0 && grp < a.ngroups && a.rows) {
            // bf16 row grp * 32 + l % 32; lane half h reads inputs [16h, 16h + 16) and [32 + 16h, 48 + 16h) of each
            // K-step, 32 bytes each (the two half-waves together cover 128 contiguous bytes of the row).
            const bf16_t* wr = a.rows + ((size_t)grp * 32 + (lane & 31)) * a.H + (lane >> 5) * 16;
            const float* xp = xrow + (lane >> 5) * 16;
            const int k0 = sp * KS / SPL, k1 = (sp + 1) * KS / SPL;
#pragma unroll 2
            for (int ks = k0; ks < k1; ++ks) {
#pragma unroll
                for (int blk = 0; blk < 2; ++blk) {
                    const uint4* src = (const uint4*)(wr + ks * 64 + blk * 32);
                    const uint4 q0 = src[0], q1 = src[1];
                    const uint32_t wv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                    const float* xv = xp + ks * 64 + blk * 32;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        acc += __uint_as_float(wv[e] << 16) * xv[2 * e];
                        acc += __uint_as_float(wv[e] & 0xffff0000u) * xv[2 * e + 1];
                    }
                }
            }
        } else if (grp >= 0 && grp < a.ngroups) {
            const uint8_t* tile = a.w + (size_t)grp * KS * 2048 + lane * 8;
            const uint8_t* sc = a.ws + (size_t)grp * KS * 64 + (lane & 31) * 2;
            const float* xp = xrow + (lane >> 5) * 16;
            const int k0 = sp * KS / SPL, k1 = (sp + 1) * KS / SPL;
#pragma unroll 4
            for (int ks = k0; ks < k1; ++ks) {
                const float s0 = __uint_as_float((uint32_t)sc[(size_t)ks * 64] << 23);
                const float s1 = __uint_as_float((uint32_t)sc[(size_t)ks * 64 + 1] << 23);
                // Word w of the lane's 32 bytes: step w / 2 of the tile, at [m][lane][8].
                uint32_t words[8];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint2 rw = *(const uint2*)(tile + (size_t)ks * 2048 + m * 512);
                    words[2 * m] = rw.x;
                    words[2 * m + 1] = rw.y;
                }
#pragma unroll
                for (int wi = 0; wi < 8; ++wi) {
                    const float scale = wi < 4 ? s0 : s1;
                    v2f f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[wi], scale, false);
                    v2f f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[wi], scale, true);
                    const float* xv = xp + ks * 64 + (wi >> 2) * 32 + (wi & 3) * 4;
                    acc += f0[0] * xv[0];
                    acc += f0[1] * xv[1];
                    acc += f1[0] * xv[2];
                    acc += f1[1] * xv[3];
                }
            }
        }
        acc += __shfl_xor(acc, 32);
        if (lane < 32) part[wave][lane] = acc;
    }
    __syncthreads();
    // 3. Per group: the K ranges added in order, the largest logit of its 32 rows (first index on ties; NaN propagates
    //    as torch.max does); then across groups the first strictly larger in top-k order.
    if (wave < G && lane < 32) {
        float v = part[wave * SPL][lane];
        for (int s2 = 1; s2 < SPL; ++s2) v += part[wave * SPL + s2][lane];
        int idx = lane;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            float ov = __shfl_xor(v, o);
            int oi = __shfl_xor(idx, o);
            bool take = (ov != ov && v == v) || (!(v != v) && (ov > v || (ov == v && oi < idx)));
            if (take) {
                v = ov;
                idx = oi;
            }
        }
        if (lane == 0) {
            const int grp = li[0][wave];
            glogit[wave] = v;
            gtoken[wave] = grp * 32 + idx;
        }
    }
    __syncthreads();
    if (tid == 0) {
        int best = -1;
        float bestv = -INFINITY;
        for (int k = 0; k < G; ++k) {
            if (glogit[k] > bestv) {
                bestv = glogit[k];
                best = gtoken[k];
            }
        }
        a.ids[r] = best;
        if (best < 0 && a.status) atomicOr(a.status, Q38_STATUS_NONFINITE);
    }
}

hipError_t q38_head_pick(const PickArgs& a, hipStream_t stream) {
    if (a.groups < 1 || a.groups > PICK_GMAX || a.H > 8192 || a.H % 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(head_pick_kernel, dim3(a.R), dim3(PICK_THREADS), 0, stream, a);
    return hipGetLastError();
}

// Greedy acceptance per row: match = leading drafts equal to the picks (at most K - 1), accepted = match + 1 for
// active rows, else 0. picks [B][K], drafts [B][K-1].
__global__ void accept_kernel(const int* picks, const int* drafts, const float* active, int B, int K, int* match,
                              int* accepted) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    int m = 0;
    while (m < K - 1 && drafts[b * (K - 1) + m] == picks[b * K + m]) ++m;
    match[b] = m;
    accepted[b] = active[b] > 0.5f ? m + 1 : 0;
}

hipError_t q38_accept(const int* picks, const int* drafts, const float* active, int B, int K, int* match, int* accepted,
                      hipStream_t stream) {
    hipLaunchKernelGGL(accept_kernel, dim3((B + 63) / 64), dim3(64), 0, stream, picks, drafts, active, B, K, match, accepted);
    return hipGetLastError();
}
