// Projection and head GEMMs of the verify step: out[T, N] = x[T, K] . W[N, K]^T with W FP8 e4m3 and one E8M0 scale per
// 32 inputs (the reference's `FP8Linear`, qwen38_inf2/model.py:211-229; its MLP, model.py:250-259; its head,
// model.py:890-900).
//
// Weights stream from HBM as FP8 (1 byte per weight plus 1/32 byte of scale) and are widened in registers to bf16 by
// v_cvt_scalef32_pk_bf16_fp8, exactly (4 significant bits times a power of two). The products run on the bf16 MFMA,
// v_mfma_f32_32x32x16_bf16, whose float32 accumulation is as precise as a float32 dot product (measured: about 1e-8 of
// sum |x w|). The FP8 MFMA, v_mfma_scale_f32_32x32x64_f8f6f4, accumulates internally to only about 2^-14 of that sum,
// and the reference's activation rounding to e5m2 at every projection input turns such last-bit differences into
// percent-level divergence within a layer; activations are therefore e5m2-rounded values held as bf16 (exact).
//
// Operands come pre-tiled (common.h), one K-step of 64 inputs at a time; each of the four MFMAs of a K-step takes
// elements [8m, 8m + 8) of every lane's 32. A workgroup of 4 waves owns (WF*FR*32 features) x (WT*TR*32 tokens) and a
// range of K-steps; weights go straight from HBM to VGPRs, activations through double-buffered LDS. Epilogues:
//   EPI_BF16     bf16 store, columns [0, n0) to out0 and [n0, N) to out1 (e.g. in_proj_qkv | in_proj_z)
//   EPI_SWIGLU   weight tiles interleave gate/up by 32 rows; writes e5m2(bf16(silu(g)) * u) as the down
//                projection's activation tiles (the chip's fused mlp_up, kernels.py:74-118)
//   EPI_PARTIAL  float32 partial sums [split][Tpad][N] for split-K; norm.hip finishes them
//   EPI_GROUPMAX largest float32 logit of each 32-row tile per token (the head's group maxima, kernels.py:126-172)
#include "kernels.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

template <int WF, int WT, int FR, int TR, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const GemmArgs a) {
    constexpr int TT = WT * TR;       // 32-token tiles per workgroup
    constexpr int STAGE = TT * 4096;  // LDS bytes per K-step of bf16 activations
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wf = wave % WF, wt = wave / WF;
    // Block order: workgroups are dealt to the 8 XCDs round-robin, so when the feature-tile count allows, the token
    // tiles of one feature tile get ids 8 apart: same XCD, same L2, launched together, and the weight tile is read
    // from HBM once.
    const int nf = a.N / (WF * FR * 32), nt = gridDim.x / nf;
    int fb, tb;
    if (nf % 8 == 0) {
        const int lo = blockIdx.x & 7, rest = blockIdx.x >> 3;
        tb = rest % nt;
        fb = (rest / nt) * 8 + lo;
    } else {
        fb = blockIdx.x % nf;
        tb = blockIdx.x / nf;
    }
    const int ft0 = fb * (WF * FR) + wf * FR;
    const int tf0 = tb * TT;
    const int KS = a.K >> 6;
    const int ks0 = blockIdx.z * a.ksteps, nks = a.ksteps;

    v16f acc[FR][TR];
#pragma unroll
    for (int f = 0; f < FR; ++f)
#pragma unroll
        for (int t = 0; t < TR; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[f][t][i] = 0.0f;

    v4i stage_regs[TT];
    auto load_act = [&](int ks) {
#pragma unroll
        for (int r = 0; r < TT; ++r) {
            int j = tid + 256 * r, tf = j >> 8, q = j & 255;
            stage_regs[r] = *(const v4i*)((const uint8_t*)a.act + ((size_t)(tf0 + tf) * KS + ks0 + ks) * 4096 + q * 16);
        }
    };
    auto store_act = [&](int buf) {
#pragma unroll
        for (int r = 0; r < TT; ++r) {
            int j = tid + 256 * r, tf = j >> 8, q = j & 255;
            // Lane q/4 holds 64 bytes; chunk q%4 is MFMA (q%4)'s 8 elements. Chunk-major, so one MFMA's operand read
            // by a wave is 1 KiB of contiguous LDS.
            *(v4i*)(lds + buf * STAGE + tf * 4096 + (q & 3) * 1024 + (q >> 2) * 16) = stage_regs[r];
        }
    };
    // Bytes 0-15 of a lane belong to the K-step's first MX block (scale byte in lane half 0), bytes 16-31 to the
    // second (lane half 1), so each lane reads both scale words. The bytes are extracted only when used: extracting
    // them at load time would make every K-step wait for the next one's loads.
    v4i wA[FR][2], wB[FR][2];
    uint32_t sA[FR][2], sB[FR][2];
    auto load_w = [&](int ks, v4i (&wr)[FR][2], uint32_t (&sr)[FR][2]) {
        const int kabs = ks0 + ks;
#pragma unroll
        for (int f = 0; f < FR; ++f) {
            const v4i* p = (const v4i*)(a.w + ((size_t)(ft0 + f) * KS + kabs) * 2048 + lane * 32);
            wr[f][0] = p[0];
            wr[f][1] = p[1];
            const uint32_t* sw = a.ws + ((size_t)(ft0 + f) * (KS >> 2) + (kabs >> 2)) * 64 + (lane & 31);
            sr[f][0] = sw[0];
            sr[f][1] = sw[32];
        }
    };
    auto compute = [&](int ks, int buf, v4i (&wr)[FR][2], uint32_t (&sr)[FR][2]) {
        const int shift = ((ks0 + ks) & 3) * 8;
        v8bf wb[FR][4];
#pragma unroll
        for (int f = 0; f < FR; ++f) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float scale = __uint_as_float(((sr[f][m >> 1] >> shift) & 0xff) << 23);  // 2^(s - 127)
                uint32_t w0 = (uint32_t)wr[f][m >> 1][(m & 1) * 2], w1 = (uint32_t)wr[f][m >> 1][(m & 1) * 2 + 1];
                v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false);
                v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true);
                v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false);
                v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true);
                wb[f][m] = (v8bf){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
            }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                v8bf xb = *(const v8bf*)(lds + buf * STAGE + (wt * TR + t) * 4096 + m * 1024 + lane * 16);
#pragma unroll
                for (int f = 0; f < FR; ++f) acc[f][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb[f][m], xb, acc[f][t], 0, 0, 0);
            }
        }
    };

    load_act(0);
    load_w(0, wA, sA);
    store_act(0);
    __syncthreads();
    for (int ks = 0; ks < nks; ks += 2) {
        if (ks + 1 < nks) {
            load_act(ks + 1);
            load_w(ks + 1, wB, sB);
        }
        compute(ks, 0, wA, sA);
        if (ks + 1 < nks) store_act(1);
        __syncthreads();
        if (ks + 1 >= nks) break;
        if (ks + 2 < nks) {
            load_act(ks + 2);
            load_w(ks + 2, wA, sA);
        }
        compute(ks + 1, 1, wB, sB);
        if (ks + 2 < nks) store_act(0);
        __syncthreads();
    }

    // Accumulator layout of a 32x32 MFMA: lane l holds token column l % 32 and feature rows
    // 8 * (i / 4) + 4 * (l / 32) + i % 4 for i = 0..15.
    const int rowq = (lane >> 5) * 4;
#pragma unroll
    for (int t = 0; t < TR; ++t) {
        const int tok = (tf0 + wt * TR + t) * 32 + (lane & 31);
        if constexpr (EPI == EPI_BF16) {
            if (tok >= a.T) continue;
#pragma unroll
            for (int f = 0; f < FR; ++f) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    int col = (ft0 + f) * 32 + g * 8 + rowq;
                    uint32_t lo = (uint32_t)f2bf(acc[f][t][g * 4 + 0]) | ((uint32_t)f2bf(acc[f][t][g * 4 + 1]) << 16);
                    uint32_t hi = (uint32_t)f2bf(acc[f][t][g * 4 + 2]) | ((uint32_t)f2bf(acc[f][t][g * 4 + 3]) << 16);
                    bf16_t* dst = col < a.n0 ? (bf16_t*)a.out0 + (size_t)tok * a.ld0 + col
                                             : (bf16_t*)a.out1 + (size_t)tok * a.ld1 + (col - a.n0);
                    *(uint2*)dst = make_uint2(lo, hi);
                }
            }
        } else if constexpr (EPI == EPI_SWIGLU) {
            static_assert(FR == 2, "gate and up tiles pair up");
            const int inner = a.N >> 1;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float gv = rbf(acc[0][t][g * 4 + e]), uv = rbf(acc[1][t][g * 4 + e]);
                    float act = rbf(gv * rbf(sigmoidf_(gv)));
                    v[e] = e5m2_round(rbf(act * uv));
                }
                int col = (ft0 >> 1) * 32 + g * 8 + rowq;
                *(uint2*)((bf16_t*)a.out0 + act_offset(tok, col, inner)) =
                    make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16), (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16));
            }
        } else if constexpr (EPI == EPI_PARTIAL) {
            float* dst = a.part + ((size_t)blockIdx.z * a.Tpad + tok) * a.N;
#pragma unroll
            for (int f = 0; f < FR; ++f)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    int col = (ft0 + f) * 32 + g * 8 + rowq;
                    *(v4f*)(dst + col) = (v4f){acc[f][t][g * 4 + 0], acc[f][t][g * 4 + 1], acc[f][t][g * 4 + 2], acc[f][t][g * 4 + 3]};
                }
        } else {
            const int groups = a.N >> 5;
#pragma unroll
            for (int f = 0; f < FR; ++f) {
                float m = acc[f][t][0];
#pragma unroll
                for (int i = 1; i < 16; ++i) m = fmaxf(m, acc[f][t][i]);
                m = fmaxf(m, __shfl_xor(m, 32));
                if (lane < 32 && tok < a.T) a.part[(size_t)tok * groups + ft0 + f] = m;
            }
        }
    }
}

template <int WF, int WT, int FR, int TR, int EPI>
static hipError_t launch_gemm(const GemmArgs& a, int splits, hipStream_t stream) {
    dim3 grid((a.N / (WF * FR * 32)) * (a.Tpad / (WT * TR * 32)), 1, splits);
    hipLaunchKernelGGL((gemm_kernel<WF, WT, FR, TR, EPI>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

// Shapes are checked by the caller (engine.cpp): N % 256 == 0, K % 256 == 0, Tpad 32, 64 or a multiple of 128,
// (K / 64) % splits == 0.
template <int EPI>
static hipError_t gemm_dispatch(const GemmArgs& a, int splits, hipStream_t stream) {
    if (a.Tpad >= 128) return launch_gemm<2, 2, 2, 2, EPI>(a, splits, stream);
    if (a.Tpad == 64) return launch_gemm<4, 1, 2, 2, EPI>(a, splits, stream);
    return launch_gemm<4, 1, 2, 1, EPI>(a, splits, stream);
}

hipError_t q38_gemm(const GemmArgs& a, int epi, int splits, hipStream_t stream) {
    switch (epi) {
        case EPI_BF16: return gemm_dispatch<EPI_BF16>(a, splits, stream);
        case EPI_SWIGLU: return gemm_dispatch<EPI_SWIGLU>(a, splits, stream);
        case EPI_PARTIAL: return gemm_dispatch<EPI_PARTIAL>(a, splits, stream);
        default: return gemm_dispatch<EPI_GROUPMAX>(a, splits, stream);
    }
}
