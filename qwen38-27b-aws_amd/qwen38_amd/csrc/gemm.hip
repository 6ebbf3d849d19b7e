// Projection GEMMs of the verify step: out[T, N] = e5m2(x)[T, K] . W[N, K]^T, W FP8 e4m3 with one E8M0 scale per 32
// inputs (the reference's `FP8Linear`, qwen38_inf2/model.py:211-229, and the chip's `fp8_linear`, kernels.py:25-71).
//
// One gfx950 scaled MFMA, v_mfma_scale_f32_32x32x64_f8f6f4, multiplies a 32-feature x 64-input weight fragment (e4m3,
// per-lane E8M0 scale) by a 64-input x 32-token activation fragment (e5m2, unit scale) into 32x32 fp32 accumulators.
// Operands arrive pre-tiled (common.h): a lane's 32 bytes are one MX block, so each fragment is a 2 KiB contiguous
// load and the scale byte is the lane's own.
//
// Work split: a workgroup of 4 waves owns (WF*FR*32 features) x (WT*TR*32 tokens) and a range of K-steps. Weights go
// from HBM straight into VGPRs (each weight byte is fetched by WT waves, WT <= 2); activations are staged through LDS
// two K-steps at a time, double buffered, and read by the WF waves that share them. Epilogues:
//   EPI_BF16    bf16 store, columns [0, n0) to out0 and [n0, N) to out1 (e.g. in_proj_qkv | in_proj_z)
//   EPI_SWIGLU  weight tiles interleave gate/up by 32 rows; writes e5m2(bf16(silu(g)) * u) as the down projection's
//               activation tiles (the MLP's `down(silu(gate(x)) * up(x))`, model.py:250-259, chip mlp_up kernels.py:74-118)
//   EPI_PARTIAL fp32 partial sums [split][Tpad][N] for split-K; reduce.hip finishes them.
#include "kernels.h"

template <int WF, int WT, int FR, int TR, int EPI>
__global__ __launch_bounds__(256) void gemm_fp8_kernel(const GemmArgs a) {
    constexpr int TT = WT * TR;             // 32-token tiles per workgroup
    constexpr int STAGE = TT * 2 * 2048;    // LDS bytes per stage of 2 K-steps
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wf = wave % WF, wt = wave / WF;
    const int ft0 = blockIdx.x * (WF * FR) + wf * FR;
    const int tf0 = blockIdx.y * TT;
    const int KS = a.K >> 6;
    const int ks0 = blockIdx.z * a.ksteps;
    const int nstages = a.ksteps >> 1;

    v16f acc[FR][TR];
#pragma unroll
    for (int f = 0; f < FR; ++f)
#pragma unroll
        for (int t = 0; t < TR; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[f][t][i] = 0.0f;

    const uint8_t* wbase[FR];
    const uint32_t* sbase[FR];
#pragma unroll
    for (int f = 0; f < FR; ++f) {
        wbase[f] = a.w + ((size_t)(ft0 + f) * KS + ks0) * 2048 + lane * 32;
        sbase[f] = a.ws + (size_t)(ft0 + f) * (KS >> 2) * 64 + lane;
    }

    v4i stage_regs[TT];
    auto load_act = [&](int s) {
#pragma unroll
        for (int r = 0; r < TT; ++r) {
            int j = tid + 256 * r, blk = j >> 7, q = j & 127;
            const uint8_t* src = a.act + ((size_t)(tf0 + (blk >> 1)) * KS + ks0 + 2 * s + (blk & 1)) * 2048 + q * 16;
            stage_regs[r] = *(const v4i*)src;
        }
    };
    auto store_act = [&](int buf) {
#pragma unroll
        for (int r = 0; r < TT; ++r) {
            int j = tid + 256 * r, blk = j >> 7, q = j & 127;
            *(v4i*)(lds + buf * STAGE + blk * 2048 + (q & 1) * 1024 + (q >> 1) * 16) = stage_regs[r];
        }
    };

    v8i wA[FR][2], wB[FR][2];
    uint32_t sA[FR], sB[FR];
    auto load_w = [&](int s, v8i (&wr)[FR][2], uint32_t (&sr)[FR]) {
#pragma unroll
        for (int f = 0; f < FR; ++f) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const v4i* p = (const v4i*)(wbase[f] + (size_t)(2 * s + kk) * 2048);
                v4i lo = p[0], hi = p[1];
                wr[f][kk] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            int kabs = ks0 + 2 * s;
            sr[f] = sbase[f][(size_t)(kabs >> 2) * 64] >> ((kabs & 2) * 8);
        }
    };
    auto compute = [&](int buf, v8i (&wr)[FR][2], uint32_t (&sr)[FR]) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            v8i af[TR];
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                const uint8_t* p = lds + buf * STAGE + ((wt * TR + t) * 2 + kk) * 2048 + lane * 16;
                v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 1024);
                af[t] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int f = 0; f < FR; ++f) {
                int sc = (sr[f] >> (8 * kk)) & 0xff;
#pragma unroll
                for (int t = 0; t < TR; ++t)
                    acc[f][t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wr[f][kk], af[t], acc[f][t], 0, 1, 0, sc, 0,
                                                                               a.unit_scale);
            }
        }
    };

    load_act(0);
    load_w(0, wA, sA);
    store_act(0);
    __syncthreads();
    for (int s = 0; s < nstages; s += 2) {
        if (s + 1 < nstages) {
            load_act(s + 1);
            load_w(s + 1, wB, sB);
        }
        compute(0, wA, sA);
        if (s + 1 < nstages) store_act(1);
        __syncthreads();
        if (s + 1 >= nstages) break;
        if (s + 2 < nstages) {
            load_act(s + 2);
            load_w(s + 2, wA, sA);
        }
        compute(1, wB, sB);
        if (s + 2 < nstages) store_act(0);
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
                uint32_t word = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float gv = rbf(acc[0][t][g * 4 + e]), uv = rbf(acc[1][t][g * 4 + e]);
                    float act = rbf(gv * rbf(sigmoidf_(gv)));
                    word |= f2e5m2(rbf(act * uv)) << (8 * e);
                }
                int col = (ft0 >> 1) * 32 + g * 8 + rowq;
                *(uint32_t*)((uint8_t*)a.out0 + act_offset(tok, col, inner)) = word;
            }
        } else {
            float* dst = a.part + ((size_t)blockIdx.z * a.Tpad + tok) * a.N;
#pragma unroll
            for (int f = 0; f < FR; ++f)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    int col = (ft0 + f) * 32 + g * 8 + rowq;
                    *(v4f*)(dst + col) = (v4f){acc[f][t][g * 4 + 0], acc[f][t][g * 4 + 1], acc[f][t][g * 4 + 2], acc[f][t][g * 4 + 3]};
                }
        }
    }
}

// ------------------------------------------------------------------------------------------------ lm_head group max
//
// `HeadStep.forward` (model.py:890-900) on the CPU path: logits = float(x_bf16) . dequant(W)^T in fp32, then the largest
// logit of each group of 32 vocabulary rows (the chip's `lm_head_group_maxima`, kernels.py:126-172). x here is bf16
// (the CPU path does not round it to e5m2), so this is a bf16 MFMA, v_mfma_f32_32x32x16_bf16, with the e4m3 weights
// widened to bf16 in registers by v_cvt_scalef32_pk_bf16_fp8 (exact: 4 significant bits times a power of two).
// One 32x32 accumulator tile is one vocabulary group for 32 rows, so the epilogue is a max over 16 registers and one
// swap of lane halves.
//
// bf16 activation tiles: [Rpad/32][K/64][64 lanes][32 bf16], lane (r % 32) + 32 * ((k % 64) / 32), element k % 32.
// The four MFMAs of a K-step take elements [8m, 8m+8) of each lane's 32, in weights and activations alike.

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

template <int WF, int WT, int FR, int TR>
__global__ __launch_bounds__(256) void head_groupmax_kernel(const HeadArgs a) {
    constexpr int TT = WT * TR;
    constexpr int STAGE = TT * 4096;        // one K-step of bf16 activations
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wf = wave % WF, wt = wave / WF;
    const int ft0 = blockIdx.x * (WF * FR) + wf * FR;
    const int tf0 = blockIdx.y * TT;
    const int KS = a.K >> 6;

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
            stage_regs[r] = *(const v4i*)((const uint8_t*)a.act + ((size_t)(tf0 + tf) * KS + ks) * 4096 + q * 16);
        }
    };
    auto store_act = [&](int buf) {
#pragma unroll
        for (int r = 0; r < TT; ++r) {
            int j = tid + 256 * r, tf = j >> 8, q = j & 255;
            // lane (q / 4) holds 64 bytes; chunk c = q % 4 is MFMA c's 8 elements. Store chunk-major so a wave's read
            // of one chunk is 1 KiB contiguous.
            *(v4i*)(lds + buf * STAGE + tf * 4096 + (q & 3) * 1024 + (q >> 2) * 16) = stage_regs[r];
        }
    };
    // Bytes 0-15 of a lane belong to the K-step's first MX block (scale held by lane half 0), bytes 16-31 to the
    // second (lane half 1): each lane reads both scale bytes.
    v4i wA[FR][2], wB[FR][2];
    uint32_t sA[FR][2], sB[FR][2];
    auto load_w = [&](int ks, v4i (&wr)[FR][2], uint32_t (&sr)[FR][2]) {
#pragma unroll
        for (int f = 0; f < FR; ++f) {
            const v4i* p = (const v4i*)(a.w + ((size_t)(ft0 + f) * KS + ks) * 2048 + lane * 32);
            wr[f][0] = p[0];
            wr[f][1] = p[1];
            const uint32_t* sw = a.ws + ((size_t)(ft0 + f) * (KS >> 2) + (ks >> 2)) * 64 + (lane & 31);
            sr[f][0] = (sw[0] >> ((ks & 3) * 8)) & 0xff;
            sr[f][1] = (sw[32] >> ((ks & 3) * 8)) & 0xff;
        }
    };
    auto compute = [&](int buf, v4i (&wr)[FR][2], uint32_t (&sr)[FR][2]) {
        v8bf wb[FR][4];
#pragma unroll
        for (int f = 0; f < FR; ++f) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float scale = __uint_as_float(sr[f][m >> 1] << 23);  // 2^(s - 127)
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
    for (int ks = 0; ks < KS; ks += 2) {
        if (ks + 1 < KS) {
            load_act(ks + 1);
            load_w(ks + 1, wB, sB);
        }
        compute(0, wA, sA);
        if (ks + 1 < KS) store_act(1);
        __syncthreads();
        if (ks + 1 >= KS) break;
        if (ks + 2 < KS) {
            load_act(ks + 2);
            load_w(ks + 2, wA, sA);
        }
        compute(1, wB, sB);
        if (ks + 2 < KS) store_act(0);
        __syncthreads();
    }

    const int groups = a.V >> 5;
#pragma unroll
    for (int t = 0; t < TR; ++t) {
        const int row = (tf0 + wt * TR + t) * 32 + (lane & 31);
#pragma unroll
        for (int f = 0; f < FR; ++f) {
            float m = acc[f][t][0];
#pragma unroll
            for (int i = 1; i < 16; ++i) m = fmaxf(m, acc[f][t][i]);
            m = fmaxf(m, __shfl_xor(m, 32));
            if (lane < 32 && row < a.R) a.maxima[(size_t)row * groups + ft0 + f] = m;
        }
    }
}

// ------------------------------------------------------------------------------------------------ launchers

static int ceil_div(int a, int b) { return (a + b - 1) / b; }

template <int WF, int WT, int FR, int TR, int EPI>
static hipError_t launch_gemm(const GemmArgs& a, int splits, hipStream_t stream) {
    dim3 grid(a.N / (WF * FR * 32), a.Tpad / (WT * TR * 32), splits);
    hipLaunchKernelGGL((gemm_fp8_kernel<WF, WT, FR, TR, EPI>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

// Shapes are checked by the caller (engine.cpp, q38_gemm_check): N % 256 == 0, K % 256 == 0, Tpad a power of two
// multiple of 32 (or of 256 above 256), (K / 64) % splits == 0 and (K / 64 / splits) even.
template <int EPI>
static hipError_t gemm_dispatch(const GemmArgs& a, int splits, hipStream_t stream) {
    if (a.Tpad >= 256) return launch_gemm<2, 2, 2, 4, EPI>(a, splits, stream);
    if (a.Tpad == 128) return launch_gemm<4, 1, 2, 4, EPI>(a, splits, stream);
    if (a.Tpad == 64) return launch_gemm<4, 1, 2, 2, EPI>(a, splits, stream);
    return launch_gemm<4, 1, 2, 1, EPI>(a, splits, stream);
}

hipError_t q38_gemm_fp8(const GemmArgs& a, int epi, int splits, hipStream_t stream) {
    switch (epi) {
        case EPI_BF16: return gemm_dispatch<EPI_BF16>(a, splits, stream);
        case EPI_SWIGLU: return gemm_dispatch<EPI_SWIGLU>(a, splits, stream);
        default: return gemm_dispatch<EPI_PARTIAL>(a, splits, stream);
    }
}

hipError_t q38_head_groupmax(const HeadArgs& a, hipStream_t stream) {
    if (a.Rpad >= 256) {
        dim3 grid(a.V / 128, a.Rpad / 256);
        hipLaunchKernelGGL((head_groupmax_kernel<2, 2, 2, 4>), grid, dim3(256), 0, stream, a);
    } else if (a.Rpad == 128) {
        dim3 grid(a.V / 256, 1);
        hipLaunchKernelGGL((head_groupmax_kernel<4, 1, 2, 4>), grid, dim3(256), 0, stream, a);
    } else if (a.Rpad == 64) {
        dim3 grid(a.V / 256, 1);
        hipLaunchKernelGGL((head_groupmax_kernel<4, 1, 2, 2>), grid, dim3(256), 0, stream, a);
    } else {
        dim3 grid(a.V / 256, 1);
        hipLaunchKernelGGL((head_groupmax_kernel<4, 1, 2, 1>), grid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}
