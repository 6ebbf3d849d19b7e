// Projection and head GEMMs of the verify step: out[T, N] = x[T, K] . W[N, K]^T with W FP8 e4m3 and one E8M0 scale per
// 32 inputs (the reference's `FP8Linear`, qwen38_inf2/model.py:211-229; its MLP, model.py:250-259; its head,
// model.py:890-900).
//
// Numerics. Weights stream from HBM as FP8 e4m3 and are widened in registers to bf16 by v_cvt_scalef32_pk_bf16_fp8,
// exactly (4 significant bits times a power of two); or, for the checkpoint's MXFP4 projections (W4), as E2M1 nibbles
// widened by v_cvt_scalef32_pk_bf16_fp4 with the same E8M0 scales, also exactly (half the weight bytes); projection activations are e5m2 bytes (the reference rounds every
// projection input to e5m2) widened exactly by v_cvt_scalef32_pk_bf16_bf8; the head's activations are bf16. Products
// run on the bf16 MFMA, v_mfma_f32_32x32x16_bf16, whose float32 accumulation is as precise as a float32 dot product
// (measured: about 1e-8 of sum |x w|). An opt-in variant (F8, the engine's projection_mfma = FP8) feeds the tiles as
// they are to the scaled FP8 MFMA, v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 weights with their E8M0 bytes as block
// scales, e5m2 activations): no conversions and half the MFMA time, but its internal accumulation is only about
// 2^-15.5 of a 64-input block's sum |x w| (about 1e-6 of the whole sum at K = 5120), so about 1% of bf16 outputs land
// on the other neighbour of the reference's, and the reference's e5m2 rounding at every projection input amplifies
// such last-bit differences to several percent per layer. The bf16 MFMA is the default.
//
// Data movement. A workgroup owns a (WF*FR*32 features) x (WT*TR*32 tokens) output tile; for every unit of KU K-steps
// of 64 inputs, its weight tiles (2 KiB of e4m3, or 1 KiB of E2M1 in the same element order per K-step), their scales
// and its activation tiles go straight from global memory into one stage of an S-deep LDS ring (global_load_lds, no
// VGPR staging), S-1 units ahead of the MFMAs. One barrier per unit: the stage a wave loads into is the one every wave
// finished reading before that barrier. Weight and activation tiles are both
// MFMA-step-major (common.h), so every operand read is 8 (or 16) contiguous bytes per lane, free of bank conflicts.
//
// Schedule. Workgroups are persistent, one per CU. For outputs that need complete sums the (feature tile, K-step) units
// are dealt out in equal contiguous ranges (stream-K): a range that ends or starts inside a tile leaves a float32 partial
// in a slot of `fix`, and the last of the tile's contributors (an arrival counter per tile) adds the partials in K order
// and runs the epilogue. For EPI_PARTIAL the units are split per tile instead (split-K) and the partials finished by the
// next row kernel. The token blocks of one workgroup group (same K range) sit on one XCD, so each weight tile is read
// from HBM once. Epilogues:
//   EPI_BF16     bf16 store, columns [0, n0) to out0 and [n0, N) to out1 (e.g. in_proj_qkv | in_proj_z)
//   EPI_SWIGLU   weight tiles interleave gate/up by 32 rows; writes e5m2(bf16(silu(g)) * u) as the down
//                projection's activation tiles (the chip's fused mlp_up, kernels.py:74-118)
//   EPI_PARTIAL  float32 partial sums [split][Tpad][N]
//   EPI_GROUPMAX largest float32 logit of each 32-row tile per token (the head's group maxima, kernels.py:126-172)
#include "kernels.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

namespace {

// Wait until at most N vector-memory operations of this wave are outstanding, then meet the other waves. The memory
// clobber keeps the compiler from moving LDS reads across.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The same, after this wave's LDS reads have also returned: for a schedule whose reads of a stage are not all consumed
// by MFMAs before the barrier that frees the stage for loading.
template <int N>
__device__ __forceinline__ void wait_all_and_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Direct global -> LDS load of BYTES per lane: lane l's bytes come from base + voff (base wave-uniform, held in SGPRs,
// voff a 32-bit per-lane offset) and land at LDS address dst + l * BYTES (dst wave-uniform). The scalar base keeps the
// per-load address arithmetic on the scalar unit (the 256-token speculative step 21.13 against 21.46 ms with 64-bit
// per-lane addresses, A/B on one box). Issued as inline assembly, so the compiler neither waits for it before unrelated
// LDS reads (it cannot tell ring stages apart) nor counts it; the main loop's own vmcnt waits cover it, and the
// compiler's waits for its own loads only get longer. NT marks the load non-temporal. The head's weight and scale
// streams (1.31 GB, read once per launch) use it: L2 then keeps the activation tiles every workgroup rereads (the
// 256-row head's HBM reads fall from 2.2 GB to 1.43 GB per launch). So does the SwiGLU pair at 64 tokens (the decode
// step: 45.4 against 50.1 us). The other decoder projections do not: at 256 tokens it changed no GEMM's time or slowed
// it, and the attention kernel that follows them ran 55 instead of 46 us.
template <int BYTES, bool NT = false>
__device__ __forceinline__ void lds_load(const void* base, uint32_t voff, uint32_t dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(dst);
    const uint64_t b = (uint64_t)(uintptr_t)base;
    // readfirstlane returns a signed int: each word goes through uint32_t so that neither is sign-extended.
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    if constexpr (BYTES == 16 && NT)
        asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sb), "{m0}"(m0) : "memory");
    else if constexpr (BYTES == 16)
        asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb), "{m0}"(m0) : "memory");
    else if constexpr (NT)
        asm volatile("global_load_lds_dword %0, %1 nt" ::"v"(voff), "s"(sb), "{m0}"(m0) : "memory");
    else
        asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(sb), "{m0}"(m0) : "memory");
}

__device__ __forceinline__ uint32_t bits(v2bf v) { return __builtin_bit_cast(uint32_t, v); }

// 8 FP8 e4m3 weights (two words) times 2^(scale byte - 127) as one bf16 MFMA operand. The packed results are used as
// whole words: element access on them is miscompiled by this hipcc.
__device__ __forceinline__ v8bf widen_e4m3(uint32_t w0, uint32_t w1, float scale) {
    u4 r = {bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true))};
    return __builtin_bit_cast(v8bf, r);
}

// 8 e5m2 activations (two words) as one bf16 MFMA operand (exact: e5m2 is a subset of bf16).
__device__ __forceinline__ v8bf widen_e5m2(uint32_t x0, uint32_t x1) {
    u4 r = {bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(x0, 1.0f, false)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(x0, 1.0f, true)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(x1, 1.0f, false)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(x1, 1.0f, true))};
    return __builtin_bit_cast(v8bf, r);
}

// 8 E2M1 weights (one word, the first input in the lowest nibble) times 2^(scale byte - 127) as one bf16 MFMA operand.
__device__ __forceinline__ v8bf widen_e2m1(uint32_t w, float scale) {
    u4 r = {bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2)),
            bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3))};
    return __builtin_bit_cast(v8bf, r);
}

template <int WF, int WT, int FR, int TR, bool A8, int S, int EPI, bool W4, bool F8, int KU>
__global__ __launch_bounds__(WF * WT * 64, 1) void gemm_kernel(const GemmArgs a) {
    constexpr int NW = WF * WT, NTH = NW * 64;
    constexpr int TT = WT * TR, FT = WF * FR;  // 32-token and 32-feature tiles per workgroup
    constexpr int AT = A8 ? 2048 : 4096;       // bytes of one activation tile (32 tokens x 64 inputs)
    constexpr int WTB = W4 ? 1024 : 2048;      // bytes of one weight tile (32 features x 64 inputs)
    constexpr int ACT_B = TT * AT, W_B = FT * WTB, SC_B = FT * 64;
    constexpr int SUB = ACT_B + W_B + SC_B;  // one K-step of 64 inputs
    constexpr int STAGE = KU * SUB;           // a unit: KU consecutive K-steps
    constexpr int ACT_DMA = ACT_B >= NW * 1024 ? 16 : 4;  // bytes per lane of one activation load
    constexpr int W_DMA = W_B >= NW * 1024 ? 16 : 4;      // bytes per lane of one weight load
    constexpr int N_ACT = ACT_B / (NW * 64 * ACT_DMA), N_W = W_B / (NW * 64 * W_DMA), SC_CHUNKS = SC_B / 256;
    constexpr int OPS = KU * (N_ACT + N_W + 1);  // loads per wave per stage
    static_assert(N_ACT >= 1 && N_ACT * NW * 64 * ACT_DMA == ACT_B, "activation stage splits evenly over the waves");
    static_assert(N_W >= 1 && N_W * NW * 64 * W_DMA == W_B && WTB % (64 * W_DMA) == 0,
                  "weight stage splits evenly over the waves, each load inside one tile");
    static_assert(SC_CHUNKS >= 1 && NW % SC_CHUNKS == 0, "scale stage splits evenly over the waves");
    static_assert(OPS * (S - 2) <= 63 && S >= 2, "vmcnt range");
    // The pipelined schedule (bf16 MFMA, units of an even number of K-steps) waits with up to S - 1 stages in flight.
    constexpr bool PIPE = !F8 && KU % 2 == 0;
    static_assert(!PIPE || OPS * (S - 1) <= 63, "vmcnt range");
    static_assert(EPI != EPI_SWIGLU || FR % 2 == 0, "gate and up tiles pair up");
    static_assert(!F8 || (A8 && !W4), "the FP8 MFMA takes e4m3 weight tiles and e5m2 activation tiles");
    constexpr int SLOT = FR * TR * 16 * NTH;  // floats of one stream-K partial
    constexpr bool NT_W = EPI == EPI_GROUPMAX || (EPI == EPI_SWIGLU && TT == 2);  // non-temporal weight streams
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STAGE];
    __shared__ unsigned long long s_arrived;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: addresses stay in scalar registers
    const int wf = wave % WF, wt = wave / WF;
    const int KS64 = a.K >> 6, KS = KS64 / KU;  // K-steps of 64 inputs, units of KU K-steps
    const int NF = a.N / (FT * 32), NTB = a.Tpad / (TT * 32);

    // Workgroup -> (group, token block). Workgroups are dealt to the 8 XCDs round-robin, so workgroups with equal
    // blockIdx.x % 8 share an XCD and its L2; when the grid allows, the NTB token blocks of one group get ids 8 apart.
    const int groups = gridDim.x / NTB;
    int grp, tb;
    if (gridDim.x % (8 * NTB) == 0) {
        const int l = blockIdx.x >> 3;
        grp = (l / NTB) * 8 + (blockIdx.x & 7);
        tb = l % NTB;
    } else {
        grp = blockIdx.x / NTB;
        tb = blockIdx.x % NTB;
    }
    // Units are (feature tile, K-step) pairs. Split-K: group (fb, z) takes a K range of tile fb. Stream-K: the tiles
    // fb = x (mod 8) belong to XCD x, and that XCD's groups (grp = 8 gi + x, gi < groups / 8) take equal contiguous
    // ranges of its units (tile-major), so the contributors of a tile share an L2. Local unit ux is tile
    // fb = x + 8 (ux / KS), K-step ux % KS.
    const int xcd = grp & 7, gi = grp >> 3, gx = groups >> 3;
    uint32_t xcc_id;  // the XCD this workgroup actually runs on (0-7 on gfx950's 8 XCDs)
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc_id));
    const unsigned long long own_byte = 0xffull << (8 * (xcc_id & 7));
    const int Ux = ((NF - xcd + 7) >> 3) * KS;
    int u0, u1, z = 0, fstep = 8, fbase = xcd;
    if constexpr (EPI == EPI_PARTIAL) {
        const int fb = grp / a.splits;
        z = grp % a.splits;
        u0 = z * KS / a.splits;
        u1 = (z + 1) * KS / a.splits;
        fstep = 1;
        fbase = fb;
    } else {
        u0 = (int)((long)gi * Ux / gx);
        u1 = (int)((long)(gi + 1) * Ux / gx);
    }
    const int n = u1 - u0;
    if (n <= 0) return;

    // Loads of one stage. Each wave moves N_ACT activation chunks, N_W weight chunks of 64 * W_DMA bytes and one scale
    // chunk of 256 bytes (waves with the same chunk index load identical bytes to the same place).
    const uint8_t* act_base = (const uint8_t*)a.act + (size_t)tb * TT * KS64 * AT;
    const int sc_c = wave % SC_CHUNKS;
    const uint32_t sc_lane = (uint32_t)((lane >> 4) * KS64 * 64 + (lane & 15) * 4);
    const uint32_t lds_addr = (uint32_t)(uintptr_t)LDS_PTR(lds);
    auto issue = [&](int fb, int k, int st) {
#pragma unroll
        for (int j = 0; j < KU; ++j) {
            const int k64 = k * KU + j;
            const uint32_t sb = lds_addr + st * STAGE + j * SUB;
#pragma unroll
            for (int i = 0; i < N_ACT; ++i) {
                const int off = (i * NW + wave) * (64 * ACT_DMA);
                const uint8_t* g = act_base + ((size_t)(off / AT) * KS64 + k64) * AT + off % AT;
                lds_load<ACT_DMA>(g, lane * ACT_DMA, sb + off);
            }
#pragma unroll
            for (int i = 0; i < N_W; ++i) {
                const int off = (i * NW + wave) * (64 * W_DMA);
                const uint8_t* g = a.w + ((size_t)(fb * FT + off / WTB) * KS64 + k64) * WTB + off % WTB;
                lds_load<W_DMA, NT_W>(g, lane * W_DMA, sb + ACT_B + off);
            }
            const uint8_t* g = a.ws + ((size_t)(fb * FT + sc_c * 4) * KS64 + k64) * 64;
            lds_load<4, NT_W>(g, sc_lane, sb + ACT_B + W_B + sc_c * 256);
        }
    };

    v16f acc[FR][TR];
    auto zero = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < FR; ++f)
#pragma unroll
            for (int t = 0; t < TR; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[f][t][i] = 0.0f;
    };

    // One K-step with the FP8 MFMA: a weight tile's 64 inputs per lane as 32 bytes (its four 8-byte MFMA-step
    // fragments: inputs 16 (l / 32) + [0, 16) and 32 + 16 (l / 32) + [0, 16), the operand order of
    // v_mfma_scale_f32_32x32x64_f8f6f4), the lane's E8M0 byte for (row l % 32, MX block l / 32) as the weight scale, the
    // activation tile's 32 bytes the same way with scale 1 (127).
    auto compute_f8 = [&](int st, int j) __attribute__((always_inline)) {
        const uint8_t* sb = lds + st * STAGE + j * SUB;
        const uint8_t* wl = sb + ACT_B + (wf * FR) * WTB + lane * 8;
        const uint8_t* sl = sb + ACT_B + W_B + (wf * FR) * 64 + (lane & 31) * 2 + (lane >> 5);
        v8i wv[FR];
        int ws[FR];
#pragma unroll
        for (int f = 0; f < FR; ++f) {
            ws[f] = sl[f * 64];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const u2 r = *(const u2*)(wl + f * 2048 + m * 512);
                wv[f][2 * m] = (int)r[0];
                wv[f][2 * m + 1] = (int)r[1];
            }
        }
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            v8i xv;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const u2 r = *(const u2*)(sb + (wt * TR + t) * 2048 + m * 512 + lane * 8);
                xv[2 * m] = (int)r[0];
                xv[2 * m + 1] = (int)r[1];
            }
#pragma unroll
            for (int f = 0; f < FR; ++f)
                acc[f][t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wv[f], xv, acc[f][t], 0, 1, 0, ws[f], 0, 127);
        }
    };

    // One K-step: per MFMA step m, each weight fragment is 8 contiguous bytes (4 for E2M1) per lane, each activation
    // fragment 8 (16 for bf16 activations).
    auto compute_sub = [&](int st, int j) __attribute__((always_inline)) {
        if constexpr (F8) {
            compute_f8(st, j);
            return;
        }
        const uint8_t* sb = lds + st * STAGE + j * SUB;
        const uint8_t* wl = sb + ACT_B + (wf * FR) * WTB + lane * (WTB / 256);
        const uint8_t* sl = sb + ACT_B + W_B + (wf * FR) * 64 + (lane & 31) * 2;
        float scl[FR][2];  // 2^(scale byte - 127) of the K-step's two MX blocks (inputs 0-31, 32-63)
#pragma unroll
        for (int f = 0; f < FR; ++f) {
            const uint32_t sc = *(const uint16_t*)(sl + f * 64);
            scl[f][0] = __uint_as_float((sc & 0xffu) << 23);
            scl[f][1] = __uint_as_float((sc >> 8) << 23);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            v8bf wb[FR];
#pragma unroll
            for (int f = 0; f < FR; ++f) {
                // Steps 0-1 are inputs of the K-step's first MX block, steps 2-3 of its second.
                const float scale = scl[f][m >> 1];
                if constexpr (W4) {
                    wb[f] = widen_e2m1(*(const uint32_t*)(wl + f * 1024 + m * 256), scale);
                } else {
                    const u2 r = *(const u2*)(wl + f * 2048 + m * 512);
                    wb[f] = widen_e4m3(r[0], r[1], scale);
                }
            }
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                v8bf xb;
                if constexpr (A8) {
                    const u2 r = *(const u2*)(sb + (wt * TR + t) * 2048 + m * 512 + lane * 8);
                    xb = widen_e5m2(r[0], r[1]);
                } else {
                    xb = *(const v8bf*)(sb + (wt * TR + t) * 4096 + m * 1024 + lane * 16);
                }
#pragma unroll
                for (int f = 0; f < FR; ++f) acc[f][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb[f], xb, acc[f][t], 0, 0, 0);
            }
        }
    };
    auto compute = [&](int st) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < KU; ++j) compute_sub(st, j);
    };

    // The same K-step split in two for the pipelined schedule: prep reads and widens all of a K-step's operands into
    // registers, mma runs its MFMAs (in compute_sub's order, so the same sums).
    struct Ops {
        v8bf w[4][FR];
        v8bf x[4][TR];
    };
    auto prep = [&](int st, int j, Ops& o) __attribute__((always_inline)) {
        const uint8_t* sb = lds + st * STAGE + j * SUB;
        const uint8_t* wl = sb + ACT_B + (wf * FR) * WTB + lane * (WTB / 256);
        const uint8_t* sl = sb + ACT_B + W_B + (wf * FR) * 64 + (lane & 31) * 2;
#pragma unroll
        for (int f = 0; f < FR; ++f) {
            const uint32_t sc = *(const uint16_t*)(sl + f * 64);
            const float s0 = __uint_as_float((sc & 0xffu) << 23), s1 = __uint_as_float((sc >> 8) << 23);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                if constexpr (W4) {
                    o.w[m][f] = widen_e2m1(*(const uint32_t*)(wl + f * 1024 + m * 256), m < 2 ? s0 : s1);
                } else {
                    const u2 r = *(const u2*)(wl + f * 2048 + m * 512);
                    o.w[m][f] = widen_e4m3(r[0], r[1], m < 2 ? s0 : s1);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TR; ++t)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                if constexpr (A8) {
                    const u2 r = *(const u2*)(sb + (wt * TR + t) * 2048 + m * 512 + lane * 8);
                    o.x[m][t] = widen_e5m2(r[0], r[1]);
                } else {
                    o.x[m][t] = *(const v8bf*)(sb + (wt * TR + t) * 4096 + m * 1024 + lane * 16);
                }
            }
    };
    // Makes the widened operands of `o` exist at this point: keeps the compiler from sinking a prep's conversions past
    // the tile-end branch, away from the MFMAs they are meant to run beside.
    auto pin = [&](Ops& o) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int f = 0; f < FR; ++f) asm volatile("" : "+v"(o.w[m][f]));
#pragma unroll
            for (int t = 0; t < TR; ++t) asm volatile("" : "+v"(o.x[m][t]));
        }
    };
    auto mma = [&](const Ops& o) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int t = 0; t < TR; ++t)
#pragma unroll
                for (int f = 0; f < FR; ++f)
                    acc[f][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o.w[m][f], o.x[m][t], acc[f][t], 0, 0, 0);
    };

    // Accumulator layout of a 32x32 MFMA: lane l holds token column l % 32 and feature rows
    // 8 * (i / 4) + 4 * (l / 32) + i % 4 for i = 0..15.
    auto epilogue = [&](int fb) __attribute__((always_inline)) {
        const int rowq = (lane >> 5) * 4;
        const int ft0 = fb * FT + wf * FR;
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            const int tok = (tb * TT + wt * TR + t) * 32 + (lane & 31);
            if constexpr (EPI == EPI_BF16) {
                if (tok >= a.T) continue;
#pragma unroll
                for (int f = 0; f < FR; ++f) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = (ft0 + f) * 32 + g * 8 + rowq;
                        bf16_t* dst = col < a.n0 ? (bf16_t*)a.out0 + (size_t)tok * a.ld0 + col
                                                 : (bf16_t*)a.out1 + (size_t)tok * a.ld1 + (col - a.n0);
                        float v[4] = {acc[f][t][g * 4 + 0], acc[f][t][g * 4 + 1], acc[f][t][g * 4 + 2], acc[f][t][g * 4 + 3]};
                        if (a.accumulate) {  // bf16(out + bf16(sum)), the reference's sum of two bf16 products
                            const uint2 old = *(const uint2*)dst;
                            v[0] = lo_bf(old.x) + rbf(v[0]);
                            v[1] = hi_bf(old.x) + rbf(v[1]);
                            v[2] = lo_bf(old.y) + rbf(v[2]);
                            v[3] = hi_bf(old.y) + rbf(v[3]);
                        }
                        *(uint2*)dst = make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]));
                    }
                }
            } else if constexpr (EPI == EPI_SWIGLU) {
                // Feature tiles 2p and 2p + 1 are the gate and up rows of the same 32 inner features.
                const int inner = a.N >> 1;
#pragma unroll
                for (int pr = 0; pr < FR / 2; ++pr)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        float h[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float gv = rbf(acc[2 * pr][t][g * 4 + e]), uv = rbf(acc[2 * pr + 1][t][g * 4 + e]);
                            const float act = rbf(gv * rbf(sigmoidf_(gv)));
                            h[e] = rbf(act * uv);
                        }
                        const uint32_t packed = pk_e5m2(h[0], h[1], h[2], h[3]);
                        const int col = ((ft0 >> 1) + pr) * 32 + g * 8 + rowq;
                        *(uint32_t*)((uint8_t*)a.out0 + act_offset(tok, col, inner)) = packed;
                    }
            } else if constexpr (EPI == EPI_PARTIAL) {
                float* dst = a.part + ((size_t)z * a.Tpad + tok) * a.N;
#pragma unroll
                for (int f = 0; f < FR; ++f)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int col = (ft0 + f) * 32 + g * 8 + rowq;
                        *(v4f*)(dst + col) = (v4f){acc[f][t][g * 4 + 0], acc[f][t][g * 4 + 1], acc[f][t][g * 4 + 2],
                                                   acc[f][t][g * 4 + 3]};
                    }
            } else {
                const int ngroups = a.N >> 5;
#pragma unroll
                for (int f = 0; f < FR; ++f) {
                    float m = acc[f][t][0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) m = fmaxf(m, acc[f][t][i]);
                    m = fmaxf(m, __shfl_xor(m, 32));
                    if (lane < 32 && tok < a.T) a.part[(size_t)tok * ngroups + ft0 + f] = m;
                }
            }
        }
    };

    // Stream-K fixup of tile (fb, tb) from a partial range. The contributors (groups g_first..g_last of index xcd, in K
    // order) are meant to share that XCD's L2. Each arrival adds one to the byte of the tile's counter that belongs to
    // the XCD it actually runs on. A partial is plain stores (through to L2) completed before the arrival; the last
    // arrival, finding every other count in its own XCD's byte, reads the others past its L1 (sc0 buffer loads), adds
    // all partials in K order and finishes the tile. Fast path: the tile's first contributor, finding every other
    // partial already counted, adds them to its own sums without storing its own (the same additions in the same
    // order). Should contributors ever run on different XCDs, their partials may sit in another L2: the last arrival
    // then reads none of them and returns true, and finishes the tile after its own range (`recompute`).
    auto start_of = [&](int g) { return (int)((long)g * Ux / gx); };  // g: group index within the XCD
    auto group_of = [&](int u) { return (int)(((long)(u + 1) * gx - 1) / Ux); };
    auto slot_of = [&](int g, int t0) {
        return ((size_t)((g * 8 + xcd) * NTB + tb) * 2 + (start_of(g) > t0 ? 0 : 1)) * SLOT;
    };
    auto store_partial = [&](size_t slot) __attribute__((always_inline)) {
        v4f* mine = (v4f*)(a.fix + slot);
#pragma unroll
        for (int f = 0; f < FR; ++f)
#pragma unroll
            for (int t = 0; t < TR; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    mine[((f * TR + t) * 4 + q) * NTH + tid] =
                        (v4f){acc[f][t][4 * q], acc[f][t][4 * q + 1], acc[f][t][4 * q + 2], acc[f][t][4 * q + 3]};
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    // acc = partial g_first + ... + partial g_last, added in that order (from g_first + 1 when acc holds g_first's).
    auto sum_partials = [&](int t0, int g_from, int g_first, int g_last) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t fix = __builtin_amdgcn_make_buffer_rsrc(a.fix, 0, 0x7fffffff, 0x00020000);
        for (int g = g_from; g <= g_last; ++g) {
            const uint32_t base = (uint32_t)(slot_of(g, t0) * 4);
#pragma unroll
            for (int f = 0; f < FR; ++f)
#pragma unroll
                for (int t = 0; t < TR; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const v4f v = __builtin_bit_cast(
                            v4f, __builtin_amdgcn_raw_buffer_load_b128(fix, base + (((f * TR + t) * 4 + q) * NTH + tid) * 16, 0, 1));
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[f][t][4 * q + e] = g == g_first ? v[e] : acc[f][t][4 * q + e] + v[e];
                    }
        }
    };
    auto fixup = [&](int fb) __attribute__((always_inline)) -> bool {
        const int t0 = ((fb - xcd) >> 3) * KS;  // first local unit of the tile
        const int g_first = group_of(t0), g_last = group_of(t0 + KS - 1);
        unsigned long long* const counter = a.counters + fb * NTB + tb;
        auto arrivals = [](unsigned long long c) {
            int total = 0;
#pragma unroll
            for (int x = 0; x < 8; ++x) total += (int)((c >> (8 * x)) & 0xff);
            return total;
        };
        unsigned long long others = 0;  // the other contributors' arrivals
        bool fast = false;
        if (gi == g_first) {
            if (tid == 0) s_arrived = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            others = s_arrived;
            fast = arrivals(others) == g_last - g_first;
            __syncthreads();  // s_arrived is read by every thread before it is written again
        }
        if (!fast) {
            store_partial(slot_of(gi, t0));
            __syncthreads();
            if (tid == 0)
                s_arrived = __hip_atomic_fetch_add(counter, own_byte & 0x0101010101010101ull, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            others = s_arrived;
            if (arrivals(others) != g_last - g_first) return false;
        }
        if (a.recompute || (others & ~own_byte) != 0) return true;
        sum_partials(t0, fast ? g_first + 1 : g_first, g_first, g_last);
        epilogue(fb);
        if (tid == 0) __hip_atomic_store(counter, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    };

    // Finishes tile fb whose contributors did not all share this workgroup's L2, after the main loop (the ring is
    // idle): each contributor's partial again, its K-steps one at a time through stage 0 from zero sums, stored in its
    // slot here; then the partials added in K order as above. The same MFMAs and additions, so the same bits.
    auto recompute = [&](int fb) __attribute__((always_inline)) {
        const int t0 = ((fb - xcd) >> 3) * KS;
        const int g_first = group_of(t0), g_last = group_of(t0 + KS - 1);
        int st0 = 0;  // stage 0, opaque to the compiler: addresses of a constant stage would be computed at the top of
        asm volatile("" : "+s"(st0));  // the kernel and held in registers through the main loop
#pragma unroll 1
        for (int g = g_first; g <= g_last; ++g) {
            const int kb = max(start_of(g) - t0, 0), ke = min(start_of(g + 1) - t0, KS);
            zero();
#pragma unroll 1
            for (int k = kb; k < ke; ++k) {
                issue(fb, k, st0);
                wait_and_barrier<0>();
                compute(st0);
                __syncthreads();  // every wave is done with stage 0 before it is loaded again
            }
            store_partial(slot_of(g, t0));
        }
        sum_partials(t0, g_first, g_first, g_last);
        epilogue(fb);
        if (tid == 0) __hip_atomic_store(a.counters + fb * NTB + tb, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // Cursors (feature tile, K-step) of the next unit to load and of the unit being computed.
    int ifb = fbase + fstep * (u0 / KS), ik = u0 % KS;
    int cfb = ifb, ck = ik;
    bool partial_start = ik != 0;  // the current tile segment began inside the tile
    int later0 = -1, later1 = -1;  // tiles to finish by recomputation (at most the range's first and last)
    // After the last K-step of unit i: the tile's epilogue or stream-K fixup when the unit ends a tile or the range.
    auto after_unit = [&](int i) __attribute__((always_inline)) {
        if (ck == KS - 1 || i == n - 1) {
            if (EPI == EPI_PARTIAL || (!partial_start && ck == KS - 1))
                epilogue(cfb);
            else if (fixup(cfb))
                (later0 < 0 ? later0 : later1) = cfb;
            zero();
            partial_start = false;
        }
        if (++ck == KS) ck = 0, cfb += fstep;
    };
    if constexpr (PIPE) {
        // Pipelined: every stage loaded up front; each K-step's operands are read and widened while the previous
        // K-step's MFMAs run. Unit i's last K-step waits for unit i + 1's stage (and the barrier after which every
        // wave has read all of unit i), refills unit i's stage with unit i + S, and preps unit i + 1's first K-step
        // beside its own MFMAs. KU is even, so K-step j of every unit uses operand set j % 2. The loop body has no
        // branch but the tile ends, so that the preps and MFMAs schedule together: past the range's last unit the
        // loads repeat that unit into stages no longer read (S - 1 extra units per range, from L2) and the last prep
        // reads a stage it never uses; every load has landed before the workgroup leaves its LDS.
        Ops ops[2];
#pragma unroll
        for (int i = 0; i < S; ++i) {
            issue(ifb, ik, i);
            if (i + 1 < n && ++ik == KS) ik = 0, ifb += fstep;
        }
        zero();
        wait_all_and_barrier<OPS*(S - 1)>();
        prep(0, 0, ops[0]);
        int st = 0;
        for (int i = 0; i < n; ++i) {
            const int nst = st + 1 == S ? 0 : st + 1;
#pragma unroll
            for (int j = 0; j < KU; ++j) {
                if (j + 1 < KU) {
                    prep(st, j + 1, ops[(j + 1) & 1]);
                    mma(ops[j & 1]);
                    pin(ops[(j + 1) & 1]);
                } else {
                    wait_all_and_barrier<OPS*(S - 2)>();  // loads issued after unit i + 1's: units i + 2 .. i + S - 1
                    issue(ifb, ik, st);                   // unit i + S, or the range's last unit again
                    // The cursor moves on while units remain (selects, not a branch).
                    const int nk = ik + (i + S + 1 < n ? 1 : 0);
                    ifb += nk == KS ? fstep : 0;
                    ik = nk == KS ? 0 : nk;
                    prep(nst, 0, ops[0]);
                    mma(ops[j & 1]);
                    pin(ops[0]);
                }
            }
            st = nst;
            after_unit(i);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
#pragma unroll
        for (int i = 0; i < S - 1; ++i)
            if (i < n) {
                issue(ifb, ik, i);
                if (++ik == KS) ik = 0, ifb += fstep;
            }
        zero();
        int st = 0, ist = S - 1;  // stage computed now, stage loaded next
        for (int i = 0; i < n; ++i) {
            if (i + S - 2 < n)
                wait_and_barrier<OPS*(S - 2)>();
            else
                wait_and_barrier<0>();
            if (i + S - 1 < n) {
                issue(ifb, ik, ist);
                if (++ik == KS) ik = 0, ifb += fstep;
                if (++ist == S) ist = 0;
            }
            compute(st);
            if (++st == S) st = 0;
            after_unit(i);
        }
    }
    if constexpr (EPI != EPI_PARTIAL) {
        if (later0 >= 0) {
            wait_all_and_barrier<0>();  // every wave is done with the ring
#pragma unroll 1
            for (int d = 0; d < 2; ++d) {
                const int fb = d ? later1 : later0;
                if (fb >= 0) recompute(fb);
            }
        }
    }
}

constexpr int MIN_UNITS = 8;  // smallest K range worth a stream-K group

template <int WF, int WT, int FR, int TR, bool A8, int S, int EPI, bool W4, bool F8, int KU = 1>
hipError_t launch(const GemmArgs& a0, int* splits_out, hipStream_t stream) {
    GemmArgs a = a0;
    constexpr int BF = WF * FR * 32, BT = WT * TR * 32, NTH = WF * WT * 64;
    if (a.N % BF || a.Tpad % BT || a.K % 64 || a.cus < 1) return hipErrorInvalidValue;
    if (a.K % (64 * KU)) return hipErrorInvalidValue;
    const int NF = a.N / BF, NTB = a.Tpad / BT, KS = a.K / (64 * KU);
    int grid;
    if (EPI == EPI_PARTIAL) {
        int s = a.cus / (NF * NTB);
        if (s < 1) {
            // More tiles than CUs (prefill widths): the split count whose rounds of workgroups come out fullest, as
            // K-steps per CU = ceil(tiles * s / cus) * KS / s (320 tiles on 256 CUs: 4 splits, 5 full rounds, instead
            // of 1 split in 1.25 rounds); ties to fewer splits (less partial traffic).
            const long tiles = (long)NF * NTB;
            const int most = a.splits_max > 0 ? a.splits_max : 1;
            s = 1;
            double best = (double)((tiles + a.cus - 1) / a.cus);
            for (int c = 2; c <= most && c <= 4 && c <= KS; ++c) {
                const double cost = (double)((tiles * c + a.cus - 1) / a.cus) / c;
                if (cost < best * 0.97) best = cost, s = c;
            }
        }
        s = s > GEMM_SPLIT_MAX ? GEMM_SPLIT_MAX : s;
        s = s > KS ? KS : s;
        if (a.splits_max > 0 && s > a.splits_max) s = a.splits_max;
        a.splits = s;
        grid = NF * NTB * s;
    } else {
        if ((size_t)NF * NTB > (size_t)a.counters_n) return hipErrorInvalidValue;
        // Groups: a multiple of 8 (an equal share per XCD), at most one workgroup per CU.
        long groups = (long)NF * KS / MIN_UNITS;
        const long most = a.cus / NTB;
        if (most < 8) return hipErrorInvalidValue;
        groups = groups > most ? most : groups;
        groups = groups < 8 ? 8 : groups - groups % 8;
        grid = (int)groups * NTB;
        if ((size_t)2 * grid * FR * TR * 16 * NTH > a.fix_floats) return hipErrorInvalidValue;
        a.splits = 1;
    }
    if (splits_out) *splits_out = a.splits;
    hipLaunchKernelGGL((gemm_kernel<WF, WT, FR, TR, A8, S, EPI, W4, F8, KU>), dim3(grid), dim3(NTH), 0, stream, a);
    return hipGetLastError();
}

// Tile shape: 256 tokens per workgroup from 256 tokens up (128 for bf16 outputs), Tpad tokens below. Features per workgroup: with e5m2
// activations 128 when N / 128 is a multiple of 8 (an equal share of tiles per XCD; as fast per tile as 256 and twice
// the tiles), else 256; with bf16 activations (the head) 256, and 512 below 256 tokens when N allows.
template <bool A8, int EPI, bool W4, bool F8>
hipError_t dispatch(const GemmArgs& a, int* splits_out, hipStream_t stream) {
    auto balanced = [&](int bf) { return a.N % bf == 0 && (a.N / bf) % 8 == 0; };
    if (a.Tpad % 256 == 0) {
        if constexpr (A8) {
            // bf16 outputs: 128 x 128 tiles, two token blocks per weight tile on one XCD (their stream-K ranges split
            // fewer tiles; measured 4-8 % faster on the 16384- and 14336-wide projections than 128 x 256). Units of
            // two K-steps (128 inputs) per ring stage when K allows: half the barriers and waits per MFMA, measured
            // 6-8 % faster on every projection of the 27B verify step than one K-step per stage with deeper rings.
            if (a.K % 128 == 0) {
                if (EPI == EPI_BF16 && balanced(128)) return launch<2, 4, 2, 1, true, 3, EPI, W4, F8, 2>(a, splits_out, stream);
                if (balanced(128) || (a.N % 256 && a.N % 128 == 0))
                    return launch<2, 4, 2, 2, true, 3, EPI, W4, F8, 2>(a, splits_out, stream);
            }
            if (EPI == EPI_BF16 && balanced(128)) return launch<2, 4, 2, 1, true, 9, EPI, W4, F8>(a, splits_out, stream);
            if (balanced(128) || (a.N % 256 && a.N % 128 == 0)) return launch<2, 4, 2, 2, true, 6, EPI, W4, F8>(a, splits_out, stream);
            return launch<4, 2, 2, 4, true, 4, EPI, W4, F8>(a, splits_out, stream);
        } else {
            return launch<4, 2, 2, 4, false, 3, EPI, W4, F8>(a, splits_out, stream);
        }
    }
    const bool wide = a.N % 512 == 0 && (balanced(512) || !balanced(256));
    switch (a.Tpad) {
        case 128:
            return wide ? launch<8, 1, 2, 4, A8, 3, EPI, W4, F8>(a, splits_out, stream)
                        : launch<4, 2, 2, 2, A8, 3, EPI, W4, F8>(a, splits_out, stream);
        case 64:
            // Measured per epilogue at 64 tokens (the decode step's projections): bf16 outputs fastest as 128 x 64
            // tiles with a deep ring (qkvz 32 against 50 us as 512 x 64), split-K partials as 128 x 64 with 5 stages,
            // the SwiGLU pair as 256 x 64 (50.9 against 56.4 us as 128 x 64).
            if constexpr (A8) {
                if (EPI == EPI_BF16 && balanced(128)) return launch<2, 2, 2, 1, true, 8, EPI, W4, F8>(a, splits_out, stream);
                if (EPI == EPI_PARTIAL && balanced(128)) return launch<2, 2, 2, 1, true, 5, EPI, W4, F8>(a, splits_out, stream);
                if (!balanced(512) && !balanced(256) && balanced(128)) return launch<2, 2, 2, 1, true, 5, EPI, W4, F8>(a, splits_out, stream);
            }
            // bf16 activations at 64 tokens (the draft heads' group maxima): 512 x 64 tiles, 64 x 64 per wave, when N
            // allows (248.3 against 261.5 us as 256 x 64 with 64 x 32 per wave, per 1.31 GB launch).
            if constexpr (!A8) {
                if (a.N % 512 == 0) return launch<8, 1, 2, 2, false, 3, EPI, W4, F8>(a, splits_out, stream);
                return launch<4, 2, 2, 1, false, 6, EPI, W4, F8>(a, splits_out, stream);
            }
            return wide ? launch<8, 1, 2, 2, A8, (A8 ? 4 : 3), EPI, W4, F8>(a, splits_out, stream)
                        : launch<4, 2, 2, 1, A8, 4, EPI, W4, F8>(a, splits_out, stream);
        case 32:
            return wide ? launch<8, 1, 2, 1, A8, 4, EPI, W4, F8>(a, splits_out, stream)
                        : launch<4, 1, 2, 1, A8, 4, EPI, W4, F8>(a, splits_out, stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t q38_gemm(const GemmArgs& a, int epi, int* splits_out, hipStream_t stream) {
    if (a.w4 && a.bf16_act) {
        // bf16 activation tiles against MXFP4 weights (the reference's FP4Linear numerics, one plane per launch)
        if (epi != EPI_BF16) return hipErrorInvalidValue;
        return dispatch<false, EPI_BF16, true, false>(a, splits_out, stream);
    }
    if (a.w4) {
        switch (epi) {
            case EPI_BF16: return dispatch<true, EPI_BF16, true, false>(a, splits_out, stream);
            case EPI_SWIGLU: return dispatch<true, EPI_SWIGLU, true, false>(a, splits_out, stream);
            case EPI_PARTIAL: return dispatch<true, EPI_PARTIAL, true, false>(a, splits_out, stream);
            default: return hipErrorInvalidValue;  // the head's weights are e4m3
        }
    }
    if (a.f8) {
        switch (epi) {
            case EPI_BF16: return dispatch<true, EPI_BF16, false, true>(a, splits_out, stream);
            case EPI_SWIGLU: return dispatch<true, EPI_SWIGLU, false, true>(a, splits_out, stream);
            case EPI_PARTIAL: return dispatch<true, EPI_PARTIAL, false, true>(a, splits_out, stream);
            default: break;  // the head's activations are bf16: the bf16 MFMA below
        }
    }
    switch (epi) {
        case EPI_BF16: return dispatch<true, EPI_BF16, false, false>(a, splits_out, stream);
        case EPI_SWIGLU: return dispatch<true, EPI_SWIGLU, false, false>(a, splits_out, stream);
        case EPI_PARTIAL: return dispatch<true, EPI_PARTIAL, false, false>(a, splits_out, stream);
        case EPI_GROUPMAX: return dispatch<false, EPI_GROUPMAX, false, false>(a, splits_out, stream);
        default: return hipErrorInvalidValue;
    }
}
