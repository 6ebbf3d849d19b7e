// Device helpers shared by every kernel of the verify path (gfx950 / CDNA4).
//
// Number formats and rounding follow the reference's CPU path (qwen38_inf2/model.py), which runs torch CPU ops in
// bf16: every bf16 result is fp32 rounded to nearest even, and activations are rounded to FP8 e5m2 at each
// projection input (model.py:85-87, 222-225).
//
// Tiles. Every GEMM reads its operands in the layout the MFMA wants, written that way by the kernel that produced
// them. One K-step of 64 inputs for 32 tokens (or 32 weight rows) is one tile; lane l holds 32 elements of token
// (row) l % 32 from lane half h = l / 32:
//     element i of lane half h  <->  input k = 32 * (i / 16) + 16 * h + i % 16  (within the K-step)
// and MFMA m (v_mfma_f32_32x32x16_bf16, 16 inputs) of the K-step takes elements [8m, 8m + 8) of every lane, so
// elements 0-15 are the K-step's first 32-input MX block and 16-31 its second. Weight tiles are FP8 e4m3 bytes, lane
// by lane (2 KiB, pack.hip), with their E8M0 scales as [row][block] bytes per tile (64 bytes). Activation tiles are
// stored MFMA-step-major, [m][lane][8], so that each MFMA's operand is one contiguous run: e5m2 bytes (2 KiB) for the
// projections, bf16 (4 KiB) for the head.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));

#define Q38_HOST_DEVICE __host__ __device__ __forceinline__

// A __shared__ object as an LDS address (its 32-bit value is the LDS byte offset the direct global -> LDS copies take).
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// The bf16 in the low / high half of a word, widened.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (c10::BFloat16's rounding; v_cvt_pk_bf16_f32); NaN stays NaN.
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Two floats rounded to bf16 and packed, a in the low half (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    const v2bf p = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, p);
}

// Round to bf16 and back: the value a torch bf16 op stores.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// 1 / (1 + e^-x) with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of a correctly rounded division.
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + expf(-x)); }

// torch.nn.functional.softplus with beta 1, threshold 20.
__device__ __forceinline__ float softplusf_(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Position of input k (0..63) within a K-step: lane half and byte (element for bf16 tiles).
Q38_HOST_DEVICE int kstep_half(int k) { return (k & 31) >> 4; }
Q38_HOST_DEVICE int kstep_byte(int k) { return ((k & 63) >> 5) * 16 + (k & 15); }

// Element offset of (token t, input k) in activation tiles with K inputs (K a multiple of 64): tile (t / 32, k / 64)
// of 2048 elements as [m][lane][8] with lane = t % 32 + 32 * kstep_half(k), element e = kstep_byte(k), m = e / 8.
// Four consecutive k from a multiple of 4 are contiguous.
Q38_HOST_DEVICE size_t act_offset(int t, int k, int K) {
    const int e = kstep_byte(k);
    return ((size_t)(t >> 5) * (K >> 6) + (k >> 6)) * 2048 +
           (size_t)((e >> 3) * 512 + ((t & 31) + kstep_half(k) * 32) * 8 + (e & 7));
}

// FP8 e5m2 bytes of floats rounded as torch's cast to float8_e5m2 does (round to nearest even, past 57344 to
// infinity; NaN stays NaN): v_cvt_pk_bf8_f32, which agrees with that rounding bit for bit on every bf16 value (all
// values converted here are bf16) and on random float32 values, NaN payloads aside.
__device__ __forceinline__ uint32_t e5m2_byte(float x) { return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(x, x, 0, false) & 0xffu; }

// Four e5m2 bytes packed into a word, a in the lowest byte.
__device__ __forceinline__ uint32_t pk_e5m2(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(c, d, lo, true);
}

// FP8 KV cache: e4m3 bytes of value / scale with one bf16 scale per layer and K or V (reference model.py:579-593).
// The cache byte of x: e4m3 (round to nearest even) of float32(x) / float32(scale), clamped to +-240 first.
__device__ __forceinline__ uint32_t kv_code(float x, float scale) {
    const float q = fminf(fmaxf(__fdiv_rn(x, scale), -240.0f), 240.0f);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q, q, 0, false) & 0xffu;
}

// Two cached bytes (the low or high half of `word`) read back as bf16 (e4m3 value x scale), packed: the e4m3 x bf16
// product is exact in float32 (4 x 8 significant bits), then rounded once to bf16.
template <bool HIGH>
__device__ __forceinline__ uint32_t kv_pk2(uint32_t word, float scale) {
    typedef float v2f_ __attribute__((ext_vector_type(2)));
    const v2f_ f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, 1.0f, HIGH);
    return pk_bf16(f[0] * scale, f[1] * scale);
}

// Eight cached bytes as one bf16 MFMA operand.
__device__ __forceinline__ v8bf16 kv_widen8(uint32_t lo, uint32_t hi, float scale) {
    typedef uint32_t u4_ __attribute__((ext_vector_type(4)));
    const u4_ r = {kv_pk2<false>(lo, scale), kv_pk2<true>(lo, scale), kv_pk2<false>(hi, scale), kv_pk2<true>(hi, scale)};
    return __builtin_bit_cast(v8bf16, r);
}

// x as a later step reads it back from the cache. Encoding the result again gives kv_code(x) (the bf16 rounding moves
// a value by at most 2^-9 relative, e4m3's rounding boundaries lie at least 2^-5 away), so kernels keep only this.
__device__ __forceinline__ float kv_round_trip(float x, float scale) {
    return lo_bf(kv_pk2<false>(kv_code(x, scale), scale));
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Sum over each aligned group of 8 (16) lanes with DPP moves (lane ^ 1, lane ^ 2, then the mirrored half row and row);
// every lane of a group ends with the same total, the same additions in the same order.
__device__ __forceinline__ float group8_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    return v;
}
__device__ __forceinline__ float group16_sum(float v) {
    v = group8_sum(v);
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
}

__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Sum over a 256-thread block; `red` is 4 floats of shared memory. Every thread gets the total.
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = warp_sum(v);
    int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
