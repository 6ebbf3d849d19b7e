// Row kernels around the GEMMs: split-K finish, residual add and RMS norm, writing the next projection's e5m2
// activation tiles directly, plus the head's norms and the embedding gather.
//
// Semantics (reference qwen38_inf2/model.py):
//   rms_norm  (model.py:54-57): float32 h * rsqrt(mean(h^2) + eps) * (1 + w), rounded to bf16
//   residual  (model.py:925-930): x + bf16(linear(...)), each a bf16 op
//   MTP tail  (model.py:858-860): bf16(float(rms_norm(x, norm)) / (1 + final_norm))
//   head norm (model.py:890-895, generate.py:196): rms_norm in bf16 for the group max, in float32 for the recheck
#include "kernels.h"

// One 256-thread block per row; H <= 8192 and H % 256 == 0 (checked by the host).
__global__ __launch_bounds__(256) void residual_norm_kernel(const NormArgs a) {
    __shared__ float row[8192];
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x, H = a.H;
    float ss = 0.0f;
    for (int c = tid * 4; c < H; c += 1024) {
        float v[4];
        if (a.part) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = 0.0f;
            for (int s = 0; s < a.splits; ++s) {
                v4f p = *(const v4f*)(a.part + ((size_t)s * a.Tpad + t) * H + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] += p[e];
            }
            uint2 r = a.resid ? *(const uint2*)(a.resid + (size_t)t * H + c) : make_uint2(0, 0);
            bf16_t rb[4] = {(bf16_t)(r.x & 0xffff), (bf16_t)(r.x >> 16), (bf16_t)(r.y & 0xffff), (bf16_t)(r.y >> 16)};
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = a.resid ? rbf(bf2f(rb[e]) + rbf(v[e])) : rbf(v[e]);
        } else {
            uint2 r = *(const uint2*)(a.xin + (size_t)t * H + c);
            v[0] = bf2f(r.x & 0xffff);
            v[1] = bf2f(r.x >> 16);
            v[2] = bf2f(r.y & 0xffff);
            v[3] = bf2f(r.y >> 16);
        }
        if (a.xout)
            *(uint2*)(a.xout + (size_t)t * H + c) =
                make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16), (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            row[c + e] = v[e];
            ss += v[e] * v[e];
        }
    }
    if (!a.act && !a.hout) return;  // residual only (the last layer)
    ss = block_sum256(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)H + a.eps);
    for (int c = tid * 4; c < H; c += 1024) {
        float h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            h[e] = rbf(row[c + e] * r * (1.0f + bf2f(a.w[c + e])));
            if (a.div_w) h[e] = rbf(h[e] / (1.0f + bf2f(a.div_w[c + e])));
        }
        if (a.hout)
            *(uint2*)(a.hout + (size_t)t * H + c) =
                make_uint2((uint32_t)f2bf(h[0]) | ((uint32_t)f2bf(h[1]) << 16), (uint32_t)f2bf(h[2]) | ((uint32_t)f2bf(h[3]) << 16));
        if (a.act)
            *(uint32_t*)(a.act + act_offset(t, a.act_col0 + c, a.Kact)) =
                e5m2_byte(h[0]) | (e5m2_byte(h[1]) << 8) | (e5m2_byte(h[2]) << 16) | (e5m2_byte(h[3]) << 24);
    }
}

hipError_t q38_residual_norm(const NormArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(residual_norm_kernel, dim3(a.T), dim3(256), 0, stream, a);
    return hipGetLastError();
}

// The head's two norms of one row: bf16 (for the group max, written as bf16 activation tiles of width H) and float32
// (for the exact recheck).
__global__ __launch_bounds__(256) void head_norm_kernel(const bf16_t* hidden, const bf16_t* w, float eps, int H, bf16_t* tiles,
                                                        float* x32) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    float ss = 0.0f;
    for (int c = tid; c < H; c += 256) {
        float v = bf2f(hidden[(size_t)t * H + c]);
        ss += v * v;
    }
    ss = block_sum256(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)H + eps);
    for (int c = tid; c < H; c += 256) {
        float v = bf2f(hidden[(size_t)t * H + c]) * r * (1.0f + bf2f(w[c]));
        x32[(size_t)t * H + c] = v;
        tiles[act_offset(t, c, H)] = f2bf(v);  // bf16 tile, same element order as the e5m2 tiles
    }
}

hipError_t q38_head_norm(const bf16_t* hidden, const bf16_t* w, float eps, int H, int rows, bf16_t* tiles, float* x32,
                         hipStream_t stream) {
    hipLaunchKernelGGL(head_norm_kernel, dim3(rows), dim3(256), 0, stream, hidden, w, eps, H, tiles, x32);
    return hipGetLastError();
}

// out[i] = table[ids[i]], rows of H bf16. Ids outside [0, V) give a zero row (the host rejects them first).
__global__ __launch_bounds__(256) void embed_kernel(const int* ids, const bf16_t* table, int V, int H, bf16_t* out) {
    const int i = blockIdx.x, id = ids[i];
    for (int c = threadIdx.x * 8; c < H; c += 2048) {
        v4i v = (id >= 0 && id < V) ? *(const v4i*)(table + (size_t)id * H + c) : (v4i){0, 0, 0, 0};
        *(v4i*)(out + (size_t)i * H + c) = v;
    }
}

hipError_t q38_embed(const int* ids, int n, const bf16_t* table, int V, int H, bf16_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, stream, ids, table, V, H, out);
    return hipGetLastError();
}

// e5m2 activation tiles of bf16 rows [T][K] (the FP8 projection's input rounding, model.py:85-87, 222-225).
__global__ __launch_bounds__(256) void act_tiles_kernel(const bf16_t* x, int T, int K, uint8_t* act) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // group of 4 elements
    if (i >= (size_t)T * K / 4) return;
    const int t = (int)(i / (K / 4)), c = (int)(i % (K / 4)) * 4;
    uint2 r = *(const uint2*)(x + (size_t)t * K + c);
    *(uint32_t*)(act + act_offset(t, c, K)) = e5m2_byte(bf2f(r.x & 0xffff)) | (e5m2_byte(bf2f(r.x >> 16)) << 8) |
                                              (e5m2_byte(bf2f(r.y & 0xffff)) << 16) | (e5m2_byte(bf2f(r.y >> 16)) << 24);
}

hipError_t q38_act_tiles(const bf16_t* x, int T, int K, uint8_t* act, hipStream_t stream) {
    size_t groups = (size_t)T * K / 4;
    hipLaunchKernelGGL(act_tiles_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, stream, x, T, K, act);
    return hipGetLastError();
}
