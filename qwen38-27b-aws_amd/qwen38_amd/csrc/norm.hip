// Row kernels around the GEMMs: split-K finish, residual add and RMS norm, writing the next projection's e5m2
// activation tiles directly, plus the head's norms and the embedding gather.
//
// Semantics (reference qwen38_inf2/model.py):
//   rms_norm  (model.py:54-57): float32 h * rsqrt(mean(h^2) + eps) * (1 + w), rounded to bf16
//   residual  (model.py:925-930): x + bf16(linear(...)), each a bf16 op
//   MTP tail  (model.py:858-860): bf16(float(rms_norm(x, norm)) / (1 + final_norm))
//   head norm (model.py:890-895, generate.py:196): rms_norm in bf16 for the group max, in float32 for the recheck
#include "kernels.h"

// One workgroup of max(64, H / 8) threads per row (H <= 8192, H % 256 == 0, checked by the host); thread tid owns
// columns 8 tid + [0, 8): 32 contiguous bytes of each split's partials, 16 of the residual, and its e5m2 activation
// bytes are one 8-byte store (8 consecutive inputs of one tile lane). All of a thread's global loads (every split's
// partials, the residual, the norm weights) are issued before any arithmetic or store: the partials come from HBM,
// and a CU reaches its share of HBM bandwidth only with its whole working set in flight.
__global__ __launch_bounds__(1024) void residual_norm_kernel(const NormArgs a) {
    __shared__ float red[16];
    const int t = blockIdx.x, tid = threadIdx.x, H = a.H;
    const bool on = tid * 8 < H;
    const int c0 = tid * 8;
    v4f p[GEMM_SPLIT_MAX][2];
    uint4 rr = make_uint4(0, 0, 0, 0), ww = rr, dd = rr;
    if (on) {
        if (!a.part)
            rr = *(const uint4*)(a.xin + (size_t)t * H + c0);
        else if (a.resid)
            rr = *(const uint4*)(a.resid + (size_t)t * H + c0);
        if (a.w) ww = *(const uint4*)(a.w + c0);
        if (a.div_w) dd = *(const uint4*)(a.div_w + c0);
#pragma unroll
        for (int s = 0; s < GEMM_SPLIT_MAX; ++s)
            if (a.part && s < a.splits) {
                const float* src = a.part + ((size_t)s * a.Tpad + t) * H + c0;
                p[s][0] = *(const v4f*)src;
                p[s][1] = *(const v4f*)(src + 4);
            }
    }
    auto unpack8 = [](uint4 r, float* f) {
        const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = bf2f((bf16_t)(w4[i] & 0xffff));
            f[2 * i + 1] = bf2f((bf16_t)(w4[i] >> 16));
        }
    };
    float v[8], rb[8];
    unpack8(rr, rb);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (a.part) {
            float sum = 0.0f;  // split order
#pragma unroll
            for (int s = 0; s < GEMM_SPLIT_MAX; ++s)
                if (s < a.splits) sum += p[s][e >> 2][e & 3];
            v[e] = a.resid ? rbf(rb[e] + rbf(sum)) : rbf(sum);
        } else {
            v[e] = rb[e];
        }
        ss += on ? v[e] * v[e] : 0.0f;
    }
    auto pack8 = [](const float* f) {
        return make_uint4(pk_bf16(f[0], f[1]), pk_bf16(f[2], f[3]), pk_bf16(f[4], f[5]), pk_bf16(f[6], f[7]));
    };
    if (on && a.xout) *(uint4*)(a.xout + (size_t)t * H + c0) = pack8(v);
    if (!a.act && !a.hout) return;  // residual only (the last layer)
    ss = warp_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += red[w];
    const float r = 1.0f / sqrtf(tot / (float)H + a.eps);
    if (!on) return;
    float wf[8], df[8], o[8];
    unpack8(ww, wf);
    unpack8(dd, df);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        o[e] = rbf(v[e] * r * (1.0f + wf[e]));
        if (a.div_w) o[e] = rbf(o[e] / (1.0f + df[e]));
    }
    if (a.hout) *(uint4*)(a.hout + (size_t)t * H + c0) = pack8(o);
    if (a.act)
        *(uint2*)(a.act + act_offset(t, a.act_col0 + c0, a.Kact)) =
            make_uint2(pk_e5m2(o[0], o[1], o[2], o[3]), pk_e5m2(o[4], o[5], o[6], o[7]));
}

hipError_t q38_residual_norm(const NormArgs& a, hipStream_t stream) {
    if (a.part && (a.splits < 1 || a.splits > GEMM_SPLIT_MAX)) return hipErrorInvalidValue;
    const int threads = a.H / 8 > 64 ? (a.H / 8 + 63) / 64 * 64 : 64;
    hipLaunchKernelGGL(residual_norm_kernel, dim3(a.T), dim3(threads), 0, stream, a);
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
    *(uint32_t*)(act + act_offset(t, c, K)) =
        pk_e5m2(bf2f(r.x & 0xffff), bf2f(r.x >> 16), bf2f(r.y & 0xffff), bf2f(r.y >> 16));
}

hipError_t q38_act_tiles(const bf16_t* x, int T, int K, uint8_t* act, hipStream_t stream) {
    size_t groups = (size_t)T * K / 4;
    hipLaunchKernelGGL(act_tiles_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, stream, x, T, K, act);
    return hipGetLastError();
}

// bf16 activation tiles of one input plane (FP4Linear's x[..., ::2] or x[..., 1::2], model.py:206-208): inputs of the
// other parity are zero, so a GEMM over all K inputs sums exactly the plane's products.
__global__ __launch_bounds__(256) void act_tiles_bf16_kernel(const bf16_t* x, int T, int K, int plane, bf16_t* act) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // group of 4 elements
    if (i >= (size_t)T * K / 4) return;
    const int t = (int)(i / (K / 4)), c = (int)(i % (K / 4)) * 4;
    const uint2 r = *(const uint2*)(x + (size_t)t * K + c);
    const uint32_t keep = plane ? 0xffff0000u : 0x0000ffffu;  // inputs c + 1, c + 3 (odd) or c, c + 2 (even)
    *(uint2*)(act + act_offset(t, c, K)) = make_uint2(r.x & keep, r.y & keep);
}

hipError_t q38_act_tiles_bf16(const bf16_t* x, int T, int K, int plane, bf16_t* act, hipStream_t stream) {
    size_t groups = (size_t)T * K / 4;
    hipLaunchKernelGGL(act_tiles_bf16_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, stream, x, T, K,
                       plane, act);
    return hipGetLastError();
}
