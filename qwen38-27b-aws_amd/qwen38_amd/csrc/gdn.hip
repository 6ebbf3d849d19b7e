// Gated delta net, multi-token verify form: `GatedDeltaNetStep.verify` (reference qwen38_inf2/model.py:376-454) with
// its chip kernel `delta_verify_state` (kernels.py:913-968), for one layer.
//
// The reference keeps a verify step's tokens out of the recurrent state and stores what each would add (key, delta,
// decay and the conv input: the "pending" snapshots, model.py:313-320); the next step first commits the accepted
// prefix of them (model.py:386-404) and then runs its own tokens against the committed state (model.py:406-448).
// Here one workgroup per (row, value head) does all of it with the 128x128 state read once and written once:
//   conv history commit and conv over the K new tokens, SiLU, l2 norms, the state commit S' = bf16(S*scale + W^T D),
//   the 2K reads [k; q] S', the K x K in-step solve, the gated RMS norm times SiLU(z), e5m2 for out_proj, and the
//   new snapshots.
// Snapshots and the conv state are double buffered (read one half, write the other) because a key head's channels
// are shared by several value heads' workgroups; the recurrent state is read and written by its own workgroup only.
// The pending input snapshot is the in_proj_qkv output itself (the GEMM writes it into the half being written).
#include "kernels.h"

// `_gates` (model.py:333-337) and the active masks (model.py:411-413): beta = bf16 sigmoid of a bf16 linear, and
// g = -exp(A_log) * softplus(float(bf16 linear) + dt_bias), both times active. Block: 8 tokens x 16 outputs
// (output o < Hv is in_proj_b's row o, else in_proj_a's row o - Hv); each wave owns 4 outputs.
__global__ __launch_bounds__(256) void gdn_gates_kernel(const GatesArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 8, o0 = blockIdx.y * 16 + wave * 4;
    float acc[4][8];
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[o][t] = 0.0f;
    const bf16_t* wrow[4];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        int oo = o0 + o;
        wrow[o] = oo < a.Hv ? a.wb + (size_t)oo * a.H : a.wa + (size_t)(oo - a.Hv) * a.H;
    }
    for (int c = lane * 4; c < a.H; c += 256) {
        float wv[4][4];
#pragma unroll
        for (int o = 0; o < 4; ++o) {
            uint2 r = *(const uint2*)(wrow[o] + c);
            wv[o][0] = bf2f(r.x & 0xffff);
            wv[o][1] = bf2f(r.x >> 16);
            wv[o][2] = bf2f(r.y & 0xffff);
            wv[o][3] = bf2f(r.y >> 16);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int tt = min(t0 + t, a.T - 1);
            uint2 r = *(const uint2*)(a.x + (size_t)tt * a.H + c);
            float xv[4] = {bf2f(r.x & 0xffff), bf2f(r.x >> 16), bf2f(r.y & 0xffff), bf2f(r.y >> 16)};
#pragma unroll
            for (int o = 0; o < 4; ++o)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[o][t] += wv[o][e] * xv[e];
        }
    }
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[o][t] = warp_sum(acc[o][t]);
    if (lane == 0) {
#pragma unroll
        for (int o = 0; o < 4; ++o) {
            int oo = o0 + o;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                int tt = t0 + t;
                if (tt >= a.T) continue;
                float on = a.active[tt / a.K];
                float lin = rbf(acc[o][t]);
                if (oo < a.Hv) {
                    a.beta[(size_t)tt * a.Hv + oo] = rbf(sigmoidf_(lin)) * on;
                } else {
                    int h = oo - a.Hv;
                    float decay = -expf(bf2f(a.a_log[h])) * softplusf_(lin + bf2f(a.dt_bias[h]));
                    a.g[(size_t)tt * a.Hv + h] = decay * on;
                }
            }
        }
    }
}

// K (tokens per row) is a template parameter so that every per-token array lives in registers.
template <int K>
__global__ __launch_bounds__(256) void gdn_verify_kernel(const GdnArgs a) {
    constexpr int D = 128;
    __shared__ float mixed[K][3 * D];   // SiLU(conv) of this head's q, k, v channels
    __shared__ float qn[K][D], kn[K][D];
    __shared__ float wk[K][D];          // committed snapshot keys times their decay weights
    __shared__ float part[4][2 * K][D]; // reads, one partial per row quarter
    __shared__ float kk[K][K], qk[K][K];
    __shared__ float ob[K][D];
    __shared__ float rms[K];

    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Hv = a.Hv, Hk = a.Hk, C = a.C;
    const int rep = Hv / Hk, kh = h / rep;
    const bool owner = (h % rep) == 0;  // writes the shared key-head channels
    const bool on = a.active[b] > 0.5f;
    const float keep = (a.position[b] == 0 && on) ? 0.0f : 1.0f;
    const int acc_n = min(max(a.accepted[b], 0), K);

    // Commit coefficients (model.py:386-398): decays of the taken snapshots, the state's scale and each snapshot's
    // weight exp(sum of later decays), all float32 in the reference's order.
    float decays[K], coef[K];
    float total = 0.0f;
#pragma unroll
    for (int s = 0; s < K; ++s) {
        decays[s] = a.decay_old[((size_t)b * K + s) * Hv + h] * (acc_n > s ? 1.0f : 0.0f);
        total = total + decays[s];
    }
    const float scale = on ? expf(total) * keep : 1.0f;
    {
        float rem = total;
#pragma unroll
        for (int s = 0; s < K; ++s) {
            rem = rem - decays[s];
            coef[s] = expf(rem) * (acc_n > s ? 1.0f : 0.0f) * keep * (on ? 1.0f : 0.0f);
        }
    }

    // Conv history and conv (model.py:399-409). Channel groups: q of key head kh, k of key head kh, v of head h.
    for (int ci = tid; ci < 3 * D; ci += 256) {
        const int grp = ci / D, j = ci % D;
        const int c = grp == 0 ? kh * D + j : grp == 1 ? Hk * D + kh * D + j : 2 * Hk * D + h * D + j;
        const bf16_t* old = a.conv_old + ((size_t)b * C + c) * 3;
        float w_old[3 + K];
        w_old[0] = bf2f(old[0]);
        w_old[1] = bf2f(old[1]);
        w_old[2] = bf2f(old[2]);
#pragma unroll
        for (int s = 0; s < K; ++s) w_old[3 + s] = bf2f(a.qkv_old[((size_t)b * K + s) * C + c]);
        float hist[3];
#pragma unroll
        for (int jj = 0; jj < 3; ++jj) {
            float v = w_old[jj];
#pragma unroll
            for (int s = 1; s <= K; ++s) v = acc_n == s ? w_old[s + jj] : v;
            hist[jj] = on ? v * keep : w_old[jj];
        }
        if (grp == 2 || owner) {
            bf16_t* dst = a.conv_new + ((size_t)b * C + c) * 3;
            dst[0] = f2bf(hist[0]);
            dst[1] = f2bf(hist[1]);
            dst[2] = f2bf(hist[2]);
        }
        float win[3 + K];
        win[0] = hist[0];
        win[1] = hist[1];
        win[2] = hist[2];
#pragma unroll
        for (int t = 0; t < K; ++t) win[3 + t] = bf2f(a.qkv_new[((size_t)b * K + t) * C + c]);
        const bf16_t* cw = a.conv_w + (size_t)c * 4;
        const float w0 = bf2f(cw[0]), w1 = bf2f(cw[1]), w2 = bf2f(cw[2]), w3 = bf2f(cw[3]);
#pragma unroll
        for (int t = 0; t < K; ++t) {
            float m = rbf(((rbf(win[t] * w0) + rbf(win[t + 1] * w1)) + rbf(win[t + 2] * w2)) + rbf(win[t + 3] * w3));
            mixed[t][ci] = rbf(m * rbf(sigmoidf_(m)));
        }
    }
    __syncthreads();

    // l2 norms (model.py:60-61, 322-331): one wave per (token, q or k) row.
    for (int r = wave; r < 2 * K; r += 4) {
        const int t = r >> 1, isk = r & 1;
        float x0 = mixed[t][isk * D + lane], x1 = mixed[t][isk * D + lane + 64];
        float ssum = warp_sum(x0 * x0 + x1 * x1);
        float rs = 1.0f / sqrtf(ssum + 1e-6f);
        if (isk) {
            kn[t][lane] = x0 * rs;
            kn[t][lane + 64] = x1 * rs;
        } else {
            qn[t][lane] = (x0 * rs) / 11.313708498984761f;
            qn[t][lane + 64] = (x1 * rs) / 11.313708498984761f;
        }
    }
    // Snapshot keys times their commit weights (model.py:397-398).
    for (int i = tid; i < K * D; i += 256) {
        const int s = i / D, j = i % D;
        float c = 0.0f;
#pragma unroll
        for (int r = 0; r < K; ++r) c = s == r ? coef[r] : c;
        wk[s][j] = a.key_old[(((size_t)b * K + s) * Hk + kh) * D + j] * c;
    }
    __syncthreads();

    // In-step dot products k_t.k_s and q_t.k_s (model.py:438, 444).
    for (int r = wave; r < 2 * K * K; r += 4) {
        const int isq = r / (K * K), t = (r % (K * K)) / K, s = r % K;
        const float* x = isq ? qn[t] : kn[t];
        float v = warp_sum(x[lane] * kn[s][lane] + x[lane + 64] * kn[s][lane + 64]);
        if (lane == 0) (isq ? qk : kk)[t][s] = v;
    }

    // State commit and reads (model.py:262-266, 419-429): thread owns columns 2*lane, 2*lane+1 of rows
    // [32*wave, 32*wave+32).
    {
        const int j0 = lane * 2, i0 = wave * 32;
        float d0[K], d1[K];
#pragma unroll
        for (int s = 0; s < K; ++s) {
            const float2 dp = *(const float2*)(a.delta_old + (((size_t)b * K + s) * Hv + h) * D + j0);
            d0[s] = dp.x;
            d1[s] = dp.y;
        }
        float p0[2 * K], p1[2 * K];
#pragma unroll
        for (int r = 0; r < 2 * K; ++r) p0[r] = p1[r] = 0.0f;
        bf16_t* st = a.state + ((size_t)b * Hv + h) * D * D;
        uint32_t sv[32];
#pragma unroll
        for (int ii = 0; ii < 32; ++ii) sv[ii] = *(const uint32_t*)(st + (size_t)(i0 + ii) * D + j0);
#pragma unroll 4
        for (int ii = 0; ii < 32; ++ii) {
            const int i = i0 + ii;
            float u0 = 0.0f, u1 = 0.0f;
#pragma unroll
            for (int s = 0; s < K; ++s) {
                u0 += wk[s][i] * d0[s];
                u1 += wk[s][i] * d1[s];
            }
            const float c0 = rbf(bf2f(sv[ii] & 0xffff) * scale + u0);
            const float c1 = rbf(bf2f(sv[ii] >> 16) * scale + u1);
            *(uint32_t*)(st + (size_t)i * D + j0) = (uint32_t)f2bf(c0) | ((uint32_t)f2bf(c1) << 16);
#pragma unroll
            for (int r = 0; r < 2 * K; ++r) {
                const float rv = r < K ? kn[r][i] : qn[r - K][i];
                p0[r] += rv * c0;
                p1[r] += rv * c1;
            }
        }
#pragma unroll
        for (int r = 0; r < 2 * K; ++r) *(float2*)&part[wave][r][j0] = make_float2(p0[r], p1[r]);
    }
    __syncthreads();

    // In-step solve (model.py:431-448), one column per thread.
    if (tid < D) {
        const int j = tid;
        float cum[K], beta[K], gl[K], dl[K];
#pragma unroll
        for (int t = 0; t < K; ++t) {
            gl[t] = a.g[((size_t)b * K + t) * Hv + h];
            beta[t] = a.beta[((size_t)b * K + t) * Hv + h];
            cum[t] = t == 0 ? gl[0] : cum[t - 1] + gl[t];
        }
#pragma unroll
        for (int t = 0; t < K; ++t) {
            const float ks = ((part[0][t][j] + part[1][t][j]) + part[2][t][j]) + part[3][t][j];
            const float qs = ((part[0][K + t][j] + part[1][K + t][j]) + part[2][K + t][j]) + part[3][K + t][j];
            float delta = mixed[t][2 * D + j] - expf(cum[t]) * ks;
#pragma unroll
            for (int s = 0; s < t; ++s) delta = delta - (expf(cum[t] - cum[s]) * kk[t][s]) * dl[s];
            dl[t] = delta * beta[t];
            float out = expf(cum[t]) * qs;
#pragma unroll
            for (int s = 0; s <= t; ++s) out = out + (expf(cum[t] - cum[s]) * qk[t][s]) * dl[s];
            ob[t][j] = rbf(out);
            a.delta_new[(((size_t)b * K + t) * Hv + h) * D + j] = dl[t];
            if (owner) a.key_new[(((size_t)b * K + t) * Hk + kh) * D + j] = kn[t][j] + 0.0f;
        }
        if (j < K) {
            float g = 0.0f;
#pragma unroll
            for (int t = 0; t < K; ++t) g = j == t ? gl[t] : g;
            a.decay_new[((size_t)b * K + j) * Hv + h] = g + 0.0f;
        }
    }
    __syncthreads();

    // Gated RMS norm (model.py:339-345): per token mean of squares over the head's 128 outputs.
    for (int t = wave; t < K; t += 4) {
        float x0 = ob[t][lane], x1 = ob[t][lane + 64];
        float ssum = warp_sum(x0 * x0 + x1 * x1);
        if (lane == 0) rms[t] = 1.0f / sqrtf(ssum / 128.0f + a.eps);
    }
    __syncthreads();
    const float nw_lo = bf2f(a.norm_w[lane]), nw_hi = bf2f(a.norm_w[lane + 64]);
    for (int r = wave; r < K; r += 4) {
        const int tok = b * K + r;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int j = lane + half * 64;
            float hv = rbf(ob[r][j] * rms[r]);
            hv = rbf((half ? nw_hi : nw_lo) * hv);
            float zf = bf2f(a.z[(size_t)tok * Hv * D + h * D + j]);
            float sz = zf * sigmoidf_(zf);
            a.act[act_offset(tok, h * D + j, Hv * D)] = (uint8_t)e5m2_byte(rbf(hv * sz));
        }
    }
}

hipError_t q38_gdn_gates(const GatesArgs& a, hipStream_t stream) {
    dim3 grid((a.T + 7) / 8, (2 * a.Hv) / 16);
    hipLaunchKernelGGL(gdn_gates_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int K>
static hipError_t launch_gdn(const GdnArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(gdn_verify_kernel<K>, dim3(a.Hv, a.B), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t q38_gdn_verify(const GdnArgs& a, hipStream_t stream) {
    switch (a.K) {
        case 1: return launch_gdn<1>(a, stream);
        case 2: return launch_gdn<2>(a, stream);
        case 3: return launch_gdn<3>(a, stream);
        case 4: return launch_gdn<4>(a, stream);
        case 5: return launch_gdn<5>(a, stream);
        case 6: return launch_gdn<6>(a, stream);
        case 7: return launch_gdn<7>(a, stream);
        default: return launch_gdn<8>(a, stream);
    }
}
