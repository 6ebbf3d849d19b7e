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
// Beta and decay projections (model.py:145-147): dot products of the bf16 normed hidden rows with the in_proj_b and
// in_proj_a rows, as partial sums over `groups` K ranges on the bf16 MFMA (float32 accumulation); gdn_verify adds the
// partials in group order and applies the bf16 rounding, sigmoid and softplus. Workgroup (token tile, output tile,
// group): 4 waves, each a 32 x 32 tile over H / (4 groups) inputs with all its loads issued up front.
__global__ __launch_bounds__(256) void gdn_gates_kernel(const GatesArgs a) {
    constexpr int MAXCH = 16;  // 16-input MFMA steps per wave, at most
    __shared__ float red[4][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int O = 2 * a.Hv, nto = (O + 31) / 32;
    const int tt = blockIdx.x / nto, ot = blockIdx.x % nto, grp = blockIdx.y;
    const int kw = a.H / (4 * a.groups), nch = kw / 16;
    const int k0 = (grp * 4 + wave) * kw + (lane >> 5) * 8;
    const int o = min(ot * 32 + (lane & 31), O - 1);
    const bf16_t* wrow = (o < a.Hv ? a.wb + (size_t)o * a.H : a.wa + (size_t)(o - a.Hv) * a.H) + k0;
    const bf16_t* xrow = a.x + (size_t)min(tt * 32 + (lane & 31), a.T - 1) * a.H + k0;
    v4i wv[MAXCH], xv[MAXCH];
#pragma unroll
    for (int c = 0; c < MAXCH; ++c)
        if (c < nch) {
            wv[c] = *(const v4i*)(wrow + c * 16);
            xv[c] = *(const v4i*)(xrow + c * 16);
        }
    v16f acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < MAXCH; ++c)
        if (c < nch)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf16, wv[c]), __builtin_bit_cast(v8bf16, xv[c]),
                                                          acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    if (wave) return;
    // Lane l holds token column l % 32 and output rows 8 * (i / 4) + 4 * (l / 32) + i % 4.
    const int tok = tt * 32 + (lane & 31);
    if (tok >= a.T) return;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int oo = ot * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (oo < O)
            a.part[((size_t)grp * a.T + tok) * O + oo] = ((red[0][i][lane] + red[1][i][lane]) + red[2][i][lane]) + red[3][i][lane];
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
    constexpr int GMAX = 8;  // gate groups, at most
    constexpr int CPT = (3 * D + 255) / 256;  // conv channels per thread

    // Every global load of the block is issued here, before the first store: a load placed after a store would wait
    // for it (the pointers may alias as far as the compiler knows), and each wait is a memory round trip.
    float gp[GMAX];
    if (tid < 2 * K) {
        const int t = tid % K, which = tid / K, O = 2 * Hv;
        const float* p = a.gate_part + ((size_t)b * K + t) * O + (which ? Hv + h : h);
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi) gp[gi] = gi < a.gate_groups ? p[(size_t)gi * a.B * K * O] : 0.0f;
    }
    float dec_in[K];
#pragma unroll
    for (int s = 0; s < K; ++s) dec_in[s] = a.decay_old[((size_t)b * K + s) * Hv + h];
    bf16_t conv_in[CPT][3 + 2 * K + 4];  // old conv state, last step's inputs, this step's inputs, conv weights
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int ci = tid + 256 * u;
        if (ci >= 3 * D) break;
        const int grp = ci / D, j = ci % D;
        const int c = grp == 0 ? kh * D + j : grp == 1 ? Hk * D + kh * D + j : 2 * Hk * D + h * D + j;
#pragma unroll
        for (int q = 0; q < 3; ++q) conv_in[u][q] = a.conv_old[((size_t)b * C + c) * 3 + q];
#pragma unroll
        for (int s = 0; s < K; ++s) {
            conv_in[u][3 + s] = a.qkv_old[((size_t)b * K + s) * C + c];
            conv_in[u][3 + K + s] = a.qkv_new[((size_t)b * K + s) * C + c];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) conv_in[u][3 + 2 * K + q] = a.conv_w[(size_t)c * 4 + q];
    }
    constexpr int KPT = (K * D + 255) / 256;  // snapshot key elements per thread
    float key_in[KPT];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
        const int i = tid + 256 * u;
        key_in[u] = i < K * D ? a.key_old[(((size_t)b * K + i / D) * Hk + kh) * D + i % D] : 0.0f;
    }
    const int j0 = lane * 2, i0 = wave * 32;
    float2 dlt_in[K];
#pragma unroll
    for (int s = 0; s < K; ++s) dlt_in[s] = *(const float2*)(a.delta_old + (((size_t)b * K + s) * Hv + h) * D + j0);
    bf16_t* st = a.state + ((size_t)b * Hv + h) * D * D;
    uint32_t sv[32];
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) sv[ii] = *(const uint32_t*)(st + (size_t)(i0 + ii) * D + j0);
    constexpr int ZPW = (K + 3) / 4;  // gated-norm rows per wave
    bf16_t z_in[ZPW][2];
#pragma unroll
    for (int u = 0; u < ZPW; ++u) {
        const int r = wave + 4 * u;
#pragma unroll
        for (int half = 0; half < 2; ++half)
            z_in[u][half] = r < K ? a.z[(size_t)(b * K + r) * Hv * D + h * D + lane + half * 64] : (bf16_t)0;
    }
    const float nw_lo = bf2f(a.norm_w[lane]), nw_hi = bf2f(a.norm_w[lane + 64]);

    // This step's gates (model.py:145-147): beta = sigmoid(bf16(x . in_proj_b)), g = -exp(A_log) softplus(bf16(x .
    // in_proj_a) + dt_bias), both times the row's active flag; the dot products are the gates kernel's partials, added
    // in group order.
    __shared__ float s_beta[K], s_g[K];
    if (tid < 2 * K) {
        const int t = tid % K, which = tid / K;
        float sum = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi)
            if (gi < a.gate_groups) sum += gp[gi];
        const float lin = rbf(sum), act = a.active[b];
        if (which)
            s_g[t] = -expf(bf2f(a.a_log[h])) * softplusf_(lin + bf2f(a.dt_bias[h])) * act;
        else
            s_beta[t] = rbf(sigmoidf_(lin)) * act;
    }

    // Commit coefficients (model.py:386-398): decays of the taken snapshots, the state's scale and each snapshot's
    // weight exp(sum of later decays), all float32 in the reference's order.
    float decays[K], coef[K];
    float total = 0.0f;
#pragma unroll
    for (int s = 0; s < K; ++s) {
        decays[s] = dec_in[s] * (acc_n > s ? 1.0f : 0.0f);
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
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
        const int ci = tid + 256 * u;
        if (ci >= 3 * D) break;
        const int grp = ci / D, j = ci % D;
        const int c = grp == 0 ? kh * D + j : grp == 1 ? Hk * D + kh * D + j : 2 * Hk * D + h * D + j;
        float w_old[3 + K];
#pragma unroll
        for (int q = 0; q < 3 + K; ++q) w_old[q] = bf2f(conv_in[u][q]);
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
        for (int t = 0; t < K; ++t) win[3 + t] = bf2f(conv_in[u][3 + K + t]);
        const float w0 = bf2f(conv_in[u][3 + 2 * K]), w1 = bf2f(conv_in[u][3 + 2 * K + 1]), w2 = bf2f(conv_in[u][3 + 2 * K + 2]),
                    w3 = bf2f(conv_in[u][3 + 2 * K + 3]);
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
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
        const int i = tid + 256 * u;
        if (i >= K * D) break;
        const int s = i / D;
        float c = 0.0f;
#pragma unroll
        for (int r = 0; r < K; ++r) c = s == r ? coef[r] : c;
        wk[s][i % D] = key_in[u] * c;
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
        float d0[K], d1[K];
#pragma unroll
        for (int s = 0; s < K; ++s) {
            d0[s] = dlt_in[s].x;
            d1[s] = dlt_in[s].y;
        }
        float p0[2 * K], p1[2 * K];
#pragma unroll
        for (int r = 0; r < 2 * K; ++r) p0[r] = p1[r] = 0.0f;
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
            *(uint32_t*)(st + (size_t)i * D + j0) = pk_bf16(c0, c1);
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
            gl[t] = s_g[t];
            beta[t] = s_beta[t];
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
#pragma unroll
    for (int u = 0; u < ZPW; ++u) {
        const int r = wave + 4 * u;
        if (r >= K) break;
        const int tok = b * K + r;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int j = lane + half * 64;
            float hv = rbf(ob[r][j] * rms[r]);
            hv = rbf((half ? nw_hi : nw_lo) * hv);
            float zf = bf2f(z_in[u][half]);
            float sz = zf * sigmoidf_(zf);
            a.act[act_offset(tok, h * D + j, Hv * D)] = (uint8_t)e5m2_byte(rbf(hv * sz));
        }
    }
}

hipError_t q38_gdn_gates(const GatesArgs& a, hipStream_t stream) {
    if (a.H % (64 * a.groups) || a.H / (64 * a.groups) > 16) return hipErrorInvalidValue;
    dim3 grid(((a.T + 31) / 32) * ((2 * a.Hv + 31) / 32), a.groups);
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
