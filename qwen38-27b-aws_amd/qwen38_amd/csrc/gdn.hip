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
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(K <= 4 ? 3 : 1))) void gdn_verify_kernel(const GdnArgs a) {
    constexpr int D = 128;
    constexpr int RS = (2 * K + 7) / 8 * 8;  // rows between the three bf16 parts of [k; q] (a multiple of 8)
    constexpr int MB = (3 * RS + 31) / 32;   // 32-row MFMA blocks holding them
    __shared__ float mixed[K][3 * D];   // SiLU(conv) of this head's q, k, v channels
    __shared__ float qn[K][D], kn[K][D];
    constexpr int WKS = K | 1;          // odd row stride of wk: the commit's column reads hit 32 different banks
    __shared__ float wk[D][WKS];        // committed snapshot keys times their decay weights, input-major
    __shared__ float part[2][2 * K][D]; // reads, one partial per half of the state rows
    // [k_0..k_K-1, q_0..q_K-1] as three bf16 parts (rows r, RS + r, 2 RS + r) whose sum is the float32 value to 2^-27:
    // the A operand of the reads on the bf16 MFMA (products exact, float32 sums). Rows past them are never read out.
    __shared__ __attribute__((aligned(16))) bf16_t kq3[32 * MB][D + 8];
    __shared__ float ck[K][K], cq[K][K], ecum[K];
    __shared__ float ob[K][D];
    __shared__ float rms[K];

    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Hv = a.Hv, Hk = a.Hk, C = a.C;
    const int rep = Hv / Hk, kh = h / rep;
    const bool owner = (h % rep) == 0;  // writes the shared key-head channels
    const float act = a.active[b];
    const bool on = act > 0.5f;
    const float keep = (a.position[b] == 0 && on) ? 0.0f : 1.0f;
    const int acc_n = min(max(a.accepted[b], 0), K);
    constexpr int GMAX = 8;  // gate groups, at most
    // Conv channels: thread tid < 3 D / 2 owns channels cc, cc + 1 of one group (q of key head kh, k of key head kh,
    // v of head h), so that every conv load and store is a word or wider.
    const bool conv_thread = tid < 3 * D / 2;
    const int cgrp = (2 * tid) / D, cj = (2 * tid) % D;
    const int cc = cgrp == 0 ? kh * D + cj : cgrp == 1 ? Hk * D + kh * D + cj : 2 * Hk * D + h * D + cj;

    // Every global load of the block is issued here, before the first store (a load placed after a store would wait
    // for it: the pointers may alias as far as the compiler knows), and in the order the phases use them, the state
    // last: the memory counter is in order, so each phase's wait leaves the later loads in flight. All of them are
    // unconditional, at clamped valid addresses, so that none sits in a branch whose end waits for it.
    float gp[GMAX];
    {
        const int t = tid % K, which = (tid / K) & 1, O = 2 * Hv;
        const float* p = a.gate_part + ((size_t)b * K + t) * O + (which ? Hv + h : h);
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi) gp[gi] = p[(size_t)min(gi, a.gate_groups - 1) * a.B * K * O];
    }
    const bf16_t a_log = a.a_log[h], dt_bias = a.dt_bias[h];
    float dec_in[K];
#pragma unroll
    for (int s = 0; s < K; ++s) dec_in[s] = a.decay_old[((size_t)b * K + s) * Hv + h];
    // Old conv state (3 bf16 per channel, so 3 words for the pair), last step's and this step's inputs (a word per
    // token), conv weights (4 bf16 per channel: 16 bytes). Threads past the conv channels load the v group's.
    uint32_t cv_old[3], cv_prev[K], cv_new[K];
    uint4 cv_w;
    {
        const uint32_t* po = (const uint32_t*)(a.conv_old + ((size_t)b * C + cc) * 3);
#pragma unroll
        for (int q = 0; q < 3; ++q) cv_old[q] = po[q];
#pragma unroll
        for (int s = 0; s < K; ++s) {
            cv_prev[s] = *(const uint32_t*)(a.qkv_old + ((size_t)b * K + s) * C + cc);
            cv_new[s] = *(const uint32_t*)(a.qkv_new + ((size_t)b * K + s) * C + cc);
        }
        cv_w = *(const uint4*)(a.conv_w + (size_t)cc * 4);
    }
    constexpr int KPT = (K * D + 255) / 256;  // snapshot key elements per thread
    float key_in[KPT];
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
        const int i = min(tid + 256 * u, K * D - 1);
        key_in[u] = a.key_old[(((size_t)b * K + i / D) * Hk + kh) * D + i % D];
    }
    // State ownership: wave w holds columns [64 (w & 1), +64) and rows [64 (w >> 1), +64); lane l the two columns jc,
    // jc + 1 and, in each of 4 MFMA K-steps ks, the 8 rows ir + 16 ks + [0, 8), as the bf16 MFMA's B operand wants
    // them (column l % 32, inputs 8 (l / 32) + [0, 8)); even and odd columns go to two MFMAs.
    const int jc = 64 * (wave & 1) + 2 * (lane & 31), ir = 64 * (wave >> 1) + 8 * (lane >> 5);
    // The commit's snapshot deltas, as the f32 MFMA's B operand: lane l holds snapshot 2 mi + l / 32 of columns jc,
    // jc + 1 (zero past the last snapshot, set after the loads).
    constexpr int MI = (K + 1) / 2;
    float2 dlt_in[MI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
        const int s = min(2 * mi + (lane >> 5), K - 1);
        dlt_in[mi] = *(const float2*)(a.delta_old + (((size_t)b * K + s) * Hv + h) * D + jc);
    }
    constexpr int ZPW = (K + 3) / 4;  // gated-norm rows per wave
    bf16_t z_in[ZPW][2];
#pragma unroll
    for (int u = 0; u < ZPW; ++u) {
        const int r = min(wave + 4 * u, K - 1);
#pragma unroll
        for (int half = 0; half < 2; ++half) z_in[u][half] = a.z[(size_t)(b * K + r) * Hv * D + h * D + lane + half * 64];
    }
    const bf16_t nw_lo_b = a.norm_w[lane], nw_hi_b = a.norm_w[lane + 64];
    // Compiler barriers around the state loads keep every load above in place (rather than sunk into the branch that
    // uses it, behind the state) and the state loads before the first use of anything.
    asm volatile("" ::: "memory");
    bf16_t* st = a.state + ((size_t)b * Hv + h) * D * D;
    uint32_t sv[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[ks][e] = *(const uint32_t*)(st + (size_t)(ir + 16 * ks + e) * D + jc);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
        if (2 * mi + (lane >> 5) >= K) dlt_in[mi] = make_float2(0.0f, 0.0f);

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
        const float lin = rbf(sum);
        if (which)
            s_g[t] = -expf(bf2f(a_log)) * softplusf_(lin + bf2f(dt_bias)) * act;
        else
            s_beta[t] = rbf(sigmoidf_(lin)) * act;
    }

    // Commit coefficients (model.py:386-398): decays of the taken snapshots, the state's scale and each snapshot's
    // weight exp(sum of later decays), all float32 in the reference's order; thread 192 + s of the last wave (which
    // has no conv channels) computes snapshot s's weight, thread 192 + K the scale.
    __shared__ float s_coef[K], s_scale;
    if (tid >= 192 && tid <= 192 + K) {
        const int s0 = tid - 192;
        float decays[K];
        float total = 0.0f;
#pragma unroll
        for (int s = 0; s < K; ++s) {
            decays[s] = dec_in[s] * (acc_n > s ? 1.0f : 0.0f);
            total = total + decays[s];
        }
        if (s0 == K) {
            s_scale = on ? expf(total) * keep : 1.0f;
        } else {
            float rem = total;
#pragma unroll
            for (int s = 0; s < K; ++s)
                if (s <= s0) rem = rem - decays[s];
            s_coef[s0] = expf(rem) * (acc_n > s0 ? 1.0f : 0.0f) * keep * (on ? 1.0f : 0.0f);
        }
    }

    // Conv history and conv (model.py:399-409). Channel groups: q of key head kh, k of key head kh, v of head h.
    if (conv_thread) {
        const float old6[6] = {lo_bf(cv_old[0]), hi_bf(cv_old[0]), lo_bf(cv_old[1]),
                               hi_bf(cv_old[1]), lo_bf(cv_old[2]), hi_bf(cv_old[2])};
        const uint32_t cw[4] = {cv_w.x, cv_w.y, cv_w.z, cv_w.w};
        float hist2[2][3];
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            float w_old[3 + K];  // the channel's old conv state, then the last step's inputs
#pragma unroll
            for (int q = 0; q < 3; ++q) w_old[q] = old6[3 * ch + q];
#pragma unroll
            for (int s = 0; s < K; ++s) w_old[3 + s] = ch ? hi_bf(cv_prev[s]) : lo_bf(cv_prev[s]);
            float hist[3];
#pragma unroll
            for (int jj = 0; jj < 3; ++jj) {
                float v = w_old[jj];
#pragma unroll
                for (int s = 1; s <= K; ++s) v = acc_n == s ? w_old[s + jj] : v;
                hist[jj] = hist2[ch][jj] = on ? v * keep : w_old[jj];
            }
            float win[3 + K];
            win[0] = hist[0];
            win[1] = hist[1];
            win[2] = hist[2];
#pragma unroll
            for (int t = 0; t < K; ++t) win[3 + t] = ch ? hi_bf(cv_new[t]) : lo_bf(cv_new[t]);
            const float w0 = lo_bf(cw[2 * ch]), w1 = hi_bf(cw[2 * ch]), w2 = lo_bf(cw[2 * ch + 1]), w3 = hi_bf(cw[2 * ch + 1]);
#pragma unroll
            for (int t = 0; t < K; ++t) {
                float m = rbf(((rbf(win[t] * w0) + rbf(win[t + 1] * w1)) + rbf(win[t + 2] * w2)) + rbf(win[t + 3] * w3));
                mixed[t][2 * tid + ch] = rbf(m * rbf(sigmoidf_(m)));
            }
        }
        if (cgrp == 2 || owner) {
            uint32_t* dst = (uint32_t*)(a.conv_new + ((size_t)b * C + cc) * 3);
            dst[0] = pk_bf16(hist2[0][0], hist2[0][1]);
            dst[1] = pk_bf16(hist2[0][2], hist2[1][0]);
            dst[2] = pk_bf16(hist2[1][1], hist2[1][2]);
        }
    }
    __syncthreads();

    // l2 norms (model.py:60-61, 322-331): one wave per (token, q or k) row.
    for (int r = wave; r < 2 * K; r += 4) {
        const int t = r >> 1, isk = r & 1;
        float x0 = mixed[t][isk * D + lane], x1 = mixed[t][isk * D + lane + 64];
        float ssum = warp_sum(x0 * x0 + x1 * x1);
        float rs = 1.0f / sqrtf(ssum + 1e-6f);
        float y0, y1;
        if (isk) {
            y0 = kn[t][lane] = x0 * rs;
            y1 = kn[t][lane + 64] = x1 * rs;
        } else {
            y0 = qn[t][lane] = (x0 * rs) / 11.313708498984761f;
            y1 = qn[t][lane + 64] = (x1 * rs) / 11.313708498984761f;
        }
        const int row = isk ? t : K + t;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const float y = half ? y1 : y0;
            const bf16_t hi = f2bf(y);
            const float r1 = y - bf2f(hi);  // exact
            const bf16_t mid = f2bf(r1);
            kq3[row][lane + 64 * half] = hi;
            kq3[RS + row][lane + 64 * half] = mid;
            kq3[2 * RS + row][lane + 64 * half] = f2bf(r1 - bf2f(mid));
        }
    }
    // Snapshot keys times their commit weights (model.py:397-398).
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
        const int i = tid + 256 * u;
        if (i >= K * D) break;
        const int s = i / D;
        wk[i % D][s] = key_in[u] * s_coef[s];
    }
    __syncthreads();

    // In-step couplings (model.py:438, 444): e^(cum_t - cum_s) times k_t.k_s and q_t.k_s, the dot products over 8
    // lanes of 16 inputs each; and e^cum_t. cum is the running float32 sum of this step's log decays.
    float cum[K];
#pragma unroll
    for (int t = 0; t < K; ++t) cum[t] = t == 0 ? s_g[0] : cum[t - 1] + s_g[t];
    if (tid < K) {
        float c = 0.0f;
#pragma unroll
        for (int t = 0; t < K; ++t) c = tid == t ? cum[t] : c;
        ecum[tid] = expf(c);
    }
    for (int p = tid >> 3; p < 2 * K * K; p += 32) {
        const int isq = p / (K * K), t = (p % (K * K)) / K, s = p % K;
        const float* x = (isq ? qn[t] : kn[t]) + (tid & 7) * 16;
        const float* y = kn[s] + (tid & 7) * 16;
        float v = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const float4 xv = *(const float4*)(x + e), yv = *(const float4*)(y + e);
            v += xv.x * yv.x;
            v += xv.y * yv.y;
            v += xv.z * yv.z;
            v += xv.w * yv.w;
        }
        v = group8_sum(v);
        if ((tid & 7) == 0) {
            float ct = 0.0f, cs = 0.0f;
#pragma unroll
            for (int u = 0; u < K; ++u) {
                ct = t == u ? cum[u] : ct;
                cs = s == u ? cum[u] : cs;
            }
            (isq ? cq : ck)[t][s] = expf(ct - cs) * v;
        }
    }

    // State commit and reads (model.py:262-266, 419-429). Commit S' = bf16(S * scale + U) with the rank-K update
    // U = sum_s wk_s d_s on the f32 MFMA, stored; reads [k; q] S' on the bf16 MFMA, S' (exact in bf16) against the
    // three bf16 parts of [k; q], so every product is exact and the sums are float32. Each wave sums its 64 rows; the
    // two row halves are added in the solve.
    // U's 32 x 32 blocks (bi, bj) of the wave's quadrant are laid out to match the state registers: MFMA column n is
    // state column jc + bj of lane n; MFMA row 8 q + 4 hh + t of block bi is state row ir0 + 32 bi + 16 (q / 2) + 8 hh
    // + 4 (q % 2) + t, so accumulator register 4 q + t of lane l holds U at the row ir + 16 ks + e of sv[ks][e] with
    // ks = 2 bi + q / 2, e = 4 (q % 2) + t.
    {
        const float scale = s_scale;
        const int m = lane & 31, hl = lane >> 5;
        const int arow = 64 * (wave >> 1) + 16 * (m >> 4) + 8 * ((m >> 2) & 1) + 4 * ((m >> 3) & 1) + (m & 3);
        v16f acc[MB][2];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[mb][0][q] = acc[mb][1][q] = 0.0f;
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            v16f u0, u1;
#pragma unroll
            for (int q = 0; q < 16; ++q) u0[q] = u1[q] = 0.0f;
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
                const int s = 2 * mi + hl;
                const float av = s < K ? wk[arow + 32 * bi][s] : 0.0f;
                u0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, dlt_in[mi].x, u0, 0, 0, 0);
                u1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, dlt_in[mi].y, u1, 0, 0, 0);
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int ks = 2 * bi + half;
                const int i = ir + 16 * ks;
                uint32_t pk[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int r = 4 * (2 * half + (e >> 2)) + (e & 3);
                    pk[e] = pk_bf16(__uint_as_float(sv[ks][e] << 16) * scale + u0[r],
                                    __uint_as_float(sv[ks][e] & 0xffff0000u) * scale + u1[r]);
                    *(uint32_t*)(st + (size_t)(i + e) * D + jc) = pk[e];
                }
                v4i be, bo;  // column jc (low halves) and jc + 1 (high halves), rows i .. i + 7
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    be[q] = (int)__builtin_amdgcn_perm(pk[2 * q + 1], pk[2 * q], 0x05040100u);
                    bo[q] = (int)__builtin_amdgcn_perm(pk[2 * q + 1], pk[2 * q], 0x07060302u);
                }
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const v8bf16 av = *(const v8bf16*)&kq3[32 * mb + (lane & 31)][i];
                    acc[mb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(v8bf16, be), acc[mb][0], 0, 0, 0);
                    acc[mb][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(v8bf16, bo), acc[mb][1], 0, 0, 0);
                }
            }
        }
        // Accumulator register 4 q + t of block mb holds row 32 mb + 8 q + 4 (lane / 32) + t; row r of [k; q] is the
        // sum of rows r, RS + r and 2 RS + r, which all sit in this lane (RS is a multiple of 8).
#pragma unroll
        for (int a8 = 0; a8 < (2 * K + 7) / 8; ++a8)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int r = 8 * a8 + 4 * (lane >> 5) + t;
                float ve = 0.0f, vo = 0.0f;
#pragma unroll
                for (int sp = 0; sp < 3; ++sp) {
                    const int base = sp * RS + 8 * a8;  // multiple of 8
                    const int mb = base / 32, reg = 4 * ((base % 32) / 8) + t;
                    ve += acc[mb][0][reg];
                    vo += acc[mb][1][reg];
                }
                if (r < 2 * K) *(float2*)&part[wave >> 1][r][jc] = make_float2(ve, vo);
            }
    }
    __syncthreads();

    // In-step solve (model.py:431-448), one column per thread.
    if (tid < D) {
        const int j = tid;
        float dl[K];
#pragma unroll
        for (int t = 0; t < K; ++t) {
            const float ks = part[0][t][j] + part[1][t][j];
            const float qs = part[0][K + t][j] + part[1][K + t][j];
            float delta = mixed[t][2 * D + j] - ecum[t] * ks;
#pragma unroll
            for (int s = 0; s < t; ++s) delta = delta - ck[t][s] * dl[s];
            dl[t] = delta * s_beta[t];
            float out = ecum[t] * qs;
#pragma unroll
            for (int s = 0; s <= t; ++s) out = out + cq[t][s] * dl[s];
            ob[t][j] = rbf(out);
            if (a.out_probe) a.out_probe[((size_t)b * K + t) * Hv * D + h * D + j] = f2bf(ob[t][j]);
            a.delta_new[(((size_t)b * K + t) * Hv + h) * D + j] = dl[t];
            if (owner) a.key_new[(((size_t)b * K + t) * Hk + kh) * D + j] = kn[t][j] + 0.0f;
        }
        if (j < K) a.decay_new[((size_t)b * K + j) * Hv + h] = s_g[j] + 0.0f;
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
            hv = rbf(bf2f(half ? nw_hi_b : nw_lo_b) * hv);
            float zf = bf2f(z_in[u][half]);
            float sz = zf * sigmoidf_(zf);
            a.act[act_offset(tok, h * D + j, Hv * D)] = (uint8_t)e5m2_byte(rbf(hv * sz));
        }
    }
}

// `GatedDeltaNetStep.forward` (model.py:347-374): one token per row, the recurrent form. One workgroup per (row, value
// head), 4 waves; wave w holds state rows [32w, 32w + 32), lane l columns 2l, 2l + 1.
//   keep = 0 for an active row at position 0; the conv window is [conv_state * keep, qkv], the new conv state its last
//   three entries (the old one for an inactive row); mixed = bf16 sum of bf16 tap products, SiLU in bf16.
//   S = float(S) * keep * e^g; delta = (v - S^T k) * beta; S += k delta^T (product, then sum: two roundings, as torch
//   computes them); S stored in bf16; out = S^T q from the float32 S; then the gated RMS norm times SiLU(z), e5m2.
__global__ __launch_bounds__(256) void gdn_decode_kernel(const GdnArgs a) {
    constexpr int D = 128, GMAX = 8;
    __shared__ float mixed[3 * D];
    __shared__ float qn[D], kn[D];
    __shared__ float part[4][D];
    __shared__ float dl[D], ob[D];
    __shared__ float s_gate[2];

    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Hv = a.Hv, Hk = a.Hk, C = a.C;
    const int rep = Hv / Hk, kh = h / rep;
    const bool owner = (h % rep) == 0;  // writes the shared key-head conv channels
    const bool on = a.active[b] > 0.5f;
    const float keep = (a.position[b] == 0 && on) ? 0.0f : 1.0f;

    // Every global load first (see gdn_verify_kernel).
    float gp[GMAX];
    if (tid < 2) {
        const float* p = a.gate_part + (size_t)b * 2 * Hv + (tid ? Hv + h : h);
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi) gp[gi] = p[(size_t)min(gi, a.gate_groups - 1) * a.B * 2 * Hv];
    }
    const bool conv_thread = tid < 3 * D / 2;
    const int cgrp = (2 * tid) / D, cj = (2 * tid) % D;
    const int cc = cgrp == 0 ? kh * D + cj : cgrp == 1 ? Hk * D + kh * D + cj : 2 * Hk * D + h * D + cj;
    uint32_t cv_old[3], cv_new = 0;
    uint4 cv_w = make_uint4(0, 0, 0, 0);
    if (conv_thread) {
        const uint32_t* po = (const uint32_t*)(a.conv_old + ((size_t)b * C + cc) * 3);
#pragma unroll
        for (int q = 0; q < 3; ++q) cv_old[q] = po[q];
        cv_new = *(const uint32_t*)(a.qkv_new + (size_t)b * C + cc);
        cv_w = *(const uint4*)(a.conv_w + (size_t)cc * 4);
    }
    const int j0 = 2 * lane, i0 = 32 * wave;
    bf16_t* st = a.state + ((size_t)b * Hv + h) * D * D;
    uint32_t sv[32];
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) sv[ii] = *(const uint32_t*)(st + (size_t)(i0 + ii) * D + j0);
    bf16_t z_in[2] = {0, 0};
    if (wave == 0) {
        z_in[0] = a.z[(size_t)b * Hv * D + h * D + lane];
        z_in[1] = a.z[(size_t)b * Hv * D + h * D + lane + 64];
    }
    const float nw_lo = bf2f(a.norm_w[lane]), nw_hi = bf2f(a.norm_w[lane + 64]);

    // Gates (model.py:333-337, 366-368), as in gdn_verify_kernel.
    if (tid < 2) {
        float sum = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi)
            if (gi < a.gate_groups) sum += gp[gi];
        const float lin = rbf(sum), act = a.active[b];
        s_gate[tid] = tid ? -expf(bf2f(a.a_log[h])) * softplusf_(lin + bf2f(a.dt_bias[h])) * act : rbf(sigmoidf_(lin)) * act;
    }

    // Conv (model.py:357-361).
    if (conv_thread) {
        const float old6[6] = {lo_bf(cv_old[0]), hi_bf(cv_old[0]), lo_bf(cv_old[1]),
                               hi_bf(cv_old[1]), lo_bf(cv_old[2]), hi_bf(cv_old[2])};
        const uint32_t cw[4] = {cv_w.x, cv_w.y, cv_w.z, cv_w.w};
        float next[2][3];
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            const float x = ch ? hi_bf(cv_new) : lo_bf(cv_new);
            const float win[4] = {old6[3 * ch] * keep, old6[3 * ch + 1] * keep, old6[3 * ch + 2] * keep, x};
#pragma unroll
            for (int q = 0; q < 3; ++q) next[ch][q] = on ? win[q + 1] : old6[3 * ch + q];
            const float w0 = lo_bf(cw[2 * ch]), w1 = hi_bf(cw[2 * ch]), w2 = lo_bf(cw[2 * ch + 1]), w3 = hi_bf(cw[2 * ch + 1]);
            const float m = rbf(((rbf(win[0] * w0) + rbf(win[1] * w1)) + rbf(win[2] * w2)) + rbf(win[3] * w3));
            mixed[2 * tid + ch] = rbf(m * rbf(sigmoidf_(m)));
        }
        if (cgrp == 2 || owner) {
            uint32_t* dst = (uint32_t*)(a.conv_new + ((size_t)b * C + cc) * 3);
            dst[0] = pk_bf16(next[0][0], next[0][1]);
            dst[1] = pk_bf16(next[0][2], next[1][0]);
            dst[2] = pk_bf16(next[1][1], next[1][2]);
        }
    }
    __syncthreads();

    // l2 norms of q and k (model.py:60-61, 322-331): waves 0 and 1.
    if (wave < 2) {
        const float x0 = mixed[wave * D + lane], x1 = mixed[wave * D + lane + 64];
        const float rs = 1.0f / sqrtf(warp_sum(x0 * x0 + x1 * x1) + 1e-6f);
        if (wave) {
            kn[lane] = x0 * rs;
            kn[lane + 64] = x1 * rs;
        } else {
            qn[lane] = (x0 * rs) / 11.313708498984761f;
            qn[lane + 64] = (x1 * rs) / 11.313708498984761f;
        }
    }
    __syncthreads();

    // Decayed state and its read with k.
    const float eg = expf(s_gate[1]);
    float s0[32], s1[32];
    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) {
        s0[ii] = (lo_bf(sv[ii]) * keep) * eg;
        s1[ii] = (hi_bf(sv[ii]) * keep) * eg;
        const float k = kn[i0 + ii];
        p0 += s0[ii] * k;
        p1 += s1[ii] * k;
    }
    *(float2*)&part[wave][j0] = make_float2(p0, p1);
    __syncthreads();
    if (tid < D) dl[tid] = (mixed[2 * D + tid] - (((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid])) * s_gate[0];
    __syncthreads();

    // S += k delta^T, stored in bf16; out = S^T q from the float32 state.
    {
        const float d0 = dl[j0], d1 = dl[j0 + 1];
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 32; ++ii) {
            const float k = kn[i0 + ii], q = qn[i0 + ii];
            const float n0 = __fadd_rn(s0[ii], __fmul_rn(k, d0)), n1 = __fadd_rn(s1[ii], __fmul_rn(k, d1));
            *(uint32_t*)(st + (size_t)(i0 + ii) * D + j0) = pk_bf16(n0, n1);
            o0 += n0 * q;
            o1 += n1 * q;
        }
        __syncthreads();  // part's first use is read
        *(float2*)&part[wave][j0] = make_float2(o0, o1);
    }
    __syncthreads();
    if (tid < D) ob[tid] = rbf(((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid]);
    __syncthreads();

    // Gated RMS norm (model.py:339-345) and the e5m2 input of out_proj.
    if (wave == 0) {
        const float x0 = ob[lane], x1 = ob[lane + 64];
        const float r = 1.0f / sqrtf(warp_sum(x0 * x0 + x1 * x1) / 128.0f + a.eps);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int j = lane + half * 64;
            float hv = rbf((half ? x1 : x0) * r);
            hv = rbf((half ? nw_hi : nw_lo) * hv);
            const float zf = bf2f(z_in[half]);
            a.act[act_offset(b, h * D + j, Hv * D)] = (uint8_t)e5m2_byte(rbf(hv * (zf * sigmoidf_(zf))));
        }
    }
}

hipError_t q38_gdn_decode(const GdnArgs& a, hipStream_t stream) {
    if (a.gate_groups < 1 || a.gate_groups > 8 || a.K != 1 || a.Hv % a.Hk || a.C != 2 * a.Hk * 128 + a.Hv * 128)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_decode_kernel, dim3(a.Hv, a.B), dim3(256), 0, stream, a);
    return hipGetLastError();
}

// Row `slot` of each layer's recurrent and conv state, live <-> saved (GatedDeltaNetStep.copy_states, model.py:456-464).
// Grid (workgroups per layer, layers); 16-byte copies.
__global__ __launch_bounds__(256) void copy_states_kernel(const CopyStatesArgs a) {
    const int layer = blockIdx.y, slot = *a.slot;
    if (slot < 0 || slot >= a.rows) return;
    const bf16_t* src_s = a.to_saved ? a.state[layer] : a.saved_state[layer];
    bf16_t* dst_s = a.to_saved ? a.saved_state[layer] : a.state[layer];
    const size_t n16 = a.state_row / 8;  // 16-byte chunks of the row
    const uint4* src = (const uint4*)(src_s + (size_t)slot * a.state_row);
    uint4* dst = (uint4*)(dst_s + (size_t)slot * a.state_row);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) dst[i] = src[i];
    if (blockIdx.x == 0) {
        const bf16_t* src_c = (a.to_saved ? a.conv[layer] : a.saved_conv[layer]) + (size_t)slot * a.conv_row;
        bf16_t* dst_c = (a.to_saved ? a.saved_conv[layer] : a.conv[layer]) + (size_t)slot * a.conv_row;
        for (size_t i = threadIdx.x; i < a.conv_row; i += 256) dst_c[i] = src_c[i];
    }
}

hipError_t q38_copy_states(const CopyStatesArgs& a, hipStream_t stream) {
    if (a.n < 1 || a.n > COPY_STATES_MAX || a.state_row % 8 || a.rows < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_states_kernel, dim3(64, a.n), dim3(256), 0, stream, a);
    return hipGetLastError();
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
    if (a.gate_groups < 1 || a.gate_groups > 8 || a.K < 1 || a.K > 8 || a.Hv % a.Hk || a.C != 2 * a.Hk * 128 + a.Hv * 128)
        return hipErrorInvalidValue;
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
