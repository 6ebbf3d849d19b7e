// Prefill form of the verify path's layers: one chunk of L tokens of one row (`slot`) from position `start`, tokens
// from `n_valid` on being padding (reference qwen38_inf2/model.py:476-521 for the gated delta net, 704-799 for
// attention, 843-855 for the MTP layer's cache-only form).
//
// Gated delta net, after the qkvz GEMM and the gates kernel over the chunk:
//   gdn_prefill_prep   (token, key head): conv over the chunk with the row's conv history (bf16 tap products summed
//                      by bf16 additions, model.py:514), SiLU, l2 norms of q and k, the gates times `valid`
//   gdn_prefill_scan   (value head, 32 state columns): the gated delta rule token by token in float32 from the row's
//                      state (times `start > 0`), the state kept in registers, the tokens' k, q, v, beta and g staged
//                      through LDS a round ahead; per token S = e^g S, delta = (v - S^T
//                      k) beta, S += k delta^T, o = S^T q. The reference runs the same rule in pieces of 128 tokens
//                      (chunked_gated_delta, model.py:88-124); both are the same sums in float32, in another order.
//   gdn_prefill_finish (token, 4 value heads): o to bf16, gated RMS norm times SiLU(z), e5m2 tiles for out_proj
//   gdn_prefill_carry  the row's new conv state: the three inputs from n_valid on of [history, chunk]
//
// Attention, after the qkv GEMM over the chunk:
//   attn_prefill_prep  (token): q and k RMS norms and RoPE in bf16 (model.py:565-577), q times 1/16 (exact) to scratch;
//                      the chunk's keys and values into row slot's cache at start .. start + L - 1 (model.py:791-799;
//                      the other rows' junk writes at the cache's end are left out: nothing reads them)
//   attn_prefill       (128 tokens, query head), four waves of 32 tokens sharing each 32-position K/V sub-block through
//                      LDS: blocked_attention (model.py:170-191) over the row's cached
//                      positions before `start` and the chunk's own tokens causally, in the reference's blocks of 2048
//                      positions of [cache, chunk]: per block the running max, e^(s - max) summed in float32, the
//                      weights in bf16 times V on the MFMA (float32 sums, rounded to bf16 once per block, as the
//                      reference's bf16 matmul), output and sum rescaled across blocks; then out / sum, the gate, e5m2.
//                      Positions a row cannot see are skipped: the reference gives them weights of exactly zero.
#include "kernels.h"

namespace {

__device__ __forceinline__ float conv_window(const PrefillGdnArgs& a, const bf16_t* hist, float keep, int c, int w) {
    // Input w of channel c's window: the row's conv history (times keep) for w < 3, then the chunk's inputs.
    return w < 3 ? bf2f(hist[(size_t)c * 3 + w]) * keep : bf2f(a.qkv[(size_t)(w - 3) * a.C + c]);
}

}  // namespace

__global__ __launch_bounds__(256) void gdn_prefill_prep_kernel(const PrefillGdnArgs a) {
    constexpr int D = 128, GMAX = 8;
    __shared__ float red[4];
    const int t = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Hk = a.Hk, Hv = a.Hv, C = a.C, rep = Hv / Hk;
    const int slot = *a.slot;
    if (slot < 0 || slot >= a.rows) return;
    const float keep = *a.start > 0 ? 1.0f : 0.0f, valid = t < *a.n_valid ? 1.0f : 0.0f;
    const bf16_t* hist = a.conv + (size_t)slot * C * 3;

    // Gates of this key head's value heads (model.py:333-337, 499-500).
    if (tid < 2 * rep) {
        const int h = kh * rep + tid % rep, which = tid / rep, O = 2 * Hv;
        const float* p = a.gate_part + (size_t)t * O + (which ? Hv + h : h);
        float sum = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GMAX; ++gi)
            if (gi < a.gate_groups) sum += p[(size_t)gi * a.L * O];
        const float lin = rbf(sum);
        if (which)
            a.g[(size_t)t * Hv + h] = -expf(bf2f(a.a_log[h])) * softplusf_(lin + bf2f(a.dt_bias[h])) * valid;
        else
            a.beta[(size_t)t * Hv + h] = rbf(sigmoidf_(lin)) * valid;
    }

    // Channel ci of this block: q (0..127) and k (128..255) of key head kh, then v of its value heads.
    auto mixed = [&](int ci) {
        const int c = ci < D ? kh * D + ci : ci < 2 * D ? Hk * D + kh * D + ci - D : 2 * Hk * D + kh * rep * D + ci - 2 * D;
        const bf16_t* wc = a.conv_w + (size_t)c * 4;
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float p = rbf(conv_window(a, hist, keep, c, t + j) * bf2f(wc[j]));
            m = j == 0 ? p : rbf(m + p);
        }
        return rbf(m * rbf(sigmoidf_(m)));
    };

    // q and k: one channel per thread, l2 norms over each 128 (waves 0-1: q, 2-3: k).
    const float x = mixed(tid);
    float ss = warp_sum(x * x);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float tot = wave < 2 ? red[0] + red[1] : red[2] + red[3];
    const float rs = 1.0f / sqrtf(tot + 1e-6f);
    if (wave < 2)
        a.qn[((size_t)t * Hk + kh) * D + tid] = (x * rs) / 11.313708498984761f;
    else
        a.kn[((size_t)t * Hk + kh) * D + tid - D] = x * rs;
    // v of the rep value heads.
    for (int ci = 2 * D + tid; ci < (2 + rep) * D; ci += 256) {
        const int h = kh * rep + (ci - 2 * D) / D, d = (ci - 2 * D) % D;
        a.v[((size_t)t * Hv + h) * D + d] = mixed(ci);
    }
}

// Grid (value head, group of 32 state columns); thread (column c = tid / 8, rows 16 (tid % 8) + [0, 16)). Tokens are
// staged through LDS 16 at a time in two buffers: each round's loads are issued into registers before the round
// before it runs, so their latency hides behind its 16 token steps.
__global__ __launch_bounds__(256) void gdn_prefill_scan_kernel(const PrefillGdnArgs a) {
    constexpr int D = 128, TB = 16;  // tokens staged per round
    __shared__ __attribute__((aligned(16))) float sk[2][TB][D], sq[2][TB][D];
    __shared__ float sv[2][TB][32], sb[2][TB], sg[2][TB];
    const int h = blockIdx.x, grp = blockIdx.y, tid = threadIdx.x;
    const int Hk = a.Hk, Hv = a.Hv, kh = h / (Hv / Hk);
    const int c = tid >> 3, r = tid & 7, j = grp * 32 + c, i0 = r * 16;
    const int slot = *a.slot;
    if (slot < 0 || slot >= a.rows) return;
    const float keep = *a.start > 0 ? 1.0f : 0.0f;
    bf16_t* st = a.state + ((size_t)slot * Hv + h) * D * D;
    float s[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = bf2f(st[(size_t)(i0 + e) * D + j]) * keep;

    // One round's loads: 2 float4 of k and of q, 2 values of v, and beta and g for threads 0 .. TB - 1; tokens past
    // the chunk load its last token (never used).
    static_assert(TB * D / 4 == 2 * 256 && TB * 32 == 2 * 256, "two pieces per thread");
    float4 rk[2], rq[2];
    float rv[2], rb = 0.0f, rg = 0.0f;
    auto load = [&](int t0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = tid + 256 * u, t = min(t0 + e / (D / 4), a.L - 1), d = (e % (D / 4)) * 4;
            rk[u] = *(const float4*)(a.kn + ((size_t)t * Hk + kh) * D + d);
            rq[u] = *(const float4*)(a.qn + ((size_t)t * Hk + kh) * D + d);
            const int tv = min(t0 + e / 32, a.L - 1);
            rv[u] = a.v[((size_t)tv * Hv + h) * D + grp * 32 + e % 32];
        }
        const int tb = min(t0 + (tid & (TB - 1)), a.L - 1);
        rb = a.beta[(size_t)tb * Hv + h];
        rg = a.g[(size_t)tb * Hv + h];
    };
    load(0);
    for (int t0 = 0, buf = 0; t0 < a.L; t0 += TB, buf ^= 1) {
        // Buffer buf was last read two rounds ago, before every thread passed the last round's barrier.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = tid + 256 * u, tt = e / (D / 4), d = (e % (D / 4)) * 4;
            *(float4*)&sk[buf][tt][d] = rk[u];
            *(float4*)&sq[buf][tt][d] = rq[u];
            sv[buf][e / 32][e % 32] = rv[u];
        }
        if (tid < TB) {
            sb[buf][tid] = rb;
            sg[buf][tid] = rg;
        }
        __syncthreads();
        if (t0 + TB < a.L) load(t0 + TB);
        const int nt = min(TB, a.L - t0);
        for (int tt = 0; tt < nt; ++tt) {
            const float e = expf(sg[buf][tt]);
            float kv[16], qv[16];
#pragma unroll
            for (int q = 0; q < 16; q += 4) {
                *(float4*)&kv[q] = *(const float4*)&sk[buf][tt][i0 + q];
                *(float4*)&qv[q] = *(const float4*)&sq[buf][tt][i0 + q];
            }
            float ks = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                s[q] *= e;
                ks += s[q] * kv[q];
            }
            ks = group8_sum(ks);
            const float delta = (sv[buf][tt][c] - ks) * sb[buf][tt];
            float os = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                s[q] += kv[q] * delta;
                os += s[q] * qv[q];
            }
            os = group8_sum(os);
            if (r == 0) a.o[((size_t)(t0 + tt) * Hv + h) * D + j] = os;
        }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) st[(size_t)(i0 + e) * D + j] = f2bf(s[e]);
}

// Grid (token, value heads / 4): wave w takes value head 4 blockIdx.y + w (model.py:339-345).
__global__ __launch_bounds__(256) void gdn_prefill_finish_kernel(const PrefillGdnArgs a) {
    constexpr int D = 128;
    const int t = blockIdx.x, lane = threadIdx.x & 63, h = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int Hv = a.Hv;
    if (h >= Hv) return;
    const float o0 = rbf(a.o[((size_t)t * Hv + h) * D + lane]), o1 = rbf(a.o[((size_t)t * Hv + h) * D + lane + 64]);
    const float r = 1.0f / sqrtf(warp_sum(o0 * o0 + o1 * o1) / 128.0f + a.eps);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int jj = lane + half * 64;
        float hv = rbf((half ? o1 : o0) * r);
        hv = rbf(bf2f(a.norm_w[jj]) * hv);
        const float zf = bf2f(a.z[(size_t)t * Hv * D + h * D + jj]);
        a.act[act_offset(t, h * D + jj, Hv * D)] = (uint8_t)e5m2_byte(rbf(hv * (zf * sigmoidf_(zf))));
    }
}

// The row's new conv state (model.py:492-495): inputs n_valid .. n_valid + 2 of [history * keep, chunk].
__global__ __launch_bounds__(256) void gdn_prefill_carry_kernel(const PrefillGdnArgs a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.C) return;
    const int slot = *a.slot, n = *a.n_valid;
    if (slot < 0 || slot >= a.rows || n < 1 || n > a.L) return;
    const float keep = *a.start > 0 ? 1.0f : 0.0f;
    bf16_t* hist = a.conv + (size_t)slot * a.C * 3;
    float w[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) w[q] = conv_window(a, hist, keep, c, n + q);
#pragma unroll
    for (int q = 0; q < 3; ++q) hist[(size_t)c * 3 + q] = f2bf(w[q]);
}

namespace {

constexpr int QP = 256;  // bf16 per scaled query row in the scratch

__device__ __forceinline__ v8bf16 load8p(const bf16_t* p) { return *(const v8bf16*)p; }
__device__ __forceinline__ int drow(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

// Direct global -> LDS copy of one dword per lane from base + off (base wave-uniform, in scalar registers): lane l's 4
// bytes land at LDS address dst + 4 l (dst wave-uniform). Inline assembly, so the compiler neither counts it nor waits
// for it; the ring's own vmcnt waits below cover it.
__device__ __forceinline__ void lds_dword(const void* base, uint32_t off, uint32_t dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(dst);
    asm volatile("global_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(m0) : "memory");
}

// Wait until at most N of this wave's vector-memory operations are outstanding (its copies into the stage about to be
// read have landed) and its LDS reads have returned, then meet the other waves: after it the stage read one step
// before is free. The memory clobber keeps LDS reads after it.
template <int N>
__device__ __forceinline__ void ring_ready() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Every LDS read of this wave has returned; then meet the other waves, so the stage just read can be refilled.
__device__ __forceinline__ void ring_release() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS layout of one 32-position sub-block (E bytes per element), swizzled at the granularity the MFMA operand reads use
// so that they are free of bank conflicts, and filled by coalesced dword copies (each copy instruction of a wave takes
// 256 contiguous bytes of the cache, permuted within rows). The maps are their own inverses.
//   K [32 positions][256 dims]: bf16 16-byte chunk c of row r at chunk c ^ (r & 15); e4m3 8-byte chunk c at c ^ r.
//   V [256 dims][32 positions]: bf16 8-byte chunk c of row d at c ^ ((d >> 2) & 7); e4m3 4-byte chunk c at
//   c ^ (((d >> 3) & 3) << 1).
template <int E>
__device__ __forceinline__ uint32_t k_swz(uint32_t byte) {  // byte offset in the sub-block, either direction
    if constexpr (E == 2) {
        const uint32_t r = byte >> 9;
        return byte ^ ((r & 15) << 4);
    } else {
        const uint32_t r = byte >> 8;
        return byte ^ ((r & 31) << 3);
    }
}
template <int E>
__device__ __forceinline__ uint32_t v_swz(uint32_t byte) {
    if constexpr (E == 2) {
        const uint32_t d = byte >> 6;
        return byte ^ (((d >> 2) & 7) << 3);
    } else {
        const uint32_t d = byte >> 5;
        return byte ^ (((d >> 3) & 3) << 3);
    }
}

}  // namespace

// Grid (token): wave w normalises and rotates rows w, w + 4, ...: query heads (scaled by 1/16 into qs), then the KV
// heads' keys (into the cache) and values (into the cache, transposed per 32 positions), as e4m3 bytes of value / scale
// with KV8. Lane l holds dims 4l .. 4l+3.
template <bool KV8>
__global__ __launch_bounds__(256) void attn_prefill_prep_kernel(const PrefillAttnArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int Hq = a.Hq, Hkv = a.Hkv, S = a.S, d0 = lane * 4;
    const int slot = *a.slot, p = *a.start + t;
    if (slot < 0 || slot >= a.rows) return;
    const int rows = a.keys_only ? 2 * Hkv : Hq + 2 * Hkv;
    const float ksc = KV8 ? bf2f(*a.k_scale) : 0.0f, vsc = KV8 ? bf2f(*a.v_scale) : 0.0f;
    float cs[4], sn[4];
    {
        const uint2 rc = *(const uint2*)(a.cos + (size_t)t * 64 + (d0 & 63));
        const uint2 rsn = *(const uint2*)(a.sin + (size_t)t * 64 + (d0 & 63));
        cs[0] = lo_bf(rc.x); cs[1] = hi_bf(rc.x); cs[2] = lo_bf(rc.y); cs[3] = hi_bf(rc.y);
        sn[0] = lo_bf(rsn.x); sn[1] = hi_bf(rsn.x); sn[2] = lo_bf(rsn.y); sn[3] = hi_bf(rsn.y);
    }
    for (int r0 = wave; r0 < rows; r0 += 4) {
        const int r = a.keys_only ? Hq + r0 : r0;  // 0..Hq-1 query heads, then keys, then values
        const bf16_t* src = r < Hq ? a.qkv + (size_t)t * a.ld + (size_t)r * 512
                                   : a.qkv + (size_t)t * a.ld + a.kv_col + (size_t)(r - Hq) * 256;
        const uint2 raw = *(const uint2*)(src + d0);
        float v[4] = {lo_bf(raw.x), hi_bf(raw.x), lo_bf(raw.y), hi_bf(raw.y)};
        if (r >= Hq + Hkv) {  // a value: stored as is
            const int kvh = r - Hq - Hkv;
            if (p < S) {
                const size_t vo = (((size_t)slot * Hkv + kvh) * S + (p & ~31)) * 256 + (p & 31);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (KV8)
                        ((uint8_t*)a.v_cache)[vo + (size_t)(d0 + e) * 32] = (uint8_t)kv_code(v[e], vsc);
                    else
                        a.v_cache[vo + (size_t)(d0 + e) * 32] = f2bf(v[e]);
                }
            }
            continue;
        }
        const bf16_t* nw = r < Hq ? a.q_norm : a.k_norm;
        const float ss = warp_sum(v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3]);
        const float rsq = 1.0f / sqrtf(ss / 256.0f + a.eps);
        float hn[4], out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) hn[e] = rbf(v[e] * rsq * (1.0f + bf2f(nw[d0 + e])));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float part = __shfl_xor(hn[e], 8);
            const int d = d0 + e;
            out[e] = d < 64 ? rbf(rbf(hn[e] * cs[e]) + rbf((d < 32 ? -part : part) * sn[e])) : hn[e];
        }
        if (r < Hq) {
            *(uint2*)(a.qs + ((size_t)r * a.L + t) * QP + d0) =
                make_uint2(pk_bf16(out[0] * 0.0625f, out[1] * 0.0625f), pk_bf16(out[2] * 0.0625f, out[3] * 0.0625f));
        } else if (p < S) {
            const int kvh = r - Hq;
            const size_t ko = (((size_t)slot * Hkv + kvh) * S + p) * 256 + d0;
            if constexpr (KV8)
                *(uint32_t*)((uint8_t*)a.k_cache + ko) = kv_code(out[0], ksc) | kv_code(out[1], ksc) << 8 |
                                                         kv_code(out[2], ksc) << 16 | kv_code(out[3], ksc) << 24;
            else
                *(uint2*)(a.k_cache + ko) = make_uint2(pk_bf16(out[0], out[1]), pk_bf16(out[2], out[3]));
        }
    }
}

// Grid (query head, tiles of 128 tokens), four waves: wave w takes tokens T0 + 32 w .. + 31. The four waves see the
// same cached positions, so each sub-block of 32 positions is copied into LDS once per workgroup (a ring of three
// stages: the next two sub-blocks' copies are in flight while the current one is used, one barrier per sub-block) and
// read by all four.
// Scores by v_mfma_f32_32x32x16_bf16 with the keys as A (32 positions) and the queries as B (32 tokens): lane l holds
// token t0 + l % 32 and positions drow(i, l); MFMA step m takes dims 8 m .. 8 m + 7 in lanes 0-31 and 128 + 8 m .. in
// lanes 32-63 (the queries in the same order). The weights go straight from those registers into the A operand of
// weights x V (two MFMA steps of 16 positions: rows drow(0..7) and drow(8..15) of the lane), with V's B operand read in
// the same position order from the transposed sub-block. With KV8 the cached bytes (the chunk's own included, written by
// the prep kernel) widen to bf16(e4m3 x scale) as they are read from LDS. Every wave runs all of the workgroup's
// sub-blocks: those past its own tokens (at most three, on the diagonal, where the workgroup waits for its last wave
// anyway) hold chunk positions the prep kernel wrote, so they add weights of exactly zero times finite values, which
// leaves the sums as they were (none of them is -0: they start at +0). A block none of a wave's tokens sees leaves
// its state alone. The output so far stays in registers.
template <bool KV8>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const PrefillAttnArgs a) {
    constexpr int E = KV8 ? 1 : 2;        // bytes per cached element
    constexpr int SUB = 32 * 256 * E;     // bytes of one K (or V) sub-block
    constexpr int NCP = SUB / 1024;       // dword copies per wave per sub-block of one array
    __shared__ __attribute__((aligned(1024))) uint8_t ring[3][2][SUB];  // [stage][K, V]
    __shared__ float s_row[4][32];
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroups start in the order of their linear id, x fastest, and go to the XCDs in turn: the last (heaviest,
    // causally) tiles start first, and with 8 | Hq the query heads of one XCD are consecutive (one KV head's, when
    // G >= Hq / 8), so its L2 holds few KV heads' keys and values.
    const int T0 = (gridDim.y - 1 - blockIdx.y) * 128;
    const int hq = a.Hq % 8 ? blockIdx.x : (blockIdx.x % 8) * (a.Hq / 8) + blockIdx.x / 8;
    const int L = a.L, S = a.S, G = a.Hq / a.Hkv, kvh = hq / G, t0 = T0 + 32 * wv;
    const int slot = *a.slot, start = *a.start;
    if (start < 0 || start + L > S || slot < 0 || slot >= a.rows) return;  // the host checks these too
    const bool live = t0 < L;         // wave-uniform: the wave has tokens
    const int tq = t0 + (lane & 31);  // this lane's token (query)
    const size_t head = (size_t)slot * a.Hkv + kvh;
    const float ksc = KV8 ? bf2f(*a.k_scale) : 0.0f, vsc = KV8 ? bf2f(*a.v_scale) : 0.0f;
    const uint8_t* kg = (const uint8_t*)a.k_cache + head * S * 256 * E;
    const uint8_t* vg = (const uint8_t*)a.v_cache + head * S * 256 * E;
    const uint32_t lds0 = (uint32_t)(uintptr_t)LDS_PTR(&ring[0][0][0]);

    v8bf16 qf[16];
    if (live) {
        const bf16_t* qp = a.qs + ((size_t)hq * L + tq) * QP + (lane >> 5) * 128;
#pragma unroll
        for (int m = 0; m < 16; ++m) qf[m] = load8p(qp + m * 8);
    } else {
#pragma unroll
        for (int m = 0; m < 16; ++m)
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[m][e] = (__bf16)0.0f;
    }
    v16f so[8];  // output so far: so[db][i] is token drow(i, l), dim 32 db + l % 32
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) so[db][i] = 0.0f;
    float best = 2.0f * -1e4f, total = 0.0f;

    // This wave's dword copies of the sub-block at p0 into stage st: copy j of lane l fills LDS byte at + 4 l of the
    // stage, at = 256 (4 j + w), from the cache byte the swizzle maps there. A wave's 256 bytes lie in rows that share
    // one swizzle (K rows hold 256 or 512 bytes; V rows 64 or 32 bytes, in groups of 4 or 8 with one pattern), so that
    // byte is at + (4 l ^ X) with X = swz(at) ^ at uniform over the wave.
    auto copy = [&](int p0, int st, bool with_v) {
        const uint32_t dst = lds0 + (uint32_t)st * 2 * SUB;
        const uint8_t* ks = kg + (size_t)p0 * 256 * E;
#pragma unroll
        for (int j = 0; j < NCP; ++j) {
            const uint32_t at = (j * 4 + wv) * 256;
            lds_dword(ks + at, (uint32_t)(lane * 4) ^ (k_swz<E>(at) ^ at), dst + at);
        }
        if (with_v) {
            const uint8_t* vs = vg + (size_t)(p0 >> 5) * SUB;
#pragma unroll
            for (int j = 0; j < NCP; ++j) {
                const uint32_t at = (j * 4 + wv) * 256;
                lds_dword(vs + at, (uint32_t)(lane * 4) ^ (v_swz<E>(at) ^ at), dst + SUB + at);
            }
        }
    };
    // Scores of the sub-block in stage st against the wave's 32 tokens.
    auto score = [&](int st, v16f& acc) {
        const uint8_t* kl = &ring[st][0][0];
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            v8bf16 kf;
            if constexpr (KV8) {
                const uint2 r = *(const uint2*)(kl + k_swz<1>((lane & 31) * 256 + (lane >> 5) * 128 + m * 8));
                kf = kv_widen8(r.x, r.y, ksc);
            } else {
                kf = *(const v8bf16*)(kl + k_swz<2>((lane & 31) * 512 + (lane >> 5) * 256 + m * 16));
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[m], acc, 0, 0, 0);
        }
    };
    const int t_max = min(t0 + 31, L - 1), t_top = min(T0 + 127, L - 1);  // the wave's and the workgroup's last token
    const int nblocks = (S + L + 2047) / 2048;
    for (int b = 0; b < nblocks; ++b) {
        // Sub-blocks of 32 cache positions (aligned, as the transposed V cache is): the cached positions [c_lo, c_hi),
        // then the positions [p_lo, p_hi) the chunk's own tokens o_lo .. o_hi - 1 were written to. n counts the
        // workgroup's sub-blocks, nw this wave's (a prefix of them: the same positions in the same order).
        const int c_lo = 2048 * b, c_hi = min(min(2048 * (b + 1), S), start);
        const int o_lo = max(0, 2048 * b - S), o_end = min(2048 * (b + 1) - S, L);
        const int o_hi = min(o_end, t_max + 1), o_top = min(o_end, t_top + 1);
        const int p_lo = start + o_lo, p_hi = start + o_hi, p_al = p_lo & ~31;
        const int n_c = c_hi > c_lo ? (c_hi - c_lo + 31) / 32 : 0;
        const int n = n_c + (o_top > o_lo ? (start + o_top - p_al + 31) / 32 : 0);
        const int nw = live ? n_c + (o_hi > o_lo ? (p_hi - p_al + 31) / 32 : 0) : 0;
        if (n == 0) continue;
        auto base = [&](int sb) { return sb < n_c ? c_lo + 32 * sb : p_al + 32 * (sb - n_c); };
        // The rows r (positions base(sb) + r) of sub-block sb this lane's token sees: rlo <= r < rhi. Cached
        // positions below c_hi; the chunk's from p_lo, below p_hi and up to the token's own.
        auto window = [&](int sb, int& rlo, int& rhi) {
            const int p0 = base(sb);
            rlo = sb < n_c ? 0 : p_lo - p0;
            rhi = (sb < n_c ? c_hi : min(p_hi, start + tq + 1)) - p0;
        };
        // Pass 1: the block's maximum per token.
        float mx = -INFINITY;
        copy(base(0), 0, false);
        if (n > 1) copy(base(1), 1, false);
        for (int sb = 0, st = 0; sb < n; ++sb, st = st == 2 ? 0 : st + 1) {
            if (sb + 1 < n)
                ring_ready<NCP>();
            else
                ring_ready<0>();
            if (sb + 2 < n) copy(base(sb + 2), st == 0 ? 2 : st - 1, false);
            v16f acc;
            score(st, acc);
            int rlo, rhi;
            window(sb, rlo, rhi);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = drow(i, lane);
                mx = ((r >= rlo) & (r < rhi)) ? fmaxf(mx, rbf(acc[i])) : mx;
            }
        }
        ring_release();
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float nb = fmaxf(best, mx);  // a token with nothing visible here keeps its maximum
        const float scale = expf(best - nb);
        // Pass 2: weights e^(s - max), their float32 sum, bf16 weights x V.
        v16f pv[8];
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) pv[db][i] = 0.0f;
        float wsum = 0.0f;
        copy(base(0), 0, true);
        if (n > 1) copy(base(1), 1, true);
        for (int sb = 0, st = 0; sb < n; ++sb, st = st == 2 ? 0 : st + 1) {
            if (sb + 1 < n)
                ring_ready<2 * NCP>();
            else
                ring_ready<0>();
            if (sb + 2 < n) copy(base(sb + 2), st == 0 ? 2 : st - 1, true);
            {
                v16f acc;
                score(st, acc);
                int rlo, rhi;
                window(sb, rlo, rhi);
                float w[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int r = drow(i, lane);
                    const float e = expf(rbf(acc[i]) - nb);
                    w[i] = ((r >= rlo) & (r < rhi)) ? e : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) wsum += w[i];
                const uint8_t* vl = &ring[st][1][0];
                typedef unsigned u4_ __attribute__((ext_vector_type(4)));
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const u4_ pw = {pk_bf16(w[8 * ks + 0], w[8 * ks + 1]), pk_bf16(w[8 * ks + 2], w[8 * ks + 3]),
                                    pk_bf16(w[8 * ks + 4], w[8 * ks + 5]), pk_bf16(w[8 * ks + 6], w[8 * ks + 7])};
                    const v8bf16 pa = __builtin_bit_cast(v8bf16, pw);
                    // Positions of this step in this lane: 16 ks + 4 (l / 32) + [0, 4) and 16 ks + 8 + 4 (l / 32) + [0, 4).
                    const int q0 = 16 * ks + 4 * (lane >> 5);
#pragma unroll
                    for (int db = 0; db < 8; ++db) {
                        const int d = db * 32 + (lane & 31);
                        v8bf16 vw;
                        if constexpr (KV8) {
                            const uint32_t lo = *(const uint32_t*)(vl + v_swz<1>(d * 32 + q0));
                            const uint32_t hi = *(const uint32_t*)(vl + v_swz<1>(d * 32 + q0 + 8));
                            vw = kv_widen8(lo, hi, vsc);
                        } else {
                            const uint2 lo = *(const uint2*)(vl + v_swz<2>(d * 64 + q0 * 2));
                            const uint2 hi = *(const uint2*)(vl + v_swz<2>(d * 64 + q0 * 2 + 16));
                            vw = __builtin_bit_cast(v8bf16, (u4_){lo.x, lo.y, hi.x, hi.y});
                        }
                        pv[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa, vw, pv[db], 0, 0, 0);
                    }
                }
            }
        }
        ring_release();
        if (nw == 0) continue;  // nothing of this block is visible to the wave: it keeps its state
        wsum += __shfl_xor(wsum, 32);
        total = total * scale + wsum;
        best = nb;
        if (lane < 32) s_row[wv][lane] = scale;
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes land before its reads
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) so[db][i] = so[db][i] * s_row[wv][drow(i, lane)] + rbf(pv[db][i]);
    }
    // out / total in bf16, times bf16 sigmoid(gate), e5m2 tiles for o_proj.
    if (!live) return;
    if (lane < 32) s_row[wv][lane] = total;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    const int act_k = a.Hq * 256;
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = drow(i, lane), d = db * 32 + (lane & 31), t = t0 + row;
            if (t >= L) continue;
            const float o = rbf(so[db][i] / s_row[wv][row]);
            const float gt = bf2f(a.qkv[(size_t)t * a.ld + (size_t)hq * 512 + 256 + d]);
            a.act[act_offset(t, hq * 256 + d, act_k)] = (uint8_t)e5m2_byte(rbf(o * rbf(sigmoidf_(gt))));
        }
}

hipError_t q38_attn_prefill(const PrefillAttnArgs& a, hipStream_t stream) {
    if (a.L < 1 || a.L % 32 || a.Hq % a.Hkv || a.S % 32) return hipErrorInvalidValue;
    if (a.kv8) {
        if (!a.k_scale || !a.v_scale) return hipErrorInvalidValue;
        hipLaunchKernelGGL(attn_prefill_prep_kernel<true>, dim3(a.L), dim3(256), 0, stream, a);
        if (!a.keys_only) hipLaunchKernelGGL(attn_prefill_kernel<true>, dim3(a.Hq, (a.L + 127) / 128), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(attn_prefill_prep_kernel<false>, dim3(a.L), dim3(256), 0, stream, a);
        if (!a.keys_only) hipLaunchKernelGGL(attn_prefill_kernel<false>, dim3(a.Hq, (a.L + 127) / 128), dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t q38_gdn_prefill(const PrefillGdnArgs& a, hipStream_t stream) {
    if (a.L < 1 || a.gate_groups < 1 || a.gate_groups > 8 || a.Hv % a.Hk || a.Hv % 4 || a.C != 2 * a.Hk * 128 + a.Hv * 128)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_prefill_prep_kernel, dim3(a.L, a.Hk), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(gdn_prefill_scan_kernel, dim3(a.Hv, 4), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(gdn_prefill_finish_kernel, dim3(a.L, a.Hv / 4), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(gdn_prefill_carry_kernel, dim3((a.C + 255) / 256), dim3(256), 0, stream, a);
    return hipGetLastError();
}
