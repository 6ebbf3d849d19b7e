// Host side of libq38: the C ABI declared in include/q38.h. It validates shapes, keeps the bound buffers of one loaded
// model and sequences the kernels of a verify step, an MTP step and the head on the caller's stream. It allocates no
// device memory.
//
// Per layer of a verify step (reference DecoderLayer.forward, qwen38_inf2/model.py:918-930):
//   gated delta:  qkvz GEMM -> gates -> gdn_verify -> out_proj GEMM (split-K) -> residual + post-norm
//   attention:    qkv GEMM -> attn_verify -> o_proj GEMM (split-K) -> residual + post-norm
//   MLP:          gate/up GEMM with SwiGLU epilogue -> down GEMM (split-K) -> residual + next layer's input norm
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../../include/q38.h"
#include "kernels.h"

namespace {

thread_local std::string g_error;

int fail(const std::string& msg) {
    g_error = msg;
    return 1;
}

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess) return fail(std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

struct Buf {
    void* p = nullptr;
    size_t n = 0;
};

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Token counts padded the way the GEMMs tile them: 32, 64, 128, then multiples of 256.
int pad_tokens(int t) {
    if (t <= 32) return 32;
    if (t <= 64) return 64;
    if (t <= 128) return 128;
    return (t + 255) / 256 * 256;
}

// Compute units of the current device (the GEMMs run one persistent workgroup per CU); 256 (MI355X) when no device
// answers, as on a build host.
int device_cus() {
    static int cus = 0;
    if (cus) return cus;
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n > 0)
        cus = n;
    else {
        (void)hipGetLastError();
        cus = 256;
    }
    return cus;
}

// GEMM scratch behind the activation tiles: stream-K arrival counters, then partial slots.
size_t gemm_scratch_bytes(int cus) { return (size_t)GEMM_COUNTERS * 8 + (size_t)2 * cus * GEMM_SLOT_FLOATS * 4; }

void gemm_scratch(GemmArgs& a, uint8_t* base, int cus) {
    a.counters = (unsigned long long*)base;
    a.counters_n = GEMM_COUNTERS;
    a.fix = (float*)(base + (size_t)GEMM_COUNTERS * 8);
    a.fix_floats = (size_t)2 * cus * GEMM_SLOT_FLOATS;
    a.cus = cus;
}

}  // namespace

static constexpr int TIMER_PAIRS = 4096;  // gate/up GEMM launches q38_kernel_timer can bracket

struct q38_handle {
    q38_config cfg;
    int H, I, V, B, K, S, T, Tpad;
    int Hq, Hkv, hd, Hk, Hv, dk, C;
    int cus;
    std::vector<std::map<std::string, Buf>> layer;  // num_layers + 1 (the MTP layer)
    std::map<std::string, Buf> global;
    int parity = 0;
    // workspace carve-up
    size_t off_x, off_hbf, off_tmp, off_act_h, off_act_mid, off_act_ffn, off_z, off_qkv, off_part,
        off_scores, off_astats, off_aown, off_akv, off_aq, off_apv, off_apr, off_htiles, off_x32, off_maxima, off_sp_embeds, off_sp_cos,
        off_sp_sin, off_sp_states, off_sp_out, off_sp_current, off_sp_ids, off_sp_at, off_sp_draft, off_gemm, off_gates, off_status,
        workspace_bytes;
    // prefill scratch (with a prefill chunk in the config)
    size_t off_pqn = 0, off_pkn = 0, off_pv = 0, off_po = 0, off_pbeta = 0, off_pg = 0, off_pqs = 0;
    size_t part_floats;  // capacity of the split-K partial buffer
    int gate_groups;  // K ranges of the gated-delta gate projections
    int attn_nchunks;  // chunks of ATTN_CHUNK cached positions over S
    size_t attn_pv_floats;  // capacity of the chunked attention's split sums
    // Kernel timer (q38_kernel_timer): event pairs around the gate/up GEMM launches while on.
    std::vector<hipEvent_t> timer_events;
    int timer_used = 0;
    bool timer_on = false;
    int act_h_k;  // width of act_h: 2H with the MTP layer (its fc input), else H
    // q38_spec_step_graph: the step captured once per gated-delta parity (the two halves give different kernel
    // arguments), for the argument pointers it was captured with; a private stream to capture on.
    struct StepGraph {
        hipGraphExec_t exec = nullptr;
        const void* args[8] = {};
    } graphs[2];
    hipStream_t capture_stream = nullptr;
    // A second stream for work that can run beside the main chain (a gated-delta layer's gate projections beside its
    // qkvz GEMM), forked and joined with the two events; made when the workspace is bound.
    hipStream_t side_stream = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;

    uint8_t* ws(size_t off) const { return (uint8_t*)global.at("workspace").p + off; }
    void drop_graphs() {
        for (StepGraph& g : graphs) {
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
            g = StepGraph{};
        }
    }
};

namespace {

bool is_linear(const q38_handle* h, int layer) { return layer < h->cfg.num_layers && h->cfg.layer_types[layer] == Q38_LINEAR; }

// Whether a layer's projections are bound as MXFP4 tiles: the decoder layers of an MXFP4 checkpoint. The MTP layer and
// the head come as bf16 in that checkpoint and are always e4m3.
bool fp4_layer(const q38_handle* h, int layer) {
    return h->cfg.weight_format == Q38_WEIGHTS_MXFP4 && layer >= 0 && layer < h->cfg.num_layers;
}

// The optional per-layer probe a verify call fills when it is bound, for the step's T = B*K tokens: as bf16, the
// layer's normed input [T][H] (gated-delta layers; left as it is for attention layers), the mixer's projection output
// [T][P] (the gated-delta in_proj_z part, P = Hv*dk, or the attention q|gate|k|v projection, P = Hq*hd*2 + 2*Hkv*hd),
// the gated-delta in-step output before its gated norm [T][Hv*dk] (gated-delta layers only), and the residual stream
// after the mixer [T][H]; then, as the e5m2 activation tiles the GEMMs read (for the first T32 = T rounded up to 32
// tokens), the out_proj input (M = Hv*dk or Hq*hd inputs), the MLP input (H) and the down projection's input (I). For
// comparing the layer stage by stage against another implementation; a verify call with no probe bound does no extra
// work. Last, as bf16 [T][H], the residual stream entering the layer (its input). The MTP layer (index num_layers)
// takes a probe too, filled by q38_mtp_step: its layer input is the fc output.
size_t probe_width(const q38_handle* h, int layer) {
    return is_linear(h, layer) ? (size_t)h->Hv * h->dk : (size_t)h->Hq * h->hd * 2 + 2 * (size_t)h->Hkv * h->hd;
}

size_t probe_mid(const q38_handle* h, int layer) { return is_linear(h, layer) ? (size_t)h->Hv * h->dk : (size_t)h->Hq * h->hd; }

size_t probe_inner(const q38_handle* h, int layer) { return is_linear(h, layer) ? (size_t)h->Hv * h->dk : 0; }

size_t probe_tiles_at(const q38_handle* h, int layer) {
    const size_t T = (size_t)h->cfg.batch_size * h->cfg.verify_tokens;
    return T * (2 * (size_t)h->H + probe_width(h, layer) + probe_inner(h, layer)) * 2;
}

size_t probe_input_at(const q38_handle* h, int layer) {
    const size_t T32 = ((size_t)h->cfg.batch_size * h->cfg.verify_tokens + 31) / 32 * 32;
    return probe_tiles_at(h, layer) + T32 * (probe_mid(h, layer) + h->H + h->I);
}

size_t probe_bytes(const q38_handle* h, int layer) {
    return probe_input_at(h, layer) + (size_t)h->cfg.batch_size * h->cfg.verify_tokens * h->H * 2;
}

// Layers that take a probe: the decoder layers and, when present, the MTP layer.
bool probed_layer(const q38_handle* h, int layer) { return layer < h->cfg.num_layers || (h->cfg.mtp && layer == h->cfg.num_layers); }

uint16_t* probe_of(q38_handle* h, int layer) {
    auto it = h->layer[layer].find("probe");
    return it == h->layer[layer].end() ? nullptr : (uint16_t*)it->second.p;
}

// Expected size of a named buffer, or 0 if the name does not exist for that layer.
size_t expected_size(const q38_handle* h, const std::string& name, int layer) {
    const size_t H = h->H, I = h->I, V = h->V, B = h->B, K = h->K, S = h->S;
    const size_t Hq = h->Hq, Hkv = h->Hkv, hd = h->hd, Hk = h->Hk, Hv = h->Hv, dk = h->dk, C = h->C;
    auto fp8 = [&](const std::string& base, size_t n, size_t k) -> size_t {
        if (name == base + ".tiles") return fp4_layer(h, layer) ? n * k / 2 : n * k;
        if (name == base + ".scales") return n * k / 32;
        return 0;
    };
    size_t r;
    if (layer == -1) {
        if (name == "head.norm") return H * 2;
        if ((r = fp8("head.lm_head", V, H))) return r;
        if (name == "head.lm_head.rows") return V * H * 2;
        if (name == "head.probe") return (B * K + 31) / 32 * 32 * H * 2;
        if (name == "embed_tokens") return V * H * 2;
        if (name == "rope_table") return S * 2 * 64 * 2;
        if (name == "workspace") return h->workspace_bytes;
        return 0;
    }
    if (layer < 0 || layer > h->cfg.num_layers) return 0;
    if (layer == h->cfg.num_layers && !h->cfg.mtp) return 0;
    if (name == "input_layernorm" || name == "post_attention_layernorm") return H * 2;
    if (name == "probe") return probe_bytes(h, layer);
    if ((r = fp8("mlp.gate_up", 2 * I, H))) return r;
    if ((r = fp8("mlp.down", H, I))) return r;
    if (is_linear(h, layer)) {
        if ((r = fp8("linear_attn.in_proj_qkvz", C + Hv * dk, H))) return r;
        if ((r = fp8("linear_attn.out_proj", H, Hv * dk))) return r;
        if (name == "linear_attn.in_proj_a" || name == "linear_attn.in_proj_b") return Hv * H * 2;
        if (name == "linear_attn.conv_weight") return C * 4 * 2;
        if (name == "linear_attn.A_log" || name == "linear_attn.dt_bias") return Hv * 2;
        if (name == "linear_attn.norm_weight") return dk * 2;
        if (name == "linear_attn.recurrent_state") return B * Hv * dk * dk * 2;
        if (name == "linear_attn.conv_state") return 2 * B * C * 3 * 2;
        if (name == "linear_attn.pending_key") return 2 * B * K * Hk * dk * 4;
        if (name == "linear_attn.pending_delta") return 2 * B * K * Hv * dk * 4;
        if (name == "linear_attn.pending_decay") return 2 * B * K * Hv * 4;
        if (name == "linear_attn.pending_input") return 2 * B * K * C * 2;
        if (h->cfg.saved_states && name == "linear_attn.saved_state") return B * Hv * dk * dk * 2;
        if (h->cfg.saved_states && name == "linear_attn.saved_conv") return B * C * 3 * 2;
        return 0;
    }
    if ((r = fp8("self_attn.qkv", Hq * hd * 2 + 2 * Hkv * hd, H))) return r;
    if ((r = fp8("self_attn.o_proj", H, Hq * hd))) return r;
    if (name == "self_attn.q_norm" || name == "self_attn.k_norm") return hd * 2;
    const bool kv8 = h->cfg.kv_cache_format == Q38_KV_FP8;
    if (name == "self_attn.k_cache" || name == "self_attn.v_cache") return B * Hkv * S * hd * (kv8 ? 1 : 2);
    if (kv8 && (name == "self_attn.k_scale" || name == "self_attn.v_scale")) return 2;
    if (layer == h->cfg.num_layers) {
        if ((r = fp8("mtp.fc", H, 2 * H))) return r;
        if (name == "mtp.embedding_norm" || name == "mtp.hidden_norm" || name == "mtp.norm") return H * 2;
    }
    return 0;
}

// Pointer of a bound buffer; sets the error and returns null when it was never bound.
template <typename T>
T* get(q38_handle* h, const std::string& name, int layer, bool* ok) {
    const auto& m = layer < 0 ? h->global : h->layer[layer];
    auto it = m.find(name);
    if (it == m.end() || !it->second.p) {
        if (*ok) g_error = "buffer '" + name + "' of layer " + std::to_string(layer) + " is not bound";
        *ok = false;
        return nullptr;
    }
    return (T*)it->second.p;
}

// A projection of layer li (its weight format decides the GEMM variant).
int gemm(q38_handle* h, int li, const uint8_t* tiles, const uint8_t* scales, const uint8_t* act, int K, int N, int epi,
         void* out0, int ld0, int n0, void* out1, int ld1, hipStream_t stream, int* splits_out = nullptr) {
    if (N % 256 || K % 256) return fail("GEMM shape N=" + std::to_string(N) + " K=" + std::to_string(K) + " not tileable");
    GemmArgs a{};
    a.w = tiles;
    a.w4 = fp4_layer(h, li);
    a.f8 = !a.w4 && h->cfg.projection_mfma == Q38_MFMA_FP8;
    a.ws = scales;
    a.act = act;
    a.K = K;
    a.N = N;
    a.T = h->T;
    a.Tpad = h->Tpad;
    a.out0 = out0;
    a.ld0 = ld0;
    a.n0 = n0;
    a.out1 = out1;
    a.ld1 = ld1;
    if (epi == EPI_PARTIAL) {
        a.part = (float*)h->ws(h->off_part);
        a.splits_max = (int)std::max<size_t>(1, h->part_floats / ((size_t)h->Tpad * N));
    }
    gemm_scratch(a, h->ws(h->off_gemm), h->cus);
    int splits = 1;
    HIP_TRY(q38_gemm(a, epi, &splits, stream));
    if (splits_out) *splits_out = splits;
    return 0;
}

int norm_rows(q38_handle* h, const float* part, int splits, const uint16_t* xin, const uint16_t* resid, uint16_t* xout,
              const uint16_t* w, uint8_t* act, int kact, int col0, uint16_t* hout, const uint16_t* div_w, hipStream_t stream) {
    NormArgs a{};
    a.part = part;
    a.splits = splits;
    a.Tpad = h->Tpad;
    a.xin = xin;
    a.resid = resid;
    a.xout = xout;
    a.w = w;
    a.eps = h->cfg.rms_norm_eps;
    a.act = act;
    a.Kact = kact;
    a.act_col0 = col0;
    a.hout = hout;
    a.div_w = div_w;
    a.H = h->H;
    a.T = h->T;
    HIP_TRY(q38_residual_norm(a, stream));
    return 0;
}

struct StepIO {
    const uint16_t* cos;
    const uint16_t* sin;
    const int32_t* position;
    const float* active;
    const int32_t* accepted;
    bool decode = false;  // one token per row, the gated-delta layers' recurrent form
    const int32_t* slot = nullptr;  // prefill: one chunk of row *slot from position *start, *n_valid real tokens
    const int32_t* start = nullptr;
    const int32_t* n_valid = nullptr;
};

// Tokens per row of the call in progress: the verify width by default, 1 for a decode step (restored on exit).
struct TokensScope {
    q38_handle* h;
    int K, T, Tpad;
    TokensScope(q38_handle* h_, int k, int t = 0) : h(h_), K(h_->K), T(h_->T), Tpad(h_->Tpad) {
        h->K = k;
        h->T = t ? t : h->B * k;
        h->Tpad = pad_tokens(h->T);
    }
    ~TokensScope() {
        h->K = K;
        h->T = T;
        h->Tpad = Tpad;
    }
};

// Mixer of layer `li` on act_h; leaves x += mixer and act_h = e5m2(post_attention_layernorm(x)).
int run_mixer(q38_handle* h, int li, const StepIO& io, int rd, int wr, hipStream_t stream) {
    bool ok = true;
    const int H = h->H;
    uint16_t* probe = probed_layer(h, li) ? probe_of(h, li) : nullptr;
    uint8_t* act_h = h->ws(h->off_act_h);
    uint8_t* act_mid = h->ws(h->off_act_mid);
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    int splits, kmid;
    if (probe && !io.decode && !io.slot)
        HIP_TRY(hipMemcpyAsync((uint8_t*)probe + probe_input_at(h, li), x, (size_t)h->T * H * 2, hipMemcpyDeviceToDevice, stream));
    const uint8_t* otiles;
    const uint8_t* oscales;
    if (is_linear(h, li)) {
        auto qkvz_t = get<uint8_t>(h, "linear_attn.in_proj_qkvz.tiles", li, &ok);
        auto qkvz_s = get<uint8_t>(h, "linear_attn.in_proj_qkvz.scales", li, &ok);
        auto pin = get<uint16_t>(h, "linear_attn.pending_input", li, &ok);
        auto wa = get<uint16_t>(h, "linear_attn.in_proj_a", li, &ok);
        auto wb = get<uint16_t>(h, "linear_attn.in_proj_b", li, &ok);
        auto alog = get<uint16_t>(h, "linear_attn.A_log", li, &ok);
        auto dtb = get<uint16_t>(h, "linear_attn.dt_bias", li, &ok);
        auto convw = get<uint16_t>(h, "linear_attn.conv_weight", li, &ok);
        auto normw = get<uint16_t>(h, "linear_attn.norm_weight", li, &ok);
        auto state = get<uint16_t>(h, "linear_attn.recurrent_state", li, &ok);
        auto conv = get<uint16_t>(h, "linear_attn.conv_state", li, &ok);
        auto pkey = get<float>(h, "linear_attn.pending_key", li, &ok);
        auto pdelta = get<float>(h, "linear_attn.pending_delta", li, &ok);
        auto pdecay = get<float>(h, "linear_attn.pending_decay", li, &ok);
        otiles = get<uint8_t>(h, "linear_attn.out_proj.tiles", li, &ok);
        oscales = get<uint8_t>(h, "linear_attn.out_proj.scales", li, &ok);
        if (!ok) return 1;
        const size_t BKC = (size_t)h->B * h->K * h->C;
        uint16_t* z = (uint16_t*)h->ws(h->off_z);
        // A verify step's qkv output is also its pending input snapshot; a decode step's or a prefill chunk's goes to
        // scratch.
        uint16_t* qkv_out = io.decode || io.slot ? (uint16_t*)h->ws(h->off_qkv) : pin + wr * BKC;
        // The gate projections (x . in_proj_b, x . in_proj_a) read only the normed input: they run on the side stream
        // beside the qkvz GEMM, whose persistent workgroups leave room for theirs on every CU.
        GatesArgs ga{};
        ga.x = (const bf16_t*)h->ws(h->off_hbf);
        ga.wb = wb;
        ga.wa = wa;
        ga.T = h->T;
        ga.H = H;
        ga.Hv = h->Hv;
        ga.groups = h->gate_groups;
        ga.part = (float*)h->ws(h->off_gates);
        const bool fork = h->side_stream != nullptr;
        if (fork) {
            HIP_TRY(hipEventRecord(h->fork_ev, stream));
            HIP_TRY(hipStreamWaitEvent(h->side_stream, h->fork_ev, 0));
            HIP_TRY(q38_gdn_gates(ga, h->side_stream));
            HIP_TRY(hipEventRecord(h->join_ev, h->side_stream));
        } else {
            HIP_TRY(q38_gdn_gates(ga, stream));
        }
        if (gemm(h, li, qkvz_t, qkvz_s, act_h, H, h->C + h->Hv * h->dk, EPI_BF16, qkv_out, h->C, h->C, z, h->Hv * h->dk, stream))
            return 1;
        if (fork) HIP_TRY(hipStreamWaitEvent(stream, h->join_ev, 0));
        if (probe && !io.decode && !io.slot) {
            HIP_TRY(hipMemcpyAsync(probe, h->ws(h->off_hbf), (size_t)h->T * H * 2, hipMemcpyDeviceToDevice, stream));
            HIP_TRY(hipMemcpyAsync(probe + (size_t)h->T * H, z, (size_t)h->T * h->Hv * h->dk * 2, hipMemcpyDeviceToDevice, stream));
        }
        if (io.slot) {
            PrefillGdnArgs p{};
            p.L = h->T;
            p.rows = h->B;
            p.Hk = h->Hk;
            p.Hv = h->Hv;
            p.C = h->C;
            p.slot = io.slot;
            p.start = io.start;
            p.n_valid = io.n_valid;
            p.qkv = qkv_out;
            p.z = z;
            p.gate_part = ga.part;
            p.gate_groups = ga.groups;
            p.a_log = alog;
            p.dt_bias = dtb;
            p.conv_w = convw;
            p.norm_w = normw;
            p.state = state;
            p.conv = conv + (size_t)rd * h->B * h->C * 3;  // the current half, in place
            p.qn = (float*)h->ws(h->off_pqn);
            p.kn = (float*)h->ws(h->off_pkn);
            p.v = (float*)h->ws(h->off_pv);
            p.beta = (float*)h->ws(h->off_pbeta);
            p.g = (float*)h->ws(h->off_pg);
            p.o = (float*)h->ws(h->off_po);
            p.act = act_mid;
            p.eps = h->cfg.rms_norm_eps;
            HIP_TRY(q38_gdn_prefill(p, stream));
            kmid = h->Hv * h->dk;
            goto out_proj;
        }
        {
        GdnArgs g{};
        g.B = h->B;
        g.K = h->K;
        g.Hk = h->Hk;
        g.Hv = h->Hv;
        g.C = h->C;
        g.qkv_new = qkv_out;
        g.qkv_old = pin + rd * BKC;
        g.z = z;
        g.gate_part = ga.part;
        g.gate_groups = ga.groups;
        g.a_log = alog;
        g.dt_bias = dtb;
        g.conv_w = convw;
        g.norm_w = normw;
        g.position = io.position;
        g.active = io.active;
        g.accepted = io.accepted;
        g.state = state;
        const size_t convn = (size_t)h->B * h->C * 3, keyn = (size_t)h->B * h->K * h->Hk * h->dk,
                     deltan = (size_t)h->B * h->K * h->Hv * h->dk, decayn = (size_t)h->B * h->K * h->Hv;
        g.conv_old = conv + rd * convn;
        g.conv_new = conv + wr * convn;
        g.key_old = pkey + rd * keyn;
        g.key_new = pkey + wr * keyn;
        g.delta_old = pdelta + rd * deltan;
        g.delta_new = pdelta + wr * deltan;
        g.decay_old = pdecay + rd * decayn;
        g.decay_new = pdecay + wr * decayn;
        g.act = act_mid;
        g.eps = h->cfg.rms_norm_eps;
        g.out_probe = probe && !io.decode ? (bf16_t*)probe + (size_t)h->T * (H + h->Hv * h->dk) : nullptr;
        HIP_TRY(io.decode ? q38_gdn_decode(g, stream) : q38_gdn_verify(g, stream));
        kmid = h->Hv * h->dk;
        }
    } else {
        auto qkv_t = get<uint8_t>(h, "self_attn.qkv.tiles", li, &ok);
        auto qkv_s = get<uint8_t>(h, "self_attn.qkv.scales", li, &ok);
        auto qn = get<uint16_t>(h, "self_attn.q_norm", li, &ok);
        auto kn = get<uint16_t>(h, "self_attn.k_norm", li, &ok);
        auto kc = get<uint16_t>(h, "self_attn.k_cache", li, &ok);
        auto vc = get<uint16_t>(h, "self_attn.v_cache", li, &ok);
        const bool kv8 = h->cfg.kv_cache_format == Q38_KV_FP8;
        const uint16_t* ks = kv8 ? get<uint16_t>(h, "self_attn.k_scale", li, &ok) : nullptr;
        const uint16_t* vs = kv8 ? get<uint16_t>(h, "self_attn.v_scale", li, &ok) : nullptr;
        otiles = get<uint8_t>(h, "self_attn.o_proj.tiles", li, &ok);
        oscales = get<uint8_t>(h, "self_attn.o_proj.scales", li, &ok);
        if (!ok) return 1;
        const int nqkv = h->Hq * h->hd * 2 + 2 * h->Hkv * h->hd;
        uint16_t* qkv = (uint16_t*)h->ws(h->off_qkv);
        if (gemm(h, li, qkv_t, qkv_s, act_h, H, nqkv, EPI_BF16, qkv, nqkv, nqkv, nullptr, 0, stream)) return 1;
        if (probe && !io.decode && !io.slot)
            HIP_TRY(hipMemcpyAsync(probe + (size_t)h->T * H, qkv, (size_t)h->T * nqkv * 2, hipMemcpyDeviceToDevice, stream));
        if (io.slot) {
            PrefillAttnArgs p{};
            p.L = h->T;
            p.rows = h->B;
            p.Hq = h->Hq;
            p.Hkv = h->Hkv;
            p.S = h->S;
            p.slot = io.slot;
            p.start = io.start;
            p.qkv = qkv;
            p.ld = nqkv;
            p.kv_col = h->Hq * h->hd * 2;
            p.q_norm = qn;
            p.k_norm = kn;
            p.cos = io.cos;
            p.sin = io.sin;
            p.k_cache = kc;
            p.v_cache = vc;
            p.kv8 = kv8;
            p.k_scale = ks;
            p.v_scale = vs;
            p.qs = (uint16_t*)h->ws(h->off_pqs);
            p.act = act_mid;
            p.eps = h->cfg.rms_norm_eps;
            HIP_TRY(q38_attn_prefill(p, stream));
            kmid = h->Hq * h->hd;
            goto out_proj;
        }
        AttnArgs a{};
        a.B = h->B;
        a.K = h->K;
        a.Hq = h->Hq;
        a.Hkv = h->Hkv;
        a.S = h->S;
        a.qkv = qkv;
        a.ld = nqkv;
        a.q_norm = qn;
        a.k_norm = kn;
        a.cos = io.cos;
        a.sin = io.sin;
        a.position = io.position;
        a.active = io.active;
        a.k_cache = kc;
        a.v_cache = vc;
        a.kv8 = kv8;
        a.k_scale = ks;
        a.v_scale = vs;
        a.nchunks = h->attn_nchunks;
        a.scores = (bf16_t*)h->ws(h->off_scores);
        a.stats = (float*)h->ws(h->off_astats);
        a.own = (float*)h->ws(h->off_aown);
        a.kv_own = (float*)h->ws(h->off_akv);
        a.qprep = (bf16_t*)h->ws(h->off_aq);
        a.pv_part = (float*)h->ws(h->off_apv);
        a.pv_part_floats = h->attn_pv_floats;
        a.pv_rows = (float*)h->ws(h->off_apr);
        a.cus = device_cus();
        a.act = act_mid;
        a.eps = h->cfg.rms_norm_eps;
        HIP_TRY(q38_attn_verify(a, stream));
        kmid = h->Hq * h->hd;
    }
out_proj:
    if (probe && !io.decode && !io.slot)
        HIP_TRY(hipMemcpyAsync((uint8_t*)probe + probe_tiles_at(h, li), act_mid, (size_t)(h->T + 31) / 32 * 32 * kmid,
                               hipMemcpyDeviceToDevice, stream));
    // x += o_proj(mixer): split-K partials, then residual add and the post-mixer norm in one row kernel.
    if (gemm(h, li, otiles, oscales, act_mid, kmid, H, EPI_PARTIAL, nullptr, 0, 0, nullptr, 0, stream, &splits)) return 1;
    auto post = get<uint16_t>(h, "post_attention_layernorm", li, &ok);
    if (!ok) return 1;
    if (norm_rows(h, (const float*)h->ws(h->off_part), splits, nullptr, x, x, post, act_h, H, 0, nullptr, nullptr, stream)) return 1;
    if (probe && !io.decode && !io.slot)
        HIP_TRY(hipMemcpyAsync(probe + (size_t)h->T * (H + probe_width(h, li) + probe_inner(h, li)), x, (size_t)h->T * H * 2,
                               hipMemcpyDeviceToDevice, stream));
    return 0;
}

// MLP of layer `li` on act_h, then the residual; `next` is the following layer (its input norm is fused), or -1 for
// the last layer, whose x goes to `final_out` (or, with `tail_norm`, the MTP output tail).
int run_mlp(q38_handle* h, int li, int next, uint16_t* final_out, bool mtp_tail, hipStream_t stream) {
    bool ok = true;
    const int H = h->H, I = h->I;
    auto gu_t = get<uint8_t>(h, "mlp.gate_up.tiles", li, &ok);
    auto gu_s = get<uint8_t>(h, "mlp.gate_up.scales", li, &ok);
    auto dn_t = get<uint8_t>(h, "mlp.down.tiles", li, &ok);
    auto dn_s = get<uint8_t>(h, "mlp.down.scales", li, &ok);
    if (!ok) return 1;
    uint8_t* act_h = h->ws(h->off_act_h);
    uint8_t* act_ffn = h->ws(h->off_act_ffn);
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    hipEvent_t* timed = h->timer_on && h->timer_used < TIMER_PAIRS ? &h->timer_events[2 * h->timer_used++] : nullptr;
    if (timed) HIP_TRY(hipEventRecord(timed[0], stream));
    if (gemm(h, li, gu_t, gu_s, act_h, H, 2 * I, EPI_SWIGLU, act_ffn, 0, 0, nullptr, 0, stream)) return 1;
    if (timed) HIP_TRY(hipEventRecord(timed[1], stream));
    uint8_t* probe = probed_layer(h, li) && h->T == h->cfg.batch_size * h->cfg.verify_tokens ? (uint8_t*)probe_of(h, li) : nullptr;
    if (probe) {
        const size_t t32 = (size_t)(h->T + 31) / 32 * 32, at = probe_tiles_at(h, li) + t32 * probe_mid(h, li);
        HIP_TRY(hipMemcpyAsync(probe + at, act_h, t32 * H, hipMemcpyDeviceToDevice, stream));
        HIP_TRY(hipMemcpyAsync(probe + at + t32 * H, act_ffn, t32 * I, hipMemcpyDeviceToDevice, stream));
    }
    int splits = 0;
    if (gemm(h, li, dn_t, dn_s, act_ffn, I, H, EPI_PARTIAL, nullptr, 0, 0, nullptr, 0, stream, &splits)) return 1;
    const float* part = (const float*)h->ws(h->off_part);
    if (mtp_tail) {
        auto nw = get<uint16_t>(h, "mtp.norm", li, &ok);
        auto fw = get<uint16_t>(h, "head.norm", -1, &ok);
        if (!ok) return 1;
        return norm_rows(h, part, splits, nullptr, x, nullptr, nw, nullptr, 0, 0, final_out, fw, stream);
    }
    if (next < 0) return norm_rows(h, part, splits, nullptr, x, final_out, nullptr, nullptr, 0, 0, nullptr, nullptr, stream);
    auto nw = get<uint16_t>(h, "input_layernorm", next, &ok);
    if (!ok) return 1;
    uint16_t* hbf = is_linear(h, next) ? (uint16_t*)h->ws(h->off_hbf) : nullptr;
    return norm_rows(h, part, splits, nullptr, x, x, nw, act_h, H, 0, hbf, nullptr, stream);
}

}  // namespace

int q38_report(const char* msg) { return fail(msg); }

int q38_device_cus() { return device_cus(); }

// One projection outside a handle: e5m2 tiles of x into `act` (unless x is null: act already holds them), then the
// GEMM with its counters and partial slots at `gemm` (fix_floats floats of slots after the counters).
int q38_projection(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n, int epi,
                   uint8_t* act, uint8_t* gemm, size_t fix_floats, void* out, int splits_max, hipStream_t stream, int w4,
                   int f8, int recompute) {
    if (!tiles || !tile_scales || !act || !gemm || !out) return fail("null argument");
    if (rows < 1 || n % 256 || k % 256) return fail("projection needs rows >= 1, N % 256 == 0 and K % 256 == 0");
    if (x) HIP_TRY(q38_act_tiles(x, rows, k, act, stream));
    GemmArgs a{};
    a.w = tiles;
    a.ws = tile_scales;
    a.act = act;
    a.K = k;
    a.N = n;
    a.T = rows;
    a.Tpad = pad_tokens(rows);
    a.splits_max = splits_max;
    a.w4 = w4;
    a.f8 = f8;
    a.recompute = recompute;
    if (epi == EPI_PARTIAL)
        a.part = (float*)out;
    else {
        a.out0 = out;
        a.ld0 = n;
        a.n0 = n;
    }
    gemm_scratch(a, gemm, device_cus());
    a.fix_floats = fix_floats;
    HIP_TRY(q38_gemm(a, epi, nullptr, stream));
    return 0;
}

extern "C" {

const char* q38_last_error(void) { return g_error.c_str(); }

int q38_create(const q38_config* cfg, q38_handle** out) {
    if (!cfg || !out) return fail("null argument");
    const q38_config& c = *cfg;
    std::string bad;
    if (c.num_layers < 1 || c.num_layers > Q38_MAX_LAYERS) bad += "num_layers out of range; ";
    if (c.linear_key_head_dim != 128 || c.linear_value_head_dim != 128) bad += "gated-delta head dims must be 128; ";
    if (c.head_dim != 256) bad += "head_dim must be 256; ";
    if (c.rotary_dim != 64) bad += "rotary_dim must be 64; ";
    if (c.linear_conv_kernel_dim != 4) bad += "conv width must be 4; ";
    if (c.num_key_value_heads <= 0 || c.num_attention_heads % c.num_key_value_heads) bad += "query heads per KV head; ";
    if (c.linear_num_key_heads <= 0 || c.linear_num_value_heads % c.linear_num_key_heads) bad += "value heads per key head; ";
    if (c.linear_num_value_heads % 8) bad += "value heads must be a multiple of 8; ";
    if (c.hidden_size % 256 || c.hidden_size > 8192) bad += "hidden_size must be a multiple of 256, at most 8192; ";
    if (c.intermediate_size % 256) bad += "intermediate_size must be a multiple of 256; ";
    if (c.vocab_size % 256) bad += "vocab_size must be a multiple of 256; ";
    if (c.verify_tokens < 1 || c.verify_tokens > 8) bad += "verify_tokens must be 1..8; ";
    if (c.num_attention_heads / c.num_key_value_heads * c.verify_tokens > 64) bad += "query rows per KV head above 64; ";
    if (c.batch_size < 1) bad += "batch_size must be positive; ";
    if (c.max_seq_len % 32 || c.max_seq_len < 64) bad += "max_seq_len must be a multiple of 32; ";
    if (c.prefill_chunk < 0 || c.prefill_chunk % 32 || c.prefill_chunk > c.max_seq_len) bad += "prefill_chunk must be a multiple of 32 up to max_seq_len; ";
    if (c.weight_format != Q38_WEIGHTS_E4M3 && c.weight_format != Q38_WEIGHTS_MXFP4) bad += "unknown weight_format; ";
    if (c.kv_cache_format != Q38_KV_BF16 && c.kv_cache_format != Q38_KV_FP8) bad += "unknown kv_cache_format; ";
    if (c.projection_mfma != Q38_MFMA_BF16 && c.projection_mfma != Q38_MFMA_FP8) bad += "unknown projection_mfma; ";
    for (int i = 0; i < c.num_layers && i < Q38_MAX_LAYERS; ++i)
        if (c.layer_types[i] != Q38_LINEAR && c.layer_types[i] != Q38_FULL) bad += "unknown layer type; ";
    if (!bad.empty()) return fail(bad);

    auto* h = new q38_handle();
    h->cfg = c;
    h->H = c.hidden_size;
    h->I = c.intermediate_size;
    h->V = c.vocab_size;
    h->B = c.batch_size;
    h->K = c.verify_tokens;
    h->S = c.max_seq_len;
    h->T = h->B * h->K;
    h->Tpad = pad_tokens(h->T);
    h->Hq = c.num_attention_heads;
    h->Hkv = c.num_key_value_heads;
    h->hd = c.head_dim;
    h->Hk = c.linear_num_key_heads;
    h->Hv = c.linear_num_value_heads;
    h->dk = c.linear_key_head_dim;
    h->C = 2 * h->Hk * h->dk + h->Hv * h->dk;
    h->cus = device_cus();
    h->layer.resize(c.num_layers + 1);
    h->act_h_k = c.mtp ? 2 * h->H : h->H;

    // Per-token buffers of the layer chain hold a verify step or a prefill chunk; the head and the speculative step's
    // buffers hold a verify step.
    const size_t Tv = h->Tpad, Tc = c.prefill_chunk ? pad_tokens(c.prefill_chunk) : 0, Tp = std::max(Tv, Tc), H = h->H;
    const size_t mid = std::max((size_t)h->Hv * h->dk, (size_t)h->Hq * h->hd);
    const size_t nqkv = (size_t)h->Hq * h->hd * 2 + 2 * (size_t)h->Hkv * h->hd;
    size_t o = 0;
    auto take = [&](size_t n) {
        size_t at = o;
        o += align256(n);
        return at;
    };
    h->off_x = take(Tp * H * 2);
    h->off_hbf = take(Tp * H * 2);
    h->off_tmp = take(Tp * H * 2);
    h->off_act_h = take(Tp * h->act_h_k);
    h->off_act_mid = take(Tp * mid);
    h->off_act_ffn = take(Tp * h->I);
    h->off_z = take(Tp * h->Hv * h->dk * 2);
    h->off_qkv = take(Tp * nqkv * 2);
    h->gate_groups = 8;
    while (h->gate_groups > 1 && (h->H % (64 * h->gate_groups) || h->H / (64 * h->gate_groups) > 16)) h->gate_groups /= 2;
    h->off_gates = take((size_t)h->gate_groups * Tp * 2 * h->Hv * 4);
    const size_t heads = (size_t)h->B * h->Hkv;
    h->attn_nchunks = (h->S + ATTN_CHUNK - 1) / ATTN_CHUNK;
    h->off_scores = take(heads * ATTN_QMAX * h->S * 2);
    h->off_astats = take(heads * h->attn_nchunks * ATTN_QMAX * 2 * 4);
    h->off_aown = take(heads * ATTN_QMAX * ATTN_KMAX * 4);
    h->off_akv = take(heads * 2 * ATTN_KMAX * 256 * 4);
    h->off_aq = take(heads * ATTN_QMAX * 256 * 2);
    // attn_pv's split sums: at most about two workgroups per CU of 64 query rows x 256 dims each.
    h->attn_pv_floats = h->attn_nchunks > 1 ? (size_t)2 * device_cus() * ATTN_QMAX * 256 : 0;
    h->off_apv = take(h->attn_pv_floats * 4);
    h->off_apr = take(heads * ATTN_QMAX * (2 + ATTN_KMAX) * 4);
    h->off_htiles = take(Tv * H * 2);
    h->off_x32 = take(Tv * H * 4);
    h->off_maxima = take(Tv * (h->V / 32) * 4);
    h->off_sp_embeds = take(Tv * H * 2);
    h->off_sp_cos = take(Tv * 64 * 2);
    h->off_sp_sin = take(Tv * 64 * 2);
    h->off_sp_states = take(Tv * H * 2);
    h->off_sp_out = take(Tv * H * 2);
    h->off_sp_current = take(Tv * H * 2);
    h->off_sp_ids = take(Tv * 4);
    h->off_sp_at = take(Tv * 4);
    h->off_sp_draft = take(Tv * 4);
    h->off_gemm = take(gemm_scratch_bytes(h->cus));
    h->off_status = take(16);
    // Split-K partials: up to GEMM_SPLIT_MAX splits at the verify width, 4 at a prefill chunk's (whose tiles
    // outnumber the CUs: the split count is chosen so the last round of workgroups is full); gemm() caps the splits at
    // what fits.
    h->part_floats = std::max((size_t)GEMM_SPLIT_MAX * Tv, 4 * Tc) * H;
    h->off_part = take(h->part_floats * 4);
    if (Tc) {
        h->off_pqn = take(Tc * h->Hk * h->dk * 4);
        h->off_pkn = take(Tc * h->Hk * h->dk * 4);
        h->off_pv = take(Tc * h->Hv * h->dk * 4);
        h->off_po = take(Tc * h->Hv * h->dk * 4);
        h->off_pbeta = take(Tc * h->Hv * 4);
        h->off_pg = take(Tc * h->Hv * 4);
        h->off_pqs = take((size_t)h->Hq * Tc * 256 * 2);
    }
    h->workspace_bytes = o;
    *out = h;
    return 0;
}

void q38_destroy(q38_handle* h) {
    if (!h) return;
    for (hipEvent_t e : h->timer_events) (void)hipEventDestroy(e);
    h->drop_graphs();
    if (h->capture_stream) (void)hipStreamDestroy(h->capture_stream);
    if (h->side_stream) (void)hipStreamDestroy(h->side_stream);
    if (h->fork_ev) (void)hipEventDestroy(h->fork_ev);
    if (h->join_ev) (void)hipEventDestroy(h->join_ev);
    delete h;
}

int q38_kernel_timer(q38_handle* h, int on, int* launches, float* total_ms) {
    if (!h) return fail("null argument");
    if (on) {
        if (h->timer_events.empty()) {
            h->timer_events.resize(2 * TIMER_PAIRS);
            for (hipEvent_t& e : h->timer_events)
                if (hipEventCreate(&e) != hipSuccess) return fail("hipEventCreate failed");
        }
        h->timer_used = 0;
        h->timer_on = true;
        return 0;
    }
    h->timer_on = false;
    float total = 0.0f;
    for (int i = 0; i < h->timer_used; ++i) {
        HIP_TRY(hipEventSynchronize(h->timer_events[2 * i + 1]));
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, h->timer_events[2 * i], h->timer_events[2 * i + 1]));
        total += ms;
    }
    if (launches) *launches = h->timer_used;
    if (total_ms) *total_ms = total;
    return 0;
}

int q38_buffer_size(q38_handle* h, const char* name, int layer, size_t* nbytes) {
    if (!h || !name || !nbytes) return fail("null argument");
    size_t n = expected_size(h, name, layer);
    if (!n) return fail(std::string("no buffer '") + name + "' for layer " + std::to_string(layer));
    *nbytes = n;
    return 0;
}

int q38_bind(q38_handle* h, const char* name, int layer, void* dev_ptr, size_t nbytes) {
    if (!h || !name || !dev_ptr) return fail("null argument");
    size_t n = expected_size(h, name, layer);
    if (!n) return fail(std::string("no buffer '") + name + "' for layer " + std::to_string(layer));
    if (nbytes != n)
        return fail(std::string("buffer '") + name + "' needs " + std::to_string(n) + " bytes, got " + std::to_string(nbytes));
    if ((uintptr_t)dev_ptr % 16) return fail(std::string("buffer '") + name + "' is not 16-byte aligned");
    if (layer < 0 && std::string(name) == "workspace") {
        // The GEMMs' arrival counters and the step status word start at zero.
        HIP_TRY(hipMemset((uint8_t*)dev_ptr + h->off_gemm, 0, (size_t)GEMM_COUNTERS * 8));
        HIP_TRY(hipMemset((uint8_t*)dev_ptr + h->off_status, 0, 16));
        if (!h->side_stream) {
            HIP_TRY(hipStreamCreateWithFlags(&h->side_stream, hipStreamNonBlocking));
            HIP_TRY(hipEventCreateWithFlags(&h->fork_ev, hipEventDisableTiming));
            HIP_TRY(hipEventCreateWithFlags(&h->join_ev, hipEventDisableTiming));
        }
    }
    Buf b;
    b.p = dev_ptr;
    b.n = nbytes;
    (layer < 0 ? h->global : h->layer[layer])[name] = b;
    h->drop_graphs();  // captured steps hold the old pointers
    return 0;
}

int q38_parity(q38_handle* h, int* parity) {
    if (!h || !parity) return fail("null argument");
    *parity = h->parity;
    return 0;
}

int q38_set_parity(q38_handle* h, int parity) {
    if (!h || (parity != 0 && parity != 1)) return fail("parity must be 0 or 1");
    h->parity = parity;
    return 0;
}

int q38_pack_weight(const uint8_t* coded, const uint8_t* scales, int n, int k, uint8_t* tiles, uint8_t* tile_scales,
                    void* stream) {
    if (!coded || !scales || !tiles || !tile_scales) return fail("null argument");
    if (n <= 0 || k <= 0 || n % 32 || k % 256) return fail("pack needs N % 32 == 0 and K % 256 == 0");
    HIP_TRY(q38_pack(coded, scales, n, k, tiles, tile_scales, (hipStream_t)stream));
    return 0;
}

int q38_pack_weight_fp4(const uint8_t* packed, const uint8_t* scales, int n, int k, uint8_t* tiles, uint8_t* tile_scales,
                        void* stream) {
    if (!packed || !scales || !tiles || !tile_scales) return fail("null argument");
    if (n <= 0 || k <= 0 || n % 32 || k % 256) return fail("pack needs N % 32 == 0 and K % 256 == 0");
    HIP_TRY(q38_pack_fp4(packed, scales, n, k, tiles, tile_scales, (hipStream_t)stream));
    return 0;
}

size_t q38_tiles_size(int rows, int k) { return align256((size_t)pad_tokens(rows) * k); }

size_t q38_fp8_linear_scratch(int rows, int k) { return q38_tiles_size(rows, k) + gemm_scratch_bytes(device_cus()); }

namespace {

// A projection with the caller's scratch: the input tiles, then the GEMM's counters and slots for every CU.
int standalone(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n, int epi,
               uint8_t* scratch, void* out, int splits_max, hipStream_t stream, int w4 = 0, int f8 = 0, int recompute = 0) {
    if (!scratch) return fail("null argument");
    return q38_projection(x, rows, k, tiles, tile_scales, n, epi, scratch, scratch + q38_tiles_size(rows, k),
                          (size_t)2 * device_cus() * GEMM_SLOT_FLOATS, out, splits_max, stream, w4, f8, recompute);
}

}  // namespace

int q38_fp8_linear(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                   uint8_t* scratch, uint16_t* out, void* stream) {
    return standalone(x, rows, k, tiles, tile_scales, n, EPI_BF16, scratch, out, 0, (hipStream_t)stream);
}

int q38_fp8_linear_mfma(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n, int mfma,
                        int f32_out, uint8_t* scratch, void* out, void* stream) {
    const int kind = mfma & ~Q38_GEMM_RECOMPUTE;
    if (kind != Q38_MFMA_FP8 && kind != Q38_MFMA_BF16) return fail("mfma must be Q38_MFMA_FP8 or Q38_MFMA_BF16");
    if (f32_out && pad_tokens(rows) != rows) return fail("float32 output needs rows in {32, 64, 128} or a multiple of 256");
    return standalone(x, rows, k, tiles, tile_scales, n, f32_out ? EPI_PARTIAL : EPI_BF16, scratch, out, f32_out ? 1 : 0,
                      (hipStream_t)stream, 0, kind == Q38_MFMA_FP8, (mfma & Q38_GEMM_RECOMPUTE) != 0);
}

size_t q38_fp4_linear_scratch(int rows, int k) {
    return align256((size_t)pad_tokens(rows) * k * 2) + gemm_scratch_bytes(device_cus());
}

// FP4Linear.forward (model.py:206-208): each parity plane of x through the whole weight (the other plane's inputs are
// zero in the tiles, so the sum is the plane's), the first plane's sums stored as bf16, the second's added to them.
int q38_fp4_linear(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                   uint8_t* scratch, uint16_t* out, void* stream_) {
    if (!x || !tiles || !tile_scales || !scratch || !out) return fail("null argument");
    if (rows < 1 || n % 256 || k % 256) return fail("fp4_linear needs rows >= 1, N % 256 == 0 and K % 256 == 0");
    const hipStream_t stream = (hipStream_t)stream_;
    bf16_t* act = (bf16_t*)scratch;
    uint8_t* gemm_base = scratch + align256((size_t)pad_tokens(rows) * k * 2);
    for (int plane = 0; plane < 2; ++plane) {
        HIP_TRY(q38_act_tiles_bf16((const bf16_t*)x, rows, k, plane, act, stream));
        GemmArgs a{};
        a.w = tiles;
        a.ws = tile_scales;
        a.act = act;
        a.K = k;
        a.N = n;
        a.T = rows;
        a.Tpad = pad_tokens(rows);
        a.w4 = 1;
        a.bf16_act = 1;
        a.accumulate = plane;
        a.out0 = out;
        a.ld0 = n;
        a.n0 = n;
        gemm_scratch(a, gemm_base, device_cus());
        HIP_TRY(q38_gemm(a, EPI_BF16, nullptr, stream));
    }
    return 0;
}

int q38_mxfp4_linear(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                     uint8_t* scratch, uint16_t* out, void* stream) {
    return standalone(x, rows, k, tiles, tile_scales, n, EPI_BF16, scratch, out, 0, (hipStream_t)stream, 1);
}

int q38_fp8_linear_f32(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                       uint8_t* scratch, float* out, void* stream) {
    if (pad_tokens(rows) != rows) return fail("fp8_linear_f32 needs rows in {32, 64, 128} or a multiple of 256");
    return standalone(x, rows, k, tiles, tile_scales, n, EPI_PARTIAL, scratch, out, 1, (hipStream_t)stream);
}

int q38_mlp_up(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int inter,
               uint8_t* scratch, uint8_t* out_tiles, void* stream) {
    if (inter % 64) return fail("mlp_up needs inter % 64 == 0");
    return standalone(x, rows, k, tiles, tile_scales, 2 * inter, EPI_SWIGLU, scratch, out_tiles, 0, (hipStream_t)stream);
}

int q38_verify(q38_handle* h, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin, const int32_t* position,
               const float* active, const int32_t* accepted, uint16_t* out_hidden, void* stream_) {
    if (!h || !embeds || !cos || !sin || !position || !active || !accepted || !out_hidden) return fail("null argument");
    hipStream_t stream = (hipStream_t)stream_;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto in0 = get<uint16_t>(h, "input_layernorm", 0, &ok);
    if (!ok) return 1;
    const int L = h->cfg.num_layers, rd = h->parity, wr = 1 - h->parity;
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    uint16_t* hbf = is_linear(h, 0) ? (uint16_t*)h->ws(h->off_hbf) : nullptr;
    if (norm_rows(h, nullptr, 0, embeds, nullptr, x, in0, h->ws(h->off_act_h), h->H, 0, hbf, nullptr, stream)) return 1;
    StepIO io{cos, sin, position, active, accepted};
    for (int li = 0; li < L; ++li) {
        if (run_mixer(h, li, io, rd, wr, stream)) return 1;
        if (run_mlp(h, li, li + 1 < L ? li + 1 : -1, out_hidden, false, stream)) return 1;
    }
    h->parity = wr;
    return 0;
}

int q38_decode(q38_handle* h, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin, const int32_t* position,
               const float* active, uint16_t* out_hidden, void* stream_) {
    if (!h || !embeds || !cos || !sin || !position || !active || !out_hidden) return fail("null argument");
    hipStream_t stream = (hipStream_t)stream_;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto in0 = get<uint16_t>(h, "input_layernorm", 0, &ok);
    if (!ok) return 1;
    TokensScope one(h, 1);
    const int L = h->cfg.num_layers, rd = h->parity, wr = 1 - h->parity;
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    uint16_t* hbf = is_linear(h, 0) ? (uint16_t*)h->ws(h->off_hbf) : nullptr;
    if (norm_rows(h, nullptr, 0, embeds, nullptr, x, in0, h->ws(h->off_act_h), h->H, 0, hbf, nullptr, stream)) return 1;
    StepIO io{cos, sin, position, active, nullptr, true};
    for (int li = 0; li < L; ++li) {
        if (run_mixer(h, li, io, rd, wr, stream)) return 1;
        if (run_mlp(h, li, li + 1 < L ? li + 1 : -1, out_hidden, false, stream)) return 1;
    }
    h->parity = wr;  // the conv states were written to the other half
    return 0;
}

int q38_prefill(q38_handle* h, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin, const int32_t* slot,
                const int32_t* start, const int32_t* n_valid, int tokens, uint16_t* out_hidden, void* stream_) {
    if (!h || !embeds || !cos || !sin || !slot || !start || !n_valid || !out_hidden) return fail("null argument");
    if (!h->cfg.prefill_chunk) return fail("the handle was created without a prefill chunk (config prefill_chunk is 0)");
    if (tokens < 32 || tokens % 32 || tokens > h->cfg.prefill_chunk)
        return fail("prefill tokens must be a multiple of 32 up to the config's prefill_chunk");
    hipStream_t stream = (hipStream_t)stream_;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto in0 = get<uint16_t>(h, "input_layernorm", 0, &ok);
    if (!ok) return 1;
    TokensScope chunk(h, 1, tokens);
    const int L = h->cfg.num_layers, rd = h->parity;
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    uint16_t* hbf = is_linear(h, 0) ? (uint16_t*)h->ws(h->off_hbf) : nullptr;
    if (norm_rows(h, nullptr, 0, embeds, nullptr, x, in0, h->ws(h->off_act_h), h->H, 0, hbf, nullptr, stream)) return 1;
    StepIO io{cos, sin, nullptr, nullptr, nullptr, false, slot, start, n_valid};
    for (int li = 0; li < L; ++li) {
        if (run_mixer(h, li, io, rd, rd, stream)) return 1;
        if (run_mlp(h, li, li + 1 < L ? li + 1 : -1, out_hidden, false, stream)) return 1;
    }
    return 0;  // the row's states and cache were updated in place; the parity stays
}

int q38_mtp_prefill(q38_handle* h, const uint16_t* hidden, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin,
                    const int32_t* slot, const int32_t* start, int tokens, uint16_t* out_x, void* stream_) {
    if (!h || !hidden || !embeds || !cos || !sin || !slot || !start) return fail("null argument");
    if (!h->cfg.mtp) return fail("the handle was created without the MTP layer");
    if (!h->cfg.prefill_chunk) return fail("the handle was created without a prefill chunk (config prefill_chunk is 0)");
    if (tokens < 32 || tokens % 32 || tokens > h->cfg.prefill_chunk)
        return fail("prefill tokens must be a multiple of 32 up to the config's prefill_chunk");
    hipStream_t stream = (hipStream_t)stream_;
    const int M = h->cfg.num_layers, H = h->H;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto en = get<uint16_t>(h, "mtp.embedding_norm", M, &ok);
    auto hn = get<uint16_t>(h, "mtp.hidden_norm", M, &ok);
    auto fin = get<uint16_t>(h, "head.norm", -1, &ok);
    auto fc_t = get<uint8_t>(h, "mtp.fc.tiles", M, &ok);
    auto fc_s = get<uint8_t>(h, "mtp.fc.scales", M, &ok);
    auto in0 = get<uint16_t>(h, "input_layernorm", M, &ok);
    auto qkv_t = get<uint8_t>(h, "self_attn.qkv.tiles", M, &ok);
    auto qkv_s = get<uint8_t>(h, "self_attn.qkv.scales", M, &ok);
    auto kn = get<uint16_t>(h, "self_attn.k_norm", M, &ok);
    auto kc = get<uint16_t>(h, "self_attn.k_cache", M, &ok);
    auto vc = get<uint16_t>(h, "self_attn.v_cache", M, &ok);
    const bool kv8 = h->cfg.kv_cache_format == Q38_KV_FP8;
    const uint16_t* ks = kv8 ? get<uint16_t>(h, "self_attn.k_scale", M, &ok) : nullptr;
    const uint16_t* vs = kv8 ? get<uint16_t>(h, "self_attn.v_scale", M, &ok) : nullptr;
    if (!ok) return 1;
    TokensScope chunk(h, 1, tokens);
    uint8_t* act_h = h->ws(h->off_act_h);
    uint16_t* tmp = (uint16_t*)h->ws(h->off_tmp);
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    // [rms(embeds) | rms(rms(hidden, final norm), hidden norm)] -> fc -> x; rms(x, input norm) as e5m2 tiles
    // (model.py:845-855, the prefill form).
    if (norm_rows(h, nullptr, 0, embeds, nullptr, nullptr, en, act_h, 2 * H, 0, nullptr, nullptr, stream)) return 1;
    if (norm_rows(h, nullptr, 0, hidden, nullptr, nullptr, fin, nullptr, 0, 0, tmp, nullptr, stream)) return 1;
    if (norm_rows(h, nullptr, 0, tmp, nullptr, nullptr, hn, act_h, 2 * H, H, nullptr, nullptr, stream)) return 1;
    int splits = 0;
    if (gemm(h, M, fc_t, fc_s, act_h, 2 * H, H, EPI_PARTIAL, nullptr, 0, 0, nullptr, 0, stream, &splits)) return 1;
    if (norm_rows(h, (const float*)h->ws(h->off_part), splits, nullptr, nullptr, x, in0, act_h, H, 0, nullptr, nullptr, stream))
        return 1;
    // Keys and values only (cache_chunk, model.py:784-790): the k and v rows of the qkv weight, after the q rows.
    const size_t q_rows = (size_t)h->Hq * h->hd * 2, kt = (size_t)H / 64;
    const int nkv = 2 * h->Hkv * h->hd;
    uint16_t* kv = (uint16_t*)h->ws(h->off_qkv);
    if (gemm(h, M, qkv_t + q_rows / 32 * kt * 2048, qkv_s + q_rows / 32 * kt * 64, act_h, H, nkv, EPI_BF16, kv, nkv, nkv, nullptr, 0,
             stream))
        return 1;
    PrefillAttnArgs p{};
    p.L = h->T;
    p.rows = h->B;
    p.Hq = h->Hq;
    p.Hkv = h->Hkv;
    p.S = h->S;
    p.slot = slot;
    p.start = start;
    p.qkv = kv;
    p.ld = nkv;
    p.kv_col = 0;
    p.k_norm = kn;
    p.cos = cos;
    p.sin = sin;
    p.k_cache = kc;
    p.v_cache = vc;
    p.kv8 = kv8;
    p.k_scale = ks;
    p.v_scale = vs;
    p.eps = h->cfg.rms_norm_eps;
    p.keys_only = 1;
    HIP_TRY(q38_attn_prefill(p, stream));
    if (out_x) HIP_TRY(hipMemcpyAsync(out_x, x, (size_t)H * 2, hipMemcpyDeviceToDevice, stream));
    return 0;
}

int q38_copy_states(q38_handle* h, const int32_t* slot, int to_saved, void* stream_) {
    if (!h || !slot) return fail("null argument");
    if (!h->cfg.saved_states) return fail("this handle keeps no saved states (config saved_states is 0)");
    hipStream_t stream = (hipStream_t)stream_;
    CopyStatesArgs a{};
    a.state_row = (size_t)h->Hv * h->dk * h->dk;
    a.conv_row = (size_t)h->C * 3;
    a.slot = slot;
    a.rows = h->B;
    a.to_saved = to_saved ? 1 : 0;
    const size_t convn = (size_t)h->B * h->C * 3;
    bool ok = true;
    auto flush = [&]() -> int {
        if (a.n) HIP_TRY(q38_copy_states(a, stream));
        a.n = 0;
        return 0;
    };
    for (int li = 0; li < h->cfg.num_layers; ++li) {
        if (!is_linear(h, li)) continue;
        auto st = get<uint16_t>(h, "linear_attn.recurrent_state", li, &ok);
        auto conv = get<uint16_t>(h, "linear_attn.conv_state", li, &ok);
        auto sst = get<uint16_t>(h, "linear_attn.saved_state", li, &ok);
        auto sconv = get<uint16_t>(h, "linear_attn.saved_conv", li, &ok);
        if (!ok) return 1;
        a.state[a.n] = st;
        a.conv[a.n] = conv + h->parity * convn;  // the current half
        a.saved_state[a.n] = sst;
        a.saved_conv[a.n] = sconv;
        if (++a.n == COPY_STATES_MAX && flush()) return 1;
    }
    return flush();
}

int q38_mtp_step(q38_handle* h, const uint16_t* hidden, const uint16_t* embeds, const uint16_t* cos, const uint16_t* sin,
                 const int32_t* position, const float* active, uint16_t* out, void* stream_) {
    if (!h || !hidden || !embeds || !cos || !sin || !position || !active || !out) return fail("null argument");
    if (!h->cfg.mtp) return fail("the handle was created without the MTP layer");
    hipStream_t stream = (hipStream_t)stream_;
    const int M = h->cfg.num_layers, H = h->H;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto en = get<uint16_t>(h, "mtp.embedding_norm", M, &ok);
    auto hn = get<uint16_t>(h, "mtp.hidden_norm", M, &ok);
    auto fin = get<uint16_t>(h, "head.norm", -1, &ok);
    auto fc_t = get<uint8_t>(h, "mtp.fc.tiles", M, &ok);
    auto fc_s = get<uint8_t>(h, "mtp.fc.scales", M, &ok);
    auto in0 = get<uint16_t>(h, "input_layernorm", M, &ok);
    if (!ok) return 1;
    uint8_t* act_h = h->ws(h->off_act_h);
    uint16_t* tmp = (uint16_t*)h->ws(h->off_tmp);
    uint16_t* x = (uint16_t*)h->ws(h->off_x);
    // [rms(embeds) | rms(rms(hidden, final norm), hidden norm)] as the fc's 2H-wide e5m2 input (model.py:845-851).
    if (norm_rows(h, nullptr, 0, embeds, nullptr, nullptr, en, act_h, 2 * H, 0, nullptr, nullptr, stream)) return 1;
    if (norm_rows(h, nullptr, 0, hidden, nullptr, nullptr, fin, nullptr, 0, 0, tmp, nullptr, stream)) return 1;
    if (norm_rows(h, nullptr, 0, tmp, nullptr, nullptr, hn, act_h, 2 * H, H, nullptr, nullptr, stream)) return 1;
    int splits = 0;
    if (gemm(h, M, fc_t, fc_s, act_h, 2 * H, H, EPI_PARTIAL, nullptr, 0, 0, nullptr, 0, stream, &splits)) return 1;
    if (norm_rows(h, (const float*)h->ws(h->off_part), splits, nullptr, nullptr, x, in0, act_h, H, 0, nullptr, nullptr, stream))
        return 1;
    StepIO io{cos, sin, position, active, nullptr};
    if (run_mixer(h, M, io, 0, 0, stream)) return 1;
    return run_mlp(h, M, -1, out, true, stream);
}

int q38_head_groupmax(q38_handle* h, const uint16_t* hidden, int rows, float* maxima, void* stream_) {
    if (!h || !hidden || !maxima) return fail("null argument");
    if (rows < 1 || rows > h->T) return fail("head rows must be 1..B*K");
    hipStream_t stream = (hipStream_t)stream_;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto nw = get<uint16_t>(h, "head.norm", -1, &ok);
    auto wt = get<uint8_t>(h, "head.lm_head.tiles", -1, &ok);
    auto wsc = get<uint8_t>(h, "head.lm_head.scales", -1, &ok);
    if (!ok) return 1;
    HIP_TRY(q38_head_norm(hidden, nw, h->cfg.rms_norm_eps, h->H, rows, (bf16_t*)h->ws(h->off_htiles),
                          (float*)h->ws(h->off_x32), stream));
    // The optional head probe: the normed rows as the GEMM reads them (bf16 activation tiles of whole 32-row blocks).
    auto hp = h->global.find("head.probe");
    if (hp != h->global.end())
        HIP_TRY(hipMemcpyAsync(hp->second.p, h->ws(h->off_htiles), (size_t)(rows + 31) / 32 * 32 * h->H * 2,
                               hipMemcpyDeviceToDevice, stream));
    GemmArgs a{};
    a.w = wt;
    a.ws = wsc;
    a.act = (const bf16_t*)h->ws(h->off_htiles);
    a.K = h->H;
    a.N = h->V;
    a.T = rows;
    a.Tpad = pad_tokens(rows);
    a.part = maxima;
    gemm_scratch(a, h->ws(h->off_gemm), h->cus);
    HIP_TRY(q38_gemm(a, EPI_GROUPMAX, nullptr, stream));
    return 0;
}

int q38_head_pick(q38_handle* h, const uint16_t* hidden, int rows, int groups, int32_t* ids, void* stream_) {
    if (!h || !hidden || !ids) return fail("null argument");
    if (groups < 1 || groups > 4) return fail("recheck groups must be 1..4");
    float* maxima = (float*)h->ws(h->off_maxima);
    if (q38_head_groupmax(h, hidden, rows, maxima, stream_)) return 1;
    bool ok = true;
    auto wt = get<uint8_t>(h, "head.lm_head.tiles", -1, &ok);
    auto wsc = get<uint8_t>(h, "head.lm_head.scales", -1, &ok);
    if (!ok) return 1;
    PickArgs a{};
    a.maxima = maxima;
    a.ngroups = h->V / 32;
    a.x32 = (const float*)h->ws(h->off_x32);
    a.w = wt;
    a.ws = wsc;
    a.rows = h->global.count("head.lm_head.rows") ? (const bf16_t*)h->global.at("head.lm_head.rows").p : nullptr;
    a.status = (int*)h->ws(h->off_status);
    a.H = h->H;
    a.R = rows;
    a.groups = groups;
    a.ids = ids;
    HIP_TRY(q38_head_pick(a, (hipStream_t)stream_));
    return 0;
}

int q38_spec_step(q38_handle* h, int32_t* position, int32_t* index, int32_t* match, int32_t* accepted, const float* active,
                  uint16_t* hidden, int32_t* picks, int32_t* drafts, void* stream_) {
    if (!h || !position || !index || !match || !accepted || !active || !hidden || !picks || !drafts)
        return fail("null argument");
    if (!h->cfg.mtp) return fail("the speculative step needs the MTP layer");
    if (h->K < 2) return fail("the speculative step needs at least 2 verify tokens");
    hipStream_t stream = (hipStream_t)stream_;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto rope = get<uint16_t>(h, "rope_table", -1, &ok);
    if (!ok) return 1;
    const int B = h->B, K = h->K, H = h->H, S = h->S;
    uint16_t* embeds = (uint16_t*)h->ws(h->off_sp_embeds);
    uint16_t* cos = (uint16_t*)h->ws(h->off_sp_cos);
    uint16_t* sin = (uint16_t*)h->ws(h->off_sp_sin);
    uint16_t* states = (uint16_t*)h->ws(h->off_sp_states);
    uint16_t* out = (uint16_t*)h->ws(h->off_sp_out);
    uint16_t* current = (uint16_t*)h->ws(h->off_sp_current);
    int32_t* ids = (int32_t*)h->ws(h->off_sp_ids);
    int32_t* at = (int32_t*)h->ws(h->off_sp_at);
    int32_t* draft = (int32_t*)h->ws(h->off_sp_draft);

    // Drafts (scheduler.py:160-193): the first MTP call takes the last step's K hidden states and picks at its
    // positions; the draft comes from its output at each row's match; each further draft from an MTP call on the
    // previous draft alone.
    if (q38_embed(h, picks, B * K, embeds, stream_)) return 1;
    int* status = (int*)h->ws(h->off_status);
    HIP_TRY(q38_rope_gather(index, 1, B, K, S, rope, cos, sin, stream, active, status));
    if (q38_mtp_step(h, hidden, embeds, cos, sin, index, active, out, stream_)) return 1;
    HIP_TRY(q38_select_rows(out, match, B, K, H, current, stream));
    for (int j = 0; j < K - 1; ++j) {
        if (q38_head_pick(h, current, B, 1, draft, stream_)) return 1;
        HIP_TRY(q38_draft_column(draft, K, B, j, drafts, stream));
        if (j == K - 2) break;
        HIP_TRY(q38_mtp_followup(current, draft, B, K, H, states, ids, stream));
        if (q38_embed(h, ids, B * K, embeds, stream_)) return 1;
        HIP_TRY(q38_offset_positions(index, match, j, B, at, stream));
        HIP_TRY(q38_rope_gather(at, 1, B, K, S, rope, cos, sin, stream, active, status));
        if (q38_mtp_step(h, states, embeds, cos, sin, at, active, out, stream_)) return 1;
        HIP_TRY(q38_select_rows(out, nullptr, B, K, H, current, stream));
    }
    return q38_verify_step(h, position, index, match, accepted, active, hidden, picks, drafts, stream_);
}

int q38_verify_step(q38_handle* h, int32_t* position, int32_t* index, int32_t* match, int32_t* accepted, const float* active,
                    uint16_t* hidden, int32_t* picks, const int32_t* drafts, void* stream_) {
    if (!h || !position || !index || !match || !accepted || !active || !hidden || !picks || !drafts)
        return fail("null argument");
    if (h->K < 2) return fail("the verify step needs at least 2 verify tokens");
    hipStream_t stream = (hipStream_t)stream_;
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    auto rope = get<uint16_t>(h, "rope_table", -1, &ok);
    if (!ok) return 1;
    const int B = h->B, K = h->K, S = h->S;
    uint16_t* embeds = (uint16_t*)h->ws(h->off_sp_embeds);
    uint16_t* cos = (uint16_t*)h->ws(h->off_sp_cos);
    uint16_t* sin = (uint16_t*)h->ws(h->off_sp_sin);
    int32_t* ids = (int32_t*)h->ws(h->off_sp_ids);
    int* status = (int*)h->ws(h->off_status);
    // Verify (scheduler.py:276-301): [last emitted token, drafts] per row, the head over all B*K rows, acceptance.
    HIP_TRY(q38_verify_tokens(picks, match, drafts, B, K, ids, stream));
    if (q38_embed(h, ids, B * K, embeds, stream_)) return 1;
    HIP_TRY(q38_rope_gather(position, 0, B, K, S, rope, cos, sin, stream, active, status));
    if (q38_verify(h, embeds, cos, sin, position, active, accepted, hidden, stream_)) return 1;
    if (q38_head_pick(h, hidden, B * K, 4, picks, stream_)) return 1;
    HIP_TRY(q38_accept(picks, drafts, active, B, K, match, accepted, stream));
    HIP_TRY(q38_advance(position, index, accepted, B, stream));
    return 0;
}

int q38_spec_step_graph(q38_handle* h, int32_t* position, int32_t* index, int32_t* match, int32_t* accepted,
                        const float* active, uint16_t* hidden, int32_t* picks, int32_t* drafts, void* stream_) {
    if (!h || !position || !index || !match || !accepted || !active || !hidden || !picks || !drafts)
        return fail("null argument");
    hipStream_t stream = (hipStream_t)stream_;
    // The kernel timer records events and the probe copies per call: those steps run as launches.
    bool probed = false;
    for (const auto& l : h->layer) probed = probed || l.count("probe");
    if (h->timer_on || probed)
        return q38_spec_step(h, position, index, match, accepted, active, hidden, picks, drafts, stream_);
    const int parity = h->parity;
    q38_handle::StepGraph& g = h->graphs[parity];
    const void* args[8] = {position, index, match, accepted, active, hidden, picks, drafts};
    if (!g.exec || memcmp(g.args, args, sizeof(args))) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        g = q38_handle::StepGraph{};
        if (!h->capture_stream) HIP_TRY(hipStreamCreateWithFlags(&h->capture_stream, hipStreamNonBlocking));
        // Capturing runs nothing: the recorded step starts from the current parity, and so does the state after it.
        HIP_TRY(hipStreamBeginCapture(h->capture_stream, hipStreamCaptureModeThreadLocal));
        const int rc = q38_spec_step(h, position, index, match, accepted, active, hidden, picks, drafts, h->capture_stream);
        hipGraph_t graph = nullptr;
        const hipError_t e = hipStreamEndCapture(h->capture_stream, &graph);
        h->parity = parity;
        if (rc) {
            if (e == hipSuccess && graph) (void)hipGraphDestroy(graph);
            return 1;
        }
        HIP_TRY(e);
        const hipError_t ei = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (ei != hipSuccess) {
            g.exec = nullptr;
            return fail(std::string("hipGraphInstantiate: ") + hipGetErrorString(ei));
        }
        memcpy(g.args, args, sizeof(args));
    }
    HIP_TRY(hipGraphLaunch(g.exec, stream));
    h->parity = 1 - parity;
    return 0;
}

int q38_step_status(q38_handle* h, int* status, int clear, void* stream_) {
    if (!h || !status) return fail("null argument");
    bool ok = true;
    get<uint8_t>(h, "workspace", -1, &ok);
    if (!ok) return 1;
    hipStream_t stream = (hipStream_t)stream_;
    int* word = (int*)h->ws(h->off_status);
    HIP_TRY(hipMemcpyAsync(status, word, sizeof(int), hipMemcpyDeviceToHost, stream));
    HIP_TRY(hipStreamSynchronize(stream));
    if (clear) HIP_TRY(hipMemsetAsync(word, 0, sizeof(int), stream));
    return 0;
}

int q38_embed(q38_handle* h, const int32_t* ids, int n, uint16_t* out, void* stream) {
    if (!h || !ids || !out) return fail("null argument");
    bool ok = true;
    auto table = get<uint16_t>(h, "embed_tokens", -1, &ok);
    if (!ok) return 1;
    if (n <= 0) return 0;
    HIP_TRY(q38_embed(ids, n, table, h->V, h->H, out, (hipStream_t)stream));
    return 0;
}

int q38_accept(q38_handle* h, const int32_t* picks, const int32_t* drafts, const float* active, int32_t* match,
               int32_t* accepted, void* stream) {
    if (!h || !picks || !drafts || !active || !match || !accepted) return fail("null argument");
    if (h->K < 2) return fail("acceptance needs at least 2 verify tokens");
    HIP_TRY(q38_accept(picks, drafts, active, h->B, h->K, match, accepted, (hipStream_t)stream));
    return 0;
}

}  // extern "C"
