// runtime.cpp -- the Moonlight session API (include/moonlight_hip.h and
// include/moonlight_hip_ext.h) over the HIP kernels.
//
// Replaces floyd's moonlight_metal.m.  The per-layer graph and residual order
// are the reference's (encode_attention_block / encode_dense_residual_buffer /
// encode_moe_residual_buffer, moonlight_metal.m:442-706):
//     h = x + o_proj(MLA(RMSNorm(x)))
//     x' = h + FFN(RMSNorm(h)),  FFN = dense SwiGLU or routed + shared experts
// but a forward is ONE submission: routing and its tables stay on the device,
// so the 1 + (layers - first_dense) host waits of run_tokens_fast
// (moonlight_metal.m:1892-1986) become a single wait for the logits.
#include "container.h"
#include "device_context.h"
#include "mla.h"
#include "moe.h"
#include "qgemm.h"
#include "sample.h"
#include "../../include/moonlight_hip.h"
#include "../../include/moonlight_hip_ext.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <algorithm>
#include <atomic>
#include <thread>
#include <string>
#include <unordered_map>
#include <vector>

using namespace mlh;

namespace {

int set_error(char *error, size_t error_size, const char *format, ...) {
    if (error && error_size) {
        va_list args;
        va_start(args, format);
        vsnprintf(error, error_size, format, args);
        va_end(args);
    }
    return 0;
}

double monotonic_seconds() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct DeviceTensor {
    std::string name;
    int dtype = 0;
    int64_t numel = 0, nbytes = 0;
    uint8_t *dev = nullptr;
};

struct Matrix {
    int fmt = kQ8;
    const uint8_t *w = nullptr;
    const float *s = nullptr;
};

struct LayerPlan {
    std::string error;  // first problem found while resolving, empty if usable
    Matrix q, kv_a, kv_b, o;
    // q_proj rows followed by kv_a rows in one matrix (same format): one GEMV
    // launch produces [q | compressed] per token row; fmt -1 when not fused
    Matrix qkv_a;
    const float *input_norm = nullptr, *post_norm = nullptr, *kv_norm = nullptr;
    bool dense = false;
    Matrix gate, up, down;
    Matrix router;
    const float *bias = nullptr;
    Matrix sh_gate, sh_up, sh_down;
    int expert_fmt = kQ8;
    ExpertWeights *expert_table = nullptr;  // device [experts] (inside the model's table)
};

}  // namespace

struct MoonlightModel {
    DeviceContext *ctx = nullptr;  // the device the model lives on (current at open)
    ModelConfig cfg;
    std::vector<DeviceTensor> tensors;
    std::unordered_map<std::string, int> index;
    uint8_t *arena = nullptr;
    size_t arena_bytes = 0;
    uint64_t resident_bytes = 0;
    std::vector<LayerPlan> layers;
    ExpertWeights *expert_tables = nullptr;  // device [layers][experts]
    float *inv_freq = nullptr;               // device [rope / 2]
    const float *embed = nullptr;
    const float *final_norm = nullptr;
    Matrix lm_head;
    std::string head_error;
    std::string device_name;
    std::vector<void *> extra;  // device buffers owned by the model (fused matrices)
};

struct MoonlightSession {
    MoonlightModel *model = nullptr;
    MoonlightOptions options{};
    MoonlightStats stats{};
    int max_splits = 0;
    std::vector<void *> allocations;
    // device buffers
    float *h = nullptr, *tmp = nullptr, *query = nullptr, *compressed = nullptr;
    float *query_rope = nullptr, *query_absorbed = nullptr, *context = nullptr;
    float *part_max = nullptr, *part_sum = nullptr, *part_lc = nullptr, *latent_ctx = nullptr;
    float *value_part = nullptr;  // decode MLA value shares
    int *merge_count = nullptr;                             // zeroed at creation
    float *latent_kv = nullptr, *rope_kv = nullptr, *logits = nullptr;
    // the latent cache's f16 halves (hi, lo) per value: [L][ctx][2][latent]
    uint16_t *latent_split = nullptr;
    // per-head keys and values of one layer for prefills of many rows
    // (MlaParams::kv_expanded), expand_keys keys; none when max_batch is
    // below the expanded path's row threshold or the shape has no such form
    uint16_t *kv_expanded = nullptr;
    long expand_keys = 0;
    float *router_logits = nullptr, *route_weights = nullptr;
    // router logit partials of one token row written by o_proj for the MoE
    // layer after it ([experts + 1][hidden / 8], GemvParams router_parts)
    float *router_parts = nullptr;
    int *route_ids = nullptr, *n_unique = nullptr, *unique = nullptr, *counts = nullptr;
    int *offsets = nullptr, *list_rows = nullptr, *list_slots = nullptr, *list_pos = nullptr;
    int *route_error = nullptr, *route_trace = nullptr, *ids = nullptr;
    ExpertTask *expert_tasks = nullptr;  // [experts] per-task table of the expert GEMVs
    // pre-split limb rows of the expert GEMV inputs (batches of 2+ rows)
    unsigned char *limb_x = nullptr, *limb_xs = nullptr, *limb_h = nullptr, *limb_sh = nullptr;
    long limb_x_stride = 0, limb_h_stride = 0, limb_sh_stride = 0;
    float *expert_hidden = nullptr, *expert_out = nullptr;
    float *shared_hidden = nullptr, *shared_out = nullptr, *dense_hidden = nullptr;
    float *shared_out2 = nullptr;  // second k half of the GEMM path's shared down
    float *moe_routed = nullptr;  // routed part of moonlight_test_moe
    // MFMA path for batches of >= kMoeGemmMinRows token rows
    // quantised activations: three limb planes [3][max_batch][aq_width]
    int8_t *aq = nullptr;
    long aq_plane = 0;
    float *aq_scale = nullptr;
    int aq_width = 0;
    // quantised expert hidden: three limb planes [3][max_batch*K][inter]
    int8_t *hq = nullptr;
    long hq_plane = 0;
    float *hq_scale = nullptr;
    GemmTask *gemm_tasks = nullptr;
    int *gemm_tile_start = nullptr;
    // router logits of every MoE layer of the last forward [L][max_batch][E]
    // (moonlight_session_trace_router; nullptr: not kept)
    float *router_trace = nullptr;
    // caller-given expert ids for the MoE test / timing hooks
    int *fixed_ids = nullptr;
    int fixed_rows = 0;
    // [position, ids...] of the current forward, on the device (pos_dev =
    // step_dev, ids = step_dev + 1) and in pinned host memory (one copy)
    int *step_dev = nullptr, *pos_dev = nullptr;
    int *host_step = nullptr, *host_ids = nullptr;
    int *host_flag = nullptr;
    float *host_logits = nullptr;  // pinned [vocab]: the D2H target, copied to the caller
    mlh::SampleWork sample;        // device sampler buffers (allocated on first use)
    int *host_sample = nullptr;    // pinned: sampler flag and token
    // one-row decode step (embed .. lm_head) as a graph: captured on the
    // second decode of the session, replayed at every later position; the
    // captured graph lives as long as its executable
    hipGraph_t decode_graph = nullptr;
    hipGraphExec_t decode_exec = nullptr;
    int eager_decodes = 0;
    bool decode_graph_failed = false, decode_graph_off = false;
    std::vector<int> kv_lengths;
    int last_forward_rows = 0;
    int position = 0;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    double last_device_ms = 0.0;
};

namespace {

// The model's device made current for the duration of an API call (the
// caller's current device is restored afterwards).
struct ApiScope : DeviceScope {
    explicit ApiScope(const MoonlightModel *m) : DeviceScope(m && m->ctx ? m->ctx->device : -1) {}
    explicit ApiScope(const MoonlightSession *s) : ApiScope(s ? s->model : nullptr) {}
};

}  // namespace

namespace {

// ---------------------------------------------------------------------------
// model: tensors and layer plans
// ---------------------------------------------------------------------------

const DeviceTensor *find_tensor(const MoonlightModel *m, const std::string &name) {
    auto it = m->index.find(name);
    return it == m->index.end() ? nullptr : &m->tensors[it->second];
}

// resolve_matrix (moonlight_metal.m:129-162): f32 of in*out elements, or U8
// with a `.qs` f32 scale of `out` elements and out*in (q8) or out*ceil(in/2)
// (q4) bytes.
bool resolve(const MoonlightModel *m, const std::string &name, int in_width, int out_width,
             Matrix *mat) {
    const DeviceTensor *t = find_tensor(m, name);
    if (!t) return false;
    mat->w = t->dev;
    mat->s = nullptr;
    if (t->dtype == kDtypeF32) {
        if (t->numel != (int64_t)in_width * out_width) return false;
        mat->fmt = kF32;
        return true;
    }
    if (t->dtype != kDtypeU8) return false;
    const DeviceTensor *st = find_tensor(m, name + ".qs");
    if (!st || st->dtype != kDtypeF32 || st->numel != out_width) return false;
    mat->s = reinterpret_cast<const float *>(st->dev);
    if (t->nbytes == (int64_t)out_width * in_width) {
        mat->fmt = kQ8;
        return true;
    }
    if (t->nbytes == (int64_t)out_width * ((in_width + 1) / 2)) {
        mat->fmt = kQ4;
        return true;
    }
    return false;
}

const float *vector_f32(const MoonlightModel *m, const std::string &name, int64_t numel) {
    const DeviceTensor *t = find_tensor(m, name);
    if (!t || t->dtype != kDtypeF32 || t->numel != numel) return nullptr;
    return reinterpret_cast<const float *>(t->dev);
}

std::string layer_name(int layer, const char *suffix) {
    char buf[256];
    snprintf(buf, sizeof(buf), "model.layers.%d.%s", layer, suffix);
    return buf;
}

// Resolves every tensor a forward needs, once, at model open (the reference
// resolves them per encode, moonlight_metal.m:307-329).  A missing or
// mis-sized tensor is recorded and reported when a forward reaches it.
bool build_plans(MoonlightModel *m, std::string *error) {
    const ModelConfig &c = m->cfg;
    m->layers.assign(c.layer_count, LayerPlan());
    std::vector<ExpertWeights> host_tables((size_t)c.layer_count * c.expert_count);
    const int qw = c.head_count * (c.qk_nope_dim + c.qk_rope_dim);
    const int cw = c.kv_lora_rank + c.qk_rope_dim;
    const int sw = c.moe_intermediate_size * c.shared_expert_count;
    for (int l = 0; l < c.layer_count; ++l) {
        LayerPlan &p = m->layers[l];
        auto need = [&](bool ok, const std::string &what) {
            if (!ok && p.error.empty()) p.error = "missing or mis-sized tensor " + what;
        };
        std::string n;
        n = layer_name(l, "self_attn.q_proj.weight");
        need(resolve(m, n, c.hidden_size, qw, &p.q), n);
        n = layer_name(l, "self_attn.kv_a_proj_with_mqa.weight");
        need(resolve(m, n, c.hidden_size, cw, &p.kv_a), n);
        n = layer_name(l, "self_attn.kv_b_proj.weight");
        need(resolve(m, n, c.kv_lora_rank, c.head_count * (c.qk_nope_dim + c.value_dim), &p.kv_b),
             n);
        n = layer_name(l, "self_attn.o_proj.weight");
        need(resolve(m, n, c.head_count * c.value_dim, c.hidden_size, &p.o), n);
        n = layer_name(l, "self_attn.kv_a_layernorm.weight");
        need((p.kv_norm = vector_f32(m, n, c.kv_lora_rank)) != nullptr, n);
        n = layer_name(l, "input_layernorm.weight");
        need((p.input_norm = vector_f32(m, n, c.hidden_size)) != nullptr, n);
        n = layer_name(l, "post_attention_layernorm.weight");
        need((p.post_norm = vector_f32(m, n, c.hidden_size)) != nullptr, n);
        p.dense = l < c.first_dense_layer_count;
        if (p.dense) {
            n = layer_name(l, "mlp.gate_proj.weight");
            need(resolve(m, n, c.hidden_size, c.dense_intermediate_size, &p.gate), n);
            n = layer_name(l, "mlp.up_proj.weight");
            need(resolve(m, n, c.hidden_size, c.dense_intermediate_size, &p.up), n);
            n = layer_name(l, "mlp.down_proj.weight");
            need(resolve(m, n, c.dense_intermediate_size, c.hidden_size, &p.down), n);
            if (p.error.empty() && (p.gate.fmt != p.up.fmt))
                p.error = "gate and up projections of layer " + std::to_string(l) +
                          " use different formats";
            continue;
        }
        n = layer_name(l, "mlp.gate.weight");
        need(resolve(m, n, c.hidden_size, c.expert_count, &p.router), n);
        n = layer_name(l, "mlp.gate.e_score_correction_bias");
        need((p.bias = vector_f32(m, n, c.expert_count)) != nullptr, n);
        n = layer_name(l, "mlp.shared_experts.gate_proj.weight");
        need(resolve(m, n, c.hidden_size, sw, &p.sh_gate), n);
        n = layer_name(l, "mlp.shared_experts.up_proj.weight");
        need(resolve(m, n, c.hidden_size, sw, &p.sh_up), n);
        n = layer_name(l, "mlp.shared_experts.down_proj.weight");
        need(resolve(m, n, sw, c.hidden_size, &p.sh_down), n);
        if (p.error.empty() && (p.sh_gate.fmt != p.sh_up.fmt || p.sh_gate.fmt != p.sh_down.fmt))
            p.error = "shared expert projections of layer " + std::to_string(l) +
                      " use different formats";
        for (int e = 0; e < c.expert_count; ++e) {
            Matrix g, u, d;
            char buf[256];
            snprintf(buf, sizeof(buf), "model.layers.%d.mlp.experts.%d.", l, e);
            const std::string base = buf;
            const bool ok = resolve(m, base + "gate_proj.weight", c.hidden_size,
                                    c.moe_intermediate_size, &g) &&
                            resolve(m, base + "up_proj.weight", c.hidden_size,
                                    c.moe_intermediate_size, &u) &&
                            resolve(m, base + "down_proj.weight", c.moe_intermediate_size,
                                    c.hidden_size, &d);
            need(ok, base + "{gate,up,down}_proj.weight");
            if (!ok) continue;
            if (e == 0) p.expert_fmt = g.fmt;
            if (p.error.empty() && (g.fmt != p.expert_fmt || u.fmt != g.fmt || d.fmt != g.fmt ||
                                    g.fmt == kF32))
                p.error = "routed experts of layer " + std::to_string(l) +
                          " must all use one quantized format";
            ExpertWeights &w = host_tables[(size_t)l * c.expert_count + e];
            w.gate = g.w;
            w.up = u.w;
            w.down = d.w;
            w.gate_s = g.s;
            w.up_s = u.s;
            w.down_s = d.s;
        }
    }
    if (!resolve(m, "lm_head.weight", c.hidden_size, c.vocab_size, &m->lm_head))
        m->head_error = "missing or mis-sized tensor lm_head.weight";
    m->embed = vector_f32(m, "model.embed_tokens.weight", (int64_t)c.vocab_size * c.hidden_size);
    m->final_norm = vector_f32(m, "model.norm.weight", c.hidden_size);
    if (!m->embed && m->head_error.empty()) m->head_error = "missing tensor model.embed_tokens.weight";
    if (!m->final_norm && m->head_error.empty()) m->head_error = "missing tensor model.norm.weight";

    // device tables: expert pointers per layer, RoPE inverse frequencies
    // theta^(-2p/rope) computed with the host libm powf exactly as the
    // reference's CPU check does (tests/test_moonlight_metal_mla.c:92-108)
    const size_t table_bytes = host_tables.size() * sizeof(ExpertWeights);
    std::vector<float> inv(c.qk_rope_dim / 2 > 0 ? c.qk_rope_dim / 2 : 1);
    for (int p = 0; p < c.qk_rope_dim / 2; ++p)
        inv[p] = powf(c.rope_theta, -2.0f * (float)p / (float)c.qk_rope_dim);
    if (hipMalloc((void **)&m->expert_tables, table_bytes ? table_bytes : 1) != hipSuccess ||
        hipMalloc((void **)&m->inv_freq, inv.size() * sizeof(float)) != hipSuccess) {
        *error = "cannot allocate model tables";
        return false;
    }
    if ((table_bytes && hipMemcpy(m->expert_tables, host_tables.data(), table_bytes,
                                  hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(m->inv_freq, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice) !=
            hipSuccess) {
        *error = "cannot upload model tables";
        return false;
    }
    for (int l = 0; l < c.layer_count; ++l)
        m->layers[l].expert_table = m->expert_tables + (size_t)l * c.expert_count;
    // [q_proj ; kv_a] row concatenation per layer: each row keeps its packed
    // bytes and its scale, only the placement changes
    for (int l = 0; l < c.layer_count; ++l) {
        LayerPlan &p = m->layers[l];
        p.qkv_a.fmt = -1;
        if (!p.error.empty() || p.q.fmt != p.kv_a.fmt) continue;
        const size_t rb = (size_t)(p.q.fmt == kF32 ? c.hidden_size * 4
                                   : p.q.fmt == kQ8 ? c.hidden_size : (c.hidden_size + 1) / 2);
        const size_t wbytes = (size_t)(qw + cw) * rb;
        const size_t sbytes = p.q.fmt == kF32 ? 0 : (size_t)(qw + cw) * sizeof(float);
        uint8_t *buf = nullptr;
        if (hipMalloc((void **)&buf, align256(wbytes) + sbytes) != hipSuccess) continue;
        m->extra.push_back(buf);
        bool ok = hipMemcpy(buf, p.q.w, (size_t)qw * rb, hipMemcpyDeviceToDevice) == hipSuccess &&
                  hipMemcpy(buf + (size_t)qw * rb, p.kv_a.w, (size_t)cw * rb,
                            hipMemcpyDeviceToDevice) == hipSuccess;
        float *sc = reinterpret_cast<float *>(buf + align256(wbytes));
        if (ok && sbytes)
            ok = hipMemcpy(sc, p.q.s, (size_t)qw * 4, hipMemcpyDeviceToDevice) == hipSuccess &&
                 hipMemcpy(sc + qw, p.kv_a.s, (size_t)cw * 4, hipMemcpyDeviceToDevice) ==
                     hipSuccess;
        if (!ok) continue;
        p.qkv_a.fmt = p.q.fmt;
        p.qkv_a.w = buf;
        p.qkv_a.s = sbytes ? sc : nullptr;
    }
    return true;
}

void free_model(MoonlightModel *m) {
    if (!m) return;
    if (m->arena) (void)hipFree(m->arena);
    if (m->expert_tables) (void)hipFree(m->expert_tables);
    if (m->inv_freq) (void)hipFree(m->inv_freq);
    for (void *p : m->extra) (void)hipFree(p);
    delete m;
}

bool place_tensors(MoonlightModel *m, std::string *error) {
    size_t total = 0;
    for (auto &t : m->tensors) total += align256((size_t)(t.nbytes > 0 ? t.nbytes : 1));
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess && total > free_b * 9 / 10) {
        char buf[256];
        snprintf(buf, sizeof(buf), "model requires %.2f GiB, above the free HBM budget %.2f GiB",
                 total / 1073741824.0, free_b * 0.9 / 1073741824.0);
        *error = buf;
        return false;
    }
    if (hipMalloc((void **)&m->arena, total ? total : 256) != hipSuccess) {
        *error = "HBM allocation of the model failed";
        return false;
    }
    m->arena_bytes = total;
    size_t off = 0;
    for (size_t i = 0; i < m->tensors.size(); ++i) {
        DeviceTensor &t = m->tensors[i];
        t.dev = m->arena + off;
        off += align256((size_t)(t.nbytes > 0 ? t.nbytes : 1));
        m->resident_bytes += (uint64_t)t.nbytes;
        if (!m->index.count(t.name)) m->index[t.name] = (int)i;
    }
    return true;
}

// Container upload (moonlight_metal.m:850-871 uploads tensor by tensor).  The
// arena places tensors in container order, contiguous up to 256-byte
// alignment, so a run of consecutive tensors fills one 64 MiB pinned staging
// buffer at its arena offsets (padding bytes are don't-care) and moves to HBM
// in one copy.  A pool of reader threads preads a stage's pieces (at most
// 4 MiB each) in parallel while the other buffer's copy runs.
// MLH_LOAD_THREADS overrides the reader count (default: up to 8);
// MLH_LOAD_STAGE_BYTES and MLH_LOAD_PIECE_BYTES override the stage and piece
// sizes (read at every model open; a piece is at most a stage).
static int load_threads() {
    const char *env = getenv("MLH_LOAD_THREADS");
    int n = env ? atoi(env) : 0;
    if (n <= 0) {
        const unsigned hw = std::thread::hardware_concurrency();
        n = hw == 0 ? 4 : (int)std::min(8u, hw);
    }
    return std::max(1, std::min(n, 64));
}

static size_t load_size(const char *name, size_t fallback) {
    const char *env = getenv(name);
    const long long v = env ? atoll(env) : 0;
    return v > 0 ? (size_t)v : fallback;
}

bool upload_container(MoonlightModel *m, const Container &ct, std::string *error) {
    const size_t kStage = load_size("MLH_LOAD_STAGE_BYTES", 64u << 20);
    const size_t kPiece = std::min(kStage, load_size("MLH_LOAD_PIECE_BYTES", 4u << 20));
    struct Piece {
        int tensor;
        int64_t offset;  // within the tensor
        size_t bytes;
        size_t arena;    // arena offset of the first byte
    };
    struct Stage {
        size_t first, last;  // pieces [first, last)
        size_t lo, hi;       // arena range
    };
    std::vector<Piece> pieces;
    std::vector<Stage> stages;
    for (size_t i = 0; i < m->tensors.size(); ++i) {
        const int64_t nbytes = ct.tensors()[i].nbytes;
        const size_t base = (size_t)(m->tensors[i].dev - m->arena);
        for (int64_t off = 0; off < nbytes; off += (int64_t)kPiece) {
            const size_t n = (size_t)std::min<int64_t>((int64_t)kPiece, nbytes - off);
            const size_t a = base + (size_t)off;
            if (stages.empty() || a + n - stages.back().lo > kStage)
                stages.push_back(Stage{pieces.size(), pieces.size(), a, a});
            pieces.push_back(Piece{(int)i, off, n, a});
            stages.back().last = pieces.size();
            stages.back().hi = a + n;
        }
    }
    DeviceContext *ctx = m->ctx;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool ok = hipHostMalloc(&stage[0], kStage, hipHostMallocDefault) == hipSuccess &&
              hipHostMalloc(&stage[1], kStage, hipHostMallocDefault) == hipSuccess &&
              hipEventCreateWithFlags(&done[0], hipEventDisableTiming) == hipSuccess &&
              hipEventCreateWithFlags(&done[1], hipEventDisableTiming) == hipSuccess;
    const int nthreads = load_threads();
    bool pending[2] = {false, false};
    int which = 0;
    for (size_t si = 0; ok && si < stages.size(); ++si) {
        const Stage &sg = stages[si];
        if (pending[which]) {
            ok = hipEventSynchronize(done[which]) == hipSuccess;
            pending[which] = false;
            if (!ok) break;
        }
        unsigned char *buf = static_cast<unsigned char *>(stage[which]);
        std::atomic<size_t> next(sg.first);
        std::atomic<int> failed(-1);
        auto reader = [&]() {
            for (size_t k = next++; k < sg.last; k = next++) {
                const Piece &pc = pieces[k];
                if (!ct.read_slice(pc.tensor, pc.offset, pc.bytes, buf + (pc.arena - sg.lo))) {
                    failed = pc.tensor;
                    return;
                }
            }
        };
        const size_t work = sg.last - sg.first;
        const int extra = (int)std::min<size_t>((size_t)nthreads, work) - 1;
        std::vector<std::thread> pool;
        for (int t = 0; t < extra; ++t) pool.emplace_back(reader);
        reader();
        for (std::thread &t : pool) t.join();
        if (failed >= 0) {
            *error = "cannot upload tensor " + ct.tensors()[(size_t)failed.load()].name;
            ok = false;
            break;
        }
        ok = hipMemcpyAsync(m->arena + sg.lo, buf, sg.hi - sg.lo, hipMemcpyHostToDevice,
                            ctx->stream) == hipSuccess &&
             hipEventRecord(done[which], ctx->stream) == hipSuccess;
        pending[which] = ok;
        which ^= 1;
    }
    if (ok) ok = hipStreamSynchronize(ctx->stream) == hipSuccess;
    for (int i = 0; i < 2; ++i) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    if (!ok && error->empty()) *error = "model upload failed";
    return ok;
}

}  // namespace

// ---------------------------------------------------------------------------
// model API
// ---------------------------------------------------------------------------

extern "C" int moonlight_model_open(MoonlightModel **out, const char *path, char *error,
                                    size_t error_size) {
    if (!out) return set_error(error, error_size, "model output is required");
    *out = nullptr;
    if (!path || !path[0]) return set_error(error, error_size, "model path is required");
    DeviceContext *ctx = context();
    if (!ctx) return set_error(error, error_size, "HIP device is unavailable: %s", last_error());
    Container ct;
    std::string why;
    if (!ct.open(path, &why)) return set_error(error, error_size, "%s", why.c_str());
    MoonlightModel *m = new MoonlightModel();
    m->ctx = ctx;
    m->cfg = ct.config();
    m->device_name = ctx->name;
    for (const TensorEntry &te : ct.tensors()) {
        DeviceTensor t;
        t.name = te.name;
        t.dtype = te.dtype;
        t.numel = te.numel;
        t.nbytes = te.nbytes;
        m->tensors.push_back(t);
    }
    if (!place_tensors(m, &why) || !upload_container(m, ct, &why) || !build_plans(m, &why)) {
        free_model(m);
        return set_error(error, error_size, "%s", why.c_str());
    }
    *out = m;
    return 1;
}

extern "C" void moonlight_model_close(MoonlightModel *model) {
    ApiScope api_scope(model);
    free_model(model);
}

extern "C" const char *moonlight_device_name(const MoonlightModel *model) {
    return model ? model->device_name.c_str() : "(none)";
}

extern "C" MoonlightModelInfo moonlight_model_info(const MoonlightModel *model) {
    MoonlightModelInfo r;
    memset(&r, 0, sizeof(r));
    if (!model) return r;
    const ModelConfig &c = model->cfg;
    r.hidden_size = c.hidden_size;
    r.layer_count = c.layer_count;
    r.vocab_size = c.vocab_size;
    r.head_count = c.head_count;
    r.kv_lora_rank = c.kv_lora_rank;
    r.qk_nope_dim = c.qk_nope_dim;
    r.qk_rope_dim = c.qk_rope_dim;
    r.value_dim = c.value_dim;
    r.expert_count = c.expert_count;
    r.experts_per_token = c.experts_per_token;
    r.moe_intermediate_size = c.moe_intermediate_size;
    r.shared_expert_count = c.shared_expert_count;
    r.first_dense_layer_count = c.first_dense_layer_count;
    r.rms_norm_epsilon = c.rms_norm_epsilon;
    r.rope_theta = c.rope_theta;
    r.routed_scale = c.routed_scale;
    r.resident_bytes = model->resident_bytes;
    return r;
}

extern "C" MoonlightSyntheticConfig moonlight_synthetic_moonlight_config(void) {
    MoonlightSyntheticConfig c;
    memset(&c, 0, sizeof(c));
    c.hidden_size = 2048;
    c.layer_count = 27;
    c.head_count = 16;
    c.expert_count = 64;
    c.experts_per_token = 6;
    c.dense_intermediate_size = 11264;
    c.moe_intermediate_size = 1408;
    c.first_dense_layer_count = 1;
    c.kv_lora_rank = 512;
    c.qk_nope_dim = 128;
    c.qk_rope_dim = 64;
    c.value_dim = 128;
    c.shared_expert_count = 2;
    c.normalize_topk = 1;
    c.vocab_size = 163840;
    c.rms_norm_epsilon = 1e-5f;
    c.rope_theta = 50000.0f;
    c.routed_scale = 2.446f;
    c.expert_bits = 8;
    c.dense_bits = 8;
    c.weight_std = 0.02f;
    c.seed = 1;
    return c;
}

namespace {

// One synthetic tensor: a packed matrix, an f32 matrix, a norm (ones) or the
// selection bias.
struct SynthSpec {
    std::string name;
    enum Kind { kPacked, kF32Matrix, kOnes, kBias } kind;
    int rows = 0, cols = 0, bits = 8;
};

void add_matrix(std::vector<SynthSpec> &v, const std::string &name, int rows, int cols, int bits) {
    v.push_back({name, SynthSpec::kPacked, rows, cols, bits});
}

}  // namespace

extern "C" int moonlight_model_create_synthetic(MoonlightModel **out,
                                                const MoonlightSyntheticConfig *sc, char *error,
                                                size_t error_size) {
    if (!out || !sc) return set_error(error, error_size, "model output and config are required");
    *out = nullptr;
    DeviceContext *ctx = context();
    if (!ctx) return set_error(error, error_size, "HIP device is unavailable: %s", last_error());
    if (sc->hidden_size <= 0 || sc->layer_count <= 0 || sc->head_count <= 0 ||
        sc->expert_count <= 0 || sc->experts_per_token <= 0 || sc->kv_lora_rank <= 0 ||
        sc->qk_rope_dim <= 0 || sc->vocab_size <= 0 ||
        (sc->expert_bits != 8 && sc->expert_bits != 4) ||
        (sc->dense_bits != 8 && sc->dense_bits != 4))
        return set_error(error, error_size, "unsupported synthetic Moonlight config");
    MoonlightModel *m = new MoonlightModel();
    m->ctx = ctx;
    ModelConfig &c = m->cfg;
    c.hidden_size = sc->hidden_size;
    c.layer_count = sc->layer_count;
    c.head_count = sc->head_count;
    c.expert_count = sc->expert_count;
    c.experts_per_token = sc->experts_per_token;
    c.dense_intermediate_size = sc->dense_intermediate_size;
    c.moe_intermediate_size = sc->moe_intermediate_size;
    c.first_dense_layer_count = sc->first_dense_layer_count;
    c.kv_lora_rank = sc->kv_lora_rank;
    c.qk_nope_dim = sc->qk_nope_dim;
    c.qk_rope_dim = sc->qk_rope_dim;
    c.value_dim = sc->value_dim;
    c.shared_expert_count = sc->shared_expert_count;
    c.normalize_topk = sc->normalize_topk;
    c.vocab_size = sc->vocab_size;
    c.rms_norm_epsilon = sc->rms_norm_epsilon;
    c.rope_theta = sc->rope_theta;
    c.routed_scale = sc->routed_scale;
    m->device_name = ctx->name;

    std::vector<SynthSpec> specs;
    const int H = c.hidden_size, eb = sc->expert_bits, db = sc->dense_bits;
    specs.push_back({"model.embed_tokens.weight", SynthSpec::kF32Matrix, c.vocab_size, H, 0});
    specs.push_back({"model.norm.weight", SynthSpec::kOnes, 1, H, 0});
    specs.push_back({"lm_head.weight", SynthSpec::kF32Matrix, c.vocab_size, H, 0});
    for (int l = 0; l < c.layer_count; ++l) {
        specs.push_back({layer_name(l, "input_layernorm.weight"), SynthSpec::kOnes, 1, H, 0});
        specs.push_back({layer_name(l, "post_attention_layernorm.weight"), SynthSpec::kOnes, 1, H, 0});
        add_matrix(specs, layer_name(l, "self_attn.q_proj.weight"),
                   c.head_count * (c.qk_nope_dim + c.qk_rope_dim), H, db);
        add_matrix(specs, layer_name(l, "self_attn.kv_a_proj_with_mqa.weight"),
                   c.kv_lora_rank + c.qk_rope_dim, H, db);
        specs.push_back({layer_name(l, "self_attn.kv_a_layernorm.weight"), SynthSpec::kOnes, 1,
                         c.kv_lora_rank, 0});
        add_matrix(specs, layer_name(l, "self_attn.kv_b_proj.weight"),
                   c.head_count * (c.qk_nope_dim + c.value_dim), c.kv_lora_rank, db);
        add_matrix(specs, layer_name(l, "self_attn.o_proj.weight"), H, c.head_count * c.value_dim,
                   db);
        if (l < c.first_dense_layer_count) {
            add_matrix(specs, layer_name(l, "mlp.gate_proj.weight"), c.dense_intermediate_size, H, db);
            add_matrix(specs, layer_name(l, "mlp.up_proj.weight"), c.dense_intermediate_size, H, db);
            add_matrix(specs, layer_name(l, "mlp.down_proj.weight"), H, c.dense_intermediate_size, db);
            continue;
        }
        specs.push_back({layer_name(l, "mlp.gate.weight"), SynthSpec::kF32Matrix, c.expert_count, H, 0});
        specs.push_back({layer_name(l, "mlp.gate.e_score_correction_bias"), SynthSpec::kBias, 1,
                         c.expert_count, 0});
        const int sw = c.moe_intermediate_size * c.shared_expert_count;
        add_matrix(specs, layer_name(l, "mlp.shared_experts.gate_proj.weight"), sw, H, db);
        add_matrix(specs, layer_name(l, "mlp.shared_experts.up_proj.weight"), sw, H, db);
        add_matrix(specs, layer_name(l, "mlp.shared_experts.down_proj.weight"), H, sw, db);
        for (int e = 0; e < c.expert_count; ++e) {
            char buf[256];
            snprintf(buf, sizeof(buf), "model.layers.%d.mlp.experts.%d.", l, e);
            add_matrix(specs, std::string(buf) + "down_proj.weight", H, c.moe_intermediate_size, eb);
            add_matrix(specs, std::string(buf) + "gate_proj.weight", c.moe_intermediate_size, H, eb);
            add_matrix(specs, std::string(buf) + "up_proj.weight", c.moe_intermediate_size, H, eb);
        }
    }
    // tensor table in container order: a packed matrix is followed by its scale
    size_t scratch_elems = 1;
    for (const SynthSpec &s : specs) {
        DeviceTensor t;
        t.name = s.name;
        if (s.kind == SynthSpec::kPacked) {
            t.dtype = kDtypeU8;
            t.nbytes = (int64_t)s.rows * (s.bits == 8 ? s.cols : (s.cols + 1) / 2);
            t.numel = t.nbytes;
            m->tensors.push_back(t);
            DeviceTensor qs;
            qs.name = s.name + ".qs";
            qs.dtype = kDtypeF32;
            qs.numel = s.rows;
            qs.nbytes = (int64_t)s.rows * 4;
            m->tensors.push_back(qs);
            scratch_elems = std::max(scratch_elems, (size_t)s.rows * s.cols);
        } else {
            t.dtype = kDtypeF32;
            t.numel = (int64_t)s.rows * s.cols;
            t.nbytes = t.numel * 4;
            m->tensors.push_back(t);
        }
    }
    std::string why;
    if (!place_tensors(m, &why)) {
        free_model(m);
        return set_error(error, error_size, "%s", why.c_str());
    }
    float *scratch = nullptr;
    std::vector<float> host_small;
    bool ok = hipMalloc((void **)&scratch, scratch_elems * sizeof(float)) == hipSuccess;
    uint64_t stream_id = 0;
    for (const SynthSpec &s : specs) {
        if (!ok) break;
        const DeviceTensor &t = m->tensors[m->index[s.name]];
        const uint64_t seed = sc->seed * 0x9E3779B97F4A7C15ULL + 1000003ULL * (++stream_id);
        if (s.kind == SynthSpec::kPacked) {
            const DeviceTensor &qs = m->tensors[m->index[s.name + ".qs"]];
            ok = fill_normal(scratch, (int64_t)s.rows * s.cols, seed, 0.0f, sc->weight_std, 1,
                             ctx->stream) == kOk &&
                 quantize_rows(s.bits, scratch, s.rows, s.cols, t.dev,
                               reinterpret_cast<float *>(qs.dev), ctx->stream) == kOk;
        } else if (s.kind == SynthSpec::kF32Matrix) {
            ok = fill_normal(reinterpret_cast<float *>(t.dev), t.numel, seed, 0.0f, sc->weight_std,
                             1, ctx->stream) == kOk;
        } else {
            host_small.assign((size_t)t.numel, 1.0f);
            if (s.kind == SynthSpec::kBias)
                for (int64_t i = 0; i < t.numel; ++i)
                    host_small[i] = t.numel > 1 ? -0.1f + 0.2f * (float)i / (float)(t.numel - 1)
                                                : 0.0f;
            ok = hipMemcpyAsync(t.dev, host_small.data(), t.nbytes, hipMemcpyHostToDevice,
                                ctx->stream) == hipSuccess &&
                 hipStreamSynchronize(ctx->stream) == hipSuccess;
        }
    }
    if (ok) ok = hipStreamSynchronize(ctx->stream) == hipSuccess;
    if (scratch) (void)hipFree(scratch);
    if (!ok || !build_plans(m, &why)) {
        free_model(m);
        return set_error(error, error_size, "synthetic model generation failed: %s",
                         why.empty() ? "device error" : why.c_str());
    }
    *out = m;
    return 1;
}

extern "C" int moonlight_container_probe(const char *path, int *ints16, float *floats3,
                                         char *error, size_t error_size) {
    if (!path || !ints16 || !floats3) {
        set_error(error, error_size, "path and outputs are required");
        return -1;
    }
    Container ct;
    std::string why;
    if (!ct.open(path, &why)) {
        set_error(error, error_size, "%s", why.c_str());
        return -1;
    }
    const ModelConfig &c = ct.config();
    const int v[16] = {c.hidden_size, c.layer_count, c.head_count, c.expert_count,
                       c.experts_per_token, c.dense_intermediate_size, c.moe_intermediate_size,
                       c.first_dense_layer_count, c.q_lora_rank, c.kv_lora_rank, c.qk_nope_dim,
                       c.qk_rope_dim, c.value_dim, c.shared_expert_count, c.normalize_topk,
                       c.vocab_size};
    memcpy(ints16, v, sizeof(v));
    floats3[0] = c.rms_norm_epsilon;
    floats3[1] = c.rope_theta;
    floats3[2] = c.routed_scale;
    return (int)ct.tensors().size();
}

extern "C" int moonlight_container_tensor(const char *path, const char *name, int *dtype,
                                          int64_t *numel, int64_t *nbytes) {
    if (!path || !name) return 0;
    Container ct;
    std::string why;
    if (!ct.open(path, &why)) return 0;
    const int i = ct.find(name);
    if (i < 0) return 0;
    const TensorEntry &t = ct.tensors()[i];
    if (dtype) *dtype = t.dtype;
    if (numel) *numel = t.numel;
    if (nbytes) *nbytes = t.nbytes;
    return 1;
}

extern "C" size_t moonlight_model_read_tensor(const MoonlightModel *model, const char *name,
                                              void *dst, size_t capacity) {
    if (!model || !name || !dst) return 0;
    const DeviceTensor *t = find_tensor(model, name);
    if (!t || (size_t)t->nbytes > capacity) return 0;
    ApiScope api_scope(model);
    DeviceContext *ctx = model->ctx;
    if (!ctx || hipMemcpyAsync(dst, t->dev, (size_t)t->nbytes, hipMemcpyDeviceToHost,
                               ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess)
        return 0;
    return (size_t)t->nbytes;
}

extern "C" int moonlight_model_tensor_info(const MoonlightModel *model, const char *name,
                                           int *dtype, int64_t *numel, int64_t *nbytes) {
    if (!model || !name) return 0;
    const DeviceTensor *t = find_tensor(model, name);
    if (!t) return 0;
    if (dtype) *dtype = t->dtype;
    if (numel) *numel = t->numel;
    if (nbytes) *nbytes = t->nbytes;
    return 1;
}

// ---------------------------------------------------------------------------
// session
// ---------------------------------------------------------------------------

namespace {

bool mul_ok(size_t a, size_t b, size_t *r) {
    if (b && a > SIZE_MAX / b) return false;
    *r = a * b;
    return true;
}

template <typename T>
bool session_alloc(MoonlightSession *s, T **ptr, size_t elems, char *error, size_t error_size) {
    size_t bytes;
    if (!mul_ok(elems ? elems : 1, sizeof(T), &bytes)) {
        set_error(error, error_size, "Moonlight session size overflow");
        return false;
    }
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        set_error(error, error_size, "HBM allocation failed: %zu bytes", bytes);
        return false;
    }
    s->allocations.push_back(p);
    s->stats.buffer_allocations++;
    s->stats.resident_bytes += bytes;
    *ptr = static_cast<T *>(p);
    return true;
}

void free_session(MoonlightSession *s) {
    if (!s) return;
    for (void *p : s->allocations) (void)hipFree(p);
    if (s->decode_exec) (void)hipGraphExecDestroy(s->decode_exec);
    if (s->decode_graph) (void)hipGraphDestroy(s->decode_graph);
    if (s->router_trace) (void)hipFree(s->router_trace);
    if (s->host_step) (void)hipHostFree(s->host_step);
    if (s->host_logits) (void)hipHostFree(s->host_logits);
    if (s->host_flag) (void)hipHostFree(s->host_flag);
    if (s->host_sample) (void)hipHostFree(s->host_sample);
    mlh::sample_free(&s->sample);
    if (s->ev_start) (void)hipEventDestroy(s->ev_start);
    if (s->ev_stop) (void)hipEventDestroy(s->ev_stop);
    delete s;
}

hipStream_t stream_of(const MoonlightSession *s) { return s->model->ctx->stream; }

// Synchronises the stream (one "command buffer" in the reference's sense).
bool finish(MoonlightSession *s) {
    s->stats.command_buffers++;
    return hipStreamSynchronize(stream_of(s)) == hipSuccess;
}

bool to_device(MoonlightSession *s, void *dst, const void *src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_of(s)) == hipSuccess;
}

bool to_host(MoonlightSession *s, void *dst, const void *src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_of(s)) == hipSuccess;
}

// Batches of at least this many token rows take the int8-MFMA GEMM (weights
// read once per 32 or 128 rows) instead of the GEMV (once per 4 rows).  The
// MoE layer switches at 3 rows: the grouped GEMM streams each active
// expert once for all its rows in one launch per stage, with the routing in
// its first launch, while the grouped GEMV runs a routing launch, two stage
// launches and a combine (measured on MI355X, whole layer: equal at T = 2,
// 53.5 us; 58 against 74 us at T = 3, 64 against 92 us at T = 4).  The
// dense projections keep the GEMV up to 16 rows.
constexpr int kGemmMinRows = 16;
constexpr int kMoeGemmMinRows = 3;

bool use_gemm(const MoonlightSession *s, int fmt, int rows, int in_w) {
    return rows >= kGemmMinRows && s->aq && in_w <= s->aq_width && qgemm_shape_ok(fmt, in_w);
}

int gemm_rows(MoonlightSession *s, const Matrix &m, const Matrix *up, const float *x, int rows,
              int in_w, int out_w, float *y, const float *norm_w, const float *resid) {
    hipStream_t st = stream_of(s);
    if (int e = quantize_activations(x, in_w, rows, in_w, norm_w, s->model->cfg.rms_norm_epsilon,
                                     s->aq, s->aq_plane, s->aq_scale, st))
        return e;
    GemmTask t;
    t.w = m.w;
    t.s = m.s;
    if (up) {
        t.w2 = up->w;
        t.s2 = up->s;
    }
    t.rows = rows;
    t.n_out = out_w;
    t.k = in_w;
    t.a = s->aq;
    t.a_plane = s->aq_plane;
    t.a_scale = s->aq_scale;
    t.a_stride = in_w;
    t.y = y;
    t.y_stride = out_w;
    t.resid = resid;
    t.resid_stride = out_w;
    return qgemm_single(m.fmt, up != nullptr, t, st);
}

// Router partials of a one-row GEMV's output for the next MoE layer (see
// GemvParams router_parts).
struct RouterFuse {
    const float *w = nullptr, *nw = nullptr;
    float *parts = nullptr;
    int experts = 0;
};

int gemv_rows(MoonlightSession *s, const Matrix &m, const float *x, int rows, int in_w,
              int out_w, float *y, const float *norm_w = nullptr, const float *resid = nullptr,
              const RouterFuse *rf = nullptr) {
    if (!rf && use_gemm(s, m.fmt, rows, in_w))
        return gemm_rows(s, m, nullptr, x, rows, in_w, out_w, y, norm_w, resid);
    GemvParams p;
    p.fmt = m.fmt;
    p.w = m.w;
    p.s = m.s;
    p.O = out_w;
    p.I = in_w;
    p.rows = rows;
    p.x = x;
    p.x_stride = in_w;
    p.norm_w = norm_w;
    p.eps = s->model->cfg.rms_norm_epsilon;
    p.y = y;
    p.y_stride = out_w;
    p.resid = resid;
    p.resid_stride = out_w;
    p.epilogue = resid ? kEpiResidual : kEpiPlain;
    if (rf) {
        p.router_w = rf->w;
        p.router_nw = rf->nw;
        p.router_parts = rf->parts;
        p.router_experts = rf->experts;
    }
    return gemv(p, stream_of(s));
}

int swiglu_rows(MoonlightSession *s, const Matrix &g, const Matrix &u, const float *x, int rows,
                int in_w, int width, float *h, const float *norm_w) {
    if (g.fmt == u.fmt && use_gemm(s, g.fmt, rows, in_w))
        return gemm_rows(s, g, &u, x, rows, in_w, width, h, norm_w, nullptr);
    GemvParams p;
    p.fmt = g.fmt;
    p.w = g.w;
    p.s = g.s;
    p.w2 = u.w;
    p.s2 = u.s;
    p.O = width;
    p.I = in_w;
    p.rows = rows;
    p.x = x;
    p.x_stride = in_w;
    p.norm_w = norm_w;
    p.eps = s->model->cfg.rms_norm_epsilon;
    p.y = h;
    p.y_stride = width;
    p.epilogue = kEpiSiluDual;
    return gemv(p, stream_of(s));
}

// Attention of `layer` for `rows` rows of (already normalised) x at
// `position`; writes o_proj(ctx) (+ resid) into out.
// position_dev: the position in device memory (forward); with grid_splits
// the attend grid is fixed (decode graph capture).
int attention(MoonlightSession *s, int layer, const float *x, int rows, int position,
              float *out, const float *norm_w, const float *resid,
              const int *position_dev = nullptr, int grid_splits = 0,
              const RouterFuse *rf = nullptr) {
    const ModelConfig &c = s->model->cfg;
    const LayerPlan &lp = s->model->layers[layer];
    const int qw = c.head_count * (c.qk_nope_dim + c.qk_rope_dim);
    const int cw = c.kv_lora_rank + c.qk_rope_dim;
    MlaParams p;
    if (lp.qkv_a.fmt >= 0) {
        // one launch: [q | compressed] rows of width qw + cw
        if (gemv_rows(s, lp.qkv_a, x, rows, c.hidden_size, qw + cw, s->query, norm_w))
            return kErrLaunch;
        p.query = s->query;
        p.query_stride = qw + cw;
        p.compressed = s->query + qw;
        p.compressed_stride = qw + cw;
    } else {
        if (gemv_rows(s, lp.q, x, rows, c.hidden_size, qw, s->query, norm_w)) return kErrLaunch;
        if (gemv_rows(s, lp.kv_a, x, rows, c.hidden_size, cw, s->compressed, norm_w))
            return kErrLaunch;
        p.query = s->query;
        p.query_stride = qw;
        p.compressed = s->compressed;
        p.compressed_stride = cw;
    }
    p.rows = rows;
    p.position = position;
    p.position_dev = position_dev;
    p.grid_splits = grid_splits;
    p.heads = c.head_count;
    p.nope = c.qk_nope_dim;
    p.rope = c.qk_rope_dim;
    p.vdim = c.value_dim;
    p.latent = c.kv_lora_rank;
    p.eps = c.rms_norm_epsilon;
    p.scale = 1.0f / sqrtf((float)(c.qk_nope_dim + c.qk_rope_dim));
    p.kv_norm = lp.kv_norm;
    p.inv_freq = s->model->inv_freq;
    p.kv_b.fmt = lp.kv_b.fmt;
    p.kv_b.w = lp.kv_b.w;
    p.kv_b.s = lp.kv_b.s;
    p.latent_cache = s->latent_kv + (size_t)layer * s->options.context_size * c.kv_lora_rank;
    p.latent_split =
        s->latent_split + (size_t)layer * s->options.context_size * 2 * c.kv_lora_rank;
    p.rope_cache = s->rope_kv + (size_t)layer * s->options.context_size * c.qk_rope_dim;
    p.query_rope = s->query_rope;
    p.query_absorbed = s->query_absorbed;
    p.max_splits = s->max_splits;
    p.part_max = s->part_max;
    p.part_sum = s->part_sum;
    p.part_lc = s->part_lc;
    p.latent_context = s->latent_ctx;
    p.kv_expanded = s->kv_expanded;
    p.expand_keys = s->expand_keys;
    p.context = s->context;
    p.value_part = s->value_part;
    p.merge_count = s->merge_count;
    p.range_error = s->route_error;  // the forward's error word (route errors: layer + 1)
    p.range_code = -(layer + 1);
    if (int e = mla_attention_core(p, stream_of(s))) return e;
    return gemv_rows(s, lp.o, s->context, rows, c.head_count * c.value_dim, c.hidden_size, out,
                     nullptr, resid, rf);
}

// Expert GEMV batches of at least this many token rows split their inputs
// into limb rows once per stage (limb_quantise_rows) rather than in every
// workgroup.
constexpr int kPresplitMinRows = 2;

// The MFMA router (32 x 32 tiles, one workgroup per tile) has the
// parallelism for prefill batches.  Up to 16 rows take router_logits_small
// (one workgroup per expert; measured on MI355X, MoE layer at T = 8: 7.5
// against 8.4 us for the GEMV; at T = 64, four row groups, 12.0 against
// 11.2 us), the rows between the GEMV.
constexpr int kRouterMfmaMinRows = 256;
constexpr int kRouterSmallMaxRows = 16;

// fixed: the MoE test / timing hooks take the caller's expert ids when set
// (moonlight_session_fix_routes); forward passes always route by top-k.
// Single-row batches with at most 64 experts route inside the first expert
// launch, and their down projections and combine run as one launch.

// With `inline_route`, a single-row batch with at most 64 experts gets only
// its router logits here; the selection and the route tables are left to
// the first expert launch, which takes *inline_route (route.logits unset
// when routing ran here).
// Whether the MoE layer of a batch of `rows` token rows runs on the grouped
// int8-MFMA GEMM (moe_gemm) rather than the grouped GEMV.
static bool moe_uses_gemm(const MoonlightSession *s, int layer, int rows) {
    const ModelConfig &c = s->model->cfg;
    const LayerPlan &lp = s->model->layers[layer];
    const int sw = c.moe_intermediate_size * c.shared_expert_count;
    return rows >= kMoeGemmMinRows && s->hq && qgemm_shape_ok(lp.expert_fmt, c.hidden_size) &&
           qgemm_shape_ok(lp.expert_fmt, c.moe_intermediate_size) &&
           qgemm_shape_ok(lp.sh_gate.fmt, c.hidden_size) && qgemm_shape_ok(lp.sh_gate.fmt, sw) &&
           c.hidden_size <= s->aq_width && sw <= s->aq_width;
}

// Partials per expert that o_proj of `layer` writes for the router of the
// same layer when one token row can take the fused router (the layer is an
// MoE layer routed inside its first expert launch, f32 router, o_proj on the
// int8 matrix-core GEMV), else 0.
int router_fuse_parts(const MoonlightSession *s, int layer) {
    const ModelConfig &c = s->model->cfg;
    const LayerPlan &lp = s->model->layers[layer];
    if (lp.dense || lp.router.fmt != kF32 || c.expert_count > 64 || c.experts_per_token > 64 ||
        !lp.post_norm || ((uintptr_t)lp.router.w & 15u) ||
        c.hidden_size % 4)
        return 0;
    GemvParams p;
    p.fmt = lp.o.fmt;
    p.w = lp.o.w;
    p.O = c.hidden_size;
    p.I = c.head_count * c.value_dim;
    p.rows = 1;
    p.x = s->context;
    p.x_stride = p.I;
    p.epilogue = kEpiResidual;
    if (!gemv_router_ok(p)) return 0;
    const int n = gemv_router_parts(p);
    // logits_from_parts: a power of two from 16 to 256
    return n >= 16 && n <= 256 && (n & (n - 1)) == 0 && n <= c.hidden_size / 8 + 1 ? n : 0;
}

// fused_parts > 0 (one token row, router_fuse_parts): o_proj has written
// the router logit partials; no router launch, the first expert launch
// derives the logits (and stores them in router_logits).
int route(MoonlightSession *s, int layer, const float *x, int rows, const float *norm_w,
          int *trace, bool fixed = false, RouteParams *inline_route = nullptr,
          int fused_parts = 0) {
    const ModelConfig &c = s->model->cfg;
    const LayerPlan &lp = s->model->layers[layer];
    const bool f32_router = lp.router.fmt == kF32;
    const float *router_w = reinterpret_cast<const float *>(lp.router.w);
    if (fused_parts > 0) {
        if (rows != 1 || !inline_route || fixed) return kErrArgs;
    } else if (rows >= kRouterMfmaMinRows && f32_router && c.hidden_size % 16 == 0) {
        if (router_logits(x, norm_w, c.rms_norm_epsilon, router_w, rows, c.expert_count,
                          c.hidden_size, s->router_logits, stream_of(s)))
            return kErrLaunch;
    } else if (f32_router && rows <= kRouterSmallMaxRows && c.hidden_size % 8 == 0) {
        if (router_logits_small(x, norm_w, c.rms_norm_epsilon, router_w, rows, c.expert_count,
                                c.hidden_size, s->router_logits, stream_of(s)))
            return kErrLaunch;
    } else if (gemv_rows(s, lp.router, x, rows, c.hidden_size, c.expert_count,
                         s->router_logits, norm_w)) {
        return kErrLaunch;
    }
    RouteParams r;
    r.logits = s->router_logits;
    r.bias = lp.bias;
    r.rows = rows;
    r.experts = c.expert_count;
    r.top_k = c.experts_per_token;
    r.normalize = c.normalize_topk;
    r.routed_scale = c.routed_scale;
    r.ids = s->route_ids;
    r.weights = s->route_weights;
    r.trace = trace;
    r.n_unique = s->n_unique;
    r.unique = s->unique;
    r.counts = s->counts;
    r.offsets = s->offsets;
    r.list_rows = s->list_rows;
    r.list_slots = s->list_slots;
    r.list_pos = s->list_pos;
    r.error = s->route_error;
    r.error_code = layer + 1;
    r.fixed_ids = fixed && s->fixed_rows >= rows ? s->fixed_ids : nullptr;
    r.expert_table = lp.expert_table;
    r.tasks = s->expert_tasks;
    r.task_slots = rows * r.top_k < r.experts ? rows * r.top_k : r.experts;
    if (inline_route) *inline_route = RouteParams{};
    if (fused_parts > 0) {
        r.logit_parts = s->router_parts;
        r.logits_out = s->router_logits;
        r.n_parts = fused_parts;
        r.width = c.hidden_size;
        r.eps = c.rms_norm_epsilon;
        *inline_route = r;
        return kOk;
    }
    if (inline_route && rows == 1 && c.expert_count <= 64 && rows < kPresplitMinRows) {
        *inline_route = r;
        return kOk;
    }
    // a few rows on the GEMM path: the first GEMM launch routes them
    if (inline_route && rows <= kRouteOneGroupRows &&
        rows * r.top_k <= kRouteFusedMaxPositions && r.top_k <= kMaxTopK && r.experts <= 64 &&
        moe_uses_gemm(s, layer, rows)) {
        *inline_route = r;
        inline_route->tasks = nullptr;  // the GEMM path builds its own task tables
        return kOk;
    }
    return route_topk(r, stream_of(s));
}

int experts(MoonlightSession *s, int layer, const float *x, int rows, const float *norm_w,
            const float *resid, float *out, float *routed_copy,
            const RouteParams *inline_route = nullptr) {
    const ModelConfig &c = s->model->cfg;
    const LayerPlan &lp = s->model->layers[layer];
    ExpertFfnParams f;
    f.rows = rows;
    f.experts = c.expert_count;
    f.top_k = c.experts_per_token;
    f.hidden = c.hidden_size;
    f.inter = c.moe_intermediate_size;
    f.shared_width = c.moe_intermediate_size * c.shared_expert_count;
    f.expert_fmt = lp.expert_fmt;
    f.shared_fmt = lp.sh_gate.fmt;
    f.has_shared = 1;
    f.expert_table = lp.expert_table;
    f.shared_gate = lp.sh_gate.w;
    f.shared_up = lp.sh_up.w;
    f.shared_down = lp.sh_down.w;
    f.shared_gate_s = lp.sh_gate.s;
    f.shared_up_s = lp.sh_up.s;
    f.shared_down_s = lp.sh_down.s;
    f.n_unique = s->n_unique;
    f.unique = s->unique;
    f.counts = s->counts;
    f.offsets = s->offsets;
    f.list_rows = s->list_rows;
    f.tasks = s->expert_tasks;  // written by route() (or by stage 0 routing inline)
    if (inline_route && inline_route->logits) f.route = *inline_route;
    if (rows >= kPresplitMinRows && c.hidden_size % 32 == 0 &&
        c.moe_intermediate_size % 32 == 0) {
        f.limb_x = s->limb_x;
        f.limb_xs = s->limb_xs;
        f.limb_h = s->limb_h;
        f.limb_sh = s->limb_sh;
        f.limb_x_stride = s->limb_x_stride;
        f.limb_h_stride = s->limb_h_stride;
        f.limb_sh_stride = s->limb_sh_stride;
    }
    f.x = x;
    f.norm_w = norm_w;
    f.eps = c.rms_norm_epsilon;
    f.expert_hidden = s->expert_hidden;
    f.expert_out = s->expert_out;
    f.shared_hidden = s->shared_hidden;
    f.shared_out = s->shared_out;
    const bool gemm = moe_uses_gemm(s, layer, rows);
    // the GEMM path runs a shared down projection twice inter wide as two k
    // halves into shared_out and shared_out2 (moe_shared_down_parts)
    const bool split_shared = gemm && f.shared_width == 2 * f.inter;
    if (gemm) {
        MoeGemmParams g;
        g.rows = f.rows;
        g.experts = f.experts;
        g.top_k = f.top_k;
        g.hidden = f.hidden;
        g.inter = f.inter;
        g.shared_width = f.shared_width;
        g.expert_fmt = f.expert_fmt;
        g.shared_fmt = f.shared_fmt;
        g.has_shared = 1;
        if (inline_route && inline_route->logits) {
            g.route = *inline_route;  // route() left the routing to the first launch
            g.route_in_prep = 1;
        }
        g.expert_table = f.expert_table;
        g.shared_gate = f.shared_gate;
        g.shared_up = f.shared_up;
        g.shared_down = f.shared_down;
        g.shared_gate_s = f.shared_gate_s;
        g.shared_up_s = f.shared_up_s;
        g.shared_down_s = f.shared_down_s;
        g.n_unique = f.n_unique;
        g.unique = f.unique;
        g.counts = f.counts;
        g.offsets = f.offsets;
        g.list_rows = f.list_rows;
        g.x = f.x;
        g.norm_w = f.norm_w;
        g.eps = f.eps;
        // the token-row quantisation is consumed by stage 0 before the shared
        // hidden is quantised into the same buffer
        g.xq = g.sq = s->aq;
        g.xq_plane = g.sq_plane = s->aq_plane;
        g.xq_scale = g.sq_scale = s->aq_scale;
        g.hq = s->hq;
        g.hq_plane = s->hq_plane;
        g.hq_scale = s->hq_scale;
        g.tasks = s->gemm_tasks;
        g.tile_start = s->gemm_tile_start;
        g.expert_hidden = f.expert_hidden;
        g.expert_out = f.expert_out;
        g.shared_hidden = f.shared_hidden;
        g.shared_out = f.shared_out;
        g.shared_out2 = split_shared ? s->shared_out2 : nullptr;
        if (int e = moe_gemm(g, stream_of(s))) return e;
    } else {
        const bool fused_down = down_combine_ok(f);
        if (fused_down) {
            f.combine_out = out;
            f.combine_resid = resid;
            f.combine_routed = routed_copy;
            f.combine_shared = routed_copy ? s->shared_out : nullptr;  // test hook reads it
            f.route_weights = s->route_weights;
            f.list_pos = s->list_pos;
        }
        if (int e = expert_ffn(f, stream_of(s))) return e;
        if (fused_down) return kOk;
    }
    CombineParams cb;
    cb.rows = rows;
    cb.hidden = c.hidden_size;
    cb.top_k = c.experts_per_token;
    cb.weights = s->route_weights;
    cb.list_pos = s->list_pos;
    cb.expert_out = s->expert_out;
    cb.shared_out = s->shared_out;
    cb.shared_out2 = split_shared ? s->shared_out2 : nullptr;
    cb.resid = resid;
    cb.routed_copy = routed_copy;
    cb.out = out;
    return moe_combine(cb, stream_of(s));
}

// Token rows of one routing call: each routes at most kRouteMaxPositions
// (row, slot) positions (the route-table kernels keep them in LDS).
int moe_chunk_rows(const ModelConfig &c) {
    const int k = c.experts_per_token > 0 ? c.experts_per_token : 1;
    return kRouteMaxPositions / k;
}

// The kernels of one forward over `count` token rows at `start` (embed,
// layers, final norm + lm_head), reading the ids and the position uploaded
// to step_dev.  With `graph` the attend grids are sized for the whole
// context so the captured launches fit every later position.
bool enqueue_forward(MoonlightSession *s, int count, int start, float *layer_outputs, bool graph) {
    MoonlightModel *m = s->model;
    const ModelConfig &c = m->cfg;
    hipStream_t st = stream_of(s);
    const size_t H = (size_t)c.hidden_size;
    const int grid_splits = graph ? s->max_splits : 0;
    bool ok = embed_rows(m->embed, s->ids, s->h, count, c.hidden_size, c.vocab_size,
                         s->route_error, st) == kOk;
    for (int l = 0; ok && l < c.layer_count; ++l) {
        const LayerPlan &lp = m->layers[l];
        // one row: o_proj also writes the router logit partials of the MoE
        // layer's router (no router launch)
        const int fused = count == 1 ? router_fuse_parts(s, l) : 0;
        RouterFuse rf;
        if (fused) {
            rf.w = reinterpret_cast<const float *>(lp.router.w);
            rf.nw = lp.post_norm;
            rf.parts = s->router_parts;
            rf.experts = c.expert_count;
        }
        ok = attention(s, l, s->h, count, start, s->h, lp.input_norm, s->h, s->pos_dev,
                       grid_splits, fused ? &rf : nullptr) == kOk;
        if (ok && lp.dense) {
            ok = swiglu_rows(s, lp.gate, lp.up, s->h, count, c.hidden_size,
                             c.dense_intermediate_size, s->dense_hidden, lp.post_norm) == kOk &&
                 gemv_rows(s, lp.down, s->dense_hidden, count, c.dense_intermediate_size,
                           c.hidden_size, s->h, nullptr, s->h) == kOk;
        } else if (ok) {
            // one routing call covers at most kRouteMaxPositions (row, slot)
            // positions: larger batches run the MoE block in row chunks (a
            // row's experts are summed in its slot order, so the chunks do
            // not change any row's arithmetic)
            const int chunk = moe_chunk_rows(c);
            for (int r0 = 0; ok && r0 < count; r0 += chunk) {
                const int n = std::min(chunk, count - r0);
                float *hr = s->h + (size_t)r0 * H;
                const size_t row_base = (size_t)l * s->options.max_batch + (size_t)r0;
                int *trace = s->route_trace + row_base * c.experts_per_token;
                RouteParams inline_r;
                ok = route(s, l, hr, n, lp.post_norm, trace, false, &inline_r, fused) == kOk;
                ok = ok && experts(s, l, hr, n, lp.post_norm, hr, hr, nullptr, &inline_r) == kOk;
                // the router logits exist once the first expert launch has run
                // (they come from o_proj's partials there when fused)
                if (ok && s->router_trace)
                    ok = hipMemcpyAsync(s->router_trace + row_base * c.expert_count,
                                        s->router_logits, (size_t)n * c.expert_count * 4,
                                        hipMemcpyDeviceToDevice, st) == hipSuccess;
            }
        }
        if (ok && layer_outputs)
            ok = to_host(s, layer_outputs + (size_t)l * count * H, s->h, (size_t)count * H * 4);
    }
    return ok && gemv_rows(s, m->lm_head, s->h + (size_t)(count - 1) * H, 1, c.hidden_size,
                           c.vocab_size, s->logits, m->final_norm) == kOk;
}

// Captures the one-row decode kernels into s->decode_exec.  The capture runs
// nothing; a failure leaves the session on the eager path.  The graph is kept
// until the executable is destroyed (drop_decode_graph / free_session).
bool capture_decode(MoonlightSession *s, int start) {
    hipStream_t st = stream_of(s);
    if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) return false;
    const bool ok = enqueue_forward(s, 1, start, nullptr, true);
    hipGraph_t graph = nullptr;
    const bool ended = hipStreamEndCapture(st, &graph) == hipSuccess;
    hipGraphExec_t exec = nullptr;
    const bool built = ok && ended && graph &&
                       hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    (void)hipGetLastError();
    if (!built) {
        if (graph) (void)hipGraphDestroy(graph);
        return false;
    }
    s->decode_graph = graph;
    s->decode_exec = exec;
    return true;
}

// Drops the captured decode graph (its launches baked in state that changed).
void drop_decode_graph(MoonlightSession *s) {
    if (s->decode_exec) (void)hipGraphExecDestroy(s->decode_exec);
    if (s->decode_graph) (void)hipGraphDestroy(s->decode_graph);
    s->decode_exec = nullptr;
    s->decode_graph = nullptr;
}

// A next-token choice made on the device after the forward (choose_token,
// moonlight_chat.c:96-131); u is the caller's draw.
struct SampleRequest {
    float temperature = 0.0f, top_p = 1.0f;
    double u = 0.0;
    int *token = nullptr;
};

static bool sampler_ready(MoonlightSession *s) {
    if (s->sample.ctl && s->host_sample) return true;
    if (!s->host_sample &&
        hipHostMalloc((void **)&s->host_sample, 2 * sizeof(int), hipHostMallocDefault) != hipSuccess) {
        s->host_sample = nullptr;
        return false;
    }
    return mlh::sample_alloc(&s->sample, s->model->cfg.vocab_size) == 0;
}

// run_tokens_fast (moonlight_metal.m:1892-1986) as one device submission: a
// graph replay for one-row decode steps, else the launches in stream order.
// With `pick` the step ends in a device-side token choice and the logits stay
// on the device (last_logits may then be null).
int forward(MoonlightSession *s, const int *ids, int count, int start, float *last_logits,
            float *layer_outputs, char *error, size_t error_size,
            const SampleRequest *pick = nullptr) {
    MoonlightModel *m = s->model;
    const ModelConfig &c = m->cfg;
    if (!m->head_error.empty())
        return set_error(error, error_size, "Moonlight fast final projection failed: %s",
                         m->head_error.c_str());
    for (int i = 0; i < count; ++i)
        if (ids[i] < 0 || ids[i] >= c.vocab_size)
            return set_error(error, error_size, "Moonlight fast embedding failed");
    for (int l = 0; l < c.layer_count; ++l) {
        if (!m->layers[l].error.empty())
            return set_error(error, error_size, "Moonlight fast %s failed at layer %d: %s",
                             l < c.first_dense_layer_count ? "dense block" : "MoE", l,
                             m->layers[l].error.c_str());
        if (s->kv_lengths[l] != start)
            return set_error(error, error_size,
                             "Moonlight fast sparse attention failed at layer %d", l);
    }
    if (pick && !sampler_ready(s))
        return set_error(error, error_size, "Moonlight sampler allocation failed");
    hipStream_t st = stream_of(s);
    // MOONLIGHT_PROFILE (moonlight_metal.m:1899, 1932-1937, 1972-1979): one
    // line per submission on stderr; a forward here is one submission
    const bool profile = getenv("MOONLIGHT_PROFILE") != nullptr;
    const double command_start = profile ? monotonic_seconds() : 0.0;
    double wait_start = 0.0;
    s->host_step[0] = start;
    memcpy(s->host_ids, ids, (size_t)count * sizeof(int));
    const bool decode = count == 1 && !layer_outputs &&
                        !s->decode_graph_off && !s->decode_graph_failed;
    // the first decode runs eagerly (lazy per-kernel set-up happens outside
    // any capture); the second captures
    if (decode && !s->decode_exec && s->eager_decodes >= 1 && !capture_decode(s, start))
        s->decode_graph_failed = true;
    bool ok = hipEventRecord(s->ev_start, st) == hipSuccess &&
              to_device(s, s->step_dev, s->host_step, (size_t)(count + 1) * sizeof(int));
    if (ok && decode && s->decode_exec) {
        ok = hipGraphLaunch(s->decode_exec, st) == hipSuccess;
    } else if (ok) {
        ok = enqueue_forward(s, count, start, layer_outputs, false);
        if (decode) s->eager_decodes++;
    }
    if (ok && pick)
        ok = mlh::sample_enqueue(&s->sample, s->logits, pick->temperature, pick->top_p, pick->u,
                                 st) == kOk &&
             to_host(s, s->host_sample, s->sample.ctl + 2, 2 * sizeof(int));
    ok = ok && hipEventRecord(s->ev_stop, st) == hipSuccess &&
         (!last_logits ||
          to_host(s, s->host_logits, s->logits, (size_t)c.vocab_size * sizeof(float))) &&
         to_host(s, s->host_flag, s->route_error, sizeof(int));
    if (profile) wait_start = monotonic_seconds();
    if (!finish(s) || !ok) {
        // the device state of a partial forward is unusable: invalidate the caches
        for (int l = 0; l < c.layer_count; ++l)
            if (s->kv_lengths[l] > start) s->kv_lengths[l] = start;
        return set_error(error, error_size, "Moonlight forward failed on the device: %s",
                         hipGetErrorString(hipGetLastError()));
    }
    const double wait_end = profile ? monotonic_seconds() : 0.0;
    for (int l = 0; l < c.layer_count; ++l) s->kv_lengths[l] = start + count;
    if (last_logits) memcpy(last_logits, s->host_logits, (size_t)c.vocab_size * sizeof(float));
    if (*s->host_flag > 0)
        return set_error(error, error_size, "Moonlight fast route table failed at layer %d",
                         *s->host_flag - 1);
    if (*s->host_flag < 0)
        return set_error(error, error_size,
                         "Moonlight attention failed at layer %d: a query or key value is "
                         "outside the f16 range of the split-f16 attention products",
                         -*s->host_flag - 1);
    // the forward is committed: a failed token choice below leaves the
    // session at the new position, ready for the next decode
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, s->ev_start, s->ev_stop) == hipSuccess) s->last_device_ms = ms;
    if (profile)
        fprintf(stderr,
                "moonlight profile rows=%d start=%d layers=%d graph=%d encode=%.3f wait=%.3f "
                "gpu=%.3f ms\n",
                count, start, c.layer_count, decode && s->decode_exec ? 1 : 0,
                (wait_start - command_start) * 1000.0, (wait_end - wait_start) * 1000.0,
                s->last_device_ms);
    s->position = start + count;
    s->last_forward_rows = count;
    if (pick) {
        if (s->host_sample[0])
            return set_error(error, error_size, "Moonlight sampler: logits are not finite");
        *pick->token = s->host_sample[1];
    }
    return 1;
}

}  // namespace

extern "C" int moonlight_session_create(MoonlightSession **out, MoonlightModel *model,
                                        const MoonlightOptions *options, char *error,
                                        size_t error_size) {
    ApiScope api_scope(model);
    if (!out || !model || !options)
        return set_error(error, error_size, "model and session options are required");
    *out = nullptr;
    if (options->context_size <= 0 || options->max_batch <= 0 ||
        options->max_batch > options->context_size)
        return set_error(error, error_size, "invalid context or batch size");
    const ModelConfig &c = model->cfg;
    if (c.kv_lora_rank > 512 || c.qk_rope_dim > 256 || (c.qk_rope_dim & 1) ||
        c.expert_count > 256 || c.experts_per_token > c.expert_count ||
        // limits of the HIP kernels (mla.h, moe.hip)
        // (the attention's fp32-MFMA score tiles take the rope part 16 dims
        // at a time)
        c.head_count > kMlaMaxHeads || c.kv_lora_rank % 64 || c.qk_rope_dim > 64 ||
        c.qk_rope_dim % 16 ||
        c.qk_nope_dim > 256 || c.qk_nope_dim <= 0 || c.value_dim <= 0 || c.experts_per_token > 16)
        return set_error(error, error_size, "unsupported Moonlight MLA dimensions");
    if (c.q_lora_rank)
        return set_error(error, error_size, "unsupported Moonlight MLA dimensions");
    MoonlightSession *s = new MoonlightSession();
    s->model = model;
    s->options = *options;
    s->stats.resident_bytes = model->resident_bytes;
    const size_t mb = (size_t)options->max_batch, ctx = (size_t)options->context_size;
    const size_t H = (size_t)c.hidden_size, L = (size_t)c.layer_count, E = (size_t)c.expert_count;
    const size_t K = (size_t)c.experts_per_token;
    const size_t heads = (size_t)c.head_count;
    // attend partials per row: one per workgroup, at most one per key tile
    s->max_splits = (int)std::min<size_t>((ctx + kMlaTileKeys - 1) / kMlaTileKeys,
                                          (size_t)kMlaAttendGroups);
    const size_t splits = (size_t)s->max_splits;
    // the split-attention (decode) path runs at most kMlaDecodeRows rows per launch group
    const size_t dr = mb < (size_t)kMlaDecodeRows ? mb : (size_t)kMlaDecodeRows;
    const size_t sw = (size_t)c.moe_intermediate_size * c.shared_expert_count;
    // the expanded prefill keys: the whole context up to kMlaExpandMaxKeys,
    // when every layer's kv_b has the expanded form
    size_t expand_bytes = 0;
    for (int l = 0; l < c.layer_count; ++l) {
        const size_t b = mla_expand_kv_bytes(c.head_count, c.qk_nope_dim, c.qk_rope_dim,
                                             c.value_dim, c.kv_lora_rank,
                                             s->model->layers[l].kv_b.fmt);
        if (!b) {
            expand_bytes = 0;
            break;
        }
        expand_bytes = b;
    }
    if (expand_bytes && mb >= (size_t)kMlaExpandMinRows)
        s->expand_keys = (long)std::min<size_t>((ctx + 63) / 64 * 64, (size_t)kMlaExpandMaxKeys);
    size_t lat_elems, rope_elems, lc_elems, logit_elems;
    if (!mul_ok(L * ctx, (size_t)c.kv_lora_rank, &lat_elems) ||
        !mul_ok(L * ctx, (size_t)c.qk_rope_dim, &rope_elems) ||
        !mul_ok(dr * splits * kMlaMaxHeads, (size_t)c.kv_lora_rank, &lc_elems) ||
        !mul_ok(mb, (size_t)c.vocab_size, &logit_elems)) {
        delete s;
        return set_error(error, error_size, "Moonlight session size overflow");
    }
    const bool ok =
        session_alloc(s, &s->h, mb * H, error, error_size) &&
        session_alloc(s, &s->tmp, mb * H, error, error_size) &&
        session_alloc(s, &s->latent_kv, lat_elems, error, error_size) &&
        session_alloc(s, &s->latent_split, 2 * lat_elems, error, error_size) &&
        session_alloc(s, &s->rope_kv, rope_elems, error, error_size) &&
        session_alloc(s, &s->step_dev, mb + 1, error, error_size) &&
        (s->pos_dev = s->step_dev, s->ids = s->step_dev + 1, true) &&
        session_alloc(s, &s->logits, logit_elems, error, error_size) &&
        session_alloc(s, &s->query,
                      mb * (heads * (c.qk_nope_dim + c.qk_rope_dim) + c.kv_lora_rank +
                            c.qk_rope_dim),
                      error, error_size) &&
        session_alloc(s, &s->compressed, mb * (c.kv_lora_rank + c.qk_rope_dim), error,
                      error_size) &&
        session_alloc(s, &s->context, mb * heads * c.value_dim, error, error_size) &&
        session_alloc(s, &s->query_rope, mb * heads * c.qk_rope_dim, error, error_size) &&
        session_alloc(s, &s->query_absorbed, mb * heads * c.kv_lora_rank, error, error_size) &&
        session_alloc(s, &s->part_max, dr * splits * kMlaMaxHeads, error, error_size) &&
        session_alloc(s, &s->part_sum, dr * splits * kMlaMaxHeads, error, error_size) &&
        session_alloc(s, &s->part_lc, lc_elems, error, error_size) &&
        session_alloc(s, &s->value_part,
                      dr * heads * (c.kv_lora_rank / kMlaValueDims) * (size_t)c.value_dim, error,
                      error_size) &&
        session_alloc(s, &s->merge_count, dr * heads * kMlaCountStride, error, error_size) &&
        hipMemset(s->merge_count, 0, dr * heads * kMlaCountStride * sizeof(int)) == hipSuccess &&
        session_alloc(s, &s->latent_ctx, mb * heads * c.kv_lora_rank, error, error_size) &&
        (s->expand_keys == 0 ||
         session_alloc(s, &s->kv_expanded, (size_t)s->expand_keys * expand_bytes / sizeof(uint16_t),
                       error, error_size)) &&
        session_alloc(s, &s->router_logits, mb * E, error, error_size) &&
        session_alloc(s, &s->router_parts, (size_t)(E + 1) * (c.hidden_size / 8 + 1), error,
                      error_size) &&
        session_alloc(s, &s->route_ids, mb * K, error, error_size) &&
        session_alloc(s, &s->route_weights, mb * K, error, error_size) &&
        session_alloc(s, &s->n_unique, 1, error, error_size) &&
        session_alloc(s, &s->unique, E, error, error_size) &&
        session_alloc(s, &s->counts, E, error, error_size) &&
        session_alloc(s, &s->offsets, E, error, error_size) &&
        session_alloc(s, &s->list_rows, mb * K, error, error_size) &&
        session_alloc(s, &s->list_slots, mb * K, error, error_size) &&
        session_alloc(s, &s->list_pos, mb * K, error, error_size) &&
        session_alloc(s, &s->route_error, 1, error, error_size) &&
        session_alloc(s, &s->expert_tasks, E, error, error_size) &&
        // limb rows sized for q8 (the larger layout) so any format fits
        (s->limb_x_stride = limb_row_lds(kQ8, c.hidden_size),
         s->limb_h_stride = limb_row_lds(kQ8, c.moe_intermediate_size > 0 ? c.moe_intermediate_size : 16),
         s->limb_sh_stride = limb_row_lds(kQ8, sw > 0 ? (int)sw : 16), true) &&
        session_alloc(s, &s->limb_x, mb * s->limb_x_stride, error, error_size) &&
        session_alloc(s, &s->limb_xs, mb * s->limb_x_stride, error, error_size) &&
        session_alloc(s, &s->limb_h, mb * K * s->limb_h_stride, error, error_size) &&
        session_alloc(s, &s->limb_sh, mb * s->limb_sh_stride, error, error_size) &&
        session_alloc(s, &s->route_trace, L * mb * K, error, error_size) &&
        session_alloc(s, &s->expert_hidden, mb * K * (size_t)c.moe_intermediate_size, error,
                      error_size) &&
        session_alloc(s, &s->expert_out, mb * K * H, error, error_size) &&
        session_alloc(s, &s->shared_hidden, mb * (sw ? sw : 1), error, error_size) &&
        session_alloc(s, &s->shared_out, mb * H, error, error_size) &&
        session_alloc(s, &s->shared_out2, mb * H, error, error_size) &&
        session_alloc(s, &s->moe_routed, mb * H, error, error_size) &&
        session_alloc(s, &s->dense_hidden,
                      mb * (size_t)(c.dense_intermediate_size > 0 ? c.dense_intermediate_size : 1),
                      error, error_size) &&
        session_alloc(s, &s->fixed_ids, mb * K, error, error_size) &&
        hipHostMalloc((void **)&s->host_step, (mb + 1) * sizeof(int), hipHostMallocDefault) ==
            hipSuccess &&
        (s->host_ids = s->host_step + 1, true) &&
        hipHostMalloc((void **)&s->host_flag, sizeof(int), hipHostMallocDefault) == hipSuccess &&
        hipHostMalloc((void **)&s->host_logits, (size_t)c.vocab_size * sizeof(float),
                      hipHostMallocDefault) == hipSuccess &&
        hipEventCreate(&s->ev_start) == hipSuccess && hipEventCreate(&s->ev_stop) == hipSuccess;
    bool gemm_ok = ok;
    if (ok && options->max_batch >= kMoeGemmMinRows) {
        // MFMA prefill scratch: quantised activations of the widest matmul
        // input, quantised expert hidden rows, per-stage task tables
        const int widths[] = {c.hidden_size, c.head_count * c.value_dim,
                              c.dense_intermediate_size, (int)sw};
        int aw = 0;
        for (int w : widths) aw = w > aw ? w : aw;
        s->aq_width = aw;
        s->aq_plane = (long)(mb * (size_t)aw);
        s->hq_plane = (long)(mb * K * (size_t)c.moe_intermediate_size);
        gemm_ok = session_alloc(s, &s->aq, 3 * (size_t)s->aq_plane, error, error_size) &&
                  session_alloc(s, &s->aq_scale, mb, error, error_size) &&
                  session_alloc(s, &s->hq, 3 * (size_t)s->hq_plane, error, error_size) &&
                  session_alloc(s, &s->hq_scale, mb * K, error, error_size) &&
                  session_alloc(s, &s->gemm_tasks, 2 * (size_t)kQgMaxTasks, error, error_size) &&
                  session_alloc(s, &s->gemm_tile_start, 2 * (size_t)(kQgMaxTasks + 1), error,
                                error_size);
    }
    if (!ok || !gemm_ok) {
        free_session(s);
        if (error && error_size && !error[0]) set_error(error, error_size, "session allocation failed");
        return 0;
    }
    s->kv_lengths.assign(c.layer_count, 0);
    *out = s;
    return 1;
}

extern "C" void moonlight_session_destroy(MoonlightSession *session) {
    ApiScope api_scope(session);
    free_session(session);
}

extern "C" void moonlight_session_reset(MoonlightSession *s) {
    ApiScope api_scope(s);
    if (!s) return;
    s->position = 0;
    s->last_forward_rows = 0;
    std::fill(s->kv_lengths.begin(), s->kv_lengths.end(), 0);
    s->stats.command_buffers = 0;
    s->stats.prefill_tokens = 0;
    s->stats.decode_tokens = 0;
    s->stats.cpu_fallbacks = 0;
    s->stats.prefill_ms = 0;
    s->stats.decode_ms = 0;
}

extern "C" int moonlight_session_position(const MoonlightSession *s) {
    return s ? s->position : 0;
}

extern "C" MoonlightStats moonlight_session_stats(const MoonlightSession *s) {
    MoonlightStats r;
    memset(&r, 0, sizeof(r));
    return s ? s->stats : r;
}

extern "C" int moonlight_session_prefill(MoonlightSession *s, const int *ids, int count,
                                         float *last_logits, char *error, size_t error_size) {
    ApiScope api_scope(s);
    if (!s || !ids || !last_logits || count <= 0 || count > s->options.max_batch ||
        count > s->options.context_size)
        return set_error(error, error_size, "invalid Moonlight prefill request");
    if (s->position != 0)
        return set_error(error, error_size, "Moonlight prefill requires an empty session");
    const double t0 = monotonic_seconds();
    if (!forward(s, ids, count, 0, last_logits, nullptr, error, error_size)) return 0;
    s->stats.prefill_tokens += (uint64_t)count;
    s->stats.prefill_ms += (monotonic_seconds() - t0) * 1000.0;
    return 1;
}

extern "C" int moonlight_session_append(MoonlightSession *s, const int *ids, int count,
                                        float *last_logits, char *error, size_t error_size) {
    ApiScope api_scope(s);
    if (!s || !ids || !last_logits || count <= 0 || count > s->options.max_batch ||
        s->position <= 0 || s->position + count > s->options.context_size)
        return set_error(error, error_size, "invalid Moonlight append request");
    const double t0 = monotonic_seconds();
    if (!forward(s, ids, count, s->position, last_logits, nullptr, error, error_size)) return 0;
    s->stats.prefill_tokens += (uint64_t)count;
    s->stats.prefill_ms += (monotonic_seconds() - t0) * 1000.0;
    return 1;
}

extern "C" int moonlight_session_decode(MoonlightSession *s, int token, float *logits,
                                        char *error, size_t error_size) {
    ApiScope api_scope(s);
    if (!s || !logits || s->position < 0 || s->position >= s->options.context_size)
        return set_error(error, error_size, "invalid Moonlight decode request");
    const double t0 = monotonic_seconds();
    if (!forward(s, &token, 1, s->position, logits, nullptr, error, error_size)) return 0;
    s->stats.decode_tokens++;
    s->stats.decode_ms += (monotonic_seconds() - t0) * 1000.0;
    return 1;
}

// random_unit (moonlight_chat.c:89-94): one xorshift64 (13, 7, 17) step, top
// 53 bits as a double in [0, 1).
static double random_unit(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (double)(x >> 11) * (1.0 / 9007199254740992.0);
}

extern "C" int moonlight_session_sample(MoonlightSession *s, float temperature, float top_p,
                                        uint64_t *rng_state, int *token, char *error,
                                        size_t error_size) {
    ApiScope api_scope(s);
    if (!s || !token || s->position <= 0 || (temperature > 0.0f && !rng_state))
        return set_error(error, error_size, "invalid Moonlight sample request");
    if (!sampler_ready(s)) return set_error(error, error_size, "Moonlight sampler allocation failed");
    // the caller's state advances only when a token is returned
    uint64_t state = rng_state ? *rng_state : 0;
    const double u = temperature > 0.0f ? random_unit(&state) : 0.0;
    bool ok = mlh::sample_enqueue(&s->sample, s->logits, temperature, top_p, u, stream_of(s)) ==
                  kOk &&
              to_host(s, s->host_sample, s->sample.ctl + 2, 2 * sizeof(int));
    if (!finish(s) || !ok)
        return set_error(error, error_size, "Moonlight sampler failed on the device: %s",
                         hipGetErrorString(hipGetLastError()));
    if (s->host_sample[0]) return set_error(error, error_size, "Moonlight sampler: logits are not finite");
    *token = s->host_sample[1];
    if (temperature > 0.0f) *rng_state = state;
    return 1;
}

extern "C" int moonlight_session_decode_sample(MoonlightSession *s, int token, float temperature,
                                               float top_p, uint64_t *rng_state, int *next_token,
                                               char *error, size_t error_size) {
    ApiScope api_scope(s);
    if (!s || !next_token || s->position < 0 || s->position >= s->options.context_size ||
        (temperature > 0.0f && !rng_state))
        return set_error(error, error_size, "invalid Moonlight decode request");
    SampleRequest pick;
    pick.temperature = temperature;
    pick.top_p = top_p;
    uint64_t state = rng_state ? *rng_state : 0;
    pick.u = temperature > 0.0f ? random_unit(&state) : 0.0;
    pick.token = next_token;
    const double t0 = monotonic_seconds();
    const int before = s->position;
    const bool chosen =
        forward(s, &token, 1, s->position, nullptr, nullptr, error, error_size, &pick) != 0;
    if (s->position == before) return 0;  // the forward itself failed
    // the step is decoded (KV appended, position advanced) even when the
    // token choice failed; the caller's state advances only with a token
    s->stats.decode_tokens++;
    s->stats.decode_ms += (monotonic_seconds() - t0) * 1000.0;
    if (!chosen) return 0;
    if (temperature > 0.0f) *rng_state = state;
    return 1;
}

extern "C" int moonlight_test_prefill_layers(MoonlightSession *s, const int *ids, int count,
                                             float *layer_outputs, float *last_logits,
                                             char *error, size_t error_size) {
    ApiScope api_scope(s);
    if (!s || !ids || !layer_outputs || !last_logits || count <= 0 ||
        count > s->options.max_batch || s->position != 0)
        return set_error(error, error_size, "invalid Moonlight layer trace request");
    const double t0 = monotonic_seconds();
    if (!forward(s, ids, count, 0, last_logits, layer_outputs, error, error_size)) return 0;
    s->stats.prefill_tokens += (uint64_t)count;
    s->stats.prefill_ms += (monotonic_seconds() - t0) * 1000.0;
    return 1;
}

// ---------------------------------------------------------------------------
// test hooks (moonlight_metal.m:1188-1812, 2055-2070)
// ---------------------------------------------------------------------------

extern "C" int moonlight_test_embed(MoonlightSession *s, const int *ids, int count, float *output) {
    ApiScope api_scope(s);
    if (!s || !ids || !output || count <= 0 || count > s->options.max_batch) return 0;
    const ModelConfig &c = s->model->cfg;
    if (!s->model->embed) return 0;
    for (int i = 0; i < count; ++i)
        if (ids[i] < 0 || ids[i] >= c.vocab_size) return 0;
    memcpy(s->host_ids, ids, (size_t)count * sizeof(int));
    const size_t bytes = (size_t)count * c.hidden_size * sizeof(float);
    bool ok = to_device(s, s->ids, s->host_ids, (size_t)count * sizeof(int)) &&
              embed_rows(s->model->embed, s->ids, s->h, count, c.hidden_size, c.vocab_size,
                         nullptr, stream_of(s)) == kOk &&
              to_host(s, output, s->h, bytes);
    return finish(s) && ok;
}

extern "C" int moonlight_test_rmsnorm(MoonlightSession *s, const float *input,
                                      const char *weight_name, int rows, int width,
                                      float *output) {
    ApiScope api_scope(s);
    if (!s || !input || !weight_name || !output || rows <= 0 || width <= 0 ||
        rows > s->options.max_batch)
        return 0;
    const float *w = vector_f32(s->model, weight_name, width);
    if (!w) return 0;
    const size_t bytes = (size_t)rows * width * sizeof(float);
    if (bytes > (size_t)s->options.max_batch * s->model->cfg.hidden_size * sizeof(float))
        return 0;
    bool ok = to_device(s, s->tmp, input, bytes) &&
              rmsnorm_rows(s->tmp, w, s->h, rows, width, s->model->cfg.rms_norm_epsilon, width,
                           width, stream_of(s)) == kOk &&
              to_host(s, output, s->h, bytes);
    return finish(s) && ok;
}

extern "C" int moonlight_test_matmul(MoonlightSession *s, const char *weight_name,
                                     const float *input, int rows, int input_width,
                                     int output_width, float *output) {
    ApiScope api_scope(s);
    if (!s || !weight_name || !input || !output || rows <= 0 || input_width <= 0 ||
        output_width <= 0 || rows > s->options.max_batch)
        return 0;
    Matrix m;
    if (!resolve(s->model, weight_name, input_width, output_width, &m)) return 0;
    const ModelConfig &c = s->model->cfg;
    const size_t in_bytes = (size_t)rows * input_width * sizeof(float);
    const size_t out_bytes = (size_t)rows * output_width * sizeof(float);
    if (in_bytes > (size_t)s->options.max_batch * c.hidden_size * sizeof(float) ||
        out_bytes > (size_t)s->options.max_batch * c.vocab_size * sizeof(float))
        return 0;
    bool ok = to_device(s, s->tmp, input, in_bytes) &&
              gemv_rows(s, m, s->tmp, rows, input_width, output_width, s->logits) == kOk &&
              to_host(s, output, s->logits, out_bytes);
    return finish(s) && ok;
}

extern "C" int moonlight_test_attention(MoonlightSession *s, int layer, const float *input,
                                        int rows, int position, float *output) {
    ApiScope api_scope(s);
    if (!s || !input || !output || rows <= 0 || position < 0 || rows > s->options.max_batch)
        return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer < 0 || layer >= c.layer_count || position != s->kv_lengths[layer] ||
        position + rows > s->options.context_size || c.q_lora_rank)
        return 0;
    if (!s->model->layers[layer].error.empty()) return 0;
    const size_t bytes = (size_t)rows * c.hidden_size * sizeof(float);
    hipStream_t st = stream_of(s);
    bool ok = to_device(s, s->tmp, input, bytes) &&
              hipMemsetAsync(s->route_error, 0, sizeof(int), st) == hipSuccess &&
              attention(s, layer, s->tmp, rows, position, s->h, nullptr, nullptr) == kOk &&
              to_host(s, output, s->h, bytes) &&
              to_host(s, s->host_flag, s->route_error, sizeof(int));
    if (!finish(s) || !ok || *s->host_flag) return 0;
    s->kv_lengths[layer] = position + rows;
    if (s->position < position + rows) s->position = position + rows;
    return 1;
}

extern "C" int moonlight_test_kv_length(const MoonlightSession *s, int layer) {
    if (!s || layer < 0 || layer >= s->model->cfg.layer_count) return 0;
    return s->kv_lengths[layer];
}

extern "C" int moonlight_test_copy_kv(const MoonlightSession *s, int layer, float *latent,
                                      float *rope, int capacity) {
    ApiScope api_scope(s);
    if (!s || !latent || !rope || capacity < 0) return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer < 0 || layer >= c.layer_count || capacity < s->kv_lengths[layer]) return 0;
    const size_t n = (size_t)s->kv_lengths[layer];
    const size_t ctx = (size_t)s->options.context_size;
    hipStream_t st = s->model->ctx->stream;
    bool ok = hipMemcpyAsync(latent, s->latent_kv + (size_t)layer * ctx * c.kv_lora_rank,
                             n * c.kv_lora_rank * sizeof(float), hipMemcpyDeviceToHost,
                             st) == hipSuccess &&
              hipMemcpyAsync(rope, s->rope_kv + (size_t)layer * ctx * c.qk_rope_dim,
                             n * c.qk_rope_dim * sizeof(float), hipMemcpyDeviceToHost,
                             st) == hipSuccess &&
              hipStreamSynchronize(st) == hipSuccess;
    return ok ? 1 : 0;
}

extern "C" int moonlight_test_moe(MoonlightSession *s, int layer, const float *input, int rows,
                                  int *route_ids, float *route_weights, float *router_scores,
                                  float *routed_output, float *shared_output, float *output) {
    ApiScope api_scope(s);
    if (!s || !input || !output || rows <= 0 || rows > s->options.max_batch) return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer < c.first_dense_layer_count || layer >= c.layer_count || c.expert_count <= 0 ||
        c.experts_per_token <= 0 || c.shared_expert_count <= 0)
        return 0;
    if (!s->model->layers[layer].error.empty()) return 0;
    const size_t hidden_bytes = (size_t)rows * c.hidden_size * sizeof(float);
    hipStream_t st = stream_of(s);
    if (!to_device(s, s->tmp, input, hidden_bytes)) return 0;
    // two submissions per routing chunk (moe_chunk_rows rows; one chunk up to
    // 2730 Moonlight rows): router + top-k (+ device route tables), then the
    // experts, the shared expert and routed + shared (no residual)
    const int chunk = moe_chunk_rows(c);
    const size_t H = (size_t)c.hidden_size, K = (size_t)c.experts_per_token;
    const size_t E = (size_t)c.expert_count;
    for (int r0 = 0; r0 < rows; r0 += chunk) {
        const int n = std::min(chunk, rows - r0);
        const float *x = s->tmp + (size_t)r0 * H;
        bool ok = hipMemsetAsync(s->route_error, 0, sizeof(int), st) == hipSuccess &&
                  route(s, layer, x, n, nullptr, nullptr, true) == kOk &&
                  to_host(s, s->host_flag, s->route_error, sizeof(int));
        if (!finish(s) || !ok || *s->host_flag) return 0;
        float *out_dev = s->h + (size_t)r0 * H;
        float *routed_dev = s->moe_routed + (size_t)r0 * H;
        ok = experts(s, layer, x, n, nullptr, nullptr, out_dev, routed_dev) == kOk;
        const size_t rb = (size_t)n * K * sizeof(float), hb = (size_t)n * H * sizeof(float);
        if (ok && route_ids) ok = to_host(s, route_ids + r0 * K, s->route_ids, rb);
        if (ok && route_weights) ok = to_host(s, route_weights + r0 * K, s->route_weights, rb);
        if (ok && router_scores)
            ok = to_host(s, router_scores + r0 * E, s->router_logits, (size_t)n * E * sizeof(float));
        if (ok && shared_output) ok = to_host(s, shared_output + r0 * H, s->shared_out, hb);
        if (r0 + n == rows) {
            if (ok && routed_output) ok = to_host(s, routed_output, s->moe_routed, hidden_bytes);
            if (ok) ok = to_host(s, output, s->h, hidden_bytes);
        }
        if (!finish(s) || !ok) return 0;
    }
    return 1;
}

extern "C" int moonlight_test_dense_mlp(MoonlightSession *s, int layer, const float *input,
                                        int rows, float *output) {
    ApiScope api_scope(s);
    if (!s || !input || !output || rows <= 0 || rows > s->options.max_batch) return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer < 0 || layer >= c.layer_count || !s->model->layers[layer].dense ||
        !s->model->layers[layer].error.empty())
        return 0;
    const LayerPlan &lp = s->model->layers[layer];
    const size_t bytes = (size_t)rows * c.hidden_size * sizeof(float);
    bool ok = to_device(s, s->tmp, input, bytes) &&
              swiglu_rows(s, lp.gate, lp.up, s->tmp, rows, c.hidden_size,
                          c.dense_intermediate_size, s->dense_hidden, nullptr) == kOk &&
              gemv_rows(s, lp.down, s->dense_hidden, rows, c.dense_intermediate_size,
                        c.hidden_size, s->h) == kOk &&
              to_host(s, output, s->h, bytes);
    return finish(s) && ok;
}

extern "C" int moonlight_test_copy_routes(const MoonlightSession *s, int layer, int *route_ids,
                                          int capacity) {
    ApiScope api_scope(s);
    if (!s || !route_ids || capacity < s->last_forward_rows) return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer < c.first_dense_layer_count || layer >= c.layer_count) return 0;
    hipStream_t st = s->model->ctx->stream;
    const size_t n = (size_t)s->last_forward_rows * c.experts_per_token;
    const int *src = s->route_trace + (size_t)layer * s->options.max_batch * c.experts_per_token;
    return hipMemcpyAsync(route_ids, src, n * sizeof(int), hipMemcpyDeviceToHost, st) ==
                   hipSuccess &&
                   hipStreamSynchronize(st) == hipSuccess
               ? 1
               : 0;
}

// ---------------------------------------------------------------------------
// extensions
// ---------------------------------------------------------------------------

extern "C" int moonlight_session_fill_kv(MoonlightSession *s, int layer, int length,
                                         uint64_t seed) {
    ApiScope api_scope(s);
    if (!s || length < 0 || length > s->options.context_size) return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer >= c.layer_count) return 0;
    const size_t ctx = (size_t)s->options.context_size;
    hipStream_t st = stream_of(s);
    const int first = layer < 0 ? 0 : layer, last = layer < 0 ? c.layer_count : layer + 1;
    for (int l = first; l < last; ++l) {
        const uint64_t sd = seed + (uint64_t)l * 2;
        if (length > 0 &&
            (fill_normal(s->latent_kv + (size_t)l * ctx * c.kv_lora_rank,
                         (int64_t)length * c.kv_lora_rank, sd, 0.0f, 1.0f, 0, st) != kOk ||
             mla_split_cache(s->latent_kv + (size_t)l * ctx * c.kv_lora_rank,
                             s->latent_split + (size_t)l * ctx * 2 * c.kv_lora_rank, length,
                             c.kv_lora_rank, st) != kOk ||
             fill_normal(s->rope_kv + (size_t)l * ctx * c.qk_rope_dim,
                         (int64_t)length * c.qk_rope_dim, sd + 1, 0.0f, 1.0f, 0, st) != kOk))
            return 0;
        s->kv_lengths[l] = length;
    }
    if (layer < 0) s->position = length;
    return hipStreamSynchronize(st) == hipSuccess ? 1 : 0;
}

namespace {

// Inputs of the timing hooks: `count` blocks of rows x hidden values ~N(0, 1),
// block b drawn from seed + b (one block when count is 1).  Device memory of
// the hook's own, released by the caller with hipFree.
float *timing_inputs(MoonlightSession *s, int rows, int count, uint64_t seed) {
    const ModelConfig &c = s->model->cfg;
    const size_t block = (size_t)rows * c.hidden_size;
    float *pool = nullptr;
    if (hipMalloc(&pool, block * count * sizeof(float)) != hipSuccess) return nullptr;
    for (int b = 0; b < count; ++b)
        if (fill_normal(pool + block * b, (int64_t)block, seed + (uint64_t)b, 0.0f, 1.0f, 0,
                        stream_of(s)) != kOk) {
            (void)hipFree(pool);
            return nullptr;
        }
    return pool;
}

// The layers a timing hook cycles through: `layer` alone, or with layer < 0
// every usable layer of the kind (MoE layers when `moe`).
std::vector<int> timing_layers(const MoonlightSession *s, int layer, bool moe) {
    const ModelConfig &c = s->model->cfg;
    std::vector<int> out;
    for (int l = 0; l < c.layer_count; ++l) {
        const LayerPlan &lp = s->model->layers[l];
        if ((layer >= 0 && l != layer) || !lp.error.empty() ||
            (moe && (l < c.first_dense_layer_count || lp.dense)))
            continue;
        out.push_back(l);
    }
    return out;
}

}  // namespace

extern "C" int moonlight_session_time_moe(MoonlightSession *s, int layer, int rows, uint64_t seed,
                                          int warmup, int iters, double *avg_us,
                                          int *unique_experts) {
    ApiScope api_scope(s);
    if (!s || !avg_us || rows <= 0 || rows > s->options.max_batch || iters <= 0 || warmup < 0)
        return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer >= c.layer_count || rows > moe_chunk_rows(c)) return 0;
    const std::vector<int> layers = timing_layers(s, layer, true);
    if (layers.empty() || (layer >= 0 && layers[0] != layer)) return 0;
    hipStream_t st = stream_of(s);
    // a fixed layer reads one input block; a rotation draws a fresh block for
    // every pass (warm-up passes included)
    const int passes = warmup + iters;
    const int blocks = layer >= 0 ? 1 : passes;
    const size_t block = (size_t)rows * c.hidden_size;
    float *inputs = timing_inputs(s, rows, blocks, seed);
    if (!inputs) return 0;
    auto pass = [&](int i) {
        const int l = layers[(size_t)i % layers.size()];
        const LayerPlan &lp = s->model->layers[l];
        const float *x = inputs + block * (size_t)(i % blocks);
        RouteParams inline_r;
        return route(s, l, x, rows, lp.post_norm, nullptr, true, &inline_r) == kOk &&
               experts(s, l, x, rows, lp.post_norm, x, s->h, nullptr, &inline_r) == kOk;
    };
    bool ok = hipMemsetAsync(s->route_error, 0, sizeof(int), st) == hipSuccess;
    for (int i = 0; ok && i < warmup; ++i) ok = pass(i);
    ok = ok && hipEventRecord(s->ev_start, st) == hipSuccess;
    for (int i = warmup; ok && i < passes; ++i) ok = pass(i);
    ok = ok && hipEventRecord(s->ev_stop, st) == hipSuccess &&
         to_host(s, s->host_flag, s->route_error, sizeof(int));
    float ms = 0.0f;
    ok = finish(s) && ok && !*s->host_flag &&
         hipEventElapsedTime(&ms, s->ev_start, s->ev_stop) == hipSuccess;
    // the distinct experts of every timed pass, from an untimed replay of the
    // same passes (routing is deterministic)
    int *counts = nullptr;
    if (ok && unique_experts) {
        ok = hipHostMalloc((void **)&counts, (size_t)iters * sizeof(int), hipHostMallocDefault) ==
             hipSuccess;
        for (int i = warmup; ok && i < passes; ++i)
            ok = pass(i) && to_host(s, counts + (i - warmup), s->n_unique, sizeof(int));
        ok = finish(s) && ok;
        long total = 0;
        for (int i = 0; ok && i < iters; ++i) total += counts[i];
        if (ok) *unique_experts = (int)total;
    }
    if (counts) (void)hipHostFree(counts);
    (void)hipFree(inputs);
    if (!ok) return 0;
    *avg_us = (double)ms * 1000.0 / iters;
    return 1;
}

extern "C" int moonlight_session_time_attention(MoonlightSession *s, int layer, int rows,
                                                int position, uint64_t seed, int warmup,
                                                int iters, double *avg_us) {
    ApiScope api_scope(s);
    if (!s || !avg_us || rows <= 0 || rows > s->options.max_batch || iters <= 0 || warmup < 0 ||
        position < 0 || position + rows > s->options.context_size)
        return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer >= c.layer_count || c.q_lora_rank) return 0;
    const std::vector<int> layers = timing_layers(s, layer, false);
    if (layers.empty() || (layer >= 0 && layers[0] != layer)) return 0;
    hipStream_t st = stream_of(s);
    const int passes = warmup + iters;
    const int blocks = layer >= 0 ? 1 : passes;
    const size_t block = (size_t)rows * c.hidden_size;
    float *inputs = timing_inputs(s, rows, blocks, seed);
    if (!inputs) return 0;
    auto pass = [&](int i) {
        const int l = layers[(size_t)i % layers.size()];
        const float *x = inputs + block * (size_t)(i % blocks);
        return attention(s, l, x, rows, position, s->h, s->model->layers[l].input_norm, x) ==
               kOk;
    };
    bool ok = true;
    for (int i = 0; ok && i < warmup; ++i) ok = pass(i);
    ok = ok && hipEventRecord(s->ev_start, st) == hipSuccess;
    for (int i = warmup; ok && i < passes; ++i) ok = pass(i);
    ok = ok && hipEventRecord(s->ev_stop, st) == hipSuccess;
    float ms = 0.0f;
    ok = finish(s) && ok && hipEventElapsedTime(&ms, s->ev_start, s->ev_stop) == hipSuccess;
    (void)hipFree(inputs);
    if (!ok) return 0;
    *avg_us = (double)ms * 1000.0 / iters;
    return 1;
}

extern "C" int moonlight_session_fix_routes(MoonlightSession *s, const int *expert_ids,
                                            int rows) {
    ApiScope api_scope(s);
    if (!s) return 0;
    const ModelConfig &c = s->model->cfg;
    if (!expert_ids || rows <= 0) {
        s->fixed_rows = 0;
        return 1;
    }
    if (rows > s->options.max_batch) return 0;
    const size_t n = (size_t)rows * c.experts_per_token;
    for (size_t i = 0; i < n; ++i)
        if (expert_ids[i] < 0 || expert_ids[i] >= c.expert_count) return 0;
    // the experts of a row must be distinct, as a top-k selection makes them
    // (the device route tables rely on it)
    for (int r = 0; r < rows; ++r)
        for (int a = 0; a < c.experts_per_token; ++a)
            for (int b = a + 1; b < c.experts_per_token; ++b)
                if (expert_ids[(size_t)r * c.experts_per_token + a] ==
                    expert_ids[(size_t)r * c.experts_per_token + b])
                    return 0;
    if (hipMemcpy(s->fixed_ids, expert_ids, n * sizeof(int), hipMemcpyHostToDevice) !=
        hipSuccess)
        return 0;
    s->fixed_rows = rows;
    return 1;
}

extern "C" int moonlight_session_decode_graph(MoonlightSession *s, int enable) {
    ApiScope api_scope(s);
    if (!s) return 0;
    if (enable == 0) {
        s->decode_graph_off = true;
        drop_decode_graph(s);
    } else if (enable > 0) {
        s->decode_graph_off = false;
    }
    return s->decode_exec ? 1 : 0;
}

extern "C" int moonlight_session_copy_route_tables(const MoonlightSession *s, int rows,
                                                   int *n_unique, int *unique, int *counts,
                                                   int *offsets, int *list_rows,
                                                   int *list_slots, int *list_pos) {
    ApiScope api_scope(s);
    if (!s || rows <= 0 || rows > s->options.max_batch) return 0;
    const ModelConfig &c = s->model->cfg;
    const size_t E = (size_t)c.expert_count, n = (size_t)rows * c.experts_per_token;
    hipStream_t st = s->model->ctx->stream;
    bool ok = true;
    auto copy = [&](int *dst, const int *src, size_t count) {
        if (ok && dst)
            ok = hipMemcpyAsync(dst, src, count * sizeof(int), hipMemcpyDeviceToHost, st) ==
                 hipSuccess;
    };
    copy(n_unique, s->n_unique, 1);
    copy(unique, s->unique, E);
    copy(counts, s->counts, E);
    copy(offsets, s->offsets, E);
    copy(list_rows, s->list_rows, n);
    copy(list_slots, s->list_slots, n);
    copy(list_pos, s->list_pos, n);
    return ok && hipStreamSynchronize(st) == hipSuccess ? 1 : 0;
}

extern "C" int moonlight_session_trace_router(MoonlightSession *s, int enable) {
    ApiScope api_scope(s);
    if (!s) return 0;
    drop_decode_graph(s);
    if (!enable) {
        if (s->router_trace) (void)hipFree(s->router_trace);
        s->router_trace = nullptr;
        return 1;
    }
    if (s->router_trace) return 1;
    const ModelConfig &c = s->model->cfg;
    const size_t n = (size_t)c.layer_count * s->options.max_batch * (size_t)c.expert_count;
    void *p = nullptr;
    if (hipMalloc(&p, n * sizeof(float)) != hipSuccess) return 0;
    s->router_trace = static_cast<float *>(p);
    return 1;
}

extern "C" int moonlight_session_copy_router_trace(const MoonlightSession *s, int layer,
                                                   float *logits, int capacity_rows) {
    ApiScope api_scope(s);
    if (!s || !logits || !s->router_trace || capacity_rows < s->last_forward_rows) return 0;
    const ModelConfig &c = s->model->cfg;
    if (layer < c.first_dense_layer_count || layer >= c.layer_count ||
        s->model->layers[layer].dense)
        return 0;
    hipStream_t st = s->model->ctx->stream;
    const size_t E = (size_t)c.expert_count;
    return hipMemcpyAsync(logits, s->router_trace + (size_t)layer * s->options.max_batch * E,
                          (size_t)s->last_forward_rows * E * sizeof(float),
                          hipMemcpyDeviceToHost, st) == hipSuccess &&
                   hipStreamSynchronize(st) == hipSuccess
               ? 1
               : 0;
}

extern "C" int moonlight_session_device_time(MoonlightSession *s, double *ms) {
    if (!s || !ms) return 0;
    *ms = s->last_device_ms;
    return 1;
}
