// capi.cpp -- extern "C" entry points of include/cactus_engine.h, random
// weight generation, and the FFI-style generate loop
// (cactus/ffi/cactus_complete.cpp:185-298).
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "cact_file.h"
#include "cactus_hip.h"
#include "engine.h"
#include "loader.h"

namespace cactus {

static thread_local std::string g_engine_error;

template <typename F>
static int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_engine_error = e.what();
        return -1;
    }
}

// ---------------------------------------------------------------- random init
static inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint16_t f2h_host(float f) {
    const double d = (double)f;
    uint64_t b;
    std::memcpy(&b, &d, 8);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const uint64_t a = b & 0x7FFFFFFFFFFFFFFFull;
    const int e = (int)(a >> 52);
    if (e == 0x7FF) return sign | ((a & 0xFFFFFFFFFFFFFull) ? 0x7E00 : 0x7C00);
    if (a == 0) return sign;
    const uint64_t mant = (a & 0xFFFFFFFFFFFFFull) | (1ull << 52);
    const int ex = e - 1023;
    if (ex > 15) return sign | 0x7C00;
    const int shift = ex >= -14 ? 42 : 42 + (-14 - ex);
    if (shift > 63) return sign;
    uint64_t q = mant >> shift;
    const uint64_t rem = mant & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    const uint32_t r = ex >= -14 ? ((uint32_t)(ex + 15) << 10) + (uint32_t)(q - 1024) : (uint32_t)q;
    return r >= 0x7C00 ? (sign | 0x7C00) : (sign | (uint16_t)r);
}

// Deterministic parallel fill: element i of tensor `tag` draws from stream
// (seed, tag, i / 65536), so the values do not depend on the thread count.
template <typename Fn>
static void parallel_fill(size_t n, uint64_t seed, uint64_t tag, Fn fn) {
    const size_t blk = 65536;
    const size_t nblk = (n + blk - 1) / blk;
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 4;
    if (nt > 16) nt = 16;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++) {
        th.emplace_back([&, t] {
            for (size_t b = t; b < nblk; b += nt) {
                uint64_t s = seed * 0x100000001B3ull ^ (tag << 40) ^ (b * 0x9E3779B97F4A7C15ull);
                const size_t e = std::min(n, (b + 1) * blk);
                for (size_t i = b * blk; i < e; i++) fn(i, s);
            }
        });
    }
    for (auto& x : th) x.join();
}

static inline double unif01(uint64_t& s) { return (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0); }
static inline double normal(uint64_t& s) {
    double u1 = unif01(s), u2 = unif01(s);
    if (u1 < 1e-300) u1 = 1e-300;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

struct HostWeights {
    std::vector<std::vector<int8_t>> q_w, k_w, v_w, o_w;
    std::vector<std::vector<uint8_t>> gate_w, up_w, down_w;
    std::vector<std::vector<uint16_t>> q_s, k_s, v_s, o_s, gate_s, up_s, down_s;
    std::vector<std::vector<uint16_t>> in_norm, post_norm, q_norm, k_norm;
    std::vector<uint16_t> emb, out_norm;
    std::vector<cactus_qwen_layer_weights> layers;
};

// Two scales differ from the other tensors' 0.02.  With every tensor at 0.02
// the attention's context average becomes a component shared by all positions
// that grows layer over layer, and with tied embeddings a residual stream
// still dominated by the input row's embedding predicts that same token: a
// greedy decode then repeats one id forever.  A wider down-projection scale
// makes the MLP's token-dependent output dominate the residual stream and
// smaller embeddings keep the input row from predicting itself, so greedy
// decode walks through distinct ids (128 of 128 at the 28-layer, 4096-token
// shape; every id of the 2-layer test shapes' short decodes).
static constexpr double kDownScaleSd = 0.1;
static constexpr double kEmbeddingSd = 0.005;

static void make_random(const cactus_qwen_config& c, uint64_t seed, HostWeights& w) {
    const size_t H = c.hidden, F = c.ffn, hd = c.head_dim, gs = c.group_size;
    const size_t nq = (size_t)c.heads * hd, nkv = (size_t)c.kv_heads * hd;
    uint64_t tag = 1;
    auto codes8 = [&](size_t n) {
        std::vector<int8_t> v(n);
        parallel_fill(n, seed, tag++, [&](size_t i, uint64_t& s) { v[i] = (int8_t)((int)(splitmix64(s) % 255) - 127); });
        return v;
    };
    auto codes4 = [&](size_t rows, size_t cols) {  // packed, low nibble = even column
        std::vector<uint8_t> v(rows * cols / 2);
        parallel_fill(v.size(), seed, tag++, [&](size_t i, uint64_t& s) {
            const int lo = (int)(splitmix64(s) % 15) - 7, hi = (int)(splitmix64(s) % 15) - 7;
            v[i] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
        });
        return v;
    };
    auto scales = [&](size_t n, double qmax, double sd) {
        std::vector<uint16_t> v(n);
        parallel_fill(n, seed, tag++, [&](size_t i, uint64_t& s) { v[i] = f2h_host((float)(std::fabs(normal(s) * sd) / qmax)); });
        return v;
    };
    auto gauss = [&](size_t n, double mean, double sd) {
        std::vector<uint16_t> v(n);
        parallel_fill(n, seed, tag++, [&](size_t i, uint64_t& s) { v[i] = f2h_host((float)(mean + sd * normal(s))); });
        return v;
    };
    const uint32_t L = c.num_layers;
    for (uint32_t l = 0; l < L; l++) {
        w.in_norm.push_back(gauss(H, 1.0, 0.02));
        w.post_norm.push_back(gauss(H, 1.0, 0.02));
        w.q_norm.push_back(gauss(hd, 1.0, 0.02));
        w.k_norm.push_back(gauss(hd, 1.0, 0.02));
        w.q_w.push_back(codes8(nq * H));
        w.q_s.push_back(scales(nq * (H / gs), 127.0, 0.02));
        w.k_w.push_back(codes8(nkv * H));
        w.k_s.push_back(scales(nkv * (H / gs), 127.0, 0.02));
        w.v_w.push_back(codes8(nkv * H));
        w.v_s.push_back(scales(nkv * (H / gs), 127.0, 0.02));
        w.o_w.push_back(codes8(H * nq));
        w.o_s.push_back(scales(H * (nq / gs), 127.0, 0.02));
        w.gate_w.push_back(codes4(F, H));
        w.gate_s.push_back(scales(F * (H / gs), 7.0, 0.02));
        w.up_w.push_back(codes4(F, H));
        w.up_s.push_back(scales(F * (H / gs), 7.0, 0.02));
        w.down_w.push_back(codes4(H, F));
        w.down_s.push_back(scales(H * (F / gs), 7.0, kDownScaleSd));
    }
    w.emb = gauss((size_t)c.vocab * H, 0.0, kEmbeddingSd);
    w.out_norm = gauss(H, 1.0, 0.02);
    w.layers.resize(L);
    for (uint32_t l = 0; l < L; l++) {
        cactus_qwen_layer_weights& x = w.layers[l];
        x.input_norm = w.in_norm[l].data();
        x.post_norm = w.post_norm[l].data();
        x.q_norm = w.q_norm[l].data();
        x.k_norm = w.k_norm[l].data();
        x.q_w = w.q_w[l].data(); x.q_s = w.q_s[l].data();
        x.k_w = w.k_w[l].data(); x.k_s = w.k_s[l].data();
        x.v_w = w.v_w[l].data(); x.v_s = w.v_s[l].data();
        x.o_w = w.o_w[l].data(); x.o_s = w.o_s[l].data();
        x.gate_w = w.gate_w[l].data(); x.gate_s = w.gate_s[l].data();
        x.up_w = w.up_w[l].data(); x.up_s = w.up_s[l].data();
        x.down_w = w.down_w[l].data(); x.down_s = w.down_s[l].data();
    }
}

static void fill_info(const CactHeader& h, cactus_cact_info* info) {
    if (!info) return;
    std::memset(info, 0, sizeof(*info));
    info->version = h.version;
    info->flags = h.flags;
    info->alignment = h.alignment;
    info->ndim = h.ndim;
    for (int i = 0; i < 4; i++) info->shape[i] = h.dims[i];
    info->precision = h.precision;
    info->group_size = h.group_size;
    info->num_groups = h.num_groups;
    info->data_bytes = h.data_bytes;
    info->scales_bytes = h.scales_bytes;
    info->scales_offset = h.scales_offset;
    info->data_offset = h.data_offset;
}

// A graph of the file API with a stream of its own.
struct GraphHandle {
    void* stream = nullptr;
    std::unique_ptr<CactusGraph> g;
    ~GraphHandle() {
        g.reset();
        if (stream) cactus_hip_stream_destroy(stream);
    }
};

static void validate(const cactus_qwen_config* c) {
    if (!c) throw std::runtime_error("null config");
    if (!c->num_layers || !c->hidden || !c->ffn || !c->heads || !c->kv_heads || !c->head_dim ||
        !c->vocab || !c->group_size || !c->max_seq)
        throw std::runtime_error("config fields must be non-zero");
}

}  // namespace cactus

using namespace cactus;

extern "C" {

const char* cactus_engine_last_error(void) { return g_engine_error.c_str(); }

int cactus_qwen_create(const cactus_qwen_config* cfg, const cactus_qwen_layer_weights* layers,
                       const uint16_t* embedding, const uint16_t* output_norm, void** model) {
    return guarded([&] {
        validate(cfg);
        if (!model || !layers || !embedding || !output_norm) throw std::runtime_error("null argument");
        *model = new QwenModel(*cfg, layers, embedding, output_norm);
    });
}

int cactus_qwen_create_random(const cactus_qwen_config* cfg, uint64_t seed, void** model) {
    return guarded([&] {
        validate(cfg);
        if (!model) throw std::runtime_error("null argument");
        HostWeights w;
        make_random(*cfg, seed, w);
        *model = new QwenModel(*cfg, w.layers.data(), w.emb.data(), w.out_norm.data());
    });
}

int cactus_qwen_random_weights(const cactus_qwen_config* cfg, uint64_t seed,
                               cactus_qwen_layer_weights* layers_out_buffers, uint16_t* embedding,
                               uint16_t* output_norm) {
    return guarded([&] {
        validate(cfg);
        if (!layers_out_buffers || !embedding || !output_norm) throw std::runtime_error("null argument");
        HostWeights w;
        make_random(*cfg, seed, w);
        const size_t H = cfg->hidden, F = cfg->ffn, hd = cfg->head_dim, gs = cfg->group_size;
        const size_t nq = (size_t)cfg->heads * hd, nkv = (size_t)cfg->kv_heads * hd;
        auto put = [](const void* dst, const void* src, size_t bytes) {
            if (!dst) throw std::runtime_error("null weight buffer");
            std::memcpy(const_cast<void*>(dst), src, bytes);
        };
        for (uint32_t l = 0; l < cfg->num_layers; l++) {
            const cactus_qwen_layer_weights& s = w.layers[l];
            const cactus_qwen_layer_weights& d = layers_out_buffers[l];
            put(d.input_norm, s.input_norm, 2 * H);
            put(d.post_norm, s.post_norm, 2 * H);
            put(d.q_norm, s.q_norm, 2 * hd);
            put(d.k_norm, s.k_norm, 2 * hd);
            put(d.q_w, s.q_w, nq * H); put(d.q_s, s.q_s, 2 * nq * (H / gs));
            put(d.k_w, s.k_w, nkv * H); put(d.k_s, s.k_s, 2 * nkv * (H / gs));
            put(d.v_w, s.v_w, nkv * H); put(d.v_s, s.v_s, 2 * nkv * (H / gs));
            put(d.o_w, s.o_w, H * nq); put(d.o_s, s.o_s, 2 * H * (nq / gs));
            put(d.gate_w, s.gate_w, F * H / 2); put(d.gate_s, s.gate_s, 2 * F * (H / gs));
            put(d.up_w, s.up_w, F * H / 2); put(d.up_s, s.up_s, 2 * F * (H / gs));
            put(d.down_w, s.down_w, H * F / 2); put(d.down_s, s.down_s, 2 * H * (F / gs));
        }
        std::memcpy(embedding, w.emb.data(), 2 * w.emb.size());
        std::memcpy(output_norm, w.out_norm.data(), 2 * H);
    });
}

int cactus_qwen_destroy(void* model) {
    return guarded([&] { delete static_cast<QwenModel*>(model); });
}

int cactus_qwen_reset(void* model) {
    return guarded([&] { static_cast<QwenModel*>(model)->reset(); });
}

int cactus_qwen_set_decode_mode(void* model, int mode) {
    return guarded([&] { static_cast<QwenModel*>(model)->set_decode_mode(mode); });
}

int cactus_qwen_set_attention_mode(void* model, int mode) {
    return guarded([&] { static_cast<QwenModel*>(model)->set_attention_mode(mode); });
}

int cactus_qwen_set_kv_window(void* model, size_t window, size_t sink) {
    return guarded([&] { static_cast<QwenModel*>(model)->set_kv_window(window, sink); });
}

int cactus_qwen_set_sampling(void* model, float temperature, float top_p, size_t top_k, size_t random_seed) {
    return guarded([&] { static_cast<QwenModel*>(model)->set_sampling(temperature, top_p, top_k, random_seed); });
}

int cactus_qwen_total_len(void* model, size_t* len) {
    return guarded([&] { *len = static_cast<QwenModel*>(model)->cache().total_seq_len; });
}

int cactus_qwen_prefill(void* model, const uint32_t* tokens, size_t n) {
    return guarded([&] {
        static_cast<QwenModel*>(model)->prefill(std::vector<uint32_t>(tokens, tokens + n));
    });
}

int cactus_qwen_decode(void* model, uint32_t token, uint32_t* next) {
    return guarded([&] { *next = static_cast<QwenModel*>(model)->decode(token); });
}

int cactus_qwen_generate(void* model, const uint32_t* prompt, size_t n, size_t max_new,
                         uint32_t* out, cactus_qwen_timing* timing) {
    return guarded([&] {
        if (n == 0) throw std::runtime_error("Cannot generate from empty prompt");
        QwenModel* m = static_cast<QwenModel*>(model);
        using clk = std::chrono::steady_clock;
        auto ms = [](clk::time_point a, clk::time_point b) {
            return std::chrono::duration<double, std::milli>(b - a).count();
        };
        auto t0 = clk::now();
        if (n > 1) m->prefill(std::vector<uint32_t>(prompt, prompt + n - 1));
        check_hip(cactus_hip_stream_sync(m->stream()), "sync");
        auto t1 = clk::now();
        uint32_t tok = max_new ? m->decode(prompt[n - 1]) : 0;
        if (max_new) out[0] = tok;
        auto t2 = clk::now();
        if (max_new > 1) m->decode_many(tok, max_new - 1, out + 1);
        check_hip(cactus_hip_stream_sync(m->stream()), "sync");
        auto t3 = clk::now();
        if (timing) {
            timing->prefill_ms = ms(t0, t1);
            timing->first_decode_ms = ms(t1, t2);
            timing->decode_ms = ms(t2, t3);
            timing->prefill_tokens = (uint32_t)(n - 1);
            timing->decode_tokens = (uint32_t)(max_new ? max_new - 1 : 0);
        }
    });
}

int cactus_qwen_last_hidden(void* model, uint16_t* out, size_t max_rows, size_t* rows) {
    return guarded([&] {
        QwenModel* m = static_cast<QwenModel*>(model);
        if (m->last_hidden_node() == SIZE_MAX)
            throw std::runtime_error("no graph forward has run since the last reset or fused decode step");
        const BufferDesc& b = m->graph().get_output_buffer(m->last_hidden_node());
        const size_t r = b.shape[0];
        if (rows) *rows = r;
        const size_t n = std::min(r, max_rows) * m->config().hidden;
        check_hip(cactus_hip_memcpy_d2h(out, b.data, n * 2, m->stream()), "last_hidden");
    });
}

int cactus_qwen_last_logits(void* model, uint16_t* out) {
    return guarded([&] {
        QwenModel* m = static_cast<QwenModel*>(model);
        if (!out) throw std::runtime_error("null argument");
        const void* src = m->last_logits_data();
        if (!src) throw std::runtime_error("no decode step has run since the last reset or prefill");
        check_hip(cactus_hip_memcpy_d2h(out, src, (size_t)m->config().vocab * 2, m->stream()), "last_logits");
    });
}

int cactus_qwen_last_entropy(void* model, float* entropy) {
    return guarded([&] {
        QwenModel* m = static_cast<QwenModel*>(model);
        if (!entropy) throw std::runtime_error("null argument");
        const void* src = m->last_logits_data();
        if (!src) throw std::runtime_error("no decode step has run since the last reset or prefill");
        DevBuf e(4);
        check_hip(cactus_hip_logits_entropy_f16(static_cast<const uint16_t*>(src), m->config().vocab, e.as<float>(),
                                                m->stream()),
                  "entropy");
        check_hip(cactus_hip_memcpy_d2h(entropy, e.ptr, 4, m->stream()), "entropy");
    });
}

int cactus_qwen_cache_len(void* model, size_t* len) {
    return guarded([&] { *len = static_cast<QwenModel*>(model)->cache().current_seq_len; });
}

int cactus_qwen_read_kv(void* model, size_t layer, int8_t* k, int8_t* v, float* ks, float* vs) {
    return guarded([&] {
        QwenModel* m = static_cast<QwenModel*>(model);
        KVCache& c = m->cache();
        if (layer >= c.num_layers) throw std::runtime_error("layer out of range");
        const size_t n = c.current_seq_len * c.num_kv_heads * c.head_dim;
        const size_t ns = c.current_seq_len * c.num_kv_heads * c.groups() * sizeof(float);
        check_hip(cactus_hip_memcpy_d2h(k, c.keys(layer), n, m->stream()), "read_kv");
        check_hip(cactus_hip_memcpy_d2h(v, c.values(layer), n, m->stream()), "read_kv");
        check_hip(cactus_hip_memcpy_d2h(ks, c.key_scales(layer), ns, m->stream()), "read_kv");
        check_hip(cactus_hip_memcpy_d2h(vs, c.value_scales(layer), ns, m->stream()), "read_kv");
    });
}

int cactus_qwen_read_weights(void* model, cactus_qwen_layer_weights* lw, uint16_t* emb,
                             uint16_t* out_norm) {
    return guarded([&] {
        QwenModel* m = static_cast<QwenModel*>(model);
        void* st = m->stream();
        auto rd = [&](const void* dst, const DevBuf& b) {
            if (dst) check_hip(cactus_hip_memcpy_d2h(const_cast<void*>(dst), b.ptr, b.bytes, st), "read_weights");
        };
        if (emb) rd(emb, m->embedding());
        if (out_norm) rd(out_norm, m->output_norm());
        if (!lw) return;
        for (uint32_t l = 0; l < m->config().num_layers; l++) {
            const QwenLayer& L = m->layer(l);
            const cactus_qwen_layer_weights& w = lw[l];
            rd(w.input_norm, L.input_norm); rd(w.post_norm, L.post_norm);
            rd(w.q_norm, L.q_norm); rd(w.k_norm, L.k_norm);
            rd(w.q_w, L.q_w); rd(w.q_s, L.q_s); rd(w.k_w, L.k_w); rd(w.k_s, L.k_s);
            rd(w.v_w, L.v_w); rd(w.v_s, L.v_s); rd(w.o_w, L.o_w); rd(w.o_s, L.o_s);
            rd(w.gate_w, L.gate_w); rd(w.gate_s, L.gate_s); rd(w.up_w, L.up_w); rd(w.up_s, L.up_s);
            rd(w.down_w, L.down_w); rd(w.down_s, L.down_s);
        }
    });
}

// ---------------------------------------------------------------- tensor files
int cactus_cact_read_info(const char* path, cactus_cact_info* info) {
    return guarded([&] {
        if (!path || !info) throw std::runtime_error("null argument");
        CactFile f(path);
        fill_info(f.header(), info);
    });
}

int cactus_cact_save(const char* path, const uint64_t* shape, uint32_t ndim, uint32_t precision,
                     const void* data, uint64_t data_bytes, const uint16_t* scales, uint32_t group_size,
                     uint32_t num_groups) {
    return guarded([&] {
        if (!path || (ndim && !shape) || (data_bytes && !data)) throw std::runtime_error("null argument");
        if (precision > static_cast<uint32_t>(Precision::INT4)) throw std::runtime_error("unknown precision");
        std::vector<size_t> sh(shape, shape + ndim);
        save_cact(path, sh, static_cast<Precision>(precision), data, data_bytes, scales, group_size, num_groups);
    });
}

int cactus_cact_load_device(const char* path, cactus_cact_info* info, void** data, void** scales) {
    return guarded([&] {
        if (!path || !data) throw std::runtime_error("null argument");
        CactFile f(path);
        void* st = nullptr;
        check_hip(cactus_hip_stream_create(&st), "stream_create");
        DeviceTensor t;
        try {
            t = upload_cact(f, st);
        } catch (...) {
            cactus_hip_stream_destroy(st);
            throw;
        }
        cactus_hip_stream_destroy(st);
        fill_info(f.header(), info);
        *data = t.data;
        if (scales) *scales = t.scales;
        else if (t.scales) cactus_hip_free(t.scales);
    });
}

int cactus_qwen_read_config(const char* folder, cactus_qwen_config* cfg) {
    return guarded([&] {
        if (!folder || !cfg) throw std::runtime_error("null argument");
        *cfg = read_qwen_config(folder);
    });
}

int cactus_qwen_create_from_folder(const char* folder, size_t context_size, void** model) {
    return guarded([&] {
        if (!folder || !model) throw std::runtime_error("null argument");
        *model = load_qwen_folder(folder, context_size);
    });
}

int cactus_graph_create(void** graph) {
    return guarded([&] {
        if (!graph) throw std::runtime_error("null argument");
        auto h = std::make_unique<GraphHandle>();
        check_hip(cactus_hip_stream_create(&h->stream), "stream_create");
        h->g = std::make_unique<CactusGraph>(h->stream);
        *graph = h.release();
    });
}

int cactus_graph_destroy(void* graph) {
    return guarded([&] { delete static_cast<GraphHandle*>(graph); });
}

int cactus_graph_load_weights(void* graph, const char* path, size_t* node) {
    return guarded([&] {
        if (!graph || !path || !node) throw std::runtime_error("null argument");
        *node = static_cast<GraphHandle*>(graph)->g->load_weights(path);
    });
}

int cactus_graph_mmap_embeddings(void* graph, const char* path, size_t* node) {
    return guarded([&] {
        if (!graph || !path || !node) throw std::runtime_error("null argument");
        *node = static_cast<GraphHandle*>(graph)->g->mmap_embeddings(path);
    });
}

int cactus_graph_save_node(void* graph, size_t node, const char* path) {
    return guarded([&] {
        if (!graph || !path) throw std::runtime_error("null argument");
        static_cast<GraphHandle*>(graph)->g->save_node(node, path);
    });
}

int cactus_graph_node_info(void* graph, size_t node, cactus_graph_node_desc* desc) {
    return guarded([&] {
        if (!graph || !desc) throw std::runtime_error("null argument");
        const BufferDesc& b = static_cast<GraphHandle*>(graph)->g->get_output_buffer(node);
        std::memset(desc, 0, sizeof(*desc));
        if (b.shape.size() > 4) throw std::runtime_error("node has more than 4 dimensions");
        desc->ndim = (uint32_t)b.shape.size();
        for (size_t i = 0; i < b.shape.size(); i++) desc->shape[i] = b.shape[i];
        desc->precision = b.is_packed_int4() ? static_cast<uint32_t>(Precision::INT4) : static_cast<uint32_t>(b.precision);
        desc->data_bytes = b.is_packed_int4() ? b.packed_int4_size : b.byte_size;
        desc->group_size = (uint32_t)b.group_size;
        desc->num_groups = (uint32_t)b.num_groups;
    });
}

int cactus_graph_read_node(void* graph, size_t node, void* data, uint64_t capacity, uint16_t* scales,
                           uint64_t scales_capacity) {
    return guarded([&] {
        if (!graph) throw std::runtime_error("null argument");
        GraphHandle* h = static_cast<GraphHandle*>(graph);
        const BufferDesc& b = h->g->get_output_buffer(node);
        const bool packed = b.is_packed_int4();
        const void* src = packed ? b.packed_int4 : b.data;
        const size_t n = packed ? b.packed_int4_size : b.byte_size;
        if (!src) throw std::runtime_error("node has no data");
        if (data) {
            if (capacity < n) throw std::runtime_error("data capacity too small");
            check_hip(cactus_hip_memcpy_d2h(data, src, n, h->stream), "read_node");
        }
        if (scales && b.scales && b.num_groups) {
            const size_t sb = (b.shape.empty() ? 1 : b.shape[0]) * b.num_groups * 2;
            if (scales_capacity < sb) throw std::runtime_error("scales capacity too small");
            check_hip(cactus_hip_memcpy_d2h(scales, b.scales, sb, h->stream), "read_node scales");
        }
        check_hip(cactus_hip_stream_sync(h->stream), "read_node sync");
    });
}

}  // extern "C"
