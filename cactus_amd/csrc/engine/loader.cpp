// loader.cpp -- Qwen3 model folders (config.txt + one CACT file per tensor)
// to device memory; file names and defaults follow the reference
// (model_qwen.cpp:17-49, engine_model.cpp:47-55 and :403-520).
#include "loader.h"

#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <fstream>
#include <memory>
#include <stdexcept>
#include <string>

#include "cactus_hip.h"
#include "engine.h"

namespace cactus {

DeviceTensor upload_cact(const CactFile& f, void* stream) {
    const CactHeader& h = f.header();
    DeviceTensor t;
    auto up = [&](void** dst, const void* src, size_t n) {
        check_hip(cactus_hip_malloc(dst, n ? n : 1), "cact upload: malloc");
        if (n) check_hip(cactus_hip_memcpy_h2d(*dst, src, n, stream), "cact upload: copy");
    };
    try {
        up(&t.data, f.data(), h.data_bytes);
        if (h.scales_bytes) up(&t.scales, f.scales(), h.scales_bytes);
        check_hip(cactus_hip_stream_sync(stream), "cact upload: sync");
    } catch (...) {
        if (t.data) cactus_hip_free(t.data);
        if (t.scales) cactus_hip_free(t.scales);
        throw;
    }
    return t;
}

namespace {

std::string trim(const std::string& s) {
    const size_t a = s.find_first_not_of(" \t\r");
    if (a == std::string::npos) return "";
    const size_t b = s.find_last_not_of(" \t\r");
    return s.substr(a, b - a + 1);
}

std::string lower(std::string s) {
    std::transform(s.begin(), s.end(), s.begin(), [](unsigned char c) { return (char)std::tolower(c); });
    return s;
}

const char* precision_name(uint32_t p) {
    switch (p) {
        case 0: return "INT8";
        case 1: return "FP16";
        case 2: return "FP32";
        case 3: return "INT4";
        default: return "unknown";
    }
}

// One tensor file of the folder, checked against the layout the engine runs.
struct Tensor {
    std::unique_ptr<CactFile> f;
    const void* data() const { return f->data(); }
    const uint16_t* scales() const { return f->scales(); }
};

Tensor open_checked(const std::string& path, Precision want, std::vector<size_t> shape, size_t gs) {
    Tensor t{std::make_unique<CactFile>(path)};
    const CactHeader& h = t.f->header();
    auto fail = [&](const std::string& what) { throw std::runtime_error(path + ": " + what); };
    if (h.precision != static_cast<uint32_t>(want))
        fail(std::string("precision ") + precision_name(h.precision) + ", this engine runs " +
             precision_name(static_cast<uint32_t>(want)) + " here");
    if (h.shape != shape) {
        std::string s;
        for (size_t d : h.shape) s += (s.empty() ? "" : "x") + std::to_string(d);
        std::string w;
        for (size_t d : shape) w += (w.empty() ? "" : "x") + std::to_string(d);
        fail("shape " + s + ", expected " + w);
    }
    size_t elems = 1;
    for (size_t d : shape) elems *= d;
    const size_t bytes = want == Precision::INT4 ? elems / 2 : elems * precision_size(want);
    if (h.data_bytes != bytes) fail("data bytes " + std::to_string(h.data_bytes) + ", expected " + std::to_string(bytes));
    if (want == Precision::INT8 || want == Precision::INT4) {
        const size_t cols = shape[1];
        if (h.group_size != gs || h.num_groups * (uint64_t)gs != cols)
            fail("group size " + std::to_string(h.group_size) + " x " + std::to_string(h.num_groups) +
                 " groups, expected " + std::to_string(gs) + " x " + std::to_string(cols / gs));
        if (h.scales_bytes != (uint64_t)shape[0] * h.num_groups * 2) fail("scales bytes do not match the groups");
    }
    return t;
}

}  // namespace

cactus_qwen_config read_qwen_config(const std::string& folder) {
    const std::string path = folder + "/config.txt";
    std::ifstream in(path);
    if (!in) throw std::runtime_error("Failed to open config file: " + path);
    // engine.h:42-58 defaults
    cactus_qwen_config c{};
    c.vocab = 151936;
    c.num_layers = 28;
    c.hidden = 1024;
    c.ffn = 3072;
    c.heads = 16;
    c.kv_heads = 8;
    c.head_dim = 128;
    c.eps = 1e-6f;
    c.rope_theta = 1000000.0f;
    c.prefill_chunk = 256;
    c.max_seq = 0;
    bool tied = true;
    std::string model_type = "qwen";
    uint32_t experts = 0;
    std::string line;
    auto u32 = [&](const std::string& key, const std::string& v) -> uint32_t {
        try {
            return (uint32_t)std::stoul(v);
        } catch (const std::exception&) {
            throw std::runtime_error(path + ": bad value for " + key + ": " + v);
        }
    };
    auto f32 = [&](const std::string& key, const std::string& v) -> float {
        try {
            return std::stof(v);
        } catch (const std::exception&) {
            throw std::runtime_error(path + ": bad value for " + key + ": " + v);
        }
    };
    while (std::getline(in, line)) {
        if (line.empty() || line[0] == '#') continue;
        const size_t eq = line.find('=');
        if (eq == std::string::npos) continue;
        const std::string key = trim(line.substr(0, eq)), v = trim(line.substr(eq + 1));
        if (key == "vocab_size") c.vocab = u32(key, v);
        else if (key == "num_layers") c.num_layers = u32(key, v);
        else if (key == "hidden_dim") c.hidden = u32(key, v);
        else if (key == "ffn_intermediate_dim") c.ffn = u32(key, v);
        else if (key == "attention_heads") c.heads = u32(key, v);
        else if (key == "attention_kv_heads") c.kv_heads = u32(key, v);
        else if (key == "attention_head_dim") c.head_dim = u32(key, v);
        else if (key == "layer_norm_eps") c.eps = f32(key, v);
        else if (key == "rope_theta") c.rope_theta = f32(key, v);
        else if (key == "tie_word_embeddings") tied = (v == "true" || v == "1");
        else if (key == "num_experts") experts = u32(key, v);
        else if (key == "model_type") model_type = lower(v);
    }
    // engine_model.cpp:474-481: unknown names fall back to Qwen
    for (const char* other : {"gemma", "lfm2", "smol", "bert", "whisper"})
        if (model_type == other)
            throw std::runtime_error(path + ": model_type " + model_type + " is not built here (Qwen3 only)");
    if (!tied) throw std::runtime_error(path + ": untied output weights are not built here (tie_word_embeddings=true only)");
    if (experts) throw std::runtime_error(path + ": mixture-of-experts layers are not built here");
    if (!c.num_layers || !c.hidden || !c.ffn || !c.heads || !c.kv_heads || !c.head_dim || !c.vocab)
        throw std::runtime_error(path + ": dimensions must be non-zero");
    // the quantization group is a property of the tensor files
    CactFile q(folder + "/layer_0_attn_q.weights");
    if (!q.header().group_size) throw std::runtime_error(q.path() + ": no group scales");
    c.group_size = q.header().group_size;
    return c;
}

QwenModel* load_qwen_folder(const std::string& folder, size_t context_size) {
    if (context_size == 0) throw std::runtime_error("context size must be non-zero");
    cactus_qwen_config c = read_qwen_config(folder);
    c.max_seq = (uint32_t)context_size;
    const size_t H = c.hidden, F = c.ffn, hd = c.head_dim, gs = c.group_size;
    const size_t nq = (size_t)c.heads * hd, nkv = (size_t)c.kv_heads * hd;
    const std::string base = folder + "/";
    // model_qwen.cpp:17-42 names; engine_model.cpp:53 embedding file
    Tensor emb = open_checked(base + "token_embeddings.weights", Precision::FP16, {c.vocab, H}, 0);
    Tensor out_norm = open_checked(base + "output_norm.weights", Precision::FP16, {H}, 0);
    std::vector<Tensor> keep;
    keep.reserve((size_t)c.num_layers * 11);
    std::vector<cactus_qwen_layer_weights> lw(c.num_layers);
    for (uint32_t l = 0; l < c.num_layers; l++) {
        const std::string p = base + "layer_" + std::to_string(l) + "_";
        auto take = [&](const std::string& name, Precision pr, std::vector<size_t> shape, size_t g) -> const Tensor& {
            keep.push_back(open_checked(p + name, pr, std::move(shape), g));
            return keep.back();
        };
        cactus_qwen_layer_weights& w = lw[l];
        w.input_norm = static_cast<const uint16_t*>(take("input_norm.weights", Precision::FP16, {H}, 0).data());
        w.post_norm = static_cast<const uint16_t*>(take("post_attn_norm.weights", Precision::FP16, {H}, 0).data());
        w.q_norm = static_cast<const uint16_t*>(take("attn_q_norm.weights", Precision::FP16, {hd}, 0).data());
        w.k_norm = static_cast<const uint16_t*>(take("attn_k_norm.weights", Precision::FP16, {hd}, 0).data());
        const Tensor& q = take("attn_q.weights", Precision::INT8, {nq, H}, gs);
        w.q_w = static_cast<const int8_t*>(q.data());
        w.q_s = q.scales();
        const Tensor& k = take("attn_k.weights", Precision::INT8, {nkv, H}, gs);
        w.k_w = static_cast<const int8_t*>(k.data());
        w.k_s = k.scales();
        const Tensor& v = take("attn_v.weights", Precision::INT8, {nkv, H}, gs);
        w.v_w = static_cast<const int8_t*>(v.data());
        w.v_s = v.scales();
        const Tensor& o = take("attn_output.weights", Precision::INT8, {H, nq}, gs);
        w.o_w = static_cast<const int8_t*>(o.data());
        w.o_s = o.scales();
        const Tensor& gt = take("ffn_gate.weights", Precision::INT4, {F, H}, gs);
        w.gate_w = static_cast<const uint8_t*>(gt.data());
        w.gate_s = gt.scales();
        const Tensor& up = take("ffn_up.weights", Precision::INT4, {F, H}, gs);
        w.up_w = static_cast<const uint8_t*>(up.data());
        w.up_s = up.scales();
        const Tensor& dn = take("ffn_down.weights", Precision::INT4, {H, F}, gs);
        w.down_w = static_cast<const uint8_t*>(dn.data());
        w.down_s = dn.scales();
    }
    // the constructor uploads and synchronizes before the maps close
    std::unique_ptr<QwenModel> m(new QwenModel(c, lw.data(), static_cast<const uint16_t*>(emb.data()),
                                               static_cast<const uint16_t*>(out_norm.data())));
    // engine_model.cpp:136-146: window min(context, 512), 4 sinks, both
    // overridable from the environment
    size_t window = std::min(context_size, (size_t)512), sink = 4;
    auto env = [](const char* name, size_t& v) {
        const char* e = std::getenv(name);
        if (!e) return;
        try {
            v = std::stoul(e);
        } catch (const std::exception&) {
            throw std::runtime_error(std::string(name) + ": not a number: " + e);
        }
    };
    env("CACTUS_KV_WINDOW_SIZE", window);
    env("CACTUS_KV_SINK_SIZE", sink);
    m->set_kv_window(window, sink);
    return m.release();
}

}  // namespace cactus
