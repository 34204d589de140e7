// Oracle: GGUF reader, Llama model, f32 KV cache, single/batched forward and the
// speculative decode loops.  TEST INFRASTRUCTURE ONLY (see nc_oracle.h).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "oracle_internal.h"

namespace {

// ---------------------------------------------------------------- GGUF (gguf.rs:454-763)
struct MetaVal {
    int type = -1;  // gguf.rs:652-668 value type ids
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;  // absolute
    uint64_t nbytes = 0;
};

struct Gguf {
    const uint8_t* data = nullptr;
    size_t size = 0;
    std::map<std::string, MetaVal> meta;
    std::vector<Tensor> tensors;
    const Tensor* find(const std::string& n) const {
        for (auto& t : tensors)
            if (t.name == n) return &t;
        return nullptr;
    }
};

struct Cursor {
    const uint8_t* p;
    size_t n, pos = 0;
    bool ok = true;
    bool need(size_t k) {
        if (pos + k > n) ok = false;
        return ok;
    }
    uint64_t u(int bytes) {
        if (!need(bytes)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < bytes; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += bytes;
        return v;
    }
    std::string str() {
        uint64_t len = u(8);
        if (!need(len)) return "";
        std::string s((const char*)p + pos, len);
        pos += len;
        return s;
    }
};

// gguf.rs:154-185 GgufTensorType::layout (block size, type size) for the types used here.
// gguf.rs:154-185 GgufTensorType::layout: (values per block, bytes per block)
bool type_layout(uint32_t t, uint64_t* bs, uint64_t* ts) {
    static const uint32_t tab[][3] = {
        {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},
        {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74}, {18, 256, 98}, {19, 256, 50},
        {20, 32, 18},  {21, 256, 110}, {22, 256, 82}, {23, 256, 136}, {24, 1, 1},   {25, 1, 2},
        {26, 1, 4},    {27, 1, 8},    {28, 1, 8},    {29, 256, 56}, {30, 1, 2},
    };
    for (auto& e : tab)
        if (e[0] == t) {
            *bs = e[1];
            *ts = e[2];
            return true;
        }
    return false;
}

bool read_value(Cursor& c, uint32_t type, MetaVal& v, int depth = 0) {
    v.type = (int)type;
    switch (type) {
        case 0: v.u = c.u(1); break;
        case 1: v.i = (int8_t)c.u(1); break;
        case 2: v.u = c.u(2); break;
        case 3: v.i = (int16_t)c.u(2); break;
        case 4: v.u = c.u(4); break;
        case 5: v.i = (int32_t)c.u(4); break;
        case 6: { uint32_t b = (uint32_t)c.u(4); v.f = bits_f32(b); break; }
        case 7: v.u = c.u(1); if (v.u > 1) return false; break;
        case 8: v.s = c.str(); break;
        case 9: {
            if (depth > 0) return false;
            uint32_t it = (uint32_t)c.u(4);
            uint64_t len = c.u(8);
            for (uint64_t k = 0; k < len && c.ok; k++) {
                MetaVal tmp;
                if (!read_value(c, it, tmp, depth + 1)) return false;
            }
            break;
        }
        case 10: v.u = c.u(8); break;
        case 11: v.i = (int64_t)c.u(8); break;
        case 12: { uint64_t b = c.u(8); double d; std::memcpy(&d, &b, 8); v.f = d; break; }
        default: return false;
    }
    return c.ok;
}

bool parse_gguf(const uint8_t* data, size_t size, Gguf& g, std::string& err) {
    g.data = data;
    g.size = size;
    Cursor c{data, size};
    if (size < 4 || std::memcmp(data, "GGUF", 4) != 0) { err = "invalid GGUF magic"; return false; }
    c.pos = 4;
    uint32_t version = (uint32_t)c.u(4);
    if (version < 2 || version > 3) { err = "unsupported GGUF version"; return false; }
    uint64_t tcount = c.u(8), mcount = c.u(8);
    for (uint64_t i = 0; i < mcount && c.ok; i++) {
        std::string key = c.str();
        uint32_t vt = (uint32_t)c.u(4);
        MetaVal v;
        if (!read_value(c, vt, v)) { err = "bad metadata value for " + key; return false; }
        g.meta[key] = v;
    }
    uint64_t alignment = 32;  // gguf.rs:10
    auto it = g.meta.find("general.alignment");
    if (it != g.meta.end()) {
        if (it->second.type == 4 || it->second.type == 10) alignment = it->second.u;
        else if (it->second.type == 5) alignment = (uint64_t)it->second.i;
    }
    if (alignment == 0 || (alignment & (alignment - 1))) { err = "invalid alignment"; return false; }
    struct Raw { std::string n; std::vector<uint64_t> d; uint32_t t; uint64_t off; };
    std::vector<Raw> raws;
    for (uint64_t i = 0; i < tcount && c.ok; i++) {
        Raw r;
        r.n = c.str();
        uint32_t nd = (uint32_t)c.u(4);
        if (nd == 0 || nd > 4) { err = "invalid dimension count"; return false; }
        for (uint32_t k = 0; k < nd; k++) r.d.push_back(c.u(8));
        r.t = (uint32_t)c.u(4);
        r.off = c.u(8);
        raws.push_back(r);
    }
    if (!c.ok) { err = "truncated GGUF header"; return false; }
    uint64_t start = (c.pos + alignment - 1) & ~(alignment - 1);
    for (auto& r : raws) {
        uint64_t bs, ts;
        if (!type_layout(r.t, &bs, &ts)) { err = "unsupported tensor type in " + r.n; return false; }
        if (r.d[0] % bs) { err = "first dim not divisible by block size: " + r.n; return false; }
        uint64_t el = 1;
        for (auto d : r.d) el *= d;
        Tensor t{r.n, r.d, r.t, start + r.off, el / bs * ts};
        if (t.offset + t.nbytes > size) { err = "tensor out of file bounds: " + r.n; return false; }
        g.tensors.push_back(t);
    }
    return true;
}

bool meta_u32(const Gguf& g, const std::string& k, uint32_t* out) {  // gguf.rs:230-237
    auto it = g.meta.find(k);
    if (it == g.meta.end()) return false;
    const MetaVal& v = it->second;
    if (v.type == 4) { *out = (uint32_t)v.u; return true; }
    if (v.type == 10 && v.u <= 0xffffffffull) { *out = (uint32_t)v.u; return true; }
    if (v.type == 5 && v.i >= 0) { *out = (uint32_t)v.i; return true; }
    return false;
}
bool meta_f32(const Gguf& g, const std::string& k, float* out) {  // gguf.rs:239-245
    auto it = g.meta.find(k);
    if (it == g.meta.end()) return false;
    if (it->second.type == 6 || it->second.type == 12) { *out = (float)it->second.f; return true; }
    return false;
}

// ---------------------------------------------------------------- model (model.rs)
struct QMat {
    uint32_t type = 2;  // 2 = Q4_0 (GGUF blocks [rows][cols/32][18]), 12 = Q4_K
    int64_t rows = 0, cols = 0;
    std::vector<uint8_t> blocks;
};

struct Layer {
    std::vector<float> attn_norm, ffn_norm;
    QMat wq, wk, wv, wo, w1, w3, w2;
};

}  // namespace

struct or_model {
    std::vector<uint8_t> owned;  // memory image copy (or empty when mmapped)
    void* map = nullptr;
    size_t map_size = 0;
    int nthreads = 1;
    // config (model.rs:26-186)
    int64_t ctx = 0, d = 0, L = 0, F = 0, H = 0, Hkv = 0, hd = 0, rope_dim = 0, V = 0;
    int64_t attn_w = 0, kv_w = 0;
    float rope_base = 10000.0f, eps = 1e-5f;
    bool has_rope_scaling = false;
    float rope_scaling[4] = {0, 0, 0, 0};  // factor, original_context_length, low, high
    bool has_output = false;
    uint32_t wtype = 2;
    std::vector<float> tok_emb, out_norm;
    QMat head;
    std::vector<Layer> layers;
    ~or_model() {
        if (map) munmap(map, map_size);
    }
};

struct or_session {
    or_model* m;
    int64_t max_ctx, max_batch;
    std::vector<float> kc, vc;  // [L][max_ctx][kv_w]
    // batch workspace (inference.rs:624-695)
    std::vector<float> hidden, residual, norm_x, q, k, v, attn, gate, up, gu, scores;
    std::vector<int8_t> xq;
    std::vector<float> xs;
    std::vector<float> logits;  // single-token workspace logits [V]
    std::vector<float> row_hidden;
    int attn_order = 0;  // 0: or_attention_head, 1: or_attention_head_split
};

namespace {

bool load_f32_tensor(const Gguf& g, const std::string& name, std::vector<float>& out, std::string& err) {
    // model.rs:1081-1230 load_f32_or_f16
    const Tensor* t = g.find(name);
    if (!t) { err = "missing tensor " + name; return false; }
    uint64_t el = 1;
    for (auto dd : t->dims) el *= dd;
    out.resize(el);
    if (or_dequantize_f32((int)t->type, g.data + t->offset, (int64_t)el, out.data()) != 0) {
        err = "unsupported f32 source type for " + name;
        return false;
    }
    return true;
}

bool load_qmat(const Gguf& g, const std::string& name, int64_t rows, int64_t cols, QMat& q, std::string& err,
               bool allow_q6k = false) {
    const Tensor* t = g.find(name);
    if (!t) { err = "missing tensor " + name; return false; }
    if (t->dims.size() != 2 || (int64_t)t->dims[0] != cols || (int64_t)t->dims[1] != rows) {
        err = "bad shape for " + name;
        return false;
    }
    if (t->type != 2 && t->type != 12 && t->type != 8 && t->type != 13 && !(allow_q6k && t->type == 14)) {
        err = "unsupported matrix type for " + name;
        return false;
    }
    q.type = t->type;
    q.rows = rows;
    q.cols = cols;
    q.blocks.assign(g.data + t->offset, g.data + t->offset + t->nbytes);
    return true;
}

bool build_model(or_model* m, const uint8_t* data, size_t size, std::string& err) {
    Gguf g;
    if (!parse_gguf(data, size, g, err)) return false;
    auto it = g.meta.find("general.architecture");
    if (it == g.meta.end() || it->second.s != "llama") { err = "unsupported architecture"; return false; }
    const std::string P = "llama.";
    uint32_t v32;
    if (!meta_u32(g, P + "context_length", &v32)) { err = "missing llama.context_length"; return false; }
    m->ctx = v32;
    if (!meta_u32(g, P + "embedding_length", &v32)) { err = "missing embedding_length"; return false; }
    m->d = v32;
    if (!meta_u32(g, P + "block_count", &v32)) { err = "missing block_count"; return false; }
    m->L = v32;
    if (!meta_u32(g, P + "feed_forward_length", &v32)) { err = "missing feed_forward_length"; return false; }
    m->F = v32;
    if (!meta_u32(g, P + "attention.head_count", &v32) || v32 == 0) { err = "bad head_count"; return false; }
    m->H = v32;
    m->Hkv = meta_u32(g, P + "attention.head_count_kv", &v32) ? v32 : m->H;
    if (m->d % m->H || m->Hkv == 0 || m->H % m->Hkv) { err = "bad head geometry"; return false; }
    float f;
    m->rope_base = meta_f32(g, P + "rope.freq_base", &f) ? f : 10000.0f;
    {  // rope_scaling_from_gguf (main.rs:8522-8535)
        float fac = 0, lo = 0, hi = 0;
        uint32_t orig = 0;
        m->has_rope_scaling = meta_f32(g, P + "rope.scaling.factor", &fac) &&
                              meta_u32(g, P + "rope.scaling.original_context_length", &orig) &&
                              meta_f32(g, P + "rope.scaling.low_freq_factor", &lo) &&
                              meta_f32(g, P + "rope.scaling.high_freq_factor", &hi);
        if (m->has_rope_scaling) {
            m->rope_scaling[0] = fac;
            m->rope_scaling[1] = (float)orig;
            m->rope_scaling[2] = lo;
            m->rope_scaling[3] = hi;
        }
    }
    m->eps = meta_f32(g, P + "attention.layer_norm_rms_epsilon", &f) ? f : 1e-5f;
    const Tensor* te = g.find("token_embd.weight");
    if (!te) { err = "missing token_embd.weight"; return false; }
    if (meta_u32(g, P + "vocab_size", &v32)) m->V = v32;
    else m->V = (int64_t)(te->dims[0] == (uint64_t)m->d ? te->dims[1] : te->dims[0]);
    m->hd = meta_u32(g, P + "attention.key_length", &v32) ? v32 : m->d / m->H;
    m->rope_dim = meta_u32(g, P + "rope.dimension_count", &v32) ? v32 : m->hd;
    m->attn_w = m->H * m->hd;
    m->kv_w = m->Hkv * m->hd;
    if (!load_f32_tensor(g, "token_embd.weight", m->tok_emb, err)) return false;
    if (!load_f32_tensor(g, "output_norm.weight", m->out_norm, err)) return false;
    m->has_output = g.find("output.weight") != nullptr;
    if (m->has_output) {
        if (!load_qmat(g, "output.weight", m->V, m->d, m->head, err, true)) return false;
    } else {
        // model.rs:471-532 tied head -> Q4_0 requantisation of the f32 embeddings.
        m->head.type = 2;
        m->head.rows = m->V;
        m->head.cols = m->d;
        m->head.blocks.resize((size_t)m->V * (m->d / 32) * 18);
        parallel_rows(m->V, m->nthreads, [&](int64_t lo, int64_t hi) {
            or_quantize_q4_0_tied(m->tok_emb.data() + lo * m->d, hi - lo, m->d,
                                  m->head.blocks.data() + (size_t)lo * (m->d / 32) * 18);
        });
    }
    m->layers.resize(m->L);
    for (int64_t i = 0; i < m->L; i++) {
        Layer& ly = m->layers[i];
        std::string b = "blk." + std::to_string(i) + ".";
        if (!load_f32_tensor(g, b + "attn_norm.weight", ly.attn_norm, err)) return false;
        if (!load_f32_tensor(g, b + "ffn_norm.weight", ly.ffn_norm, err)) return false;
        // each matrix in its own type (Q4_0, Q4_K or Q6_K), as matmul_quantized_batch dispatches
        if (!load_qmat(g, b + "attn_q.weight", m->attn_w, m->d, ly.wq, err, true)) return false;
        if (!load_qmat(g, b + "attn_k.weight", m->kv_w, m->d, ly.wk, err, true)) return false;
        if (!load_qmat(g, b + "attn_v.weight", m->kv_w, m->d, ly.wv, err, true)) return false;
        if (!load_qmat(g, b + "attn_output.weight", m->d, m->attn_w, ly.wo, err, true)) return false;
        if (!load_qmat(g, b + "ffn_gate.weight", m->F, m->d, ly.w1, err, true)) return false;
        if (!load_qmat(g, b + "ffn_up.weight", m->F, m->d, ly.w3, err, true)) return false;
        if (!load_qmat(g, b + "ffn_down.weight", m->d, m->F, ly.w2, err, true)) return false;
        m->wtype = ly.wq.type;
    }
    return true;
}

void matmul(const or_model* m, float* out, const int8_t* x, const float* xs, const QMat& w, int64_t N) {
    // inference.rs:1246-1303 matmul_quantized_batch dispatch
    if (w.type == 2) or_matmul_q4_0(out, x, xs, w.blocks.data(), N, w.rows, w.cols, m->nthreads);
    else if (w.type == 14) or_matmul_q6_k(out, x, xs, w.blocks.data(), N, w.rows, w.cols, m->nthreads);
    else if (w.type == 8) or_matmul_q8_0(out, x, xs, w.blocks.data(), N, w.rows, w.cols, m->nthreads);
    else if (w.type == 13) or_matmul_q5_k(out, x, xs, w.blocks.data(), N, w.rows, w.cols, m->nthreads);
    else or_matmul_q4_k(out, x, xs, w.blocks.data(), N, w.rows, w.cols, m->nthreads);
}

void quantize_rows(const float* x, int64_t N, int64_t dim, int8_t* q, float* s) {
    // inference.rs:967-989 quantize_f32_to_q8_0_batch
    for (int64_t t = 0; t < N; t++) or_quantize_q8_0(x + t * dim, dim, q + t * dim, s + t * (dim / 32));
}

// inference.rs:3747-4111 run_layer_range_batch (dense llama layers).  N == 1 is the
// single-token run_layer_range (inference.rs:4505-4781), identical per row.
void run_layers(or_session* s, int64_t N, int64_t start_pos) {
    or_model* m = s->m;
    const int64_t d = m->d, aw = m->attn_w, kw = m->kv_w, F = m->F;
    const float scale = 1.0f / std::sqrt((float)m->hd);
    const int64_t kv_mul = m->H / m->Hkv;
    for (int64_t li = 0; li < m->L; li++) {
        const Layer& ly = m->layers[li];
        std::copy(s->hidden.begin(), s->hidden.begin() + N * d, s->residual.begin());
        for (int64_t t = 0; t < N; t++)
            or_rms_norm(&s->norm_x[t * d], &s->hidden[t * d], ly.attn_norm.data(), d, m->eps);
        quantize_rows(s->norm_x.data(), N, d, s->xq.data(), s->xs.data());
        matmul(m, s->q.data(), s->xq.data(), s->xs.data(), ly.wq, N);
        matmul(m, s->k.data(), s->xq.data(), s->xs.data(), ly.wk, N);
        matmul(m, s->v.data(), s->xq.data(), s->xs.data(), ly.wv, N);
        for (int64_t t = 0; t < N; t++) {
            int64_t pos = start_pos + t;
            const float* rs = m->has_rope_scaling ? m->rope_scaling : nullptr;
            or_rope_scaled(&s->q[t * aw], pos, m->H, m->hd, m->rope_dim, m->rope_base, 0, rs);
            or_rope_scaled(&s->k[t * kw], pos, m->Hkv, m->hd, m->rope_dim, m->rope_base, 0, rs);
            size_t off = ((size_t)li * s->max_ctx + pos) * kw;  // inference.rs:539-548
            std::copy(&s->k[t * kw], &s->k[t * kw] + kw, &s->kc[off]);
            std::copy(&s->v[t * kw], &s->v[t * kw] + kw, &s->vc[off]);
        }
        std::fill(s->attn.begin(), s->attn.begin() + N * aw, 0.0f);
        const float* kc = &s->kc[(size_t)li * s->max_ctx * kw];
        const float* vc = &s->vc[(size_t)li * s->max_ctx * kw];
        for (int64_t t = 0; t < N; t++) {
            int64_t pos = start_pos + t;
            parallel_rows(m->H, m->H >= 8 ? std::min<int>(m->nthreads, 8) : 1, [&](int64_t lo, int64_t hi) {
                std::vector<float> sc(pos + 1);
                for (int64_t h = lo; h < hi; h++) {
                    if (s->attn_order == 1)
                        or_attention_head_split(&s->attn[t * aw + h * m->hd], &s->q[t * aw + h * m->hd], kc, vc, pos,
                                                start_pos + N - 1, kw, h / kv_mul, m->hd, scale);
                    else
                        or_attention_head(&s->attn[t * aw + h * m->hd], sc.data(), &s->q[t * aw + h * m->hd], kc, vc,
                                          pos, kw, h / kv_mul, m->hd, scale);
                }
            });
        }
        quantize_rows(s->attn.data(), N, aw, s->xq.data(), s->xs.data());
        matmul(m, s->hidden.data(), s->xq.data(), s->xs.data(), ly.wo, N);
        for (int64_t i = 0; i < N * d; i++) s->hidden[i] += s->residual[i];
        std::copy(s->hidden.begin(), s->hidden.begin() + N * d, s->residual.begin());
        for (int64_t t = 0; t < N; t++)
            or_rms_norm(&s->norm_x[t * d], &s->hidden[t * d], ly.ffn_norm.data(), d, m->eps);
        quantize_rows(s->norm_x.data(), N, d, s->xq.data(), s->xs.data());
        matmul(m, s->gate.data(), s->xq.data(), s->xs.data(), ly.w1, N);
        matmul(m, s->up.data(), s->xq.data(), s->xs.data(), ly.w3, N);
        or_silu_mul(s->gu.data(), s->gate.data(), s->up.data(), N * F);
        quantize_rows(s->gu.data(), N, F, s->xq.data(), s->xs.data());
        matmul(m, s->hidden.data(), s->xq.data(), s->xs.data(), ly.w2, N);
        for (int64_t i = 0; i < N * d; i++) s->hidden[i] += s->residual[i];
    }
}

void embed(or_session* s, const uint32_t* toks, int64_t N) {
    const or_model* m = s->m;
    for (int64_t t = 0; t < N; t++)
        std::copy(&m->tok_emb[(size_t)toks[t] * m->d], &m->tok_emb[(size_t)toks[t] * m->d] + m->d,
                  &s->hidden[t * m->d]);
}

// inference.rs:4783-4832 compute_logits_from_hidden on one hidden row.
void logits_from_hidden(or_session* s, const float* h, float* out) {
    const or_model* m = s->m;
    std::vector<float> nx(m->d);
    std::vector<int8_t> q(m->d);
    std::vector<float> xs(m->d / 32);
    or_rms_norm(nx.data(), h, m->out_norm.data(), m->d, m->eps);
    or_quantize_q8_0(nx.data(), m->d, q.data(), xs.data());
    matmul(m, out, q.data(), xs.data(), m->head, 1);
}

// ---------------------------------------------------------------- spec helpers
constexpr uint32_t PURPOSE_DRAFT = 1, PURPOSE_ACCEPT = 2, PURPOSE_RESAMPLE = 3, PURPOSE_BONUS = 7;
constexpr uint32_t PURPOSE_PROMPT = 4, PURPOSE_ORACLE_U = 5, PURPOSE_ORACLE_ID = 6;

uint32_t philox_word(uint64_t seed, uint64_t pos, uint32_t purpose) {
    uint32_t ctr[4] = {(uint32_t)pos, (uint32_t)(pos >> 32), purpose, 0};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    or_philox4x32_10(ctr, key, out);
    return out[0];
}
// u in [0,1) from the top 24 bits.
float philox_uniform(uint64_t seed, uint64_t pos, uint32_t purpose) {
    return (float)(philox_word(seed, pos, purpose) >> 8) * (1.0f / 16777216.0f);
}

void prefill(or_session* s, const uint32_t* toks, int64_t n, int64_t start_pos, int64_t chunk) {
    // main.rs:9415-9485 prefill_tokens: chunks of the batch width; a lone token takes the
    // single-token path.  Per-row numerics are identical either way.
    int64_t pos = start_pos;
    for (int64_t i = 0; i < n; i += chunk) {
        int64_t len = std::min(chunk, n - i);
        or_prefill_pass_batch(s, toks + i, len, pos);
        pos += len;
    }
}

}  // namespace

extern "C" {

static or_model* finish_load(or_model* m, const uint8_t* data, size_t size, char* err, int errlen) {
    std::string e;
    if (!build_model(m, data, size, e)) {
        if (err && errlen > 0) std::snprintf(err, errlen, "%s", e.c_str());
        delete m;
        return nullptr;
    }
    return m;
}

or_model* or_model_load(const char* path, int nthreads, char* err, int errlen) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        if (err) std::snprintf(err, errlen, "cannot open %s", path);
        return nullptr;
    }
    struct stat st;
    fstat(fd, &st);
    void* p = mmap(nullptr, st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) {
        if (err) std::snprintf(err, errlen, "mmap failed");
        return nullptr;
    }
    or_model* m = new or_model();
    m->nthreads = nthreads;
    m->map = p;
    m->map_size = st.st_size;
    return finish_load(m, (const uint8_t*)p, st.st_size, err, errlen);
}

or_model* or_model_load_memory(const void* data, size_t size, int nthreads, char* err, int errlen) {
    or_model* m = new or_model();
    m->nthreads = nthreads;
    return finish_load(m, (const uint8_t*)data, size, err, errlen);
}

void or_model_free(or_model* m) { delete m; }

void or_model_info(const or_model* m, int64_t* o) {
    int64_t v[16] = {m->ctx, m->d, m->L, m->F, m->H, m->Hkv, m->hd, m->rope_dim, m->V, m->attn_w,
                     m->kv_w, m->has_output ? 1 : 0, (int64_t)m->wtype, 0, 0, 0};
    std::memcpy(o, v, sizeof(v));
}
void or_model_info_f(const or_model* m, float* o) {
    o[0] = m->rope_base;
    o[1] = m->eps;
}

int64_t or_model_head_q4_0(const or_model* m, uint8_t* out, int64_t cap) {
    if (m->head.type != 2 || (int64_t)m->head.blocks.size() > cap) return -1;
    std::memcpy(out, m->head.blocks.data(), m->head.blocks.size());
    return (int64_t)m->head.blocks.size();
}

or_session* or_session_create(or_model* m, int64_t max_ctx, int64_t max_batch) {
    or_session* s = new or_session();
    s->m = m;
    s->max_ctx = max_ctx;
    s->max_batch = max_batch;
    s->kc.assign((size_t)m->L * max_ctx * m->kv_w, 0.0f);
    s->vc.assign((size_t)m->L * max_ctx * m->kv_w, 0.0f);
    int64_t B = max_batch;
    s->hidden.resize(B * m->d);
    s->residual.resize(B * m->d);
    s->norm_x.resize(B * m->d);
    s->q.resize(B * m->attn_w);
    s->k.resize(B * m->kv_w);
    s->v.resize(B * m->kv_w);
    s->attn.resize(B * m->attn_w);
    s->gate.resize(B * m->F);
    s->up.resize(B * m->F);
    s->gu.resize(B * m->F);
    int64_t mx = std::max({m->d, m->F, m->attn_w});
    s->xq.resize(B * mx);
    s->xs.resize(B * (mx / 32 + 1));
    s->logits.resize(m->V);
    return s;
}

void or_session_free(or_session* s) { delete s; }
void or_session_set_attention(or_session* s, int order) { s->attn_order = order == 1 ? 1 : 0; }

void or_model_set_threads(or_model* m, int nthreads) { m->nthreads = nthreads > 0 ? nthreads : 1; }

void or_synth_kv_values(uint64_t seed, int32_t layer, int32_t kind, int64_t start, int64_t count, float* out) {
    // No reference counterpart: BASELINE config 4's KV cache "filled with N(0, 1) keys and
    // values".  Pair j = element / 2 of stream 2 * layer + kind: Philox4x32-10 with counter
    // (j low, j high, stream, purpose 10) and key (seed low, seed high); two 53-bit uniforms
    // u1 in (0, 1] and u2 in [0, 1); Box-Muller in double, z0 = r cos(2 pi u2), z1 = r sin(2 pi u2)
    // with r = sqrt(-2 ln u1); each rounded to f32.
    const uint32_t stream = (uint32_t)(2 * layer + kind);
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int64_t e = 0; e < count; e += 2) {
        const uint64_t j = (uint64_t)(start + e) / 2;
        const uint32_t ctr[4] = {(uint32_t)j, (uint32_t)(j >> 32), stream, 10u};
        uint32_t w[4];
        or_philox4x32_10(ctr, key, w);
        const double u1 = ((double)(((uint64_t)(w[0] >> 5) << 26) | (w[1] >> 6)) + 1.0) / 9007199254740992.0;
        const double u2 = (double)(((uint64_t)(w[2] >> 5) << 26) | (w[3] >> 6)) / 9007199254740992.0;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double a = 6.283185307179586 * u2;
        out[e] = (float)(r * std::cos(a));
        out[e + 1] = (float)(r * std::sin(a));
    }
}

void or_session_fill_kv(or_session* s, int64_t n, uint64_t seed) {
    // rows [0, n) of every layer: key row p = elements [p * kv_width, (p + 1) * kv_width) of
    // stream (layer, 0), value row p the same of stream (layer, 1)
    const int64_t kw = s->m->kv_w, L = s->m->L;
    n = std::min(n, s->max_ctx);
    const int nth = std::max(1, s->m->nthreads);
    std::vector<std::thread> th;
    for (int t = 0; t < nth; t++)
        th.emplace_back([=] {
            for (int64_t l = t; l < L; l += nth)
                for (int64_t p = 0; p < n; p++) {
                    or_synth_kv_values(seed, (int32_t)l, 0, p * kw, kw, &s->kc[((size_t)l * s->max_ctx + p) * kw]);
                    or_synth_kv_values(seed, (int32_t)l, 1, p * kw, kw, &s->vc[((size_t)l * s->max_ctx + p) * kw]);
                }
        });
    for (auto& x : th) x.join();
}

void or_prefill_pass_batch(or_session* s, const uint32_t* toks, int64_t n, int64_t start_pos) {
    if (n <= 0) return;
    if (n > s->max_batch || start_pos + n > s->max_ctx) {  // inference.rs:3712-3722
        std::fprintf(stderr, "oracle: batch out of bounds\n");
        std::abort();
    }
    embed(s, toks, n);
    run_layers(s, n, start_pos);
}

void or_forward_pass(or_session* s, uint32_t tok, int64_t pos) {
    or_prefill_pass_batch(s, &tok, 1, pos);
    logits_from_hidden(s, s->hidden.data(), s->logits.data());
}

void or_batch_row_logits(or_session* s, int64_t row, float* out) {
    logits_from_hidden(s, &s->hidden[row * s->m->d], out);
}

const float* or_session_logits(const or_session* s) { return s->logits.data(); }
const float* or_session_batch_hidden(const or_session* s) { return s->hidden.data(); }

static float top2_margin(const float* l, int64_t V, int64_t best) {
    float second = -INFINITY;
    for (int64_t i = 0; i < V; i++)
        if (i != best && l[i] > second) second = l[i];
    return l[best] - second;
}

void or_verify_greedy(or_session* s, const uint32_t* toks, int64_t n, int64_t start_pos,
                      uint32_t* preds, float* margins, float* logits_out) {
    or_prefill_pass_batch(s, toks, n, start_pos);
    std::vector<float> lg(s->m->V);
    for (int64_t i = 0; i < n; i++) {
        float* dst = logits_out ? logits_out + i * s->m->V : lg.data();
        or_batch_row_logits(s, i, dst);
        int64_t a = or_argmax(dst, s->m->V);
        preds[i] = (uint32_t)a;
        if (margins) margins[i] = top2_margin(dst, s->m->V, a);
    }
}

int or_generate_greedy(or_session* s, const uint32_t* prompt, int64_t n_prompt, int64_t n_new,
                       int64_t prefill_batch, uint32_t* out) {
    // main.rs:9676-9706: prefix via prefill_tokens, last prompt token via forward_pass,
    // then the plain greedy loop (sample, emit, forward).
    prefill(s, prompt, n_prompt - 1, 0, prefill_batch);
    int64_t pos = n_prompt - 1;
    or_forward_pass(s, prompt[n_prompt - 1], pos);
    pos++;
    for (int64_t i = 0; i < n_new; i++) {
        uint32_t t = (uint32_t)or_argmax(s->logits.data(), s->m->V);
        out[i] = t;
        if (i + 1 < n_new) {
            or_forward_pass(s, t, pos);
            pos++;
        }
    }
    return 0;
}

int64_t or_generate_plain(or_session* s, const uint32_t* prompt, int64_t n_prompt, int64_t n_new, float temp,
                          uint64_t* rng_state, const uint32_t* stop, int64_t n_stop, int64_t prefill_batch,
                          uint32_t* out) {
    // main.rs:9676-9706 prefill, then the plain loop (main.rs:9894-9928): sample, end at a stop
    // token, the context end or n_new, emit, end at n_new, forward
    uint64_t st_unused = 0;
    uint64_t* rs = rng_state ? rng_state : &st_unused;
    prefill(s, prompt, n_prompt - 1, 0, prefill_batch);
    int64_t pos = n_prompt - 1;
    or_forward_pass(s, prompt[n_prompt - 1], pos);
    pos++;
    int64_t produced = 0;
    for (;;) {
        const uint32_t t = (uint32_t)or_sample_logits(s->logits.data(), s->m->V, temp, rs);
        if (std::find(stop, stop + n_stop, t) != stop + n_stop || pos >= s->max_ctx || produced >= n_new) break;
        out[produced++] = t;
        if (produced >= n_new) break;
        or_forward_pass(s, t, pos);
        pos++;
    }
    return produced;
}

int64_t or_generate_speculative_draft(or_session* tg, or_session* dr, const uint32_t* prompt,
                                      int64_t n_prompt, int64_t n_new, int64_t draft_k,
                                      int64_t prefill_batch, uint32_t* out, int64_t* stats,
                                      int64_t* steps_out) {
    return or_generate_speculative_draft_temp(tg, dr, prompt, n_prompt, n_new, draft_k, 0.0f, nullptr, nullptr, 0,
                                              prefill_batch, out, stats, steps_out);
}

int64_t or_generate_speculative_draft_temp(or_session* tg, or_session* dr, const uint32_t* prompt,
                                           int64_t n_prompt, int64_t n_new, int64_t draft_k, float temp,
                                           uint64_t* rng_state, const uint32_t* stop, int64_t n_stop,
                                           int64_t prefill_batch, uint32_t* out, int64_t* stats,
                                           int64_t* steps_out) {
    // main.rs:9643-9706 prefill of both models, then speculative.rs:299-494 per step with the
    // generate loop's turn end (main.rs:9852-9866); every sample is sample_logits (argmax at
    // temp <= 0).
    const int64_t V = tg->m->V;
    uint64_t st_unused = 0;
    uint64_t* rs = rng_state ? rng_state : &st_unused;
    auto sample = [&](const float* l) { return (uint32_t)or_sample_logits(l, V, temp, rs); };
    auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    prefill(dr, prompt, n_prompt - 1, 0, std::min(prefill_batch, dr->max_batch));
    or_forward_pass(dr, prompt[n_prompt - 1], n_prompt - 1);
    prefill(tg, prompt, n_prompt - 1, 0, prefill_batch);
    or_forward_pass(tg, prompt[n_prompt - 1], n_prompt - 1);
    int64_t pos = n_prompt, dpos = n_prompt, produced = 0, steps = 0;
    stats[0] = stats[1] = 0;
    std::vector<float> lg(V);
    bool saw_stop = false;
    while (!saw_stop && produced < n_new && pos < tg->max_ctx) {
        int64_t k = std::min(draft_k, n_new - produced);
        k = std::min(k, tg->max_batch);
        k = std::min(k, tg->max_ctx - (pos + 1));
        k = std::min(k, dr->max_ctx - (pos + 1));
        if (k <= 0) break;
        std::vector<uint32_t> drafts;
        int64_t cdp = pos;
        while ((int64_t)drafts.size() < k) {
            uint32_t t = sample(dr->logits.data());
            drafts.push_back(t);
            if (is_stop(t)) break;  // speculative.rs:336-338: drafted, never run on the draft
            or_forward_pass(dr, t, cdp);
            cdp++;
        }
        k = (int64_t)drafts.size();
        or_prefill_pass_batch(tg, drafts.data(), k, pos);
        std::vector<uint32_t> acc;
        bool rejected = false;
        stats[0] += k;
        for (int64_t i = 0; i < k; i++) {
            const float* l;
            if (i > 0) {
                or_batch_row_logits(tg, i - 1, lg.data());
                l = lg.data();
            } else {
                l = tg->logits.data();
            }
            uint32_t tt = sample(l);
            if (drafts[i] == tt) {
                acc.push_back(tt);
                stats[1]++;
                if (is_stop(tt)) {  // speculative.rs:404-412: verification ends, no trailing token
                    pos = dpos = pos + i + 1;
                    rejected = true;
                    break;
                }
            } else {
                rejected = true;
                acc.push_back(tt);
                or_forward_pass(tg, tt, pos + i);
                or_forward_pass(dr, tt, pos + i);
                pos = dpos = pos + i + 1;
                break;
            }
        }
        if (!rejected) {
            or_batch_row_logits(tg, k - 1, lg.data());
            uint32_t tt = sample(lg.data());
            acc.push_back(tt);
            or_forward_pass(tg, tt, pos + k);
            or_forward_pass(dr, tt, pos + k);
            pos = dpos = pos + k + 1;
        }
        for (auto t : acc) {
            if (is_stop(t)) {  // the turn ends; the stop token is not part of the stream
                saw_stop = true;
                break;
            }
            if (produced < n_new) out[produced++] = t;
        }
        steps++;
    }
    (void)dpos;
    if (steps_out) *steps_out = steps;
    return produced;
}

uint32_t or_oracle_draft(uint64_t seed, int64_t p, float alpha, const uint32_t* greedy,
                         int64_t n_prompt, int64_t n_greedy, uint32_t vocab) {
    float u = philox_uniform(seed, (uint64_t)p, PURPOSE_ORACLE_U);
    int64_t gi = p - n_prompt;
    if (u < alpha && gi >= 0 && gi < n_greedy) return greedy[gi];
    return philox_word(seed, (uint64_t)p, PURPOSE_ORACLE_ID) % vocab;
}

void or_uniform_prompt(uint64_t seed, int64_t n, uint32_t vocab, uint32_t* ids) {
    for (int64_t i = 0; i < n; i++) ids[i] = philox_word(seed, (uint64_t)i, PURPOSE_PROMPT) % vocab;
}

int64_t or_generate_speculative_oracle(or_session* s, const uint32_t* prompt, int64_t n_prompt,
                                       int64_t n_new, int64_t k, float alpha, uint64_t seed,
                                       const uint32_t* greedy, int64_t prefill_batch, uint32_t* out,
                                       int64_t* stats, int64_t* steps_out) {
    // k+1 form (cluster_tcp_smoke.rs:905-979): batch = [pending] + drafts, preds after
    // every row, accepted = longest prefix with draft[i] == pred[i], next = pred[accepted].
    const int64_t V = s->m->V;
    prefill(s, prompt, n_prompt - 1, 0, prefill_batch);
    or_forward_pass(s, prompt[n_prompt - 1], n_prompt - 1);
    uint32_t pending = (uint32_t)or_argmax(s->logits.data(), V);
    int64_t pos = n_prompt, produced = 0, steps = 0;
    stats[0] = stats[1] = 0;
    out[produced++] = pending;
    std::vector<uint32_t> batch, preds;
    while (produced < n_new) {
        int64_t kk = std::min(k, s->max_batch - 1);
        kk = std::min(kk, s->max_ctx - pos - 1);
        if (kk < 0) break;
        batch.assign(1, pending);
        for (int64_t i = 1; i <= kk; i++)
            batch.push_back(or_oracle_draft(seed, pos + i, alpha, greedy, n_prompt, n_new, (uint32_t)V));
        preds.resize(kk + 1);
        or_verify_greedy(s, batch.data(), kk + 1, pos, preds.data(), nullptr, nullptr);
        int64_t a = 0;
        while (a < kk && batch[a + 1] == preds[a]) a++;
        stats[0] += kk;
        stats[1] += a;
        for (int64_t i = 1; i <= a && produced < n_new; i++) out[produced++] = batch[i];
        pending = preds[a];
        if (produced < n_new) out[produced++] = pending;
        pos += a + 1;
        steps++;
    }
    if (steps_out) *steps_out = steps;
    return produced;
}

int64_t or_ngram_draft(const uint32_t* history, int64_t len, int64_t min_ngram, int64_t max_ngram,
                       int64_t max_tokens, uint32_t* out) {
    // NGramDrafter::draft (speculative.rs:81-103): longest suffix n-gram (max_ngram down to
    // min_ngram) with an earlier occurrence, most recent occurrence first; propose what
    // followed it, at most max_tokens and never past the end of the history.
    if (max_tokens <= 0 || min_ngram <= 0 || len <= min_ngram) return 0;
    const int64_t max_n = std::min(max_ngram, len - 1);
    for (int64_t n = max_n; n >= min_ngram; n--) {
        const uint32_t* pat = history + len - n;
        for (int64_t start = len - n - 1; start >= 0; start--) {
            if (std::equal(pat, pat + n, history + start)) {
                const int64_t cs = start + n, ce = std::min(cs + max_tokens, len);
                if (cs < ce) {
                    std::copy(history + cs, history + ce, out);
                    return ce - cs;
                }
                break;
            }
        }
    }
    return 0;
}

int64_t or_generate_speculative_ngram(or_session* s, const uint32_t* prompt, int64_t n_prompt, int64_t n_new,
                                      int64_t k, int64_t min_ngram, int64_t max_ngram, const uint32_t* stop,
                                      int64_t n_stop, int64_t prefill_batch, uint32_t* out, int64_t* stats,
                                      int64_t* steps_out) {
    // ngram_speculative_step (speculative.rs:122-286) driven by main.rs:9729-9776, greedy, in
    // the k+1 verify form (cluster_tcp_smoke.rs:905-979): each step verifies [pending] + drafts
    // drawn from the history that ends with pending, and the corrective token is the next
    // step's pending (no separate forward); the emitted stream is the target's greedy stream,
    // cut before the first stop token (stop tokens are neither emitted nor consumed).
    const int64_t V = s->m->V;
    auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    prefill(s, prompt, n_prompt - 1, 0, prefill_batch);
    or_forward_pass(s, prompt[n_prompt - 1], n_prompt - 1);
    uint32_t pending = (uint32_t)or_argmax(s->logits.data(), V);
    std::vector<uint32_t> history(prompt, prompt + n_prompt), batch, preds, drafts(std::max<int64_t>(k, 1));
    int64_t pos = n_prompt, produced = 0, steps = 0;
    stats[0] = stats[1] = 0;
    bool stopped = false;
    while (produced < n_new && !stopped) {
        if (is_stop(pending)) break;
        out[produced++] = pending;
        history.push_back(pending);
        if (produced >= n_new) break;
        // main.rs:9736-9737: a step emits at most the token budget (pending is counted)
        int64_t kk = std::min(k, n_new - produced);
        kk = std::min(kk, s->max_batch - 1);
        kk = std::min(kk, s->max_ctx - pos - 1);
        if (kk < 0) break;
        const int64_t nd = kk > 0 ? or_ngram_draft(history.data(), (int64_t)history.size(), min_ngram, max_ngram,
                                                   kk, drafts.data())
                                  : 0;
        batch.assign(1, pending);
        batch.insert(batch.end(), drafts.begin(), drafts.begin() + nd);
        preds.resize(nd + 1);
        or_verify_greedy(s, batch.data(), nd + 1, pos, preds.data(), nullptr, nullptr);
        int64_t a = 0;
        while (a < nd && batch[a + 1] == preds[a]) a++;
        stats[0] += nd;
        int64_t counted = a;  // the step stops counting at a stop prediction
        for (int64_t i = 1; i <= a && produced < n_new; i++) {
            if (is_stop(batch[i])) {
                stopped = true;
                counted = i;
                break;
            }
            out[produced++] = batch[i];
            history.push_back(batch[i]);
        }
        stats[1] += counted;
        pending = preds[a];
        pos += a + 1;
        steps++;
    }
    if (steps_out) *steps_out = steps;
    return produced;
}

int64_t or_generate_speculative_ngram_temp(or_session* s, const uint32_t* prompt, int64_t n_prompt, int64_t n_new,
                                           int64_t k, int64_t min_ngram, int64_t max_ngram, float temp,
                                           uint64_t* rng_state, const uint32_t* stop, int64_t n_stop,
                                           int64_t prefill_batch, uint32_t* out, int64_t* stats,
                                           int64_t* steps_out) {
    if (!(temp > 0.0f))
        return or_generate_speculative_ngram(s, prompt, n_prompt, n_new, k, min_ngram, max_ngram, stop, n_stop,
                                             prefill_batch, out, stats, steps_out);
    // The generate loop of main.rs:9729-9776 over ngram_speculative_step (speculative.rs:122-286):
    // t0 drawn from the live logits (a stop token ends the turn unemitted), drafts from the
    // history that ends in t0 (k clamped to the token budget minus one, then to the batch and
    // the context), one batched pass over t0 + drafts, one draw per verified row in order:
    // a stop prediction ends the turn, a mismatch emits the prediction and runs it as a
    // corrective forward, and when every draft matches the last row's logits are the next
    // step's live logits.
    const int64_t V = s->m->V;
    uint64_t st_unused = 0;
    uint64_t* rs = rng_state ? rng_state : &st_unused;
    auto sample = [&](const float* l) { return (uint32_t)or_sample_logits(l, V, temp, rs); };
    auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    prefill(s, prompt, n_prompt - 1, 0, prefill_batch);
    or_forward_pass(s, prompt[n_prompt - 1], n_prompt - 1);
    std::vector<uint32_t> history(prompt, prompt + n_prompt), drafts(std::max<int64_t>(k, 1)), emitted;
    std::vector<float> lg(V);
    int64_t live_row = -1;  // -1: s->logits; else that row of the last batched pass
    int64_t pos = n_prompt, produced = 0, steps = 0;
    stats[0] = stats[1] = 0;
    for (;;) {
        if (pos >= s->max_ctx || produced >= n_new) break;
        const int64_t ck = std::min(k, n_new - produced - 1);
        if (live_row >= 0) or_batch_row_logits(s, live_row, lg.data());
        const uint32_t t0 = sample(live_row >= 0 ? lg.data() : s->logits.data());
        if (is_stop(t0)) break;
        history.push_back(t0);
        int64_t nd = ck > 0 ? or_ngram_draft(history.data(), (int64_t)history.size(), min_ngram, max_ngram, ck,
                                             drafts.data())
                            : 0;
        nd = std::min(nd, std::min(s->max_batch - 1, s->max_ctx - (pos + 1)));
        steps++;
        if (nd <= 0) {
            or_forward_pass(s, t0, pos);
            live_row = -1;
            out[produced++] = t0;
            pos++;
            continue;
        }
        stats[0] += nd;
        std::vector<uint32_t> batch(1, t0);
        batch.insert(batch.end(), drafts.begin(), drafts.begin() + nd);
        or_prefill_pass_batch(s, batch.data(), nd + 1, pos);
        emitted.assign(1, t0);
        bool hit_stop = false, done = false;
        for (int64_t i = 0; i < nd; i++) {
            or_batch_row_logits(s, i, lg.data());
            const uint32_t tt = sample(lg.data());
            if (drafts[i] == tt) stats[1]++;
            if (is_stop(tt)) {  // neither emitted nor consumed
                hit_stop = done = true;
                pos += i + 1;
                break;
            }
            if (drafts[i] == tt) {
                emitted.push_back(tt);
            } else {
                emitted.push_back(tt);
                or_forward_pass(s, tt, pos + i + 1);
                live_row = -1;
                pos += i + 2;
                done = true;
                break;
            }
        }
        if (!done) {
            live_row = nd;
            pos += nd + 1;
        }
        for (size_t j = 1; j < emitted.size(); j++) history.push_back(emitted[j]);
        for (uint32_t t : emitted) out[produced++] = t;  // at most ck + 1 <= the budget
        if (hit_stop) break;
    }
    if (steps_out) *steps_out = steps;
    return produced;
}

void or_temperature_probs(const float* logits, int64_t V, float temp, float* probs) {
    // Max, exp((l - max) / T) (as inference.rs:4857-4862), sequential sum, then the
    // softmax normalisation (inference.rs:3535-3539): p = e * (1 / sum).
    float mx = logits[0];
    for (int64_t i = 0; i < V; i++)
        if (logits[i] > mx) mx = logits[i];
    float sum = 0.0f;
    for (int64_t i = 0; i < V; i++) {
        probs[i] = expf((logits[i] - mx) / temp);
        sum += probs[i];
    }
    float inv = 1.0f / sum;
    for (int64_t i = 0; i < V; i++) probs[i] *= inv;
}

// Fixed-point inverse CDF (this build's stochastic specification; the reference samples with
// a sequential f32 walk, inference.rs:4865-4872, and has no speculative sampler).  Weights
// W_j = floor(w_j * 2^40) are exact integers, so their prefix sums do not depend on the
// summation order: the GPU evaluates the same sampler with a parallel scan.  With
// total = sum W_j and u = k24 / 2^24, the sample is the first j whose inclusive prefix
// exceeds target = floor(k24 * total / 2^24) (< total, so such a j exists and W_j > 0).
// Returns false when every weight is zero.
static inline uint64_t fixed_weight(float w) { return w > 0.0f ? (uint64_t)(w * 1099511627776.0f) : 0u; }

static bool sample_fixed(const float* w, int64_t V, uint32_t k24, uint32_t* out) {
    uint64_t total = 0;
    for (int64_t i = 0; i < V; i++) total += fixed_weight(w[i]);
    if (total == 0) return false;
    const uint64_t th = total >> 32, tl = total & 0xffffffffu;
    const uint64_t target = ((k24 * th) << 8) + ((k24 * tl) >> 24);
    uint64_t c = 0;
    for (int64_t i = 0; i < V; i++) {
        c += fixed_weight(w[i]);
        if (c > target) {
            *out = (uint32_t)i;
            return true;
        }
    }
    return false;  // unreachable: target < total
}

static uint32_t philox_u24(uint64_t seed, uint64_t pos, uint32_t purpose) { return philox_word(seed, pos, purpose) >> 8; }

uint32_t or_sample_inverse_cdf(const float* probs, int64_t V, float u) {
    uint32_t k24 = (uint32_t)((double)u * 16777216.0), out = 0;
    if (k24 > 0xffffffu) k24 = 0xffffffu;
    return sample_fixed(probs, V, k24, &out) ? out : 0u;
}

void or_stochastic_accept(const float* p_logits, const float* q_probs, const uint32_t* drafts,
                          int64_t k, int64_t V, float temp, uint64_t seed, int64_t start_pos,
                          int64_t* n_accepted, uint32_t* next_token) {
    // Row i of the k+1 verify batch sits at position start_pos + i and scores draft i.
    // Draft i is accepted iff u * q_i(x) < p_i(x) (probability min(1, p/q)); at the first
    // rejection the next token is drawn from max(0, p_i - q_i) (from p_i if that residual
    // has no fixed-point mass); after k acceptances the bonus token is drawn from p_k.
    std::vector<float> p(V), r(V);
    for (int64_t i = 0; i < k; i++) {
        or_temperature_probs(p_logits + i * V, V, temp, p.data());
        const float* q = q_probs + i * V;
        const uint32_t x = drafts[i];
        const float u = philox_uniform(seed, (uint64_t)(start_pos + i), PURPOSE_ACCEPT);
        if (u * q[x] < p[x]) continue;
        for (int64_t j = 0; j < V; j++) {
            const float dlt = p[j] - q[j];
            r[j] = dlt > 0.0f ? dlt : 0.0f;
        }
        const uint32_t k24 = philox_u24(seed, (uint64_t)(start_pos + i), PURPOSE_RESAMPLE);
        uint32_t t = 0;
        if (!sample_fixed(r.data(), V, k24, &t)) sample_fixed(p.data(), V, k24, &t);
        *n_accepted = i;
        *next_token = t;
        return;
    }
    or_temperature_probs(p_logits + k * V, V, temp, p.data());
    uint32_t t = 0;
    sample_fixed(p.data(), V, philox_u24(seed, (uint64_t)(start_pos + k), PURPOSE_BONUS), &t);
    *n_accepted = k;
    *next_token = t;
}

int64_t or_generate_speculative_stochastic(or_session* tg, or_session* dr, const uint32_t* prompt,
                                           int64_t n_prompt, int64_t n_new, int64_t k, float temp,
                                           uint64_t seed, int64_t prefill_batch, uint32_t* out,
                                           int64_t* stats, int64_t* steps_out) {
    // Draft-model speculative sampling in the k+1 form (no reference counterpart: the
    // reference's temperature path matches tokens, speculative.rs:403).  Per step at
    // position pos with the pending token t0: the draft runs t0, d_0, .., d_{k-2} at
    // pos .. pos+k-1 and samples d_i from q_i = softmax(draft logits / T) with
    // u(seed, pos+i, draft); the target verifies [t0, d_0 .. d_{k-1}] at pos .. pos+k;
    // or_stochastic_accept decides.  After a full acceptance the draft first catches up
    // on d_{k-1}.  The first token is drawn from the target's last prompt row with
    // u(seed, n_prompt-1, bonus).
    const int64_t V = tg->m->V;
    prefill(dr, prompt, n_prompt, 0, std::min(prefill_batch, dr->max_batch));
    prefill(tg, prompt, n_prompt - 1, 0, prefill_batch);
    or_forward_pass(tg, prompt[n_prompt - 1], n_prompt - 1);
    std::vector<float> p(V), q, lg;
    or_temperature_probs(tg->logits.data(), V, temp, p.data());
    uint32_t pending = 0;
    sample_fixed(p.data(), V, philox_u24(seed, (uint64_t)(n_prompt - 1), PURPOSE_BONUS), &pending);
    int64_t pos = n_prompt, produced = 0, steps = 0;
    uint32_t last_draft = 0;
    bool catch_up = false;  // the last step accepted all of its drafts (and drafted some)
    stats[0] = stats[1] = 0;
    out[produced++] = pending;
    std::vector<uint32_t> batch;
    while (produced < n_new) {
        int64_t kk = std::min(k, tg->max_batch - 1);
        kk = std::min(kk, tg->max_ctx - pos - 1);
        kk = std::min(kk, dr->max_ctx - pos - 1);
        if (kk < 0) break;
        if (kk > 0 && catch_up) or_forward_pass(dr, last_draft, pos - 1);  // d_{k-1} at pos - 1
        batch.assign(1, pending);
        q.resize((size_t)kk * V);
        uint32_t x = pending;
        for (int64_t i = 0; i < kk; i++) {
            or_forward_pass(dr, x, pos + i);
            or_temperature_probs(dr->logits.data(), V, temp, &q[(size_t)i * V]);
            sample_fixed(&q[(size_t)i * V], V, philox_u24(seed, (uint64_t)(pos + i), PURPOSE_DRAFT), &x);
            batch.push_back(x);
        }
        or_prefill_pass_batch(tg, batch.data(), kk + 1, pos);
        lg.resize((size_t)(kk + 1) * V);
        for (int64_t i = 0; i <= kk; i++) or_batch_row_logits(tg, i, &lg[(size_t)i * V]);
        int64_t a = 0;
        uint32_t next = 0;
        or_stochastic_accept(lg.data(), q.data(), batch.data() + 1, kk, V, temp, seed, pos, &a, &next);
        stats[0] += kk;
        stats[1] += a;
        for (int64_t i = 1; i <= a && produced < n_new; i++) out[produced++] = batch[i];
        if (produced < n_new) out[produced++] = next;
        if (kk > 0) last_draft = batch[kk];
        catch_up = kk > 0 && a == kk;
        pos += a + 1;
        pending = next;
        steps++;
    }
    if (steps_out) *steps_out = steps;
    return produced;
}

}  // extern "C"
