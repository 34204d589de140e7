// GGUF v2/v3 reader and the seeded synthetic-model writer.
//
// Reader: same header walk as gguf::read_file (src/gguf.rs:454-551): magic, version
// 2..3, tensor/metadata counts, metadata key/values, tensor infos, data start
// aligned to general.alignment (default 32, gguf.rs:10), byte sizes from the type
// layout table (gguf.rs:154-185, tensor_nbytes gguf.rs:737-763).
#include "gguf.h"

#include <cmath>
#include <cstring>
#include <set>
#include <thread>

namespace nc {

namespace {

struct Cur {
    const uint8_t* p;
    size_t n, pos = 0;
    bool ok = true;
    uint64_t u(int b) {
        if (pos + b > n) {
            ok = false;
            return 0;
        }
        uint64_t v = 0;
        for (int i = 0; i < b; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += b;
        return v;
    }
    std::string s() {
        uint64_t len = u(8);
        if (!ok || pos + len > n) {
            ok = false;
            return "";
        }
        std::string r((const char*)p + pos, len);
        pos += len;
        return r;
    }
};

bool skip_or_read(Cur& c, uint32_t type, GgufValue& v, int depth) {
    v.type = (int)type;
    switch (type) {
        case 0: v.u = c.u(1); return c.ok;
        case 1: v.i = (int8_t)c.u(1); return c.ok;
        case 2: v.u = c.u(2); return c.ok;
        case 3: v.i = (int16_t)c.u(2); return c.ok;
        case 4: v.u = c.u(4); return c.ok;
        case 5: v.i = (int32_t)c.u(4); return c.ok;
        case 6: { uint32_t b = (uint32_t)c.u(4); float f; std::memcpy(&f, &b, 4); v.f = f; return c.ok; }
        case 7: v.u = c.u(1); return c.ok && v.u <= 1;
        case 8: v.s = c.s(); return c.ok;
        case 9: {
            if (depth) return false;
            uint32_t it = (uint32_t)c.u(4);
            uint64_t len = c.u(8);
            v.item_type = (int)it;
            v.count = len;
            for (uint64_t k = 0; k < len && c.ok; k++) {
                GgufValue t;
                if (!skip_or_read(c, it, t, 1)) return false;
                if (it == 8) v.strs.push_back(std::move(t.s));  // string arrays are kept (tokens)
            }
            return c.ok;
        }
        case 10: v.u = c.u(8); return c.ok;
        case 11: v.i = (int64_t)c.u(8); return c.ok;
        case 12: { uint64_t b = c.u(8); double d; std::memcpy(&d, &b, 8); v.f = d; return c.ok; }
        default: return false;
    }
}

}  // namespace

// GgufTensorType::layout (gguf.rs:154-185): (values per block, bytes per block); false for
// type ids that have no layout (removed or unknown types).
bool gguf_type_layout(uint32_t t, uint64_t* block, uint64_t* bytes) {
    struct L {
        uint32_t id;
        uint16_t block, bytes;
    };
    static const L table[] = {
        {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
        {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
        {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
        {26, 1, 4},     {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},
    };
    for (const L& e : table)
        if (e.id == t) {
            *block = e.block;
            *bytes = e.bytes;
            return true;
        }
    return false;
}

// tensor_nbytes (gguf.rs:737-763): the first dimension must be a whole number of blocks, and
// neither the element count nor the byte size may overflow 64 bits.
bool gguf_tensor_nbytes(const std::string& name, const std::vector<uint64_t>& dims, uint32_t type, uint64_t* out,
                        std::string& err) {
    uint64_t bs, ts;
    if (!gguf_type_layout(type, &bs, &ts)) {
        err = "tensor " + name + " has unknown or removed GGML type " + std::to_string(type);
        return false;
    }
    const uint64_t first = dims.empty() ? 1 : dims[0];
    if (first % bs) {
        err = "tensor " + name + " first dimension " + std::to_string(first) + " is not divisible by block size " +
              std::to_string(bs);
        return false;
    }
    uint64_t el = 1;
    for (uint64_t d : dims) {
        if (d != 0 && el > UINT64_MAX / d) {
            err = "tensor " + name + " element count overflow";
            return false;
        }
        el *= d;
    }
    const uint64_t blocks = el / bs;
    if (blocks != 0 && ts > UINT64_MAX / blocks) {
        err = "tensor " + name + " byte size overflow";
        return false;
    }
    *out = blocks * ts;
    return true;
}

bool gguf_parse(const uint8_t* data, size_t size, GgufFile& g, std::string& err) {
    g.data = data;
    g.size = size;
    Cur c{data, size};
    if (size < 8 || std::memcmp(data, "GGUF", 4) != 0) {
        err = "invalid GGUF magic";
        return false;
    }
    c.pos = 4;
    uint32_t ver = (uint32_t)c.u(4);
    if (ver < 2 || ver > 3) {
        err = "unsupported GGUF version " + std::to_string(ver);
        return false;
    }
    uint64_t nt = c.u(8), nm = c.u(8);
    for (uint64_t i = 0; i < nm && c.ok; i++) {
        std::string k = c.s();
        uint32_t vt = (uint32_t)c.u(4);
        GgufValue v;
        if (!skip_or_read(c, vt, v, 0)) {
            err = "malformed metadata value for key " + k;
            return false;
        }
        g.meta[k] = v;
    }
    if (!c.ok) {
        err = "truncated GGUF metadata";
        return false;
    }
    uint64_t align = 32;  // DEFAULT_ALIGNMENT (gguf.rs:10)
    auto a = g.meta.find("general.alignment");
    if (a != g.meta.end()) {
        if (a->second.type == 4 || a->second.type == 10) align = a->second.u;
        else if (a->second.type == 5) align = (uint64_t)a->second.i;
    }
    if (align == 0 || (align & (align - 1))) {
        err = "invalid GGUF alignment: " + std::to_string(align);
        return false;
    }
    g.alignment = align;
    struct Raw {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t type;
        uint64_t off;
    };
    std::vector<Raw> raws;
    for (uint64_t i = 0; i < nt && c.ok; i++) {
        Raw r;
        r.name = c.s();
        uint32_t nd = (uint32_t)c.u(4);
        if (!c.ok) break;
        if (nd == 0 || nd > 4) {
            err = "tensor " + r.name + " has invalid dimension count " + std::to_string(nd);
            return false;
        }
        for (uint32_t k = 0; k < nd; k++) r.dims.push_back(c.u(8));
        r.type = (uint32_t)c.u(4);
        r.off = c.u(8);
        raws.push_back(std::move(r));
    }
    if (!c.ok) {
        err = "truncated GGUF header";
        return false;
    }
    if (c.pos > UINT64_MAX - (align - 1) || ((c.pos + align - 1) & ~(align - 1)) > size) {
        err = "aligned tensor data start overflows file";
        return false;
    }
    const uint64_t start = (c.pos + align - 1) & ~(align - 1);
    g.data_start = start;
    std::set<std::string> seen;
    for (auto& r : raws) {
        if (!seen.insert(r.name).second) {
            err = "duplicate tensor name " + r.name;
            return false;
        }
        uint64_t nbytes;
        if (!gguf_tensor_nbytes(r.name, r.dims, r.type, &nbytes, err)) return false;
        if (r.off > UINT64_MAX - start) {
            err = "tensor " + r.name + " absolute offset overflow";
            return false;
        }
        g.tensors.push_back(GgufTensor{r.name, r.dims, r.type, start + r.off, nbytes});
    }
    return true;
}

// tensor_bytes (model.rs:1054-1079): the tensor's byte range must lie inside the image.
const uint8_t* GgufFile::bytes(const GgufTensor& t, std::string& err) const {
    if (t.offset > size || t.nbytes > size - t.offset) {
        err = "tensor " + t.name + " byte range " + std::to_string(t.offset) + ".." + std::to_string(t.offset + t.nbytes) +
              " exceeds mapped GGUF size " + std::to_string(size);
        return nullptr;
    }
    return data + t.offset;
}

const GgufTensor* GgufFile::find(const std::string& name) const {
    for (auto& t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

bool GgufFile::get_u32(const std::string& k, uint32_t* out) const {  // gguf.rs:230-237
    auto it = meta.find(k);
    if (it == meta.end()) return false;
    const GgufValue& v = it->second;
    if (v.type == 4) { *out = (uint32_t)v.u; return true; }
    if (v.type == 10 && v.u <= 0xffffffffull) { *out = (uint32_t)v.u; return true; }
    if (v.type == 5 && v.i >= 0) { *out = (uint32_t)v.i; return true; }
    return false;
}

bool GgufFile::get_f32(const std::string& k, float* out) const {  // gguf.rs:239-245
    auto it = meta.find(k);
    if (it == meta.end()) return false;
    if (it->second.type == 6 || it->second.type == 12) {
        *out = (float)it->second.f;
        return true;
    }
    return false;
}

std::string GgufFile::get_str(const std::string& k) const {
    auto it = meta.find(k);
    return (it == meta.end() || it->second.type != 8) ? std::string() : it->second.s;
}

// ---------------------------------------------------------------- tokenizer end-of-generation ids
// Tokenizer::from_gguf (src/tokenizer.rs:203-360), the parts that decide SpecialTokens::eog:
// the tokenizer model ("llama": SentencePiece ids, "gpt2": BPE), the token texts, and the
// special ids from metadata or their defaults (eos: 2 / "<|end_of_text|>", eot: "<|eot_id|>",
// Phi-3's "<|end|>"); every special id must lie inside the vocabulary (validate_token_id,
// :1180-1189).  A text lookup takes the last token with that text, as the reference's
// text -> id map is filled in id order.  The rest of the tokenizer (pre-tokenizer, scores,
// merges) is not read: text <-> id conversion stays with the caller.
bool gguf_stop_tokens(const GgufFile& g, std::vector<uint32_t>& out, std::string& err) {
    out.clear();
    auto mit = g.meta.find("tokenizer.ggml.model");
    if (mit == g.meta.end() || mit->second.type != 8) {
        err = "tokenizer.ggml.model missing";
        return false;
    }
    const std::string& model = mit->second.s;
    if (model != "llama" && model != "gpt2") {
        err = "unsupported tokenizer model: " + model;
        return false;
    }
    const bool spm = model == "llama";
    auto tit = g.meta.find("tokenizer.ggml.tokens");
    if (tit == g.meta.end() || tit->second.type != 9 || (tit->second.count > 0 && tit->second.item_type != 8)) {
        err = "tokenizer.ggml.tokens missing or invalid";
        return false;
    }
    const std::vector<std::string>& texts = tit->second.strs;
    if (texts.empty()) {
        err = "tokenizer.ggml.tokens must not be empty";
        return false;
    }
    const auto find_text = [&](const char* t, int64_t* id) {
        for (int64_t i = (int64_t)texts.size() - 1; i >= 0; i--)
            if (texts[i] == t) {
                *id = i;
                return true;
            }
        return false;
    };
    // (id or -1) from a metadata key, else a default
    const auto meta_id = [&](const char* key, int64_t dflt) {
        uint32_t v;
        return g.get_u32(key, &v) ? (int64_t)v : dflt;
    };
    int64_t tmp;
    const int64_t bos = meta_id("tokenizer.ggml.bos_token_id", spm ? 1 : (find_text("<|begin_of_text|>", &tmp) ? tmp : -1));
    const int64_t eos = meta_id("tokenizer.ggml.eos_token_id", spm ? 2 : (find_text("<|end_of_text|>", &tmp) ? tmp : -1));
    const int64_t unk = meta_id("tokenizer.ggml.unknown_token_id", spm ? 0 : -1);
    const int64_t eot = meta_id("tokenizer.ggml.eot_token_id", find_text("<|eot_id|>", &tmp) ? tmp : -1);
    const int64_t eom = meta_id("tokenizer.ggml.eom_token_id", -1);
    const int64_t phi_end = find_text("<|end|>", &tmp) ? tmp : -1;
    const int64_t sep = meta_id("tokenizer.ggml.separator_token_id", meta_id("tokenizer.ggml.seperator_token_id", -1));
    const int64_t pad = meta_id("tokenizer.ggml.padding_token_id", -1);
    const int64_t mask = meta_id("tokenizer.ggml.mask_token_id", -1);
    const std::pair<const char*, int64_t> special[] = {{"bos", bos}, {"eos", eos}, {"unk", unk},  {"eot", eot},
                                                       {"eom", eom}, {"sep", sep}, {"pad", pad}, {"mask", mask}};
    for (const auto& [name, id] : special)
        if (id >= (int64_t)texts.size()) {
            err = std::string(name) + " token id " + std::to_string(id) + " out of range for vocab size " +
                  std::to_string(texts.size());
            return false;
        }
    for (int64_t id : {eos, eot, eom, phi_end})
        if (id >= 0) out.push_back((uint32_t)id);
    std::sort(out.begin(), out.end());
    out.erase(std::unique(out.begin(), out.end()), out.end());
    return true;
}

// ---------------------------------------------------------------- Philox4x32-10
void philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    // Salmon et al., SC'11: multipliers 0xD2511F53 / 0xCD9E8D57, key bumps 0x9E3779B9 / 0xBB67AE85.
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

uint32_t philox_word(uint64_t seed, uint64_t ctr, uint32_t purpose) {
    const uint32_t c[4] = {(uint32_t)ctr, (uint32_t)(ctr >> 32), purpose, 0};
    const uint32_t k[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    philox4x32_10(c, k, o);
    return o[0];
}

float philox_uniform(uint64_t seed, uint64_t ctr, uint32_t purpose) {
    return (float)(philox_word(seed, ctr, purpose) >> 8) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------- synthetic writer
namespace {

uint16_t f32_to_f16_rne(float f) {
    // IEEE round-to-nearest-even binary32 -> binary16 (what llama.cpp's F16C path does).
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
    for (int i = 0; i < 4; i++) b.push_back((uint8_t)(v >> (8 * i)));
}
void put_u64(std::vector<uint8_t>& b, uint64_t v) {
    for (int i = 0; i < 8; i++) b.push_back((uint8_t)(v >> (8 * i)));
}
void put_str(std::vector<uint8_t>& b, const std::string& s) {
    put_u64(b, s.size());
    b.insert(b.end(), s.begin(), s.end());
}
void kv_str(std::vector<uint8_t>& b, const std::string& k, const std::string& v) {
    put_str(b, k);
    put_u32(b, 8);
    put_str(b, v);
}
void kv_u32(std::vector<uint8_t>& b, const std::string& k, uint32_t v) {
    put_str(b, k);
    put_u32(b, 4);
    put_u32(b, v);
}
void kv_f32(std::vector<uint8_t>& b, const std::string& k, float v) {
    put_str(b, k);
    put_u32(b, 6);
    uint32_t u;
    std::memcpy(&u, &v, 4);
    put_u32(b, u);
}

struct TSpec {
    std::string name;
    uint64_t cols, rows;  // rows == 1 for vectors
    uint32_t type;
    int kind;             // 0 = weight N(0, std), 1 = norm
    uint64_t offset = 0, bytes = 0;
};

std::vector<TSpec> synth_tensors(const nc_synth_spec& s) {
    const uint64_t d = s.embedding_length, F = s.feed_forward_length, V = s.vocab_size;
    const uint64_t hd = d / s.head_count, aw = s.head_count * hd, kw = s.head_count_kv * hd;
    const uint32_t wt = (uint32_t)s.weight_type;
    std::vector<TSpec> t;
    t.push_back({"token_embd.weight", d, V, wt, 0});
    t.push_back({"output_norm.weight", d, 1, 0, 1});
    if (!s.tied) t.push_back({"output.weight", d, V, NC_TYPE_Q4_0, 0});
    for (int i = 0; i < s.layers; i++) {
        const std::string b = "blk." + std::to_string(i) + ".";
        t.push_back({b + "attn_norm.weight", d, 1, 0, 1});
        t.push_back({b + "attn_q.weight", d, aw, wt, 0});
        t.push_back({b + "attn_k.weight", d, kw, wt, 0});
        t.push_back({b + "attn_v.weight", d, kw, wt, 0});
        t.push_back({b + "attn_output.weight", aw, d, wt, 0});
        t.push_back({b + "ffn_norm.weight", d, 1, 0, 1});
        t.push_back({b + "ffn_gate.weight", d, F, wt, 0});
        t.push_back({b + "ffn_up.weight", d, F, wt, 0});
        t.push_back({b + "ffn_down.weight", F, d, wt, 0});
    }
    for (auto& x : t) {
        uint64_t bs, ts;
        gguf_type_layout(x.type, &bs, &ts);
        x.bytes = x.cols * x.rows / bs * ts;
    }
    return t;
}

std::vector<uint8_t> synth_header(const nc_synth_spec& s, std::vector<TSpec>& ts, uint64_t* data_start) {
    std::vector<uint8_t> h = {'G', 'G', 'U', 'F'};
    put_u32(h, 3);
    put_u64(h, ts.size());
    const bool scaled = s.rope_scaling_factor > 0.0f;
    put_u64(h, scaled ? 17 : 13);
    kv_str(h, "general.architecture", "llama");
    kv_u32(h, "general.alignment", 32);
    kv_u32(h, "llama.context_length", (uint32_t)s.context_length);
    kv_u32(h, "llama.embedding_length", (uint32_t)s.embedding_length);
    kv_u32(h, "llama.block_count", (uint32_t)s.layers);
    kv_u32(h, "llama.feed_forward_length", (uint32_t)s.feed_forward_length);
    kv_u32(h, "llama.attention.head_count", (uint32_t)s.head_count);
    kv_u32(h, "llama.attention.head_count_kv", (uint32_t)s.head_count_kv);
    kv_f32(h, "llama.rope.freq_base", s.rope_freq_base);
    kv_f32(h, "llama.attention.layer_norm_rms_epsilon", s.rms_norm_epsilon);
    kv_u32(h, "llama.vocab_size", (uint32_t)s.vocab_size);
    kv_u32(h, "llama.rope.dimension_count", (uint32_t)(s.embedding_length / s.head_count));
    kv_str(h, "general.name", "nanocamelid-synthetic");
    if (scaled) {  // Llama-3 RoPE frequency scaling keys (read by rope_scaling_from_gguf, main.rs:8522-8535)
        kv_f32(h, "llama.rope.scaling.factor", s.rope_scaling_factor);
        kv_u32(h, "llama.rope.scaling.original_context_length", s.rope_scaling_original_context_length);
        kv_f32(h, "llama.rope.scaling.low_freq_factor", s.rope_scaling_low_freq_factor);
        kv_f32(h, "llama.rope.scaling.high_freq_factor", s.rope_scaling_high_freq_factor);
    }
    uint64_t off = 0;
    for (auto& t : ts) {
        put_str(h, t.name);
        const bool vec = t.rows == 1;
        put_u32(h, vec ? 1 : 2);
        put_u64(h, t.cols);
        if (!vec) put_u64(h, t.rows);
        put_u32(h, t.type);
        put_u64(h, off);
        t.offset = off;
        off += (t.bytes + 31) & ~31ull;
    }
    *data_start = (h.size() + 31) & ~31ull;
    return h;
}

constexpr uint32_t kPurposeWeight = 8, kPurposeNorm = 9;

// Two N(0,1) draws per Philox call (Box-Muller on two 53-bit uniforms) for elements
// 2j and 2j+1 of tensor `tid`.
inline void normal_pair(uint64_t seed, uint32_t tid, uint64_t j, uint32_t purpose, double* z0, double* z1) {
    const uint32_t c[4] = {(uint32_t)j, (uint32_t)(j >> 32), tid, purpose};
    const uint32_t k[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    philox4x32_10(c, k, o);
    const double u1 = ((double)(((uint64_t)(o[0] >> 5) << 26) | (o[1] >> 6)) + 1.0) * 0x1p-53;
    const double u2 = (double)(((uint64_t)(o[2] >> 5) << 26) | (o[3] >> 6)) * 0x1p-53;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double a = 6.283185307179586 * u2;
    *z0 = r * std::cos(a);
    *z1 = r * std::sin(a);
}

void gen_values(uint64_t seed, uint32_t tid, uint64_t start, uint64_t count, float stdv, float mean, uint32_t purpose,
                float* out) {
    // start and count are even (blocks of 32/256 values)
    for (uint64_t e = 0; e < count; e += 2) {
        double z0, z1;
        normal_pair(seed, tid, (start + e) / 2, purpose, &z0, &z1);
        out[e] = (float)(mean + stdv * z0);
        out[e + 1] = (float)(mean + stdv * z1);
    }
}

// llama.cpp quantize_row_q4_0_ref: d = max / -8 (max = signed value of largest |x|),
// q = min(15, (int8)(x/d + 8.5)), f16 scale rounded to nearest even.
void quant_q4_0_block(const float* x, uint8_t* out) {
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++)
        if (amax < std::fabs(x[j])) {
            amax = std::fabs(x[j]);
            mx = x[j];
        }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t h = f32_to_f16_rne(d);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 16; j++) {
        int q0 = (int)(int8_t)(x[j] * id + 8.5f), q1 = (int)(int8_t)(x[16 + j] * id + 8.5f);
        q0 = q0 > 15 ? 15 : q0;
        q1 = q1 > 15 ? 15 : q1;
        out[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

// llama.cpp quantize_row_q8_0_ref: d = max|x| / 127, q = round(x / d) (half away from zero),
// f16 scale rounded to nearest even.
void quant_q8_0_block(const float* x, uint8_t* out) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std::fmax(amax, std::fabs(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t h = f32_to_f16_rne(d);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; j++) out[2 + j] = (uint8_t)(int8_t)std::round(x[j] * id);
}

// A valid Q4_K encoding: per 32-sub-block affine [min, max] range, 6-bit scales/mins
// relative to f16 super-block factors d, dmin; packing as llama.cpp's get_scale_min_k4
// inverse.
void quant_q4_k_block(const float* x, uint8_t* out) {
    float scale[8], minv[8];
    float maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = 0.0f;
        for (int l = 0; l < 32; l++) {
            lo = std::fmin(lo, x[j * 32 + l]);
            hi = std::fmax(hi, x[j * 32 + l]);
        }
        scale[j] = (hi - lo) / 15.0f;
        minv[j] = -lo;
        maxs = std::fmax(maxs, scale[j]);
        maxm = std::fmax(maxm, minv[j]);
    }
    const uint16_t dh = f32_to_f16_rne(maxs / 63.0f), mh = f32_to_f16_rne(maxm / 63.0f);
    const float d = (float)__builtin_bit_cast(_Float16, dh), dmin = (float)__builtin_bit_cast(_Float16, mh);
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        int a = d > 0 ? (int)std::nearbyint(scale[j] / d) : 0;
        int b = dmin > 0 ? (int)std::nearbyint(minv[j] / dmin) : 0;
        ls[j] = (uint8_t)(a < 0 ? 0 : (a > 63 ? 63 : a));
        lm[j] = (uint8_t)(b < 0 ? 0 : (b > 63 ? 63 : b));
    }
    uint8_t* sc = out + 4;
    std::memset(sc, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = ls[j];
            sc[j + 4] = lm[j];
        } else {
            sc[j + 4] = (uint8_t)((ls[j] & 0x0f) | ((lm[j] & 0x0f) << 4));
            sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 0xff);
    out[3] = (uint8_t)(mh >> 8);
    uint8_t* qs = out + 16;
    std::memset(qs, 0, 128);
    for (int j = 0; j < 8; j++) {
        const float sj = d * (float)ls[j], mj = dmin * (float)lm[j];
        const int pair = j / 2, half = j % 2;
        for (int l = 0; l < 32; l++) {
            int q = sj > 0 ? (int)std::nearbyint((x[j * 32 + l] + mj) / sj) : 0;
            q = q < 0 ? 0 : (q > 15 ? 15 : q);
            qs[pair * 32 + l] |= (uint8_t)(half ? (q << 4) : q);
        }
    }
}

// A valid Q5_K encoding: the Q4_K scheme with 31 levels per sub-block; the fifth bit of the
// value of element 64*pair + 32*half + l goes to bit 2*pair + half of qh[l] (q8.rs:1380-1397).
void quant_q5_k_block(const float* x, uint8_t* out) {
    float scale[8], minv[8];
    float maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = 0.0f;
        for (int l = 0; l < 32; l++) {
            lo = std::fmin(lo, x[j * 32 + l]);
            hi = std::fmax(hi, x[j * 32 + l]);
        }
        scale[j] = (hi - lo) / 31.0f;
        minv[j] = -lo;
        maxs = std::fmax(maxs, scale[j]);
        maxm = std::fmax(maxm, minv[j]);
    }
    const uint16_t dh = f32_to_f16_rne(maxs / 63.0f), mh = f32_to_f16_rne(maxm / 63.0f);
    const float d = (float)__builtin_bit_cast(_Float16, dh), dmin = (float)__builtin_bit_cast(_Float16, mh);
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        int a = d > 0 ? (int)std::nearbyint(scale[j] / d) : 0;
        int b = dmin > 0 ? (int)std::nearbyint(minv[j] / dmin) : 0;
        ls[j] = (uint8_t)(a < 0 ? 0 : (a > 63 ? 63 : a));
        lm[j] = (uint8_t)(b < 0 ? 0 : (b > 63 ? 63 : b));
    }
    uint8_t* sc = out + 4;
    std::memset(sc, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = ls[j];
            sc[j + 4] = lm[j];
        } else {
            sc[j + 4] = (uint8_t)((ls[j] & 0x0f) | ((lm[j] & 0x0f) << 4));
            sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    out[2] = (uint8_t)(mh & 0xff);
    out[3] = (uint8_t)(mh >> 8);
    uint8_t* qh = out + 16;
    uint8_t* qs = out + 48;
    std::memset(qh, 0, 32);
    std::memset(qs, 0, 128);
    for (int j = 0; j < 8; j++) {
        const float sj = d * (float)ls[j], mj = dmin * (float)lm[j];
        const int pair = j / 2, half = j % 2;
        for (int l = 0; l < 32; l++) {
            int q = sj > 0 ? (int)std::nearbyint((x[j * 32 + l] + mj) / sj) : 0;
            q = q < 0 ? 0 : (q > 31 ? 31 : q);
            qs[pair * 32 + l] |= (uint8_t)(half ? ((q & 15) << 4) : (q & 15));
            if (q & 16) qh[l] |= (uint8_t)(1u << j);
        }
    }
}

}  // namespace

void synth_normal_values(uint64_t seed, uint32_t tid, uint64_t start, uint64_t count, uint32_t purpose, float* out) {
    // elements [start, start + count) of stream tid (start and count even): (float) z
    for (uint64_t e = 0; e < count; e += 2) {
        double z0, z1;
        normal_pair(seed, tid, (start + e) / 2, purpose, &z0, &z1);
        out[e] = (float)z0;
        out[e + 1] = (float)z1;
    }
}

int synth_size(const nc_synth_spec& s, uint64_t* size) {
    auto ts = synth_tensors(s);
    uint64_t start;
    synth_header(s, ts, &start);
    const auto& last = ts.back();
    *size = start + last.offset + last.bytes;
    return NC_OK;
}

int synth_write(const nc_synth_spec& s, uint8_t* dst, uint64_t size, int nthreads) {
    auto ts = synth_tensors(s);
    uint64_t start;
    auto hdr = synth_header(s, ts, &start);
    const auto& last = ts.back();
    if (size < start + last.offset + last.bytes) return fail(NC_EINVAL, "synth: destination too small");
    std::memset(dst, 0, start);
    std::memcpy(dst, hdr.data(), hdr.size());
    // Work items: (tensor, block range) chunks, processed by nthreads workers.
    struct Item {
        uint32_t tid;
        uint64_t b0, b1;
    };
    std::vector<Item> items;
    for (uint32_t tid = 0; tid < ts.size(); tid++) {
        const auto& t = ts[tid];
        uint64_t bs, tb;
        gguf_type_layout(t.type, &bs, &tb);
        const uint64_t nblk = t.cols * t.rows / (t.type == 0 ? 32 : bs);
        const uint64_t step = 1 << 14;
        for (uint64_t b = 0; b < nblk; b += step) items.push_back({tid, b, std::min(nblk, b + step)});
        // zero the alignment padding after the tensor
        uint8_t* tp = dst + start + t.offset;
        std::memset(tp + t.bytes, 0, ((t.bytes + 31) & ~31ull) - t.bytes);
    }
    std::atomic<size_t> next{0};
    auto worker = [&]() {
        std::vector<float> buf(256);
        for (;;) {
            const size_t i = next.fetch_add(1);
            if (i >= items.size()) break;
            const Item it = items[i];
            const TSpec& t = ts[it.tid];
            uint8_t* tp = dst + start + t.offset;
            if (t.type == 0) {  // f32 norm vector, 32 values per block
                float* o = (float*)tp;
                for (uint64_t b = it.b0; b < it.b1; b++) {
                    if (s.norm_mode == 0) {
                        for (int j = 0; j < 32; j++) o[b * 32 + j] = 1.0f;
                    } else {
                        gen_values(s.seed, it.tid, b * 32, 32, 0.1f, 1.0f, kPurposeNorm, o + b * 32);
                    }
                }
            } else if (t.type == NC_TYPE_Q4_0) {
                for (uint64_t b = it.b0; b < it.b1; b++) {
                    gen_values(s.seed, it.tid, b * 32, 32, s.weight_std, 0.0f, kPurposeWeight, buf.data());
                    quant_q4_0_block(buf.data(), tp + b * 18);
                }
            } else if (t.type == NC_TYPE_Q5_K) {
                for (uint64_t b = it.b0; b < it.b1; b++) {
                    gen_values(s.seed, it.tid, b * 256, 256, s.weight_std, 0.0f, kPurposeWeight, buf.data());
                    quant_q5_k_block(buf.data(), tp + b * 176);
                }
            } else if (t.type == NC_TYPE_Q8_0) {
                for (uint64_t b = it.b0; b < it.b1; b++) {
                    gen_values(s.seed, it.tid, b * 32, 32, s.weight_std, 0.0f, kPurposeWeight, buf.data());
                    quant_q8_0_block(buf.data(), tp + b * 34);
                }
            } else {
                for (uint64_t b = it.b0; b < it.b1; b++) {
                    gen_values(s.seed, it.tid, b * 256, 256, s.weight_std, 0.0f, kPurposeWeight, buf.data());
                    quant_q4_k_block(buf.data(), tp + b * 144);
                }
            }
        }
    };
    if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
    std::vector<std::thread> th;
    for (int i = 0; i < nthreads; i++) th.emplace_back(worker);
    for (auto& t : th) t.join();
    return NC_OK;
}

}  // namespace nc
