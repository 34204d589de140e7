// GGUF reader/writer and Philox helpers (host side of libnanocamelid_hip).
#pragma once

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "nc_internal.h"

namespace nc {

struct GgufValue {
    int type = -1;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    // arrays (type 9): the item type and count; the items themselves only for strings
    int item_type = -1;
    uint64_t count = 0;
    std::vector<std::string> strs;
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;  // dims[0] = columns (contiguous), dims[1] = rows
    uint32_t type = 0;
    uint64_t offset = 0;  // absolute byte offset in the image
    uint64_t nbytes = 0;
};

struct GgufFile {
    const uint8_t* data = nullptr;
    size_t size = 0;
    uint64_t alignment = 32, data_start = 0;
    std::map<std::string, GgufValue> meta;
    std::vector<GgufTensor> tensors;
    const GgufTensor* find(const std::string& name) const;
    // the tensor's bytes, or null (err set) when its range does not lie inside the image
    const uint8_t* bytes(const GgufTensor& t, std::string& err) const;
    bool get_u32(const std::string& k, uint32_t* out) const;
    bool get_f32(const std::string& k, float* out) const;
    std::string get_str(const std::string& k) const;
};

bool gguf_type_layout(uint32_t type, uint64_t* block, uint64_t* bytes);
bool gguf_tensor_nbytes(const std::string& name, const std::vector<uint64_t>& dims, uint32_t type, uint64_t* out,
                        std::string& err);
bool gguf_parse(const uint8_t* data, size_t size, GgufFile& out, std::string& err);

// SpecialTokens::eog of the file's tokenizer (src/tokenizer.rs:203-323): sorted, distinct ids.
bool gguf_stop_tokens(const GgufFile& g, std::vector<uint32_t>& out, std::string& err);

// Tensor bytes -> f32 as the reference's load_f32_or_f16 (dequant.cpp); n values.
bool dequant_supported(uint32_t type);
int dequant_f32(uint32_t type, const uint8_t* src, uint64_t n, float* out, int nthreads);

void philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint32_t philox_word(uint64_t seed, uint64_t ctr, uint32_t purpose);
float philox_uniform(uint64_t seed, uint64_t ctr, uint32_t purpose);

// Philox purposes (counter word 2) shared by the drafter, prompts and sampling.
constexpr uint32_t kPurposeDraft = 1, kPurposeAccept = 2, kPurposeResample = 3, kPurposePrompt = 4;
constexpr uint32_t kPurposeOracleU = 5, kPurposeOracleId = 6, kPurposeBonus = 7;

// N(0, 1) values (Philox4x32-10 counter (pair index, stream tid, purpose), Box-Muller in double,
// rounded to f32) of elements [start, start + count) of stream tid; start and count even.
constexpr uint32_t kPurposeKvFill = 10;
void synth_normal_values(uint64_t seed, uint32_t tid, uint64_t start, uint64_t count, uint32_t purpose, float* out);

int synth_size(const nc_synth_spec& s, uint64_t* size);
int synth_write(const nc_synth_spec& s, uint8_t* dst, uint64_t size, int nthreads);

}  // namespace nc
