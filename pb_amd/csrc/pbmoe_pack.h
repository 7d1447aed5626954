// On-disk expert packs (layer_NN.bin + layer_NN.json) -- internal interface
// between the metadata reader (pbmoe_pack.cpp) and the C ABI.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace pbmoe {
namespace pack {

// Metadata format names (experts/mod.rs:46-52).
extern const char* const FORMAT_PBQ4_V1;
extern const char* const FORMAT_PBQ4_V2;
extern const char* const FORMAT_FIXED_Q4;
extern const char* const FORMAT_FIXED_MXFP4;
extern const char* const FORMAT_FIXED_DENSE;
extern const char* const FORMAT_FIXED_DEEPSEEK_GGUF;

// ExpertPackRecord (experts/mod.rs:440-454); scale_bias_dtype defaults to
// "F32" (default_expert_scale_bias_dtype, experts/mod.rs:936-938).
struct Record {
    std::string tensor, dtype, scale_bias_dtype;
    std::vector<uint64_t> shape;
    uint64_t record_offset = 0, packed_bytes = 0, groups = 0, group_size = 0;
};

// ExpertPackMetadata (experts/mod.rs:431-438); packed_bytes defaults to 0.
struct Pack {
    uint64_t layer = 0, expert = 0, packed_bytes = 0;
    std::vector<Record> records;
};

// ExpertLayerPackMetadata (experts/mod.rs:283-290).
struct LayerMeta {
    std::string format;
    uint64_t layer = 0, expert_size = 0, experts = 0;
    std::vector<Pack> packs;
    const Pack* pack_for(uint64_t expert) const;
};

// root/layer_NN.bin and root/layer_NN.json (experts/mod.rs:2478-2484).
std::string layer_bin_path(const std::string& root, uint32_t layer);
std::string layer_json_path(const std::string& root, uint32_t layer);

// Read, parse and validate root/layer_NN.json the way
// read_expert_layer_pack_metadata + ExpertLayerPackMetadata::validate do
// (experts/mod.rs:2501-2519, 372-429).  Returns 0 or a pbmoe_status code
// with the reason in *err.
int read_layer_meta(const std::string& root, uint32_t layer, LayerMeta* out, std::string* err);

// Size of a regular file, or -1 with errno set.
int64_t file_size(const std::string& path);

} // namespace pack
} // namespace pbmoe
