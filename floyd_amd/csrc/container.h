// container.h -- reader of the Moonlight container (config.json + *.safetensors)
// that tools/convert_moonlight.py writes (internal).
//
// Behaviour follows floyd's moonlight_model.c:41-190 and st.h:114-168: the
// config fields and defaults of read_config, every *.safetensors file of the
// directory in sorted order, tensors addressed by name (first occurrence
// wins), raw bytes read with pread.
#pragma once

#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace mlh {

// dtype codes of moonlight_model.h:10-15 (plus st.h's extra codes).
enum TensorDtype {
    kDtypeBF16 = 0, kDtypeF16 = 1, kDtypeF32 = 2, kDtypeU8 = 3, kDtypeI64 = 4,
    kDtypeF8E8M0 = 5, kDtypeF8E4M3 = 6
};

struct ModelConfig {
    int hidden_size = 0, layer_count = 0, head_count = 0, expert_count = 0;
    int experts_per_token = 0, dense_intermediate_size = 0, moe_intermediate_size = 0;
    int first_dense_layer_count = 0, q_lora_rank = 0, kv_lora_rank = 0;
    int qk_nope_dim = 0, qk_rope_dim = 0, value_dim = 0, shared_expert_count = 0;
    int normalize_topk = 1, vocab_size = 0;
    float rms_norm_epsilon = 1e-5f, rope_theta = 10000.0f, routed_scale = 1.0f;
};

struct TensorEntry {
    std::string name;
    int dtype = 0;
    int64_t numel = 0;
    int64_t nbytes = 0;
    int file = -1;        // index into Container::files
    int64_t offset = 0;   // absolute byte offset in the file
};

class Container {
public:
    ~Container();
    // Parses config.json and every shard header; false + message on failure.
    bool open(const std::string &dir, std::string *error);
    const ModelConfig &config() const { return config_; }
    const std::vector<TensorEntry> &tensors() const { return tensors_; }
    int find(const std::string &name) const;
    uint64_t total_bytes() const { return total_bytes_; }
    // Reads the raw bytes of tensor `index` into dst (nbytes of it).
    bool read(int index, void *dst, size_t capacity) const;
    // Reads bytes [offset, offset + n) of tensor `index` into dst.
    bool read_slice(int index, int64_t offset, size_t n, void *dst) const;

private:
    ModelConfig config_;
    std::vector<TensorEntry> tensors_;
    std::unordered_map<std::string, int> index_;
    std::vector<int> fds_;
    uint64_t total_bytes_ = 0;
};

// Config parsing on its own (used by open(); exposed for tests).
bool parse_config_json(const std::string &text, ModelConfig *config, std::string *error);

}  // namespace mlh
