// mxh_gguf.h — GGUF v2/v3 reader (mmap, exact tensor names) and the seeded
// synthetic-model writer.  Host-only C++17; no HIP headers.
//
// Reference counterparts: third_party/gguf/gguf_reader.cpp:224-676 (open,
// metadata, tensor directory) and src/io/gguf_loader.cpp (role lookup).  The
// differences are deliberate: one mmap instead of a whole-file read per role
// group (gguf_loader.cpp:70-71), exact names instead of substring matches
// (gguf_reader.cpp:741-750), `attention.key_length` honoured, and Q5_K / F16
// accepted.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace mxh {

struct GgufTensor {
    std::string name;
    int type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
    const uint8_t* data = nullptr;
    size_t nbytes = 0;
    int64_t rows() const { return n_dims > 1 ? ne[1] : 1; }
    int64_t cols() const { return ne[0]; }
};

class GgufFile {
public:
    GgufFile() = default;
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;
    ~GgufFile();

    // Returns false with *err set on failure.
    bool open(const std::string& path, std::string* err);

    const GgufTensor* find(const std::string& name) const;
    // Numeric metadata `<arch>.<suffix>` (e.g. "attention.head_count"); def if absent.
    double arch_num(const std::string& suffix, double def) const;
    const std::string& arch() const { return arch_; }
    const std::vector<GgufTensor>& tensors() const { return tensors_; }
    const std::map<std::string, double>& nums() const { return nums_; }

private:
    void* map_ = nullptr;
    size_t size_ = 0;
    std::string arch_;
    std::map<std::string, double> nums_;
    std::map<std::string, std::string> strs_;
    std::vector<GgufTensor> tensors_;
    std::unordered_map<std::string, size_t> index_;
};

// Bytes of a [rows x cols] tensor of `type`; 0 when cols is not a whole number of blocks.
size_t tensor_bytes(int type, int64_t rows, int64_t cols);

// Architecture of a synthetic model (llama.cpp tensor names, `<arch>.*` keys).
struct SynthArch {
    const char* arch = "qwen3";
    int n_layer = 2, n_embd = 256, n_head = 4, n_head_kv = 2, head_dim = 64, n_ff = 512, n_vocab = 512;
    int ctx = 4096;
    float rope_theta = 1e6f, eps = 1e-6f;
    int qk_norm = 1, tied = 0;
    int wtype = 12, out_type = 8, embd_type = 8;
    int attn_v_type = -1, ffn_down_type = -1;  // per-role overrides (-1: wtype)
};

// Write a seeded synthetic GGUF: 2D weights N(0, 0.02) quantized to their
// type, norms F32 near 1.  Deterministic in `seed` whatever `threads` is.
bool write_synthetic_gguf(const std::string& path, const SynthArch& a, uint64_t seed, int threads, std::string* err);

// Row quantizers (affine min/max K-quants packed in the ggml scale layout,
// symmetric Q8_0); n is a whole number of blocks.
void quantize_row(int type, const float* x, int64_t n, uint8_t* out);

}  // namespace mxh
