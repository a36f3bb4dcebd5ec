// Reader for .rlm model files (the format tools/convert.py and tools/quantize.py write):
// "RLM1", a u32 version, a u64 header length, a JSON header (config, quant, sections,
// tensors), then page-aligned sections. Replaces src/model_file.{h,mm}: the file is mapped
// read-only and the tables give each tensor's absolute byte offsets in it; the engine
// (engine.hip) uploads and packs what it uses into device memory (a discrete GPU has to
// copy the weights anyway, so nothing here touches the GPU). Host code only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace rlq {

// The model configuration of the header (src/model_file.h:13-38), with the same defaults.
struct ModelConfig {
  int hidden = 0, layers = 0, intermediate = 0;
  int heads = 0, kv_heads = 0, head_dim = 0;
  int lin_v_heads = 0, lin_k_heads = 0, lin_k_dim = 0, lin_v_dim = 0, conv_taps = 0;
  int vocab = 0, full_attn_interval = 4, eos = -1;
  float norm_eps = 1e-6f;
  double rope_theta = 1e7;
  float partial_rotary = 0.25f;
  int group = 64, block = 256;
  bool native = false;     // scale-free 4-bit codebook weights instead of affine groups
  std::string book;        // native codebook: "fp4", "int15" or "int16"
  int rot_block = 0;       // residual stream rotated by signed Hadamard blocks (0: not rotated)
  int experts = 0, experts_per_tok = 0, moe_inter = 0;
  bool norm_topk = true;

  bool is_moe() const { return experts > 0; }
  int rope_dims() const { return (int)(head_dim * partial_rotary); }
};

// Tensor kinds of the file format (tools/convert.py:165-250, tools/quantize.py).
enum TensorKind { kKindQ4a = 1, kKindQ4n = 2, kKindQ4aRows = 3, kKindQ4nRows = 4, kKindF16b = 5, kKindF32 = 6 };

// A quantized or half-precision matrix [n][k] (src/model_file.h:40-55). Offsets are
// absolute byte offsets in the file: w codes (or halves), s scales, b biases (affine), c
// column scales (native). Blocked kinds (q4a, q4n, f16b) store rows in blocks of 256,
// padded to n_pad rows.
struct QTensor {
  int kind = 0, section = -1;
  uint64_t w = 0, s = 0, b = 0, c = 0;
  int k = 0, n = 0, n_pad = 0;
  bool blocked = true, native = false, dense = false;
  std::string book;                                      // q4n: the tensor's codebook when it names one
  std::vector<std::pair<std::string, std::pair<int, int>>> parts;   // name -> (first row, rows), file order

  const std::pair<int, int> *part(const std::string &name) const;
};

struct FTensor {
  int section = -1;
  uint64_t offset = 0;
  std::vector<int> shape;
  size_t count() const;
};

struct Section {
  std::string name;
  uint64_t offset = 0, nbytes = 0;
};

class ModelFile {
 public:
  // Maps and parses the file. Returns 0, or fails (fatal by default) with the reference's
  // messages: not a model file, invalid JSON, a missing header field, an unsupported mixture
  // of experts or rotation, a section past the end of the file; and, beyond the reference, a
  // header past the end, a tensor naming a missing section or reaching past the file.
  static int open(const std::string &path, std::unique_ptr<ModelFile> &out);
  ~ModelFile();
  ModelFile(const ModelFile &) = delete;
  ModelFile &operator=(const ModelFile &) = delete;

  const ModelConfig &config() const { return cfg_; }
  const QTensor *q(const std::string &name) const;      // nullptr when absent
  const FTensor *f(const std::string &name) const;
  bool has(const std::string &name) const { return q_.count(name) || f_.count(name); }
  const uint8_t *data() const { return base_; }
  size_t file_bytes() const { return size_; }
  const std::vector<Section> &sections() const { return sections_; }
  const std::map<std::string, QTensor> &qtensors() const { return q_; }
  const std::map<std::string, FTensor> &ftensors() const { return f_; }
  uint32_t version() const { return version_; }
  const std::string &path() const { return path_; }

 private:
  ModelFile() = default;
  int parse(const std::string &path);

  std::string path_;
  const uint8_t *base_ = nullptr;
  size_t size_ = 0;
  uint32_t version_ = 0;
  ModelConfig cfg_;
  std::vector<Section> sections_;
  std::map<std::string, QTensor> q_;
  std::map<std::string, FTensor> f_;
};

// The page the writer aligns sections to (tools/convert.py:30).
constexpr uint64_t kRlmPage = 16384;

}  // namespace rlq
