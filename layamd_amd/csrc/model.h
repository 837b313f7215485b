// Laya checkpoint contract: config parsing and a zero-copy safetensors view (host only).
// Mirrors the reference's loader semantics (src/laya.cpp:5-75, src/laya.hpp:19-48): the same
// JSON keys and defaults, the same tensor names, F32/BF16/F16 tensors.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace laya {

struct Config {
  int n_layers = 28, d = 1024, n_heads = 16, head_dim = 64, intermediate = 2624;
  int vocab = 50368, max_len = 512, head_max_len = 192, head_layers = 2, n_act = 2;
  int local_attention = 128;            // full window width; each side sees local_attention/2
  float norm_eps = 1e-5f;
  float rope_theta_global = 160000.f, rope_theta_local = 10000.f;
  int pad_id = 50283, cls_id = 50281, sep_id = 50282, mask_id = 50284;
  std::vector<uint8_t> global_layer;    // 1 = full attention, 0 = sliding window
  std::vector<float> temperature;       // per qtype
  std::map<std::string, float> temp_by_options;   // parsed for completeness; applied by callers
  int head_ffn = 0;                     // 4 * d
  bool sans_pos = false;

  // Reads <dir>/encoder/config.json (required) and <dir>/rl_agent_config.json (optional).
  bool load(const std::string& encoder_cfg, const std::string& agent_cfg, std::string* err);
  std::string describe() const;
};

struct TensorView {
  const void* data = nullptr;
  std::vector<int64_t> shape;
  std::string dtype;                    // "F32" | "BF16" | "F16"
  size_t nbytes = 0;
  int64_t numel() const { int64_t n = 1; for (auto s : shape) n *= s; return n; }
};

// Memory-maps a .safetensors file; tensors are views into the mapping.
class SafeTensors {
 public:
  ~SafeTensors();
  bool open(const std::string& path, std::string* err);
  const TensorView* get(const std::string& name) const;
  const std::map<std::string, TensorView>& all() const { return tensors_; }
 private:
  int fd_ = -1; void* base_ = nullptr; size_t size_ = 0;
  std::map<std::string, TensorView> tensors_;
};

// Element conversion of a tensor view to float (F32/BF16/F16 sources).
void tensor_to_f32(const TensorView& t, float* out);

}  // namespace laya
