// Config parsing and safetensors mapping (host only; built with g++ or hipcc).
// Key names and defaults follow the reference loader (src/laya.cpp:5-41) and HF's
// ModernBertConfig (rope_parameters.{full,sliding}_attention.rope_theta, layer_types or
// global_attn_every_n_layers).
#include "model.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>

#include "json_lite.h"

namespace laya {

static bool read_file(const std::string& path, std::string* out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[1 << 14];
  size_t n;
  out->clear();
  while ((n = fread(buf, 1, sizeof buf, f)) > 0) out->append(buf, n);
  fclose(f);
  return true;
}

bool Config::load(const std::string& encoder_cfg, const std::string& agent_cfg, std::string* err) {
  std::string s;
  if (!read_file(encoder_cfg, &s)) { if (err) *err = "cannot open " + encoder_cfg; return false; }
  try {
    JVal j = json_parse(s);
    n_layers = j.int_or("num_hidden_layers", 28);
    d = j.int_or("hidden_size", 1024);
    n_heads = j.int_or("num_attention_heads", 16);
    head_dim = d / n_heads;
    intermediate = j.int_or("intermediate_size", 2624);
    vocab = j.int_or("vocab_size", 50368);
    local_attention = j.int_or("local_attention", 128);
    norm_eps = (float)j.num_or("norm_eps", j.num_or("layer_norm_eps", 1e-5));
    pad_id = j.int_or("pad_token_id", 50283);
    cls_id = j.int_or("cls_token_id", 50281);
    sep_id = j.int_or("sep_token_id", 50282);
    mask_id = j.int_or("mask_token_id", 50284);
    sans_pos = j.str_or("position_embedding_type", "absolute") == "sans_pos";
    if (const JVal* rp = j.find("rope_parameters")) {
      if (const JVal* g = rp->find("full_attention")) rope_theta_global = (float)g->num_or("rope_theta", 160000.0);
      if (const JVal* l = rp->find("sliding_attention")) rope_theta_local = (float)l->num_or("rope_theta", 10000.0);
    } else {
      rope_theta_global = (float)j.num_or("global_rope_theta", 160000.0);
      rope_theta_local = (float)j.num_or("local_rope_theta", 10000.0);
    }
    global_layer.clear();
    if (const JVal* lt = j.find("layer_types"); lt && lt->kind == JVal::Arr) {
      for (auto& t : lt->arr) global_layer.push_back(t.str == "full_attention" ? 1 : 0);
    } else {
      int every = j.int_or("global_attn_every_n_layers", 3);
      for (int i = 0; i < n_layers; i++) global_layer.push_back(i % every == 0 ? 1 : 0);
    }
    if ((int)global_layer.size() != n_layers) { if (err) *err = "layer_types length != num_hidden_layers"; return false; }
  } catch (const std::exception& e) {
    if (err) *err = encoder_cfg + ": " + e.what();
    return false;
  }
  temperature.clear();
  temp_by_options.clear();
  if (read_file(agent_cfg, &s)) {
    try {
      JVal j = json_parse(s);
      max_len = j.int_or("max_len", 512);
      head_max_len = j.int_or("head_max_len", 192);
      head_layers = j.int_or("head_layers", 2);
      if (const JVal* a = j.find("act_costs"); a && a->kind == JVal::Arr) n_act = (int)a->arr.size() + 1;
      if (const JVal* t = j.find("temperature"); t && t->kind == JVal::Arr)
        for (auto& v : t->arr) temperature.push_back((float)v.num);
      if (const JVal* t = j.find("temperature_by_options"); t && t->kind == JVal::Obj)
        for (auto& kv : t->obj) temp_by_options[kv.first] = (float)kv.second.num;
    } catch (const std::exception& e) {
      if (err) *err = agent_cfg + ": " + e.what();
      return false;
    }
  }
  if (temperature.empty()) temperature = {1.f, 1.f, 1.f};
  head_ffn = 4 * d;
  return true;
}

std::string Config::describe() const {
  int ng = 0;
  for (auto g : global_layer) ng += g;
  std::ostringstream o;
  o << "[laya] layers=" << n_layers << " d=" << d << " heads=" << n_heads << " head_dim=" << head_dim
    << " ffn=" << intermediate << " vocab=" << vocab << " max_len=" << max_len << "\n"
    << "[laya] attn: " << ng << " global / " << (n_layers - ng) << " sliding (window=" << local_attention
    << ") rope theta g=" << rope_theta_global << " l=" << rope_theta_local << " eps=" << norm_eps << "\n"
    << "[laya] head: " << head_layers << " layers ffn=" << head_ffn << " n_act=" << n_act << "\n";
  return o.str();
}

SafeTensors::~SafeTensors() {
  if (base_ && base_ != MAP_FAILED) munmap(base_, size_);
  if (fd_ >= 0) close(fd_);
}

bool SafeTensors::open(const std::string& path, std::string* err) {
  fd_ = ::open(path.c_str(), O_RDONLY);
  if (fd_ < 0) { if (err) *err = "cannot open " + path; return false; }
  struct stat st;
  if (fstat(fd_, &st) != 0 || st.st_size < 8) { if (err) *err = "bad file " + path; return false; }
  size_ = (size_t)st.st_size;
  base_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (base_ == MAP_FAILED) { base_ = nullptr; if (err) *err = "mmap failed " + path; return false; }
  uint64_t hlen;
  memcpy(&hlen, base_, 8);
  if (hlen > size_ - 8) { if (err) *err = "bad safetensors header length"; return false; }
  const size_t data_off = 8 + hlen;
  try {
    JVal j = json_parse(std::string((const char*)base_ + 8, hlen));
    for (auto& kv : j.obj) {
      if (kv.first == "__metadata__") continue;
      TensorView t;
      t.dtype = kv.second["dtype"].str;
      for (auto& s : kv.second["shape"].arr) t.shape.push_back((int64_t)s.num);
      const JVal& off = kv.second["data_offsets"];
      size_t a = (size_t)off.arr.at(0).num, b = (size_t)off.arr.at(1).num;
      if (b < a || data_off + b > size_) { if (err) *err = "tensor " + kv.first + " out of file bounds"; return false; }
      size_t esz = t.dtype == "F32" ? 4 : (t.dtype == "BF16" || t.dtype == "F16") ? 2 : 0;
      if (!esz) { if (err) *err = "tensor " + kv.first + ": unsupported dtype " + t.dtype; return false; }
      if ((size_t)t.numel() * esz != b - a) { if (err) *err = "tensor " + kv.first + ": size mismatch"; return false; }
      t.nbytes = b - a;
      t.data = (const char*)base_ + data_off + a;
      tensors_[kv.first] = t;
    }
  } catch (const std::exception& e) {
    if (err) *err = path + ": " + e.what();
    return false;
  }
  return true;
}

const TensorView* SafeTensors::get(const std::string& name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

static float half_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF, u;
  if (e == 0) {
    if (m == 0) u = s;
    else { float f = std::ldexp((float)m, -24); memcpy(&u, &f, 4); u |= s; }
  } else if (e == 31) {
    u = s | 0x7F800000u | (m << 13);
  } else {
    u = s | ((e + 112) << 23) | (m << 13);
  }
  float f; memcpy(&f, &u, 4); return f;
}

void tensor_to_f32(const TensorView& t, float* out) {
  const int64_t n = t.numel();
  if (t.dtype == "F32") { memcpy(out, t.data, (size_t)n * 4); return; }
  const uint16_t* s = (const uint16_t*)t.data;
  if (t.dtype == "BF16") {
    for (int64_t i = 0; i < n; i++) { uint32_t u = (uint32_t)s[i] << 16; memcpy(&out[i], &u, 4); }
  } else {
    for (int64_t i = 0; i < n; i++) out[i] = half_to_f32(s[i]);
  }
}

}  // namespace laya
