// Host-only entry points over the engine's C++ packer and checkpoint loader, built with g++ into
// liblaya_host.so so the CPU test suite can check them without a GPU.  Not part of laya_api.h.
#include <cstring>
#include <string>
#include <vector>

#include "model.h"
#include "pack.h"

using namespace laya;

extern "C" {

// Plans a laya_forward_batch call.  Returns -1 on invalid input, else the number of passes.
// For pass `which` it fills (when the pointers are non-null and large enough):
//   dims[10] = first, B, T, valid, KT, R, ntiles, ngtiles, len(gq), ngltiles
//   rows[3*T] = ids | pos | seq; seqs[5*B+1] = soff(B+1) | vlen | qt | nm | moff
//   tiles[4*ntiles] (sliding-window query tiles of <= q_tile), gltiles[4*ngltiles] (global query
//   tiles of <= q_tile_global), gtiles[4*ngtiles], gq[len], grow[R]
int laya_host_plan(int B, const int* lens, const int* ids, const int* nmark, const int* markers, const int* qtypes,
                   int max_len, int pass_tokens, int max_seqs, int max_grows, int vocab, int pad_id, int q_tile,
                   int q_tile_global, int which, int* dims,
                   int* rows, int* seqs, int* tiles, int* gltiles, int* gtiles, int* gq, int* grow) {
  PackLimits lim;
  lim.max_len = max_len; lim.pass_tokens = pass_tokens; lim.max_seqs = max_seqs; lim.max_grows = max_grows;
  lim.vocab = vocab;
  lim.pad_id = pad_id;
  lim.q_tile = q_tile;
  lim.q_tile_global = q_tile_global;
  std::vector<PassPlan> ps;
  if (plan_passes(B, lens, ids, nmark, markers, qtypes, lim, &ps) != 0) return -1;
  if (which >= 0 && which < (int)ps.size()) {
    const PassPlan& p = ps[which];
    if (dims) {
      int d[10] = {p.first, p.B, p.T, p.valid, p.KT, p.R, (int)p.tiles.size(), (int)p.gtiles.size(), (int)p.gq.size(),
                   (int)p.gltiles.size()};
      memcpy(dims, d, sizeof d);
    }
    if (rows) {
      memcpy(rows, p.ids.data(), p.T * 4); memcpy(rows + p.T, p.pos.data(), p.T * 4);
      memcpy(rows + 2 * p.T, p.seq.data(), p.T * 4);
    }
    if (seqs) {
      int* s = seqs;
      memcpy(s, p.soff.data(), (p.B + 1) * 4); s += p.B + 1;
      memcpy(s, p.vlen.data(), p.B * 4); s += p.B;
      memcpy(s, p.qt.data(), p.B * 4); s += p.B;
      memcpy(s, p.nm.data(), p.B * 4); s += p.B;
      memcpy(s, p.moff.data(), p.B * 4);
    }
    if (tiles) memcpy(tiles, p.tiles.data(), p.tiles.size() * sizeof(AttnTile));
    if (gltiles) memcpy(gltiles, p.gltiles.data(), p.gltiles.size() * sizeof(AttnTile));
    if (gtiles) memcpy(gtiles, p.gtiles.data(), p.gtiles.size() * sizeof(AttnTile));
    if (gq) memcpy(gq, p.gq.data(), p.gq.size() * 4);
    if (grow) memcpy(grow, p.grow.data(), p.R * 4);
  }
  return (int)ps.size();
}

// Parses <dir>'s configs.  out[16] = n_layers, d, n_heads, head_dim, intermediate, vocab, max_len,
// head_max_len, head_layers, n_act, local_attention, pad, cls, sep, mask, number of global layers;
// fout[6] = eps, theta_global, theta_local, temperature[0..2].  Returns 0, or -1 with err filled.
int laya_host_config(const char* dir, int* out, float* fout, char* err, int err_len) {
  Config c;
  std::string e;
  if (!c.load(std::string(dir) + "/encoder/config.json", std::string(dir) + "/rl_agent_config.json", &e)) {
    if (err && err_len > 0) { strncpy(err, e.c_str(), err_len - 1); err[err_len - 1] = 0; }
    return -1;
  }
  int ng = 0;
  for (auto g : c.global_layer) ng += g;
  int v[16] = {c.n_layers, c.d, c.n_heads, c.head_dim, c.intermediate, c.vocab, c.max_len, c.head_max_len,
               c.head_layers, c.n_act, c.local_attention, c.pad_id, c.cls_id, c.sep_id, c.mask_id, ng};
  memcpy(out, v, sizeof v);
  float f[6] = {c.norm_eps, c.rope_theta_global, c.rope_theta_local, c.temperature[0], c.temperature[1],
                c.temperature[2]};
  memcpy(fout, f, sizeof f);
  return 0;
}

// Global-attention flag of layer i (after laya_host_config succeeded on the same dir), -1 if out of range.
int laya_host_layer_is_global(const char* dir, int i) {
  Config c;
  std::string e;
  if (!c.load(std::string(dir) + "/encoder/config.json", std::string(dir) + "/rl_agent_config.json", &e)) return -1;
  return i >= 0 && i < (int)c.global_layer.size() ? c.global_layer[i] : -1;
}

// Reads tensor `name` of a safetensors file as float32 into out (numel values).  Returns numel,
// or -1 (missing tensor / bad file); shape (up to 8 dims) goes to shape_out, ndim to *ndim.
long long laya_host_read_tensor(const char* path, const char* name, float* out, long long cap, long long* shape_out,
                                int* ndim) {
  SafeTensors st;
  std::string e;
  if (!st.open(path, &e)) return -1;
  const TensorView* t = st.get(name);
  if (!t) return -1;
  if (ndim) *ndim = (int)t->shape.size();
  if (shape_out) for (size_t i = 0; i < t->shape.size() && i < 8; i++) shape_out[i] = t->shape[i];
  if (out && t->numel() <= cap) tensor_to_f32(*t, out);
  return t->numel();
}
}

// ---------------------------------------------------------------- counter-based normal draws
// The weight/workload generator of layamd_amd/rng.py, in C++ (same definition, multithreaded):
//   z = splitmix64_mix(key + (i + 1) * 0x9E3779B97F4A7C15)
//   u1 = ((z >> 32) + 0.5) * 2^-32, u2 = ((z & 0xffffffff) + 0.5) * 2^-32
//   out[i - start] = (float)(sqrt(-2 ln u1) * cos(2 pi u2) * std)
#include <cmath>
#include <thread>

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

extern "C" void laya_host_normal(uint64_t key, long long start, long long n, double stdv, float* out, int threads) {
  const double two32 = 1.0 / 4294967296.0, two_pi = 6.283185307179586;
  auto work = [&](long long a, long long b) {
    for (long long i = a; i < b; i++) {
      const uint64_t z = mix64(key + (uint64_t)(start + i + 1) * 0x9E3779B97F4A7C15ull);
      const double u1 = ((double)(z >> 32) + 0.5) * two32, u2 = ((double)(z & 0xFFFFFFFFull) + 0.5) * two32;
      out[i] = (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2) * stdv);
    }
  };
  if (threads < 1) threads = 1;
  if (n < (1 << 16)) threads = 1;
  std::vector<std::thread> th;
  for (int t = 0; t < threads; t++) th.emplace_back(work, n * t / threads, n * (t + 1) / threads);
  for (auto& x : th) x.join();
}

extern "C" void laya_host_u64(uint64_t key, long long start, long long n, uint64_t* out) {
  for (long long i = 0; i < n; i++) out[i] = mix64(key + (uint64_t)(start + i + 1) * 0x9E3779B97F4A7C15ull);
}
