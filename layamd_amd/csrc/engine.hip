// Laya engine for AMD Instinct MI355X (gfx950): weight upload, pass execution, HIP graphs and the
// laya_api.h C ABI.
//
// One pass runs a whole batch of questions packed densely (see pack.h), on one stream:
//
//   embeddings -> LN                                   k_layernorm (gather by token id)
//   per encoder layer:
//     QKV GEMM + RoPE + V^T write                      k_gemm_xl<EPI_QKV>
//     attention (global | sliding +-64)                k_attention_bf16
//     out-proj GEMM, x += (fp32 residual)               k_gemm_xl<EPI_RESID>
//     LN -> xn                                         k_layernorm
//     Wi GEMM + GeGLU                                  k_gemm_xl<EPI_GEGLU>
//     Wo GEMM, x +=                                    k_gemm_xl<EPI_RESID>
//     LN -> xn (next attn_norm) | final LN + type embedding into x
//   head layer 0 (all rows), head layer 1 on the gathered marker + CLS rows, scorer, act head.
// (bf16 names; the fp32 engine runs k_gemm and k_attention<float>.)  The GEMM tile shapes of a
// pass are timed before its first run (tune_pass) and the pass is then captured in a HIP graph.
//
// Semantics follow the reference's Engine::run / forward_batch (src/engine.hip:396-539) and the
// upstream model it serves (ref/rl_common.py:100-124); the kernels, data layout and fusion are
// this engine's own (weights keep their [out, in] layout; RoPE, the V transpose and GeGLU are
// GEMM epilogues; the residual add happens in the GEMM epilogue in fp32).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "common.h"
#include "kernels.h"
#include "laya_api.h"
#include "laya_ext.h"
#include "model.h"
#include "pack.h"

namespace laya {

static int env_int(const char* n, int d) { const char* s = getenv(n); return s && *s ? atoi(s) : d; }

// ---------------------------------------------------------------- profiling
thread_local LaunchTimer* g_launch_timer = nullptr;

// Per-stage device time, as the reference's stage profiler reports it (src/engine.hip:35-47), but
// measured per kernel: between begin() and end() this is the calling thread's LaunchTimer, so each
// of the stage's launches records its own start and end into an event pair from the pool.  Nothing
// waits during the pass; collect() (after the stream has been synchronized) reads the pairs and
// adds each kernel's duration to its stage.
struct Prof : LaunchTimer {
  bool on = false;
  std::vector<std::tuple<std::string, double, long long>> acc;   // stage, ms, stage executions
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pool;
  std::vector<std::pair<size_t, size_t>> pending;                  // (acc index, pool index)
  std::vector<int> seq;                                            // stage of each launch of the last pass
  size_t cur = 0;
  void init() {
    const char* p = getenv("LAYA_PROFILE");
    on = p != nullptr && *p && strcmp(p, "0") != 0;
  }
  void events(hipEvent_t* a, hipEvent_t* b) override {
    const size_t i = pending.size();
    if (i == pool.size()) {
      hipEvent_t x, y;
      LAYA_HIP(hipEventCreate(&x));
      LAYA_HIP(hipEventCreate(&y));
      pool.emplace_back(x, y);
    }
    pending.emplace_back(cur, i);
    seq.push_back((int)cur);
    *a = pool[i].first;
    *b = pool[i].second;
  }
  void begin(const char* name) {
    if (!on) return;
    size_t i = 0;
    while (i < acc.size() && std::get<0>(acc[i]) != name) i++;
    if (i == acc.size()) acc.emplace_back(name, 0.0, 0LL);
    std::get<2>(acc[i]) += 1;
    cur = i;
    g_launch_timer = this;
  }
  void end() { g_launch_timer = nullptr; }
  // after the stream has finished every pending launch
  void collect() {
    for (const auto& pr : pending) {
      float ms = 0.f;
      LAYA_HIP(hipEventElapsedTime(&ms, pool[pr.second].first, pool[pr.second].second));
      std::get<1>(acc[pr.first]) += ms;
    }
    pending.clear();
  }
  void report(int iters) {
    if (acc.empty()) { printf("[laya] profile is empty (set LAYA_PROFILE or call laya_ext_prof_enable)\n"); return; }
    if (iters < 1) iters = 1;
    double tot = 0;
    for (auto& e : acc) tot += std::get<1>(e);
    auto v = acc;
    std::sort(v.begin(), v.end(), [](auto& x, auto& y) { return std::get<1>(x) > std::get<1>(y); });
    printf("\n%-28s %10s %8s %7s\n", "stage", "ms/fwd", "calls", "%");
    for (auto& e : v)
      printf("%-28s %10.4f %8lld %6.1f%%\n", std::get<0>(e).c_str(), std::get<1>(e) / iters, std::get<2>(e),
             100.0 * std::get<1>(e) / tot);
    printf("%-28s %10.4f (serialized sum of kernel time)\n", "TOTAL", tot / iters);
  }
};

// ---------------------------------------------------------------- engine interface
struct EngineIface {
  Config cfg;
  Prof prof;
  virtual ~EngineIface() {}
  virtual int forward_batch(int B, const int* lens, const int* ids, const int* nmark, const int* markers,
                            const int* qtypes, float* logits, float* act) = 0;
  virtual int replay(int iters, float* ms) = 0;
  virtual void warmup() = 0;
  virtual void tune_all() = 0;
  virtual const char* precision() const = 0;
  // graphs cached, graphs captured so far, tuned GEMM plans, pass buckets tuned
  virtual void stats(long long* out) const = 0;
};

template <typename T>
struct Engine : EngineIface {
  // With the LayerNorm fold (bf16 engine), the weights read after a LayerNorm hold its weight
  // already (rows W[n] * w) and the c_* arrays their row sums; a LayerNorm bias b is in the
  // following GEMM's bias (bias + W . b).
  struct EncLayer {
    float* attn_norm = nullptr; T* Wqkv; T* Wo; float* mlp_norm; T* Wi; T* Wmo;
    float* c_qkv = nullptr; float* c_wi = nullptr;
  };
  struct HeadLayer {
    float *n1w, *n1b, *n2w, *n2b, *inB, *outB, *l1B, *l2B; T *inW, *outW, *l1W, *l2W;
    float* c_in = nullptr; float* c_l1 = nullptr;
  };

  hipStream_t stream = nullptr;
  PackLimits lim;
  PassCaps caps{};
  bool use_graphs = true, capturing = false, verbose = false;
  std::string dump_dir;                       // LAYA_DUMP_DIR at laya_create (empty: no dumps)

  // weights
  float* tok_emb = nullptr;            // fp32 in both engines, as the reference's embedding output is
  float *emb_norm = nullptr, *final_norm = nullptr, *type_emb = nullptr;
  std::vector<EncLayer> enc;
  std::vector<HeadLayer> head;
  float *sc0w, *sc0b, *sc1b, *sc3w, *sc3b;
  T* sc1W;
  float *ah0W, *ah0b, *ah2W, *ah2b;
  float *cos_g, *sin_g, *cos_l, *sin_l;

  // activations
  int64_t MT = 0, RG = 0, VTC = 0;   // rows, gathered rows, V^T columns (rows + one key block)
  float *x = nullptr, *xg = nullptr, *d_logits = nullptr, *d_act = nullptr, *d_act_hidden = nullptr;
  T *xn, *q, *k, *vt, *ao, *mg, *ff, *aog, *xng, *sh;

  // per-pass index arrays: one device block and its pinned host mirror, laid out per pass shape
  // (so a captured graph's addresses hold for every replay of that shape) and uploaded by one copy
  int *d_ids, *d_pos, *d_seq, *d_soff, *d_vlen, *d_qt, *d_nm, *d_moff, *d_gq, *d_grow;
  int *h_ids, *h_pos, *h_seq, *h_soff, *h_vlen, *h_qt, *h_nm, *h_moff, *h_gq, *h_grow;
  AttnTile *d_tiles, *d_gltiles, *d_gtiles, *h_tiles, *h_gltiles, *h_gtiles;
  char *d_blob = nullptr, *h_blob = nullptr;
  size_t blob_cap = 0;
  float *h_logits, *h_act;

  // A pass bucket: rows (a multiple of kRowBucket), questions, marker rows (a multiple of
  // kMarkerBucket).  Everything a pass launches and every index array's size follow from it: the
  // gathered rows R = KT + B and the attention grids (the tile capacities of pack.h).
  struct Shape {
    int rows, B, KT;
    int R() const { return KT + B; }
    int nt() const { return tiles_cap(rows, B); }
    int ngt() const { return gtiles_cap(R(), B); }
    bool operator<(const Shape& o) const { return std::tie(rows, B, KT) < std::tie(o.rows, o.B, o.KT); }
  };
  std::map<Shape, hipGraphExec_t> graphs;
  size_t max_graphs = 512;                // the reference's cache limit (src/engine.hip:477)
  long long n_captures = 0;               // graphs captured so far (cache misses that were captured)
  bool have_last = false;
  Shape last{};

  // measured bf16 tile configuration per (epilogue, activation, N, K, RoPE, M bucket), filled before
  // the first pass of a shape (or by tune_all); every configuration gives bit-identical results
  using TuneKey = std::tuple<int, int, int, int, int, int, int>;
  // a tuned launch: tile configuration, and optionally the first `split_tiles` tile rows in it and
  // the remaining rows in a second launch with configuration `tail`
  struct TilePlan { int cfg = -1, split_tiles = 0, tail = -1; };
  std::map<TuneKey, TilePlan> tuned;
  int n_cu = 256;
  std::set<Shape> tuned_shapes;
  bool tune_on = true;
  // LAYA_GEMM_CFG / LAYA_GEMM_SPLIT, read at laya_create: one tile configuration (and row split)
  // for every bf16 GEMM of this engine instead of the tuned plans
  int pin_cfg = -1, pin_split = 0, pin_tail = -1;
  std::vector<std::pair<int, GemmArgs>>* collecting = nullptr;   // set while a pass's GEMMs are listed

  const char* precision() const override { return sizeof(T) == 2 ? "bf16" : "fp32"; }
  void stats(long long* out) const override {
    out[0] = (long long)graphs.size(); out[1] = n_captures; out[2] = (long long)tuned.size();
    out[3] = (long long)tuned_shapes.size();
  }

  // ------------------------------------------------------------ allocation helpers
  template <typename U> U* dalloc(size_t n, bool zero = false) {
    U* p = nullptr;
    LAYA_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(U)));
    if (zero) LAYA_HIP(hipMemset(p, 0, std::max<size_t>(n, 1) * sizeof(U)));
    return p;
  }
  template <typename U> U* halloc(size_t n) {
    U* p = nullptr;
    LAYA_HIP(hipHostMalloc(&p, std::max<size_t>(n, 1) * sizeof(U), hipHostMallocDefault));
    return p;
  }

  static const TensorView& must(const SafeTensors& st, const std::string& n) {
    const TensorView* t = st.get(n);
    if (!t) { fprintf(stderr, "[laya] missing tensor %s\n", n.c_str()); exit(1); }
    return *t;
  }
  static void check_shape(const TensorView& t, std::vector<int64_t> s, const std::string& n) {
    if (t.shape != s) {
      fprintf(stderr, "[laya] tensor %s has an unexpected shape\n", n.c_str());
      exit(1);
    }
  }
  static std::vector<float> host_f32(const TensorView& t) {
    std::vector<float> v((size_t)t.numel());
    tensor_to_f32(t, v.data());
    return v;
  }
  float* up_f32(const SafeTensors& st, const std::string& n, std::vector<int64_t> shape) {
    const TensorView& t = must(st, n);
    check_shape(t, shape, n);
    std::vector<float> v = host_f32(t);
    float* d = dalloc<float>(v.size());
    LAYA_HIP(hipMemcpy(d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return d;
  }
  // matrix [rows, cols] with stored row i taken from source row perm[i] (identity when empty)
  T* up_mat(const SafeTensors& st, const std::string& n, int64_t rows, int64_t cols, const std::vector<int>& perm = {}) {
    const TensorView& t = must(st, n);
    check_shape(t, {rows, cols}, n);
    std::vector<float> v = host_f32(t);
    std::vector<T> o((size_t)(rows * cols));
    auto work = [&](int64_t r0, int64_t r1) {
      for (int64_t r = r0; r < r1; r++) {
        const float* s = v.data() + (perm.empty() ? r : perm[r]) * cols;
        T* d = o.data() + r * cols;
        for (int64_t c = 0; c < cols; c++) {
          if constexpr (sizeof(T) == 2) d[c] = f2bf(s[c]); else d[c] = s[c];
        }
      }
    };
    const int nth = rows * cols > (1 << 22) ? 8 : 1;
    std::vector<std::thread> th;
    for (int i = 0; i < nth; i++) th.emplace_back(work, rows * i / nth, rows * (i + 1) / nth);
    for (auto& x : th) x.join();
    T* d = dalloc<T>(o.size());
    LAYA_HIP(hipMemcpy(d, o.data(), o.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
  }
  // The matrix [rows, cols] of the GEMM that reads LayerNorm(x) (weight lnw [cols], bias lnb or
  // null) through the fold: stored row r = bf16(W[perm[r]] * lnw) (weights multiplied in fp32 and
  // rounded once); c[r] = the sum of stored row r (exact sum of the bf16 values, rounded to fp32);
  // bias[r] += W[perm[r]] . lnb (fp64, from the checkpoint's values) when lnb is given.
  T* up_mat_ln(const SafeTensors& st, const std::string& n, int64_t rows, int64_t cols, const std::string& lnw_name,
               const std::string& lnb_name, float** c_out, float** bias_io, const std::vector<int>& perm = {}) {
    const TensorView& t = must(st, n);
    check_shape(t, {rows, cols}, n);
    std::vector<float> v = host_f32(t);
    const TensorView& tw = must(st, lnw_name);
    check_shape(tw, {cols}, lnw_name);
    const std::vector<float> lw = host_f32(tw);
    std::vector<float> lb;
    if (!lnb_name.empty()) {
      const TensorView& tb = must(st, lnb_name);
      check_shape(tb, {cols}, lnb_name);
      lb = host_f32(tb);
    }
    std::vector<T> o((size_t)(rows * cols));
    std::vector<float> c((size_t)rows), add((size_t)rows, 0.f);
    for (int64_t r = 0; r < rows; r++) {
      const float* s = v.data() + (perm.empty() ? r : perm[r]) * cols;
      T* d = o.data() + r * cols;
      double cs = 0.0, bs = 0.0;
      for (int64_t k = 0; k < cols; k++) {
        d[k] = f2bf(s[k] * lw[k]);
        cs += (double)bf2f(d[k]);
        if (!lb.empty()) bs += (double)s[k] * (double)lb[k];
      }
      c[r] = (float)cs;
      add[r] = (float)bs;
    }
    T* dev = dalloc<T>(o.size());
    LAYA_HIP(hipMemcpy(dev, o.data(), o.size() * sizeof(T), hipMemcpyHostToDevice));
    float* dc = dalloc<float>(c.size());
    LAYA_HIP(hipMemcpy(dc, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    *c_out = dc;
    if (!lb.empty()) {
      // the bias (already on the device) gains W . lnb
      std::vector<float> b((size_t)rows);
      LAYA_HIP(hipMemcpy(b.data(), *bias_io, rows * 4, hipMemcpyDeviceToHost));
      for (int64_t r = 0; r < rows; r++) b[r] = (float)((double)b[r] + (double)add[r]);
      LAYA_HIP(hipMemcpy(*bias_io, b.data(), rows * 4, hipMemcpyHostToDevice));
    }
    return dev;
  }

  // Wi rows as alternating 32-row blocks of input rows and gate rows (GeGLU epilogue pairs)
  std::vector<int> geglu_perm() const {
    const int I = cfg.intermediate;
    std::vector<int> p(2 * I);
    for (int r = 0; r < 2 * I; r++) {
      const int pair = r / 64, within = r % 64;
      p[r] = within < 32 ? pair * 32 + within : I + pair * 32 + (within - 32);
    }
    return p;
  }

  // ------------------------------------------------------------ load
  void load(const std::string& dir) {
    std::string err;
    if (!cfg.load(dir + "/encoder/config.json", dir + "/rl_agent_config.json", &err)) {
      fprintf(stderr, "[laya] %s\n", err.c_str());
      exit(1);
    }
    verbose = getenv("LAYA_VERBOSE") != nullptr;
    printf("%s[laya] precision=%s (gfx950 MFMA path)\n", cfg.describe().c_str(), precision());
    const int D = cfg.d, I = cfg.intermediate, FF = cfg.head_ffn, H = cfg.n_heads, HD = cfg.head_dim, V = cfg.vocab;
    if (HD != 64 || D % 64 || I % 32 || cfg.head_layers < 1 || cfg.n_act < 1 || cfg.n_act > 256) {
      fprintf(stderr, "[laya] unsupported model shape (needs head_dim 64, d %% 64 == 0, intermediate %% 32 == 0, "
                      "head_layers >= 1)\n");
      exit(1);
    }
    SafeTensors st;
    if (!st.open(dir + "/model.safetensors", &err)) { fprintf(stderr, "[laya] %s\n", err.c_str()); exit(1); }

    // The token embeddings stay fp32 in the bf16 engine too (0.2 GB for the large model's 50k-token
    // vocabulary, 0.8 GB for the 256k one): the embedding LayerNorm reads only the pass's rows, and
    // its output, the start of the fp32 residual stream, then carries no bf16 rounding, as in the
    // reference's bf16 autocast, where the embedding and its LayerNorm run in fp32.
    tok_emb = up_f32(st, "encoder.embeddings.tok_embeddings.weight", {V, D});
    emb_norm = up_f32(st, "encoder.embeddings.norm.weight", {D});
    final_norm = up_f32(st, "encoder.final_norm.weight", {D});
    type_emb = up_f32(st, "type_emb.weight", {3, D});
    const std::vector<int> gp = geglu_perm();
    // With LAYA_LN_FOLD=1 the bf16 engine folds every LayerNorm that feeds a GEMM over all rows into
    // that GEMM (see GemmArgs in kernels.h): the encoder's attn_norm (layers >= 1) and mlp_norm, the
    // head's norm1 and, but for the last head layer (gathered rows), norm2.  Off by default: on
    // MI355X at 9.5k rows the residual GEMMs' extra outputs (+3.5 us), the row-statistics kernels
    // (4.8 us) and the consumers' per-element fold (+2.6 to +5 us) cost more than the 12.7 us
    // LayerNorm kernels they replace.
    fold_ln = sizeof(T) == 2 && D % 64 == 0 && D <= 2048 && env_int("LAYA_LN_FOLD", 0) != 0;
    latency = sizeof(T) == 2 && env_int("LAYA_LATENCY", 0) != 0;
    enc.resize(cfg.n_layers);
    for (int i = 0; i < cfg.n_layers; i++) {
      const std::string p = "encoder.layers." + std::to_string(i) + ".";
      if (st.get(p + "attn_norm.weight") || i > 0) enc[i].attn_norm = up_f32(st, p + "attn_norm.weight", {D});
      // layer 0's attn_norm (optional in a checkpoint) runs as its own LayerNorm after the
      // embeddings, so only later layers' are folded into Wqkv
      if (fold_ln && enc[i].attn_norm && i > 0)
        enc[i].Wqkv = up_mat_ln(st, p + "attn.Wqkv.weight", 3 * D, D, p + "attn_norm.weight", "", &enc[i].c_qkv, nullptr);
      else
        enc[i].Wqkv = up_mat(st, p + "attn.Wqkv.weight", 3 * D, D);
      enc[i].Wo = up_mat(st, p + "attn.Wo.weight", D, D);
      enc[i].mlp_norm = up_f32(st, p + "mlp_norm.weight", {D});
      if (fold_ln)
        enc[i].Wi = up_mat_ln(st, p + "mlp.Wi.weight", 2 * I, D, p + "mlp_norm.weight", "", &enc[i].c_wi, nullptr, gp);
      else
        enc[i].Wi = up_mat(st, p + "mlp.Wi.weight", 2 * I, D, gp);
      enc[i].Wmo = up_mat(st, p + "mlp.Wo.weight", D, I);
    }
    head.resize(cfg.head_layers);
    for (int i = 0; i < cfg.head_layers; i++) {
      const std::string p = "head.layers." + std::to_string(i) + ".";
      HeadLayer& h = head[i];
      h.n1w = up_f32(st, p + "norm1.weight", {D}); h.n1b = up_f32(st, p + "norm1.bias", {D});
      h.n2w = up_f32(st, p + "norm2.weight", {D}); h.n2b = up_f32(st, p + "norm2.bias", {D});
      h.inB = up_f32(st, p + "self_attn.in_proj_bias", {3 * D});
      if (fold_ln)
        h.inW = up_mat_ln(st, p + "self_attn.in_proj_weight", 3 * D, D, p + "norm1.weight", p + "norm1.bias", &h.c_in, &h.inB);
      else
        h.inW = up_mat(st, p + "self_attn.in_proj_weight", 3 * D, D);
      h.outW = up_mat(st, p + "self_attn.out_proj.weight", D, D);
      h.outB = up_f32(st, p + "self_attn.out_proj.bias", {D});
      h.l1B = up_f32(st, p + "linear1.bias", {FF});
      if (fold_ln && i + 1 < cfg.head_layers)
        h.l1W = up_mat_ln(st, p + "linear1.weight", FF, D, p + "norm2.weight", p + "norm2.bias", &h.c_l1, &h.l1B);
      else
        h.l1W = up_mat(st, p + "linear1.weight", FF, D);
      h.l2W = up_mat(st, p + "linear2.weight", D, FF); h.l2B = up_f32(st, p + "linear2.bias", {D});
    }
    sc0w = up_f32(st, "scorer.0.weight", {D}); sc0b = up_f32(st, "scorer.0.bias", {D});
    sc1W = up_mat(st, "scorer.1.weight", D, D); sc1b = up_f32(st, "scorer.1.bias", {D});
    sc3w = up_f32(st, "scorer.3.weight", {1, D}); sc3b = up_f32(st, "scorer.3.bias", {1});
    ah0W = up_f32(st, "act_head.0.weight", {256, D + 4}); ah0b = up_f32(st, "act_head.0.bias", {256});
    ah2W = up_f32(st, "act_head.2.weight", {cfg.n_act, 256}); ah2b = up_f32(st, "act_head.2.bias", {cfg.n_act});

    // RoPE tables [max_len][HD/2], as HF builds them (modeling_modernbert.py:136-163): fp32
    // inverse frequencies theta^(-2i/HD), fp32 position products, cos/sin of those.
    {
      const int L = cfg.max_len + kRowAlign, H2 = HD / 2;   // padding rows continue past max_len
      std::vector<float> cg((size_t)L * H2), sg(cg.size()), cl(cg.size()), sl(cg.size());
      for (int i = 0; i < H2; i++) {
        const float ig = 1.0f / powf(cfg.rope_theta_global, (float)(2 * i) / (float)HD);
        const float il = 1.0f / powf(cfg.rope_theta_local, (float)(2 * i) / (float)HD);
        for (int p = 0; p < L; p++) {
          const float fg = (float)p * ig, fl = (float)p * il;
          cg[(size_t)p * H2 + i] = (float)cos((double)fg); sg[(size_t)p * H2 + i] = (float)sin((double)fg);
          cl[(size_t)p * H2 + i] = (float)cos((double)fl); sl[(size_t)p * H2 + i] = (float)sin((double)fl);
        }
      }
      auto upv = [&](std::vector<float>& v) {
        float* d = dalloc<float>(v.size());
        LAYA_HIP(hipMemcpy(d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
        return d;
      };
      cos_g = upv(cg); sin_g = upv(sg); cos_l = upv(cl); sin_l = upv(sl);
    }

    // limits and buffers
    lim.max_len = cfg.max_len;
    lim.vocab = V;
    lim.pad_id = cfg.pad_id;
    if (cfg.pad_id < 0 || cfg.pad_id >= V) { fprintf(stderr, "[laya] pad_token_id outside the vocabulary\n"); exit(1); }
    lim.pass_tokens = std::max(env_int("LAYA_MAX_TOKENS", 65536), cfg.max_len);
    {
      // The kernels read their row operands through buffer resources with 32-bit offsets: every
      // [rows][width] activation (width up to max(D, I, head FFN)) and V^T must stay below 2 GiB,
      // with room for a pass's bucket padding.  Larger capacities are capped here.
      const int64_t width = std::max<int64_t>({(int64_t)D, (int64_t)I, (int64_t)FF});
      const int64_t cap = (((int64_t)1 << 31) - (1 << 20)) / ((int64_t)sizeof(T) * width) / 64 * 64 - 1024;
      if (lim.pass_tokens > cap) {
        fprintf(stderr, "[laya] LAYA_MAX_TOKENS=%d exceeds what 32-bit buffer offsets reach for this model; using %lld\n",
                lim.pass_tokens, (long long)cap);
        lim.pass_tokens = (int)cap;
      }
    }
    lim.pass_tokens = std::min(std::max(env_int("LAYA_PASS_TOKENS", lim.pass_tokens), cfg.max_len), lim.pass_tokens);
    lim.max_seqs = std::max(1, env_int("LAYA_MAX_SEQS", 512));
    lim.max_grows = std::max(env_int("LAYA_MAX_GATHERED", 32768), kMaxMarkers + 1);
    {
      // the gathered rows feed the same kernels (head FFN width), under the same 2 GiB bound
      const int64_t cap = (((int64_t)1 << 31) - (1 << 20)) / ((int64_t)sizeof(T) * std::max(D, FF)) / 64 * 64 - 1024;
      if (lim.max_grows > cap) {
        fprintf(stderr, "[laya] LAYA_MAX_GATHERED=%d exceeds what 32-bit buffer offsets reach; using %lld\n",
                lim.max_grows, (long long)cap);
        lim.max_grows = (int)cap;
      }
    }
    // attention query tiles.  bf16: 64 queries (two waves) in the sliding-window layers and 128
    // (four waves, four per SIMD) in the global ones, the faster tiling of each (same bits either
    // way); LAYA_ATTN_QTILE=64 or 128 puts every layer on one of them.  fp32: 64.
    {
      const int qt = sizeof(T) == 2 ? env_int("LAYA_ATTN_QTILE", 0) : 64;
      lim.q_tile = qt == 128 ? 128 : 64;
      lim.q_tile_global = sizeof(T) == 2 && qt != 64 ? 128 : 64;
    }
    if (lim.q_tile == 128 && (cfg.local_attention / 2) % 64 != 0) {
      // 128-query tiles visit the same key blocks as 64-query tiles only when the sliding window's
      // half width is a multiple of 64 (both tilings then start every query's keys on the same
      // 64-key boundaries); otherwise the tiling would change the bits
      fprintf(stderr, "[laya] LAYA_ATTN_QTILE=128 needs local_attention / 2 to be a multiple of 64; using 64\n");
      lim.q_tile = 64;
    }
    caps = pass_caps(lim);
    MT = caps.rows; RG = caps.grows; VTC = (MT + 64 + 63) / 64 * 64;
    x = dalloc<float>((size_t)MT * D);
    // zeroed once: rows that no kernel of a pass writes (bucket padding after the last question, the
    // attention output of padding rows) are still read, with weight 0, and must hold finite values
    xn = dalloc<T>((size_t)MT * D, true); q = dalloc<T>((size_t)MT * D, true); k = dalloc<T>((size_t)MT * D, true);
    ao = dalloc<T>((size_t)MT * D, true);
    vt = dalloc<T>((size_t)D * VTC, true);      // zeroed once: unread gaps must stay finite
    mg = dalloc<T>((size_t)MT * I);
    ff = dalloc<T>((size_t)std::max(MT, RG) * FF);
    xg = dalloc<float>((size_t)RG * D);
    // the gathered buffers are zeroed once: rows past a pass's gathered queries (the marker padding)
    // are read by the row-wise head GEMMs, which must see finite values
    aog = dalloc<T>((size_t)RG * D, true); xng = dalloc<T>((size_t)RG * D, true); sh = dalloc<T>((size_t)RG * D, true);
    if (sizeof(T) == 2) sk_ws = dalloc<float>(kSplitKBytes / sizeof(float));
    // LayerNorm statistics of the rows the fold's GEMMs read: [D / 64][rows][2] (group-major)
    if (fold_ln) {
      ln_stats = dalloc<float>((size_t)MT * (D / 64) * 2, true);
      ln_mr = dalloc<float>((size_t)MT * 2, true);
    }
    d_logits = dalloc<float>((size_t)RG);
    d_act = dalloc<float>((size_t)lim.max_seqs * cfg.n_act);
    d_act_hidden = dalloc<float>((size_t)lim.max_seqs * 256);
    h_logits = halloc<float>((size_t)RG);
    h_act = halloc<float>((size_t)lim.max_seqs * cfg.n_act);
    {
      blob_cap = blob_layout((int)MT, caps.seqs, (int)RG, (int)caps.tiles, (int)caps.gtiles).total;
      d_blob = dalloc<char>(blob_cap, true);
      h_blob = halloc<char>(blob_cap);
      memset(h_blob, 0, blob_cap);
      bind(Shape{(int)MT, 1, 0});
    }

    LAYA_HIP(hipStreamCreate(&stream));
    {
      int dev = 0;
      LAYA_HIP(hipGetDevice(&dev));
      LAYA_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    }
    prof.init();
    use_graphs = env_int("LAYA_GRAPHS", 1) != 0;
    max_graphs = (size_t)std::max(0, env_int("LAYA_MAX_GRAPHS", 512));
    tune_on = env_int("LAYA_TUNE", 1) != 0;
    if (const char* e = getenv("LAYA_GEMM_CFG")) {
      pin_cfg = atoi(e);
      if (pin_cfg < 0 || pin_cfg >= kGemmConfigs) pin_cfg = -1;
      int rows = 0, tail = -1;
      const char* sp = getenv("LAYA_GEMM_SPLIT");
      if (pin_cfg >= 0 && sp && sscanf(sp, "%d,%d", &rows, &tail) == 2 && rows > 0 && tail >= 0 && tail < kGemmConfigs) {
        pin_split = rows;
        pin_tail = tail;
      }
    }
    if (const char* dd = getenv("LAYA_DUMP_DIR")) dump_dir = dd;
    LAYA_HIP(hipDeviceSynchronize());
    printf("[laya] ready: rows/pass=%lld gathered rows/pass=%lld graphs=%d\n", (long long)MT, (long long)RG,
           (int)use_graphs);
  }

  // ------------------------------------------------------------ one pass
  // byte offsets of the index arrays of a pass bucket in the blocks (256-byte aligned)
  struct BlobLayout { size_t ids, pos, seq, soff, vlen, qt, nm, moff, gq, grow, tiles, gltiles, gtiles, total; };
  static BlobLayout blob_layout(int rows, int B, int R, int nt, int ngt) {
    BlobLayout L;
    size_t o = 0;
    auto take = [&](size_t bytes) { const size_t r = o; o += (bytes + 255) & ~(size_t)255; return r; };
    L.ids = take((size_t)rows * 4); L.pos = take((size_t)rows * 4); L.seq = take((size_t)rows * 4);
    L.soff = take((size_t)(B + 1) * 4); L.vlen = take((size_t)B * 4); L.qt = take((size_t)B * 4);
    L.nm = take((size_t)B * 4); L.moff = take((size_t)B * 4);
    L.gq = take((size_t)R * 4); L.grow = take((size_t)R * 4);
    L.tiles = take((size_t)nt * sizeof(AttnTile)); L.gltiles = take((size_t)nt * sizeof(AttnTile));
    L.gtiles = take((size_t)ngt * sizeof(AttnTile));
    L.total = o;
    return L;
  }
  static BlobLayout blob_layout(const Shape& s) { return blob_layout(s.rows, s.B, s.R(), s.nt(), s.ngt()); }
  void bind(const Shape& s) {
    const BlobLayout L = blob_layout(s);
    auto at = [&](size_t off, int** d, int** h) { *d = (int*)(d_blob + off); *h = (int*)(h_blob + off); };
    at(L.ids, &d_ids, &h_ids); at(L.pos, &d_pos, &h_pos); at(L.seq, &d_seq, &h_seq);
    at(L.soff, &d_soff, &h_soff); at(L.vlen, &d_vlen, &h_vlen); at(L.qt, &d_qt, &h_qt);
    at(L.nm, &d_nm, &h_nm); at(L.moff, &d_moff, &h_moff); at(L.gq, &d_gq, &h_gq); at(L.grow, &d_grow, &h_grow);
    d_tiles = (AttnTile*)(d_blob + L.tiles); h_tiles = (AttnTile*)(h_blob + L.tiles);
    d_gltiles = (AttnTile*)(d_blob + L.gltiles); h_gltiles = (AttnTile*)(h_blob + L.gltiles);
    d_gtiles = (AttnTile*)(d_blob + L.gtiles); h_gtiles = (AttnTile*)(h_blob + L.gtiles);
  }

  void stage_inputs(const PassPlan& p) {
    const Shape s{p.T, p.B, p.KT};
    if ((int)p.tiles.size() != s.nt() || (int)p.gltiles.size() != s.nt() || (int)p.gtiles.size() != s.ngt() ||
        p.R != s.R() || (int)p.gq.size() > p.R) {
      fprintf(stderr, "[laya] internal error: pass arrays do not match their bucket\n");
      exit(1);
    }
    memcpy(h_ids, p.ids.data(), p.T * 4); memcpy(h_pos, p.pos.data(), p.T * 4);
    memcpy(h_seq, p.seq.data(), p.T * 4);
    memcpy(h_soff, p.soff.data(), (p.B + 1) * 4); memcpy(h_vlen, p.vlen.data(), p.B * 4);
    memcpy(h_qt, p.qt.data(), p.B * 4);
    memcpy(h_nm, p.nm.data(), p.B * 4); memcpy(h_moff, p.moff.data(), p.B * 4);
    memcpy(h_gq, p.gq.data(), p.gq.size() * 4); memcpy(h_grow, p.grow.data(), p.R * 4);
    memcpy(h_tiles, p.tiles.data(), p.tiles.size() * sizeof(AttnTile));
    memcpy(h_gltiles, p.gltiles.data(), p.gltiles.size() * sizeof(AttnTile));
    memcpy(h_gtiles, p.gtiles.data(), p.gtiles.size() * sizeof(AttnTile));
  }

  void dump(const char* name, const float* dev, size_t rows) {
    if (dump_dir.empty() || capturing || collecting) return;
    LAYA_HIP(hipStreamSynchronize(stream));
    std::vector<float> buf(rows * cfg.d);
    LAYA_HIP(hipMemcpy(buf.data(), dev, buf.size() * 4, hipMemcpyDeviceToHost));
    std::string fn = dump_dir + "/" + name + ".bin";
    FILE* f = fopen(fn.c_str(), "wb");
    if (f) { fwrite(buf.data(), 4, buf.size(), f); fclose(f); }
  }

  // Split-K for the GEMMs on the gathered rows and the scorer (a few hundred rows, so without it
  // a handful of tiles would each walk the whole K).  The factor depends only on K, never on how
  // many rows a batch gathered, so a row's result is the same in every batch.
  static constexpr size_t kSplitKBytes = (size_t)64 << 20;
  float* sk_ws = nullptr;
  bool fold_ln = false;
  float* ln_stats = nullptr;                          // per-group statistics (the residual GEMMs' scratch)
  float* ln_mr = nullptr;                             // mean and rstd of each row of xn
  void splitk(GemmArgs& g) const {
    if (sizeof(T) != 2 || !sk_ws) return;
    g.ksplit = g.K >= 2048 ? 16 : 8;
    g.ws = sk_ws;
    g.ws_bytes = kSplitKBytes;
  }
  // LAYA_LATENCY=1 (bf16, read at laya_create): the residual GEMMs over all rows (the encoder's
  // out-projection and MLP down-projection, the first head layers' out-projection and FFN
  // down-projection) also split K, into chunks of kLatencyStages 64-deep stages, whatever the
  // pass's size.  A pass of a few hundred rows then puts several workgroups on each of the 8-16
  // tiles these N = 1024 GEMMs have, instead of walking all of K on a few CUs.  The chunking
  // depends only on K, so every row's result is the same in every batch (and differs from the
  // default engine's in the last bits: the partial sums are added in chunk order).  Larger
  // passes pay for the fp32 partials: the mode is for latency-bound serving of small batches.
  // When a pass's partial products fit the workspace in one piece, the GEMM only writes them and
  // the LayerNorm that follows adds them to x (in the reduction's order, so the same bits) before
  // normalising: no reduction launch, and x is read and written once instead of twice.
  static constexpr int kLatencyStages = 4;
  bool latency = false;
  PendingPartials pend;                               // partials the next LayerNorm over all rows adds
  void splitk_latency(GemmArgs& g) {
    if (!latency || sizeof(T) != 2 || !sk_ws || g.Xh || g.K % 64) return;
    const int stages = g.K / 64;
    if (stages <= kLatencyStages) return;
    g.ksplit = (stages + kLatencyStages - 1) / kLatencyStages;
    g.ws = sk_ws;
    g.ws_bytes = kSplitKBytes;
    const int ch = gemm_splitk_chunks(g.K, g.ksplit);
    if (dump_dir.empty() && !fold_ln && (size_t)g.M * ch * g.N * sizeof(float) <= kSplitKBytes) {
      g.partials_only = true;
      pend = PendingPartials{sk_ws, ch, (size_t)g.M * g.N, g.bias, g.X};
    }
  }
  // the pending partials for the next LayerNorm (null when none), handed over once
  const PendingPartials* take_pending() {
    if (!pend.p) return nullptr;
    pend_taken = pend;
    pend = PendingPartials{};
    return &pend_taken;
  }
  PendingPartials pend_taken;

  GemmArgs gemm_args(const T* A, int lda, const T* W, int M, int N, int K, const float* bias) {
    GemmArgs g;
    g.A = A; g.lda = lda; g.W = W; g.ldw = K; g.M = M; g.N = N; g.K = K; g.bias = bias;
    return g;
  }

  // ------------------------------------------------------------ GEMM tile tuning
  // M buckets: multiples of 64 rows up to 1024, then 16 buckets per octave up to 8192 rows and 8
  // per octave above (88 buckets up to 65536 rows); every bucket bound is a multiple of 64
  static int m_bucket(int M) {
    if (M <= 1024) return (M + 63) / 64 * 64;
    const int lg = 31 - __builtin_clz((unsigned)(M - 1));          // 2^lg < M <= 2^(lg + 1)
    const int step = (1 << lg) / (lg < 13 ? 16 : 8);
    return (M + step - 1) / step * step;
  }
  static TuneKey tune_key(int epi, const GemmArgs& g) {
    return TuneKey(epi, g.act, g.N, g.K, g.rope_cos != nullptr, m_bucket(g.M),
                   (g.ln_mr ? 1 : 0) + (g.stats ? 2 : 0) + (g.bias ? 4 : 0));
  }

  // one GEMM of the pass: listed while the pass is collected for tuning, otherwise launched with
  // the measured configuration of its bucket (the analytic planner's where none was measured)
  void gemm(int epi, GemmArgs g, hipStream_t st) {
    if (collecting) { collecting->emplace_back(epi, g); return; }
    if (pin_cfg >= 0) {
      g.cfg = pin_cfg; g.split_rows = pin_split; g.cfg_tail = pin_tail;
    } else {
      auto it = tuned.find(tune_key(epi, g));
      if (it != tuned.end()) apply_plan(g, it->second);
    }
    launch_gemm<T>(epi, g, st);
  }

  static void apply_plan(GemmArgs& g, const TilePlan& p) {
    g.cfg = p.cfg;
    const int rows = p.split_tiles * gemm_config_bm(p.cfg);
    if (p.split_tiles > 0 && rows < g.M) { g.split_rows = rows; g.cfg_tail = p.tail; }
    else { g.split_rows = 0; g.cfg_tail = -1; }
  }

  // Times every tile configuration this GEMM can use, at its own M, on its own buffers (which hold
  // nothing live before a pass), and returns the fastest: the analytic pick unless another one is
  // more than 1% faster.  Besides single launches, the candidates include row splits: large tiles
  // over the rows that fill whole rounds of the CUs (the last one, or the last two), and 128x128
  // or 128x256 tiles over the rest, so that a partial last round of large tiles is not paid in
  // full.  The operand rows are first filled with a finite pattern so the timing sees realistic
  // MFMA power and the V^T rows a QKV candidate writes stay finite.
  TilePlan tune_gemm(int epi, GemmArgs g) {
    TilePlan first;
    first.cfg = gemm_planned(epi, g);
    if (first.cfg < 0) return first;
    std::vector<TilePlan> cands = {first};
    for (int c = 0; c < kGemmConfigs; c++)
      if (c != first.cfg && gemm_config_valid(epi, g, c)) cands.push_back(TilePlan{c, 0, -1});
    for (int c1 : {0, 4, 5}) {
      if (!gemm_config_valid(epi, g, c1)) continue;
      const int bm = gemm_config_bm(c1), tn = (g.N + gemm_config_bn(c1) - 1) / gemm_config_bn(c1);
      const int rounds = ((g.M + bm - 1) / bm) * tn / n_cu;
      int last_kb = -1;
      for (int r = rounds; r >= std::max(1, rounds - 1); r--) {
        const int kb = r * n_cu / tn;
        if (kb < 1 || kb == last_kb || kb * bm >= g.M) continue;
        last_kb = kb;
        for (int c2 : {3, 2})
          if (gemm_split_valid(epi, g, c1, kb * bm, c2)) cands.push_back(TilePlan{c1, kb, c2});
      }
    }
    // GeGLU: 192x128 tiles (two per CU) over the rows that fill whole rounds of the CUs' slots, and
    // 128x64 or 128x128 tiles over the rest in the same launch, filling the slots that the partial
    // last round of 192x128 tiles would leave idle
    if (epi == EPI_GEGLU && !g.ln_mr && gemm_config_valid(epi, g, 7)) {
      const int tn = (g.N + 127) / 128, slots = 2 * n_cu;
      const int kb = ((g.M + 191) / 192) * tn / slots * slots / tn;
      if (kb >= 1 && kb * 192 < g.M)
        for (int c2 : {8, 3})
          if (gemm_split_valid(epi, g, 7, kb * 192, c2)) cands.push_back(TilePlan{7, kb, c2});
    }
    launch_fill_pattern((T*)const_cast<void*>(g.A), (size_t)g.M * g.lda, 0x9E3779B9u ^ (uint32_t)g.K, stream);
    hipEvent_t a, b;
    LAYA_HIP(hipEventCreate(&a));
    LAYA_HIP(hipEventCreate(&b));
    // two rounds over the candidates, the second in reverse order (the clock drifts while the chip
    // warms up), keeping each candidate's best time; the planner's pick keeps a 1% preference
    const int reps = g.M >= 2048 ? 4 : 8;
    std::vector<float> t(cands.size(), 1e30f);
    for (int round = 0; round < 2; round++)
      for (size_t n = 0; n < cands.size(); n++) {
        const size_t i = round ? cands.size() - 1 - n : n;
        apply_plan(g, cands[i]);
        launch_gemm<T>(epi, g, stream);
        LAYA_HIP(hipEventRecord(a, stream));
        for (int r = 0; r < reps; r++) launch_gemm<T>(epi, g, stream);
        LAYA_HIP(hipEventRecord(b, stream));
        LAYA_HIP(hipEventSynchronize(b));
        float ms = 0.f;
        LAYA_HIP(hipEventElapsedTime(&ms, a, b));
        t[i] = std::min(t[i], ms / reps);
      }
    LAYA_HIP(hipEventDestroy(a));
    LAYA_HIP(hipEventDestroy(b));
    size_t bi = 0;
    for (size_t i = 1; i < cands.size(); i++)
      if (t[i] < t[bi] * (bi == 0 ? 0.99f : 1.0f)) bi = i;
    if (verbose)
      for (size_t i = 0; i < cands.size(); i++)
        printf("[laya] tune epi %d %5dx%5dx%5d cfg %d split %5d tail %2d: %8.1f us%s\n", epi, g.M, g.N, g.K, cands[i].cfg,
               cands[i].split_tiles * gemm_config_bm(cands[i].cfg), cands[i].tail, t[i] * 1e3f, i == bi ? "  <- picked" : "");
    return cands[bi];
  }

  // lists the GEMMs of pass shape s (uploading its index arrays, which the QKV epilogue reads) and
  // tunes the buckets not yet measured
  void tune_pass(const Shape& s) {
    if (!tune_on || sizeof(T) != 2 || gemm_pinned() >= 0 || pin_cfg >= 0 || capturing || tuned_shapes.count(s)) return;
    std::vector<std::pair<int, GemmArgs>> list;
    collecting = &list;
    run(s);
    collecting = nullptr;
    for (auto& eg : list) {
      const TuneKey key = tune_key(eg.first, eg.second);
      if (eg.second.ksplit <= 1 && !tuned.count(key)) tuned[key] = tune_gemm(eg.first, eg.second);
    }
    LAYA_HIP(hipStreamSynchronize(stream));
    tuned_shapes.insert(s);
  }

  // every M bucket up to the pass capacity, for every GEMM of the model (the gathered head rows and
  // the scorer share the encoder's and head's (N, K) shapes at other M)
  void tune_all() override {
    if (tune_on && sizeof(T) == 2 && gemm_pinned() < 0 && pin_cfg < 0) {
      // the listing run uploads the host block: all zeros (position 0) keeps the RoPE table reads
      // in range whatever the layout.  The gathered-row GEMMs (KT + 1 rows) and the scorer (KT rows)
      // are listed at the largest marker bucket below the row bucket.
      memset(h_blob, 0, blob_cap);
      for (int mb = 64; mb <= MT; mb = m_bucket(mb + 1)) {
        const int kt = (int)std::max<int64_t>(kMarkerBucket, std::min<int64_t>(mb, RG - 1) / kMarkerBucket * kMarkerBucket);
        tune_pass(Shape{mb, 1, kt});
      }
    }
    warmup();
  }

  void run(const Shape& s) {
    const int D = cfg.d, H = cfg.n_heads, HD = cfg.head_dim, I = cfg.intermediate, FF = cfg.head_ffn;
    const float eps = cfg.norm_eps, scale = 1.0f / sqrtf((float)HD);
    const int T_ = s.rows, B = s.B, KT = s.KT, R = s.R();
    hipStream_t st = stream;
    auto h2d = [&](void* d, const void* h, size_t n) { LAYA_HIP(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, st)); };
    bind(s);
    h2d(d_blob, h_blob, blob_layout(s).total);
    pend = PendingPartials{};
    if (prof.on && !collecting) prof.seq.clear();

    // while the pass is only being listed for tuning, GEMMs are recorded and nothing else runs
#define STAGE(name, ...) do { if (!collecting) { prof.begin(name); __VA_ARGS__; prof.end(); } } while (0)
#define GSTAGE(name, ...) do { if (collecting) { __VA_ARGS__; } else { prof.begin(name); __VA_ARGS__; prof.end(); } } while (0)
    STAGE("enc:embed_ln", launch_layernorm<float, T>(tok_emb, d_ids, T_, D, eps, emb_norm, nullptr, nullptr, nullptr,
                                                 nullptr, x, enc[0].attn_norm ? nullptr : xn, st));
    dump("emb", x, T_);
    // LayerNorm fold (bf16): a residual GEMM leaves x, its bf16 copy in xn and each row's mean and rstd;
    // the next GEMM reads xn with the LayerNorm weight folded into its own weight
    auto fold_in = [&](GemmArgs& g, const float* c) { g.ln_mr = ln_mr; g.ln_c = c; };
    auto fold_out = [&](GemmArgs& g) {
      if constexpr (sizeof(T) == 2) {
        g.Xh = xn; g.ldxh = D; g.stats = ln_stats; g.ldst = (int)MT;
      }
    };
    for (int L = 0; L < cfg.n_layers; L++) {
      const EncLayer& e = enc[L];
      const bool glob = cfg.global_layer[L] != 0;
      const bool last_layer = L + 1 == cfg.n_layers;
      if (L == 0 && e.attn_norm)            // later layers' attn_norm runs after the previous layer, or is folded
        STAGE("enc:ln", launch_layernorm<float, T>(x, nullptr, T_, D, eps, e.attn_norm, nullptr, nullptr, nullptr,
                                                   nullptr, nullptr, xn, st));
      {
        GemmArgs g = gemm_args(xn, D, e.Wqkv, T_, 3 * D, D, nullptr);
        g.Q = q; g.Kt = k; g.ldqk = D; g.Vt = vt; g.ldv = (int)VTC; g.H = H; g.HD = HD; g.pos = d_pos;
        g.rope_cos = glob ? cos_g : cos_l; g.rope_sin = glob ? sin_g : sin_l;
        if (e.c_qkv && L > 0) fold_in(g, e.c_qkv);
        GSTAGE("enc:gemm_qkv_rope", gemm(EPI_QKV, g, st));
      }
      STAGE(glob ? "enc:attn_global" : "enc:attn_sliding",
            launch_attention<T>(q, k, D, (int)MT, vt, (int)VTC, ao, D, glob ? d_gltiles : d_tiles, s.nt(),
                                glob ? lim.q_tile_global : lim.q_tile, H, d_soff, d_vlen, nullptr, nullptr,
                                glob ? 0 : cfg.local_attention / 2, scale, st));
      {
        GemmArgs g = gemm_args(ao, D, e.Wo, T_, D, D, nullptr);
        g.X = x; g.ldx = D;
        if (fold_ln) fold_out(g);
        splitk_latency(g);
        GSTAGE("enc:gemm_attn_out_res", gemm(EPI_RESID, g, st));
        if (fold_ln) STAGE("enc:ln_rowstats", launch_ln_rowstats(ln_stats, (int)MT, D / 64, T_, eps, ln_mr, st));
      }
      if (!fold_ln)
        STAGE("enc:ln", launch_layernorm<float, T>(x, nullptr, T_, D, eps, e.mlp_norm, nullptr, nullptr, nullptr, nullptr,
                                                   nullptr, xn, st, nullptr, take_pending()));
      {
        GemmArgs g = gemm_args(xn, D, e.Wi, T_, 2 * I, D, nullptr);
        g.C = mg; g.ldc = I;
        if (fold_ln) fold_in(g, e.c_wi);
        GSTAGE("enc:gemm_mlp_in_geglu", gemm(EPI_GEGLU, g, st));
      }
      {
        GemmArgs g = gemm_args(mg, I, e.Wmo, T_, D, I, nullptr);
        g.X = x; g.ldx = D;
        if (fold_ln && !last_layer) fold_out(g);
        splitk_latency(g);
        GSTAGE("enc:gemm_mlp_out_res", gemm(EPI_RESID, g, st));
        if (fold_ln && !last_layer)
          STAGE("enc:ln_rowstats", launch_ln_rowstats(ln_stats, (int)MT, D / 64, T_, eps, ln_mr, st));
      }
      if (!dump_dir.empty() && !capturing) { char nm[32]; snprintf(nm, sizeof nm, "enc%d", L); dump(nm, x, T_); }
      if (!last_layer) {
        if (!fold_ln)
          STAGE("enc:ln", launch_layernorm<float, T>(x, nullptr, T_, D, eps, enc[L + 1].attn_norm, nullptr, nullptr,
                                                     nullptr, nullptr, nullptr, xn, st, nullptr, take_pending()));
      } else {
        // final_norm then + type_emb[qtype of the row's question] (ref/rl_common.py:104), in place;
        // with the fold also its bf16 copy and statistics, which the head's first GEMM reads
        const PendingPartials* pp = take_pending();
        if (pp) pend_taken.xout = nullptr;              // x is overwritten by the normalised rows here
        STAGE("enc:final_ln_type", launch_layernorm<float, T>(x, nullptr, T_, D, eps, final_norm, nullptr, type_emb,
                                                              d_qt, d_seq, x, fold_ln ? xn : (T*)nullptr, st,
                                                              fold_ln ? ln_mr : nullptr, pp));
      }
    }
    dump("final", x, T_);

    for (int L = 0; L < cfg.head_layers; L++) {
      const HeadLayer& hl = head[L];
      const bool last = L == cfg.head_layers - 1;
      if (!fold_ln)
        STAGE("head:ln", launch_layernorm<float, T>(x, nullptr, T_, D, eps, hl.n1w, hl.n1b, nullptr, nullptr, nullptr,
                                                    nullptr, xn, st, nullptr, take_pending()));
      {
        GemmArgs g = gemm_args(xn, D, hl.inW, T_, 3 * D, D, hl.inB);
        g.Q = q; g.Kt = k; g.ldqk = D; g.Vt = vt; g.ldv = (int)VTC; g.H = H; g.HD = HD; g.pos = d_pos;
        if (fold_ln) fold_in(g, hl.c_in);
        GSTAGE("head:gemm_qkv", gemm(EPI_QKV, g, st));
      }
      if (!last) {
        STAGE("head:attn", launch_attention<T>(q, k, D, (int)MT, vt, (int)VTC, ao, D, d_gltiles, s.nt(), lim.q_tile_global, H, d_soff,
                                               d_vlen, nullptr, nullptr, 0, scale, st));
        { GemmArgs g = gemm_args(ao, D, hl.outW, T_, D, D, hl.outB); g.X = x; g.ldx = D;
          if (fold_ln) fold_out(g);
          splitk_latency(g);
          GSTAGE("head:gemm_out_res", gemm(EPI_RESID, g, st)); }
        if (fold_ln) STAGE("head:ln_rowstats", launch_ln_rowstats(ln_stats, (int)MT, D / 64, T_, eps, ln_mr, st));
        if (!fold_ln)
          STAGE("head:ln", launch_layernorm<float, T>(x, nullptr, T_, D, eps, hl.n2w, hl.n2b, nullptr, nullptr, nullptr,
                                                      nullptr, xn, st, nullptr, take_pending()));
        { GemmArgs g = gemm_args(xn, D, hl.l1W, T_, FF, D, hl.l1B); g.C = ff; g.ldc = FF; g.act = ACT_RELU;
          if (fold_ln) fold_in(g, hl.c_l1);
          GSTAGE("head:gemm_ffn1_relu", gemm(EPI_STORE, g, st)); }
        { GemmArgs g = gemm_args(ff, FF, hl.l2W, T_, D, FF, hl.l2B); g.X = x; g.ldx = D;
          if (fold_ln) fold_out(g);
          splitk_latency(g);
          GSTAGE("head:gemm_ffn2_res", gemm(EPI_RESID, g, st)); }
        if (fold_ln) STAGE("head:ln_rowstats", launch_ln_rowstats(ln_stats, (int)MT, D / 64, T_, eps, ln_mr, st));
        if (!dump_dir.empty() && !capturing) { char nm[32]; snprintf(nm, sizeof nm, "head%d", L); dump(nm, x, T_); }
      } else {
        // queries, out-proj and FFN only for the R = KT + B rows read afterwards
        STAGE("head:attn_gathered", launch_attention<T>(q, k, D, (int)MT, vt, (int)VTC, aog, D, d_gtiles, s.ngt(), kQTile, H, d_soff,
                                                        d_vlen, d_gq, d_grow, 0, scale, st));
        STAGE("head:gather", launch_gather_rows(x, d_grow, xg, R, D, st));
        { GemmArgs g = gemm_args(aog, D, hl.outW, R, D, D, hl.outB); g.X = xg; g.ldx = D; splitk(g);
          GSTAGE("head:gemm_out_res", gemm(EPI_RESID, g, st)); }
        STAGE("head:ln", launch_layernorm<float, T>(xg, nullptr, R, D, eps, hl.n2w, hl.n2b, nullptr, nullptr, nullptr,
                                                    nullptr, xng, st));
        { GemmArgs g = gemm_args(xng, D, hl.l1W, R, FF, D, hl.l1B); g.C = ff; g.ldc = FF; g.act = ACT_RELU;
          GSTAGE("head:gemm_ffn1_relu", gemm(EPI_STORE, g, st)); }
        { GemmArgs g = gemm_args(ff, FF, hl.l2W, R, D, FF, hl.l2B); g.X = xg; g.ldx = D; splitk(g);
          GSTAGE("head:gemm_ffn2_res", gemm(EPI_RESID, g, st)); }
        if (!dump_dir.empty() && !capturing) { char nm[32]; snprintf(nm, sizeof nm, "head%d_gathered", L); dump(nm, xg, R); }
      }
    }
    // scorer on the KT marker rows: LN(+bias) -> Linear + GELU -> Linear(D -> 1)
    STAGE("scorer:ln", launch_layernorm<float, T>(xg, nullptr, KT, D, eps, sc0w, sc0b, nullptr, nullptr, nullptr,
                                                  nullptr, xng, st));
    { GemmArgs g = gemm_args(xng, D, sc1W, KT, D, D, sc1b); g.C = sh; g.ldc = D; g.act = ACT_GELU; splitk(g);
      GSTAGE("scorer:gemm_gelu", gemm(EPI_STORE, g, st)); }
    STAGE("scorer:dot", launch_row_dot<T>(sh, D, sc3w, sc3b, d_logits, KT, D, st));
    STAGE("act_head", launch_act_head(xg + (size_t)KT * D, D, d_logits, d_moff, d_nm, ah0W, ah0b, ah2W, ah2b,
                                      cfg.n_act, d_act, d_act_hidden, B, st));
#undef STAGE
#undef GSTAGE
    if (collecting) return;
    LAYA_HIP(hipMemcpyAsync(h_logits, d_logits, (size_t)KT * 4, hipMemcpyDeviceToHost, st));
    LAYA_HIP(hipMemcpyAsync(h_act, d_act, (size_t)B * cfg.n_act * 4, hipMemcpyDeviceToHost, st));
  }

  // graph replay on a hit; on a miss run eagerly, then capture the same sequence
  void execute(const Shape& s) {
    last = s; have_last = true;
    const bool graphs_on = use_graphs && !prof.on && dump_dir.empty();
    if (graphs_on) {
      auto it = graphs.find(s);
      if (it != graphs.end()) {
        LAYA_HIP(hipGraphLaunch(it->second, stream));
        LAYA_HIP(hipStreamSynchronize(stream));
        return;
      }
    }
    tune_pass(s);
    run(s);
    LAYA_HIP(hipStreamSynchronize(stream));
    if (prof.on) prof.collect();
    if (!graphs_on || graphs.size() >= max_graphs) return;
    hipGraph_t g;
    hipGraphExec_t ex;
    if (hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal) != hipSuccess) { use_graphs = false; return; }
    capturing = true;
    run(s);
    capturing = false;
    if (hipStreamEndCapture(stream, &g) != hipSuccess || hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess) {
      fprintf(stderr, "[laya] graph capture failed; continuing without graphs\n");
      (void)hipGetLastError();
      use_graphs = false;
      return;
    }
    LAYA_HIP(hipGraphDestroy(g));
    graphs[s] = ex;
    n_captures++;
  }

  int forward_batch(int B, const int* lens, const int* ids, const int* nmark, const int* markers, const int* qtypes,
                    float* logits, float* act) override {
    std::vector<PassPlan> passes;
    if (plan_passes(B, lens, ids, nmark, markers, qtypes, lim, &passes) != 0) return -1;
    std::vector<int64_t> moff(B + 1, 0);
    for (int b = 0; b < B; b++) moff[b + 1] = moff[b] + nmark[b];
    for (const PassPlan& p : passes) {
      const Shape s{p.T, p.B, p.KT};
      bind(s);
      stage_inputs(p);
      execute(s);
      for (int i = 0; i < p.B; i++) {
        const int b = p.first + i;
        memcpy(logits + moff[b], h_logits + p.moff[i], (size_t)nmark[b] * 4);
        memcpy(act + (size_t)b * cfg.n_act, h_act + (size_t)i * cfg.n_act, (size_t)cfg.n_act * 4);
      }
    }
    return 0;
  }

  int replay(int iters, float* ms) override {
    if (!have_last || iters < 1) return -1;
    hipEvent_t a, b;
    LAYA_HIP(hipEventCreate(&a));
    LAYA_HIP(hipEventCreate(&b));
    auto it = graphs.find(last);
    const bool g = use_graphs && !prof.on && dump_dir.empty() && it != graphs.end();
    LAYA_HIP(hipEventRecord(a, stream));
    for (int i = 0; i < iters; i++) {
      if (g) LAYA_HIP(hipGraphLaunch(it->second, stream));
      else run(last);
    }
    LAYA_HIP(hipEventRecord(b, stream));
    LAYA_HIP(hipEventSynchronize(b));
    LAYA_HIP(hipEventElapsedTime(ms, a, b));
    LAYA_HIP(hipEventDestroy(a));
    LAYA_HIP(hipEventDestroy(b));
    if (prof.on) prof.collect();
    return 0;
  }

  void warmup() override {
    std::vector<int> ids(std::min(cfg.max_len, 64), cfg.cls_id), mk = {0};
    int len = (int)ids.size(), nm = 1, qt = 0;
    std::vector<float> lo(1), ac(cfg.n_act);
    forward_batch(1, &len, ids.data(), &nm, mk.data(), &qt, lo.data(), ac.data());
  }
};

}  // namespace laya

// ---------------------------------------------------------------- C ABI
using laya::EngineIface;
static EngineIface* E(void* h) { return static_cast<EngineIface*>(h); }

extern "C" {
void* laya_create(const char* dir) {
  const char* p = getenv("LAYA_PRECISION");
  const std::string prec = p ? p : "bf16";
  EngineIface* e = nullptr;
  if (prec == "fp32") { auto* x = new laya::Engine<float>(); x->load(dir); e = x; }
  else if (prec == "bf16") { auto* x = new laya::Engine<laya::bf16_t>(); x->load(dir); e = x; }
  else { fprintf(stderr, "[laya] LAYA_PRECISION must be bf16 or fp32\n"); exit(1); }
  return e;
}
int laya_forward_batch(void* h, int B, const int* lens, const int* ids, const int* nmark, const int* markers,
                       const int* qtypes, float* logits, float* act) {
  return E(h)->forward_batch(B, lens, ids, nmark, markers, qtypes, logits, act);
}
void laya_forward(void* h, const int* ids, int S, int valid_len, const int* markers, int K, int qtype, float* logits,
                  float* act) {
  (void)S;
  E(h)->forward_batch(1, &valid_len, ids, &K, markers, &qtype, logits, act);
}
int laya_n_act(void* h) { return E(h)->cfg.n_act; }
int laya_max_len(void* h) { return E(h)->cfg.max_len; }
int laya_max_markers(void* h) { (void)h; return laya::kMaxMarkers; }
float laya_temperature(void* h, int qtype) {
  const auto& t = E(h)->cfg.temperature;
  return qtype >= 0 && qtype < (int)t.size() ? t[qtype] : 1.0f;
}
void laya_prof_report(void* h, int iters) { E(h)->prof.report(iters); }
void laya_prof_reset(void* h) { E(h)->prof.acc.clear(); E(h)->prof.pending.clear(); }
void laya_tune_all(void* h) { E(h)->tune_all(); }

int laya_ext_prof_enable(void* h, int on) { int was = E(h)->prof.on; E(h)->prof.on = on != 0; return was; }
int laya_ext_prof_stage(void* h, int i, char* name, int name_len, double* ms, long long* calls) {
  auto& acc = E(h)->prof.acc;
  if (i < 0 || i >= (int)acc.size()) return -1;
  if (name && name_len > 0) { strncpy(name, std::get<0>(acc[i]).c_str(), name_len - 1); name[name_len - 1] = 0; }
  if (ms) *ms = std::get<1>(acc[i]);
  if (calls) *calls = std::get<2>(acc[i]);
  return 0;
}
int laya_ext_replay(void* h, int iters, float* ms) { return E(h)->replay(iters, ms); }
int laya_ext_prof_sequence(void* h, int* stages, int cap) {
  if (!h || cap < 0 || (cap > 0 && !stages)) return -1;
  const auto& q = E(h)->prof.seq;
  for (int i = 0; i < cap && i < (int)q.size(); i++) stages[i] = q[i];
  return (int)q.size();
}
static float* g_ext_ws = nullptr;          // split-K workspace of laya_ext_gemm (caller's memory)
static size_t g_ext_ws_bytes = 0;

// The measurement hooks run inside the caller's process, which shares the HIP runtime (and its
// per-thread last error) with the caller: a stale error that the caller's own HIP calls left must
// not be reported as this launch's, so each hook clears it first and then checks its own launches.

// launch only: the caller times it with its own events on its stream
int laya_ext_mfma_loop(float* out, int blocks, int iters, void* stream, double* flops) {
  using namespace laya;
  if (!out || blocks < 1 || iters < 1) return -1;
  (void)hipGetLastError();
  launch_mfma_loop(out, blocks, iters, (hipStream_t)stream);
  LAYA_HIP(hipGetLastError());
  if (flops) *flops = (double)blocks * 4.0 * iters * 8.0 * 32768.0;
  return 0;
}

// launch only, like the MFMA loop: two workgroups per CU
int laya_ext_hbm_copy(const void* src, void* dst, size_t bytes, void* stream) {
  using namespace laya;
  if (!src || !dst || bytes == 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return -1;
  const char* s = static_cast<const char*>(src);
  const char* d = static_cast<const char*>(dst);
  if (s < d + bytes && d < s + bytes) return -1;         // overlapping ranges
  (void)hipGetLastError();
  int dev = 0, cus = 0;
  LAYA_HIP(hipGetDevice(&dev));
  LAYA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  launch_hbm_copy(src, dst, bytes / 16, 2 * (cus > 0 ? cus : 256), (hipStream_t)stream);
  LAYA_HIP(hipGetLastError());
  return 0;
}

int laya_ext_gemm(int dtype, int epi, const void* A, const void* W, void* C, const float* bias, int act, int M, int N,
                  int K, void* stream, int iters, float* ms) {
  using namespace laya;
  if ((dtype != 0 && dtype != 1) || (epi != 0 && epi != 1) || iters < 1) return -1;
  GemmArgs g;
  g.A = A; g.lda = K; g.W = W; g.ldw = K; g.M = M; g.N = N; g.K = K; g.bias = bias; g.act = act;
  if (epi == 0) { g.C = C; g.ldc = N; } else { g.X = (float*)C; g.ldx = N; }
  const char* why = "";
  if (!gemm_shape_ok(epi == 0 ? EPI_STORE : EPI_RESID, g, dtype == 0 ? 4 : 2, &why)) return -1;
  hipStream_t st = (hipStream_t)stream;
  (void)hipGetLastError();
  // a pinned split-K factor runs in the caller's workspace (laya_ext_gemm_ksplit)
  g.ws = g_ext_ws;
  g.ws_bytes = g_ext_ws_bytes;
  hipEvent_t a, b;
  if (ms) { LAYA_HIP(hipEventCreate(&a)); LAYA_HIP(hipEventCreate(&b)); LAYA_HIP(hipEventRecord(a, st)); }
  for (int i = 0; i < iters; i++) {
    if (dtype == 0) launch_gemm<float>(epi == 0 ? EPI_STORE : EPI_RESID, g, st);
    else launch_gemm<bf16_t>(epi == 0 ? EPI_STORE : EPI_RESID, g, st);
  }
  if (ms) {
    LAYA_HIP(hipEventRecord(b, st));
    LAYA_HIP(hipEventSynchronize(b));
    LAYA_HIP(hipEventElapsedTime(ms, a, b));
    LAYA_HIP(hipEventDestroy(a)); LAYA_HIP(hipEventDestroy(b));
  }
  LAYA_HIP(hipGetLastError());
  return 0;
}
const char* laya_ext_precision(void* h) { return E(h)->precision(); }

int laya_ext_stats(void* h, long long* out, int n) {
  if (!h || !out || n < 1) return -1;
  long long v[4];
  E(h)->stats(v);
  for (int i = 0; i < n && i < 4; i++) out[i] = v[i];
  return 0;
}

// largest K or V^T operand (bytes) of the attention kernels, whose buffer offsets are 32-bit
static constexpr size_t kMaxAttnOperandBytes = (size_t)1 << 31;

int laya_ext_attention(int dtype, const void* Q, const void* K, int ldqk, int kv_rows, const void* Vt, int ldv, void* O,
                       int ldo, const int* tiles, int ntiles, int qtile, int H, const int* soff, const int* vlen,
                       const int* gq, const int* grow, int window_half, float scale, void* stream) {
  using namespace laya;
  const int elt = dtype == 0 ? 4 : 2;
  if ((dtype != 0 && dtype != 1) || !Q || !K || !Vt || !O || !tiles || !soff || !vlen || ntiles < 0 || H < 1 ||
      kv_rows < 1 || window_half < 0 || !(scale > 0.f) || (gq == nullptr) != (grow == nullptr))
    return -1;
  // 128-query tiles: bf16, not gathered, and a window (if any) whose half width is a multiple of the
  // 64-key block; the gathered mode attends to every key of the question (no window)
  if (qtile != 64 && !(qtile == 128 && dtype == 1 && !gq && window_half % 64 == 0)) return -1;
  if (gq && window_half > 0) return -1;
  if (ldqk < H * 64 || ldo < H * 64 || ldv < 64 || (ldqk * elt) % 16 || (ldo * elt) % 16 || (ldv * elt) % 16) return -1;
  // K and V^T are read through buffer resources with 32-bit record counts and offsets
  if ((size_t)kv_rows * ldqk * elt >= kMaxAttnOperandBytes || (size_t)H * 64 * ldv * elt >= kMaxAttnOperandBytes) return -1;
  if ((reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) | reinterpret_cast<uintptr_t>(Vt) |
       reinterpret_cast<uintptr_t>(O)) & 15)
    return -1;
  hipStream_t st = (hipStream_t)stream;
  (void)hipGetLastError();
  const AttnTile* t = reinterpret_cast<const AttnTile*>(tiles);
  if (dtype == 0)
    launch_attention<float>((const float*)Q, (const float*)K, ldqk, kv_rows, (const float*)Vt, ldv, (float*)O, ldo, t,
                            ntiles, qtile, H, soff, vlen, gq, grow, window_half, scale, st);
  else
    launch_attention<bf16_t>((const bf16_t*)Q, (const bf16_t*)K, ldqk, kv_rows, (const bf16_t*)Vt, ldv, (bf16_t*)O, ldo,
                             t, ntiles, qtile, H, soff, vlen, gq, grow, window_half, scale, st);
  LAYA_HIP(hipGetLastError());
  return 0;
}
int laya_ext_gemm_ksplit(int ks, void* ws, size_t ws_bytes) {
  if (ks < 0 || ks > 64 || (ks > 1 && (!ws || ws_bytes == 0))) return -2;
  g_ext_ws = static_cast<float*>(ws);
  g_ext_ws_bytes = ws_bytes;
  return laya::gemm_pin_ksplit(ks);
}
}  // extern "C"

// ---------------------------------------------------------------- split-K GEMM without allocation
// Partial products of laya_ext_gemm_splitk_static live in this file-scope device array, one copy
// per GPU, held until the process ends.  Host code never passes the array's name to a kernel (in
// host code it is only a stand-in symbol): each device's address comes from hipGetSymbolAddress,
// taken once per device with that device current, and only that address is used.
static constexpr size_t kStaticScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];
static constexpr int kMaxDevices = 64;
static std::atomic<float*> g_scratch_ptr[kMaxDevices];

// the calling thread's current device's copy of `scratch`, or null (with the error printed)
static float* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fprintf(stderr, "[laya] laya_ext_gemm_splitk_static: no usable current device\n");
    return nullptr;
  }
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || addr == nullptr) {
      fprintf(stderr, "[laya] laya_ext_gemm_splitk_static: hipGetSymbolAddress failed: %s\n", hipGetErrorString(e));
      return nullptr;
    }
    p = static_cast<float*>(addr);
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

extern "C" {
int laya_ext_gemm_splitk_static(int epi, const void* A, const void* W, void* C, const float* bias, int act, int M,
                                int N, int K, int ksplit, void* stream) {
  using namespace laya;
  if ((epi != 0 && epi != 1) || ksplit < 2 || ksplit > 64 || act < 0 || act > 2) return -1;
  GemmArgs g;
  g.A = A; g.lda = K; g.W = W; g.ldw = K; g.M = M; g.N = N; g.K = K; g.bias = bias; g.act = act;
  if (epi == 0) { g.C = C; g.ldc = N; } else { g.X = (float*)C; g.ldx = N; }
  const char* why = "";
  const int e = epi == 0 ? EPI_STORE : EPI_RESID;
  // the split-K path of launch_gemm: the tiled kernel, K a multiple of 64 per chunk
  if (!gemm_shape_ok(e, g, 2, &why) || gemm_planned(e, g) < 0 || K % (64 * ksplit) != 0) return -1;
  // rows run in chunks whose ksplit x N fp32 partials fit the array; one row must fit
  if ((size_t)ksplit * (size_t)N * sizeof(float) > kStaticScratchBytes) {
    fprintf(stderr, "[laya] laya_ext_gemm_splitk_static: ksplit * N * 4 = %zu bytes exceeds the %zu-byte static "
                    "scratch\n", (size_t)ksplit * N * sizeof(float), kStaticScratchBytes);
    return -2;
  }
  float* ws = device_scratch();
  if (ws == nullptr) return -3;
  g.ksplit = ksplit;
  g.ws = ws;
  g.ws_bytes = kStaticScratchBytes;
  (void)hipGetLastError();
  launch_gemm<bf16_t>(e, g, (hipStream_t)stream);
  LAYA_HIP(hipGetLastError());
  return 0;
}

int laya_ext_gemm_config(int cfg) {
  if (cfg < -1 || cfg >= laya::kGemmConfigs) return -2;
  return laya::gemm_config(cfg);
}
int laya_ext_gemm_split(int split_rows, int cfg_tail) {
  if (split_rows < 0 || (split_rows > 0 && (cfg_tail < 0 || cfg_tail >= laya::kGemmConfigs))) return -2;
  laya::gemm_pin_split(split_rows, split_rows > 0 ? cfg_tail : -1);
  return 0;
}
}
