// laya-parity: checks a Laya engine library against golden vectors in the reference's golden
// format, through laya_api.h only (the counterpart of the reference's src/test_parity.cpp).
//
//   laya-parity <model_dir> <golden_dir> [--prob-tol P] [--act-tol A] [--logit-tol L]
//
// <golden_dir>/manifest.json lists cases {name, shapes{...}}; each case directory holds int32
// input_ids [n, L], attention_mask [n, L], marker_pos [n, kmax], marker_mask [n, kmax], qtype [n]
// and float32 logits [n, kmax], act_logits [n, n_act] (little-endian .bin files).  Every case runs
// as one laya_forward_batch call of its n questions, twice: the first call runs eagerly (and
// captures a graph), the second replays it.  Per question it reports max |dlogit|, max |dprob| of
// the softmax over its markers and max |dact| / max(1, |act|); a question passes when dprob <= P
// (default 0.01, the reference tool's bar), dact <= A (default 0.05) and dlogit <= L (default: no
// bound), and every engine logit and act value is finite.  Exit status 0 when every question
// passes, 1 otherwise, 2 on a bad input.  `laya-parity --self-check` runs the comparison on planted
// values (NaN, Inf, out-of-bar) without an engine.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "json_lite.h"
#include "laya_api.h"

namespace {

template <typename T>
bool read_bin(const std::string& path, size_t n, std::vector<T>* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) { fprintf(stderr, "laya-parity: cannot open %s\n", path.c_str()); return false; }
  out->resize(n);
  f.read(reinterpret_cast<char*>(out->data()), (std::streamsize)(n * sizeof(T)));
  if ((size_t)f.gcount() != n * sizeof(T)) { fprintf(stderr, "laya-parity: %s is short\n", path.c_str()); return false; }
  return true;
}

size_t numel(const laya::JVal& shape) {
  size_t n = 1;
  for (const auto& d : shape.arr) n *= (size_t)d.num;
  return n;
}

void softmax(const float* z, int k, std::vector<double>* p) {
  double m = -INFINITY, s = 0.0;
  for (int i = 0; i < k; i++) m = std::max(m, (double)z[i]);
  p->assign(k, 0.0);
  for (int i = 0; i < k; i++) { (*p)[i] = std::exp((double)z[i] - m); s += (*p)[i]; }
  for (int i = 0; i < k; i++) (*p)[i] /= s;
}

// running maximum that keeps a NaN once one is seen (std::max(acc, NaN) would return acc)
double worse(double acc, double x) { return std::isnan(acc) || std::isnan(x) ? NAN : std::max(acc, x); }

struct QuestionDiff {
  double dl = 0.0, dp = 0.0, da = 0.0;
  bool finite = true;                    // every engine logit and act value is finite
};

// One question: K engine logits lo against golden gl, n_act act values against gact.
QuestionDiff compare_question(const float* lo, const float* gl, int K, const float* act, const float* gact, int n_act) {
  QuestionDiff q;
  for (int i = 0; i < K; i++) q.finite = q.finite && std::isfinite(lo[i]);
  for (int i = 0; i < n_act; i++) q.finite = q.finite && std::isfinite(act[i]);
  std::vector<double> pe, pg;
  softmax(lo, K, &pe);
  softmax(gl, K, &pg);
  for (int i = 0; i < K; i++) {
    q.dl = worse(q.dl, std::fabs((double)lo[i] - gl[i]));
    q.dp = worse(q.dp, std::fabs(pe[i] - pg[i]));
  }
  for (int i = 0; i < n_act; i++) {
    const double g = gact[i];
    q.da = worse(q.da, std::fabs(act[i] - g) / std::max(1.0, std::fabs(g)));
  }
  return q;
}

// A question passes only with finite engine outputs and every difference within its bar (a NaN
// difference compares false, so it fails too).
bool question_passes(const QuestionDiff& q, double prob_tol, double act_tol, double logit_tol) {
  return q.finite && q.dp <= prob_tol && q.da <= act_tol && q.dl <= logit_tol;
}

// --self-check: the comparison on planted values, no engine or GPU involved.  Exit 0 when a clean
// question passes and NaN, +-Inf or out-of-bar values in logits or act values each fail.
int self_check() {
  const float gl[3] = {0.1f, -0.2f, 0.3f}, ga[2] = {1.0f, -2.0f};
  auto run = [&](const float* lo, const float* act) {
    return question_passes(compare_question(lo, gl, 3, act, ga, 2), 0.01, 0.05, INFINITY);
  };
  const float ok_lo[3] = {0.1f, -0.2f, 0.3001f}, ok_act[2] = {1.0f, -2.0f};
  const float nan_lo[3] = {0.1f, NAN, 0.3f}, inf_lo[3] = {INFINITY, -0.2f, 0.3f}, ninf_lo[3] = {0.1f, -INFINITY, 0.3f};
  const float nan_act[2] = {1.0f, NAN}, inf_act[2] = {INFINITY, -2.0f}, far_lo[3] = {2.0f, -0.2f, 0.3f};
  const float far_act[2] = {1.5f, -2.0f};
  int bad = 0;
  bad += !run(ok_lo, ok_act);
  bad += run(nan_lo, ok_act);
  bad += run(inf_lo, ok_act);
  bad += run(ninf_lo, ok_act);
  bad += run(ok_lo, nan_act);
  bad += run(ok_lo, inf_act);
  bad += run(far_lo, ok_act);
  bad += run(ok_lo, far_act);
  printf("laya-parity self-check: %s\n", bad ? "FAILED" : "ok");
  return bad ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc == 2 && strcmp(argv[1], "--self-check") == 0) return self_check();
  if (argc < 3) {
    fprintf(stderr, "usage: laya-parity <model_dir> <golden_dir> [--prob-tol P] [--act-tol A] [--logit-tol L]\n");
    return 2;
  }
  const std::string model = argv[1], gold = argv[2];
  double prob_tol = 0.01, act_tol = 0.05, logit_tol = INFINITY;
  for (int i = 3; i + 1 < argc; i += 2) {
    const std::string k = argv[i];
    const double v = atof(argv[i + 1]);
    if (k == "--prob-tol") prob_tol = v;
    else if (k == "--act-tol") act_tol = v;
    else if (k == "--logit-tol") logit_tol = v;
    else { fprintf(stderr, "laya-parity: unknown option %s\n", k.c_str()); return 2; }
  }
  laya::JVal man;
  try {
    std::ifstream mf(gold + "/manifest.json");
    std::stringstream ss;
    ss << mf.rdbuf();
    man = laya::json_parse(ss.str());
  } catch (const std::exception& e) {
    fprintf(stderr, "laya-parity: %s/manifest.json: %s\n", gold.c_str(), e.what());
    return 2;
  }
  void* eng = laya_create(model.c_str());
  const int n_act = laya_n_act(eng);
  printf("%-22s %4s %5s %4s %12s %12s %12s  %s\n", "case", "q", "len", "K", "max|dlogit|", "max|dprob|", "rel|dact|",
         "result");
  int total = 0, failed = 0;
  double worst_p = 0.0, worst_l = 0.0, worst_a = 0.0;
  for (int round = 0; round < 2; round++) {
    for (const auto& c : man["cases"].arr) {
      const std::string name = c["name"].str, dir = gold + "/" + name;
      const auto& sh = c["shapes"];
      const int n = (int)sh["input_ids"].arr[0].num, L = (int)sh["input_ids"].arr[1].num;
      const int kmax = (int)sh["marker_pos"].arr[1].num;
      std::vector<int> ids, att, mpos, mmask, qt;
      std::vector<float> glog, gact;
      if (!read_bin(dir + "/input_ids.bin", numel(sh["input_ids"]), &ids) ||
          !read_bin(dir + "/attention_mask.bin", numel(sh["attention_mask"]), &att) ||
          !read_bin(dir + "/marker_pos.bin", numel(sh["marker_pos"]), &mpos) ||
          !read_bin(dir + "/marker_mask.bin", numel(sh["marker_mask"]), &mmask) ||
          !read_bin(dir + "/qtype.bin", numel(sh["qtype"]), &qt) ||
          !read_bin(dir + "/logits.bin", numel(sh["logits"]), &glog) ||
          !read_bin(dir + "/act_logits.bin", numel(sh["act_logits"]), &gact))
        return 2;
      if ((int)sh["act_logits"].arr[1].num != n_act) { fprintf(stderr, "laya-parity: n_act mismatch\n"); return 2; }
      // unpad: each question's valid tokens and markers, concatenated (the ABI's layout)
      std::vector<int> lens(n), nmark(n), flat_ids, flat_mk;
      for (int q = 0; q < n; q++) {
        for (int j = 0; j < L; j++) lens[q] += att[(size_t)q * L + j] != 0;
        for (int j = 0; j < kmax; j++) nmark[q] += mmask[(size_t)q * kmax + j] != 0;
        flat_ids.insert(flat_ids.end(), ids.begin() + (size_t)q * L, ids.begin() + (size_t)q * L + lens[q]);
        flat_mk.insert(flat_mk.end(), mpos.begin() + (size_t)q * kmax, mpos.begin() + (size_t)q * kmax + nmark[q]);
      }
      std::vector<float> logits(std::max<size_t>(1, flat_mk.size())), act((size_t)n * n_act);
      if (laya_forward_batch(eng, n, lens.data(), flat_ids.data(), nmark.data(), flat_mk.data(), qt.data(), logits.data(),
                             act.data()) != 0) {
        fprintf(stderr, "laya-parity: %s rejected by laya_forward_batch\n", name.c_str());
        return 2;
      }
      size_t off = 0;
      for (int q = 0; q < n; q++) {
        const int K = nmark[q];
        const QuestionDiff d = compare_question(logits.data() + off, glog.data() + (size_t)q * kmax, K,
                                                act.data() + (size_t)q * n_act, gact.data() + (size_t)q * n_act, n_act);
        const bool ok = question_passes(d, prob_tol, act_tol, logit_tol);
        total++;
        failed += !ok;
        worst_p = worse(worst_p, d.dp); worst_l = worse(worst_l, d.dl); worst_a = worse(worst_a, d.da);
        printf("%-22s %4d %5d %4d %12.3e %12.3e %12.3e  %s\n", (name + (round ? " (replay)" : "")).c_str(), q, lens[q], K,
               d.dl, d.dp, d.da, ok ? "pass" : (d.finite ? "FAIL" : "FAIL (non-finite output)"));
        off += K;
      }
    }
  }
  printf("%d/%d questions pass; worst dlogit %.3e, dprob %.3e, dact %.3e\n", total - failed, total, worst_l, worst_p,
         worst_a);
  return failed ? 1 : 0;
}
