// laya-bench: wall-clock latency of laya_forward_batch through laya_api.h (the counterpart of the
// reference's src/bench_engine.cpp), host packing, copies and synchronisation included.
//
//   laya-bench <model_dir> [--tune-all] [--iters N]
//
// Prints the p50 over N calls (default 30; 15 for the batched table), after three untimed calls of
// the same shape, for one question of 64 .. 1024 tokens (up to the model's max_len) and for
// 1, 2, 4, 8, 16, 32 questions of 256 tokens.  Every question has 5 options at positions 5 + 4k
// and deterministic token ids.  With --tune-all it first times laya_tune_all.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "laya_api.h"

namespace {

using Clock = std::chrono::steady_clock;

double p50_ms(void* eng, int len, int B, int iters, int n_act) {
  std::vector<int> lens(B, len), nmark(B, 5), qt(B, 1), ids((size_t)B * len), mk((size_t)B * 5);
  for (size_t i = 0; i < ids.size(); i++) ids[i] = 1000 + (int)((i * 2654435761u) % 40000u);
  for (int b = 0; b < B; b++)
    for (int k = 0; k < 5; k++) mk[(size_t)b * 5 + k] = std::min(len - 1, 5 + 4 * k);
  std::vector<float> logits((size_t)B * 5), act((size_t)B * n_act);
  auto call = [&] {
    if (laya_forward_batch(eng, B, lens.data(), ids.data(), nmark.data(), mk.data(), qt.data(), logits.data(),
                           act.data()) != 0) {
      fprintf(stderr, "laya-bench: call rejected (len %d, B %d)\n", len, B);
      exit(1);
    }
  };
  for (int i = 0; i < 3; i++) call();
  std::vector<double> t(iters);
  for (int i = 0; i < iters; i++) {
    const auto a = Clock::now();
    call();
    t[i] = std::chrono::duration<double, std::milli>(Clock::now() - a).count();
  }
  std::sort(t.begin(), t.end());
  return t[iters / 2];
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: laya-bench <model_dir> [--tune-all] [--iters N]\n");
    return 2;
  }
  bool tune = false;
  int iters = 30;
  for (int i = 2; i < argc; i++) {
    if (!strcmp(argv[i], "--tune-all")) tune = true;
    else if (!strcmp(argv[i], "--iters") && i + 1 < argc) iters = std::max(1, atoi(argv[++i]));
    else { fprintf(stderr, "laya-bench: unknown option %s\n", argv[i]); return 2; }
  }
  void* eng = laya_create(argv[1]);
  const int max_len = laya_max_len(eng), n_act = laya_n_act(eng);
  if (tune) {
    const auto a = Clock::now();
    laya_tune_all(eng);
    printf("laya_tune_all: %.2f s\n", std::chrono::duration<double>(Clock::now() - a).count());
  }
  printf("\none question\n%-8s %10s %10s\n", "tokens", "p50_ms", "q/s");
  for (int len : {64, 128, 256, 384, 512, 768, 1024}) {
    if (len > max_len) break;
    const double m = p50_ms(eng, len, 1, iters, n_act);
    printf("%-8d %10.3f %10.1f\n", len, m, 1000.0 / m);
  }
  const int blen = std::min(256, max_len);
  printf("\nbatched, %d tokens per question\n%-8s %10s %10s %12s\n", blen, "questions", "p50_ms", "q/s", "ms/question");
  for (int B : {1, 2, 4, 8, 16, 32}) {
    const double m = p50_ms(eng, blen, B, std::max(1, iters / 2), n_act);
    printf("%-8d %10.3f %10.1f %12.3f\n", B, m, 1000.0 * B / m, m / B);
  }
  fflush(stdout);
  return 0;
}
