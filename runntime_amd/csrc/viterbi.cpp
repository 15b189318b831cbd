// Host-side constrained Viterbi decode of the privacy filter (plain C++,
// no GPU): the best-scoring label path under start, end and transition
// scores, ties to the lower previous label and the lower last label; when no
// path is finite, the per-token argmax.
//
// Reference: src/zoo/privacy-filter/viterbi.ts:85-148 (decode), with the
// scores in f64 and the log-probabilities as f32.
#include <math.h>
#include <stdint.h>

#include <vector>

#include "../../include/runntime_moe.h"

extern "C" int moe_viterbi_decode(const double *start, const double *end, const double *trans,
                                  const float *log_probs, int T, int n, int32_t *path) {
  if (T < 0 || n < 1 || (T > 0 && (!start || !end || !trans || !log_probs || !path)))
    return MOE_INVALID_ARGUMENT;
  if (T == 0) return MOE_OK;
  std::vector<double> scores(n), next(n);
  std::vector<int32_t> back((size_t)(T > 1 ? T - 1 : 0) * n);
  for (int j = 0; j < n; j++) scores[j] = (double)log_probs[j] + start[j];
  for (int t = 1; t < T; t++) {
    for (int j = 0; j < n; j++) {
      double best = -INFINITY;
      int bi = 0;
      for (int i = 0; i < n; i++) {
        const double s = scores[i] + trans[(size_t)i * n + j];
        if (s > best) {
          best = s;
          bi = i;
        }
      }
      next[j] = best + (double)log_probs[(size_t)t * n + j];
      back[(size_t)(t - 1) * n + j] = bi;
    }
    scores.swap(next);
  }
  bool finite = false;
  for (int j = 0; j < n; j++) finite |= isfinite(scores[j]) != 0;
  if (!finite) {
    for (int t = 0; t < T; t++) {
      float best = -INFINITY;
      int bj = 0;
      for (int j = 0; j < n; j++)
        if (log_probs[(size_t)t * n + j] > best) {
          best = log_probs[(size_t)t * n + j];
          bj = j;
        }
      path[t] = bj;
    }
    return MOE_OK;
  }
  int last = 0;
  double best = -INFINITY;
  for (int j = 0; j < n; j++) {
    const double s = scores[j] + end[j];
    if (s > best) {
      best = s;
      last = j;
    }
  }
  path[T - 1] = last;
  for (int t = T - 2; t >= 0; t--) {
    last = back[(size_t)t * n + path[t + 1]];
    path[t] = last;
  }
  return MOE_OK;
}
