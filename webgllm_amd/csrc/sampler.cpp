// The host sampler over a pick's candidates (the reference's createSampler,
// draw and drawAt, src/sampler.ts:27-242): top-k by a
// min-heap of slots, top-p over a stable descending order, min-p, then the
// temperature, in llama.cpp's order, with the reference's float32 stores
// (Float32Array) and double arithmetic (JavaScript numbers) in between, so
// a given uniform draw picks the reference's token.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "status.h"

namespace {

// Whether slot a holds less than slot b, ties to the lower slot (sampler.ts:147-149).
inline bool below(const std::vector<float> &kept, int a, int b) {
  return kept[a] < kept[b] || (kept[a] == kept[b] && a < b);
}

// Indices of the positive weights, largest first, ties in index order
// (descending, sampler.ts:157-185: a stable order on the weights' bits).
std::vector<int> descending(const std::vector<float> &w) {
  std::vector<int> order;
  for (int j = 0; j < (int)w.size(); j++)
    if (w[j] > 0.0f) order.push_back(j);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
    uint32_t ba, bb;
    memcpy(&ba, &w[a], 4);
    memcpy(&bb, &w[b], 4);
    return ba > bb;  // positive floats order as their bits
  });
  return order;
}

}  // namespace

extern "C" {

int wg_sample_distribution(const wg_sampling *s, const float *logits, const int32_t *ids_in,
                           int32_t n, int32_t *ids_out, float *p_out, int32_t *n_out) {
  WG_REQUIRE(s && logits && ids_out && p_out && n_out && n >= 1,
             "wg_sample_distribution: bad arguments");
  const int k = std::max(1, std::min(s->top_k > 0 ? s->top_k : n, n));
  std::vector<int> kept_ids(k);
  std::vector<float> kept(k);
  if (k >= n) {
    for (int i = 0; i < k; i++) {
      kept_ids[i] = ids_in ? ids_in[i] : i;
      kept[i] = logits[i];
    }
  } else {
    // The k largest: replace the smallest kept when beaten; a min-heap of
    // slots finds it, ties to the lowest slot.
    std::fill(kept.begin(), kept.end(), -INFINITY);
    std::vector<int> heap(k);
    for (int j = 0; j < k; j++) heap[j] = j;
    for (int i = 0; i < n; i++) {
      const float x = logits[i];
      const int slot = heap[0];
      if (!(x > kept[slot])) continue;
      kept[slot] = x;
      kept_ids[slot] = ids_in ? ids_in[i] : i;
      int at = 0;
      for (;;) {
        int child = 2 * at + 1;
        if (child >= k) break;
        const int right = child + 1;
        if (right < k && below(kept, heap[right], heap[child])) child = right;
        if (!below(kept, heap[child], slot)) break;
        heap[at] = heap[child];
        at = child;
      }
      heap[at] = slot;
    }
  }
  int best = 0;
  for (int j = 1; j < k; j++)
    if (kept[j] > kept[best]) best = j;
  if (s->temperature <= 0.0) {
    ids_out[0] = kept_ids[best];
    p_out[0] = 1.0f;
    *n_out = 1;
    return WG_OK;
  }
  const double max = kept[best];
  std::vector<float> weight(k);
  double total = 0;
  for (int j = 0; j < k; j++) {
    weight[j] = (float)exp((double)kept[j] - max);
    total += weight[j];
  }
  if (s->top_p < 1.0) {
    const std::vector<int> order = descending(weight);
    double share = 0;
    bool cut = false;
    for (int j : order) {
      if (cut) {
        weight[j] = 0.0f;
      } else {
        share += (double)weight[j] / total;
        cut = share >= s->top_p;
      }
    }
  }
  if (s->min_p > 0.0)
    for (int j = 0; j < k; j++)
      if ((double)weight[j] < s->min_p) weight[j] = 0.0f;
  double left = 0;
  for (int j = 0; j < k; j++) {
    kept[j] = weight[j] > 0.0f ? (float)exp(((double)kept[j] - max) / s->temperature) : 0.0f;
    left += kept[j];
  }
  for (int j = 0; j < k; j++) {
    ids_out[j] = kept_ids[j];
    p_out[j] = (float)((double)kept[j] / left);
  }
  *n_out = k;
  return WG_OK;
}

int32_t wg_sample_draw(const int32_t *ids, const float *p, int32_t n, double u) {
  if (!ids || !p || n < 1) return -1;
  double left = u;
  int best = 0;
  for (int j = 0; j < n; j++) {
    if (p[j] > p[best]) best = j;
    left -= p[j];
    if (left <= 0 && p[j] > 0) return ids[j];
  }
  return ids[best];
}

int32_t wg_sample_draw_at(const int32_t *ids, const float *p, int32_t n, double u) {
  if (!ids || !p || n < 1) return -1;
  std::vector<int> order(n);
  for (int j = 0; j < n; j++) order[j] = j;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return ids[a] < ids[b]; });
  double left = u;
  int best = order[0];
  for (int k = 0; k < n; k++) {
    const int j = order[k];
    if (p[j] > p[best]) best = j;
    left -= p[j];
    if (left < 0 && p[j] > 0) return ids[j];
  }
  return ids[best];
}

}  // extern "C"
