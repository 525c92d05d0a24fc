// Route-history retention policy of the slot cache (host code).
//
// Observable behaviour, as the reference's RouteCachePolicy
// (runtime/deepseek_v4_ssd/route_cache.py:12-120) defines it:
//  - per (layer, expert), two decayed decode routing rates with half-lives of 16 and 256
//    of that layer's tokens: a token routed to the expert adds 1 - 2^(-1/h) at its own age,
//    so an expert routed every token approaches rate 1;
//  - the current prompt's routing counts per prompt token form a prior of weight 0.1 that
//    fades as 2^(-t/32) with the request's decode tokens t;
//  - a per-layer expert read cost (first sample, then a running mean of weight 0.05),
//    taken relative to the median sampled layer and clipped to [0.5, 2] (unsampled layers
//    count as the median);
//  - retention score = (0.75 short + 0.25 long + prior) * relative cost;
//  - the cache's slots are split over layers by marginal value: every layer's scores sorted
//    in descending order are its values for a first, second, ... slot, and the capacity
//    goes to the largest values overall, equal values to the lower rank, then the lower
//    layer;
//  - rebalanced every 16 * layers decode tokens, when a prefill ends, and on demand.
//
// Mechanics of this implementation:
//  - rates are stored lazily against a per-layer time base b: A_h[l][e] holds
//    sum over routed tokens tau of (1 - 2^(-1/h)) 2^((tau - b) / h), and the rate at the
//    layer's token count n is A_h 2^(-(n - b) / h). A routed token therefore costs O(1)
//    instead of decaying every expert of the layer; the rates are materialised only when
//    the scores are rebuilt, and the base moves forward before 2^((n - b) / 16) nears the
//    top of the double range;
//  - the quota split selects the capacity-th key with nth_element over all (layer, rank)
//    keys (linear time) instead of popping a heap once per slot.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <stdexcept>
#include <vector>

namespace wm {

class RoutePolicy {
 public:
  static constexpr double kShortHalfLife = 16.0, kLongHalfLife = 256.0;
  static constexpr int kRebalanceTokens = 16;     // per layer
  static constexpr double kPriorWeight = 0.1, kPriorFadeTokens = 32.0;
  static constexpr double kReadCostStep = 0.05;
  static constexpr double kShortShare = 0.75, kLongShare = 0.25;
  static constexpr double kRebaseExponent = 600.0;  // 2^600 << DBL_MAX

  RoutePolicy(int layers, int experts, int slots, int top_k)
      : L_(layers), E_(experts), k_(top_k), capacity_(std::min<int64_t>(slots, (int64_t)layers * experts)) {
    if (layers < 1 || experts < 1 || slots < 1 || top_k < 1 || top_k > experts)
      throw std::runtime_error("route policy: invalid dimensions");
    const size_t n = (size_t)layers * experts;
    acc_short_.assign(n, 0.0);
    acc_long_.assign(n, 0.0);
    prompt_.assign(n, 0.0);
    score_.assign(n, 0.0);
    base_.assign(layers, 0);
    decode_.assign(layers, 0);
    request_decode_.assign(layers, 0);
    prompt_tokens_.assign(layers, 0);
    cost_.assign(layers, 0.0);
    cost_samples_.assign(layers, 0);
    quota_.assign(layers, 0);
    rebalance();
  }

  // A new prompt: its routes become the prior; the decode history is kept.
  void begin_request() {
    std::fill(prompt_.begin(), prompt_.end(), 0.0);
    std::fill(prompt_tokens_.begin(), prompt_tokens_.end(), 0);
    std::fill(request_decode_.begin(), request_decode_.end(), 0);
  }

  // Routes of `layer`, token-major with top_k ids per token (the last token may be short).
  // Returns true when the observation triggered a rebalance.
  bool observe(int layer, const int32_t* ids, int64_t n, bool prefill) {
    if (layer < 0 || layer >= L_) throw std::runtime_error("route policy: layer out of range");
    for (int64_t i = 0; i < n; ++i)
      if (ids[i] < 0 || ids[i] >= E_) throw std::runtime_error("route policy: routed expert outside the model");
    if (n == 0) return false;
    const int64_t tokens = (n + k_ - 1) / k_;
    double* prompt = &prompt_[(size_t)layer * E_];
    if (prefill) {
      for (int64_t i = 0; i < n; ++i) prompt[ids[i]] += 1.0;
      prompt_tokens_[layer] += tokens;
      return false;
    }
    const int64_t first = decode_[layer] + 1;  // time of the batch's first token
    decode_[layer] += tokens;
    request_decode_[layer] += tokens;
    if ((double)(decode_[layer] - base_[layer]) / kShortHalfLife > kRebaseExponent) rebase(layer);
    const double add_s = 1.0 - std::exp2(-1.0 / kShortHalfLife), add_l = 1.0 - std::exp2(-1.0 / kLongHalfLife);
    double* as = &acc_short_[(size_t)layer * E_];
    double* al = &acc_long_[(size_t)layer * E_];
    for (int64_t i = 0; i < n; ++i) {
      const double rel = (double)(first + i / k_ - base_[layer]);
      as[ids[i]] += add_s * std::exp2(rel / kShortHalfLife);
      al[ids[i]] += add_l * std::exp2(rel / kLongHalfLife);
    }
    const int64_t total = std::accumulate(decode_.begin(), decode_.end(), (int64_t)0);
    if (total - last_rebalance_ >= (int64_t)kRebalanceTokens * L_) {
      last_rebalance_ = total;
      rebalance();
      return true;
    }
    return false;
  }

  void record_read(int layer, double seconds) {
    if (layer < 0 || layer >= L_) throw std::runtime_error("route policy: layer out of range");
    if (!std::isfinite(seconds) || seconds <= 0.0) return;
    cost_[layer] = cost_samples_[layer] == 0 ? seconds : cost_[layer] + kReadCostStep * (seconds - cost_[layer]);
    ++cost_samples_[layer];
  }

  void rebalance() {
    // relative read cost per layer
    std::vector<double> sampled;
    for (int l = 0; l < L_; ++l)
      if (cost_samples_[l] > 0) sampled.push_back(cost_[l]);
    double typical = 1.0;
    if (!sampled.empty()) {
      std::sort(sampled.begin(), sampled.end());
      const size_t m = sampled.size();
      typical = m % 2 ? sampled[m / 2] : 0.5 * (sampled[m / 2 - 1] + sampled[m / 2]);
    }
    for (int l = 0; l < L_; ++l) {
      const double c = cost_samples_[l] > 0 ? cost_[l] : typical;
      const double relative = std::min(2.0, std::max(0.5, c / std::max(typical, 1e-9)));
      const double prior = kPriorWeight * std::exp2(-(double)request_decode_[l] / kPriorFadeTokens) /
                           (double)std::max<int64_t>(prompt_tokens_[l], 1);
      for (int e = 0; e < E_; ++e) {
        const size_t i = (size_t)l * E_ + e;
        score_[i] = (kShortShare * rate(l, e, false) + kLongShare * rate(l, e, true) + prior * prompt_[i]) * relative;
      }
    }
    split_quotas();
    ++rebalances_;
  }

  // The decayed rate of (layer, expert) at the layer's current token count.
  double rate(int l, int e, bool long_rate) const {
    const double h = long_rate ? kLongHalfLife : kShortHalfLife;
    const double a = (long_rate ? acc_long_ : acc_short_)[(size_t)l * E_ + e];
    return a == 0.0 ? 0.0 : a * std::exp2(-(double)(decode_[l] - base_[l]) / h);
  }

  const std::vector<double>& scores() const { return score_; }
  const std::vector<int32_t>& quotas() const { return quota_; }
  int64_t decode_tokens(int l) const { return decode_[l]; }
  int64_t prompt_tokens(int l) const { return prompt_tokens_[l]; }
  double read_cost(int l) const { return cost_[l]; }
  int64_t rebalances() const { return rebalances_; }
  int64_t capacity() const { return capacity_; }

 private:
  void rebase(int l) {
    const double shift = (double)(decode_[l] - base_[l]);
    const double fs = std::exp2(-shift / kShortHalfLife), fl = std::exp2(-shift / kLongHalfLife);
    for (int e = 0; e < E_; ++e) {
      acc_short_[(size_t)l * E_ + e] *= fs;
      acc_long_[(size_t)l * E_ + e] *= fl;
    }
    base_[l] = decode_[l];
  }

  // Slots per layer by marginal value (see the file comment).
  void split_quotas() {
    std::vector<double> sorted(score_);
    for (int l = 0; l < L_; ++l)
      std::sort(sorted.begin() + (size_t)l * E_, sorted.begin() + (size_t)(l + 1) * E_, std::greater<double>());
    std::fill(quota_.begin(), quota_.end(), 0);
    const int64_t n = (int64_t)L_ * E_;
    if (capacity_ >= n) {
      std::fill(quota_.begin(), quota_.end(), E_);
      return;
    }
    // key (l, r) = value sorted[l][r]; earlier = larger value, then lower rank, then lower layer
    std::vector<int32_t> keys(n);
    for (int64_t i = 0; i < n; ++i) keys[i] = (int32_t)i;
    auto earlier = [&](int32_t a, int32_t b) {
      const double va = sorted[a], vb = sorted[b];
      if (va != vb) return va > vb;
      const int ra = a % E_, rb = b % E_;
      if (ra != rb) return ra < rb;
      return a / E_ < b / E_;
    };
    std::nth_element(keys.begin(), keys.begin() + capacity_, keys.end(), earlier);
    for (int64_t i = 0; i < capacity_; ++i) ++quota_[keys[i] / E_];
  }

  int L_, E_, k_;
  int64_t capacity_;
  std::vector<double> acc_short_, acc_long_, prompt_, score_;
  std::vector<int64_t> base_, decode_, request_decode_, prompt_tokens_;
  std::vector<double> cost_;
  std::vector<int64_t> cost_samples_;
  std::vector<int32_t> quota_;
  int64_t last_rebalance_ = 0, rebalances_ = 0;
};

}  // namespace wm
