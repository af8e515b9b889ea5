// Token sampling.  Reference: src/core/sampling.cpp:10-113.
//
// The draw is defined by its steps, so a seed gives the reference's tokens:
// logits * (1/T) in float; top-k keeps values >= the k-th largest; softmax
// with float exp(x - max), a double sum and a float reciprocal; top-p keeps the
// most probable tokens (descending, std::sort order) until their double
// cumulative sum reaches p and renormalises; then one
// uniform_real_distribution<double>(0, 1) draw walks the double CDF in index
// order (the last index if rounding leaves the draw above the total).
#include "ctd/sampling.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>
#include <stdexcept>

#include "ctd/runtime.h"
#include "ember_hip.h"

namespace ctd {

namespace {

int64_t host_argmax(const float* x, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

// Keeps the values >= the k-th largest (ties at the threshold all stay).
void keep_top_k(std::vector<float>& z, int k) {
  std::vector<float> sorted(z);
  std::nth_element(sorted.begin(), sorted.begin() + (k - 1), sorted.end(), std::greater<float>());
  const float thresh = sorted[k - 1];
  for (float& x : z)
    if (x < thresh) x = -std::numeric_limits<float>::infinity();
}

void softmax(std::vector<float>& z) {
  const float mx = *std::max_element(z.begin(), z.end());
  double total = 0.0;
  for (float& x : z) {
    x = std::exp(x - mx);
    total += x;
  }
  const float inv = static_cast<float>(1.0 / total);
  for (float& x : z) x *= inv;
}

void keep_top_p(std::vector<float>& p, float top_p) {
  const int64_t V = static_cast<int64_t>(p.size());
  std::vector<int64_t> order(V);
  std::iota(order.begin(), order.end(), int64_t{0});
  std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return p[a] > p[b]; });
  std::vector<char> kept(V, 0);
  double cum = 0.0;
  for (int64_t r = 0; r < V; ++r) {
    cum += p[order[r]];
    kept[order[r]] = 1;
    if (cum >= top_p) break;
  }
  double total = 0.0;
  for (int64_t i = 0; i < V; ++i) {
    if (!kept[i]) p[i] = 0.0f;
    total += p[i];
  }
  if (total > 0.0) {
    const float inv = static_cast<float>(1.0 / total);
    for (float& x : p) x *= inv;
  }
}

}  // namespace

int64_t sample_row(const float* logits, int64_t V, const SamplerConfig& cfg,
                   std::mt19937_64& rng) {
  if (V <= 0) throw std::runtime_error("sample: empty vocabulary");
  if (cfg.temperature <= 0.0f) return host_argmax(logits, V);
  std::vector<float> z(logits, logits + V);
  const float inv_t = 1.0f / cfg.temperature;
  for (float& x : z) x *= inv_t;
  if (cfg.top_k > 0 && cfg.top_k < V) keep_top_k(z, cfg.top_k);
  softmax(z);
  if (cfg.top_p > 0.0f && cfg.top_p < 1.0f) keep_top_p(z, cfg.top_p);
  std::uniform_real_distribution<double> unif(0.0, 1.0);
  const double u = unif(rng);
  double cdf = 0.0;
  for (int64_t i = 0; i < V; ++i) {
    cdf += z[i];
    if (u < cdf) return i;
  }
  return V - 1;
}

std::vector<int64_t> sample(const Tensor& logits_last, const SamplerConfig& cfg,
                            std::mt19937_64& rng) {
  if (logits_last.dtype() != DType::kFloat32)
    throw std::runtime_error("sample: fp32 logits only");
  if (logits_last.dim() != 3 || logits_last.shape()[1] != 1)
    throw std::runtime_error("sample: expected logits shape [B, 1, V]");
  if (!logits_last.is_contiguous()) throw std::runtime_error("sample: logits must be contiguous");
  const int64_t B = logits_last.shape()[0];
  const int64_t V = logits_last.shape()[2];
  std::vector<int64_t> out(B);
  if (B == 0) return out;
  if (V <= 0) throw std::runtime_error("sample: empty vocabulary");
  if (cfg.temperature <= 0.0f && logits_last.device().is_hip()) {
    Tensor idx = Tensor::empty({B}, DType::kInt64, logits_last.device());
    const size_t wsb = ember_argmax_rows_workspace_bytes(B, V);
    Tensor ws = wsb ? Tensor::empty({static_cast<int64_t>((wsb + 7) / 8)}, DType::kInt64,
                                    logits_last.device())
                    : Tensor{};
    CTD_CHECK(ember_argmax_rows_ws(static_cast<const float*>(logits_last.data_ptr()), B, V,
                                   static_cast<int64_t*>(idx.data_ptr()),
                                   wsb ? ws.data_ptr() : nullptr, wsb,
                                   runtime::compute_stream()));
    idx.copy_to_host(out.data());
    return out;
  }
  std::vector<float> host(static_cast<size_t>(B * V));
  logits_last.copy_to_host(host.data());
  for (int64_t b = 0; b < B; ++b) out[b] = sample_row(host.data() + b * V, V, cfg, rng);
  return out;
}

}  // namespace ctd
