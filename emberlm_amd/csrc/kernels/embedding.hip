// Token embedding gather and its deterministic scatter-add backward.
//
// Reference: embedding_kernel_f32 / embedding_backward_kernel_f32
// (src/ops/embedding.cu:15-39), whose backward atomically adds every token's
// gradient row into dW[id] (order-dependent fp32 sums).  Both backward forms
// here sum each dW row in a fixed order, so it is the same on every run:
//   - with a workspace (ember_embedding_bwd_workspace_bytes): the token
//     positions are sorted by id with a stable radix sort (hipCUB), cut into
//     windows of 64 sorted entries; one workgroup per window sums each run of
//     equal ids in position order and adds it into dW when the run lies in
//     the window, or keeps it as a partial row when the run crosses a window
//     edge; a second pass adds, for every crossing run, the partials of the
//     windows it spans, in window order, into dW.  The work per token is
//     bounded however the ids repeat: a batch of one repeated id (padding)
//     spreads over n/64 workgroups instead of one serial chain.
//   - without one: each block owns kIdsPerBlock vocabulary rows, scans the id
//     list in order, compacts the positions that hit its range with a wave
//     ballot (keeping ascending order), and adds those dy rows into its dW
//     rows one after another.
#include <hipcub/hipcub.hpp>

#include "common.h"

using namespace ember;

namespace {

constexpr int kThreads = 256;
constexpr int kIdsPerBlock = 128;

template <int VEC>
__global__ __launch_bounds__(kThreads) void embedding_fwd_kernel(const int64_t* __restrict__ ids,
                                                                 const float* __restrict__ w,
                                                                 float* __restrict__ out,
                                                                 int64_t n, int64_t H, int64_t V) {
  // One block per token row (grid-stride), VEC columns per thread; ids
  // outside [0,V) give zero rows.
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
    const int64_t id = ids[r];
    const bool ok = id >= 0 && id < V;
    for (int64_t c = static_cast<int64_t>(threadIdx.x) * VEC; c < H; c += kThreads * VEC) {
      if constexpr (VEC == 4) {
        *reinterpret_cast<f32x4*>(out + r * H + c) =
            ok ? *reinterpret_cast<const f32x4*>(w + id * H + c) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        out[r * H + c] = ok ? w[id * H + c] : 0.f;
      }
    }
  }
}

__global__ __launch_bounds__(kThreads) void embedding_bwd_kernel(const int64_t* __restrict__ ids,
                                                                 const float* __restrict__ dy,
                                                                 float* __restrict__ dw, int64_t n,
                                                                 int64_t H, int64_t V) {
  __shared__ int hits[kThreads];
  __shared__ int wave_base[kThreads / kWave + 1];
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * kIdsPerBlock;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int64_t base = 0; base < n; base += kThreads) {
    const int64_t i = base + threadIdx.x;
    const int64_t id = i < n ? ids[i] : -1;
    const bool hit = id >= v0 && id < v0 + kIdsPerBlock && id < V;
    const uint64_t ballot = __ballot(hit);
    const int before = __popcll(ballot & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    if (lane == 0) wave_base[wid] = __popcll(ballot);
    __syncthreads();
    if (threadIdx.x == 0) {
      int acc = 0;
      for (int w_ = 0; w_ < kThreads / kWave; ++w_) {
        const int c = wave_base[w_];
        wave_base[w_] = acc;
        acc += c;
      }
      wave_base[kThreads / kWave] = acc;
    }
    __syncthreads();
    if (hit) hits[wave_base[wid] + before] = static_cast<int>(threadIdx.x);
    __syncthreads();
    const int nh = wave_base[kThreads / kWave];
    for (int h = 0; h < nh; ++h) {  // ascending token order
      const int64_t r = base + hits[h];
      const int64_t row = ids[r];
      for (int64_t c = threadIdx.x; c < H; c += kThreads) dw[row * H + c] += dy[r * H + c];
    }
    __syncthreads();
  }
}

// --- sorted form -----------------------------------------------------------
constexpr int kWin = 64;  // sorted entries per window

// keys = ids (out-of-range ids become V and sort last), vals = positions.
__global__ __launch_bounds__(kThreads) void emb_sort_prep(const int64_t* __restrict__ ids,
                                                          uint32_t* __restrict__ keys,
                                                          uint32_t* __restrict__ vals, int64_t n,
                                                          int64_t V) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t id = ids[i];
  keys[i] = static_cast<uint32_t>(id >= 0 && id < V ? id : V);
  vals[i] = static_cast<uint32_t>(i);
}

// Columns a thread handles at once: four (float4) when rows allow it.
template <int VEC>
struct Cols;
template <>
struct Cols<4> {
  using T = f32x4;
  static __device__ __forceinline__ T zero() { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  static __device__ __forceinline__ T load(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  }
  static __device__ __forceinline__ T get(const float* p) {
    return *reinterpret_cast<const f32x4*>(p);
  }
  static __device__ __forceinline__ void put(float* p, T v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <>
struct Cols<1> {
  using T = float;
  static __device__ __forceinline__ T zero() { return 0.f; }
  static __device__ __forceinline__ T load(const float* p) { return *p; }
  static __device__ __forceinline__ T get(const float* p) { return *p; }
  static __device__ __forceinline__ void put(float* p, T v) { *p = v; }
};

constexpr int kAhead = 8;  // dy rows a thread loads before adding them up

// Window w: the sum, in position order, of the dy rows of each run of equal
// keys among sorted entries [64w, 64w + 64).  A run that lies wholly in the
// window is added into dW[key] here (its only owner); the window's first run
// when it continues one from the window before, and its last run when it
// continues into the next window, go to part[64w + k] (the window's k-th run)
// for emb_window_combine.
template <int VEC>
__global__ __launch_bounds__(kThreads) void emb_window_sums(const uint32_t* __restrict__ keys,
                                                            const uint32_t* __restrict__ vals,
                                                            const float* __restrict__ dy,
                                                            float* __restrict__ part,
                                                            float* __restrict__ dw, int64_t n,
                                                            int64_t H, int64_t V) {
  using C = Cols<VEC>;
  __shared__ uint32_t k_s[kWin], v_s[kWin];
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kWin;
  const int cnt = static_cast<int>(n - e0 < kWin ? n - e0 : kWin);
  if (threadIdx.x < cnt) {
    k_s[threadIdx.x] = keys[e0 + threadIdx.x];
    v_s[threadIdx.x] = vals[e0 + threadIdx.x];
  }
  const uint32_t prev_key = e0 > 0 ? keys[e0 - 1] : 0xffffffffu;
  const uint32_t next_key = e0 + cnt < n ? keys[e0 + cnt] : 0xffffffffu;
  __syncthreads();
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * VEC; c < H; c += kThreads * VEC) {
    typename C::T acc = C::zero();
    int k = 0;
    for (int b = 0; b < cnt; b += kAhead) {
      typename C::T row[kAhead];
#pragma unroll
      for (int i = 0; i < kAhead; ++i)
        row[i] = b + i < cnt && k_s[b + i] < V
                     ? C::load(dy + static_cast<int64_t>(v_s[b + i]) * H + c)
                     : C::zero();
#pragma unroll
      for (int i = 0; i < kAhead; ++i) {
        const int e = b + i;
        if (e >= cnt) break;
        const uint32_t key = k_s[e];
        if (key >= V) break;  // invalid ids sort last
        acc += row[i];
        if (e + 1 == cnt || k_s[e + 1] != key) {
          const bool spans = (k == 0 && prev_key == key) || (e + 1 == cnt && next_key == key);
          if (spans) {
            C::put(part + (e0 + k) * H + c, acc);
          } else {
            float* d = dw + static_cast<int64_t>(key) * H + c;
            C::put(d, C::get(d) + acc);
          }
          acc = C::zero();
          ++k;
        }
      }
    }
  }
}

// Window w: if its last run starts in it (not a continuation of the previous
// window's last run) and continues into the next window, dW[key] += its
// partial + the partials of the following windows the run continues into, in
// window order.  Every other run was added by emb_window_sums.
template <int VEC>
__global__ __launch_bounds__(kThreads) void emb_window_combine(const uint32_t* __restrict__ keys,
                                                               const float* __restrict__ part,
                                                               float* __restrict__ dw, int64_t n,
                                                               int64_t H, int64_t V) {
  using C = Cols<VEC>;
  const int64_t nwin = (n + kWin - 1) / kWin;
  const int64_t w = blockIdx.x;
  const int64_t e0 = w * kWin;
  const int cnt = static_cast<int>(n - e0 < kWin ? n - e0 : kWin);
  if (e0 + cnt >= n) return;  // the last window: nothing continues past it
  const uint32_t key = keys[e0 + cnt - 1];
  if (key >= V || keys[e0 + cnt] != key) return;
  // the run's first entry in this window, and the window's number of runs
  // before it (its part slot)
  int first = cnt - 1;
  while (first > 0 && keys[e0 + first - 1] == key) --first;
  if (first == 0 && w > 0 && keys[e0 - 1] == key) return;  // owned by an earlier window
  int k = 0;
  for (int e = 1; e <= first; ++e) k += keys[e0 + e] != keys[e0 + e - 1];
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * VEC; c < H; c += kThreads * VEC) {
    typename C::T t = C::get(part + (e0 + k) * H + c);
    for (int64_t w2 = w + 1; w2 < nwin; ++w2) {
      const int64_t f = w2 * kWin;
      if (keys[f] != key) break;
      t += C::get(part + f * H + c);  // the continuation is window w2's first run
      const int64_t fend = f + kWin < n ? f + kWin : n;
      if (keys[fend - 1] != key) break;  // the run ends inside window w2
    }
    float* d = dw + static_cast<int64_t>(key) * H + c;
    C::put(d, C::get(d) + t);
  }
}

int emb_key_bits(int64_t V) {
  int b = 1;
  while ((int64_t{1} << b) <= V) ++b;  // keys run up to V (invalid ids)
  return b;
}

size_t emb_sort_temp_bytes(int64_t n, int64_t V) {
  size_t b = 0;
  const hipError_t e = hipcub::DeviceRadixSort::SortPairs(
      nullptr, b, static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
      static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr), static_cast<int>(n),
      0, emb_key_bits(V));
  return e == hipSuccess ? b : 0;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

}  // namespace

extern "C" int ember_embedding_fwd(const int64_t* ids, const float* w, float* out, int64_t n,
                                   int64_t H, int64_t V, ember_stream_t s) {
  if (n < 0 || H <= 0 || V <= 0) return EMBER_EINVAL;
  if (n == 0) return EMBER_OK;
  if (!ids || !w || !out) return EMBER_EINVAL;
  const unsigned g = static_cast<unsigned>(n < 65536 * 4 ? n : 65536 * 4);
  if (H % 4 == 0 && aligned16(w) && aligned16(out))
    embedding_fwd_kernel<4><<<g, kThreads, 0, as_stream(s)>>>(ids, w, out, n, H, V);
  else
    embedding_fwd_kernel<1><<<g, kThreads, 0, as_stream(s)>>>(ids, w, out, n, H, V);
  return launch_status();
}

extern "C" size_t ember_embedding_bwd_workspace_bytes(int64_t n, int64_t H, int64_t V) {
  if (n <= 0 || H <= 0 || V <= 0 || n > 0x7fffffff || V >= 0x7fffffff) return 0;
  const size_t temp = emb_sort_temp_bytes(n, V);
  if (!temp) return 0;
  return 4 * align256(static_cast<size_t>(n) * 4) + align256(static_cast<size_t>(n * H) * 4) +
         align256(temp);
}

extern "C" int ember_embedding_bwd(const int64_t* ids, const float* dy, float* dw, int64_t n,
                                   int64_t H, int64_t V, int accumulate, void* workspace,
                                   size_t workspace_bytes, ember_stream_t s) {
  if (n < 0 || H <= 0 || V <= 0 || !dw) return EMBER_EINVAL;
  if (n > 0 && (!ids || !dy)) return EMBER_EINVAL;
  if (!accumulate) {
    const int rc = ember_fill(dw, V * H, 0.f, s);
    if (rc) return rc;
  }
  if (n == 0) return EMBER_OK;
  hipStream_t st = as_stream(s);
  const size_t need = workspace ? ember_embedding_bwd_workspace_bytes(n, H, V) : 0;
  if (need && workspace_bytes >= need) {
    char* p = static_cast<char*>(workspace);
    const size_t keyb = align256(static_cast<size_t>(n) * 4);
    uint32_t* keys_in = reinterpret_cast<uint32_t*>(p);
    uint32_t* vals_in = reinterpret_cast<uint32_t*>(p + keyb);
    uint32_t* keys = reinterpret_cast<uint32_t*>(p + 2 * keyb);
    uint32_t* vals = reinterpret_cast<uint32_t*>(p + 3 * keyb);
    float* part = reinterpret_cast<float*>(p + 4 * keyb);
    char* temp = p + 4 * keyb + align256(static_cast<size_t>(n * H) * 4);
    size_t temp_bytes = need - 4 * keyb - align256(static_cast<size_t>(n * H) * 4);
    emb_sort_prep<<<static_cast<unsigned>((n + kThreads - 1) / kThreads), kThreads, 0, st>>>(
        ids, keys_in, vals_in, n, V);
    int rc = launch_status();
    if (rc) return rc;
    rc = status_of(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys_in, keys, vals_in,
                                                      vals, static_cast<int>(n), 0,
                                                      emb_key_bits(V), st));
    if (rc) return rc;
    const unsigned nwin = static_cast<unsigned>((n + kWin - 1) / kWin);
    if (H % 4 == 0 && aligned16(dy) && aligned16(dw)) {
      emb_window_sums<4><<<nwin, kThreads, 0, st>>>(keys, vals, dy, part, dw, n, H, V);
      if ((rc = launch_status())) return rc;
      emb_window_combine<4><<<nwin, kThreads, 0, st>>>(keys, part, dw, n, H, V);
    } else {
      emb_window_sums<1><<<nwin, kThreads, 0, st>>>(keys, vals, dy, part, dw, n, H, V);
      if ((rc = launch_status())) return rc;
      emb_window_combine<1><<<nwin, kThreads, 0, st>>>(keys, part, dw, n, H, V);
    }
    return launch_status();
  }
  const int64_t nb = (V + kIdsPerBlock - 1) / kIdsPerBlock;
  if (nb > 0x7fffffff) return EMBER_EINVAL;
  embedding_bwd_kernel<<<static_cast<unsigned>(nb), kThreads, 0, st>>>(ids, dy, dw, n, H, V);
  return launch_status();
}
