// Runtime half of the C ABI: memory, copies, streams, events, seeded fills.
#include <cstring>
#include <mutex>

#include "common.h"

using namespace ember;

namespace ember {

namespace {
struct Staging {
  std::mutex mu;
  void* host = nullptr;
  size_t cap = 0;
  hipEvent_t copied = nullptr;
};
Staging& staging() {
  static Staging* s = new Staging();  // lives as long as the process
  return *s;
}
}  // namespace

int upload_async(void* dev_dst, const void* host_src, size_t bytes, hipStream_t st) {
  if (bytes == 0) return EMBER_OK;
  if (!dev_dst || !host_src) return EMBER_EINVAL;
  Staging& sg = staging();
  std::lock_guard<std::mutex> lk(sg.mu);
  hipError_t e = hipSuccess;
  if (sg.copied) {
    e = hipEventSynchronize(sg.copied);  // the previous table has left the buffer
  } else {
    e = hipEventCreateWithFlags(&sg.copied, hipEventDisableTiming);
  }
  if (e != hipSuccess) return status_of(e);
  if (sg.cap < bytes) {
    if (sg.host) (void)hipHostFree(sg.host);
    sg.host = nullptr;
    sg.cap = 0;
    if ((e = hipHostMalloc(&sg.host, bytes)) != hipSuccess) return status_of(e);
    sg.cap = bytes;
  }
  std::memcpy(sg.host, host_src, bytes);
  e = hipMemcpyAsync(dev_dst, sg.host, bytes, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipEventRecord(sg.copied, st);
  return status_of(e);
}

}  // namespace ember

extern "C" const char* ember_status_string(int status) {
  switch (status) {
    case EMBER_OK: return "ok";
    case EMBER_EINVAL: return "invalid argument";
    case EMBER_EWORKSPACE: return "workspace missing or too small";
    case EMBER_EALIGN: return "pointer alignment not met";
    case EMBER_EMASKSUM: return "sum(loss_mask) == 0 in cross-entropy backward";
    case EMBER_ESCRATCH: return "problem larger than the entry point's fixed scratch";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

extern "C" int ember_get_device_count(int* count) {
  if (!count) return EMBER_EINVAL;
  return status_of(hipGetDeviceCount(count));
}
extern "C" int ember_set_device(int device) { return status_of(hipSetDevice(device)); }
extern "C" int ember_get_device(int* device) {
  if (!device) return EMBER_EINVAL;
  return status_of(hipGetDevice(device));
}

extern "C" int ember_device_malloc(void** ptr, size_t bytes) {
  if (!ptr) return EMBER_EINVAL;
  *ptr = nullptr;
  if (bytes == 0) return EMBER_OK;
  return status_of(hipMalloc(ptr, bytes));
}
extern "C" int ember_device_free(void* ptr) { return ptr ? status_of(hipFree(ptr)) : EMBER_OK; }

extern "C" int ember_host_malloc_pinned(void** ptr, size_t bytes) {
  if (!ptr) return EMBER_EINVAL;
  *ptr = nullptr;
  if (bytes == 0) return EMBER_OK;
  return status_of(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}
extern "C" int ember_host_free_pinned(void* ptr) {
  return ptr ? status_of(hipHostFree(ptr)) : EMBER_OK;
}

static bool kind_of(int kind, hipMemcpyKind* k) {
  switch (kind) {
    case 0: *k = hipMemcpyHostToDevice; return true;
    case 1: *k = hipMemcpyDeviceToHost; return true;
    case 2: *k = hipMemcpyDeviceToDevice; return true;
    case 3: *k = hipMemcpyHostToHost; return true;
    default: return false;
  }
}

extern "C" int ember_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                                  ember_stream_t s) {
  hipMemcpyKind k;
  if (!kind_of(kind, &k)) return EMBER_EINVAL;
  if (bytes == 0) return EMBER_OK;
  if (!dst || !src) return EMBER_EINVAL;
  return status_of(hipMemcpyAsync(dst, src, bytes, k, as_stream(s)));
}

extern "C" int ember_memcpy(void* dst, const void* src, size_t bytes, int kind) {
  hipMemcpyKind k;
  if (!kind_of(kind, &k)) return EMBER_EINVAL;
  if (bytes == 0) return EMBER_OK;
  if (!dst || !src) return EMBER_EINVAL;
  return status_of(hipMemcpy(dst, src, bytes, k));
}

extern "C" int ember_mem_get_info(size_t* free_bytes, size_t* total_bytes) {
  if (!free_bytes || !total_bytes) return EMBER_EINVAL;
  return status_of(hipMemGetInfo(free_bytes, total_bytes));
}

extern "C" int ember_device_synchronize(void) { return status_of(hipDeviceSynchronize()); }

extern "C" int ember_stream_create(ember_stream_t* s) {
  if (!s) return EMBER_EINVAL;
  hipStream_t st = nullptr;
  int rc = status_of(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  *s = reinterpret_cast<ember_stream_t>(st);
  return rc;
}
extern "C" int ember_stream_destroy(ember_stream_t s) {
  return s ? status_of(hipStreamDestroy(as_stream(s))) : EMBER_OK;
}
extern "C" int ember_stream_synchronize(ember_stream_t s) {
  return status_of(hipStreamSynchronize(as_stream(s)));
}

extern "C" int ember_event_create(ember_event_t* e) {
  if (!e) return EMBER_EINVAL;
  hipEvent_t ev = nullptr;
  int rc = status_of(hipEventCreate(&ev));
  *e = reinterpret_cast<ember_event_t>(ev);
  return rc;
}
extern "C" int ember_event_destroy(ember_event_t e) {
  return e ? status_of(hipEventDestroy(reinterpret_cast<hipEvent_t>(e))) : EMBER_OK;
}
extern "C" int ember_event_record(ember_event_t e, ember_stream_t s) {
  if (!e) return EMBER_EINVAL;
  return status_of(hipEventRecord(reinterpret_cast<hipEvent_t>(e), as_stream(s)));
}
extern "C" int ember_event_synchronize(ember_event_t e) {
  if (!e) return EMBER_EINVAL;
  return status_of(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e)));
}
extern "C" int ember_event_query(ember_event_t e) {
  if (!e) return EMBER_EINVAL;
  const hipError_t rc = hipEventQuery(reinterpret_cast<hipEvent_t>(e));
  if (rc == hipErrorNotReady) return EMBER_NOTREADY;
  return status_of(rc);
}
extern "C" int ember_stream_wait_event(ember_stream_t s, ember_event_t e) {
  if (!e) return EMBER_EINVAL;
  return status_of(hipStreamWaitEvent(as_stream(s), reinterpret_cast<hipEvent_t>(e), 0));
}
extern "C" int ember_event_elapsed_ms(float* ms, ember_event_t start, ember_event_t stop) {
  if (!ms || !start || !stop) return EMBER_EINVAL;
  return status_of(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                       reinterpret_cast<hipEvent_t>(stop)));
}

extern "C" int ember_device_info(char* name, size_t name_cap, int* cu_count, size_t* hbm_bytes) {
  int dev = 0;
  int rc = status_of(hipGetDevice(&dev));
  if (rc) return rc;
  hipDeviceProp_t prop;
  rc = status_of(hipGetDeviceProperties(&prop, dev));
  if (rc) return rc;
  if (name && name_cap) {
    std::strncpy(name, prop.gcnArchName, name_cap - 1);
    name[name_cap - 1] = '\0';
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
  return EMBER_OK;
}

// ----------------------------------------------------------------- fills
namespace {

// SplitMix64 finaliser: a bijective mix of the counter (Steele et al. 2014).
__host__ __device__ inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Element i: two 32-bit uniforms from one 64-bit draw, Box-Muller cosine branch.
__global__ void fill_normal_kernel(float* __restrict__ p, int64_t n, uint64_t seed,
                                   uint64_t offset, float mean, float stddev) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    const uint64_t r = splitmix64(seed * 0xD1B54A32D192ED03ull + offset + static_cast<uint64_t>(i));
    const double u1 = (static_cast<double>(r >> 40) + 1.0) * (1.0 / 16777217.0);  // (0,1]
    const double u2 = static_cast<double>(r & 0xFFFFFFull) * (1.0 / 16777216.0);   // [0,1)
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    p[i] = mean + stddev * static_cast<float>(z);
  }
}

__global__ void fill_kernel(float* __restrict__ p, int64_t n, float value) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = value;
}

}  // namespace

extern "C" int ember_fill_normal(float* p, int64_t n, uint64_t seed, uint64_t offset, float mean,
                                 float stddev, ember_stream_t s) {
  if (n < 0 || (n > 0 && !p)) return EMBER_EINVAL;
  if (n == 0) return EMBER_OK;
  fill_normal_kernel<<<grid_1d(n, 256, 65536), 256, 0, as_stream(s)>>>(p, n, seed, offset, mean,
                                                                       stddev);
  return launch_status();
}

extern "C" int ember_fill(float* p, int64_t n, float value, ember_stream_t s) {
  if (n < 0 || (n > 0 && !p)) return EMBER_EINVAL;
  if (n == 0) return EMBER_OK;
  fill_kernel<<<grid_1d(n, 256, 65536), 256, 0, as_stream(s)>>>(p, n, value);
  return launch_status();
}
