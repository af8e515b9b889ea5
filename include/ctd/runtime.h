#pragma once
// Device runtime glue over the C ABI (include/ember_hip.h): error checking,
// the compute stream every op is enqueued on, and the copy streams used by
// the offloaded optimizer.  Replaces the reference's cuda_utils.h /
// cublas_utils.h (CTD_CUDA_CHECK*, the call_once cuBLAS handle).

#include <string>
#include <vector>

#include "ctd/storage.h"
#include "ember_hip.h"

namespace ctd::runtime {

// Throws std::runtime_error("<what>: <status text>") when status != 0.
void check(int status, const char* what);

// Process-wide streams, created on first use at the default priority.
ember_stream_t compute_stream();
ember_stream_t h2d_stream();
ember_stream_t d2h_stream();

// Blocks until all work on the compute stream is done.
void synchronize();

// Makes the compute stream wait for the storage's pending writer event (see
// Storage::set_ready_event) and clears it.
void wait_ready(Storage& s);

// Keeps `keep` alive until `done` has completed, then drops the references
// (their device blocks return to the cache).  Used for buffers that a side
// stream still reads after their owner let go of them, e.g. gradients the
// offloaded optimizer consumes while zero_grad() has already released them.
// Pending entries are checked on every device allocation.
void release_after(ember_event_t done, std::vector<StoragePtr> keep);
// Drops every pending entry whose event has completed; returns how many remain.
size_t collect_released();
// Waits for every pending entry's event and drops them all.
void drain_released();
// Waits for the oldest pending entry's event and drops it; false when none
// is pending.
bool wait_oldest_released();

// Whether a HIP device is present (without creating a context on failure).
bool device_available();

// GEMM timing for the roofline figure: while enabled, the ops layer brackets
// every GEMM launch with HIP events on the compute stream.
void gemm_profile_enable(bool on);
bool gemm_profiling();
void* gemm_profile_begin();                     // null when disabled
// variant of the launch: 2*transa + transb for a GEMM (which kernel
// instantiation ran), kProfileAttnFwd / kProfileAttnBwd for fused attention.
void gemm_profile_end(void* begin, double flops, int variant);
// The same for a launch sized on the device: its flops are flops_per_row times
// clamp(*count - base, 0, max_rows), the count read when the record is collected.
void gemm_profile_end_rows(void* begin, double flops_per_row, const int64_t* count,
                           int64_t base, int64_t max_rows, int variant);
constexpr int kProfileAttnFwd = 4;
constexpr int kProfileAttnBwd = 5;
constexpr int kProfileVariants = 6;
// Resolves the recorded events (synchronises) and resets the record; the
// arrays have kProfileVariants entries, one per variant.
void gemm_profile_collect(int64_t* launches, double* flops, double* total_ms);

}  // namespace ctd::runtime

#define CTD_CHECK(expr) ::ctd::runtime::check((expr), #expr)
