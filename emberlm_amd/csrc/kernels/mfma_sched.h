#pragma once
// Instruction scheduling and wait helpers shared by the MFMA kernels that
// stage their operands through LDS with DMA loads (gemm.hip, attention.hip).
#include <hip/hip_runtime.h>

namespace ember {

// Schedules NM MFMAs of the current region with NX instructions of class
// `mask` spread evenly among them (0x100 LDS read, 0x200 LDS write, 0x020 VMEM
// read, 0x008 MFMA).
// The same with each group's MFMAs first: groups of (up to) two MFMAs, then
// one NX instruction, so the reads are issued early in the region and the
// region's first MFMAs wait only for reads issued before it (the compiler's
// wait for LDS results is lgkmcnt(0): a read placed ahead of them would be
// waited for too).  0.5-0.7% faster on the 256-row tiles' slab 0.
template <int NX, int NM, int MASK>
__device__ __forceinline__ void interleave_mfma_first() {
  constexpr int per = NM / NX >= 2 ? 2 : 1;
#pragma unroll
  for (int t = 0; t < NX; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, per, 0);
    __builtin_amdgcn_sched_group_barrier(MASK, 1, 0);
  }
  if (NM > NX * per) __builtin_amdgcn_sched_group_barrier(0x008, NM - NX * per, 0);
}

template <int NX, int NM, int MASK>
__device__ __forceinline__ void interleave() {
  constexpr int per = NM / NX > 0 ? NM / NX : 1;
#pragma unroll
  for (int t = 0; t < NX; ++t) {
    __builtin_amdgcn_sched_group_barrier(MASK, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, per, 0);
  }
  if (NM > NX * per) __builtin_amdgcn_sched_group_barrier(0x008, NM - NX * per, 0);
}

// s_waitcnt with vmcnt <= N (loads still in flight: the newest N) and
// lgkmcnt = 0; expcnt left alone.  gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4, lgkmcnt 11:8.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
}
// Workgroup barrier with no implied memory wait (the waits above are explicit);
// the empty asm keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// NR LDS reads (mask 0x100) and NV VMEM loads (0x020) spread evenly among
// NM MFMAs of the current region.
template <int NR, int NV, int NM>
__device__ __forceinline__ void interleave2() {
  constexpr int per = NM / (NR + NV) > 0 ? NM / (NR + NV) : 1;
  constexpr int n = NR > NV ? NR : NV;
#pragma unroll
  for (int t = 0; t < n; ++t) {
    if (t < NR) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, per, 0);
    }
    if (t < NV) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, per, 0);
    }
  }
  if (NM > (NR + NV) * per) __builtin_amdgcn_sched_group_barrier(0x008, NM - (NR + NV) * per, 0);
}

}  // namespace ember
