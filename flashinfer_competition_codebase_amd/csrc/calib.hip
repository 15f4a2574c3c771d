// calib.hip - reference kernels for bench.py's floor measurements on gfx950.
//
// Not part of the decode step.  These kernels move the same bytes as a
// decode step's state stream with nothing else, so the benchmark can report
// how far the decode kernel sits from the practical floor of its traffic:
//   * gdn_calib_rmw: in-place read-modify-write of an fp32 buffer (x *= c),
//     read once and written once, 16 floats per thread as four coalesced
//     128-bit accesses, 128 threads (8 KiB) per workgroup -- the decode
//     kernel's workgroup size and bytes per workgroup at small batch;
//   * gdn_calib_empty: a kernel that does nothing, on the same grid: the
//     dispatch-and-retire floor the timers see.
// Both take optional hipEvent_t stamps (hipExtLaunchKernelGGL) so the elapsed
// time is the kernel's own duration.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn_calib {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 128;
constexpr int kFloatsPerThread = 16;
constexpr long long kFloatsPerBlock = kThreads * kFloatsPerThread;  // 8 KiB

// Chunk i of a workgroup's 8 KiB is read by its 128 threads as 128
// consecutive 16-byte vectors, so every access instruction covers 2 KiB of
// contiguous memory.
template <bool NT>
__global__ __launch_bounds__(kThreads) void rmw(float* buf, float c) {
  f32x4* p = reinterpret_cast<f32x4*>(buf + static_cast<long long>(blockIdx.x) * kFloatsPerBlock) +
             threadIdx.x;
  f32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v[i] = NT ? __builtin_nontemporal_load(p + i * kThreads) : p[i * kThreads];
  // All four loads in flight before the first wait (left to itself the
  // scheduler waits on the first pair before issuing the second: two
  // memory round trips instead of one).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] *= c;
    if constexpr (NT) {
      __builtin_nontemporal_store(v[i], p + i * kThreads);
    } else {
      p[i * kThreads] = v[i];
    }
  }
}

__global__ __launch_bounds__(kThreads) void empty() {}

}  // namespace gdn_calib

extern "C" {

// In-place buf[i] *= c over n_floats floats (a multiple of 2048, buf 16-byte
// aligned), nontemporal (1) or ordinary (0) accesses.  Returns a hipError_t.
int gdn_calib_rmw(float* buf, long long n_floats, float c, int nontemporal,
                  void* start_event, void* stop_event, void* hip_stream) {
  using namespace gdn_calib;
  if (!buf || n_floats <= 0 || n_floats % kFloatsPerBlock != 0 ||
      (reinterpret_cast<uintptr_t>(buf) & 15) != 0 || (nontemporal != 0 && nontemporal != 1))
    return hipErrorInvalidValue;
  const long long blocks = n_floats / kFloatsPerBlock;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  auto* kern = nontemporal ? rmw<true> : rmw<false>;
  hipExtLaunchKernelGGL(kern, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                        static_cast<hipStream_t>(hip_stream),
                        static_cast<hipEvent_t>(start_event),
                        static_cast<hipEvent_t>(stop_event), 0, buf, c);
  return hipGetLastError();
}

// An empty kernel on `blocks` workgroups of 128 threads.
int gdn_calib_empty(long long blocks, void* start_event, void* stop_event,
                    void* hip_stream) {
  using namespace gdn_calib;
  if (blocks <= 0 || blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipExtLaunchKernelGGL(empty, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                        static_cast<hipStream_t>(hip_stream),
                        static_cast<hipEvent_t>(start_event),
                        static_cast<hipEvent_t>(stop_event), 0);
  return hipGetLastError();
}

}  // extern "C"
