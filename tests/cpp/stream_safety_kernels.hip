// stream_safety_kernels.hip -- TEST SUPPORT: the device side of the allocator
// stream-safety race test (test_stream_safety.cpp), the MI355X counterpart of the
// reference's tests/test_stream_safety.cu kernels.
//
//   ss_fill_f32        buf[i] = v (grid-stride);
//   ss_gated_read_f32  one workgroup: lane 0 polls a host-written flag (bounded:
//                      it gives up after kMaxPolls polls, so the kernel always
//                      finishes even if the host never releases it), then every
//                      lane counts elements != 1.0f; reads are agent-scope atomic
//                      loads, so they see what other CUs / XCDs wrote after this
//                      kernel started, not a stale cached copy;
//   ss_gate_*          the flag: pinned, mapped, coherent host memory.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kMaxPolls = 2000000;   // ~seconds of polling at most, then give up

__global__ void ss_fill_kernel(float* __restrict__ buf, int n, float v) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += blockDim.x * gridDim.x) buf[i] = v;
}

__global__ void ss_gated_read_kernel(const float* buf, int n, const int* gate, unsigned* bad_out,
                                     int* gate_seen_out) {
  __shared__ int seen;
  if (threadIdx.x == 0) {
    int g = 0;
    for (int p = 0; p < kMaxPolls; ++p) {
      g = __hip_atomic_load(gate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (g != 0) break;
      __builtin_amdgcn_s_sleep(2);
    }
    seen = g;
    *gate_seen_out = g;
  }
  __syncthreads();
  unsigned bad = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = __hip_atomic_load(buf + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v != 1.0f) ++bad;
  }
  if (bad) atomicAdd(bad_out, bad);
  (void)seen;
}

}  // namespace

extern "C" {

int ss_fill_f32(float* buf, int n, float v, void* stream) {
  ss_fill_kernel<<<256, 256, 0, static_cast<hipStream_t>(stream)>>>(buf, n, v);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

int ss_gated_read_f32(const float* buf, int n, const int* gate_dev, unsigned* bad_out,
                      int* gate_seen_out, void* stream) {
  ss_gated_read_kernel<<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(buf, n, gate_dev, bad_out,
                                                                       gate_seen_out);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

int ss_gate_create(int** host_ptr, int** dev_ptr) {
  void* h = nullptr;
  if (hipHostMalloc(&h, sizeof(int), hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) return 1;
  *static_cast<volatile int*>(h) = 0;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
    (void)hipHostFree(h);
    return 1;
  }
  *host_ptr = static_cast<int*>(h);
  *dev_ptr = static_cast<int*>(d);
  return 0;
}

int ss_gate_destroy(int* host_ptr) { return hipHostFree(host_ptr) == hipSuccess ? 0 : 1; }

}  // extern "C"
