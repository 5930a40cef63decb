// Measurement probes: an empty kernel (the per-launch floor of dependent
// launches) and a plain streaming read of device memory (what a launch that
// only reads B bytes takes).  Benchmarks time them in the same harness as the
// GEMVs, so a GEMV's time can be stated against what any launch of its size
// can reach.  They compute nothing the hot path uses.
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

constexpr int kProbeThreads = 256;

size_t probe_read_wgs(size_t bytes, int per_thread) {
  const size_t per_wg = static_cast<size_t>(kProbeThreads) * 16 * per_thread;
  return (bytes + per_wg - 1) / per_wg;
}

__global__ __launch_bounds__(kProbeThreads) void probe_empty_kernel() {}

// U 16-byte loads per thread, all issued before the first add; a workgroup
// covers U * 4 KB.  Raw buffer loads with the streaming (nontemporal) hint,
// as the GEMVs load their weights: of the forms measured for a 7.1 MB read
// from HBM in a graph of dependent launches (global or buffer loads, every
// combination of the cache-policy bits, 64-1024 threads, 1-16 loads per
// thread) this is the fastest (3.02 us at 8 loads per thread against 3.26 us
// for buffer loads without the hint and 3.42 us for global loads).  Every
// loaded float is summed and one f32 per workgroup is stored, so no load can
// be dropped; offsets past `bytes` read 0 (hardware range check).
template <int U>
__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const void *__restrict__ src, uint32_t bytes,
                                                                   float *__restrict__ out) {
  const auto rs = make_rsrc(src, bytes);
  const uint32_t base = (blockIdx.x * static_cast<uint32_t>(kProbeThreads * U) + threadIdx.x) * 16u;
  uint4 v[U];
#pragma unroll
  for (int u = 0; u < U; u++) v[u] = buf_load16<kAuxNT>(rs, base + static_cast<uint32_t>(u * kProbeThreads) * 16u);
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < U; u++)
    s += (__uint_as_float(v[u].x) + __uint_as_float(v[u].y)) + (__uint_as_float(v[u].z) + __uint_as_float(v[u].w));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  __shared__ float part[kProbeThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

template <int U>
hipError_t read_u(const void *src, size_t bytes, float *out, hipStream_t st) {
  const size_t wgs = probe_read_wgs(bytes, U);
  hipLaunchKernelGGL(probe_read_kernel<U>, dim3(static_cast<unsigned>(wgs)), dim3(kProbeThreads), 0, st, src,
                     static_cast<uint32_t>(bytes), out);
  return hipGetLastError();
}

}  // namespace

size_t probe_read_workgroups(size_t bytes, int per_thread) { return probe_read_wgs(bytes, per_thread); }

hipError_t launch_probe_empty(int wgs, hipStream_t st) {
  hipLaunchKernelGGL(probe_empty_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kProbeThreads), 0, st);
  return hipGetLastError();
}

hipError_t launch_probe_read(const void *src, size_t bytes, int per_thread, float *out, hipStream_t st) {
  if (bytes >= (size_t{1} << 31)) return hipErrorInvalidValue;  // 32-bit buffer offsets
  switch (per_thread) {
    case 1: return read_u<1>(src, bytes, out, st);
    case 2: return read_u<2>(src, bytes, out, st);
    case 4: return read_u<4>(src, bytes, out, st);
    case 8: return read_u<8>(src, bytes, out, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace lgh
