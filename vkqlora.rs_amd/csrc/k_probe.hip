// k_probe.hip -- measurement kernels for the benchmark (libqh_probe.so, not
// part of the product library): what one launch of a plain streaming read
// reaches on this GPU, the ceiling the decode GEMV's weight stream is
// compared against.
//
// qh_probe_read: `groups` workgroups of `threads` threads read `bytes` of
// HBM (a multiple of 16) with 16-byte loads (non-temporal ones when `nt`),
// `unroll` of them in flight per thread, each workgroup a contiguous slice;
// every thread folds what it read into one word so the loads cannot be
// dropped, and workgroup g writes one word to sink[g].
#include <hip/hip_runtime.h>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int U, bool NT>
__global__ void k_read(const uint4 *__restrict__ src, int64_t n16, uint32_t *__restrict__ sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = per * blockIdx.x;
  const int64_t b1 = b0 + per < n16 ? b0 + per : n16;
  uint32_t acc = 0;
  int64_t i = b0 + threadIdx.x;
  for (; i + (int64_t)(U - 1) * blockDim.x < b1; i += (int64_t)U * blockDim.x) {
    u32x4 v[U];
    const u32x4 *p = (const u32x4 *)src;
#pragma unroll
    for (int u = 0; u < U; ++u)
      v[u] = NT ? __builtin_nontemporal_load(p + i + (int64_t)u * blockDim.x)
                : p[i + (int64_t)u * blockDim.x];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < b1; i += blockDim.x) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off);
  __shared__ uint32_t red[16];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) a ^= red[w];
    sink[blockIdx.x] = a;
  }
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int qh_probe_read(const void *src, size_t bytes,
                                                                    uint32_t *sink, int groups,
                                                                    int threads, int unroll,
                                                                    int nt, void *stream) {
  if (!src || !sink || groups <= 0 || threads <= 0 || threads > 1024 || threads % 64 != 0 ||
      bytes % 16 != 0)
    return (int)hipErrorInvalidValue;
  const int64_t n16 = (int64_t)(bytes / 16);
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)groups), b((unsigned)threads);
#define QH_PROBE(U)                                                                  \
  case U:                                                                            \
    if (nt)                                                                          \
      k_read<U, true><<<g, b, 0, s>>>((const uint4 *)src, n16, sink);                \
    else                                                                             \
      k_read<U, false><<<g, b, 0, s>>>((const uint4 *)src, n16, sink);               \
    break;
  switch (unroll) {
    QH_PROBE(1)
    QH_PROBE(2)
    QH_PROBE(4)
    QH_PROBE(8)
    default: return (int)hipErrorInvalidValue;
  }
#undef QH_PROBE
  return (int)hipGetLastError();
}
