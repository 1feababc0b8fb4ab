// k_adam.hip -- paged 8-bit block-wise Adam step for gfx950.
//
// Bit-exact restatement of qlora-core/src/optim.rs:206-248 (step_param) with
// quantize_block_i8 / dequant_block_i8 (:84-100).  Compiled with
// -ffp-contract=off; sqrt and division are IEEE (correctly rounded).
// The host computes b1t = 1 - beta1^t and b2t = 1 - beta2^t with the same
// libm powf the reference calls and passes them in.
//
// One workgroup per state block (all tensors of one step in one launch):
// dequantize m and v, update p, stage the new m and v in LDS, reduce the
// block absmax, requantize.  16 B of HBM traffic per element.
#include "qh_internal.h"
#include "qh_nf4.h"

namespace qh {
namespace {

constexpr int kMaxTensors = 24;
struct AdamBatch {
  AdamTensor t[kMaxTensors];
  int n;
};

__device__ __forceinline__ float deq_i8(uint8_t c, float absmax) {
  return (float)(int8_t)c / 127.0f * absmax;
}

__device__ float block_max(float v, float *red) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, red[i]);
  return r;
}

__global__ __launch_bounds__(256) void k_adam(AdamBatch B, int64_t first_block,
                                              int64_t bs, float lr, float beta1,
                                              float beta2, float eps) {
  extern __shared__ float smem[];  // m[bs], v[bs]
  __shared__ float red[8];
  const int64_t gb = first_block + blockIdx.x;
  int ti = 0;
  while (ti + 1 < B.n && B.t[ti + 1].block_offset <= gb) ++ti;
  const AdamTensor &T = B.t[ti];
  const int64_t b = gb - T.block_offset;
  const int64_t s = b * bs;
  const int64_t len = (s + bs < T.numel ? s + bs : T.numel) - s;
  float *sm = smem, *sv = smem + bs;
  const float ms = T.m_scales[b], vs = T.v_scales[b];
  const float one_m_b1 = 1.0f - beta1, one_m_b2 = 1.0f - beta2;
  float am = 0.0f, av = 0.0f;
  for (int64_t j = threadIdx.x; j < len; j += blockDim.x) {
    const float gj = T.g[s + j];
    float m = deq_i8(T.m_codes[s + j], ms);
    float v = deq_i8(T.v_codes[s + j], vs);
    m = beta1 * m + one_m_b1 * gj;
    const float var = beta2 * v * v + one_m_b2 * gj * gj;
    v = sqrtf(var);
    const float mh = m / T.b1t;
    const float vh = var / T.b2t;
    T.p[s + j] = T.p[s + j] - lr * mh / (sqrtf(vh) + eps);
    sm[j] = m;
    sv[j] = v;
    am = fmaxf(am, fabsf(m));
    av = fmaxf(av, fabsf(v));
  }
  am = block_max(am, red);
  av = block_max(av, red + 4);
  for (int64_t j = threadIdx.x; j < len; j += blockDim.x) {
    int32_t qm = 0, qv = 0;
    if (am != 0.0f) qm = qh_round_clamp127(sm[j] / am * 127.0f);
    if (av != 0.0f) qv = qh_round_clamp127(sv[j] / av * 127.0f);
    T.m_codes[s + j] = (uint8_t)(int8_t)qm;
    T.v_codes[s + j] = (uint8_t)(int8_t)qv;
  }
  if (threadIdx.x == 0) {
    T.m_scales[b] = am;
    T.v_scales[b] = av;
  }
}

}  // namespace

hipError_t launch_adam(const AdamTensor *tensors, int ntensors,
                       int64_t total_blocks, int64_t block_size, float lr,
                       float beta1, float beta2, float eps, hipStream_t s) {
  (void)total_blocks;
  const size_t shmem = (size_t)block_size * 2 * sizeof(float);
  for (int i0 = 0; i0 < ntensors; i0 += kMaxTensors) {
    AdamBatch B;
    B.n = ntensors - i0 < kMaxTensors ? ntensors - i0 : kMaxTensors;
    int64_t blocks = 0;
    for (int i = 0; i < B.n; ++i) {
      B.t[i] = tensors[i0 + i];
      B.t[i].block_offset = blocks;
      blocks += B.t[i].nblocks;
    }
    if (blocks == 0) continue;
    for (int64_t b0 = 0; b0 < blocks; b0 += 65535) {
      int64_t nbk = blocks - b0 < 65535 ? blocks - b0 : 65535;
      hipError_t e = qh_launch(k_adam, dim3((unsigned)nbk), dim3(256), (uint32_t)shmem, s,
                               B, b0, block_size, lr, beta1, beta2, eps);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

}  // namespace qh
