// k_quant.hip -- NF4 quantize (+ double quantization), scale decode and
// dequantize for gfx950.  All three are bit-exact restatements of
// qlora-core/src/quant.rs (quantize :104-154, nearest_nf4_code :263-278,
// double_quantize_scales :283-299, block_scales :212-221, dequantize
// :157-167).  This file is compiled with -ffp-contract=off: every f32
// operation must round where the reference rounds.
#include "qh_internal.h"
#include "qh_nf4.h"

namespace qh {
namespace {

__constant__ float c_lut17[17] = QH_NF4_LUT17_INIT;

// Decoded scale of block b (quant.rs:212-221): fp32, or
// fl(fl(i8 / 127) * absmax[b / 256]).
__device__ __forceinline__ float block_scale(const DevQW &w, int64_t b) {
  if (w.kind == 0) return w.scales[b];
  float c = (float)(int8_t)w.scale_codes[b];
  return c / 127.0f * w.absmax[b >> 8];
}

__device__ __forceinline__ float wave_max8(float v) {
  // max over the 8 consecutive lanes of a group
  v = fmaxf(v, __shfl_xor(v, 1, 8));
  v = fmaxf(v, __shfl_xor(v, 2, 8));
  v = fmaxf(v, __shfl_xor(v, 4, 8));
  return v;
}

// Super-block double quantization of the 256 (or fewer) block absmaxes held
// in `sblk`; the whole workgroup (256 threads) participates.
__device__ void dq_superblock(const float *sblk, int nhere, int64_t sb,
                              uint8_t *scale_codes, float *absmax,
                              float *red) {
  const int tid = threadIdx.x;
  float s = tid < nhere ? sblk[tid] : 0.0f;
  float a = fabsf(s);
  for (int off = 32; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
  if ((tid & 63) == 0) red[tid >> 6] = a;
  __syncthreads();
  float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (tid < nhere) {
    int32_t q = 0;
    if (amax != 0.0f) q = qh_round_clamp127(s / amax * 127.0f);
    scale_codes[sb * QH_DQ_BLOCK + tid] = (uint8_t)(int8_t)q;
  }
  if (tid == 0) absmax[sb] = amax;
}

// block_size == 64.  One workgroup per super-block of 256 blocks (16384
// elements); 8 lanes per block, 8 contiguous elements per lane, 32 blocks
// per pass, 8 passes.
__global__ __launch_bounds__(256) void k_quantize64(
    const float *__restrict__ w, int64_t n, int dq, uint8_t *__restrict__ codes,
    int64_t codes_len, float *__restrict__ scales,
    uint8_t *__restrict__ scale_codes, float *__restrict__ absmax, int64_t nb) {
  __shared__ float lut[17];
  __shared__ float sblk[256];
  __shared__ float red[4];
  const int tid = threadIdx.x;
  if (tid < 17) lut[tid] = c_lut17[tid];
  __syncthreads();
  const int64_t sb = blockIdx.x;
  const int l8 = tid & 7, grp = tid >> 3;
#pragma unroll 1
  for (int pass = 0; pass < 8; ++pass) {
    const int64_t blk = sb * 256 + pass * 32 + grp;
    const int64_t e0 = blk * 64 + l8 * 8;
    float v[8];
    if (e0 + 8 <= n) {
      const float4 *p = reinterpret_cast<const float4 *>(w + e0);
      float4 a = p[0];
      float4 b = p[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (e0 + i < n) ? w[e0 + i] : 0.0f;
    }
    // Padding with 0 leaves the fold max(0, |w|...) unchanged.
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    am = wave_max8(am);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t code = QH_NF4_ZERO_CODE;
      if (am != 0.0f) code = qh_nf4_code_of_target(v[i] / am, lut);
      if (e0 + i >= n) code = 0;
      word |= code << (4 * i);
    }
    const int64_t byte0 = e0 >> 1;
    if (byte0 + 4 <= codes_len) {
      *reinterpret_cast<uint32_t *>(codes + byte0) = word;
    } else {
      for (int i = 0; i < 4; ++i)
        if (byte0 + i < codes_len) codes[byte0 + i] = (uint8_t)(word >> (8 * i));
    }
    if (l8 == 0 && blk < nb) {
      if (dq)
        sblk[pass * 32 + grp] = am;
      else
        scales[blk] = am;
    }
  }
  if (dq) {
    __syncthreads();
    int64_t rem = nb - sb * 256;
    int nhere = rem < 256 ? (int)rem : 256;
    dq_superblock(sblk, nhere, sb, scale_codes, absmax, red);
  }
}

// Generic block size: (1) per-block absmax, (2) codes per byte, (3) DQ.
__global__ void k_block_absmax(const float *__restrict__ w, int64_t n,
                               int64_t bs, int64_t nb, float *__restrict__ out) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nb) return;
  int64_t s = b * bs, e = s + bs < n ? s + bs : n;
  float am = 0.0f;
  for (int64_t i = s; i < e; ++i) am = fmaxf(am, fabsf(w[i]));
  out[b] = am;
}

__global__ void k_codes_generic(const float *__restrict__ w, int64_t n,
                                int64_t bs, const float *__restrict__ am,
                                uint8_t *__restrict__ codes, int64_t codes_len) {
  __shared__ float lut[17];
  if (threadIdx.x < 17) lut[threadIdx.x] = c_lut17[threadIdx.x];
  __syncthreads();
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= codes_len) return;
  uint32_t byte = 0;
  for (int h = 0; h < 2; ++h) {
    int64_t e = 2 * i + h;
    if (e >= n) break;
    float a = am[e / bs];
    uint32_t code = QH_NF4_ZERO_CODE;
    if (a != 0.0f) code = qh_nf4_code_of_target(w[e] / a, lut);
    byte |= code << (4 * h);
  }
  codes[i] = (uint8_t)byte;
}

__global__ __launch_bounds__(256) void k_double_quant(
    const float *__restrict__ sc, int64_t nb, uint8_t *__restrict__ scale_codes,
    float *__restrict__ absmax) {
  __shared__ float sblk[256];
  __shared__ float red[4];
  const int64_t sb = blockIdx.x;
  int64_t rem = nb - sb * 256;
  int nhere = rem < 256 ? (int)rem : 256;
  if ((int)threadIdx.x < nhere) sblk[threadIdx.x] = sc[sb * 256 + threadIdx.x];
  __syncthreads();
  dq_superblock(sblk, nhere, sb, scale_codes, absmax, red);
}

__global__ void k_block_scales(DevQW w, float *__restrict__ out) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b < w.nb) out[b] = block_scale(w, b);
}

// One thread per 4 code bytes (8 elements).
__global__ __launch_bounds__(256) void k_dequantize(DevQW w,
                                                    float *__restrict__ out) {
  __shared__ float lut[16];
  if (threadIdx.x < 16) lut[threadIdx.x] = c_lut17[threadIdx.x];
  __syncthreads();
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t e0 = q * 8;
  if (e0 >= w.n) return;
  const int64_t codes_len = (w.n + 1) / 2;
  uint32_t word = 0;
  if (q * 4 + 4 <= codes_len) {
    word = *reinterpret_cast<const uint32_t *>(w.codes + q * 4);
  } else {
    for (int i = 0; i < 4; ++i)
      if (q * 4 + i < codes_len) word |= (uint32_t)w.codes[q * 4 + i] << (8 * i);
  }
  float v[8];
  if (w.bs % 8 == 0) {
    const float s = block_scale(w, e0 / w.bs);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = lut[(word >> (4 * i)) & 15u] * s;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int64_t e = e0 + i < w.n ? e0 + i : w.n - 1;
      v[i] = lut[(word >> (4 * i)) & 15u] * block_scale(w, e / w.bs);
    }
  }
  if (e0 + 8 <= w.n) {
    float4 *o = reinterpret_cast<float4 *>(out + e0);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    for (int i = 0; i < 8; ++i)
      if (e0 + i < w.n) out[e0 + i] = v[i];
  }
}

}  // namespace

hipError_t launch_quantize(const float *w, int64_t n, int64_t bs, int dq,
                           uint8_t *codes, float *scales, uint8_t *scale_codes,
                           float *absmax, float *scratch, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int64_t nb = (n + bs - 1) / bs;
  const int64_t codes_len = (n + 1) / 2;
  const int64_t nsb = (nb + 255) / 256;
  if (bs == 64 && (((uintptr_t)w) & 15) == 0 && (((uintptr_t)codes) & 3) == 0) {
    return qh_launch(k_quantize64, dim3((unsigned)nsb), dim3(256), 0, s, w, n, dq, codes,
                     codes_len, scales, scale_codes, absmax, nb);
  }
  float *am = dq ? scratch : scales;
  k_block_absmax<<<dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s>>>(
      w, n, bs, nb, am);
  k_codes_generic<<<dim3((unsigned)((codes_len + 255) / 256)), dim3(256), 0,
                    s>>>(w, n, bs, am, codes, codes_len);
  if (dq)
    k_double_quant<<<dim3((unsigned)nsb), dim3(256), 0, s>>>(am, nb,
                                                             scale_codes, absmax);
  return hipGetLastError();
}

hipError_t launch_block_scales(const DevQW &w, float *out, hipStream_t s) {
  if (w.nb == 0) return hipSuccess;
  k_block_scales<<<dim3((unsigned)((w.nb + 255) / 256)), dim3(256), 0, s>>>(
      w, out);
  return hipGetLastError();
}

hipError_t launch_dequantize(const DevQW &w, float *out, hipStream_t s) {
  if (w.n == 0) return hipSuccess;
  int64_t threads = (w.n + 7) / 8;
  return qh_launch(k_dequantize, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                   w, out);
}

}  // namespace qh
