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

__constant__ QhNf4Buckets c_buckets = qh_nf4_make_buckets();


// 1 / (double)a for a finite a > 0 within 2^-51 (relative): the hardware
// reciprocal (within 2^-23) and two Newton steps, each squaring the error.
__device__ __forceinline__ double inv_f64(float a) {
  const double d = (double)a;
  double y = __builtin_amdgcn_rcp(d);
  y = __builtin_fma(__builtin_fma(-d, y, 1.0), y, y);
  y = __builtin_fma(__builtin_fma(-d, y, 1.0), y, y);
  return y;
}

// block_size == 64.  One workgroup per super-block of 256 blocks (16384
// elements); 8 lanes per block, 8 contiguous elements per lane, 32 blocks
// per pass, 8 passes, every pass's loads issued before the first is used
// (measured: 213 us at 28672 x 8192 against 262 us for persistent
// workgroups that reload each pass's registers with the next super-block).
// The target t = fl(w / absmax) is the double product of w with the block's
// reciprocal rounded to float: the IEEE quotient bit for bit when t is a
// normal float (an exact quotient of two floats lies at least 2^-49
// relative from every float midpoint; the product is within 2^-51), and
// any subnormal t is nearest to level 0 (code 7) whatever its last bits.
// |t| <= 1 (the absmax bounds |w|), so the bucketed search applies: one LDS
// byte (the bucket's c0) and one 16-byte LDS read (L[c0 .. c0 + 2]).
__global__ __launch_bounds__(256) void k_quantize64(
    const float *__restrict__ w, int64_t n, int dq, uint8_t *__restrict__ codes,
    int64_t codes_len, float *__restrict__ scales,
    uint8_t *__restrict__ scale_codes, float *__restrict__ absmax, int64_t nb) {
  __shared__ __align__(16) uint8_t bkt[QH_NF4_BUCKETS];
  __shared__ __align__(16) float lq[16][4];  // L[c], L[c+1], L[c+2], unused
  __shared__ float sblk[256];
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t sb = blockIdx.x;
  const int l8 = tid & 7, grp = tid >> 3;
  // every pass's data first: 16 float4 per lane in flight
  float4 va[8], vb[8];
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {
    const int64_t e0 = (sb * 256 + pass * 32 + grp) * 64 + l8 * 8;
    if (e0 + 8 <= n) {
      const float4 *p = reinterpret_cast<const float4 *>(w + e0);
      va[pass] = p[0];
      vb[pass] = p[1];
    } else {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (e0 + i < n) ? w[e0 + i] : 0.0f;
      va[pass] = make_float4(v[0], v[1], v[2], v[3]);
      vb[pass] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  reinterpret_cast<uint4 *>(bkt)[tid] = reinterpret_cast<const uint4 *>(c_buckets.c0)[tid];
  if (tid < 16)
    *reinterpret_cast<float4 *>(lq[tid]) =
        make_float4(qh_nf4_levels[tid], qh_nf4_levels[tid + 1], qh_nf4_levels[tid + 2], 0.0f);
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {
    const int64_t blk = sb * 256 + pass * 32 + grp;
    const int64_t e0 = blk * 64 + l8 * 8;
    const float v[8] = {va[pass].x, va[pass].y, va[pass].z, va[pass].w,
                        vb[pass].x, vb[pass].y, vb[pass].z, vb[pass].w};
    // Padding with 0 leaves the fold max(0, |w|...) unchanged.
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    am = wave_max8(am);
    // w / inf is 0 (NaN for inf / inf): a zero reciprocal gives both
    const double inv = __builtin_isinf(am) ? 0.0 : inv_f64(am != 0.0f ? am : 1.0f);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float t = (float)((double)v[i] * inv);
      const uint32_t c0 = bkt[qh_nf4_bucket(t)];
      const float4 L = *reinterpret_cast<const float4 *>(lq[c0]);
      uint32_t code = qh_nf4_code_bucketed(t, c0, L.x, L.y, L.z);
      if (am == 0.0f) code = QH_NF4_ZERO_CODE;
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
