// k_gemv.hip -- decode-shaped fused NF4 dequant-GEMV for gfx950.
//
// Replaces, for small batches, the reference forward's dequant dispatch +
// mm_nt (qlora-wgpu/src/kernels.rs:281-282, shaders/gemm.wgsl:68-98) and its
// LoRA branch (kernels.rs:284-294):
//
//   y[m][n] = sum_b s_{n,b} * (sum_{k in b} x[m][k] * L[code_{n,k}])
//           + s * sum_j t1[m][j] * B[n][j]
//
// HBM-bound on the packed weight stream: every code byte is read once, with
// the per-block scale hoisted out of the inner product (one multiply per
// 16 elements instead of one per element).  A workgroup owns R weight rows
// and spreads their K range over all 256 threads, so each thread reuses the
// x values it loaded for all R rows.
#include "qh_internal.h"
#include "qh_nf4.h"

namespace qh {
namespace {

__constant__ float c_lut[17] = QH_NF4_LUT17_INIT;

__device__ __forceinline__ float bf16f(uint32_t h) { return __uint_as_float(h << 16); }

template <int M>
__device__ __forceinline__ void load_x16(const void *x, int x_bf16, int64_t K,
                                         int64_t k, float (&xv)[M][16]) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (!x_bf16) {
      const float4 *p = (const float4 *)((const float *)x + m * K + k);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float4 t = p[q];
        xv[m][4 * q + 0] = t.x; xv[m][4 * q + 1] = t.y;
        xv[m][4 * q + 2] = t.z; xv[m][4 * q + 3] = t.w;
      }
    } else {
      const uint4 *p = (const uint4 *)((const uint16_t *)x + m * K + k);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint4 t = p[q];
        uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xv[m][8 * q + 2 * i] = bf16f(u[i] & 0xffffu);
          xv[m][8 * q + 2 * i + 1] = bf16f(u[i] >> 16);
        }
      }
    }
  }
}

template <int M, int R>
__global__ __launch_bounds__(256) void k_gemv(DevQW w, const void *__restrict__ x,
                                              int x_bf16,
                                              const float *__restrict__ t1,
                                              const float *__restrict__ lb,
                                              int r, float s, float *__restrict__ y) {
  __shared__ float lut[16];
  __shared__ float red[4][M * R];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < 16) lut[tid] = c_lut[tid];
  __syncthreads();

  const int64_t N = w.rows, K = w.cols;
  const int64_t n0 = (int64_t)blockIdx.x * R;
  const int64_t nch = K >> 4;  // 16-element chunks per row
  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int rr = 0; rr < R; ++rr) acc[m][rr] = 0.0f;

  for (int64_t c = tid; c < nch; c += 256) {
    const int64_t k = c << 4;
    uint2 code[R];
    float sc[R];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const int64_t n = n0 + rr < N ? n0 + rr : N - 1;
      const int64_t e = n * K + k;
      code[rr] = *(const uint2 *)(w.codes + (e >> 1));
      const int64_t b = e >> 6;
      if (w.kind == 0) {
        sc[rr] = w.scales[b];
      } else {
        sc[rr] = (float)(int8_t)w.scale_codes[b] / 127.0f * w.absmax[b >> 8];
      }
    }
    float xv[M][16];
    load_x16<M>(x, x_bf16, K, k, xv);
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      float lv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        lv[e] = lut[((e < 8 ? code[rr].x : code[rr].y) >> (4 * (e & 7))) & 15u];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float p = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) p = fmaf(xv[m][e], lv[e], p);
        acc[m][rr] = fmaf(p, sc[rr], acc[m][rr]);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      float v = acc[m][rr];
      for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
      if (lane == 0) red[wave][m * R + rr] = v;
    }
  __syncthreads();
  if (tid < M * R) {
    const int m = tid / R, rr = tid % R;
    const int64_t n = n0 + rr;
    if (n < N) {
      float base = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
      if (r > 0) {
        float l = 0.0f;
        for (int j = 0; j < r; ++j) l += t1[m * r + j] * lb[n * r + j];
        base += s * l;
      }
      y[m * N + n] = base;
    }
  }
}

// out[m][j] = sum_k x[m][k] * a[j][k]: one workgroup per (m, j).
__global__ __launch_bounds__(256) void k_dot_rows(const void *__restrict__ x, int x_bf16,
                                                  const float *__restrict__ a,
                                                  int64_t K, int r,
                                                  float *__restrict__ out) {
  __shared__ float red[4];
  const int j = blockIdx.x, m = blockIdx.y;
  float acc = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    float xv = x_bf16 ? bf16f(((const uint16_t *)x)[m * K + k])
                      : ((const float *)x)[m * K + k];
    acc = fmaf(xv, a[(int64_t)j * K + k], acc);
  }
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[m * r + j] = (red[0] + red[1]) + (red[2] + red[3]);
}

template <int M>
hipError_t run_gemv(const DevQW &w, const void *x, int x_bf16, const float *t1,
                    const float *lb, int64_t r, float s, float *y,
                    hipStream_t st) {
  constexpr int R = 4;
  dim3 grid((unsigned)((w.rows + R - 1) / R));
  k_gemv<M, R><<<grid, dim3(256), 0, st>>>(w, x, x_bf16, t1, lb, (int)r, s, y);
  return hipGetLastError();
}

}  // namespace

bool gemv_ok(const DevQW &w, int64_t M) {
  return M >= 1 && M <= 4 && w.bs == 64 && w.cols % 64 == 0;
}

hipError_t launch_dot_rows(const void *x, int x_bf16, const float *a,
                           int64_t M, int64_t K, int64_t r, float *out,
                           hipStream_t st) {
  if (M == 0 || r == 0) return hipSuccess;
  k_dot_rows<<<dim3((unsigned)r, (unsigned)M), dim3(256), 0, st>>>(x, x_bf16, a, K,
                                                                   (int)r, out);
  return hipGetLastError();
}

hipError_t launch_gemv(const DevQW &w, const void *x, int x_bf16, int64_t M,
                       const float *t1, const float *lb, int64_t r, float s,
                       float *y, hipStream_t st) {
  if (w.rows == 0) return hipSuccess;
  switch (M) {
    case 1: return run_gemv<1>(w, x, x_bf16, t1, lb, r, s, y, st);
    case 2: return run_gemv<2>(w, x, x_bf16, t1, lb, r, s, y, st);
    case 3: return run_gemv<3>(w, x, x_bf16, t1, lb, r, s, y, st);
    case 4: return run_gemv<4>(w, x, x_bf16, t1, lb, r, s, y, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qh
