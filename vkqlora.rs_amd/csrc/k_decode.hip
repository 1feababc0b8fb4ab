// k_decode.hip -- decode-shaped fused NF4 dequant-GEMV on gfx950 MFMA.
//
// Replaces, for batches of at most 16 tokens, the reference forward's
// dequant + mm_nt + LoRA mm_nt dispatches (qlora-wgpu/src/kernels.rs:262-296,
// shaders/gemm.wgsl:68-98):
//
//   y[m][n] = sum_b s_{n,b} sum_{k in b} x[m][k] L[c_{n,k}]
//           + (alpha/r) sum_j T1[m][j] B[n][j],      T1 = X A^T.
//
// The weight stream is the only large input, so the kernel is built to keep
// VALU work per packed byte small:
//  * Codes are turned into MFMA operands by table lookup: a byte (two
//    nibbles) indexes a 256-entry table whose entry holds the two codebook
//    levels split into bf16 hi and lo parts (L = hi + lo + O(2^-18 L)).  The
//    table is replicated 32 times in LDS so that lane l always reads the
//    bank pair 2*(l%32): lookups are free of bank conflicts for any data.
//  * x is split the same way (prep kernel), and three bf16 MFMAs
//    (xh*Lh + xl*Lh + xh*Ll, fp32 accumulate) give each product to about
//    2^-16 relative -- far inside the 1e-4 parity bar -- at bf16 MFMA rate.
//  * The 64-element block scale is applied once per block to the MFMA
//    partial (scale hoisting): lane l's outputs all belong to weight row
//    l%16, so one scale decode per lane per block.
// Layout of one wave's work unit: 16 weight rows (MFMA N) x 16 batch rows
// (MFMA M, zero-padded) x one 64-element block (two K=32 MFMA steps).  Lane
// group g = l/16 supplies elements {8g..8g+7} and {32+8g..32+8g+7} of the
// block: two dword loads per lane.  A workgroup (8 waves) owns 16 rows and
// interleaves the row's blocks over its waves; partial tiles are reduced in
// LDS in a fixed order.
#include "qh_internal.h"
#include "qh_nf4.h"

namespace qh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kCopies = 32;
constexpr int kDepth = 4;  // blocks loaded together per wave

constexpr uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
constexpr float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
constexpr uint32_t bf16_rne(float f) {
  const uint32_t u = f2u(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

struct PairTable {
  uint32_t hi[256], lo[256];
};

constexpr PairTable make_pair_table() {
  PairTable t{};
  constexpr float L[16] = {
      -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
      -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
      0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
      0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
      0.7229568362236023f, 1.0f};
  for (int v = 0; v < 256; ++v) {
    uint32_t h[2] = {0, 0}, l[2] = {0, 0};
    for (int q = 0; q < 2; ++q) {
      const float x = L[q == 0 ? (v & 15) : (v >> 4)];
      h[q] = bf16_rne(x);
      l[q] = bf16_rne(x - u2f(h[q] << 16));
    }
    t.hi[v] = h[0] | (h[1] << 16);
    t.lo[v] = l[0] | (l[1] << 16);
  }
  return t;
}

__constant__ PairTable c_pairs = make_pair_table();

__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// ---------------------------------------------------------------------------
// Prep: X -> (Xh, Xl) bf16 split, and T1 = X A^T.  grid = (max(r,1), M),
// 256 threads: workgroup (j, m) splits its 1/gridDim.x share of X row m and,
// if r > 0, computes T1[m][j] over the whole K.  Loads are issued in
// unconditional batches of 8 per thread (clamped index, zero weight).
template <int XBF16>
__device__ __forceinline__ float4 load_x4(const void *x, int64_t e) {
  if (XBF16) {
    const uint2 q = *(const uint2 *)((const uint16_t *)x + e);
    return make_float4(__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xffff0000u),
                       __uint_as_float(q.y << 16), __uint_as_float(q.y & 0xffff0000u));
  }
  return *(const float4 *)((const float *)x + e);
}

template <int XBF16>
__global__ __launch_bounds__(256) void k_decode_prep(
    const void *__restrict__ x, int M, int64_t K, const float *__restrict__ a,
    int r, uint16_t *__restrict__ xh, uint16_t *__restrict__ xl,
    float *__restrict__ t1) {
  __shared__ float red[4];
  const int j = blockIdx.x, J = gridDim.x, m = blockIdx.y, tid = threadIdx.x;
  const int64_t units = K >> 3;  // 8-element units of row m
  const int64_t u0 = units * j / J, u1 = xh ? units * (j + 1) / J : u0;
  for (int64_t u = u0 + tid; u < u1; u += 256) {
    const int64_t e = (int64_t)m * K + u * 8;
    const float4 p0 = load_x4<XBF16>(x, e), p1 = load_x4<XBF16>(x, e + 4);
    const float v[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t h0 = bf16_bits_rne(v[2 * q]), h1 = bf16_bits_rne(v[2 * q + 1]);
      const uint32_t l0 = bf16_bits_rne(v[2 * q] - __uint_as_float(h0 << 16));
      const uint32_t l1 = bf16_bits_rne(v[2 * q + 1] - __uint_as_float(h1 << 16));
      hw[q] = h0 | (h1 << 16);
      lw[q] = l0 | (l1 << 16);
    }
    *(uint4 *)(xh + e) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(xl + e) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  }
  if (r == 0) return;
  const int64_t nk4 = K >> 2;
  const float4 *a4 = (const float4 *)(a + (int64_t)j * K);
  float s = 0.0f;
  for (int64_t base = tid; base < nk4; base += 256 * 8) {
    float4 xv[8], av[8];
    float ok[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t k4 = base + 256 * q;
      ok[q] = k4 < nk4 ? 1.0f : 0.0f;
      const int64_t kc = k4 < nk4 ? k4 : 0;
      av[q] = a4[kc];
      xv[q] = load_x4<XBF16>(x, (int64_t)m * K + 4 * kc);
    }
    __builtin_amdgcn_sched_barrier(0);  // loads stay batched ahead of uses
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float p = xv[q].x * av[q].x;
      p = fmaf(xv[q].y, av[q].y, p);
      p = fmaf(xv[q].z, av[q].z, p);
      p = fmaf(xv[q].w, av[q].w, p);
      s = fmaf(p, ok[q], s);
    }
  }
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) t1[m * r + j] = (red[0] + red[1]) + (red[2] + red[3]);
}

// ---------------------------------------------------------------------------
template <int XLO, int KIND>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_decode(
    DevQW w, int M, const uint16_t *__restrict__ xh,
    const uint16_t *__restrict__ xl, const float *__restrict__ t1,
    const float *__restrict__ lb, int r, float s_lora, float *__restrict__ y) {
  __shared__ uint2 tab[256 * kCopies];  // 64 KB; reused for the epilogue
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t N = w.rows, K = w.cols, KB = K >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16;

  // Replicate the pair table: each thread writes copies of one byte's entry.
  {
    constexpr int kPer = 256 * kCopies / kThreads;
    const int v = tid / (kCopies / kPer), c0 = (tid % (kCopies / kPer)) * kPer;
    const uint2 e = make_uint2(c_pairs.hi[v], c_pairs.lo[v]);
#pragma unroll
    for (int c = 0; c < kPer; ++c) tab[v * kCopies + c0 + c] = e;
  }
  __syncthreads();
  // LoRA epilogue operands (16 rows of B, and T1): loaded before the main
  // loop, consumed after it, so their latency hides behind it.
  float lbv[2] = {0.0f, 0.0f}, t1v[2] = {0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int idx = tid + q * kThreads;
    if (idx < 16 * r) {
      int64_t row = n0 + idx / r;
      row = row < N ? row : N - 1;
      lbv[q] = lb[row * r + idx % r];
    }
    if (idx < M * r) t1v[q] = t1[idx];
  }

  const int i = lane & 15, g = lane >> 4;
  const int64_t n = (n0 + i < N) ? n0 + i : N - 1;
  const uint32_t *c32 = (const uint32_t *)w.codes + n * (K >> 3);
  const int copy = lane & 31;
  const bool xrow = i < M;
  const uint16_t *xhr = xh + (int64_t)i * K + 8 * g;
  const uint16_t *xlr = xl + (int64_t)i * K + 8 * g;

  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t kb0 = wave; kb0 < KB; kb0 += kWaves * kDepth) {
    // Issue every load of kDepth blocks before using any of them: raw scale
    // fields are decoded only at use so no wait sits between the loads.
    uint32_t cw[kDepth][2];
    float sa[kDepth], okm[kDepth];
    int32_t sq[kDepth];
    uint4 ah[kDepth][2], al[kDepth][2];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int64_t kb = kb0 + (int64_t)d * kWaves;
      const bool ok = kb < KB;
      const int64_t kbc = ok ? kb : 0;
      okm[d] = ok ? 1.0f : 0.0f;
      cw[d][0] = c32[kbc * 8 + g];
      cw[d][1] = c32[kbc * 8 + 4 + g];
      const int64_t b = n * KB + kbc;
      if (KIND == 0) {
        sa[d] = w.scales[b];
        sq[d] = 0;
      } else {
        sq[d] = (int8_t)w.scale_codes[b];
        sa[d] = w.absmax[b >> 8];
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        ah[d][t] = make_uint4(0, 0, 0, 0);
        al[d][t] = make_uint4(0, 0, 0, 0);
        if (xrow) {
          ah[d][t] = *(const uint4 *)(xhr + kbc * 64 + 32 * t);
          if (XLO) al[d][t] = *(const uint4 *)(xlr + kbc * 64 + 32 * t);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // loads stay batched ahead of uses
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      floatx4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t bh[4], bl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint2 e = tab[((cw[d][t] >> (8 * q)) & 255u) * kCopies + copy];
          bh[q] = e.x;
          bl[q] = e.y;
        }
        const bf16x8 Bh = __builtin_bit_cast(bf16x8, make_uint4(bh[0], bh[1], bh[2], bh[3]));
        const bf16x8 Bl = __builtin_bit_cast(bf16x8, make_uint4(bl[0], bl[1], bl[2], bl[3]));
        const bf16x8 Ah = __builtin_bit_cast(bf16x8, ah[d][t]);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bh, c, 0, 0, 0);
        if (XLO) {
          const bf16x8 Al = __builtin_bit_cast(bf16x8, al[d][t]);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bh, c, 0, 0, 0);
        }
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bl, c, 0, 0, 0);
      }
      // block scale (within 1 ulp of quant.rs:218's decode; only the GEMV
      // sum depends on it, never a stored weight)
      const float sc = (KIND == 0 ? sa[d] : (float)sq[d] * (sa[d] * (1.0f / 127.0f))) * okm[d];
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = fmaf(sc, c[v], acc[v]);
    }
  }

  // Lane holds D[batch 4g+v][row i]; reduce the waves in LDS (fixed order).
  __syncthreads();
  float *red = (float *)tab;          // kWaves x 256 floats
  float *lbs = red + kWaves * 256;    // 16 x r
  float *t1s = lbs + 16 * 64;         // M x r
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave * 256 + (4 * g + v) * 16 + i] = acc[v];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int idx = tid + q * kThreads;
    if (idx < 16 * r) lbs[idx] = lbv[q];
    if (idx < M * r) t1s[idx] = t1v[q];
  }
  __syncthreads();
  if (tid < 256) {
    const int bm = tid >> 4, ri = tid & 15;
    const int64_t nn = n0 + ri;
    if (bm < M && nn < N) {
      float sum = 0.0f;
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv) sum += red[wv * 256 + tid];
      if (r > 0) {
        float l = 0.0f;
        for (int j = 0; j < r; ++j) l += t1s[bm * r + j] * lbs[ri * r + j];
        sum += s_lora * l;
      }
      y[(int64_t)bm * N + nn] = sum;
    }
  }
}

}  // namespace

bool decode_ok(const DevQW &w, int64_t M, int64_t r) {
  return M >= 1 && M <= 16 && r <= 64 && w.bs == 64 && w.cols % 256 == 0 &&
         (((uintptr_t)w.codes) & 3) == 0;
}

size_t decode_scratch_bytes(int64_t M, int64_t K, int64_t r) {
  const size_t xs = ((size_t)M * K * 2 + 255) / 256 * 256;
  return 2 * xs + (size_t)M * (r ? r : 1) * 4 + 256;
}

hipError_t launch_decode_prep(const DevQW &w, const void *x, int x_bf16, int64_t M,
                              const float *a, int64_t r, float *t1_out, void *scratch,
                              hipStream_t st) {
  const int64_t K = w.cols;
  const size_t xs = ((size_t)M * K * 2 + 255) / 256 * 256;
  uint16_t *xh = (uint16_t *)scratch;
  uint16_t *xl = (uint16_t *)((char *)scratch + xs);
  float *t1 = t1_out ? t1_out : (float *)((char *)scratch + 2 * xs);
  const dim3 grid((unsigned)(r > 0 ? r : 8), (unsigned)M);
  if (x_bf16)
    return qh_launch(k_decode_prep<1>, grid, dim3(256), 0, st, x, (int)M, K, a, (int)r,
                     xh, xl, t1);
  return qh_launch(k_decode_prep<0>, grid, dim3(256), 0, st, x, (int)M, K, a, (int)r,
                   xh, xl, t1);
}

hipError_t launch_lora_t1(const void *x, int x_bf16, int64_t M, int64_t K, const float *a,
                          int64_t r, float *t1, hipStream_t st) {
  if (M == 0 || r == 0) return hipSuccess;
  const dim3 grid((unsigned)r, (unsigned)M);
  uint16_t *none = nullptr;
  if (x_bf16)
    return qh_launch(k_decode_prep<1>, grid, dim3(256), 0, st, x, (int)M, K, a, (int)r,
                     none, none, t1);
  return qh_launch(k_decode_prep<0>, grid, dim3(256), 0, st, x, (int)M, K, a, (int)r,
                   none, none, t1);
}

hipError_t launch_decode(const DevQW &w, int x_bf16, int64_t M, const float *lb,
                         int64_t r, float s, float *y, const float *t1_out, void *scratch,
                         hipStream_t st) {
  const int64_t K = w.cols, N = w.rows;
  const size_t xs = ((size_t)M * K * 2 + 255) / 256 * 256;
  uint16_t *xh = (uint16_t *)scratch;
  uint16_t *xl = (uint16_t *)((char *)scratch + xs);
  const float *t1 = t1_out ? t1_out : (const float *)((char *)scratch + 2 * xs);
  dim3 grid((unsigned)((N + 15) / 16));
  const dim3 blk(kThreads);
  if (x_bf16) {
    if (w.kind == 0)
      return qh_launch(k_decode<0, 0>, grid, blk, 0, st, w, (int)M, xh, xl, t1, lb, (int)r, s, y);
    return qh_launch(k_decode<0, 1>, grid, blk, 0, st, w, (int)M, xh, xl, t1, lb, (int)r, s, y);
  }
  if (w.kind == 0)
    return qh_launch(k_decode<1, 0>, grid, blk, 0, st, w, (int)M, xh, xl, t1, lb, (int)r, s, y);
  return qh_launch(k_decode<1, 1>, grid, blk, 0, st, w, (int)M, xh, xl, t1, lb, (int)r, s, y);
}

}  // namespace qh
