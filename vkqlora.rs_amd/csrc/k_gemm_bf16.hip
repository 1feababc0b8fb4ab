// k_gemm_bf16.hip -- the large NF4 GEMMs of a QLoRA layer on bf16 MFMA (gfx950).
//
// The forward and the input gradient (qlora-core/src/qlora.rs:86-165, the
// reference's mm_nt / mm_nn WGSL kernels qlora-wgpu/shaders/gemm.wgsl:34-98):
//
//   forward  C = X . W^T + T1 . (s B)^T    (W: N x K, C: M x N)
//   grad_x   C = dY . W + Ds . A           (W: K x N as stored, C: M x N)
//
// on v_mfma_f32_32x32x16_bf16 with fp32 accumulation.  The dequantized
// weight w = L[code] * block_scale (fp32, bit-exact with quant.rs:157-167)
// is split into two bf16 parts, w = wh + wl + d with |d| <= 2^-16 |w|.
//  * bf16 activations (XF = 0) are exact in bf16: a product runs as two
//    MFMAs, x.wh + x.wl.
//  * fp32 activations (XF = 1) are split the same way: xh.wh + xh.wl +
//    xl.wh, three MFMAs, leaving out xl.wl (~2^-16 of the product); the
//    bf16 MFMA rate is 16 times the fp32 one, so three of them still beat
//    one fp32 MFMA five-fold.
//  * The LoRA segment (fp32 operands) always runs as three MFMAs.
//
// Tiles: 512 threads = 8 waves (two per SIMD, so that one wave's dequant
// work and waits overlap the other's MFMAs) in a 2 x 4 grid; a block
// computes 256 x BN outputs (BN = 256 or 128), a wave 128 x BN/4 of 32 x 32
// MFMA tiles whose accumulators stay in registers for the whole reduction.
// The reduction runs in steps of 32 through two LDS stages: while the MFMAs
// read one stage, the next step's activations and codes are already in
// registers (loaded at the top of the step) and are dequantized, split and
// written to the other stage after the MFMAs; one barrier per step.
// LDS rows hold 32 bf16 (64 bytes) as four 16-byte granules; granule g of
// row r sits at position g ^ ((r >> 1) & 3), so that the fragment reads of
// 8 consecutive rows that one LDS cycle serves fall in 8 distinct bank
// groups without padding.
#include <type_traits>

#include "qh_internal.h"
#include "qh_nf4.h"

namespace qh {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 512;    // 8 waves: two per SIMD
constexpr int kBM = 256;         // output rows per block
constexpr int kBK = 32;          // reduction per step = one LDS row

__constant__ float c_lut_bf[17] = QH_NF4_LUT17_INIT;  // the codebook (quant.rs:27-44)

// Element offset of granule g (8 elements) of LDS row `row`.
__device__ __forceinline__ int sw(int row, int g) { return row * kBK + 8 * (g ^ ((row >> 1) & 3)); }

// Two floats as a bf16 pair (round to nearest even).
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const bf16x2_t h = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ float bf16_lo_f(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi_f(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// hi and lo bf16 parts of two floats: hi = bf16(v), lo = bf16(v - hi).
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
  hi = pk_bf16(a, b);
  lo = pk_bf16(a - bf16_lo_f(hi), b - bf16_hi_f(hi));
}

// Block scale (quant.rs:212-221): fp32, or fl(fl(c / 127) * absmax).  c / 127
// is the double product with the double reciprocal of 127 rounded once to
// float, which is the IEEE float quotient bit for bit (an exact quotient of
// two floats lies at least 2^-49 relatively from every float midpoint; the
// product is within 2^-52), without a float division.
struct ScaleRef {
  float a;    // the fp32 scale, or the super-block absmax
  int32_t c;  // the int8 scale code
};
__device__ __forceinline__ ScaleRef load_scale(const DevQW &w, int64_t blk) {
  if (w.kind == 0) return ScaleRef{w.scales[blk], 127};
  return ScaleRef{w.absmax[blk >> 8], (int32_t)(int8_t)w.scale_codes[blk]};
}
__device__ __forceinline__ float decode_scale(int kind, ScaleRef r) {
  if (kind == 0) return r.a;
  return (float)((double)(float)r.c * (1.0 / 127.0)) * r.a;
}

// ---- activation tile: 256 rows x 32 of a row-major (rows x K) matrix ---------
// Thread t owns rows t / 4 + 128 v and granule t % 4 (elements 8 (t % 4) ...
// + 8).  bf16 (XF = 0) is copied; fp32 (XF = 1) is split into hi and lo.
template <int XF>
struct ActTile;

template <>
struct ActTile<0> {
  uint4 v[2];
  __device__ __forceinline__ void load(const void *pv, int64_t ld, int64_t m0, int64_t M,
                                       int64_t k0, int64_t K, bool vec) {
    const uint16_t *p = (const uint16_t *)pv;
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t row = m0 + (threadIdx.x >> 2) + 128 * i, k = k0 + 8 * c;
      if (vec && row < M && k + 8 <= K) {
        v[i] = *(const uint4 *)(p + row * ld + k);
      } else {
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = (row < M && k + j < K) ? p[row * ld + k + j] : 0u;
        v[i] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                          e[6] | (e[7] << 16));
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t *Sh, uint16_t *) const {
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) *(uint4 *)(Sh + sw((threadIdx.x >> 2) + 128 * i, c)) = v[i];
  }
};

template <>
struct ActTile<1> {
  float4 v[2][2];
  __device__ __forceinline__ void load(const void *pv, int64_t ld, int64_t m0, int64_t M,
                                       int64_t k0, int64_t K, bool vec) {
    const float *p = (const float *)pv;
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t row = m0 + (threadIdx.x >> 2) + 128 * i, k = k0 + 8 * c;
      if (vec && row < M && k + 8 <= K) {
        v[i][0] = *(const float4 *)(p + row * ld + k);
        v[i][1] = *(const float4 *)(p + row * ld + k + 4);
      } else {
        float e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = (row < M && k + j < K) ? p[row * ld + k + j] : 0.0f;
        v[i][0] = make_float4(e[0], e[1], e[2], e[3]);
        v[i][1] = make_float4(e[4], e[5], e[6], e[7]);
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t *Sh, uint16_t *Sl) const {
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint32_t h[4], l[4];
      split2(v[i][0].x, v[i][0].y, h[0], l[0]);
      split2(v[i][0].z, v[i][0].w, h[1], l[1]);
      split2(v[i][1].x, v[i][1].y, h[2], l[2]);
      split2(v[i][1].z, v[i][1].w, h[3], l[3]);
      const int o = sw((threadIdx.x >> 2) + 128 * i, c);
      *(uint4 *)(Sh + o) = make_uint4(h[0], h[1], h[2], h[3]);
      *(uint4 *)(Sl + o) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
};

// ---- NF4 tile, forward orientation: BN W rows (output columns) x 32 ----------
// W row n = n0 + t / TPR, elements (t % TPR) * EPT ... + EPT of the step
// (within one 64-element block, so one scale).
template <int BN>
struct WTileRow {
  static constexpr int TPR = kThreads / BN;     // threads per W row: 2 or 4
  static constexpr int EPT = kBK / TPR;         // elements per thread: 16 or 8
  uint2 c;        // EPT / 2 code bytes
  ScaleRef sr;
  __device__ __forceinline__ void load(const DevQW &w, int64_t n0, int64_t k0) {
    const int64_t n = n0 + threadIdx.x / TPR;
    const int64_t k = k0 + (threadIdx.x % TPR) * EPT;
    c = make_uint2(0, 0);
    sr = ScaleRef{0.0f, 0};
    if (n < w.rows) {
      const int64_t e = n * w.cols + k;
      if (EPT == 16) c = *(const uint2 *)(w.codes + (e >> 1));
      else c.x = *(const uint32_t *)(w.codes + (e >> 1));
      sr = load_scale(w, e >> 6);
    }
  }
  __device__ __forceinline__ void store(uint16_t *Sh, uint16_t *Sl, const float *lut,
                                        int kind) const {
    const int row = threadIdx.x / TPR, g0 = (threadIdx.x % TPR) * (EPT / 8);
    const float s = decode_scale(kind, sr);
    const uint32_t cw[2] = {c.x, c.y};
#pragma unroll
    for (int q = 0; q < EPT / 8; ++q) {  // 8 elements = one code word = one granule
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = lut[(cw[q] >> (4 * e)) & 15u] * s;
      uint32_t h[4], l[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split2(f[2 * e], f[2 * e + 1], h[e], l[e]);
      const int o = sw(row, g0 + q);
      *(uint4 *)(Sh + o) = make_uint4(h[0], h[1], h[2], h[3]);
      *(uint4 *)(Sl + o) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
};

// ---- NF4 tile, input-gradient orientation: 32 W rows (reduction) x BN W
// columns (outputs), written transposed (LDS row = W column).  Lane l of
// wave w holds one code byte (W columns c0 + 128 (w / 4) + 2 l, + 1) of the
// RPT W rows n0 + RPT (w % RG) ... + RPT, so consecutive lanes write LDS
// rows two apart (BN = 256; BN = 128 folds the column halves into the row
// groups).
template <int BN>
struct WTileCol {
  static constexpr int RG = BN == 256 ? 4 : 8;  // row groups
  static constexpr int RPT = kBK / RG;          // rows per thread: 8 or 4
  uint8_t c[RPT];
  ScaleRef sr[RPT];
  __device__ __forceinline__ void load(const DevQW &w, int64_t c0, int64_t n0) {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t col = c0 + (BN == 256 ? 128 * (wv / RG) : 0) + 2 * lane;
    const int64_t row0 = n0 + RPT * (wv % RG);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int64_t n = row0 + i;
      c[i] = 0;
      sr[i] = ScaleRef{0.0f, 0};
      if (n < w.rows && col < w.cols) {
        const int64_t e = n * w.cols + col;
        c[i] = w.codes[e >> 1];
        sr[i] = load_scale(w, e >> 6);
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t *Sh, uint16_t *Sl, const float *lut,
                                        int kind) const {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cl = (BN == 256 ? 128 * (wv / RG) : 0) + 2 * lane, rl = RPT * (wv % RG);
    float s[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) s[i] = decode_scale(kind, sr[i]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {  // W column cl + j: RPT consecutive reduction rows
      float f[RPT];
#pragma unroll
      for (int i = 0; i < RPT; ++i) f[i] = lut[((uint32_t)c[i] >> (4 * j)) & 15u] * s[i];
      uint32_t h[RPT / 2], l[RPT / 2];
#pragma unroll
      for (int e = 0; e < RPT / 2; ++e) split2(f[2 * e], f[2 * e + 1], h[e], l[e]);
      const int o = sw(cl + j, rl >> 3) + (rl & 7);
      if constexpr (RPT == 8) {
        *(uint4 *)(Sh + o) = make_uint4(h[0], h[1], h[2], h[3]);
        *(uint4 *)(Sl + o) = make_uint4(l[0], l[1], l[2], l[3]);
      } else {
        *(uint2 *)(Sh + o) = make_uint2(h[0], h[1]);
        *(uint2 *)(Sl + o) = make_uint2(l[0], l[1]);
      }
    }
  }
};

// ---- LoRA segment tiles (fp32 operands, split into hi / lo) -----------------
// R rows x 32 of a row-major fp32 matrix (element (row, k) at p[row * ld + k]),
// scaled by `scale`: thread t owns rows t / 8 + 64 v, elements 4 (t % 8) ... + 4.
template <int R>
__device__ __forceinline__ void stage_f32_rowk(const float *p, int64_t ld, int64_t r0, int64_t rlim,
                                               int64_t k0, int64_t klim, float scale,
                                               uint16_t *Sh, uint16_t *Sl) {
  const int c = threadIdx.x & 7;
#pragma unroll
  for (int i = 0; i < R / 64; ++i) {
    const int rl = (threadIdx.x >> 3) + 64 * i;
    const int64_t row = r0 + rl, k = k0 + 4 * c;
    float f[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = (row < rlim && k + j < klim) ? p[row * ld + k + j] * scale : 0.0f;
    uint32_t h0, h1, l0, l1;
    split2(f[0], f[1], h0, l0);
    split2(f[2], f[3], h1, l1);
    const int o = sw(rl, c >> 1) + 4 * (c & 1);
    *(uint2 *)(Sh + o) = make_uint2(h0, h1);
    *(uint2 *)(Sl + o) = make_uint2(l0, l1);
  }
}

// 32 x R of a row-major fp32 matrix read transposed (element (col, k) at
// p[k * ld + col]): thread t owns reduction rows t / (R / 4) + KS v and
// columns 4 (t % (R / 4)) ... + 4.
template <int R>
__device__ __forceinline__ void stage_f32_krow(const float *p, int64_t ld, int64_t c0, int64_t clim,
                                               int64_t k0, int64_t klim, float scale,
                                               uint16_t *Sh, uint16_t *Sl) {
  constexpr int CG = R / 4, KS = kThreads / CG;
  const int cl = 4 * (threadIdx.x % CG);
#pragma unroll
  for (int i = 0; i < kBK / KS; ++i) {
    const int kl = threadIdx.x / CG + KS * i;
    const int64_t k = k0 + kl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = c0 + cl + j;
      const float f = (k < klim && col < clim) ? p[k * ld + col] * scale : 0.0f;
      const __bf16 h = (__bf16)f;
      const __bf16 l = (__bf16)(f - (float)h);
      const int o = sw(cl + j, kl >> 3) + (kl & 7);
      Sh[o] = __builtin_bit_cast(uint16_t, h);
      Sl[o] = __builtin_bit_cast(uint16_t, l);
    }
  }
}

// ---- the kernel --------------------------------------------------------------
// WF = ROWK: forward (W rows are the output columns); WF = KROW: grad_x (W
// rows are the reduction).  XF: activations bf16 (0) or fp32 (1).  8 waves
// in a 2 x 4 grid, each 128 x BN/4 of the block's 256 x BN outputs.  LDS
// per stage: Ah[256][32], Al[256][32], Bh[BN][32], Bl[BN][32]; two stages,
// then the 16-entry codebook.
template <int BN, int WF, int XF>
__global__ __launch_bounds__(kThreads, 2) void k_nf4_bf16(Bf16GemmArgs g, int tiles_n) {
  constexpr int TM = 4, TN = BN / 128;  // 32 x 32 tiles per wave
  constexpr int WN = BN / 4;
  constexpr int A_ELEMS = kBM * kBK, B_ELEMS = BN * kBK;
  constexpr int STAGE = 2 * A_ELEMS + 2 * B_ELEMS;
  extern __shared__ __align__(16) uint16_t smem[];
  float *lut = (float *)(smem + 2 * STAGE);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int wm0 = (wave >> 2) * 128, wn0 = (wave & 3) * WN;
  // Blocks go to the 8 XCDs round robin (block b to XCD b % 8): give each
  // XCD a contiguous run of tiles (whole rows of them), so that the blocks
  // sharing an activation panel share an L2.
  const int nb = (int)gridDim.x;
  int tb = (int)blockIdx.x;
  if (nb % 8 == 0) tb = (tb % 8) * (nb / 8) + tb / 8;
  const int64_t m0 = (int64_t)(tb / tiles_n) * kBM, n0 = (int64_t)(tb % tiles_n) * BN;
  if (tid < 16) lut[tid] = c_lut_bf[tid];

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // 2 x 16 of the reduction from one stage: ah.bh + ah.bl (+ al.bh when the
  // A operand has a lo part).
  auto mma = [&](const uint16_t *Ah, const uint16_t *Al, const uint16_t *Bh, const uint16_t *Bl,
                 bool a_lo) {
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t ah[TM], al[TM], bh[TN], bl[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        ah[i] = *(const bf16x8_t *)(Ah + sw(wm0 + 32 * i + l32, 2 * kk + h));
        if (a_lo) al[i] = *(const bf16x8_t *)(Al + sw(wm0 + 32 * i + l32, 2 * kk + h));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        bh[j] = *(const bf16x8_t *)(Bh + sw(wn0 + 32 * j + l32, 2 * kk + h));
        bl[j] = *(const bf16x8_t *)(Bl + sw(wn0 + 32 * j + l32, 2 * kk + h));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
      if (a_lo) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // ---- segment 1: activations x dequantized weight ---------------------------
  const bool a_vec = (g.lda % 8 == 0) && ((((uintptr_t)g.A) & 15) == 0);
  const int kind = g.w.kind;
  ActTile<XF> at;
  typename std::conditional<WF == ROWK, WTileRow<BN>, WTileCol<BN>>::type wt;
  const int64_t steps = (g.K + kBK - 1) / kBK;
  auto stage = [&](uint16_t *D) {
    at.store(D, D + A_ELEMS);
    wt.store(D + 2 * A_ELEMS, D + 2 * A_ELEMS + B_ELEMS, lut, kind);
  };
  if (steps > 0) {
    at.load(g.A, g.lda, m0, g.M, 0, g.K, a_vec);
    wt.load(g.w, n0, 0);
    __syncthreads();  // codebook
    stage(smem);
    __syncthreads();
    for (int64_t t = 0; t < steps; ++t) {
      const bool more = t + 1 < steps;
      if (more) {
        at.load(g.A, g.lda, m0, g.M, (t + 1) * kBK, g.K, a_vec);
        wt.load(g.w, n0, (t + 1) * kBK);
      }
      const uint16_t *S = smem + (t & 1) * STAGE;
      mma(S, S + A_ELEMS, S + 2 * A_ELEMS, S + 2 * A_ELEMS + B_ELEMS, XF == 1);
      if (more) stage(smem + ((t + 1) & 1) * STAGE);
      __syncthreads();
    }
  }

  // ---- segment 2: the LoRA term, three MFMAs per tile ------------------------
  if (g.K2 > 0) {
    uint16_t *Ah = smem, *Al = smem + A_ELEMS;
    uint16_t *Bh = smem + 2 * A_ELEMS, *Bl = smem + 2 * A_ELEMS + B_ELEMS;
    for (int64_t k0 = 0; k0 < g.K2; k0 += kBK) {
      stage_f32_rowk<kBM>(g.A2, g.lda2, m0, g.M, k0, g.K2, 1.0f, Ah, Al);
      if (g.b2form == ROWK)
        stage_f32_rowk<BN>(g.B2, g.ldb2, n0, g.N, k0, g.K2, g.b2scale, Bh, Bl);
      else
        stage_f32_krow<BN>(g.B2, g.ldb2, n0, g.N, k0, g.K2, g.b2scale, Bh, Bl);
      __syncthreads();
      mma(Ah, Al, Bh, Bl, true);
      __syncthreads();
    }
  }

  // ---- epilogue ---------------------------------------------------------------
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm0 + 32 * i + 8 * (v / 4) + 4 * h + (v % 4);
        const int64_t n = n0 + wn0 + 32 * j + l32;
        if (m < g.M && n < g.N) g.C[m * g.ldc + n] = g.alpha * acc[i][j][v];
      }
}

template <int BN, int WF, int XF>
hipError_t run_bf16(const Bf16GemmArgs &g, hipStream_t s) {
  auto k = k_nf4_bf16<BN, WF, XF>;
  constexpr uint32_t lds = (uint32_t)(2 * (2 * kBM + 2 * BN) * kBK * 2 + 16 * 4);
  static bool attr = false;  // per instantiation
  if (!attr) {
    const hipError_t e =
        hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const int tiles_n = (int)((g.N + BN - 1) / BN);
  const int tiles_m = (int)((g.M + kBM - 1) / kBM);
  return qh_launch(k, dim3((unsigned)(tiles_n * tiles_m)), dim3(kThreads), lds, s, g, tiles_n);
}

template <int WF, int XF>
hipError_t pick_bn(const Bf16GemmArgs &g, hipStream_t s) {
  // 256 x 256 tiles when they leave no GPU-wide wave of blocks mostly empty
  // (one block per CU: 256 CUs), else 256 x 128
  const int64_t t256 = ((g.M + 255) / 256) * ((g.N + 255) / 256);
  const int64_t waves = (t256 + 255) / 256;
  const bool wide = t256 >= 192 && (double)t256 / (double)(waves * 256) >= 0.75;
  return wide ? run_bf16<256, WF, XF>(g, s) : run_bf16<128, WF, XF>(g, s);
}

}  // namespace

// The bf16-MFMA path needs whole 64-element blocks per W row and enough
// output tiles to fill the GPU (smaller problems stay on the fp32 tile
// engine).
bool bf16_gemm_ok(const DevQW &w, int64_t M, int64_t N) {
  return w.bs == 64 && w.cols % 64 == 0 && M >= 256 && N >= 256 && (M / 256) * (N / 128) >= 128;
}

hipError_t launch_gemm_bf16(const Bf16GemmArgs &g, int w_form, int a_f32, hipStream_t s) {
  if (g.M == 0 || g.N == 0) return hipSuccess;
  if (w_form == ROWK) return a_f32 ? pick_bn<ROWK, 1>(g, s) : pick_bn<ROWK, 0>(g, s);
  return a_f32 ? pick_bn<KROW, 1>(g, s) : pick_bn<KROW, 0>(g, s);
}

}  // namespace qh
