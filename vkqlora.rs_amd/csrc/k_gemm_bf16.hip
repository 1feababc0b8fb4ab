// k_gemm_bf16.hip -- NF4 GEMMs on bf16 MFMA for bf16 activations (gfx950).
//
// The forward and the input gradient of a QLoRA layer with bf16 activations
// (qlora-core/src/qlora.rs:86-165, the reference's mm_nt / mm_nn WGSL
// kernels qlora-wgpu/shaders/gemm.wgsl:34-98):
//
//   forward  C = X . W^T + T1 . (s B)^T    (W: N x K, C: M x N)
//   grad_x   C = dY . W + Ds . A           (W: K x N as stored, C: M x N)
//
// X and dY are bf16, so they enter v_mfma_f32_32x32x16_bf16 exactly.  The
// dequantized weight w = L[code] * block_scale (fp32, bit-exact with
// quant.rs:157-167) is split into two bf16 parts, w = hi + lo + d with
// |d| <= 2^-16 |w|, and every product runs as two MFMAs (x.hi + x.lo) with
// fp32 accumulation.  The LoRA segment has fp32 operands on both sides and
// runs as three MFMAs (ah.bh + ah.bl + al.bh).
//
// Tiles: 512 threads = 8 waves (two per SIMD, so that one wave's dequant
// work and waits overlap the other's MFMAs) in a 2 x 4 grid; a block
// computes 256 x BN outputs (BN = 256 or 128), a wave 128 x BN/4 of 32 x 32
// MFMA tiles whose accumulators stay in registers for the whole reduction.  The reduction
// runs in steps of 32 through two LDS stages: while the MFMAs read one
// stage, the next step's activations and codes are already in registers
// (loaded at the top of the step) and are dequantized, split and written to
// the other stage after the MFMAs; one barrier per step.  LDS rows are 32
// bf16 plus 8 of padding (80 bytes), so the 16-byte fragment reads of 8
// lanes that one LDS cycle serves fall in distinct banks.
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
constexpr int kBK = 32;          // reduction per step
constexpr int kRow = kBK + 8;    // LDS row, in bf16 elements (80 bytes)

__constant__ float c_lut_bf[17] = QH_NF4_LUT17_INIT;  // the codebook (quant.rs:27-44)

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

// ---- activation tile (bf16, row-major rows x K) -----------------------------
// 256 rows x 32: thread t owns rows t / 4 + 128 v and elements 8 (t % 4) ... + 8.
struct ActTile {
  uint4 v[2];
  __device__ __forceinline__ void load(const uint16_t *p, int64_t ld, int64_t m0, int64_t M,
                                       int64_t k0, int64_t K, bool vec) {
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
  __device__ __forceinline__ void store(uint16_t *S) const {
    const int c = threadIdx.x & 3;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *(uint4 *)(S + ((threadIdx.x >> 2) + 128 * i) * kRow + 8 * c) = v[i];
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
    const int row = threadIdx.x / TPR, k = (threadIdx.x % TPR) * EPT;
    const float s = decode_scale(kind, sr);
    const uint32_t cw[2] = {c.x, c.y};
#pragma unroll
    for (int q = 0; q < EPT / 8; ++q) {  // 8 elements = one code word
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = lut[(cw[q] >> (4 * e)) & 15u] * s;
      uint32_t h[4], l[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split2(f[2 * e], f[2 * e + 1], h[e], l[e]);
      *(uint4 *)(Sh + row * kRow + k + 8 * q) = make_uint4(h[0], h[1], h[2], h[3]);
      *(uint4 *)(Sl + row * kRow + k + 8 * q) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
};

// ---- NF4 tile, input-gradient orientation: 32 W rows (reduction) x BN W
// columns (outputs), written transposed (LDS row = W column).  Lane l of
// wave w holds one code byte (W columns c0 + 128 (w / 4) + 2 l, + 1) of the
// 8 W rows n0 + 8 (w % 4) ... + 8, so consecutive lanes write LDS rows two
// apart (BN = 256; BN = 128 folds the column halves into the row groups).
template <int BN>
struct WTileCol {
  static constexpr int RG = BN == 256 ? 4 : 8;  // row groups
  static constexpr int RPT = kBK / RG;          // rows per thread: 8 or 4
  uint8_t c[RPT];
  ScaleRef sr[RPT];
  __device__ __forceinline__ int wave_() const { return threadIdx.x >> 6; }
  __device__ __forceinline__ void load(const DevQW &w, int64_t c0, int64_t n0) {
    const int wv = wave_(), lane = threadIdx.x & 63;
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
    const int wv = wave_(), lane = threadIdx.x & 63;
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
      if constexpr (RPT == 8) {
        *(uint4 *)(Sh + (cl + j) * kRow + rl) = make_uint4(h[0], h[1], h[2], h[3]);
        *(uint4 *)(Sl + (cl + j) * kRow + rl) = make_uint4(l[0], l[1], l[2], l[3]);
      } else {
        *(uint2 *)(Sh + (cl + j) * kRow + rl) = make_uint2(h[0], h[1]);
        *(uint2 *)(Sl + (cl + j) * kRow + rl) = make_uint2(l[0], l[1]);
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
    *(uint2 *)(Sh + rl * kRow + 4 * c) = make_uint2(h0, h1);
    *(uint2 *)(Sl + rl * kRow + 4 * c) = make_uint2(l0, l1);
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
      Sh[(cl + j) * kRow + kl] = __builtin_bit_cast(uint16_t, h);
      Sl[(cl + j) * kRow + kl] = __builtin_bit_cast(uint16_t, l);
    }
  }
}

// ---- the kernel --------------------------------------------------------------
// WF = ROWK: forward (W rows are the output columns); WF = KROW: grad_x (W
// rows are the reduction).  8 waves in a 2 x 4 grid, each 128 x BN/4 of the
// block's 256 x BN outputs.  LDS per stage: A[256][kRow], Bh[BN][kRow],
// Bl[BN][kRow]; two stages, then the 16-entry codebook.
template <int BN, int WF>
__global__ __launch_bounds__(kThreads, 2) void k_nf4_bf16(Bf16GemmArgs g, int tiles_n) {
  constexpr int TM = 4, TN = BN / 128;  // 32 x 32 tiles per wave
  constexpr int WN = BN / 4;
  constexpr int A_ELEMS = kBM * kRow, B_ELEMS = BN * kRow;
  constexpr int STAGE = A_ELEMS + 2 * B_ELEMS;
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

  // 2 x 16 of the reduction from one stage: A fragments of the wave's rows
  // and hi / lo fragments of its columns, two MFMAs per tile.
  auto mma = [&](const uint16_t *A, const uint16_t *Bh, const uint16_t *Bl) {
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t a[TM], bh[TN], bl[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *(const bf16x8_t *)(A + (wm0 + 32 * i + l32) * kRow + 16 * kk + 8 * h);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        bh[j] = *(const bf16x8_t *)(Bh + (wn0 + 32 * j + l32) * kRow + 16 * kk + 8 * h);
        bl[j] = *(const bf16x8_t *)(Bl + (wn0 + 32 * j + l32) * kRow + 16 * kk + 8 * h);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bl[j], acc[i][j], 0, 0, 0);
    }
  };

  // ---- segment 1: activations x dequantized weight ---------------------------
  const bool a_vec = (g.lda % 8 == 0) && ((((uintptr_t)g.A) & 15) == 0);
  const int kind = g.w.kind;
  ActTile at;
  typename std::conditional<WF == ROWK, WTileRow<BN>, WTileCol<BN>>::type wt;
  const int64_t steps = (g.K + kBK - 1) / kBK;
  if (steps > 0) {
    at.load(g.A, g.lda, m0, g.M, 0, g.K, a_vec);
    wt.load(g.w, n0, 0);
    __syncthreads();  // codebook
    at.store(smem);
    wt.store(smem + A_ELEMS, smem + A_ELEMS + B_ELEMS, lut, kind);
    __syncthreads();
    for (int64_t t = 0; t < steps; ++t) {
      const bool more = t + 1 < steps;
      if (more) {
        at.load(g.A, g.lda, m0, g.M, (t + 1) * kBK, g.K, a_vec);
        wt.load(g.w, n0, (t + 1) * kBK);
      }
      const uint16_t *S = smem + (t & 1) * STAGE;
      mma(S, S + A_ELEMS, S + A_ELEMS + B_ELEMS);
      if (more) {
        uint16_t *D = smem + ((t + 1) & 1) * STAGE;
        at.store(D);
        wt.store(D + A_ELEMS, D + A_ELEMS + B_ELEMS, lut, kind);
      }
      __syncthreads();
    }
  }

  // ---- segment 2: the LoRA term, three MFMAs per tile ------------------------
  if (g.K2 > 0) {
    uint16_t *Ah = smem, *Al = smem + STAGE;
    uint16_t *Bh = smem + A_ELEMS, *Bl = smem + A_ELEMS + B_ELEMS;
    for (int64_t k0 = 0; k0 < g.K2; k0 += kBK) {
      stage_f32_rowk<kBM>(g.A2, g.lda2, m0, g.M, k0, g.K2, 1.0f, Ah, Al);
      if (g.b2form == ROWK)
        stage_f32_rowk<BN>(g.B2, g.ldb2, n0, g.N, k0, g.K2, g.b2scale, Bh, Bl);
      else
        stage_f32_krow<BN>(g.B2, g.ldb2, n0, g.N, k0, g.K2, g.b2scale, Bh, Bl);
      __syncthreads();
      mma(Ah, Bh, Bl);  // ah.bh + ah.bl
#pragma unroll
      for (int kk = 0; kk < kBK / 16; ++kk) {  // al.bh
        bf16x8_t a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a[i] = *(const bf16x8_t *)(Al + (wm0 + 32 * i + l32) * kRow + 16 * kk + 8 * h);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          b[j] = *(const bf16x8_t *)(Bh + (wn0 + 32 * j + l32) * kRow + 16 * kk + 8 * h);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
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

template <int BN, int WF>
hipError_t run_bf16(const Bf16GemmArgs &g, hipStream_t s) {
  auto k = k_nf4_bf16<BN, WF>;
  constexpr uint32_t lds = (uint32_t)(2 * (kBM + 2 * BN) * kRow * 2 + 16 * 4);
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

}  // namespace

// The bf16 path needs whole 64-element blocks per W row and enough output
// tiles to fill the GPU (smaller problems stay on the fp32 tile engine).
bool bf16_gemm_ok(const DevQW &w, int64_t M, int64_t N) {
  return w.bs == 64 && w.cols % 64 == 0 && M >= 256 && N >= 256 && (M / 256) * (N / 128) >= 128;
}

hipError_t launch_gemm_bf16(const Bf16GemmArgs &g, int w_form, hipStream_t s) {
  if (g.M == 0 || g.N == 0) return hipSuccess;
  // 256 x 256 tiles when they leave no GPU-wide wave of blocks mostly empty
  // (one block per CU: 256 CUs), else 256 x 128
  const int64_t t256 = ((g.M + 255) / 256) * ((g.N + 255) / 256);
  const int64_t waves = (t256 + 255) / 256;
  const bool wide = t256 >= 192 && (double)t256 / (double)(waves * 256) >= 0.75;
  if (w_form == ROWK)
    return wide ? run_bf16<256, ROWK>(g, s) : run_bf16<128, ROWK>(g, s);
  return wide ? run_bf16<256, KROW>(g, s) : run_bf16<128, KROW>(g, s);
}

}  // namespace qh
