// k_decode.hip -- decode-shaped fused NF4 dequant-GEMV on gfx950 MFMA.
//
// Replaces, for batches of at most 16 tokens, the reference forward's
// dequant + mm_nt + LoRA mm_nt dispatches (qlora-wgpu/src/kernels.rs:262-296,
// shaders/gemm.wgsl:68-98):
//
//   y[m][n] = sum_b s_{n,b} sum_{k in b} x[m][k] L[c_{n,k}]
//           + (alpha/r) sum_j T1[m][j] B[n][j],      T1 = X A^T.
//
// Two kernels:
//  * k_dprep -- one workgroup per 256-element line of K.  It splits X into
//    bf16 hi/lo parts laid out as MFMA A-fragments, computes the line's
//    partial of T1, and the last workgroup to finish (atomic ticket, no
//    waiting) sums the partials in line order: T1 is deterministic.
//  * k_dmain -- the weight stream.  A workgroup owns 16 weight rows; its 4
//    waves split K into contiguous line ranges.  Per line, lane (n, g)
//    (n = lane % 16, g = lane / 16) loads bytes [16g, 16g+16) and
//    [64+16g, 64+16g+16) of row n's 128-byte line: every load instruction
//    reads 16 rows x 64 contiguous bytes.  Two v_permlane32_swap per 16 bytes
//    regroup the dwords so that each K=32 MFMA step covers 32 elements of ONE
//    64-element block (one scale per output column per step; k-slot order
//    step_koff below).  Nibbles become bf16 hi/lo operands by LDS table
//    lookup (L = Lh + Ll + O(2^-18 L)); three bf16 MFMAs
//    (xh*Lh + xl*Lh + xh*Ll, fp32 accumulate) give each product to ~2^-16
//    relative.  The block scale multiplies the per-block MFMA partial once.
// The double-quant scale decode c*(absmax/127) is within 1 ulp of
// quant.rs:218's fl(fl(c/127)*absmax); it only enters this sum, never a
// stored weight.
#include <algorithm>
#include <type_traits>

#include "decode_common.h"

namespace qh {
namespace {

constexpr int kWaves = 4;

// Index (in uint4 units) of the A-fragment of (line, step, part, m, g);
// part 0 = hi, 1 = lo.  One line holds kFragsPerLine * M uint4.
constexpr int kFragsPerLine = 8 * 2 * 4;
__device__ __forceinline__ int64_t frag_index(int64_t line, int s, int part, int M, int m, int g) {
  return ((line * 8 + s) * 2 + part) * (int64_t)M * 4 + m * 4 + g;
}

constexpr int kRedFloats = 8192;  // LDS of the prep's final T1 reduction
constexpr int kRedBatch = 16;     // loads in flight per thread there

// ---------------------------------------------------------------------------
// Prep: grid = K / 256 workgroups of 256 threads (workgroup c = line c).
template <int XBF16>
__global__ __launch_bounds__(256) void k_dprep(const void *__restrict__ x, int M, int64_t K,
                                               const float *__restrict__ a, int r,
                                               uint4 *__restrict__ xf, float *__restrict__ t1p,
                                               float *__restrict__ t1,
                                               unsigned *__restrict__ ticket) {
  __shared__ int last;
  __shared__ float red[kRedFloats];
  const int c = blockIdx.x, P = gridDim.x, tid = threadIdx.x, lane = tid & 63,
            wave = tid >> 6;
  const int64_t k0 = (int64_t)c * kLine;
  // 1. A-fragments of X for this line (bf16 X is its own hi part).
  for (int idx = tid; idx < M * 32; idx += 256) {
    const int m = idx >> 5, u = idx & 31, s = u >> 2, g = u & 3;
    const int64_t e = (int64_t)m * K + k0 + step_koff(s, g);
    uint4 hi, lo = make_uint4(0, 0, 0, 0);
    if (XBF16) {
      hi = *(const uint4 *)((const uint16_t *)x + e);
    } else {
      const float4 p0 = *(const float4 *)((const float *)x + e);
      const float4 p1 = *(const float4 *)((const float *)x + e + 4);
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
      hi = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      lo = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
    xf[frag_index(c, s, 0, M, m, g)] = hi;
    if (!XBF16) xf[frag_index(c, s, 1, M, m, g)] = lo;
  }
  if (r == 0) return;
  // 2. This line's partial of T1[m][j]: a lane covers 4 elements; rows j of
  //    A are spread over the waves (all loads issued first); the 16 padded
  //    batch rows are reduced at once.
  float4 xv[16], av[16];
#pragma unroll
  for (int m = 0; m < 16; ++m)
    xv[m] = m < M ? load_x4<XBF16>(x, (int64_t)m * K + k0 + 4 * lane)
                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int j = wave + kWaves * q;
    av[q] = j < r ? *(const float4 *)(a + (int64_t)j * K + k0 + 4 * lane)
                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int j = wave + kWaves * q;
    if (kWaves * q >= r) break;  // uniform: q stays a compile-time index
    float p[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      float t = xv[m].x * av[q].x;
      t = fmaf(xv[m].y, av[q].y, t);
      t = fmaf(xv[m].z, av[q].z, t);
      p[m] = fmaf(xv[m].w, av[q].w, t);
    }
    const float s = reduce16(p);
    const int m = lane >> 2;
    if ((lane & 3) == 0 && m < M && j < r) st_dev(t1p + ((int64_t)c * M + m) * r + j, s);
  }
  // 3. The last workgroup to arrive sums the partials in line order.  The
  //    partials go through LDS in output chunks; every thread issues its
  //    loads of a chunk together.
  if (!last_arrival(ticket, (unsigned)P, &last)) return;
  const int MR = M * r;
  const int oc = MR < kRedFloats / P ? MR : (kRedFloats / P > 0 ? kRedFloats / P : 1);
  for (int o0 = 0; o0 < MR; o0 += oc) {
    const int on = MR - o0 < oc ? MR - o0 : oc;
    const int cnt = P * on;  // partial (cc, o) at red[cc * on + (o - o0)]
    for (int base = 0; base < cnt; base += 256 * kRedBatch) {
      float v[kRedBatch];
#pragma unroll
      for (int q = 0; q < kRedBatch; ++q) {
        int i = base + tid + 256 * q;
        i = i < cnt ? i : cnt - 1;
        v[q] = ld_dev(t1p + (int64_t)(i / on) * MR + o0 + i % on);
      }
#pragma unroll
      for (int q = 0; q < kRedBatch; ++q) {
        const int i = base + tid + 256 * q;
        if (i < cnt) red[i] = v[q];
      }
    }
    __syncthreads();
    for (int o = tid; o < on; o += 256) {
      float sum = 0.0f;
      for (int cc = 0; cc < P; ++cc) sum += red[cc * on + o];
      t1[o0 + o] = sum;
    }
    __syncthreads();
  }
}

// Copies n 16-byte (W16) or 4-byte units from global to LDS with
// global_load_lds: no VGPR round trip, so nothing for the compiler to sink
// next to a use.  The LDS destination of a wave is its first lane's slot
// (wave-uniform, in M0); the caller waits (vmcnt) and syncs before reading.
// Straight-line code (at most MAXIT exec-masked copies per thread, 256
// threads): a loop would hide the number of later loads from the
// compiler's wait-count tracking.
template <bool W16, int MAXIT>
__device__ __forceinline__ void copy_to_lds(void *lds, const void *src, int n) {
  using Unit = typename std::conditional<W16, uint4, uint32_t>::type;
  typedef __attribute__((address_space(3))) void lds_void;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < MAXIT; ++q) {
    const int i = threadIdx.x + 256 * q;
    if (i < n) {
      const void *g = (const Unit *)src + i;
      lds_void *l = (lds_void *)((Unit *)lds + (i - lane));
      if (W16)
        __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------

// LDS operands of one 64-element block (MFMA steps 2j and 2j+1).
struct BlockOps {
  uint32_t h[2][4], l[2][4];  // weight hi / lo bf16 pairs per step
  uint4 xh[2], xl[2];         // A-fragments (X hi / lo) per step
};

template <int XLO>
__device__ __forceinline__ void fetch_block(BlockOps &o, const uint32_t (&sw)[8], int j,
                                            const uint4 *xl, int part, int xo,
                                            const uint32_t *tab1) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int s = 2 * j + t;
    const uint32_t wd = sw[s];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t0 = tab1[(wd >> (8 * i)) & 15u];
      const uint32_t t1 = tab1[(wd >> (8 * i + 4)) & 15u];
      o.h[t][i] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
      o.l[t][i] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
    }
    o.xh[t] = xl[s * 2 * part + xo];
    o.xl[t] = XLO ? xl[s * 2 * part + part + xo] : make_uint4(0, 0, 0, 0);
  }
}

template <int XLO>
__device__ __forceinline__ floatx4 mfma_block(const BlockOps &o) {
  floatx4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const bf16x8 bh = __builtin_bit_cast(bf16x8, make_uint4(o.h[t][0], o.h[t][1], o.h[t][2], o.h[t][3]));
    const bf16x8 bl = __builtin_bit_cast(bf16x8, make_uint4(o.l[t][0], o.l[t][1], o.l[t][2], o.l[t][3]));
    const bf16x8 ah = __builtin_bit_cast(bf16x8, o.xh[t]);
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, d, 0, 0, 0);
    if (XLO) {
      const bf16x8 al = __builtin_bit_cast(bf16x8, o.xl[t]);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, d, 0, 0, 0);
    }
    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, d, 0, 0, 0);
  }
  return d;
}

// One line of one 16-row group: xl points at the line's staged A-fragments
// (hi parts at [s*2*M*4], lo parts M*4 further).  The LDS operands of block
// j+1 are requested before block j's MFMAs so their latency overlaps.
template <int XLO, int KIND>
__device__ __forceinline__ void compute_line(const LineRegs &R, float amax, const uint4 *xl,
                                             int M, int xo, const uint32_t *tab1, floatx4 &acc) {
  uint32_t sw[8];
  {
    auto p = __builtin_amdgcn_permlane32_swap(R.c0.x, R.c0.y, false, false);
    sw[0] = p[0];
    sw[2] = p[1];
    p = __builtin_amdgcn_permlane32_swap(R.c0.z, R.c0.w, false, false);
    sw[1] = p[0];
    sw[3] = p[1];
    p = __builtin_amdgcn_permlane32_swap(R.c1.x, R.c1.y, false, false);
    sw[4] = p[0];
    sw[6] = p[1];
    p = __builtin_amdgcn_permlane32_swap(R.c1.z, R.c1.w, false, false);
    sw[5] = p[0];
    sw[7] = p[1];
  }
  const float amax127 = amax * (1.0f / 127.0f);
  const int part = M * 4;
  BlockOps ops[2];
  fetch_block<XLO>(ops[0], sw, 0, xl, part, xo, tab1);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < 3) fetch_block<XLO>(ops[(j + 1) & 1], sw, j + 1, xl, part, xo, tab1);
    const floatx4 d = mfma_block<XLO>(ops[j & 1]);
    float sc;
    if (KIND == 0) {
      sc = __uint_as_float(j == 0 ? R.sf.x : j == 1 ? R.sf.y : j == 2 ? R.sf.z : R.sf.w);
    } else {
      sc = (float)(int8_t)((R.sf.x >> (8 * j)) & 255u) * amax127;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = fmaf(sc, d[v], acc[v]);
  }
}

constexpr int kRing = 4;       // code lines per wave (at most)
constexpr int kInFlight = 2;   // of which in flight at once (small-batch path)
constexpr int kStage = 12;     // staged A-fragment uint4 per thread (48 KB)
constexpr int kMaxSplits = 8;   // K split the grid-size target may ask for
constexpr int kSplitBatch = 8;  // slice partials loaded together

// Main: grid = ntiles * S workgroups of 256 threads; workgroup (tile, slice)
// covers rows [16 tile, 16 tile + 16) and lines [NL slice / S, NL (slice+1) / S).
// Dynamic LDS: the slice's A-fragments (lines * kFragsPerLine * M uint4),
// reused by the epilogue.
template <int XLO, int KIND>
__global__ __launch_bounds__(256) void k_dmain(DevQW w, int M, int S, const uint4 *__restrict__ xf,
                                               const float *__restrict__ t1,
                                               const float *__restrict__ lb, int r,
                                               float s_lora, float *__restrict__ part,
                                               unsigned *__restrict__ counters,
                                               float *__restrict__ y) {
  extern __shared__ uint4 xs[];
  __shared__ uint32_t tab1[16];
  __shared__ float lbs[16 * 64];  // rows n0.. of B (16 x r)
  __shared__ float t1s[16 * 64];  // T1 (M x r)
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t N = w.rows, K = w.cols, KB = K >> 6, NL = K / kLine;
  const int64_t ntiles = (N + 15) / 16;
  const int64_t tile = blockIdx.x % ntiles, slice = blockIdx.x / ntiles;
  const int64_t n0 = tile * 16;
  const int64_t SL0 = NL * slice / S, SL1 = NL * (slice + 1) / S, nls = SL1 - SL0;
  const int64_t wl0 = SL0 + nls * wave / kWaves, wl1 = SL0 + nls * (wave + 1) / kWaves;
  const int64_t nw = wl1 - wl0;

  const int nl = lane & 15, g = lane >> 4;
  const int64_t n = n0 + nl < N ? n0 + nl : N - 1;
  const uint8_t *crow = w.codes + n * (K >> 1);

  // Load order matters: vmcnt retires loads in issue order.  The slice's
  // A-fragments and the LoRA epilogue operands (L2-resident, small) go to
  // LDS first, then every code line of this wave (<= kRing of them: each
  // line's MFMAs wait only for its own bytes).
  // Every LDS fill of the prologue is a global_load_lds: an ordinary LDS
  // store here would make the compiler wait for all of them (and, in
  // issue order, for the code lines behind them).
  copy_to_lds<false, 1>(tab1, c_tab.nib, 16);
  const int64_t per_line = kFragsPerLine * (int64_t)M;
  copy_to_lds<true, kStage>(xs, xf + SL0 * per_line, (int)(nls * per_line));
  const int nrows = (int)(N - n0 < 16 ? N - n0 : 16);
  if (r > 0) {
    copy_to_lds<false, 4>(lbs, lb + n0 * r, nrows * r);
    copy_to_lds<false, 4>(t1s, t1, M * r);
  }
  __builtin_amdgcn_sched_barrier(0);  // the code loads stay behind the copies
  // absmax: a 256-block group spans 64 lines of a row, so the wave's lines
  // see at most two values (loaded before the lines: the first line needs
  // them).
  float am0 = 0.0f, am1 = 0.0f;
  if (KIND == 1) {
    const int64_t lf = nw > 0 ? wl0 : SL0, ll = nw > 0 ? wl1 - 1 : SL0;
    am0 = w.absmax[(n * KB + 4 * lf) >> 8];
    am1 = w.absmax[(n * KB + 4 * ll) >> 8];
  }
  __builtin_amdgcn_sched_barrier(0);
  LineRegs R[kRing];
#pragma unroll
  for (int d = 0; d < kRing; ++d) {
    const int64_t L = wl0 + d;
    load_line<KIND>(R[d], w, n, KB, crow, L < wl1 ? L : (nw > 0 ? wl1 - 1 : SL0), g);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Wait for the LDS copies only: the kAfter loads issued after them (the
  // code lines) stay in flight through the barrier.
  __builtin_amdgcn_s_waitcnt(vmcnt_only(KIND == 1 ? 3 * kRing + 2 : 3 * kRing));
  __builtin_amdgcn_s_barrier();  // no fence: a fence would wait for everything

  // A-fragment rows m >= M only reach output rows that are discarded:
  // those lanes read row M-1's fragment instead of branching.
  const int xo = (nl < M ? nl : M - 1) * 4 + g;
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t g0 = (n * KB + 4 * (nw > 0 ? wl0 : SL0)) >> 8;
#pragma unroll
  for (int d = 0; d < kRing; ++d) {
    if (d < nw) {
      const float amax = ((n * KB + 4 * (wl0 + d)) >> 8) == g0 ? am0 : am1;
      compute_line<XLO, KIND>(R[d], amax, xs + (wl0 + d - SL0) * kFragsPerLine * M, M, xo,
                              tab1, acc);
    }
  }

  // Epilogue.  Lane holds D[batch 4g+v][row nl]; waves reduce in LDS in a
  // fixed order.  The staged fragments are dead: reuse their LDS.
  __syncthreads();
  float *red = (float *)xs;  // kWaves x 256
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave * 256 + (4 * g + v) * 16 + nl] = acc[v];
  __syncthreads();
  const int bm = tid >> 4, ri = tid & 15;
  const int64_t nn = n0 + ri;
  const bool mine = bm < M && nn < N;
  float sum = 0.0f;
  if (mine) sum = (red[tid] + red[256 + tid]) + (red[512 + tid] + red[768 + tid]);
  if (S > 1) {
    if (mine) st_dev(part + (slice * M + bm) * N + nn, sum);
    if (!last_arrival(counters + tile, (unsigned)S, &last)) return;
    if (!mine) return;
    sum = 0.0f;
    for (int s0 = 0; s0 < S; s0 += kSplitBatch) {
      float v[kSplitBatch];
#pragma unroll
      for (int q = 0; q < kSplitBatch; ++q) {
        const int64_t sl = s0 + q < S ? s0 + q : S - 1;
        v[q] = ld_dev(part + (sl * M + bm) * N + nn);
      }
#pragma unroll
      for (int q = 0; q < kSplitBatch; ++q)
        if (s0 + q < S) sum += v[q];
    }
  }
  if (!mine) return;
  if (r > 0) {
    float l = 0.0f;
    for (int j = 0; j < r; ++j) l = fmaf(t1s[bm * r + j], lbs[ri * r + j], l);
    sum = fmaf(s_lora, l, sum);
  }
  y[(int64_t)bm * N + nn] = sum;
}

// ===========================================================================
// Small-batch decode (at most 8 rows): k_t1p + k_dsmall.
//
// MFMA operand packing.  The A-fragment rows carry both bf16 parts of X:
// row m < M holds hi(x_m) and row M+m holds lo(x_m) = bf16(x_m - hi).  The B
// operand interleaves the weight's parts exactly as the byte-pair table
// stores them, [Lh_a Lh_b Ll_a Ll_b Lh_c Lh_d Ll_c Ll_d] for elements a..d,
// and the A slots repeat each element to match, [q_a q_b q_a q_b q_c q_d q_c
// q_d].  One MFMA therefore accumulates q*(Lh+Ll) over 4 elements in every
// row, and y[m] = D[m] + D[M+m] = (xh+xl)(Lh+Ll) minus the negligible
// xl*Ll term: two MFMAs per 8 elements per lane, table entries used in place.
//
// k_t1p writes one partial of T1 = X A^T per 256-element line of K; the GEMV
// kernel loads those partials in its prologue (after its code loads, so they
// never delay the weight stream) and sums them in line order in its
// epilogue.  Its workgroups are (16-row tile, K slice); a tile's last slice
// to finish adds the slices (fixed order) and the LoRA term.
constexpr int kFusedMaxM = 8;
constexpr int kSmallRouteMaxM = 2;
// T1 partials prefetched per thread: covers NL * M * r <= 256 * 4M, i.e.
// K <= 16384 at r = 16; the rest is read in the epilogue.
template <int M>
constexpr int t1_prefetch() { return 4 * M; }

// Fragment index (uint4) of (line-in-slice ll, step s, half p, row rho, group g).
__device__ __forceinline__ int ffrag(int ll, int s, int p, int M2, int rho, int g) {
  return ((ll * 8 + s) * 2 + p) * (M2 * 4) + rho * 4 + g;
}

template <int XBF16>
__device__ __forceinline__ void load_x4_any(const void *x, int64_t e, float (&v)[4]) {
  const float4 t = load_x4<XBF16>(x, e);
  v[0] = t.x;
  v[1] = t.y;
  v[2] = t.z;
  v[3] = t.w;
}

template <int KIND>
__device__ __forceinline__ void compute_line2(const LineRegs &R, float amax, float valid,
                                              const uint4 *xl, int M2, int xo,
                                              const uint2 *tab2, floatx4 &acc) {
  uint32_t sw[8];
  {
    auto p = __builtin_amdgcn_permlane32_swap(R.c0.x, R.c0.y, false, false);
    sw[0] = p[0];
    sw[2] = p[1];
    p = __builtin_amdgcn_permlane32_swap(R.c0.z, R.c0.w, false, false);
    sw[1] = p[0];
    sw[3] = p[1];
    p = __builtin_amdgcn_permlane32_swap(R.c1.x, R.c1.y, false, false);
    sw[4] = p[0];
    sw[6] = p[1];
    p = __builtin_amdgcn_permlane32_swap(R.c1.z, R.c1.w, false, false);
    sw[5] = p[0];
    sw[7] = p[1];
  }
  const float amax127 = amax * (1.0f / 127.0f) * valid;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    floatx4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int s = 2 * j + t;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint2 e0 = tab2[(sw[s] >> (16 * p)) & 255u];
        const uint2 e1 = tab2[(sw[s] >> (16 * p + 8)) & 255u];
        const bf16x8 b = __builtin_bit_cast(bf16x8, make_uint4(e0.x, e0.y, e1.x, e1.y));
        const bf16x8 a = __builtin_bit_cast(bf16x8, xl[(s * 2 + p) * (M2 * 4) + xo]);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, d, 0, 0, 0);
      }
    }
    float sc;
    if (KIND == 0) {
      sc = __uint_as_float(j == 0 ? R.sf.x : j == 1 ? R.sf.y : j == 2 ? R.sf.z : R.sf.w) *
           valid;
    } else {
      sc = (float)(int8_t)((R.sf.x >> (8 * j)) & 255u) * amax127;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = fmaf(sc, d[v], acc[v]);
  }
}

// T1 partial of line c (workgroup c of K / 256): a lane covers
// 4 elements, rows j of A are spread over the waves; every load is issued
// before the first use.
template <int XBF16, int M>
__global__ __launch_bounds__(256) void k_t1p(const void *__restrict__ x, int64_t K,
                                             const float *__restrict__ a, int r,
                                             float *__restrict__ t1p) {
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t k = (int64_t)c * kLine + 4 * lane;
  float4 xv[M], av[16];
#pragma unroll
  for (int m = 0; m < M; ++m) xv[m] = load_x4<XBF16>(x, (int64_t)m * K + k);
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int j = wave + kWaves * q;
    av[q] = j < r ? *(const float4 *)(a + (int64_t)j * K + k)
                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int j = wave + kWaves * q;
    if (kWaves * q >= r) break;  // uniform: q stays a compile-time index
    float p[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      p[m] = 0.0f;
      if (m < M) {
        float t = xv[m].x * av[q].x;
        t = fmaf(xv[m].y, av[q].y, t);
        t = fmaf(xv[m].z, av[q].z, t);
        p[m] = fmaf(xv[m].w, av[q].w, t);
      }
    }
    const float s = reduce16(p);
    const int m = lane >> 2;
    if ((lane & 3) == 0 && m < M && j < r) t1p[((int64_t)c * M + m) * r + j] = s;
  }
}

// grid = ntiles * S workgroups of 256 threads.  Dynamic LDS: the slice's
// A-fragments (lines * 128 * M uint4), reused by the epilogue.
template <int XBF16, int KIND, int M>
__global__ __launch_bounds__(256) void k_dsmall(DevQW w, int S, const void *__restrict__ x,
                                                const float *__restrict__ t1p,
                                                const float *__restrict__ lb, int r,
                                                float s_lora, float *__restrict__ part,
                                                unsigned *__restrict__ counters,
                                                float *__restrict__ t1_out,
                                                float *__restrict__ y) {
  extern __shared__ uint4 xs[];
  __shared__ uint2 tabs[kWaves][256];  // one codebook table per wave
  __shared__ float lbs[16 * 64];
  __shared__ float t1s[kFusedMaxM * 64];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t N = w.rows, K = w.cols, KB = K >> 6, NL = K / kLine;
  const int64_t ntiles = (N + 15) / 16;
  const int64_t tile = blockIdx.x % ntiles, slice = blockIdx.x / ntiles;
  // Until the epilogue every wave works alone: its own table copy, its own
  // lines' A-fragments in its own LDS region, no workgroup barrier, so it
  // starts on its first line as soon as its own loads land.
  uint4 *xw = xs + wave * (kRing * 128 * M);
  uint2 *tab2 = tabs[wave];
  const int64_t n0 = tile * 16;
  const int64_t SL0 = NL * slice / S, SL1 = NL * (slice + 1) / S, nls = SL1 - SL0;
  const int64_t wl0 = SL0 + nls * wave / kWaves, wl1 = SL0 + nls * (wave + 1) / kWaves;
  const int64_t nw = wl1 - wl0;
  const int M2 = 2 * M;
  const int nl = lane & 15, g = lane >> 4;
  const int64_t n = n0 + nl < N ? n0 + nl : N - 1;
  const uint8_t *crow = w.codes + n * (K >> 1);

  // Prologue, all straight-line.  Phase 1: the codebook table and this
  // wave's X, converted into A-fragments.  Phase 2: the wave's code lines
  // and scales, then the LoRA operands of the epilogue (vmcnt retires loads
  // in issue order, so each line's MFMAs wait only for that line).
  uint2 tv[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    tv[q] = make_uint2(c_tab.pair[lane + 64 * q][0], c_tab.pair[lane + 64 * q][1]);
  // Unit u = t * 4M + (m * 4 + gg) with t = 16 ll + 2 s + p: 4 elements of
  // row m for lane group gg in half p of step s of the wave's line ll.
  constexpr int kUnits = kRing * M;  // per lane
  const int units = (int)(nw > 0 ? nw : 1) * 64 * M;
  float xv[kUnits][4];
#pragma unroll
  for (int q = 0; q < kUnits; ++q) {
    int u = lane + 64 * q;
    u = u < units ? u : units - 1;
    const int t = u / (4 * M), wi = u % (4 * M);
    const int ll = t >> 4, s = (t >> 1) & 7, p = t & 1, m = wi >> 2, gg = wi & 3;
    const int64_t L = nw > 0 ? wl0 + ll : SL0;
    const int64_t e = (int64_t)m * K + L * kLine + step_koff(s, gg) + 4 * p;
    load_x4_any<XBF16>(x, e, xv[q]);
  }
  // Phase 1 ends here: the table and X have landed (they were alone in
  // the memory pipeline, so they come back fast); only now do the code
  // lines go out.  Issued first, they would queue the small loads of every
  // later wave behind the weight stream.
  // Convert X: hi part to row m, lo part to row M+m, elements repeated in
  // pairs to match the interleaved B operand.
#pragma unroll
  for (int q = 0; q < 4; ++q) tab2[lane + 64 * q] = tv[q];
#pragma unroll
  for (int q = 0; q < kUnits; ++q) {
    int u = lane + 64 * q;
    u = u < units ? u : units - 1;
    const int t = u / (4 * M), wi = u % (4 * M);
    uint32_t h[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = bf16_bits_rne(xv[q][i]);
      lo[i] = XBF16 ? 0u : bf16_bits_rne(xv[q][i] - __uint_as_float(h[i] << 16));
    }
    const uint32_t h01 = h[0] | (h[1] << 16), h23 = h[2] | (h[3] << 16);
    const uint32_t l01 = lo[0] | (lo[1] << 16), l23 = lo[2] | (lo[3] << 16);
    xw[t * (8 * M) + wi] = make_uint4(h01, h01, h23, h23);          // row m
    xw[t * (8 * M) + 4 * M + wi] = make_uint4(l01, l01, l23, l23);  // row M + m
  }
  // A wave's LDS operations complete in order: its lookups see its writes.
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_sched_barrier(0);
  float am0 = 0.0f, am1 = 0.0f;
  if (KIND == 1) {
    const int64_t lf = nw > 0 ? wl0 : SL0, ll = nw > 0 ? wl1 - 1 : SL0;
    am0 = w.absmax[(n * KB + 4 * lf) >> 8];
    am1 = w.absmax[(n * KB + 4 * ll) >> 8];
  }
  // The wave's lines stream through a ring of kInFlight registers sets:
  // enough to keep HBM busy, short enough to keep the memory queues short.
  auto line_of = [&](int d) -> int64_t {
    return d < nw ? wl0 + d : (nw > 0 ? wl1 - 1 : SL0);
  };
  LineRegs R[kInFlight];
#pragma unroll
  for (int d = 0; d < kInFlight; ++d) load_line<KIND>(R[d], w, n, KB, crow, line_of(d), g);
  __builtin_amdgcn_sched_barrier(0);
  const int rr = r > 0 ? r : 1;
  float lbv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (r > 0) {  // without an adapter lb is NULL
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = tid + 256 * q;
      const int i16 = idx < 16 * r ? idx : 16 * r - 1;
      int64_t row = n0 + i16 / r;
      row = row < N ? row : N - 1;
      lbv[q] = lb[row * r + i16 % r];
    }
  }
  // T1 partials (P = NL lines x M*r): the first 256 * kT1Pre are loaded now.
  const int MR = M * r, PMR = (int)NL * MR;
  constexpr int kT1Pre = t1_prefetch<M>();
  float t1v[kT1Pre];
  if (r > 0) {
#pragma unroll
    for (int q = 0; q < kT1Pre; ++q) {
      const int i = tid + 256 * q;
      t1v[q] = t1p[i < PMR ? i : PMR - 1];
    }
  }

  // A-fragment rows >= 2M only reach discarded output rows: read row 2M-1.
  const int xo = (nl < M2 ? nl : M2 - 1) * 4 + g;
  const int64_t g0 = (n * KB + 4 * (nw > 0 ? wl0 : SL0)) >> 8;
  // Straight-line over the ring (no branch per line: a branch makes the
  // compiler shuffle ring registers that still have loads in flight); a
  // padded line past the wave's range contributes with scale 0.
  floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int d = 0; d < kRing; ++d) {
    const int64_t L = line_of(d);
    const float amax = ((n * KB + 4 * L) >> 8) == g0 ? am0 : am1;
    compute_line2<KIND>(R[d % kInFlight], amax, d < nw ? 1.0f : 0.0f,
                        xw + ffrag((int)(L - (nw > 0 ? wl0 : SL0)), 0, 0, M2, 0, 0), M2, xo,
                        tab2, acc);
    if (d + kInFlight < kRing)  // compile-time: unrolled
      load_line<KIND>(R[d % kInFlight], w, n, KB, crow, line_of(d + kInFlight), g);
  }

  // Epilogue: waves reduce in LDS (fixed order), rows m and M+m add up.
  __syncthreads();
  float *red = (float *)xs;           // kWaves x 256
  float *t1all = red + kWaves * 256;  // the prefetched T1 partials
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave * 256 + (4 * g + v) * 16 + nl] = acc[v];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int idx = tid + 256 * q;
    lbs[idx < 16 * rr ? idx : 16 * rr - 1] = lbv[q];
  }
  if (r > 0) {
#pragma unroll
    for (int q = 0; q < kT1Pre; ++q) {
      const int i = tid + 256 * q;
      if (i < PMR) t1all[i] = t1v[q];
    }
  }
  __syncthreads();
  const int bm = tid >> 4, ri = tid & 15;
  const int64_t nn = n0 + ri;
  const bool mine = bm < M && nn < N;
  float sum = 0.0f;
  if (mine) {
    const int hi = bm * 16 + ri, lo = (M + bm) * 16 + ri;
    sum = ((red[hi] + red[256 + hi]) + (red[512 + hi] + red[768 + hi])) +
          ((red[lo] + red[256 + lo]) + (red[512 + lo] + red[768 + lo]));
  }
  bool finisher = true;
  if (S > 1) {
    if (mine) st_dev(part + (slice * M + bm) * N + nn, sum);
    finisher = last_arrival(counters + tile, (unsigned)S, &last);
    if (finisher && mine) {
      sum = 0.0f;
      for (int s0 = 0; s0 < S; s0 += kSplitBatch) {
        float v[kSplitBatch];
#pragma unroll
        for (int q = 0; q < kSplitBatch; ++q) {
          const int64_t sl = s0 + q < S ? s0 + q : S - 1;
          v[q] = ld_dev(part + (sl * M + bm) * N + nn);
        }
#pragma unroll
        for (int q = 0; q < kSplitBatch; ++q)
          if (s0 + q < S) sum += v[q];
      }
    }
  }
  if (!finisher) return;
  if (r > 0) {
    // T1[o] = sum of the NL line partials, in a fixed order: thread (o, q)
    // of G = 256 / MR threads per output adds lines q, q+G, ...; the G
    // sums then add up in q order (partials past the prefetched ones are
    // read now).
    const int G = 256 / MR, o = tid % MR, q = tid / MR;
    float t = 0.0f;
    if (q < G) {
      for (int c = q; c < (int)NL; c += G) {
        const int i = c * MR + o;
        t += i < 256 * kT1Pre ? t1all[i] : t1p[i];
      }
    }
    __syncthreads();  // t1all is read; reuse red[] for the G sums
    if (q < G) red[q * MR + o] = t;
    __syncthreads();
    if (tid < MR) {
      float u = 0.0f;
      for (int c = 0; c < G; ++c) u += red[c * MR + tid];
      t1s[tid] = u;
      if (t1_out && tile == 0) t1_out[tid] = u;
    }
    __syncthreads();
    if (mine) {
      float l = 0.0f;
      for (int j = 0; j < r; ++j) l = fmaf(t1s[bm * r + j], lbs[ri * r + j], l);
      sum = fmaf(s_lora, l, sum);
    }
  }
  if (mine) y[(int64_t)bm * N + nn] = sum;
}

template <int M>
hipError_t run_small(const DevQW &w, int x_bf16, int S, const void *x, const float *t1p,
                     const float *lb, int r, float s, float *part, unsigned *counters,
                     float *t1_out, float *y, dim3 grid, uint32_t lds, hipStream_t st) {
  if (x_bf16) {
    if (w.kind == 0)
      return qh_launch(k_dsmall<1, 0, M>, grid, dim3(256), lds, st, w, S, x, t1p, lb, r, s,
                       part, counters, t1_out, y);
    return qh_launch(k_dsmall<1, 1, M>, grid, dim3(256), lds, st, w, S, x, t1p, lb, r, s, part,
                     counters, t1_out, y);
  }
  if (w.kind == 0)
    return qh_launch(k_dsmall<0, 0, M>, grid, dim3(256), lds, st, w, S, x, t1p, lb, r, s, part,
                     counters, t1_out, y);
  return qh_launch(k_dsmall<0, 1, M>, grid, dim3(256), lds, st, w, S, x, t1p, lb, r, s, part,
                   counters, t1_out, y);
}

template <int M>
hipError_t run_t1p(int x_bf16, const void *x, int64_t K, const float *a, int r, float *t1p,
                   hipStream_t st) {
  const dim3 grid((unsigned)(K / kLine));
  if (x_bf16) return qh_launch(k_t1p<1, M>, grid, dim3(256), 0, st, x, K, a, r, t1p);
  return qh_launch(k_t1p<0, M>, grid, dim3(256), 0, st, x, K, a, r, t1p);
}

constexpr int kSplitTarget = 512;  // workgroups the K split aims for

// Split of K over workgroups: the grid reaches kSplitTarget workgroups
// (at most kMaxSplits slices for that), and more slices are taken while a
// slice's staged A-fragments exceed 256 * kStage uint4 of LDS or a wave
// would own more than kRing lines.
int64_t decode_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t NL = K / kLine, ntiles = (N + 15) / 16;
  int64_t s = (kSplitTarget + ntiles - 1) / ntiles;
  if (s > kMaxSplits) s = kMaxSplits;
  if (s > NL) s = NL;
  if (s < 1) s = 1;
  while (s < NL && ((NL + s - 1) / s * kFragsPerLine * M > 256 * kStage ||
                    (NL + s - 1) / s > kWaves * kRing))
    ++s;
  return s;
}

size_t main_lds_bytes(int64_t M, int64_t K, int64_t S) {
  const int64_t NL = K / kLine;
  const int64_t lines = (NL + S - 1) / S;
  size_t b = (size_t)lines * kFragsPerLine * M * 16;
  const size_t epi = kWaves * 256 * 4;  // wave reduction
  return b > epi ? b : epi;
}

template <int XLO, int KIND>
hipError_t run_main(const DevQW &w, int M, int S, const uint4 *xf, const float *t1,
                    const float *lb, int r, float s, float *part, unsigned *counters, float *y,
                    hipStream_t st) {
  const int64_t ntiles = (w.rows + 15) / 16;
  const dim3 grid((unsigned)(ntiles * S));
  const uint32_t lds = (uint32_t)main_lds_bytes(M, w.cols, S);
  return qh_launch(k_dmain<XLO, KIND>, grid, dim3(256), lds, st, w, M, S, xf, t1, lb, r, s,
                   part, counters, y);
}

struct DecodeScratch {
  uint4 *xf;
  float *t1p, *t1, *part;
};

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

DecodeScratch carve(void *scratch, int64_t M, int64_t N, int64_t K, int64_t r) {
  const int64_t P = K / kLine;
  const size_t xs = round256((size_t)P * kFragsPerLine * M * 16);
  const size_t ps = round256((size_t)P * M * (r ? r : 1) * 4);
  const size_t ts = round256((size_t)M * (r ? r : 1) * 4);
  (void)N;
  DecodeScratch d;
  d.xf = (uint4 *)scratch;
  d.t1p = (float *)((char *)scratch + xs);
  d.t1 = (float *)((char *)scratch + xs + ps);
  d.part = (float *)((char *)scratch + xs + ps + ts);
  return d;
}

// Small-batch split: waves own at most kRing lines and the grid aims at
// kSplitTarget workgroups (at most kMaxSplits slices for that).
int64_t fused_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t NL = K / kLine, ntiles = (N + 15) / 16;
  int64_t s = (kSplitTarget + ntiles - 1) / ntiles;
  if (s > kMaxSplits) s = kMaxSplits;
  if (s > NL) s = NL;
  if (s < 1) s = 1;
  while (s < NL && (NL + s - 1) / s > kWaves * kRing) ++s;
  return s;
}

}  // namespace


bool decode_ok(const DevQW &w, int64_t M, int64_t r) {
  return M >= 1 && M <= 16 && r <= 64 && w.bs == 64 && w.cols % kLine == 0 &&
         (w.rows + 15) / 16 <= kDecodeMaxTiles && (((uintptr_t)w.codes) & 15) == 0 &&
         (w.kind == 0 ? (((uintptr_t)w.scales) & 15) == 0
                      : (((uintptr_t)w.scale_codes) & 3) == 0);
}

size_t decode_scratch_bytes(int64_t M, int64_t N, int64_t K, int64_t r) {
  const int64_t P = K / kLine, S = decode_splits(M, N, K);
  return round256((size_t)P * kFragsPerLine * M * 16) + round256((size_t)P * M * (r ? r : 1) * 4) +
         round256((size_t)M * (r ? r : 1) * 4) + round256((size_t)S * M * N * 4);
}

bool decode_small_ok(const DevQW &w, int64_t M, int64_t r) {
  // Batches of 3..8 rows are supported by the kernels but measured faster
  // on the prep + main path, so the router only sends 1 and 2 here.
  return decode_ok(w, M, r) && M <= kSmallRouteMaxM && M * r <= 256;
}

size_t decode_small_scratch_bytes(int64_t M, int64_t N, int64_t K, int64_t r) {
  const int64_t NL = K / kLine, S = fused_splits(M, N, K);
  return round256((size_t)NL * M * (r ? r : 1) * 4) + round256((size_t)S * M * N * 4);
}

#define QH_SMALL_CASES(F) \
  F(1) F(2) F(3) F(4) F(5) F(6) F(7) F(8)

hipError_t launch_decode_t1(const DevQW &w, const void *x, int x_bf16, int64_t M,
                            const float *a, int64_t r, void *scratch, hipStream_t st) {
  if (r == 0) return hipSuccess;
  float *t1p = (float *)scratch;
  switch (M) {
#define QH_CASE(m) \
  case m: return run_t1p<m>(x_bf16, x, w.cols, a, (int)r, t1p, st);
    QH_SMALL_CASES(QH_CASE)
#undef QH_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_small(const DevQW &w, const void *x, int x_bf16, int64_t M,
                               const float *lb, int64_t r, float s, float *y, float *t1_out,
                               void *scratch, unsigned *tickets, hipStream_t st) {
  const int64_t N = w.rows, K = w.cols, NL = K / kLine;
  const int64_t S = fused_splits(M, N, K);
  const float *t1p = (const float *)scratch;
  float *part = (float *)((char *)scratch + round256((size_t)NL * M * (r ? r : 1) * 4));
  const size_t epi = (size_t)(kWaves * 256 + 256 * 4 * M) * 4;  // t1_prefetch<M>()
  const uint32_t lds = (uint32_t)std::max<size_t>((size_t)kWaves * kRing * 128 * M * 16, epi);
  const dim3 grid((unsigned)(((N + 15) / 16) * S));
  unsigned *counters = tickets + kDecodeTileCounterBase;
  switch (M) {
#define QH_CASE(m) \
  case m:          \
    return run_small<m>(w, x_bf16, (int)S, x, t1p, lb, (int)r, s, part, counters, t1_out, y, grid, lds, st);
    QH_SMALL_CASES(QH_CASE)
#undef QH_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_prep(const DevQW &w, const void *x, int x_bf16, int64_t M,
                              const float *a, int64_t r, float *t1_out, void *scratch,
                              unsigned *tickets, hipStream_t st) {
  const int64_t K = w.cols;
  const DecodeScratch d = carve(scratch, M, w.rows, K, r);
  float *t1 = t1_out ? t1_out : d.t1;
  const dim3 grid((unsigned)(K / kLine));
  if (x_bf16)
    return qh_launch(k_dprep<1>, grid, dim3(256), 0, st, x, (int)M, K, a, (int)r, d.xf,
                     d.t1p, t1, tickets);
  return qh_launch(k_dprep<0>, grid, dim3(256), 0, st, x, (int)M, K, a, (int)r, d.xf, d.t1p,
                   t1, tickets);
}

hipError_t launch_decode(const DevQW &w, int x_bf16, int64_t M, const float *lb, int64_t r,
                         float s, float *y, const float *t1_out, void *scratch,
                         unsigned *tickets, hipStream_t st) {
  const DecodeScratch d = carve(scratch, M, w.rows, w.cols, r);
  const float *t1 = t1_out ? t1_out : d.t1;
  const int S = (int)decode_splits(M, w.rows, w.cols);
  unsigned *counters = tickets + kDecodeTileCounterBase;
  if (x_bf16) {
    if (w.kind == 0)
      return run_main<0, 0>(w, (int)M, S, d.xf, t1, lb, (int)r, s, d.part, counters, y, st);
    return run_main<0, 1>(w, (int)M, S, d.xf, t1, lb, (int)r, s, d.part, counters, y, st);
  }
  if (w.kind == 0)
    return run_main<1, 0>(w, (int)M, S, d.xf, t1, lb, (int)r, s, d.part, counters, y, st);
  return run_main<1, 1>(w, (int)M, S, d.xf, t1, lb, (int)r, s, d.part, counters, y, st);
}

}  // namespace qh
