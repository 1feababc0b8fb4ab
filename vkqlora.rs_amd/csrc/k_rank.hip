// k_rank.hip -- the LoRA-rank GEMMs whose output is (rows x r), r <= 64:
//   T1 = X . A^T        (qlora.rs:95, 141; lora.rs:94-102)
//   Ds = s * dY . B     (qlora.rs:143, 149)
// out[m][j] = alpha * sum_k P[m][k] * Q(j, k), P (M x K) row-major in fp32
// or bf16, Q either A (r x K, Q(j,k) = q[j * ldq + k]) or B (K x r,
// Q(j,k) = q[k * ldq + j]).
//
// At training shapes these are skinny (r = 8..64 columns, K = 192..2048):
// the tile engine's 64x64 tiles waste most of each MFMA and walk K in
// dependent 32-wide steps, so they ran 10-15 us each at C4's shapes.  Here a
// workgroup of 8 waves owns 16 rows and every wave one eighth of K, so each
// wave's chain is short; the eight partial tiles are summed through LDS in
// wave order (no split-K, no second launch).
//
// v_mfma_f32_16x16x4f32 takes, per lane l, one A value A[l % 16][k_l] and one
// B value B[k_l][l % 16] with k_l one of the step's four reduction indices
// (lane quarters 0-15, 16-31, 32-47, 48-63).  The reduction order is free,
// so chunk t of 16 k values gives lane quarter g = l / 16 the indices
// 16t + 4g + e for the chunk's four steps e = 0..3: a lane's four A values
// are one float4 of its row.
#include "qh_internal.h"

namespace qh {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRankWaves = 8;
constexpr int kRankThreads = kRankWaves * 64;
constexpr int kRankRows = 16;
constexpr int kRankUnroll = 4;  // chunks of 16 k loaded before their MFMAs

__device__ __forceinline__ float bf16f(uint32_t h) { return __uint_as_float(h << 16); }

// NB blocks of 16 output columns (r <= 16 * NB); job blockIdx.y of `jobs`.
template <int QF, int PE, int NB>
__global__ __launch_bounds__(kRankThreads) void k_rank_gemm(RankJobs jobs, int64_t M) {
  __shared__ float red[kRankWaves][kRankRows][16 * NB + 1];
  const RankJob &jb = jobs.j[blockIdx.y];
  const void *__restrict__ P = jb.p;
  const float *__restrict__ Q = jb.q;
  float *__restrict__ out = jb.out;
  const int64_t ldp = jb.ldp, ldq = jb.ldq, ldo = jb.ldo, K = jb.k;
  const int r = jb.r;
  const float alpha = jb.alpha;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.x * kRankRows;
  const int64_t row = m0 + l16;
  const bool row_ok = row < M;
  // this wave's K range, whole chunks of 16
  const int64_t chunks = (K + 15) / 16;
  const int64_t c0 = chunks * wv / kRankWaves, c1 = chunks * (wv + 1) / kRankWaves;

  floatx4 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[b][v] = 0.0f;

  auto load_p = [&](int64_t k, float (&p)[4]) {
    // P[row][k .. k+3], zero past the row's end or K
    if (PE == E_F32) {
      const float *pr = (const float *)P + row * ldp;
      if (row_ok && k + 3 < K && (((uintptr_t)(pr + k)) & 15) == 0) {
        const float4 v = *(const float4 *)(pr + k);
        p[0] = v.x; p[1] = v.y; p[2] = v.z; p[3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = (row_ok && k + e < K) ? pr[k + e] : 0.0f;
      }
    } else {
      const uint16_t *pr = (const uint16_t *)P + row * ldp;
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = (row_ok && k + e < K) ? bf16f(pr[k + e]) : 0.0f;
    }
  };
  auto load_q = [&](int b, int64_t k, float (&q)[4]) {
    const int j = b * 16 + l16;
    const bool j_ok = j < r;
    if (QF == 0) {
      const float *qr = Q + (int64_t)j * ldq;
      if (j_ok && k + 3 < K && (((uintptr_t)(qr + k)) & 15) == 0) {
        const float4 v = *(const float4 *)(qr + k);
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = (j_ok && k + e < K) ? qr[k + e] : 0.0f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = (j_ok && k + e < K) ? Q[(k + e) * ldq + j] : 0.0f;
    }
  };

  for (int64_t c = c0; c < c1; c += kRankUnroll) {
    float p[kRankUnroll][4], q[kRankUnroll][NB][4];
#pragma unroll
    for (int u = 0; u < kRankUnroll; ++u) {
      const int64_t k = (c + u) * 16 + 4 * g;
      const bool live = c + u < c1;
      if (live) {
        load_p(k, p[u]);
#pragma unroll
        for (int b = 0; b < NB; ++b) load_q(b, k, q[u][b]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[u][e] = 0.0f;
#pragma unroll
          for (int b = 0; b < NB; ++b) q[u][b][e] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kRankUnroll; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[u][e], q[u][b][e], acc[b], 0, 0, 0);
  }

  // D layout of the 16x16x4 MFMA: value v of lane l is row 4(l/16) + v,
  // column l % 16
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wv][4 * g + v][b * 16 + l16] = acc[b][v];
  __syncthreads();
  for (int e = tid; e < kRankRows * 16 * NB; e += kRankThreads) {
    const int rr = e / (16 * NB), j = e % (16 * NB);
    const int64_t m = m0 + rr;
    if (m >= M || j >= r) continue;
    float s = red[0][rr][j];
#pragma unroll
    for (int w = 1; w < kRankWaves; ++w) s += red[w][rr][j];
    out[m * ldo + j] = alpha * s;
  }
}

// The LoRA-rank GEMMs that reduce over the tokens (qlora.rs:147, 151):
//   grad_B = s * dY^T . T1   (N x r)      grad_A = Ds^T . X   (r x K)
// out(c, j) = alpha * sum_m Big[m][c] * Small[m][j], Big (M x C) row-major in
// fp32 or bf16, Small (M x r) fp32; stored at out[c * ldo + j] (out_t = 0) or
// out[j * ldo + c] (out_t = 1).  A workgroup owns 16 columns c and all r, its
// 8 waves split the tokens; lane quarter g takes tokens 16t + 4g + e, so a
// lane's four A values are four rows of one column, coalesced across the
// quarter's 16 lanes.
template <int PE, int NB>
__global__ __launch_bounds__(kRankThreads) void k_rank_tgemm(RankJobs jobs, int64_t M) {
  __shared__ float red[kRankWaves][16][16 * NB + 1];
  const RankJob &jb = jobs.j[blockIdx.y];
  const void *__restrict__ Big = jb.p;
  const float *__restrict__ Small = jb.q;
  float *__restrict__ out = jb.out;
  const int64_t ldb = jb.ldp, lds = jb.ldq, ldo = jb.ldo, C = jb.k;
  const int r = jb.r, OT = jb.out_t;
  const float alpha = jb.alpha;
  if ((int64_t)blockIdx.x * 16 >= C) return;  // a shorter job of the launch
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 16;
  const int64_t col = c0 + l16;
  const bool col_ok = col < C;
  const int64_t chunks = (M + 15) / 16;
  const int64_t t0 = chunks * wv / kRankWaves, t1 = chunks * (wv + 1) / kRankWaves;
  floatx4 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[b][v] = 0.0f;
  for (int64_t t = t0; t < t1; t += kRankUnroll) {
    float p[kRankUnroll][4], q[kRankUnroll][NB][4];
#pragma unroll
    for (int u = 0; u < kRankUnroll; ++u) {
      const int64_t m = (t + u) * 16 + 4 * g;
      const bool live = t + u < t1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = live && m + e < M;
        if (PE == E_F32)
          p[u][e] = (ok && col_ok) ? ((const float *)Big)[(m + e) * ldb + col] : 0.0f;
        else
          p[u][e] = (ok && col_ok) ? bf16f(((const uint16_t *)Big)[(m + e) * ldb + col]) : 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int j = b * 16 + l16;
          q[u][b][e] = (ok && j < r) ? Small[(m + e) * lds + j] : 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kRankUnroll; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[u][e], q[u][b][e], acc[b], 0, 0, 0);
  }
  // row i of the 16x16 D (a column c of the output), column j
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wv][4 * g + v][b * 16 + l16] = acc[b][v];
  __syncthreads();
  for (int e = tid; e < 16 * 16 * NB; e += kRankThreads) {
    const int ci = e / (16 * NB), j = e % (16 * NB);
    const int64_t c = c0 + ci;
    if (c >= C || j >= r) continue;
    float s = red[0][ci][j];
#pragma unroll
    for (int w = 1; w < kRankWaves; ++w) s += red[w][ci][j];
    out[OT ? (int64_t)j * ldo + c : c * ldo + j] = alpha * s;
  }
}

}  // namespace

// Measured against the split-K tile engine: faster up to K = 2048 (C4's
// 576- and 1536-long T1 and Ds: 5-10 against 9-12 us), slower at K = 4096
// (C3's T1: 52 against 31 us), where a wave's K loop waits on its loads
// every kRankUnroll chunks and the tile engine's split-K has more waves.
bool rank_gemm_ok(int64_t K, int64_t r) { return r >= 1 && r <= 64 && K >= 1 && K <= 2048; }

hipError_t launch_rank_gemms(const RankJobs &jobs, int p_bf16, int q_kmajor, int64_t M,
                             hipStream_t s) {
  if (M == 0 || jobs.count == 0) return hipSuccess;
  int rmax = 0;
  for (int i = 0; i < jobs.count; ++i) rmax = jobs.j[i].r > rmax ? jobs.j[i].r : rmax;
  if (rmax == 0) return hipSuccess;
  const dim3 grid((unsigned)((M + kRankRows - 1) / kRankRows), (unsigned)jobs.count);
  const dim3 block(kRankThreads);
#define QH_RANK(QF, PE, NB) return qh_launch(k_rank_gemm<QF, PE, NB>, grid, block, 0, s, jobs, M)
#define QH_RANK_NB(NB)                       \
  if (q_kmajor) {                            \
    if (p_bf16) QH_RANK(1, E_BF16, NB);      \
    QH_RANK(1, E_F32, NB);                   \
  }                                          \
  if (p_bf16) QH_RANK(0, E_BF16, NB);        \
  QH_RANK(0, E_F32, NB);
  if (rmax <= 16) {
    QH_RANK_NB(1)
  }
  if (rmax <= 32) {
    QH_RANK_NB(2)
  }
  QH_RANK_NB(4)
#undef QH_RANK_NB
#undef QH_RANK
}

hipError_t launch_rank_gemm(const void *P, int p_bf16, int64_t ldp, const float *Q, int q_kmajor,
                            int64_t ldq, float *out, int64_t ldo, int64_t M, int64_t K, int64_t r,
                            float alpha, hipStream_t s) {
  RankJobs jobs{};
  jobs.count = 1;
  jobs.j[0] = RankJob{P, ldp, Q, ldq, out, ldo, K, (int)r, 0, alpha};
  return launch_rank_gemms(jobs, p_bf16, q_kmajor, M, s);
}

}  // namespace qh

namespace qh {

// Measured against the split-K tile engine: faster at 2048 tokens (C4's
// grad_A / grad_B: 8.5-9 against 10-12 us plus a reduction pass), slower at
// 4096 (C3's: 42-70 against 32 us), where each wave walks twice the tokens.
bool rank_tgemm_ok(int64_t M, int64_t r) { return r >= 1 && r <= 64 && M >= 1 && M <= 2048; }

hipError_t launch_rank_tgemms(const RankJobs &jobs, int big_bf16, int64_t M, hipStream_t s) {
  if (jobs.count == 0) return hipSuccess;
  int rmax = 0;
  int64_t cmax = 0;
  for (int i = 0; i < jobs.count; ++i) {
    rmax = jobs.j[i].r > rmax ? jobs.j[i].r : rmax;
    cmax = jobs.j[i].k > cmax ? jobs.j[i].k : cmax;
  }
  if (rmax == 0 || cmax == 0) return hipSuccess;
  const dim3 grid((unsigned)((cmax + 15) / 16), (unsigned)jobs.count), block(kRankThreads);
#define QH_RT(PE, NB) return qh_launch(k_rank_tgemm<PE, NB>, grid, block, 0, s, jobs, M)
#define QH_RT_NB(NB)                 \
  if (big_bf16) QH_RT(E_BF16, NB);   \
  QH_RT(E_F32, NB);
  if (rmax <= 16) {
    QH_RT_NB(1)
  }
  if (rmax <= 32) {
    QH_RT_NB(2)
  }
  QH_RT_NB(4)
#undef QH_RT_NB
#undef QH_RT
}

hipError_t launch_rank_tgemm(const void *Big, int big_bf16, int64_t ldb, const float *Small,
                             int64_t lds, float *out, int64_t ldo, int out_t, int64_t M,
                             int64_t C, int64_t r, float alpha, hipStream_t s) {
  RankJobs jobs{};
  jobs.count = 1;
  jobs.j[0] = RankJob{Big, ldb, Small, lds, out, ldo, C, (int)r, out_t, alpha};
  return launch_rank_tgemms(jobs, big_bf16, M, s);
}

}  // namespace qh
