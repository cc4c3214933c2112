// gfx950 kernels that fuse the elementwise steps of a layer with the
// per-group activation quantization the next W4A8 projection needs, and the
// decode/verify attention.  Same bit-exact contract as kernels.hip: every
// value is produced in the f32 operation order of rai's AVX2 path
// (rai-infer/src/layers.rs, gemm.rs).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <utility>

#include "exact_math.h"
#include "kernels.h"
#include "quant_dev.h"

namespace rai {

namespace {

// A pointer the compiler must treat as lane-varying: loads through it are
// vector loads (tracked in order by vmcnt) even when every lane reads the
// same address.  Scalar loads would be waited for all at once (lgkmcnt(0)),
// which serialises a software pipeline.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *vector_ptr(const T *p) {
  uintptr_t a = reinterpret_cast<uintptr_t>(p);
  asm volatile("" : "+v"(a));
  return reinterpret_cast<const __attribute__((address_space(1))) T *>(a);
}

// quantize_group8_to with row pointers: group at columns col0.. of the
// rows qs (block-split) and qn (natural, may be null).
template <int NB>
__device__ __forceinline__ void quantize_group8(const float (&v)[NB], int j, int col0, bool ok,
                                                int8_t *__restrict__ qs, int8_t *__restrict__ qn,
                                                float *__restrict__ scale_out,
                                                float *__restrict__ sum_out, _Float16 *qa_slot = nullptr) {
  quantize_group8_to<NB>(v, j, ok, qs + col0, qn ? qn + col0 : nullptr, scale_out, sum_out, qa_slot);
}

// ------------------------------------------------------ RMSNorm + quant --

// rms_norm_avx2 (layers.rs:325-376) of one token row followed by the
// per-group quantization of the normalised row (gemm.rs:147-374).  One
// 256-thread block per token; the row is staged in LDS.  The sum of squares
// runs as the reference's 16 FMA chains (lane c: j = c & 7 over the
// elements 16i + (c < 8 ? 0 : 8) + j, the trailing 8-block into chains
// 0..7), then lane-wise sq0 + sq1, hsum8 and the scalar tail.
template <int GS>
__global__ __launch_bounds__(256) void k_norm_quant(const float *__restrict__ x,
                                                    const float *__restrict__ w,
                                                    float *__restrict__ normed,
                                                    int8_t *__restrict__ q_split,
                                                    int8_t *__restrict__ q_nat,
                                                    float *__restrict__ scales,
                                                    float *__restrict__ sums, int n, float eps,
                                                    _Float16 *qa) {
  extern __shared__ float xs[];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *row = x + (size_t)t * n;
  if constexpr (GS > 0) {
    // n % 8 == 0 and GS | n (fused_quant_ok).
    const int groups = n / GS;
    rmsnorm_quant_block<GS>(row, w, n, eps, xs, q_split + (size_t)t * n, GS,
                            q_nat ? q_nat + (size_t)t * n : nullptr, scales + (size_t)t * groups,
                            sums + (size_t)t * groups, normed ? normed + (size_t)t * n : nullptr, qa, t);
  } else {
    // RMSNorm only (rms_norm / rms_norm_with_residual): out = (x*inv)*w.
    float *ws = xs + n;  // [n] row, then [n] weights
    __shared__ float chains[16];
    __shared__ float inv_sh;
    const int n4 = (n % 4 == 0) ? n / 4 : 0;  // rows stay 16-byte aligned
    for (int i = tid; i < n4; i += 256) {
      reinterpret_cast<float4 *>(xs)[i] = reinterpret_cast<const float4 *>(row)[i];
      reinterpret_cast<float4 *>(ws)[i] = reinterpret_cast<const float4 *>(w)[i];
    }
    for (int i = n4 * 4 + tid; i < n; i += 256) {
      xs[i] = row[i];
      ws[i] = w[i];
    }
    __syncthreads();
    const int c16 = (n / 8) / 2;
    const bool extra8 = 16 * c16 + 8 <= n;
    if (tid < 16) {
      const int j = tid & 7, off = tid < 8 ? 0 : 8;
      float a = 0.0f;
      int i = 0;
      for (; i + 32 <= c16; i += 32) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = xs[16 * (i + u) + off + j];
#pragma unroll
        for (int u = 0; u < 32; ++u) a = __fmaf_rn(v[u], v[u], a);
      }
      for (; i < c16; ++i) {
        const float v = xs[16 * i + off + j];
        a = __fmaf_rn(v, v, a);
      }
      if (tid < 8 && extra8) {
        const float v = xs[16 * c16 + j];
        a = __fmaf_rn(v, v, a);
      }
      chains[tid] = a;
    }
    __syncthreads();
    if (tid == 0) {
      float s[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] = chains[j] + chains[8 + j];
      float sum = ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
      for (int i = 16 * c16 + (extra8 ? 8 : 0); i < n; ++i) sum = sum + xs[i] * xs[i];
      // Correctly rounded sqrt and divide (the reference's sqrtss / divss).
      inv_sh = 1.0f / __builtin_sqrtf(sum / (float)n + eps);
    }
    __syncthreads();
    const float inv = inv_sh;
    float *nrow = normed + (size_t)t * n;
    for (int i = tid; i < n; i += 256) nrow[i] = (xs[i] * inv) * ws[i];
  }
}

// silu_mul_avx2 (layers.rs:850-883) on one token's gate/up rows (n a
// multiple of 8: every element takes the Schraudolph body) followed by the
// per-group quantization of the product for the down projection.  Grid
// (ceil(groups / 32), m), 256 threads, 8 lanes per group.
template <int GS>
__global__ __launch_bounds__(256) void k_silu_quant(float *__restrict__ gate,
                                                    const float *__restrict__ up, int n, int ld,
                                                    int8_t *__restrict__ q_split,
                                                    int8_t *__restrict__ q_nat,
                                                    float *__restrict__ scales,
                                                    float *__restrict__ sums, _Float16 *qa) {
  constexpr int NB = GS / 8;
  const int t = blockIdx.y;
  const int groups = n / GS;
  const int g = blockIdx.x * 32 + threadIdx.x / 8;
  const int j = threadIdx.x & 7;
  const bool ok = g < groups;
  const int col0 = (ok ? g : 0) * GS;
  float *gr = gate + (size_t)t * ld;
  const float *ur = up + (size_t)t * ld;
  float v[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) {
    const int col = col0 + 8 * c + j;
    if (ok) {
      const float xv = gr[col];
      const float e = rai_exact::schraudolph(xv * -1.0f);
      v[c] = (xv / (1.0f + e)) * ur[col];
      gr[col] = v[c];
    } else {
      v[c] = 0.0f;
    }
  }
  int8_t *qs = q_split + (size_t)t * n;
  int8_t *qn = q_nat ? q_nat + (size_t)t * n : nullptr;
  quantize_group8<NB>(v, j, col0, ok, qs, qn, scales + (size_t)t * groups + g,
                      sums + (size_t)t * groups + g, qa ? qa4_slot(qa, t, ok ? g : 0, groups) : nullptr);
}

// Per-group quantization of m rows of n (quantize_input_split +
// compute_input_sums, gemm.rs:147-374).  Grid (ceil(groups / 32), m).
template <int GS>
__global__ __launch_bounds__(256) void k_quant(const float *__restrict__ x, int n,
                                               int8_t *__restrict__ q_split,
                                               int8_t *__restrict__ q_nat,
                                               float *__restrict__ scales,
                                               float *__restrict__ sums, _Float16 *qa) {
  constexpr int NB = GS / 8;
  const int t = blockIdx.y;
  const int groups = n / GS;
  const int g = blockIdx.x * 32 + threadIdx.x / 8;
  const int j = threadIdx.x & 7;
  const bool ok = g < groups;
  const int col0 = (ok ? g : 0) * GS;
  const float *xr = x + (size_t)t * n;
  float v[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) v[c] = ok ? xr[col0 + 8 * c + j] : 0.0f;
  int8_t *qs = q_split + (size_t)t * n;
  int8_t *qn = q_nat ? q_nat + (size_t)t * n : nullptr;
  quantize_group8<NB>(v, j, col0, ok, qs, qn, scales + (size_t)t * groups + g,
                      sums + (size_t)t * groups + g, qa ? qa4_slot(qa, t, ok ? g : 0, groups) : nullptr);
}

// -------------------------------------------------------------- attention --
//
// attention_head_avx2 (layers.rs:1266-1380) for every (token, query head) in
// three kernels over a score buffer S [t][h][sstride]:
//   scores   S[s] = hsum8(8-lane FMA dot(q, k_s)) * scale for s <= pos;
//   softmax  mx = max S; e_s = Schraudolph(S_s - mx) on the first
//            8*floor(n/8) positions, expf on the tail; sum = hsum8 of the 8
//            lane chains (lane j adds e_{8i+j} in i order) plus the tail in
//            order; S[s] = e_s * (1/sum);
//   PV       out[d] = fma(p_s, v_s[d], out[d]) for s = 0..n-1 in order.

constexpr int kScoreTile = 64;  // positions per score block (one per lane)

// acc = fma(q, k, acc) with q taken from lane n of the lane's row of 16
// (DPP row_newbcast): a wave-uniform operand held once per 16 values.
template <int N>
__device__ __forceinline__ float fma_bcast(float q, float k, float acc) {
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(q), "v"(k), "n"(N));
  return acc;
}

__device__ __forceinline__ float fma_bcast_n(int n, float q, float k, float acc) {
  switch (n) {
    case 0: return fma_bcast<0>(q, k, acc);
    case 1: return fma_bcast<1>(q, k, acc);
    case 2: return fma_bcast<2>(q, k, acc);
    case 3: return fma_bcast<3>(q, k, acc);
    case 4: return fma_bcast<4>(q, k, acc);
    case 5: return fma_bcast<5>(q, k, acc);
    case 6: return fma_bcast<6>(q, k, acc);
    case 7: return fma_bcast<7>(q, k, acc);
    case 8: return fma_bcast<8>(q, k, acc);
    case 9: return fma_bcast<9>(q, k, acc);
    case 10: return fma_bcast<10>(q, k, acc);
    case 11: return fma_bcast<11>(q, k, acc);
    case 12: return fma_bcast<12>(q, k, acc);
    case 13: return fma_bcast<13>(q, k, acc);
    case 14: return fma_bcast<14>(q, k, acc);
    default: return fma_bcast<15>(q, k, acc);
  }
}

typedef float sf4 __attribute__((ext_vector_type(4)));

// One 8-column chunk C of the score chains of PB pairs (fully expanded so
// that the query register and the broadcast lane are compile-time).
template <int HD, int PB, int C>
__device__ __forceinline__ void score_chunk(const sf4 *kr4, const float (&qb)[PB][HD / 16], float (&a)[PB][8]) {
  const sf4 k0 = kr4[2 * C], k1 = kr4[2 * C + 1];
  const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
  for (int p = 0; p < PB; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) a[p][i] = fma_bcast_n((8 * C + i) & 15, qb[p][C >> 1], kv[i], a[p][i]);
}

template <int HD, int PB, int... Cs>
__device__ __forceinline__ void score_chunks(std::integer_sequence<int, Cs...>, const sf4 *kr4,
                                             const float (&qb)[PB][HD / 16], float (&a)[PB][8]) {
  (score_chunk<HD, PB, Cs>(kr4, qb, a), ...);
}

// The same with the next chunk's keys requested before this chunk's FMAs
// (k0, k1 hold chunk C's keys on entry, chunk C + 1's on exit).
template <int HD, int PB, int C>
__device__ __forceinline__ void score_chunk_p(const sf4 *kr4, const float (&qb)[PB][HD / 16], float (&a)[PB][8],
                                              sf4 &k0, sf4 &k1) {
  sf4 n0 = k0, n1 = k1;
  if constexpr (C + 1 < HD / 8) {
    n0 = kr4[2 * C + 2];
    n1 = kr4[2 * C + 3];
  }
  __builtin_amdgcn_sched_barrier(0);
  const float kv[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
  for (int p = 0; p < PB; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) a[p][i] = fma_bcast_n((8 * C + i) & 15, qb[p][C >> 1], kv[i], a[p][i]);
  __builtin_amdgcn_sched_barrier(0);
  k0 = n0;
  k1 = n1;
}

template <int HD, int PB, int... Cs>
__device__ __forceinline__ void score_chunks_pipe(std::integer_sequence<int, Cs...>, const sf4 *kr4,
                                                  const float (&qb)[PB][HD / 16], float (&a)[PB][8]) {
  sf4 k0 = kr4[0], k1 = kr4[1];
  (score_chunk_p<HD, PB, Cs>(kr4, qb, a, k0, k1), ...);
}

// grid (ceil(nmax / 64), nkv), 256 threads.  The block stages its 64 key
// rows in LDS; each wave takes (token, head) pairs of the kv group, lane =
// position.  HD > 0 (compile-time head_dim): key rows HD + 4 floats apart
// (16-byte reads, conflict-free per 16 lanes), followed by the query rows of
// the block's pairs (pair pi = (t - tfirst) * G + g at row pi, each wave's
// pairs read into registers 16 values per register and taken by the FMAs
// through DPP row_newbcast); a wave runs PB of its pairs at once, head-dim
// chunk outer, so each key value read serves PB dot products (pairs past the end repeat the
// last one and store nothing).  HD = 0: rows hd + 1 floats apart, queries
// from global memory, one pair at a time.  With a step record the token
// positions start at st[0] + toff.  grid.z splits the m tokens into groups
// of mb (the LDS holds one group's query rows): group z takes tokens
// z * mb.. as a launch of its own would.
template <int HD, int PB>
__global__ __launch_bounds__(256) void k_scores(const float *__restrict__ q, int q_ld,
                                                const float *__restrict__ kc, int cap, int pos0,
                                                int m, int nh, int nkv, int hd_rt, float scale,
                                                float *__restrict__ S, int sstride,
                                                const int *__restrict__ st, int toff, int mb) {
  extern __shared__ float ks[];
  {
    const int u0 = (int)blockIdx.z * mb;
    m = min(mb, m - u0);
    q += (size_t)u0 * q_ld;
    S += (size_t)u0 * nh * sstride;
    pos0 += u0;
    toff += u0;
  }
  if (st) pos0 = st[0] + toff;
  const int hd = HD > 0 ? HD : hd_rt;
  const int kstride = HD > 0 ? HD + 4 : hd + 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int s0 = (int)blockIdx.x * kScoreTile;
  const int kvh = blockIdx.y;
  const int G = nh / nkv;
  const int nmax = pos0 + m;
  if (s0 >= nmax) return;  // capacity-sized grids (step record) end early
  const int rows = min(kScoreTile, nmax - s0);
  const float *kb = kc + ((size_t)kvh * cap + s0) * hd;
  // Token t sees positions <= pos0 + t.
  const int tfirst = s0 > pos0 ? s0 - pos0 : 0;
  const int pairs = G * (m - tfirst);
  typedef float f4 __attribute__((ext_vector_type(4)));
  if constexpr (HD > 0) {
    // All of the thread's key loads are issued before the first LDS store.
    constexpr int NPT = kScoreTile * (HD / 4) / 256;
    f4 v4[NPT];
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int i = threadIdx.x + 256 * u;
      const int r = min(i / (HD / 4), rows - 1), c4 = i % (HD / 4);
      v4[u] = reinterpret_cast<const f4 *>(kb + (size_t)r * HD)[c4];
    }
    f4 *lq = reinterpret_cast<f4 *>(ks + kScoreTile * kstride);
    for (int i = threadIdx.x; i < pairs * (HD / 4); i += 256) {
      const int pi = i / (HD / 4), c4 = i % (HD / 4);
      const int t = tfirst + pi / G, h = kvh * G + pi % G;
      lq[i] = reinterpret_cast<const f4 *>(q + (size_t)t * q_ld + (size_t)h * HD)[c4];
    }
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int i = threadIdx.x + 256 * u;
      const int r = i / (HD / 4), c4 = i % (HD / 4);
      *reinterpret_cast<f4 *>(ks + r * kstride + 4 * c4) = v4[u];
    }
    __syncthreads();
    const int s = s0 + lane;
    const f4 *kr4 = reinterpret_cast<const f4 *>(ks + lane * kstride);
    const int npw = (pairs - wave + 3) / 4;  // this wave's pairs: wave, wave + 4, ...
    for (int b0 = 0; b0 < npw; b0 += PB) {
      // The pairs' query rows, 16 values per register: lane l holds
      // q[16 m + l % 16] in qb[p][m]; the FMAs take q[e] from lane e % 16
      // of their row (one 4-byte LDS read per 16 values instead of a
      // broadcast 16-byte read per 4).
      float qb[PB][HD / 16];
#pragma unroll
      for (int p = 0; p < PB; ++p) {
        const float *qrow = reinterpret_cast<const float *>(lq + (wave + 4 * min(b0 + p, npw - 1)) * (HD / 4));
#pragma unroll
        for (int mm = 0; mm < HD / 16; ++mm) qb[p][mm] = qrow[16 * mm + (lane & 15)];
      }
      float a[PB][8];
#pragma unroll
      for (int p = 0; p < PB; ++p)
#pragma unroll
        for (int i = 0; i < 8; ++i) a[p][i] = 0.0f;
      score_chunks<HD, PB>(std::make_integer_sequence<int, HD / 8>{}, reinterpret_cast<const sf4 *>(kr4), qb, a);
#pragma unroll
      for (int p = 0; p < PB; ++p) {
        const int pi = wave + 4 * (b0 + p);
        const int t = tfirst + pi / G, h = kvh * G + pi % G;
        if (b0 + p < npw && lane < rows && s <= pos0 + t) {
          const float d = ((a[p][0] + a[p][4]) + (a[p][1] + a[p][5])) + ((a[p][2] + a[p][6]) + (a[p][3] + a[p][7]));
          S[((size_t)t * nh + h) * sstride + s] = d * scale;
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < rows * (hd / 4); i += 256) {
      const int r = i / (hd / 4), c4 = i - r * (hd / 4);
      const float4 v4 = reinterpret_cast<const float4 *>(kb + (size_t)r * hd)[c4];
      float *d = ks + r * kstride + 4 * c4;
      d[0] = v4.x;
      d[1] = v4.y;
      d[2] = v4.z;
      d[3] = v4.w;
    }
    __syncthreads();
    const int s = s0 + lane;
    const float *kr = ks + lane * kstride;
    for (int pi = wave; pi < pairs; pi += 4) {
      const int t = tfirst + pi / G;
      const int h = kvh * G + pi % G;
      const auto *qh = vector_ptr(reinterpret_cast<const f4 *>(q + (size_t)t * q_ld + (size_t)h * hd));
      float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (lane < rows) {
        for (int c = 0; c < hd / 8; ++c) {
          const f4 q0 = qh[2 * c];
          const f4 q1 = qh[2 * c + 1];
          const float *k8 = kr + 8 * c;
          a[0] = __fmaf_rn(q0.x, k8[0], a[0]);
          a[1] = __fmaf_rn(q0.y, k8[1], a[1]);
          a[2] = __fmaf_rn(q0.z, k8[2], a[2]);
          a[3] = __fmaf_rn(q0.w, k8[3], a[3]);
          a[4] = __fmaf_rn(q1.x, k8[4], a[4]);
          a[5] = __fmaf_rn(q1.y, k8[5], a[5]);
          a[6] = __fmaf_rn(q1.z, k8[6], a[6]);
          a[7] = __fmaf_rn(q1.w, k8[7], a[7]);
        }
      }
      if (lane < rows && s <= pos0 + t) {
        const float d = ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
        S[((size_t)t * nh + h) * sstride + s] = d * scale;
      }
    }
  }
}

// Scores of batches of more than 12 tokens (compile-time head_dim, the
// prefill): k_scores' arithmetic in blocks of eight waves that stage their
// token group's query rows once and walk several 64-position key tiles, the
// next tile's keys loaded into registers while the current one is computed
// (two LDS key buffers).  Block (b, kv head, group z) takes tiles b, b + ns,
// ... of the group; wave w takes the tile's pairs w, w + 8, ..., PB at a
// time.  ns is chosen so that the grid's blocks are about one per CU.
template <int HD, int PB>
__global__ __launch_bounds__(512, 1) void k_scores_mt(const float *__restrict__ q, int q_ld,
                                                   const float *__restrict__ kc, int cap, int pos0, int m, int nh,
                                                   int nkv, float scale, float *__restrict__ S, int sstride,
                                                   const int *__restrict__ st, int mb, int ns) {
  constexpr int NT = 512, KSTR = HD + 4, KF4 = kScoreTile * (HD / 4) / NT;  // key float4 per thread and tile
  static_assert(KF4 * NT == kScoreTile * (HD / 4), "whole key tiles per block");
  extern __shared__ float ks[];  // [2][64][HD + 4] keys, then [G * mb][HD] query rows
  int toff = 0;
  {
    const int u0 = (int)blockIdx.z * mb;
    m = min(mb, m - u0);
    q += (size_t)u0 * q_ld;
    S += (size_t)u0 * nh * sstride;
    pos0 += u0;
    toff = u0;
  }
  if (st) pos0 = st[0] + toff;
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kvh = blockIdx.y, G = nh / nkv;
  const int nmax = pos0 + m;
  const int ntiles = (nmax + kScoreTile - 1) / kScoreTile;
  int t = blockIdx.x;
  if (t >= ntiles) return;  // the group's positions end before this block's first tile
  const float *kb = kc + (size_t)kvh * cap * HD;
  f4 *lq = reinterpret_cast<f4 *>(ks + 2 * kScoreTile * KSTR);
  f4 v4[KF4];
  auto kload = [&](int tt) {
    const int s0 = tt * kScoreTile, rows = min(kScoreTile, nmax - s0);
#pragma unroll
    for (int u = 0; u < KF4; ++u) {
      const int i = tid + NT * u;
      const int r = min(i / (HD / 4), rows - 1), c4 = i % (HD / 4);
      v4[u] = reinterpret_cast<const f4 *>(kb + (size_t)(s0 + r) * HD)[c4];
    }
  };
  auto kstore = [&](int b) {
    float *kt = ks + b * kScoreTile * KSTR;
#pragma unroll
    for (int u = 0; u < KF4; ++u) {
      const int i = tid + NT * u;
      *reinterpret_cast<f4 *>(kt + (i / (HD / 4)) * KSTR + 4 * (i % (HD / 4))) = v4[u];
    }
  };
  kload(t);
  // The group's query rows (pair pi = token * G + g at row pi).
  for (int i = tid; i < G * m * (HD / 4); i += NT) {
    const int pi = i / (HD / 4), c4 = i % (HD / 4);
    lq[i] = reinterpret_cast<const f4 *>(q + (size_t)(pi / G) * q_ld + (size_t)(kvh * G + pi % G) * HD)[c4];
  }
  kstore(0);
  __syncthreads();
  for (int it = 0; t < ntiles; ++it, t += ns) {
    if (t + ns < ntiles) kload(t + ns);
    const int s0 = t * kScoreTile, rows = min(kScoreTile, nmax - s0);
    // Token tk sees positions <= pos0 + tk.
    const int tfirst = s0 > pos0 ? s0 - pos0 : 0;
    const int pairs = G * (m - tfirst);
    const int s = s0 + lane;
    const f4 *kr4 = reinterpret_cast<const f4 *>(ks + (it & 1) * kScoreTile * KSTR + lane * KSTR);
    const int npw = (pairs - wave + 7) / 8;  // this wave's pairs: wave, wave + 8, ...
    for (int b0 = 0; b0 < npw; b0 += PB) {
      float qb[PB][HD / 16];
#pragma unroll
      for (int p = 0; p < PB; ++p) {
        const float *qrow =
            reinterpret_cast<const float *>(lq + (tfirst * G + wave + 8 * min(b0 + p, npw - 1)) * (HD / 4));
#pragma unroll
        for (int mm = 0; mm < HD / 16; ++mm) qb[p][mm] = qrow[16 * mm + (lane & 15)];
      }
      float a[PB][8];
#pragma unroll
      for (int p = 0; p < PB; ++p)
#pragma unroll
        for (int i = 0; i < 8; ++i) a[p][i] = 0.0f;
      // The batch's query values all read before its FMAs.
      __builtin_amdgcn_sched_barrier(0);
      score_chunks_pipe<HD, PB>(std::make_integer_sequence<int, HD / 8>{}, reinterpret_cast<const sf4 *>(kr4), qb, a);
#pragma unroll
      for (int p = 0; p < PB; ++p) {
        const int pi = wave + 8 * (b0 + p);
        const int tk = tfirst + pi / G, h = kvh * G + pi % G;
        if (b0 + p < npw && lane < rows && s <= pos0 + tk) {
          const float d = ((a[p][0] + a[p][4]) + (a[p][1] + a[p][5])) + ((a[p][2] + a[p][6]) + (a[p][3] + a[p][7]));
          S[((size_t)tk * nh + h) * sstride + s] = d * scale;
        }
      }
    }
    // The other key buffer was last read in the previous tile.
    if (t + ns < ntiles) kstore((it + 1) & 1);
    __syncthreads();
  }
}

template <int HD>
void launch_scores_mt(hipStream_t s, const float *q, int q_ld, const float *kc, int cap, int p0, int m, int nh,
                      int nkv, float scale, float *scores, int sstride, int nmax, const int *st, int mb) {
  const int G = nh / nkv, nz = (m + mb - 1) / mb;
  const int ntiles = (nmax + kScoreTile - 1) / kScoreTile;
  const int ns = std::max(1, std::min(ntiles, 256 / (nkv * nz)));
  const size_t smem = sizeof(float) * (2 * (size_t)kScoreTile * (HD + 4) + (size_t)G * mb * HD);
  static bool configured = false;
  if (!configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_scores_mt<HD, 8>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    configured = true;
  }
  hipLaunchKernelGGL((k_scores_mt<HD, 8>), dim3(ns, nkv, nz), dim3(512), smem, s, q, q_ld, kc, cap, p0, m, nh, nkv,
                     scale, scores, sstride, st, mb, ns);
}

template <int HD, int PB>
void launch_scores_t(dim3 sg, size_t ksm, hipStream_t s, const float *q, int q_ld, const float *kc, int cap, int p0,
                     int m, int nh, int nkv, float scale, float *scores, int sstride, const int *st, int toff,
                     int mb) {
  static bool configured = false;
  if (!configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_scores<HD, PB>),
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)(sizeof(float) * ((size_t)kScoreTile * (HD + 4) + 16384)));
    configured = true;
  }
  hipLaunchKernelGGL((k_scores<HD, PB>), sg, dim3(256), ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, HD, scale, scores,
                     sstride, st, toff, mb);
}

template <int HD>
void launch_scores_hd(dim3 sg, size_t ksm, int npw, hipStream_t s, const float *q, int q_ld, const float *kc, int cap,
                      int p0, int m, int nh, int nkv, float scale, float *scores, int sstride, const int *st,
                      int toff, int mb) {
  // Pairs per wave at once: all of them up to three, four for four, nine
  // for the verify batch (5..9), eight at a time beyond.
  if (npw <= 1)
    launch_scores_t<HD, 1>(sg, ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, toff, mb);
  else if (npw == 2)
    launch_scores_t<HD, 2>(sg, ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, toff, mb);
  else if (npw == 3)
    launch_scores_t<HD, 3>(sg, ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, toff, mb);
  else if (npw > 9)
    // Prefill groups: eight pairs per key read (0.577 against 0.584 s for
    // the 4095-token Mistral-7B prefill with four).
    launch_scores_t<HD, 8>(sg, ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, toff, mb);
  else if (npw <= 4)
    launch_scores_t<HD, 4>(sg, ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, toff, mb);
  else
    launch_scores_t<HD, 9>(sg, ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, toff, mb);
}

// Score launches for tokens [0, m): the compile-time head dims in sub-batches
// whose query rows fit next to the keys in LDS (at most 64 KB of them).
void launch_scores(const float *q, int q_ld, const float *kc, int cap, int p0, int m, int nh, int nkv, int hd,
                   float scale, float *scores, int sstride, int nmax, const int *st, hipStream_t s) {
  static size_t sc_configured = 0;
  const int G = nh / nkv;
  if (hd == 128 || hd == 64) {
    // Groups of mb tokens (their query rows next to the keys in LDS, at
    // most 64 KB of them) in one launch, grid.z = group; the grid's x covers
    // the last group's positions and earlier groups' blocks past their own
    // positions leave at once.
    const int mb = std::max(1, std::min(16, 16384 / (G * hd)));
    // More than 12 tokens: the multi-tile blocks (68.4 against 72.2 ms of
    // scores per 4095-token Mistral-7B prefill).
    const bool mt_ok = G * mb * hd * 4 + 2 * kScoreTile * (hd + 4) * 4 <= 160 * 1024;
    if (m > 12 && mt_ok) {
      if (hd == 128)
        launch_scores_mt<128>(s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, nmax, st, mb);
      else
        launch_scores_mt<64>(s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, nmax, st, mb);
      return;
    }
    const int nz = (m + mb - 1) / mb;
    const dim3 sg((nmax + kScoreTile - 1) / kScoreTile, nkv, nz);
    const size_t ksm = sizeof(float) * ((size_t)kScoreTile * (hd + 4) + (size_t)G * std::min(mb, m) * hd);
    const int npw = (G * std::min(mb, m) + 3) / 4;
    if (hd == 128)
      launch_scores_hd<128>(sg, ksm, npw, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, 0, mb);
    else
      launch_scores_hd<64>(sg, ksm, npw, s, q, q_ld, kc, cap, p0, m, nh, nkv, scale, scores, sstride, st, 0, mb);
    return;
  }
  const dim3 sg((nmax + kScoreTile - 1) / kScoreTile, nkv);
  const size_t ksm = sizeof(float) * (size_t)kScoreTile * (hd + 1);
  if (ksm > 48 * 1024 && ksm > sc_configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_scores<0, 1>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)ksm);
    sc_configured = ksm;
  }
  hipLaunchKernelGGL((k_scores<0, 1>), sg, dim3(256), ksm, s, q, q_ld, kc, cap, p0, m, nh, nkv, hd, scale, scores,
                     sstride, st, 0, m);
}

// The softmax of rows of any length (used past the register-resident
// kernels' 16384 positions).  grid (nh, m), 512 threads.  The row stays in
// global memory: one pass for the maximum, then chunks of kSoftLChunk
// positions.  Waves 1..7 (448 threads, 8 positions each) turn a chunk's
// scores into exponentials (Schraudolph on the 8-aligned body, expf on the
// <= 7 tail positions), store them to the row and chain-major to LDS
// (position p of the chunk at chain p % 8, step p / 8: 448 is a multiple of
// 8, so a thread's positions all belong to chain tid % 8), while lanes 0..7
// of wave 0 add the previous chunk's values into the eight chains in order
// (acc_j = sum of e[8i + j], i ascending, from +0).  Two chunk buffers, one
// block barrier per chunk.  Then hsum8 of the chains, the tail in order and
// 1/sum into S[sstride - 1], as the other softmax kernels.
constexpr int kSoftLFill = 448;                // filling threads (waves 1..7)
constexpr int kSoftLChunk = kSoftLFill * 8;    // positions per chunk
constexpr int kSoftLSteps = kSoftLChunk / 8;   // chain steps per chunk
constexpr int kSoftLStr = kSoftLSteps + 4;     // LDS row stride (floats)

__global__ __launch_bounds__(512) void k_softmax_l(float *__restrict__ S, int pos0, int nh, int sstride,
                                                   const int *__restrict__ st) {
  __shared__ __align__(16) float ech[2][8 * kSoftLStr];
  __shared__ float red[8];
  __shared__ float csum[8];
  __shared__ float tail[8];
  if (st) pos0 = st[0];
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = pos0 + t + 1, n8 = n / 8, body = 8 * n8;
  float *row = S + ((size_t)t * nh + h) * sstride;
  float mx = -INFINITY;
  for (int base = 0; base < n; base += 512 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = base + 512 * u + tid;
      v[u] = p < n ? row[p] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) mx = fmaxf(mx, v[u]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
  const int nch = (n + kSoftLChunk - 1) / kSoftLChunk;
  const int f = tid - 64;  // filling thread index (waves 1..7)
  auto fill = [&](int c) {
    const int c0 = c * kSoftLChunk;
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = c0 + kSoftLFill * u + f;
      v[u] = p < n ? row[p] : 0.0f;
    }
    float *er = &ech[c & 1][(f & 7) * kSoftLStr + (f >> 3)];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = c0 + kSoftLFill * u + f;
      if (p < body) {
        const float e = rai_exact::schraudolph(v[u] - mx);
        er[(kSoftLFill / 8) * u] = e;
        row[p] = e;
      } else if (p < n) {
        const float e = rai_exact::expf_glibc(v[u] - mx);
        tail[p - body] = e;
        row[p] = e;
      }
    }
  };
  if (wave > 0) fill(0);
  __syncthreads();
  float acc = 0.0f;
  for (int c = 0; c < nch; ++c) {
    if (wave > 0) {
      if (c + 1 < nch) fill(c + 1);
    } else if (tid < 8) {
      const int cnt = min(kSoftLSteps, n8 - c * kSoftLSteps);  // chain steps in this chunk
      const float *cr = &ech[c & 1][tid * kSoftLStr];
      int i = 0;
      if (cnt >= 32) {
        float4 cur[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = reinterpret_cast<const float4 *>(cr)[u];
        for (; i + 32 <= cnt; i += 32) {
          float4 nxt[8];
          const int nb = i + 64 <= cnt ? i + 32 : i;
#pragma unroll
          for (int u = 0; u < 8; ++u) nxt[u] = reinterpret_cast<const float4 *>(cr + nb)[u];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            acc = acc + cur[u].x;
            acc = acc + cur[u].y;
            acc = acc + cur[u].z;
            acc = acc + cur[u].w;
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
        }
      }
      for (; i < cnt; ++i) acc = acc + cr[i];
    }
    __syncthreads();
  }
  if (tid < 8) csum[tid] = acc;
  __syncthreads();
  if (tid == 0) {
    float sum = ((csum[0] + csum[4]) + (csum[1] + csum[5])) + ((csum[2] + csum[6]) + (csum[3] + csum[7]));
    for (int r = 0; r < n - body; ++r) sum = sum + tail[r];
    row[sstride - 1] = 1.0f / sum;
  }
}

// The same softmax with the row held in registers: thread t of 512 owns
// the positions p = 512u + t (u < NB, n <= 512 NB), all of them in lane
// chain t % 8 (512 is a multiple of 8) at chain step 64u + t / 8.  One load
// burst, the maximum by lane moves, the exponentials written chain-major to
// LDS (row j = chain j, row stride cstr = 4 mod 64 floats, so the 8 chain
// lanes' 16-byte reads hit distinct banks) and stored to the row.  The tail
// exponentials (expf) go to LDS for the final sum.
template <int NB>
__global__ __launch_bounds__(512) void k_softmax_r(float *__restrict__ S, int pos0, int nh, int sstride,
                                                   int cstr, const int *__restrict__ st) {
  extern __shared__ __align__(16) float ech[];  // [8][cstr]
  __shared__ float red[8];
  __shared__ float csum[8];
  __shared__ float tail[8];
  if (st) pos0 = st[0];
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = pos0 + t + 1, n8 = n / 8;
  float *row = S + ((size_t)t * nh + h) * sstride;
  float v[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u) v[u] = 512 * u < n ? row[min(512 * u + tid, n - 1)] : -INFINITY;
  float mx = v[0];
#pragma unroll
  for (int u = 1; u < NB; ++u) mx = fmaxf(mx, v[u]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
  float *erow = ech + (tid & 7) * cstr + (tid >> 3);
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int p = 512 * u + tid;
    if (p < 8 * n8) {
      v[u] = rai_exact::schraudolph(v[u] - mx);
      erow[64 * u] = v[u];
    } else if (p < n) {
      v[u] = rai_exact::expf_glibc(v[u] - mx);
      tail[p - 8 * n8] = v[u];
    }
    if (p < n) row[p] = v[u];
  }
  __syncthreads();
  if (wave != 0) return;
  if (tid < 8) {
    // Chain tid: e_{8i + tid} for i = 0..n8-1 in order, 16-byte reads kept
    // 32 values ahead.
    const float *cr = ech + tid * cstr;
    float acc = 0.0f;
    int i = 0;
    if (n8 >= 32) {
      float4 cur[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = reinterpret_cast<const float4 *>(cr)[u];
      for (; i + 32 <= n8; i += 32) {
        float4 nxt[8];
        const int nb = i + 64 <= n8 ? i + 32 : i;
#pragma unroll
        for (int u = 0; u < 8; ++u) nxt[u] = reinterpret_cast<const float4 *>(cr + nb)[u];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc = acc + cur[u].x;
          acc = acc + cur[u].y;
          acc = acc + cur[u].z;
          acc = acc + cur[u].w;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
      }
    }
    for (; i < n8; ++i) acc = acc + cr[i];
    csum[tid] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    float sum = ((csum[0] + csum[4]) + (csum[1] + csum[5])) + ((csum[2] + csum[6]) + (csum[3] + csum[7]));
    for (int r = 0; r < n - 8 * n8; ++r) sum = sum + tail[r];
    row[sstride - 1] = 1.0f / sum;
  }
}

// Chain-major row stride for k_softmax_r: at least ceil(nmax / 8) floats,
// 4 mod 64.
static int softmax_r_stride(int nmax) { return (((nmax + 7) / 8 + 63) & ~63) + 4; }

// The softmax of k_softmax_r with the eight sum chains run from registers.
// Load, maximum and exponentials as there: every position's Schraudolph
// exponential (positions past the chains give 0), stored to the row and
// chain-major to LDS; the (at most 7) tail positions take expf on lanes
// 0..6, from values loaded at the start.  Then one wave runs the chains
// over segments of 64 steps: segment q = 8s + u of chain j is read, slot s
// at a time, into the registers of lane u + 8j.  Phase q adds every lane's
// values in order (only the segment-q lanes carry a live chain; a padding
// step adds +0, which leaves a chain unchanged: it starts at +0 and adds
// non-negative values), then moves each chain to the next segment's lane
// (DPP row_shr:1, or row_shl:7 from u = 7 to u = 0 of the next slot), so a
// chain is one sequence of dependent adds with no LDS read between them.
// The last segment's lanes hold the chains; hsum8 and the tail as the
// reference, then 1/sum into S[sstride - 1].
constexpr int kSoftSeg = 64;  // chain steps per segment

__host__ __device__ constexpr int softmax_c_slots(int nb) { return nb > 8 ? nb / 8 : 1; }
__host__ __device__ constexpr int softmax_c_cstr(int nb) { return 8 * kSoftSeg * softmax_c_slots(nb) + 4; }

template <int NB>
__global__ __launch_bounds__(512) void k_softmax_c(float *__restrict__ S, int pos0, int nh, int sstride,
                                                   const int *__restrict__ st) {
  constexpr int SL = softmax_c_slots(NB), CSTR = softmax_c_cstr(NB);
  static_assert(8 * kSoftSeg * SL >= 64 * NB, "slots cover every chain step");
  __shared__ __align__(16) float ech[8 * CSTR];  // [8][CSTR], chain-major
  __shared__ float red[8];
  __shared__ float tail[8];
  if (st) pos0 = st[0];
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = pos0 + t + 1, n8 = n / 8, ntail = n - 8 * n8;
  float *row = S + ((size_t)t * nh + h) * sstride;
  float v[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u) v[u] = 512 * u < n ? row[min(512 * u + tid, n - 1)] : -INFINITY;
  const float xt = row[min(8 * n8 + (tid & 7), n - 1)];  // tail value (lanes < ntail)
  float mx = v[0];
#pragma unroll
  for (int u = 1; u < NB; ++u) mx = fmaxf(mx, v[u]);
  mx = wave_max_dpp(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
  float *erow = ech + (tid & 7) * CSTR + (tid >> 3);
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int p = 512 * u + tid;
    const float e = p < 8 * n8 ? rai_exact::schraudolph(v[u] - mx) : 0.0f;
    erow[64 * u] = e;
    if (p < 8 * n8) row[p] = e;
  }
  // Chain steps past 64 NB (slots no row reaches when NB < 8) are never
  // added by a live lane; zero them anyway.
  for (int i = 64 * NB + (tid >> 3); i < 8 * kSoftSeg * SL; i += 64) ech[(tid & 7) * CSTR + i] = 0.0f;
  if (tid < ntail) {
    const float e = rai_exact::expf_glibc(xt - mx);
    tail[tid] = e;
    row[8 * n8 + tid] = e;
  }
  __syncthreads();
  if (wave != 0) return;
  const int u8 = lane & 7, j = lane >> 3;
  const int nseg = (n8 + kSoftSeg - 1) / kSoftSeg;
  float4 r[kSoftSeg / 4];
  float acc = 0.0f;
  int q = 0;
#pragma unroll
  for (int sl = 0; sl < SL; ++sl) {
    if (q >= nseg) break;
    const float4 *cr = reinterpret_cast<const float4 *>(ech + j * CSTR + kSoftSeg * (8 * sl + u8));
#pragma unroll
    for (int g = 0; g < kSoftSeg / 4; ++g) r[g] = cr[g];
#pragma unroll 1
    for (int uu = 0; uu < 8 && q < nseg; ++uu, ++q) {
#pragma unroll
      for (int g = 0; g < kSoftSeg / 4; ++g) {
        acc = acc + r[g].x;
        acc = acc + r[g].y;
        acc = acc + r[g].z;
        acc = acc + r[g].w;
      }
      // Within each row of 16 lanes: lane l takes lane l - 1 (row_shr:1)
      // or lane l + 7 (row_shl:7); the 8 lanes of a chain share a row.
      const int ai = __float_as_int(acc);
      const float moved = __int_as_float(uu < 7 ? __builtin_amdgcn_update_dpp(ai, ai, 0x111, 0xF, 0xF, false)
                                                : __builtin_amdgcn_update_dpp(ai, ai, 0x107, 0xF, 0xF, false));
      acc = u8 == ((uu + 1) & 7) ? moved : acc;
    }
  }
  // The chains ended in the lanes of segment nseg - 1 (with n8 = 0 every
  // lane still holds +0).
  const int last = (nseg > 0 ? nseg - 1 : 0) & 7;
  float c[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) c[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), last + 8 * k));
  if (lane == 0) {
    float sum = ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
    for (int k = 0; k < ntail; ++k) sum = sum + tail[k];
    row[sstride - 1] = 1.0f / sum;
  }
}

// k_softmax_c with one wave per row, for batches of many rows (prefill):
// the wave holds positions lane + 64 k (k < NBW) of its row in registers,
// takes the maximum by DPP, writes the exponentials to the row and, chain
// by chain, to its own LDS area (position p is step p / 8 of chain p % 8,
// and every position a lane holds belongs to chain lane % 8), then runs
// k_softmax_c's lane-segment chains over that area.  RPB rows per block, no
// block barrier.  Positions past the row read the row's last value (which
// leaves the maximum unchanged) and give exponentials of 0.
template <int NBW, int RPB>
__global__ __launch_bounds__(64 * RPB) void k_softmax_w(float *__restrict__ S, int pos0, int m, int nh, int sstride,
                                                       const int *__restrict__ st) {
  static_assert(NBW <= 64, "one slot of eight 64-step segments per chain");
  constexpr int SL = 1;
  constexpr int CSTR = 8 * kSoftSeg * SL + 4;           // floats per chain
  extern __shared__ __align__(16) float ech_all[];      // [RPB][8][CSTR]
  if (st) pos0 = st[0];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = blockIdx.x * RPB + wave;
  const int t = r / nh, h = r - t * nh;
  if (t >= m) return;
  const int n = pos0 + t + 1, n8 = n / 8, n8x8 = 8 * n8, ntail = n - n8x8;
  float *row = S + ((size_t)t * nh + h) * sstride;
  float *ech = ech_all + wave * 8 * CSTR;
  float v[NBW];
#pragma unroll
  for (int k = 0; k < NBW; ++k) v[k] = row[min(lane + 64 * k, n - 1)];
  const float xt = row[min(n8x8 + (lane & 7), n - 1)];  // tail value (lanes < ntail)
  float mx = v[0];
#pragma unroll
  for (int k = 1; k < NBW; ++k) mx = fmaxf(mx, v[k]);
  mx = wave_max_dpp(mx);
  float *erow = ech + (lane & 7) * CSTR + (lane >> 3);
#pragma unroll
  for (int k = 0; k < NBW; ++k) {
    const int p = lane + 64 * k;
    // schraudolph(-inf) is +0: positions from 8 floor(n/8) on give 0.
    const float e = rai_exact::schraudolph(p < n8x8 ? v[k] - mx : -INFINITY);
    erow[8 * k] = e;
    if (p < n8x8) row[p] = e;
  }
  float et = 0.0f;
  if (lane < ntail) {
    et = rai_exact::expf_glibc(xt - mx);
    row[n8x8 + lane] = et;
  }
  // The chain-major area is read by other lanes of this wave.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int u8 = lane & 7, j = lane >> 3;
  const int nseg = (n8 + kSoftSeg - 1) / kSoftSeg;
  float4 rr[kSoftSeg / 4];
  float acc = 0.0f;
  int q = 0;
#pragma unroll
  for (int sl = 0; sl < SL; ++sl) {
    if (q >= nseg) break;
    const float4 *cr = reinterpret_cast<const float4 *>(ech + j * CSTR + kSoftSeg * (8 * sl + u8));
#pragma unroll
    for (int g = 0; g < kSoftSeg / 4; ++g) rr[g] = cr[g];
#pragma unroll 1
    for (int uu = 0; uu < 8 && q < nseg; ++uu, ++q) {
#pragma unroll
      for (int g = 0; g < kSoftSeg / 4; ++g) {
        acc = acc + rr[g].x;
        acc = acc + rr[g].y;
        acc = acc + rr[g].z;
        acc = acc + rr[g].w;
      }
      const int ai = __float_as_int(acc);
      const float moved = __int_as_float(uu < 7 ? __builtin_amdgcn_update_dpp(ai, ai, 0x111, 0xF, 0xF, false)
                                                : __builtin_amdgcn_update_dpp(ai, ai, 0x107, 0xF, 0xF, false));
      acc = u8 == ((uu + 1) & 7) ? moved : acc;
    }
  }
  const int last = (nseg > 0 ? nseg - 1 : 0) & 7;
  float c[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) c[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), last + 8 * k));
  float tl[7];
#pragma unroll
  for (int k = 0; k < 7; ++k) tl[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(et), k));
  if (lane == 0) {
    float sum = ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
#pragma unroll
    for (int k = 0; k < 7; ++k)
      if (k < ntail) sum = sum + tl[k];
    row[sstride - 1] = 1.0f / sum;
  }
}

template <int NBW, int RPB>
void launch_softmax_w(float *scores, int p0, int m, int nh, int sstride, const int *st, hipStream_t s) {
  constexpr size_t smem = sizeof(float) * RPB * 8 * (8 * kSoftSeg + 4);
  static bool configured = false;
  if (!configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_softmax_w<NBW, RPB>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = true;
  }
  hipLaunchKernelGGL((k_softmax_w<NBW, RPB>), dim3((m * nh + RPB - 1) / RPB), dim3(64 * RPB), smem, s, scores, p0, m,
                     nh, sstride, st);
}

// PV with the V stream spread over loader waves.  The V cache is d-major
// ([kv head][head dim][vstride] floats, vstride a multiple of 64), so the
// positions of one dim in a chunk are contiguous.  One block per (kv head,
// slice of DL head dims, TM tokens) with NCW compute waves and NL loader
// waves.  Compute lane L = 64w + lane owns the chain of token L / (G*DL),
// query head kvh*G + (L / DL) % G, dim d0 + L % DL, so the G heads of the kv
// group and the TM tokens share every V value.  Loader i fetches chunks
// i, i + NL, ... (CP positions: the V tile [DL][CP] and the TM*G
// probability rows) with 16-byte coalesced loads, so NL chunks are in flight
// while the compute waves work.  Each iteration the owner of the next chunk
// stores it into the free half of a double-buffered LDS tile (probabilities
// of positions past the row's token, and rows of tokens past m, stored as
// 0: fma(0, v, acc) == acc for the finite cached v, and acc is never -0),
// and the compute waves run the reference's sequential FMA chain over the
// current chunk, reading 4 positions' V values and (wave-broadcast)
// probabilities per 16-byte LDS read, 32 positions ahead of the chain.  The
// chunks run to the block's longest token.  No block barrier in the chunk
// loop: LDS flags hand each tile over (k_pv_flag).
template <int DL, int G, int CP, int TM, int NL, int TPL = 1>
struct PvCfg {
  static constexpr int NCW = TM * G * DL / (64 * TPL);  // compute waves (TPL tokens per lane)
  static constexpr int NT = 64 * (NCW + NL);         // threads
  static constexpr int NV = DL * CP / 256;           // V float4 per loader lane per chunk
  static constexpr int NP = (TM * G * CP / 4 + 63) / 64;  // P float4 per loader lane per chunk
  static constexpr int STR = CP + 4;                 // LDS row stride (floats)
  static_assert(TM * G * DL % (64 * TPL) == 0 && TM % TPL == 0, "whole compute waves");
};


// The tile hand-off without block barriers: the loader of chunk c waits
// until every compute wave has finished chunk c - 2 (the same tile half),
// publishes V and probabilities, then posts ready[c & 1] = c; a compute wave
// waits for ready[k & 1] >= k, runs the chunk's chains and posts its
// done[w] = k + 1.  Every wait is bounded (`spin` polls, kPvSpin unless a
// caller lowers it), so a wait that could not end still lets the block
// finish; a wait that gives up sets bit 0 of the error word `err`, which the
// host turns into an error for the whole call (the block's output is then
// not trusted).
constexpr int kPvSpin = 1 << 22;

// Poll an LDS word until it is at least `want` (every lane reads the same
// word; at most `spin` polls).  One asm block, so the compiler keeps the
// loads that follow inside the block that uses them.  Returns the last value
// read: below `want` when the wait gave up.
template <bool SLEEP>
__device__ __forceinline__ int lds_wait_ge(const int *flag, int want, int spin) {
  typedef const __attribute__((address_space(3))) int lds_int;
  const unsigned addr = (unsigned)(uintptr_t)((lds_int *)flag);
  int seen;
  unsigned polls;
  if constexpr (SLEEP) {
    asm volatile(
        "s_mov_b32 %1, 0\n"
        "1:\n\t"
        "ds_read_b32 %0, %2\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "v_cmp_lt_i32 vcc, %0, %3\n\t"
        "s_cbranch_vccz 2f\n\t"
        "s_sleep 1\n\t"
        "s_add_u32 %1, %1, 1\n\t"
        "s_cmp_lt_u32 %1, %4\n\t"
        "s_cbranch_scc1 1b\n"
        "2:"
        : "=&v"(seen), "=&s"(polls)
        : "v"(addr), "v"(want), "s"(spin)
        : "vcc", "scc", "memory");
  } else {
    asm volatile(
        "s_mov_b32 %1, 0\n"
        "1:\n\t"
        "ds_read_b32 %0, %2\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "v_cmp_lt_i32 vcc, %0, %3\n\t"
        "s_cbranch_vccz 2f\n\t"
        "s_add_u32 %1, %1, 1\n\t"
        "s_cmp_lt_u32 %1, %4\n\t"
        "s_cbranch_scc1 1b\n"
        "2:"
        : "=&v"(seen), "=&s"(polls)
        : "v"(addr), "v"(want), "s"(spin)
        : "vcc", "scc", "memory");
  }
  return seen;
}

// Record a wait that gave up (one lane per wave; a vector atomic).
__device__ __forceinline__ void pv_wait_failed(int *err) {
  if (err && (threadIdx.x & 63) == 0) atomicOr(err, 1);
}


// s_waitcnt lgkmcnt(N) (vmcnt and expcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt field");
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}

// The sequential PV chain over one CP-position tile for the lane's output
// (acc = fma(p_t, v_t, acc), t in order; layers.rs:1354-1379).  A wave
// issues one dependent FMA per ~8 cycles and each other instruction costs
// about 3.5 cycles more, so the loop keeps the others few: 16 positions (4
// V and 4 probability reads of 16 bytes) per group, the reads of group
// g + 2 issued together ahead of the 16 FMAs of group g, and one LDS wait
// per group (the 16 reads after group g's are the two groups ahead, so
// lgkmcnt(15) has group g landed).  64-position quarters at or past
// `nvalid` (the block's last position, in the tile's last chunk) are not
// run: their probabilities are 0, and fma(0, v, acc) == acc.
template <int CP>
__device__ __forceinline__ float pv_chunk(const float4 *__restrict__ vr, const float4 *__restrict__ pr, int nvalid,
                                          float acc) {
  constexpr int NG = CP / 16;
  static_assert(CP % 64 == 0, "whole 64-position quarters");
  float4 rv[3][4], rq[3][4];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      rv[b][u] = vr[4 * b + u];
      rq[b][u] = pr[4 * b + u];
    }
#pragma unroll
  for (int q = 0; q < NG / 4; ++q) {
    if (64 * q >= nvalid) break;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      const int b = 4 * q + bb;
      if (b + 2 < NG) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          rv[(b + 2) % 3][u] = vr[4 * (b + 2) + u];
          rq[(b + 2) % 3][u] = pr[4 * (b + 2) + u];
        }
        wait_lgkm<15>();
      } else {
        wait_lgkm<0>();
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 v4 = rv[b % 3][u], p4 = rq[b % 3][u];
        acc = __fmaf_rn(p4.x, v4.x, acc);
        acc = __fmaf_rn(p4.y, v4.y, acc);
        acc = __fmaf_rn(p4.z, v4.z, acc);
        acc = __fmaf_rn(p4.w, v4.w, acc);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  return acc;
}

// Two chains at once (tokens t and t + 1 of the lane's head and dim): each
// V read feeds both, so a wave issues two independent FMAs per position
// and the dependent latency of one hides behind the other.  Groups of 16
// positions (4 V and 2 x 4 probability reads), read one group ahead with one
// wait per group.
template <int CP>
__device__ __forceinline__ void pv_chunk2(const float4 *__restrict__ vr, const float4 *__restrict__ pr0,
                                          const float4 *__restrict__ pr1, int nvalid, float &acc0, float &acc1) {
  constexpr int NG = CP / 16;
  static_assert(CP % 64 == 0, "whole 64-position quarters");
  float4 rv[2][4], r0[2][4], r1[2][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    rv[0][u] = vr[u];
    r0[0][u] = pr0[u];
    r1[0][u] = pr1[u];
  }
#pragma unroll
  for (int q = 0; q < NG / 4; ++q) {
    if (64 * q >= nvalid) break;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      const int b = 4 * q + bb;
      if (b + 1 < NG) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          rv[(b + 1) & 1][u] = vr[4 * (b + 1) + u];
          r0[(b + 1) & 1][u] = pr0[4 * (b + 1) + u];
          r1[(b + 1) & 1][u] = pr1[4 * (b + 1) + u];
        }
        wait_lgkm<12>();
      } else {
        wait_lgkm<0>();
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 v4 = rv[b & 1][u], p4 = r0[b & 1][u], q4 = r1[b & 1][u];
        acc0 = __fmaf_rn(p4.x, v4.x, acc0);
        acc1 = __fmaf_rn(q4.x, v4.x, acc1);
        acc0 = __fmaf_rn(p4.y, v4.y, acc0);
        acc1 = __fmaf_rn(q4.y, v4.y, acc1);
        acc0 = __fmaf_rn(p4.z, v4.z, acc0);
        acc1 = __fmaf_rn(q4.z, v4.z, acc1);
        acc0 = __fmaf_rn(p4.w, v4.w, acc0);
        acc1 = __fmaf_rn(q4.w, v4.w, acc1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Four chains at once (tokens t .. t + 3 of the lane's head and dim, token
// rows PS4 float4 apart): each V read feeds four independent FMAs per
// position.  Groups of 8 positions (2 V and 4 x 2 probability reads), read
// one group ahead with one wait per group.
template <int CP, int PS4>
__device__ __forceinline__ void pv_chunk4(const float4 *__restrict__ vr, const float4 *__restrict__ pr, int nvalid,
                                          float (&acc)[4]) {
  constexpr int NG = CP / 8;
  static_assert(CP % 64 == 0, "whole 64-position quarters");
  float4 rv[2][2], rp[2][4][2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    rv[0][u] = vr[u];
#pragma unroll
    for (int t = 0; t < 4; ++t) rp[0][t][u] = pr[t * PS4 + u];
  }
#pragma unroll
  for (int q = 0; q < NG / 8; ++q) {
    if (64 * q >= nvalid) break;
#pragma unroll
    for (int bb = 0; bb < 8; ++bb) {
      const int b = 8 * q + bb;
      if (b + 1 < NG) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          rv[(b + 1) & 1][u] = vr[2 * (b + 1) + u];
#pragma unroll
          for (int t = 0; t < 4; ++t) rp[(b + 1) & 1][t][u] = pr[t * PS4 + 2 * (b + 1) + u];
        }
        wait_lgkm<10>();
      } else {
        wait_lgkm<0>();
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float4 v4 = rv[b & 1][u];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __fmaf_rn(rp[b & 1][t][u].x, v4.x, acc[t]);
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __fmaf_rn(rp[b & 1][t][u].y, v4.y, acc[t]);
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __fmaf_rn(rp[b & 1][t][u].z, v4.z, acc[t]);
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __fmaf_rn(rp[b & 1][t][u].w, v4.w, acc[t]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int DL, int G, int CP, int TM, int NL, int TPL = 1>
__global__ __launch_bounds__(TM * G * DL / TPL + 64 * NL) void k_pv_flag(
    const float *__restrict__ P, const float *__restrict__ vt_g, int vstride, int pos0, int m, int nh, int hd,
    int sstride, float *__restrict__ out, const int *__restrict__ st, int *__restrict__ err, int spin) {
  using C = PvCfg<DL, G, CP, TM, NL, TPL>;
  static_assert(TPL == 1 || TPL == 2 || TPL == 4, "one, two or four tokens per compute lane");
  if (st) pos0 = st[0];
  constexpr int NCW = C::NCW, NV = C::NV, NP = C::NP, STR = C::STR;
  constexpr int Q4 = CP / 4;  // float4 per tile row
  __shared__ __align__(16) float vt[2][DL * STR];
  __shared__ __align__(16) float pt[2][TM * G * STR];
  __shared__ int ready[2];
  __shared__ int done[NCW];
  // 1/sum of each probability row (the softmax leaves it in the row's last
  // slot): the loaders publish p = e * (1/sum).
  __shared__ float pinv[TM * G];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slices = hd / DL;
  const int kvh = blockIdx.x / slices;
  const int d0 = (blockIdx.x - kvh * slices) * DL;
  const int t0 = blockIdx.y * TM;
  const int tn = min(TM, m - t0);   // tokens of this block
  const int nmax = pos0 + t0 + tn;  // positions of its longest token
  const int nchunks = (nmax + CP - 1) / CP;
  const float *vbase = vt_g + ((size_t)kvh * hd + d0) * vstride;

  typedef float f4 __attribute__((ext_vector_type(4)));
  f4 fv[NV], fp[NP];
  auto prow = [&](int r) {
    const int rr = min((64 * r + lane) / Q4, TM * G - 1), tl = min(rr / G, tn - 1);
    return ((size_t)(t0 + tl) * nh + (size_t)kvh * G + rr % G) * sstride;
  };
  auto issue = [&](int k) {
    const int s0 = k * CP;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int f = 64 * u + lane;  // float4 index in the [DL][CP] tile
      const int q0 = min(s0 + 4 * (f % Q4), vstride - 4);
      fv[u] = *reinterpret_cast<const f4 *>(vbase + (size_t)(f / Q4) * vstride + q0);
    }
#pragma unroll
    for (int r = 0; r < NP; ++r) {
      const int f = 64 * r + lane;  // float4 index in the [TM*G][CP] tile
      const int q0 = min(s0 + 4 * (f % Q4), sstride - 4);
      fp[r] = *reinterpret_cast<const f4 *>(P + prow(r) + q0);
    }
  };
  auto publish = [&](int k) {
    const int s0 = k * CP, b = k & 1;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int f = 64 * u + lane;
      *reinterpret_cast<f4 *>(&vt[b][(f / Q4) * STR + 4 * (f % Q4)]) = fv[u];
    }
    if (tn == TM && s0 + CP <= pos0 + t0 + 1) {
      // Every row of the block covers the whole chunk: nothing to mask.
#pragma unroll
      for (int r = 0; r < NP; ++r) {
        const int f = 64 * r + lane;
        if (f < TM * G * Q4) {
          const int rr = f / Q4;
          *reinterpret_cast<f4 *>(&pt[b][rr * STR + 4 * (f % Q4)]) = fp[r] * pinv[rr];
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < NP; ++r) {
      const int f = 64 * r + lane;
      if (f < TM * G * Q4) {
        const int q = 4 * (f % Q4), rr = f / Q4, tl = rr / G;
        const int n_ = tl < tn ? pos0 + t0 + tl + 1 : 0;
        f4 v = fp[r] * pinv[rr];
        if (s0 + q + 0 >= n_) v.x = 0.0f;
        if (s0 + q + 1 >= n_) v.y = 0.0f;
        if (s0 + q + 2 >= n_) v.z = 0.0f;
        if (s0 + q + 3 >= n_) v.w = 0.0f;
        *reinterpret_cast<f4 *>(&pt[b][rr * STR + q]) = v;
      }
    }
  };

  if (threadIdx.x == 0) {
    ready[0] = 0;  // chunk 0 is published before the first barrier
    ready[1] = -1;
  }
  if (threadIdx.x < NCW) done[threadIdx.x] = 0;
  const int lw = wave - NCW;  // loader index, negative for compute waves
  if (threadIdx.x < TM * G) {
    const int i = threadIdx.x, tl = min(i / G, tn - 1);
    pinv[i] = P[((size_t)(t0 + tl) * nh + (size_t)kvh * G + i % G) * sstride + sstride - 1];
  }
  if (lw >= 0 && lw < nchunks) issue(lw);
  __syncthreads();  // pinv
  if (lw == 0) {
    publish(0);
    if (NL < nchunks) issue(NL);
  }
  __syncthreads();
  const int L = wave * 64 + lane;
  // Lane L runs tokens tl .. tl + TPL - 1 of head g, dim dd.
  const int tl = TPL * (L / (G * DL)), g = (L / DL) % G, dd = L % DL;
  // One loop per role (the role is wave-uniform), so the loaders' in-flight
  // tiles are not live in the compute loop's registers.
  if (wave < NCW) {
    float acc[TPL];
#pragma unroll
    for (int t = 0; t < TPL; ++t) acc[t] = 0.0f;
    for (int k = 0; k < nchunks; ++k) {
      if (lds_wait_ge<false>(&ready[k & 1], k, spin) < k) pv_wait_failed(err);
      const float4 *vr = reinterpret_cast<const float4 *>(&vt[k & 1][dd * STR]);
      const float4 *pr = reinterpret_cast<const float4 *>(&pt[k & 1][(tl * G + g) * STR]);
      if constexpr (TPL == 4)
        pv_chunk4<CP, G * STR / 4>(vr, pr, nmax - k * CP, acc);
      else if constexpr (TPL == 2)
        pv_chunk2<CP>(vr, pr, pr + G * STR / 4, nmax - k * CP, acc[0], acc[1]);
      else
        acc[0] = pv_chunk<CP>(vr, pr, nmax - k * CP, acc[0]);
      // The release orders this chunk's tile reads before the post.
      __hip_atomic_store(&done[wave], k + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
#pragma unroll
    for (int t = 0; t < TPL; ++t)
      if (tl + t < tn) out[((size_t)(t0 + tl + t) * nh + (size_t)kvh * G + g) * hd + d0 + dd] = acc[t];
  } else {
    // Loader lw publishes chunks lw, lw + NL, ... (loader 0 published chunk 0
    // above and holds chunk NL).  Tile half c & 1 held chunk c - 2: wait
    // until every compute wave has consumed it.
    for (int c = lw == 0 ? NL : lw; c < nchunks; c += NL) {
#pragma unroll
      for (int w = 0; w < NCW; ++w)
        if (lds_wait_ge<true>(&done[w], c - 1, spin) < c - 1) pv_wait_failed(err);
      publish(c);
      __hip_atomic_store(&ready[c & 1], c, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (c + NL < nchunks) issue(c + NL);
    }
  }
}

template <int DL, int G, int CP, int TM, int NL, int TPL = 1>
void launch_pv_flag(const float *scores, const float *vc, int vstride, int p0, int m, int nh, int nkv, int hd,
                    int sstride, float *out, const int *st, int *err, int spin, hipStream_t s) {
  const dim3 pg(nkv * (hd / DL), (m + TM - 1) / TM);
  hipLaunchKernelGGL((k_pv_flag<DL, G, CP, TM, NL, TPL>), pg, dim3(PvCfg<DL, G, CP, TM, NL, TPL>::NT), 0, s, scores,
                     vc, vstride, p0, m, nh, hd, sstride, out, st, err, spin);
}

// One-token attention over a short context in one launch: one block per kv
// head and G * HD = 512 threads, with k_scores', k_softmax_w's and
// pv_chunk's arithmetic and orders.  The block requests the kv head's V rows
// (positions up to n rounded up to 64) into registers, then wave w computes
// the scores of positions 64 w + lane for the G query heads from the lane's
// key row in registers (query values through DPP row_newbcast, as
// k_scores) and the V rows go to LDS; wave g runs head g's softmax (the row
// in registers, DPP maximum, Schraudolph on the first 8 floor(n/8)
// positions, expf on the tail; chain j on lane j over the position-major row
// at stride 8, the zeros past 8 floor(n/8) leaving it unchanged) and stores
// p = e * (1/sum) over the scores; thread (g, d) then runs the PV chain of
// head g, dim d.  Positions up to NMAX.
template <int HD, int G, int NMAX>
__global__ __launch_bounds__(512) void k_attn1s(const float *__restrict__ q, const float *__restrict__ kc,
                                                const float *__restrict__ vc, int cap, int vstride, int pos0,
                                                float scale, float *__restrict__ out, const int *__restrict__ st) {
  constexpr int NT = 512, STR = NMAX + 4, KSTR = HD + 4, KV4 = HD * (NMAX / 4) / NT;
  static_assert(G * HD == NT && NMAX % 64 == 0 && NMAX <= 64 * (NT / 64), "a lane per position and chain");
  static_assert(KV4 * NT == HD * (NMAX / 4), "whole V and key float4s per thread");
  typedef float f4 __attribute__((ext_vector_type(4)));
  // The key rows [position][HD + 4], then the V rows [dim][position].
  constexpr int XF = (NMAX * KSTR > HD * STR) ? NMAX * KSTR : HD * STR;
  __shared__ __align__(16) float xs[XF];
  __shared__ __align__(16) float ps[G * STR];  // scores, then probabilities [head][position]
  __shared__ __align__(16) float qs[G * HD];
  if (st) pos0 = st[0];
  const int n = pos0 + 1, n8x8 = n & ~7, nv = (n + 63) & ~63;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kvh = blockIdx.x;
  // Key float4 i = tid + 512 k: position i / (HD / 4), clamped to the last;
  // V float4 i: dim i / (NMAX / 4), positions 4 (i % (NMAX / 4)).., clamped
  // to the row.  Both requested before any is used.
  f4 kr[KV4], vr[KV4];
  const float *kb = kc + (size_t)kvh * cap * HD;
  const float *vb = vc + (size_t)kvh * HD * vstride;
#pragma unroll
  for (int k = 0; k < KV4; ++k) {
    const int i = tid + NT * k, r = i / (HD / 4), c4 = i % (HD / 4);
    if (r < nv) kr[k] = reinterpret_cast<const f4 *>(kb + (size_t)min(r, n - 1) * HD)[c4];
  }
#pragma unroll
  for (int k = 0; k < KV4; ++k) {
    const int i = tid + NT * k, d = i / (NMAX / 4), p = 4 * (i % (NMAX / 4));
    if (p < nv) vr[k] = *reinterpret_cast<const f4 *>(vb + (size_t)d * vstride + min(p, vstride - 4));
  }
  if (tid < G * HD / 4)
    reinterpret_cast<f4 *>(qs)[tid] = reinterpret_cast<const f4 *>(q + (size_t)kvh * G * HD)[tid];
#pragma unroll
  for (int k = 0; k < KV4; ++k) {
    const int i = tid + NT * k, r = i / (HD / 4), c4 = i % (HD / 4);
    if (r < nv) *reinterpret_cast<f4 *>(xs + r * KSTR + 4 * c4) = kr[k];
  }
  __syncthreads();
  // Scores of position s = 64 wave + lane for the G heads.
  const int s = 64 * wave + lane;
  if (64 * wave < n) {
    float qb[G][HD / 16];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int mm = 0; mm < HD / 16; ++mm) qb[g][mm] = qs[g * HD + 16 * mm + (lane & 15)];
    float a[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) a[g][i] = 0.0f;
    score_chunks<HD, G>(std::make_integer_sequence<int, HD / 8>{}, reinterpret_cast<const sf4 *>(xs + s * KSTR),
                        qb, a);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float d = ((a[g][0] + a[g][4]) + (a[g][1] + a[g][5])) + ((a[g][2] + a[g][6]) + (a[g][3] + a[g][7]));
      if (s < n) ps[g * STR + s] = d * scale;
    }
  }
  __syncthreads();  // the key rows are read: the region takes the V rows
#pragma unroll
  for (int k = 0; k < KV4; ++k) {
    const int i = tid + NT * k, d = i / (NMAX / 4), p = 4 * (i % (NMAX / 4));
    if (p < nv) *reinterpret_cast<f4 *>(xs + d * STR + p) = vr[k];
  }
  __syncthreads();
  if (wave < G) {
    float *row = ps + wave * STR;
    constexpr int NB = NMAX / 64;
    float v[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) v[k] = row[min(lane + 64 * k, n - 1)];
    const float xt = row[min(n8x8 + (lane & 7), n - 1)];  // tail value (lanes < n - n8x8)
    float mx = v[0];
#pragma unroll
    for (int k = 1; k < NB; ++k) mx = fmaxf(mx, v[k]);
    mx = wave_max_dpp(mx);
    // schraudolph(-inf) is +0: positions from 8 floor(n/8) on hold 0.
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int p = lane + 64 * k;
      v[k] = rai_exact::schraudolph(p < n8x8 ? v[k] - mx : -INFINITY);
      row[p] = v[k];
    }
    const float et = lane < n - n8x8 ? rai_exact::expf_glibc(xt - mx) : 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Chain j on lane j: e_{8i+j} for i < NMAX / 8 in order (+0 past n / 8).
    float acc = 0.0f;
    if (lane < 8) {
      float r[NMAX / 8];
#pragma unroll
      for (int i = 0; i < NMAX / 8; ++i) r[i] = row[8 * i + lane];
#pragma unroll
      for (int i = 0; i < NMAX / 8; ++i) acc = acc + r[i];
    }
    float c[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), k));
    float sum = ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
#pragma unroll
    for (int k = 0; k < 7; ++k)
      if (k < n - n8x8) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(et), k));
    const float inv = 1.0f / sum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < NB; ++k) row[lane + 64 * k] = v[k] * inv;
    if (lane < n - n8x8) row[n8x8 + lane] = et * inv;
  }
  __syncthreads();
  {
    const int g = tid / HD, d = tid % HD;
    const float acc = pv_chunk<NMAX>(reinterpret_cast<const float4 *>(xs + d * STR),
                                     reinterpret_cast<const float4 *>(ps + g * STR), n, 0.0f);
    out[(size_t)(kvh * G + g) * HD + d] = acc;
  }
}

// PV for any head_dim: thread per output element, same chain order.  V
// layout: DMAJOR [kv][hd][vstride], else [kv][cap][hd].
template <bool DMAJOR>
__global__ __launch_bounds__(64) void k_pv_any(const float *__restrict__ P,
                                               const float *__restrict__ vc, int cap, int vstride,
                                               int pos0, int m, int nh, int nkv, int hd,
                                               int sstride, float *__restrict__ out,
                                               const int *__restrict__ st) {
  if (st) pos0 = st[0];
  const int G = nh / nkv;
  const size_t gid = (size_t)blockIdx.x * 64 + threadIdx.x;
  if (gid >= (size_t)m * nh * hd) return;
  const int row = (int)(gid / hd), d = (int)(gid - (size_t)row * hd);
  const int t = row / nh, h = row - t * nh;
  const int n = pos0 + t + 1;
  const float *p = P + (size_t)row * sstride;
  const float inv = p[sstride - 1];  // the softmax's 1/sum: p_s = e_s * inv
  const size_t step = DMAJOR ? 1 : (size_t)hd;
  const float *vb = DMAJOR ? vc + ((size_t)(h / G) * hd + d) * vstride
                           : vc + (size_t)(h / G) * cap * hd + d;
  float acc = 0.0f;
  int s = 0;
  for (; s + 8 <= n; s += 8) {
    float pv[8], vv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      pv[u] = p[s + u] * inv;
      vv[u] = vb[(size_t)(s + u) * step];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = __fmaf_rn(pv[u], vv[u], acc);
  }
  for (; s < n; ++s) acc = __fmaf_rn(p[s] * inv, vb[(size_t)s * step], acc);
  out[(size_t)row * hd + d] = acc;
}

// Group 32, rows of at most 32 * P groups: the row and the norm weights in
// registers, the sum of squares over a chain-major LDS copy (one block per
// token).
template <int P>
__global__ __launch_bounds__(256) void k_norm_quant_r(const float *__restrict__ x, const float *__restrict__ w,
                                                      float *__restrict__ normed, int8_t *__restrict__ q_split,
                                                      int8_t *__restrict__ q_nat, float *__restrict__ scales,
                                                      float *__restrict__ sums, int n, float eps, _Float16 *qa) {
  extern __shared__ __align__(16) float xsr[];
  const int t = blockIdx.x, groups = n / 32;
  float xr[P][4], wr[P][4];
  rmsnorm_regs_load<32, P>(x + (size_t)t * n, w, n, xr, wr);
  rmsnorm_quant_regs<32, P>(xr, wr, n, eps, xsr, q_split + (size_t)t * n, 32, scales + (size_t)t * groups,
                            sums + (size_t)t * groups, q_nat ? q_nat + (size_t)t * n : nullptr,
                            normed ? normed + (size_t)t * n : nullptr, qa, t);
}

template <int GS>
void launch_norm_quant_t(const float *x, const float *w, float *normed, int m, int n, float eps,
                         int8_t *q_split, int8_t *q_nat, float *scales, float *sums,
                         hipStream_t s, _Float16 *qa = nullptr) {
  if (GS == 32 && n <= 32 * 32 * 4) {
    const size_t smem = sizeof(float) * (size_t)rms_scratch_floats(n);
    const int groups = n / 32;
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(m), dim3(256), smem, s, x, w, normed, q_split, q_nat, scales, sums, n, eps, qa);
    };
    if (groups <= 32) go(k_norm_quant_r<1>);
    else if (groups <= 64) go(k_norm_quant_r<2>);
    else if (groups <= 96) go(k_norm_quant_r<3>);
    else go(k_norm_quant_r<4>);
    return;
  }
  const size_t smem = (GS > 0 ? 1 : 2) * sizeof(float) * (size_t)n;
  static size_t configured = 0;
  if (smem > 48 * 1024 && smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_norm_quant<GS>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  hipLaunchKernelGGL(k_norm_quant<GS>, dim3(m), dim3(256), smem, s, x, w, normed, q_split, q_nat,
                     scales, sums, n, eps, qa);
}

template <int GS>
void launch_silu_quant_t(float *gate, const float *up, int m, int n, int ld, int8_t *q_split,
                         int8_t *q_nat, float *scales, float *sums, hipStream_t s, _Float16 *qa) {
  const int groups = n / GS;
  hipLaunchKernelGGL(k_silu_quant<GS>, dim3((groups + 31) / 32, m), dim3(256), 0, s, gate, up, n,
                     ld, q_split, q_nat, scales, sums, qa);
}

}  // namespace

void launch_rmsnorm(const float *x, const float *w, float *out, float *resid, int m, int n,
                    float eps, hipStream_t s) {
  if (resid)
    (void)hipMemcpyAsync(resid, x, sizeof(float) * (size_t)m * n, hipMemcpyDeviceToDevice, s);
  launch_norm_quant_t<0>(x, w, out, m, n, eps, nullptr, nullptr, nullptr, nullptr, s);
}

bool fused_quant_ok(int n, int gs) {
  return (gs == 32 || gs == 64 || gs == 128) && n % gs == 0 && n % 8 == 0;
}

void launch_norm_quant(const float *x, const float *w, float *normed, int m, int n, float eps,
                       int gs, int8_t *q_split, int8_t *q_nat, float *scales, float *sums,
                       hipStream_t s, _Float16 *qa) {
  if (gs == 32)
    launch_norm_quant_t<32>(x, w, normed, m, n, eps, q_split, q_nat, scales, sums, s, qa);
  else if (gs == 64)
    launch_norm_quant_t<64>(x, w, normed, m, n, eps, q_split, q_nat, scales, sums, s);
  else
    launch_norm_quant_t<128>(x, w, normed, m, n, eps, q_split, q_nat, scales, sums, s);
}

void launch_quant(const float *x, int m, int n, int gs, int8_t *q_split, int8_t *q_nat,
                  float *scales, float *sums, hipStream_t s, _Float16 *qa) {
  const dim3 grid((n / gs + 31) / 32, m);
  if (gs == 32)
    hipLaunchKernelGGL(k_quant<32>, grid, dim3(256), 0, s, x, n, q_split, q_nat, scales, sums, qa);
  else if (gs == 64)
    hipLaunchKernelGGL(k_quant<64>, grid, dim3(256), 0, s, x, n, q_split, q_nat, scales, sums, nullptr);
  else
    hipLaunchKernelGGL(k_quant<128>, grid, dim3(256), 0, s, x, n, q_split, q_nat, scales, sums, nullptr);
}

void launch_silu_quant(float *gate, const float *up, int m, int n, int ld, int gs,
                       int8_t *q_split, int8_t *q_nat, float *scales, float *sums,
                       hipStream_t s, _Float16 *qa) {
  if (gs == 32)
    launch_silu_quant_t<32>(gate, up, m, n, ld, q_split, q_nat, scales, sums, s, qa);
  else if (gs == 64)
    launch_silu_quant_t<64>(gate, up, m, n, ld, q_split, q_nat, scales, sums, s, nullptr);
  else
    launch_silu_quant_t<128>(gate, up, m, n, ld, q_split, q_nat, scales, sums, s, nullptr);
}

// Floats per score row: the positions, then a slot for the softmax's
// 1/sum, rounded up to a multiple of 4 (16-byte rows).
static int score_stride(int nmax) { return (nmax + 4) & ~3; }

size_t attention_scores_floats(int m, int nh, int ctx) {
  return (size_t)std::min(m, kAttnTokens) * nh * (size_t)score_stride(ctx);
}

static int g_pv_spin = kPvSpin;

void set_attention_spin(int polls) { g_pv_spin = polls > 0 ? polls : kPvSpin; }

void launch_attention(const float *q, int q_ld, const float *kc, const float *vc, int cap,
                      int vstride, int pos0, int m, int nh, int nkv, int hd, float scale,
                      float *out, float *scores, hipStream_t s, const int *st, int *err, int stages,
                      int span) {
  for (int t0 = 0; t0 < m; t0 += kAttnTokens) {
    const int mt = std::min(kAttnTokens, m - t0);
    const int p0 = pos0 + t0;
    // With a step record the position is on the device: the grids, the
    // score stride and the softmax kernel are those of the span of
    // positions the caller gives (by default the first span), so the
    // launch does not depend on the position.
    const int nmax = st ? (span > 0 ? std::min(cap, span) : attn_span(cap, 1)) : p0 + mt;
    const int sstride = score_stride(nmax);
    const float *qt = q + (size_t)t0 * q_ld;
    float *ot = out + (size_t)t0 * nh * hd;
    if (stages == 7 && mt == 1 && nh == 8 * nkv && hd == 64 && nmax <= 384 && vstride > 0 && vstride % 64 == 0) {
      // One token over a short context: scores, softmax and PV in one launch
      // (11.0 against 3.5 + 4.0 + 4.7 us at 128-256 positions for the
      // TinyLlama shape; the block's key and V loads, 4 CUs for 4 kv heads,
      // take 2.6 of them).
      hipLaunchKernelGGL((k_attn1s<64, 8, 384>), dim3(nkv), dim3(512), 0, s, qt, kc, vc, cap, vstride, p0, scale, ot,
                         st);
      continue;
    }
    if (stages & 1) launch_scores(qt, q_ld, kc, cap, p0, mt, nh, nkv, hd, scale, scores, sstride, nmax, st, s);
    if (!(stages & 2)) {
    } else if (mt > 12 && nmax <= 4096) {
      // Many rows (prefill): one wave per row; per 4095-token Mistral-7B
      // prefill 5.8 / 9.0 / 13.4 us per launch for rows of <= 1024 / 2048 /
      // 4096 positions against 8.3 / 10.6 / 13.8 with a block per row (the
      // longest rows are bound by the score rows' read and write).
      if (nmax <= 1024)
        launch_softmax_w<16, 4>(scores, p0, mt, nh, sstride, st, s);
      else if (nmax <= 2048)
        launch_softmax_w<32, 4>(scores, p0, mt, nh, sstride, st, s);
      else
        launch_softmax_w<64, 4>(scores, p0, mt, nh, sstride, st, s);
    } else if (nmax <= 512 * 16) {
      // Chains from registers (k_softmax_c): the chain-major rows hold
      // 64 NB steps each.
      const dim3 g(nh, mt);
      auto go = [&](auto kern, int) {
        hipLaunchKernelGGL(kern, g, dim3(512), 0, s, scores, p0, nh, sstride, st);
      };
      if (nmax <= 512 * 2)
        go(k_softmax_c<2>, 2);
      else if (nmax <= 512 * 4)
        go(k_softmax_c<4>, 4);
      else if (nmax <= 512 * 8)
        go(k_softmax_c<8>, 8);
      else
        go(k_softmax_c<16>, 16);
    } else if (nmax <= 512 * 32) {
      const int cstr = softmax_r_stride(nmax);
      const size_t rsm = sizeof(float) * 8 * (size_t)cstr;
      hipLaunchKernelGGL(k_softmax_r<32>, dim3(nh, mt), dim3(512), rsm, s, scores, p0, nh, sstride, cstr, st);
    } else {
      hipLaunchKernelGGL(k_softmax_l, dim3(nh, mt), dim3(512), 0, s, scores, p0, nh, sstride, st);
    }
    const size_t total = (size_t)mt * nh * hd;
    const int G = nh / nkv;
    const int DL = (G == 2) ? 32 : 16;
    const bool stream = vstride > 0 && vstride % 64 == 0 &&
                        (G == 1 || G == 2 || G == 4 || G == 8 || G == 16) && hd % DL == 0;
    if (!(stages & 4)) {
    } else if (stream) {
      // Tokens per block: one for one or two tokens (more blocks), three up
      // to twelve (the verify batch), four beyond; tile length and loader
      // waves measured on 4.1K-4.35K positions with V streamed from HBM (one
      // token: 512-position tiles and two loaders, 21.0 -> 20.0 us against
      // 256 and four; the loaders' registers spill from 640 positions or four
      // loaders at 512; three tokens: 256 and three).
      if (G == 4 && mt > 12 && hd % 32 == 0)
        // Prefill batches (128 tokens per launch): 32-dim slices, eight
        // tokens per block, four per compute lane (each V read feeds four
        // chains; a kv head's probability rows are read by four slice
        // blocks instead of eight), 64-position tiles and two loaders, whose
        // registers (126 per lane) let two blocks share a CU: 0.483 s per
        // 4095-token Mistral-7B prefill against 0.491 with 128-position
        // tiles (236 registers, one block per CU) and 0.506 with 64-token
        // launches.
        launch_pv_flag<32, 4, 64, 8, 2, 4>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin,
                                           s);
      else if (G == 4 && mt > 12)
        launch_pv_flag<16, 4, 128, 8, 4, 2>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin,
                                            s);
      else if (G == 4 && mt > 2)
        launch_pv_flag<16, 4, 256, 3, 3>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else if (G == 4)
        launch_pv_flag<16, 4, 512, 1, 2>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else if (G == 8 && mt == 1)
        // One token, eight query heads per kv head (TinyLlama-shaped): 8-dim
        // slices (one compute wave of 8 heads x 8 dims) with 512-position
        // tiles and two loaders: 11.97 us at 2048 positions, head_dim 64,
        // against 14.06 with 16-dim slices, 256-position tiles and six
        // loaders (12.3-14.0 for the four other shapes measured).
        launch_pv_flag<8, 8, 512, 1, 2>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else if (G == 8)
        launch_pv_flag<16, 8, 256, 1, 6>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else if (G == 16)
        launch_pv_flag<16, 16, 256, 1, 4>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else if (G == 2)
        launch_pv_flag<32, 2, 128, 1, 7>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else if (mt > 4)
        // One query head per kv head: 16-d slices, so a wave's four lane
        // rows take four tokens of one head (eight tokens in two compute
        // waves here) and a 256-position tile fits the loaders' registers
        // (64-d slices needed 64-position tiles: 22.5 -> 15.1 us at nine
        // tokens and 2100 positions, 19.1 -> 13.4 us at one).
        launch_pv_flag<16, 1, 256, 8, 3>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
      else
        launch_pv_flag<16, 1, 256, 4, 2>(scores, vc, vstride, p0, mt, nh, nkv, hd, sstride, ot, st, err, g_pv_spin, s);
    } else if (vstride > 0) {
      hipLaunchKernelGGL(k_pv_any<true>, dim3((unsigned)((total + 63) / 64)), dim3(64), 0, s, scores,
                         vc, cap, vstride, p0, mt, nh, nkv, hd, sstride, ot, st);
    } else {
      hipLaunchKernelGGL(k_pv_any<false>, dim3((unsigned)((total + 63) / 64)), dim3(64), 0, s, scores,
                         vc, cap, 0, p0, mt, nh, nkv, hd, sstride, ot, st);
    }
  }
}

}  // namespace rai
