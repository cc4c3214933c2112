// gfx950 kernels for the prompt-lookup / W4A8 hot path.
//
// Every kernel reproduces the f32 operation order of rai's AVX2 CPU path
// (rai-infer/src/gemm.rs, layers.rs), so outputs are bit-identical to it:
// the library is built with -ffp-contract=off and fuses a multiply-add only
// where the reference uses an FMA intrinsic.  Integer dot products use
// v_dot4 (exact int32).  Wavefronts are 64 lanes.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>

#include "exact_math.h"
#include "kernels.h"
#include "quant_dev.h"

namespace rai {

namespace {

__device__ __forceinline__ float f16bits(uint16_t b) { return __half2float(__ushort_as_half(b)); }

// IEEE division, correctly rounded (HIP compiles `/` that way by default;
// the helper only names the intent at the call sites that need it).
__device__ __forceinline__ float __fdiv_exact(float a, float b) { return a / b; }

// _mm256 horizontal sum order of gemm.rs:527-533 / layers.rs:1303-1310.
__device__ __forceinline__ float hsum8(const float *a) {
  return ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Integer dot of one 8-column block: low nibbles (even columns) against the
// 4 even activations, high nibbles against the 4 odd ones
// (the PMADDUBSW pairing of gemm.rs:470-476).
__device__ __forceinline__ int block_dot(uint32_t codes, uint32_t q_even, uint32_t q_odd, int acc) {
  const uint32_t lo = codes & 0x0F0F0F0Fu;
  const uint32_t hi = (codes >> 4) & 0x0F0F0F0Fu;
  return dot4(hi, q_odd, dot4(lo, q_even, acc));
}

// Column c of a block-split row: 8-column block b holds its even columns at
// 8b+0..3 and its odd columns at 8b+4..7.
__device__ __forceinline__ int split_index(int c) {
  const int j = c & 7;
  return (c & ~7) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

// ------------------------------------------------------------ quantize --

// One thread per (token, group): absmax, scale, int8 codes (RNE on the
// 8-wide body, half-away on the pair tail), and the 8-lane input sum
// (gemm.rs:172-212, 280-374).
__global__ void k_quantize(const float *__restrict__ x, int m, int k, int gs, int groups,
                           int8_t *__restrict__ q_nat, int8_t *__restrict__ q_split,
                           float *__restrict__ scales, float *__restrict__ sums) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (g >= groups || t >= m) return;
  const float *row = x + (size_t)t * k;
  const int start = g * gs;
  const int end = min(start + gs, k);
  const int len = end - start;
  const int c8 = len / 8;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float absmax = 0.0f;
  for (int i = 0; i < c8; ++i)
    for (int j = 0; j < 8; ++j) {
      const float v = row[start + i * 8 + j];
      acc[j] = acc[j] + v;
      absmax = fmaxf(absmax, fabsf(v));
    }
  float total = hsum8(acc);
  for (int i = c8 * 8; i < len; ++i) {
    const float v = row[start + i];
    total = total + v;
    const float a = fabsf(v);
    if (a > absmax) absmax = a;
  }
  sums[(size_t)t * groups + g] = total;
  const float scale = absmax > 1e-10f ? __fdiv_exact(absmax, 127.0f) : 1.0f;
  const float inv = __fdiv_exact(1.0f, scale);
  scales[(size_t)t * groups + g] = scale;
  int8_t *qn = q_nat + (size_t)t * k;
  int8_t *qs = q_split ? q_split + (size_t)t * k : nullptr;
  for (int i = 0; i < len; ++i) {
    const float v = row[start + i] * inv;
    float r = (i < c8 * 8) ? rintf(v) : roundf(v);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    const int8_t q = (int8_t)(int)r;
    qn[start + i] = q;
    if (qs) qs[split_index(start + i)] = q;
  }
}

// ---------------------------------------------------------- w4a8 simple --

// One thread per (row, token), the full reference order for any even group
// size, partial last group and unquantized f32 tail (gemm.rs:401-539).
__global__ void k_w4a8_simple(float *out, const float *add, const uint8_t *__restrict__ nib,
                              const uint8_t *__restrict__ params, const float *__restrict__ x,
                              const int8_t *__restrict__ q_nat, const float *__restrict__ scales,
                              const float *__restrict__ sums, int rows, int cols, int m, int gs,
                              int groups) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (r >= rows || t >= m) return;
  const uint8_t *nrow = nib + (size_t)r * (cols / 2);
  const uint8_t *prow = params + (size_t)r * groups * 4;
  const int8_t *q = q_nat + (size_t)t * cols;
  const float *xr = x + (size_t)t * cols;
  float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float zc = 0.0f;
  for (int g = 0; g < groups; ++g) {
    const uint16_t sb = (uint16_t)(prow[g * 4] | (prow[g * 4 + 1] << 8));
    const uint16_t zb = (uint16_t)(prow[g * 4 + 2] | (prow[g * 4 + 3] << 8));
    const float ws = f16bits(sb), wz = f16bits(zb);
    zc = zc + wz * sums[(size_t)t * groups + g];
    const float cs = ws * scales[(size_t)t * groups + g];
    const int col0 = g * gs;
    const int ags = min(gs, cols - col0);
    const int c64 = ags / 64;
    int s64[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < c64; ++c)
      for (int l = 0; l < 8; ++l)
        for (int j = 0; j < 8; ++j) {
          const int col = col0 + 64 * c + 8 * l + j;
          const uint8_t b = nrow[col >> 1];
          const int code = (col & 1) ? (b >> 4) : (b & 15);
          s64[l] += code * (int)q[col];
        }
    for (int l = 0; l < 8; ++l) f[l] = f[l] + (float)s64[l] * cs;
    const int done = c64 * 64;
    const bool has32 = done + 32 <= ags;
    if (has32) {
      for (int l = 0; l < 4; ++l) {
        int s = 0;
        for (int j = 0; j < 8; ++j) {
          const int col = col0 + done + 8 * l + j;
          const uint8_t b = nrow[col >> 1];
          const int code = (col & 1) ? (b >> 4) : (b & 15);
          s += code * (int)q[col];
        }
        f[l] = f[l] + (float)s * cs;
      }
    }
    const int done2 = done + (has32 ? 32 : 0);
    if (done2 < ags) {
      float tacc = 0.0f;
      for (int tc = done2; tc + 1 < ags; tc += 2) {
        const uint8_t b = nrow[(col0 + tc) >> 1];
        const float a0 = (float)(b & 15) * xr[col0 + tc];
        const float a1 = (float)(b >> 4) * xr[col0 + tc + 1];
        tacc = tacc + (a0 + a1);
      }
      f[0] = f[0] + ws * tacc;
    }
  }
  const size_t oi = (size_t)t * rows + r;
  const float v = hsum8(f) + zc;
  out[oi] = add ? add[oi] + v : v;
}

// ------------------------------------------------------------ w4a8 fast --

// Tiled kernel for group sizes 32, 64 and 128 with full groups.
// A block owns kRows weight rows and all m (<= MT) tokens and walks K in
// tiles of GT groups.  Phase 1: every (row, group) item computes, for each
// token, the per-lane products fl(float(S_lane) * fl(ws*as)) and the zero
// term fl(z * xsum) into LDS.  Phase 2: each (token, chain, row) accumulator
// adds its products in group order, which is exactly the reference's
// sequential per-lane f32 accumulation.  NL = reference lanes that receive
// products (4 for group 32, 8 for groups 64/128); chain NL is the zero term.
constexpr int kRows = 16;
constexpr int kThreads = 256;

template <int GS, int MT>
struct FastCfg {
  static constexpr int NL = (GS == 32) ? 4 : 8;
  static constexpr int NC = NL + 1;
  // Groups per K tile, chosen to keep the product tile within 40 KB of LDS.
  static constexpr int GT = (GS == 32) ? (MT >= 16 ? 8 : 16) : (MT >= 16 ? 4 : 8);
  static constexpr int CPT = (MT * NC * kRows + kThreads - 1) / kThreads;
};

template <int GS, int MT>
__global__ __launch_bounds__(kThreads) void k_w4a8_fast(
    float *out, const float *add, const uint8_t *__restrict__ nib, const uint8_t *__restrict__ params,
    const int8_t *__restrict__ q_split, const float *__restrict__ scales,
    const float *__restrict__ sums, int rows, int cols, int m_total, int groups) {
  using C = FastCfg<GS, MT>;
  constexpr int NL = C::NL, NC = C::NC, GT = C::GT, CPT = C::CPT;
  extern __shared__ __align__(16) unsigned char smem[];
  const int t0 = blockIdx.y * MT;
  const int m = min(MT, m_total - t0);
  const int row0 = blockIdx.x * kRows;
  const int tid = threadIdx.x;
  // LDS carve-up: q tile [MT][GT*GS] bytes, scale/sum [MT][GT], products
  // [MT][NC][kRows][GT], final chain values reuse the product area.
  int8_t *qsh = reinterpret_cast<int8_t *>(smem);
  float *ash = reinterpret_cast<float *>(smem + MT * GT * GS);
  float *ssh = ash + MT * GT;
  float *psh = ssh + MT * GT;

  float acc[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) acc[j] = 0.0f;

  const int ktiles = (groups + GT - 1) / GT;
  const size_t row_bytes = (size_t)cols / 2;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int g0 = kt * GT;
    const int gcount = min(GT, groups - g0);
    // Stage the activation tile.
    {
      const int tile_bytes = gcount * GS;  // per token, multiple of 16
      const int vec_per_tok = tile_bytes / 16;
      for (int i = tid; i < m * vec_per_tok; i += kThreads) {
        const int t = i / vec_per_tok, v = i % vec_per_tok;
        const uint4 val = *reinterpret_cast<const uint4 *>(q_split + (size_t)(t0 + t) * cols +
                                                           (size_t)g0 * GS + v * 16);
        *reinterpret_cast<uint4 *>(qsh + t * GT * GS + v * 16) = val;
      }
      for (int i = tid; i < m * gcount; i += kThreads) {
        const int t = i / gcount, g = i % gcount;
        ash[t * GT + g] = scales[(size_t)(t0 + t) * groups + g0 + g];
        ssh[t * GT + g] = sums[(size_t)(t0 + t) * groups + g0 + g];
      }
    }
    __syncthreads();
    // Phase 1: products.
    if (tid < kRows * GT) {
      const int r = tid / GT, g = tid % GT;
      const int row = row0 + r;
      if (row < rows && g < gcount) {
        const uint8_t *pp = params + ((size_t)row * groups + g0 + g) * 4;
        const uint32_t pw = *reinterpret_cast<const uint32_t *>(pp);
        const float ws = f16bits((uint16_t)(pw & 0xFFFF));
        const float wz = f16bits((uint16_t)(pw >> 16));
        constexpr int NW = GS / 8;  // 8-column blocks (code dwords) per group
        uint32_t cw[NW];
        const uint8_t *cp = nib + (size_t)row * row_bytes + (size_t)(g0 + g) * (GS / 2);
#pragma unroll
        for (int v = 0; v < NW / 4; ++v) {
          const uint4 u = *reinterpret_cast<const uint4 *>(cp + v * 16);
          cw[v * 4 + 0] = u.x;
          cw[v * 4 + 1] = u.y;
          cw[v * 4 + 2] = u.z;
          cw[v * 4 + 3] = u.w;
        }
        for (int t = 0; t < m; ++t) {
          const uint32_t *qw = reinterpret_cast<const uint32_t *>(qsh + t * GT * GS + g * GS);
          int s[NL];
#pragma unroll
          for (int l = 0; l < NL; ++l) s[l] = 0;
#pragma unroll
          for (int b = 0; b < NW; ++b) s[b % NL] = block_dot(cw[b], qw[2 * b], qw[2 * b + 1], s[b % NL]);
          const float cs = ws * ash[t * GT + g];
          float *pt = psh + ((t * NC) * kRows + r) * GT + g;
#pragma unroll
          for (int l = 0; l < NL; ++l) pt[l * kRows * GT] = (float)s[l] * cs;
          pt[NL * kRows * GT] = wz * ssh[t * GT + g];
        }
      }
    }
    __syncthreads();
    // Phase 2: ordered accumulation.
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + j * kThreads;
      if (c < m * NC * kRows) {
        const float *p = psh + c * GT;
        float a = acc[j];
        for (int g = 0; g < gcount; ++g) a = a + p[g];
        acc[j] = a;
      }
    }
    __syncthreads();
  }
  // Epilogue: lane reduction in the reference's order, plus the zero term.
  float *fin = psh;  // [m][NC][kRows]
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = tid + j * kThreads;
    if (c < m * NC * kRows) fin[c] = acc[j];
  }
  __syncthreads();
  if (tid < m * kRows) {
    const int t = tid / kRows, r = tid % kRows;
    const int row = row0 + r;
    if (row < rows) {
      float f[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) f[l] = (l < NL) ? fin[(t * NC + l) * kRows + r] : 0.0f;
      const float zc = fin[(t * NC + NL) * kRows + r];
      const size_t oi = (size_t)(t0 + t) * rows + row;
      const float v = hsum8(f) + zc;
      out[oi] = add ? add[oi] + v : v;
    }
  }
}

template <int GS, int MT>
size_t fast_smem() {
  using C = FastCfg<GS, MT>;
  return (size_t)MT * C::GT * GS + 2 * sizeof(float) * MT * C::GT +
         sizeof(float) * (size_t)MT * C::NC * kRows * C::GT;
}

template <int GS, int MT>
void launch_fast_t(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                   const float *scales, const float *sums, int rows, int cols, int m, int groups,
                   hipStream_t s) {
  const size_t smem = fast_smem<GS, MT>();
  static bool configured = false;
  if (!configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_fast<GS, MT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = true;
  }
  dim3 grid((rows + kRows - 1) / kRows, (m + MT - 1) / MT);
  hipLaunchKernelGGL((k_w4a8_fast<GS, MT>), grid, dim3(kThreads), smem, s, out, add, nib, params,
                     q_split, scales, sums, rows, cols, m, groups);
}

template <int GS>
void launch_fast_gs(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                    const float *scales, const float *sums, int rows, int cols, int m, int groups,
                    hipStream_t s) {
  if (m <= 1)
    launch_fast_t<GS, 1>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else if (m <= 2)
    launch_fast_t<GS, 2>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else if (m <= 4)
    launch_fast_t<GS, 4>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else if (m <= 8)
    launch_fast_t<GS, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else
    launch_fast_t<GS, 16>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
}

// ------------------------------------------------------ w4a8 small-M v2 --

// Small-M (<= 16 tokens) W4A8 kernel for group sizes 32/64/128 with full
// groups, same two-phase arithmetic as k_w4a8_fast:
//   phase 1: item (row r, group g) -> per-token lane products
//            fl(float(S_lane) * fl(ws*as)) and zero terms fl(z*xsum) in LDS;
//   phase 2: each (token, chain, row) accumulator adds its tile's products in
//            group order (the reference's sequential per-lane f32 sums).
// A block owns R rows; a K tile holds GT = 256/R groups, one item per thread.
// Weights are prefetched PD tiles ahead in a register ring so the block
// keeps PD tiles of HBM traffic in flight.  Activations (int8, block-split),
// scales and sums are staged in LDS once per block when they fit (WHOLE),
// else one tile at a time with a one-tile register prefetch.  LDS strides are
// padded against bank conflicts.
template <int GS, int MT, int R, int PD, bool WHOLE>
struct SmallCfg {
  static constexpr int NL = (GS == 32) ? 4 : 8;
  static constexpr int NC = NL + 1;
  static constexpr int NW = GS / 8;          // code dwords per group
  static constexpr int GT = kThreads / R;    // groups per K tile
  static constexpr int PSTR = GT + 1;        // padded product stride
  static constexpr int QSTR = GS + 8;        // padded per-group q stride (bytes)
  static constexpr int CPT = (MT * NC * R + kThreads - 1) / kThreads;
  static constexpr int QV = (MT * GT * NW + kThreads - 1) / kThreads;  // uint2 per thread per tile
};

template <int GS, int MT, int R, int PD, bool WHOLE>
__global__ __launch_bounds__(kThreads) void k_w4a8_small(
    float *out, const float *add, const uint8_t *__restrict__ nib, const uint8_t *__restrict__ params,
    const int8_t *__restrict__ q_split, const float *__restrict__ scales,
    const float *__restrict__ sums, int rows, int cols, int m_total, int groups,
    const float *__restrict__ nx, const float *__restrict__ nw, float eps) {
  using C = SmallCfg<GS, MT, R, PD, WHOLE>;
  constexpr int NL = C::NL, NC = C::NC, NW = C::NW, GT = C::GT, PSTR = C::PSTR, QSTR = C::QSTR;
  constexpr int CPT = C::CPT, QV = C::QV;
  extern __shared__ __align__(16) unsigned char smem[];
  const int t0 = blockIdx.y * MT;
  const int m = min(MT, m_total - t0);
  const int row0 = blockIdx.x * R;
  const int tid = threadIdx.x;
  const int ktiles = (groups + GT - 1) / GT;
  const int gstage = WHOLE ? groups : GT;  // groups held per staged q buffer
  const int nbuf = WHOLE ? 1 : 2;
  // LDS: q [nbuf][MT][gstage][QSTR] bytes | scale, sum [nbuf][MT][gstage] f32
  //      | products [MT][NC][R][PSTR] f32
  // Sized by the launch's token count m (<= MT), see small_smem().
  const size_t qbytes = (size_t)nbuf * m * gstage * QSTR;
  int8_t *qsh = reinterpret_cast<int8_t *>(smem);
  float *ash = reinterpret_cast<float *>(smem + ((qbytes + 15) & ~size_t(15)));
  float *ssh = ash + nbuf * m * gstage;
  float *psh = ash + ((2 * nbuf * m * gstage + 3) & ~3);  // 16-byte aligned

  const int r_item = tid / GT, g_item = tid % GT;
  const int row_item = row0 + r_item;
  const bool row_ok = row_item < rows;
  const size_t row_bytes = (size_t)cols / 2;
  const uint8_t *nrow = nib + (size_t)(row_ok ? row_item : 0) * row_bytes;
  const uint8_t *prow = params + (size_t)(row_ok ? row_item : 0) * groups * 4;

  // Fused RMSNorm input (one token, whole K staged, group 32, at most 128
  // groups): its loads go out before the weights'.
  constexpr bool NORM_OK = MT == 1 && WHOLE && GS == 32;
  constexpr int NPN = NORM_OK ? 4 : 1;
  float xr[NPN][GS / 8], wr[NPN][GS / 8];
  if (NORM_OK && nx) rmsnorm_regs_load<GS, NPN>(nx, nw, cols, xr, wr);
  // Weight ring: tile kt lives in slot kt % PD.  Every load is issued,
  // clamped into the row (items past the row are never read back), so the
  // waits on earlier loads stay exact.
  uint32_t ring_c[PD][NW];
  uint32_t ring_p[PD];
  auto load_tile = [&](int kt, uint32_t (&c)[NW], uint32_t &p) {
    const int gi = min(kt * GT + g_item, groups - 1);
    const uint4 *cp = reinterpret_cast<const uint4 *>(nrow + (size_t)gi * (GS / 2));
#pragma unroll
    for (int v = 0; v < NW / 4; ++v) {
      const uint4 u = cp[v];
      c[4 * v + 0] = u.x;
      c[4 * v + 1] = u.y;
      c[4 * v + 2] = u.z;
      c[4 * v + 3] = u.w;
    }
    p = *reinterpret_cast<const uint32_t *>(prow + (size_t)gi * 4);
  };
  // Stage activations for groups [g0, g0+gn) of tokens t0.. into buffer b.
  auto stage_direct = [&](int b, int g0, int gn) {
    int8_t *qb = qsh + (size_t)b * m * gstage * QSTR;
    const int per_tok = gn * NW;  // uint2 per token
    for (int i = tid; i < m * per_tok; i += kThreads) {
      const int t = i / per_tok, rem = i % per_tok, g = rem / NW, w = rem % NW;
      const uint2 v = *reinterpret_cast<const uint2 *>(q_split + (size_t)(t0 + t) * cols +
                                                       (size_t)(g0 + g) * GS + w * 8);
      *reinterpret_cast<uint2 *>(qb + ((size_t)t * gstage + g) * QSTR + w * 8) = v;
    }
    for (int i = tid; i < m * gn; i += kThreads) {
      const int t = i / gn, g = i % gn;
      ash[(b * m + t) * gstage + g] = scales[(size_t)(t0 + t) * groups + g0 + g];
      ssh[(b * m + t) * gstage + g] = sums[(size_t)(t0 + t) * groups + g0 + g];
    }
  };

  float acc[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) acc[j] = 0.0f;

#pragma unroll
  for (int j = 0; j < PD; ++j) load_tile(j, ring_c[j], ring_p[j]);
  if constexpr (NORM_OK) {
    if (nx)
      rmsnorm_quant_regs<GS, NPN>(xr, wr, cols, eps, psh, qsh, QSTR, ash, ssh);
    else
      stage_direct(0, 0, groups);
  } else {
    stage_direct(0, 0, WHOLE ? groups : min(GT, groups));
  }
  __syncthreads();

  uint2 qn[QV];
  float an = 0.0f, sn = 0.0f;
  for (int kt0 = 0; kt0 < ktiles; kt0 += PD) {
#pragma unroll
    for (int j = 0; j < PD; ++j) {
      const int kt = kt0 + j;
      if (kt >= ktiles) break;
      const int g0 = kt * GT;
      const int gcount = min(GT, groups - g0);
      const int buf = WHOLE ? 0 : (kt & 1);
      const int gbase = WHOLE ? g0 : 0;
      // Prefetch the next tile's activations (per-tile staging only).
      const int gn_next = (kt + 1 < ktiles) ? min(GT, groups - (kt + 1) * GT) : 0;
      if (!WHOLE && gn_next > 0) {
#pragma unroll
        for (int v = 0; v < QV; ++v) {
          const int i = tid + v * kThreads;
          if (i < m * gn_next * NW) {
            const int t = i / (gn_next * NW), rem = i % (gn_next * NW), g = rem / NW, w = rem % NW;
            qn[v] = *reinterpret_cast<const uint2 *>(q_split + (size_t)(t0 + t) * cols +
                                                     (size_t)((kt + 1) * GT + g) * GS + w * 8);
          }
        }
        if (tid < m * gn_next) {
          const int t = tid / gn_next, g = tid % gn_next;
          an = scales[(size_t)(t0 + t) * groups + (kt + 1) * GT + g];
          sn = sums[(size_t)(t0 + t) * groups + (kt + 1) * GT + g];
        }
      }
      // Phase 1: products of this thread's (row, group) item.
      if (row_ok && g_item < gcount) {
        const uint32_t pw = ring_p[j];
        const float ws = f16bits((uint16_t)(pw & 0xFFFF));
        const float wz = f16bits((uint16_t)(pw >> 16));
        const int gq = gbase + g_item;
        for (int t = 0; t < m; ++t) {
          const int8_t *qg = qsh + ((size_t)(buf * m + t) * gstage + gq) * QSTR;
          int sl[NL];
#pragma unroll
          for (int l = 0; l < NL; ++l) sl[l] = 0;
#pragma unroll
          for (int b = 0; b < NW; ++b) {
            const uint2 qv = *reinterpret_cast<const uint2 *>(qg + 8 * b);
            sl[b % NL] = block_dot(ring_c[j][b], qv.x, qv.y, sl[b % NL]);
          }
          const float cs = ws * ash[(buf * m + t) * gstage + gq];
          float *pt = psh + ((size_t)(t * NC) * R + r_item) * PSTR + g_item;
#pragma unroll
          for (int l = 0; l < NL; ++l) pt[(size_t)l * R * PSTR] = (float)sl[l] * cs;
          pt[(size_t)NL * R * PSTR] = wz * ssh[(buf * m + t) * gstage + gq];
        }
      }
      // Refill this ring slot with tile kt + PD (clamped past the row).
      load_tile(kt + PD, ring_c[j], ring_p[j]);
      // Publish the next tile's activations into the other buffer.
      if (!WHOLE && gn_next > 0) {
        int8_t *qb = qsh + (size_t)((kt + 1) & 1) * m * gstage * QSTR;
#pragma unroll
        for (int v = 0; v < QV; ++v) {
          const int i = tid + v * kThreads;
          if (i < m * gn_next * NW) {
            const int t = i / (gn_next * NW), rem = i % (gn_next * NW), g = rem / NW, w = rem % NW;
            *reinterpret_cast<uint2 *>(qb + ((size_t)t * gstage + g) * QSTR + w * 8) = qn[v];
          }
        }
        if (tid < m * gn_next) {
          const int t = tid / gn_next, g = tid % gn_next;
          ash[(((kt + 1) & 1) * m + t) * gstage + g] = an;
          ssh[(((kt + 1) & 1) * m + t) * gstage + g] = sn;
        }
      }
      __syncthreads();
      // Phase 2: ordered accumulation.
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int ch = tid + c * kThreads;
        if (ch < m * NC * R) {
          const float *p = psh + (size_t)ch * PSTR;
          float a = acc[c];
          for (int g = 0; g < gcount; ++g) a = a + p[g];
          acc[c] = a;
        }
      }
      __syncthreads();
    }
  }
  float *fin = psh;  // [m][NC][R]
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + c * kThreads;
    if (ch < m * NC * R) fin[ch] = acc[c];
  }
  __syncthreads();
  if (tid < m * R) {
    const int t = tid / R, r = tid % R;
    const int row = row0 + r;
    if (row < rows) {
      float f[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) f[l] = (l < NL) ? fin[(t * NC + l) * R + r] : 0.0f;
      const size_t oi = (size_t)(t0 + t) * rows + row;
      const float v = hsum8(f) + fin[(t * NC + NL) * R + r];
      out[oi] = add ? add[oi] + v : v;
    }
  }
}

// LDS bytes for a launch whose token tiles hold at most m tokens.
// With a fused RMSNorm (norm_cols > 0) the products area doubles as the
// row scratch.
template <int GS, int MT, int R, int PD, bool WHOLE>
size_t small_smem(int groups, int m, int norm_cols = 0) {
  using C = SmallCfg<GS, MT, R, PD, WHOLE>;
  const int gstage = WHOLE ? groups : C::GT;
  const int nbuf = WHOLE ? 1 : 2;
  const size_t qbytes = (((size_t)nbuf * m * gstage * C::QSTR) + 15) & ~size_t(15);
  return qbytes + sizeof(float) * ((2 * (size_t)nbuf * m * gstage + 3) & ~size_t(3)) +
         std::max(sizeof(float) * (size_t)m * C::NC * R * C::PSTR,
                  norm_cols ? sizeof(float) * (size_t)rms_scratch_floats(norm_cols) : size_t(0));
}

template <int GS, int MT, int R, int PD, bool WHOLE>
void launch_small_t(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                    const float *scales, const float *sums, int rows, int cols, int m, int groups,
                    hipStream_t s, const float *nx = nullptr, const float *nw = nullptr, float eps = 0.0f) {
  const size_t smem = small_smem<GS, MT, R, PD, WHOLE>(groups, std::min(m, MT), nx ? cols : 0);
  static size_t configured = 0;
  if (smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_small<GS, MT, R, PD, WHOLE>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  dim3 grid((rows + R - 1) / R, (m + MT - 1) / MT);
  hipLaunchKernelGGL((k_w4a8_small<GS, MT, R, PD, WHOLE>), grid, dim3(kThreads), smem, s, out, add,
                     nib, params, q_split, scales, sums, rows, cols, m, groups, nx, nw, eps);
}

// ---------------------------------------------------------- w4a8 M = 1 --

// (row, group) items each thread of the M = 1 kernel holds in registers.
constexpr int m1_items_per_thread(int gs) { return gs == 128 ? 4 : 8; }

// Single-token W4A8 kernel (decode), group sizes 32/64/128 with full groups.
// A block owns R rows and the whole K: its R*G (row, group) items are split
// over the 256 threads (up to IPT each) and every weight load is issued up
// front, so one HBM round trip covers the block.  Phase 1 writes each item's
// lane products fl(float(S_lane) * fl(ws*as)) and zero term fl(z*xsum) to
// LDS; phase 2 runs the NC*R sequential accumulators over all groups in
// order; the epilogue applies the reference's lane reduction.
template <int GS, int R, int IPT>
__global__ __launch_bounds__(kThreads) void k_w4a8_m1(
    float *out, const float *add, const uint8_t *__restrict__ nib, const uint8_t *__restrict__ params,
    const int8_t *__restrict__ q_split, const float *__restrict__ scales,
    const float *__restrict__ sums, int rows, int cols, int groups, const float *__restrict__ nx,
    const float *__restrict__ nw, float eps) {
  constexpr int NL = (GS == 32) ? 4 : 8;
  constexpr int NC = NL + 1;
  constexpr int NW = GS / 8;
  static_assert(NC * R <= kThreads, "one thread per accumulator chain");
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int row0 = blockIdx.x * R;
  const int pstr = groups + 1;  // padded product stride
  // LDS: q [K] (block-split) | scale, sum [G] | products [NC][R][G+1]
  // (16-byte aligned)
  int8_t *qsh = reinterpret_cast<int8_t *>(smem);
  float *ash = reinterpret_cast<float *>(smem + ((cols + 15) & ~15));
  float *ssh = ash + groups;
  float *psh = ash + ((2 * groups + 3) & ~3);  // 16-byte aligned
  const int items = R * groups;
  // Fused RMSNorm input (group 32, at most 128 groups): loaded first.
  constexpr int NP = (GS == 32) ? 4 : 1;
  float xr[NP][GS / 8], wr[NP][GS / 8];
  if (GS == 32 && nx) rmsnorm_regs_load<GS, NP>(nx, nw, cols, xr, wr);
  uint32_t cw[IPT][NW];
  uint32_t pw[IPT];
  int ir[IPT], ig[IPT];
#pragma unroll
  for (int j = 0; j < IPT; ++j) {
    const int i = tid + j * kThreads;
    ir[j] = i / groups;
    ig[j] = i - ir[j] * groups;
    // Every load is issued (clamped into the matrix; unused items are never
    // read back), so the waits on earlier loads stay exact.
    const int row = min(row0 + ir[j], rows - 1);
    const int gi = i < items ? ig[j] : 0;
    const uint4 *cp = reinterpret_cast<const uint4 *>(nib + (size_t)row * (cols / 2) + gi * (GS / 2));
#pragma unroll
    for (int v = 0; v < NW / 4; ++v) {
      const uint4 u = cp[v];
      cw[j][4 * v + 0] = u.x;
      cw[j][4 * v + 1] = u.y;
      cw[j][4 * v + 2] = u.z;
      cw[j][4 * v + 3] = u.w;
    }
    pw[j] = *reinterpret_cast<const uint32_t *>(params + ((size_t)row * groups + gi) * 4);
  }
  if (GS == 32 && nx) {
    // RMSNorm + quantization of the input row into LDS (the products area
    // serves as the row scratch) while the weight loads are in flight.
    rmsnorm_quant_regs<GS, NP>(xr, wr, cols, eps, psh, qsh, GS, ash, ssh);
  } else {
    for (int i = tid; i < cols / 16; i += kThreads)
      reinterpret_cast<uint4 *>(qsh)[i] = reinterpret_cast<const uint4 *>(q_split)[i];
    for (int i = tid; i < groups; i += kThreads) {
      ash[i] = scales[i];
      ssh[i] = sums[i];
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < IPT; ++j) {
    const int i = tid + j * kThreads;
    if (i < items && row0 + ir[j] < rows) {
      const float ws = f16bits((uint16_t)(pw[j] & 0xFFFF));
      const float wz = f16bits((uint16_t)(pw[j] >> 16));
      const uint2 *qg = reinterpret_cast<const uint2 *>(qsh + ig[j] * GS);
      int sl[NL];
#pragma unroll
      for (int l = 0; l < NL; ++l) sl[l] = 0;
#pragma unroll
      for (int b = 0; b < NW; ++b) {
        const uint2 qv = qg[b];
        sl[b % NL] = block_dot(cw[j][b], qv.x, qv.y, sl[b % NL]);
      }
      const float cs = ws * ash[ig[j]];
      float *pt = psh + ir[j] * pstr + ig[j];
#pragma unroll
      for (int l = 0; l < NL; ++l) pt[l * R * pstr] = (float)sl[l] * cs;
      pt[NL * R * pstr] = wz * ssh[ig[j]];
    }
  }
  __syncthreads();
  float acc = 0.0f;
  if (tid < NC * R) {
    const float *p = psh + tid * pstr;
    for (int g = 0; g < groups; ++g) acc = acc + p[g];
  }
  __syncthreads();
  if (tid < NC * R) psh[tid] = acc;  // chain c = l*R + r
  __syncthreads();
  if (tid < R && row0 + tid < rows) {
    float f[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) f[l] = (l < NL) ? psh[l * R + tid] : 0.0f;
    const float v = hsum8(f) + psh[NL * R + tid];
    out[row0 + tid] = add ? add[row0 + tid] + v : v;
  }
}

template <int GS, int R>
void launch_m1_t(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                 const float *scales, const float *sums, int rows, int cols, int groups,
                 hipStream_t s, const float *nx = nullptr, const float *nw = nullptr, float eps = 0.0f) {
  constexpr int NC = (GS == 32) ? 5 : 9;
  constexpr int IPT = m1_items_per_thread(GS);
  // With a fused RMSNorm the products area doubles as the row scratch.
  const size_t prod = std::max(4 * (size_t)NC * R * (groups + 1), nx ? 4 * (size_t)rms_scratch_floats(cols) : 0);
  const size_t smem = (size_t)((cols + 15) & ~15) + 4 * (size_t)((2 * groups + 3) & ~3) + prod;
  static size_t configured = 0;
  if (smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_m1<GS, R, IPT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  hipLaunchKernelGGL((k_w4a8_m1<GS, R, IPT>), dim3((rows + R - 1) / R), dim3(kThreads), smem, s,
                     out, add, nib, params, q_split, scales, sums, rows, cols, groups, nx, nw, eps);
}

// Rows per block: the largest power of two whose R*G items fit IPT per
// thread.  Returns false when one row's groups do not fit (very large K).
template <int GS>
bool launch_m1(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
               const float *scales, const float *sums, int rows, int cols, int groups,
               hipStream_t s) {
  const int cap = m1_items_per_thread(GS) * kThreads;
  if (groups > cap) return false;
  // Phase 2 gives each of the NC*R accumulator chains its own thread.
  constexpr bool allow32 = ((GS == 32) ? 5 : 9) * 32 <= kThreads;
  if constexpr (allow32) {
    if (32 * groups <= cap) {
      launch_m1_t<GS, 32>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
      return true;
    }
  }
  if (16 * groups <= cap)
    launch_m1_t<GS, 16>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
  else if (8 * groups <= cap)
    launch_m1_t<GS, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
  else if (4 * groups <= cap)
    launch_m1_t<GS, 4>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
  else if (2 * groups <= cap)
    launch_m1_t<GS, 2>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
  else
    launch_m1_t<GS, 1>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
  return true;
}

// Activation staging of the whole K fits comfortably in LDS.
constexpr size_t kWholeStageBytes = 24 * 1024;

template <int GS, int MT, int R = 16>
void launch_small_mt(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                     const float *scales, const float *sums, int rows, int cols, int m, int groups,
                     hipStream_t s) {
  constexpr int PD = 4;
  const size_t whole = (size_t)std::min(m, MT) * groups * (GS + 8 + 8);
  if (whole <= kWholeStageBytes)
    launch_small_t<GS, MT, R, PD, true>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else
    launch_small_t<GS, MT, R, PD, false>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
}

template <int GS>
void launch_small_gs(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                     const float *scales, const float *sums, int rows, int cols, int m, int groups,
                     hipStream_t s) {
  if (m <= 1)
    launch_small_mt<GS, 1>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else if (m <= 2)
    launch_small_mt<GS, 2>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else if (m <= 4)
    launch_small_mt<GS, 4>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else if (m <= 8 || GS > 32)  // groups 64/128 carry 9 chains: at most 8 tokens per tile
    launch_small_mt<GS, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
  else
    launch_small_mt<GS, 16>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
}

// --------------------------------------------------------- lane sums dbg --

__global__ void k_lane_sums(int32_t *__restrict__ out, const uint8_t *__restrict__ nib,
                            const int8_t *__restrict__ q_nat, int rows, int cols, int m, int gs,
                            int groups) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (idx >= rows * groups || t >= m) return;
  const int r = idx / groups, g = idx % groups;
  const uint8_t *nrow = nib + (size_t)r * (cols / 2);
  const int8_t *q = q_nat + (size_t)t * cols;
  int32_t *o = out + (((size_t)t * rows + r) * groups + g) * 12;
  const int col0 = g * gs;
  const int ags = min(gs, cols - col0);
  const int c64 = ags / 64;
  for (int l = 0; l < 8; ++l) {
    int s = 0;
    for (int c = 0; c < c64; ++c)
      for (int j = 0; j < 8; ++j) {
        const int col = col0 + 64 * c + 8 * l + j;
        const uint8_t b = nrow[col >> 1];
        s += ((col & 1) ? (b >> 4) : (b & 15)) * (int)q[col];
      }
    o[l] = s;
  }
  const int done = c64 * 64;
  for (int l = 0; l < 4; ++l) {
    int s = 0;
    if (done + 32 <= ags)
      for (int j = 0; j < 8; ++j) {
        const int col = col0 + done + 8 * l + j;
        const uint8_t b = nrow[col >> 1];
        s += ((col & 1) ? (b >> 4) : (b & 15)) * (int)q[col];
      }
    o[8 + l] = s;
  }
}

// -------------------------------------------------------- tied lm_head --

// quantize_hidden_i8 (gemm.rs:924-1047): +-63 per group, plus input sums.
__global__ void k_quantize63(const float *__restrict__ x, int m, int n, int gs, int groups,
                             int8_t *__restrict__ q, float *__restrict__ scales,
                             float *__restrict__ sums) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (g >= groups || t >= m) return;
  const float *row = x + (size_t)t * n;
  const int start = g * gs, end = min(start + gs, n), len = end - start, c8 = len / 8;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float absmax = 0.0f;
  for (int i = 0; i < c8; ++i)
    for (int j = 0; j < 8; ++j) {
      const float v = row[start + i * 8 + j];
      acc[j] = acc[j] + v;
      absmax = fmaxf(absmax, fabsf(v));
    }
  float total = hsum8(acc);
  for (int i = c8 * 8; i < len; ++i) {
    total = total + row[start + i];
    const float a = fabsf(row[start + i]);
    if (a > absmax) absmax = a;
  }
  sums[(size_t)t * groups + g] = total;
  const float scale = absmax > 1e-10f ? __fdiv_exact(absmax, 63.0f) : 1.0f;
  const float inv = __fdiv_exact(1.0f, scale);
  scales[(size_t)t * groups + g] = scale;
  for (int i = 0; i < len; ++i) {
    const float v = row[start + i] * inv;
    float r = (i < c8 * 8) ? rintf(v) : roundf(v);
    r = fminf(fmaxf(r, -63.0f), 63.0f);
    q[(size_t)t * n + start + i] = (int8_t)(int)r;
  }
}

// lm_head_chunk_i8 (gemm.rs:804-915): 8 lanes of 4 consecutive codes per
// 32-column chunk, scalar tail on the quantized hidden into lane 0.
__global__ void k_tied_head(float *__restrict__ logits, const uint8_t *__restrict__ codes,
                            const uint8_t *__restrict__ params, const int8_t *__restrict__ hq,
                            const float *__restrict__ hscales, const float *__restrict__ hsums,
                            int vocab, int n, int gs, int groups, int m) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (v >= vocab || t >= m) return;
  const uint8_t *row = codes + (size_t)v * n;
  const uint8_t *prow = params + (size_t)v * groups * 4;
  const int8_t *h = hq + (size_t)t * n;
  float zc = 0.0f;
  for (int g = 0; g < groups; ++g) {
    const float wz = f16bits((uint16_t)(prow[g * 4 + 2] | (prow[g * 4 + 3] << 8)));
    zc = zc + wz * hsums[(size_t)t * groups + g];
  }
  float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int g = 0; g < groups; ++g) {
    const float ws = f16bits((uint16_t)(prow[g * 4] | (prow[g * 4 + 1] << 8)));
    const float hs = hscales[(size_t)t * groups + g];
    const int col0 = g * gs, ags = min(gs, n - col0), c32 = ags / 32;
    int s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < c32; ++c)
      for (int l = 0; l < 8; ++l)
        for (int j = 0; j < 4; ++j) {
          const int col = col0 + 32 * c + 4 * l + j;
          s[l] += (int)row[col] * (int)h[col];
        }
    const float cs = ws * hs;
    for (int l = 0; l < 8; ++l) f[l] = f[l] + (float)s[l] * cs;
    if (c32 * 32 < ags) {
      float tail = 0.0f;
      for (int i = c32 * 32; i < ags; ++i) tail = tail + (float)row[col0 + i] * (float)h[col0 + i];
      f[0] = f[0] + (ws * hs) * tail;
    }
  }
  logits[(size_t)t * vocab + v] = hsum8(f) + zc;
}

// --------------------------------------------------------------- embed --

// embed_lookup (gemm.rs:1926-1970): out = fl(fl(code*scale) + zero), then
// *embed_scale when it is not 1.  Grid (m, ceil(hidden / 256)).
__global__ void k_embed(const uint32_t *__restrict__ tokens, const uint32_t *__restrict__ ctx,
                        int last, int start, const uint8_t *__restrict__ codes,
                        const uint8_t *__restrict__ params, int vocab, int hidden, int egs,
                        int egroups, float embed_scale, float *__restrict__ out, int *err,
                        const int *__restrict__ st) {
  const int t = blockIdx.x;
  if (st) {  // device step record {pos0, len, start, nd}
    last = st[1] - 1;
    start = st[2];
  }
  const int c = blockIdx.y * blockDim.x + threadIdx.x;
  uint32_t tok = tokens ? tokens[t] : (t == 0 ? ctx[last] : ctx[start + t - 1]);
  if (c >= hidden) return;
  float *o = out + (size_t)t * hidden;
  if (tok >= (uint32_t)vocab) {
    if (c == 0) atomicExch(err, 1);
    o[c] = 0.0f;
    return;
  }
  const uint8_t *row = codes + (size_t)tok * hidden;
  const uint8_t *prow = params + ((size_t)tok * egroups + c / egs) * 4;
  const float sc = f16bits((uint16_t)(prow[0] | (prow[1] << 8)));
  const float z = f16bits((uint16_t)(prow[2] | (prow[3] << 8)));
  float v = (float)row[c] * sc + z;
  if (embed_scale != 1.0f) v = v * embed_scale;
  o[c] = v;
}

// vec_add (layers.rs:503-531): h = r + a; h may alias r.
__global__ void k_vec_add(float *h, const float *r, const float *__restrict__ a, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) h[i] = r[i] + a[i];
}

// silu_mul_avx2 (layers.rs:850-883) per token row of n.
__global__ void k_silu_mul(float *__restrict__ gate, const float *__restrict__ up, int m, int n) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n || t >= m) return;
  const size_t idx = (size_t)t * n + i;
  const float x = gate[idx];
  float r;
  if (i < (n / 8) * 8) {
    const float e = rai_exact::schraudolph(x * -1.0f);
    r = __fdiv_exact(x, 1.0f + e) * up[idx];
  } else {
    r = __fdiv_exact(x, 1.0f + rai_exact::expf_glibc(-x)) * up[idx];
  }
  gate[idx] = r;
}

// RoPETable::apply_avx2 (layers.rs:689-726) for q and k, then the KV store
// (kv_cache.rs:143-172).  One thread per (token, head, pair i): rotates
// (i, i + hd/2) of a q or k head; k threads also store the rotated pair and
// the matching v pair in the cache.  Grid (m, ceil((nh + nkv) * hd/2 / 256)).
__global__ void k_rope_store(float *__restrict__ q, float *__restrict__ k,
                             const float *__restrict__ v, const float *__restrict__ cos_t,
                             const float *__restrict__ sin_t, int pos0, int nh, int nkv, int hd,
                             float *__restrict__ kc, float *__restrict__ vc, int cap,
                             int vstride, int q_ld, int kv_ld, const int *__restrict__ st) {
  const int t = blockIdx.x;
  if (st) pos0 = st[0];
  const int pos = pos0 + t;
  const int half = hd / 2;
  const int body = (half / 8) * 8;
  const int idx = blockIdx.y * blockDim.x + threadIdx.x;
  if (idx >= (nh + nkv) * half) return;
  const int h = idx / half, i = idx - h * half;
  const bool isq = h < nh;
  const int kh = h - nh;
  float *b = isq ? q + (size_t)t * q_ld + (size_t)h * hd : k + (size_t)t * kv_ld + (size_t)kh * hd;
  const float x0 = b[i], x1 = b[half + i];
  const float c = cos_t[(size_t)pos * half + i], sn = sin_t[(size_t)pos * half + i];
  float r0, r1;
  if (i < body) {
    r0 = __fmaf_rn(x0, c, -(x1 * sn));
    r1 = __fmaf_rn(x1, c, x0 * sn);
  } else {
    r0 = x0 * c - x1 * sn;
    r1 = x1 * c + x0 * sn;
  }
  b[i] = r0;
  b[half + i] = r1;
  if (!isq) {
    const size_t dst = ((size_t)kh * cap + pos) * hd;
    kc[dst + i] = r0;
    kc[dst + half + i] = r1;
    const float *vr = v + (size_t)t * kv_ld + (size_t)kh * hd;
    float *vd = vc + (size_t)kh * hd * vstride + pos;  // d-major V
    vd[(size_t)i * vstride] = vr[i];
    vd[(size_t)(half + i) * vstride] = vr[half + i];
  }
}

__global__ void k_rope_apply(float *__restrict__ heads, int nh, int hd,
                             const float *__restrict__ cr, const float *__restrict__ sr) {
  const int half = hd / 2;
  const int body = (half / 8) * 8;
  for (int idx = threadIdx.x; idx < nh * half; idx += blockDim.x) {
    const int h = idx / half, i = idx % half;
    float *b = heads + (size_t)h * hd;
    const float x0 = b[i], x1 = b[half + i], c = cr[i], s = sr[i];
    if (i < body) {
      b[i] = __fmaf_rn(x0, c, -(x1 * s));
      b[half + i] = __fmaf_rn(x1, c, x0 * s);
    } else {
      b[i] = x0 * c - x1 * s;
      b[half + i] = x1 * c + x0 * s;
    }
  }
}

// -------------------------------------------------------------- argmax --

__device__ __forceinline__ long long argmax_key(float f, int idx) {
  if (f != f) f = -INFINITY;  // sampler.rs:55-59 NaN -> -inf
  int32_t b = (int32_t)__float_as_uint(f);
  b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);  // f32::total_cmp ordering
  return ((long long)b << 32) | (long long)(uint32_t)idx;
}

// sampler.rs:201-208: max by total_cmp, the last maximal index wins (the
// key puts the index in the low bits, so the larger index wins a tie).
// One 1024-thread block per token.
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ logits, int vocab,
                                                 uint32_t *__restrict__ out) {
  const int t = blockIdx.x;
  const float *row = logits + (size_t)t * vocab;
  long long best = LLONG_MIN;
  for (int base = 0; base < vocab; base += 8 * (int)blockDim.x) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * (int)blockDim.x + (int)threadIdx.x;
      v[u] = i < vocab ? row[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * (int)blockDim.x + (int)threadIdx.x;
      if (i < vocab) {
        const long long k = argmax_key(v[u], i);
        best = k > best ? k : best;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const long long other = __shfl_xor(best, o, 64);
    best = other > best ? other : best;
  }
  __shared__ long long red[16];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    long long b = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = red[w] > b ? red[w] : b;
    out[t] = (uint32_t)(b & 0xFFFFFFFFll);
  }
}

// ------------------------------------------------------- n-gram search --

// find_ngram_draft (lookup.rs:131-171): for n = hi..lo, the largest start
// <= len-n-1 whose n tokens equal the suffix; draft = min(max_draft,
// len-start-n) tokens after it.  One 1024-thread block.
__device__ __forceinline__ void ngram_search(const uint32_t *__restrict__ ctx, int len, int min_n, int max_n,
                                             int max_draft, int *__restrict__ res) {
  __shared__ int best;
  __shared__ int done;
  if (threadIdx.x == 0) {
    done = 0;
    res[0] = 0;
    res[1] = 0;
    res[2] = 0;
  }
  __syncthreads();
  if (max_draft <= 0 || len < 2) return;
  const int hi = min(max_n, len - 1);
  const int lo = max(min_n, 1);
  for (int n = hi; n >= lo; --n) {
    if (threadIdx.x == 0) best = -1;
    __syncthreads();
    const uint32_t *suf = ctx + len - n;
    for (int s = threadIdx.x; s <= len - n - 1; s += blockDim.x) {
      bool eq = true;
      for (int i = 0; i < n && eq; ++i) eq = ctx[s + i] == suf[i];
      if (eq) atomicMax(&best, s);
    }
    __syncthreads();
    if (threadIdx.x == 0 && best >= 0) {
      const int ds = best + n;
      const int dl = min(max_draft, len - ds);
      if (dl > 0) {
        res[0] = n;
        res[1] = ds;
        res[2] = dl;
        done = 1;
      }
    }
    __syncthreads();
    if (done) return;
  }
}

__global__ void k_ngram(const uint32_t *__restrict__ ctx, int len, int min_n, int max_n,
                        int max_draft, int *__restrict__ res) {
  ngram_search(ctx, len, min_n, max_n, max_draft, res);
}

// The next decoder step's search, run at the end of a step: the context
// then holds this step's `produced` = res_acc[1] tokens past len, and the
// next step's position is pos + produced, so its draft is capped at
// max_ctx - (pos + produced) - 1 tokens (none when that is not positive).
// With a step record, pos, len and the search parameters come from it
// (st[0], st[1], st[5..7]).
__global__ void k_ngram_next(const uint32_t *__restrict__ ctx, int len, int pos, int min_n, int max_n,
                             int max_draft, int max_ctx, const int *__restrict__ res_acc, int *__restrict__ res,
                             const int *__restrict__ st) {
  if (st) {
    pos = st[0];
    len = st[1];
    min_n = st[5];
    max_n = st[6];
    max_draft = st[7];
  }
  const int produced = res_acc[1];
  const int budget = max_ctx - (pos + produced) - 1;
  ngram_search(ctx, len + produced, min_n, max_n, budget > 0 ? min(max_draft, budget) : 0, res);
}

// Greedy acceptance (the T -> 0 limit of lookup.rs:359-403).
__global__ void k_accept(const uint32_t *__restrict__ am, uint32_t *__restrict__ ctx, int len,
                         int start, int nd, int *__restrict__ res, const int *__restrict__ st) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  if (st) {
    len = st[1];
    start = st[2];
    nd = st[3];
  }
  int acc = 0, prod = 0;
  for (int i = 0; i < nd; ++i) {
    const uint32_t a = am[i];
    ctx[len + prod++] = a;
    if (a != ctx[start + i]) break;
    ++acc;
  }
  if (acc == nd) ctx[len + prod++] = am[nd];
  res[0] = acc;
  res[1] = prod;
}

// --------------------------------------------------------------- MoE --

// Router logits: block (token t, experts e0 .. e0 + 7), 256 threads.  The
// block computes the products fl(router[e][i] * x[i]) of a 256-column tile
// for its experts into LDS (coalesced row reads, issued a tile ahead; rows
// padded to 9 floats against bank conflicts); lane e adds its expert's
// products in column order.  logits[t][e] = the sequential dot from -0.0.
constexpr int kRouterEpb = 8, kRouterCols = 256, kRouterThreads = 256;
__global__ __launch_bounds__(kRouterThreads) void k_router_logits(const float *__restrict__ x,
                                                                  const float *__restrict__ router, int hidden,
                                                                  int experts, float *__restrict__ logits) {
  constexpr int EP = kRouterEpb + 1, TC = kRouterCols;
  constexpr int RI = kRouterEpb * TC / kRouterThreads;  // items per thread and tile
  __shared__ float tiles[2][TC * EP];
  const int t = blockIdx.x, e0 = blockIdx.y * kRouterEpb;
  const int ne = min(kRouterEpb, experts - e0);
  const float *xr = x + (size_t)t * hidden;
  const int tid = threadIdx.x;
  const int ntile = (hidden + TC - 1) / TC;
  // Item i = u * 256 + tid: expert i / TC, column i % TC (consecutive
  // threads read consecutive columns of one row).
  auto load = [&](int tl, float (&r)[RI], float (&xv)[RI]) {
#pragma unroll
    for (int u = 0; u < RI; ++u) {
      const int i = u * kRouterThreads + tid;
      const int e = i / TC, col = tl * TC + i % TC;
      const bool ok = e < ne && col < hidden && tl < ntile;
      r[u] = ok ? router[(size_t)(e0 + e) * hidden + col] : 0.0f;
      xv[u] = ok ? xr[col] : 0.0f;
    }
  };
  float s = -0.0f;
  auto step = [&](int tl, float (&r)[RI], float (&xv)[RI]) {
    float *cur = tiles[tl & 1];
#pragma unroll
    for (int u = 0; u < RI; ++u) {
      const int i = u * kRouterThreads + tid;
      cur[(i % TC) * EP + i / TC] = r[u] * xv[u];
    }
    load(tl + 2, r, xv);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (tid < ne) {
      const int cn = min(TC, hidden - tl * TC);
      int c = 0;
      for (; c + 8 <= cn; c += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = cur[(c + k) * EP + tid];
#pragma unroll
        for (int k = 0; k < 8; ++k) s = s + v[k];
      }
      for (; c < cn; ++c) s = s + cur[c * EP + tid];
    }
  };
  float ra[RI], rb[RI], xa[RI], xb[RI];
  load(0, ra, xa);
  load(1, rb, xb);
  for (int tl = 0; tl < ntile; tl += 2) {
    step(tl, ra, xa);
    if (tl + 1 < ntile) step(tl + 1, rb, xb);
  }
  if (tid < ne) logits[(size_t)t * experts + e0 + tid] = s;
}

// Router logits with the chains in registers, for hidden = 16 S: one wave
// per (token, 4 experts); the 16 lanes of DPP row c hold expert e0 + c's
// chain, lane q of the row the products fl(router[e][i] * x[i]) of columns
// [S q, S q + S) in registers.  Phase q adds every lane's S products in
// column order (only lane q of each row carries the live chain), then DPP
// row_shr:1 moves each chain to lane q + 1 of its row, so the dot from -0.0
// is one sequence of dependent adds with no memory access between them;
// lane 15 of each row ends with its expert's logit.
// One wave's four chains: expert e (lane row c = lane / 16) of token t;
// returns the logit on lane 15 of each row.
template <int S>
__device__ __forceinline__ float router_chain_r(const float *__restrict__ x, const float *__restrict__ router, int t,
                                                int e) {
  constexpr int hidden = 16 * S;
  const int q = threadIdx.x & 15;
  const float4 *rr = reinterpret_cast<const float4 *>(router + (size_t)e * hidden + S * q);
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)t * hidden + S * q);
  float p[S];
#pragma unroll
  for (int k = 0; k < S / 32; ++k) {
    float4 rv[8], xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      rv[u] = rr[8 * k + u];
      xv[u] = xr[8 * k + u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      p[32 * k + 4 * u] = rv[u].x * xv[u].x;
      p[32 * k + 4 * u + 1] = rv[u].y * xv[u].y;
      p[32 * k + 4 * u + 2] = rv[u].z * xv[u].z;
      p[32 * k + 4 * u + 3] = rv[u].w * xv[u].w;
    }
  }
  float acc = -0.0f;
#pragma unroll 1
  for (int ph = 0; ph < 16; ++ph) {
#pragma unroll
    for (int i = 0; i < S; ++i) acc = acc + p[i];
    if (ph < 15) {
      const int ai = __float_as_int(acc);
      const float moved = __int_as_float(__builtin_amdgcn_update_dpp(ai, ai, 0x111, 0xF, 0xF, false));
      acc = q == ph + 1 ? moved : acc;
    }
  }
  return acc;
}

template <int S>
__global__ __launch_bounds__(64) void k_router_logits_r(const float *__restrict__ x,
                                                        const float *__restrict__ router, int experts,
                                                        float *__restrict__ logits) {
  const int t = blockIdx.x, lane = threadIdx.x, c = lane >> 4;
  const int e = min((int)blockIdx.y * 4 + c, experts - 1);
  const float acc = router_chain_r<S>(x, router, t, e);
  if ((lane & 15) == 15 && (int)blockIdx.y * 4 + c < experts) logits[(size_t)t * experts + blockIdx.y * 4 + c] = acc;
}

// route_experts for at most 64 experts, one wave per token, expert e on
// lane e: the maximum by DPP moves, glibc expf, the sum as one chain in
// expert order (lane reads), the division; then each top-k pick is the
// wave maximum over the untaken finite probabilities and the lowest lane
// holding it (a ballot), which is k_router's strict-> scan with the lowest
// index winning a tie; NaN probabilities are never picked.
__device__ __forceinline__ void route64_wave(float lg_in, int t, int experts, int topk, int norm_topk,
                                             int *__restrict__ sel, float *__restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const bool live = lane < experts;
  const float lg = live ? lg_in : -INFINITY;
  const float mx = wave_max_dpp(lg);
  const float ex = live ? rai_exact::expf_glibc(lg - mx) : 0.0f;
  const int exi = __float_as_int(ex);
  float sum = 0.0f;
  for (int e = 0; e < experts; ++e) sum = sum + __int_as_float(__builtin_amdgcn_readlane(exi, e));
  const float pr = __fdiv_exact(ex, sum);
  bool taken = false;
  float total = -0.0f;
  int cnt = 0;
  for (int k = 0; k < topk; ++k) {
    const float v = (live && !taken && pr > -INFINITY) ? pr : -INFINITY;
    const float bv = wave_max_dpp(v);
    if (!(bv > -INFINITY)) break;
    const uint64_t hit = __ballot(v == bv && v > -INFINITY);
    const int best = __ffsll((unsigned long long)hit) - 1;
    if (lane == best) taken = true;
    if (lane == 0) {
      sel[t * topk + cnt] = best;
      wts[t * topk + cnt] = bv;
    }
    total = total + bv;
    ++cnt;
  }
  if (lane == 0) {
    for (int k = cnt; k < topk; ++k) {
      sel[t * topk + k] = -1;
      wts[t * topk + k] = 0.0f;
    }
    if (norm_topk && total > 0.0f)
      for (int k = 0; k < cnt; ++k) wts[t * topk + k] = __fdiv_exact(wts[t * topk + k], total);
  }
}

__global__ __launch_bounds__(64) void k_router64(const float *__restrict__ logits, int experts, int topk,
                                                 int norm_topk, int *__restrict__ sel, float *__restrict__ wts) {
  const int t = blockIdx.x, lane = threadIdx.x;
  route64_wave(lane < experts ? logits[(size_t)t * experts + lane] : 0.0f, t, experts, topk, norm_topk, sel, wts);
}

// route_experts (layers.rs:1808-1870) after the logits: softmax over all
// experts (glibc expf, the sum as one chain in expert order), then top-k by
// selection (strict >, so the lowest index wins a tie), optional
// renormalisation.  One block per token.
__global__ __launch_bounds__(1024) void k_router(const float *__restrict__ logits, int experts, int topk,
                                                 int norm_topk, int *__restrict__ sel, float *__restrict__ wts) {
  extern __shared__ float probs[];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int e = tid; e < experts; e += nt) probs[e] = logits[(size_t)t * experts + e];
  __syncthreads();
  // Softmax over every expert: max and exponentials in parallel, the sum as
  // one chain in expert order, then the division.
  __shared__ float smx, ssum;
  if (tid < 64) {
    float mx = -INFINITY;
    for (int e = tid; e < experts; e += 64) mx = fmaxf(mx, probs[e]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (tid == 0) smx = mx;
  }
  __syncthreads();
  for (int e = tid; e < experts; e += nt) probs[e] = rai_exact::expf_glibc(probs[e] - smx);
  __syncthreads();
  if (tid == 0) {
    float sum = 0.0f;
    for (int e = 0; e < experts; ++e) sum = sum + probs[e];
    ssum = sum;
  }
  __syncthreads();
  for (int e = tid; e < experts; e += nt) probs[e] = __fdiv_exact(probs[e], ssum);
  __syncthreads();
  // Top-k by selection (strict >, so the lowest index wins a tie): lane l
  // scans experts l, l + 64, ...; a wave-wide argmax picks each slot.
  if (tid < 64) {
    const int lane = tid;
    uint32_t mine = 0;  // taken bits of experts lane + 64 j
    float total = -0.0f;
    int cnt = 0;
    for (int k = 0; k < topk; ++k) {
      float bv = -INFINITY;
      int best = -1;
      for (int j = 0, e = lane; e < experts; ++j, e += 64)
        if (!((mine >> j) & 1u) && probs[e] > bv) {
          bv = probs[e];
          best = e;
        }
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int ob = __shfl_xor(best, o, 64);
        if (ob >= 0 && (best < 0 || ov > bv || (ov == bv && ob < best))) {
          bv = ov;
          best = ob;
        }
      }
      if (best < 0) break;
      if (lane == (best & 63)) mine |= 1u << (best >> 6);
      if (lane == 0) {
        sel[t * topk + cnt] = best;
        wts[t * topk + cnt] = bv;
      }
      total = total + bv;
      ++cnt;
    }
    if (lane == 0) {
      for (int k = cnt; k < topk; ++k) {
        sel[t * topk + k] = -1;
        wts[t * topk + k] = 0.0f;
      }
      if (norm_topk && total > 0.0f)
        for (int k = 0; k < cnt; ++k) wts[t * topk + k] = __fdiv_exact(wts[t * topk + k], total);
    }
  }
}

__global__ void k_moe_acc(float *__restrict__ out, const float *__restrict__ eo,
                          const float *__restrict__ w, int m, int n) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n || t >= m) return;
  out[(size_t)t * n + i] = out[(size_t)t * n + i] + w[t] * eo[(size_t)t * n + i];
}

__global__ void k_fill(float *p, float v, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

// ------------------------------------------------------------ launchers --

void launch_quantize(const float *x, int m, int k, int gs, int8_t *q_nat, int8_t *q_split,
                     float *scales, float *sums, hipStream_t s) {
  const int groups = (k + gs - 1) / gs;
  dim3 grid((groups + 63) / 64, m);
  hipLaunchKernelGGL(k_quantize, grid, dim3(64), 0, s, x, m, k, gs, groups, q_nat,
                     (k % 8 == 0) ? q_split : nullptr, scales, sums);
}

bool w4a8_norm1_path(int rows, int cols, int gs) {
  return gs == 32 && rows > 0 && cols % 32 == 0 && cols / 32 <= 128 && cols >= 256;
}

bool launch_w4a8_norm1(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const float *x,
                       const float *norm_w, float eps, int rows, int cols, int gs, hipStream_t s) {
  if (!w4a8_norm1_path(rows, cols, gs)) return false;
  if (launch_w4a8_dec(out, add, nib, params, nullptr, nullptr, nullptr, rows, cols, gs, x, norm_w, eps, s)) return true;
  const int groups = cols / 32;
  // Same tiles as the unfused one-token dispatch in launch_w4a8.
  if (rows >= 16384)
    launch_small_t<32, 1, 16, 4, true>(out, add, nib, params, nullptr, nullptr, nullptr, rows, cols, 1, groups, s,
                                       x, norm_w, eps);
  else
    launch_m1_t<32, 8>(out, add, nib, params, nullptr, nullptr, nullptr, rows, cols, groups, s, x, norm_w, eps);
  return true;
}

bool w4a8_fast_path(int cols, int gs) {
  return (gs == 32 || gs == 64 || gs == 128) && cols % gs == 0;
}

void launch_w4a8(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const float *x,
                 const int8_t *q_nat, const int8_t *q_split, const float *scales,
                 const float *sums, int rows, int cols, int m, int gs, hipStream_t s,
                 const _Float16 *qa, uint8_t *mm, const uint8_t *params_tiled) {
  const int groups = (cols + gs - 1) / gs;
  if (launch_w4a8_mfma(out, add, nib, params, qa, q_split, scales, sums, rows, cols, m, gs, s, params_tiled)) return;
  if (mm && q_split && w4a8_mm_path(rows, cols, m, gs)) {
    launch_w4a8_mm(out, add, nib, params, q_split, scales, sums, rows, cols, m, mm, s);
    return;
  }
  if (m == 1 && q_split &&
      launch_w4a8_dec(out, add, nib, params, q_split, scales, sums, rows, cols, gs, nullptr, nullptr, 0.0f, s))
    return;
  // Decode (one token) at group 32, measured on the 7B shapes (4096..32000
  // rows, K 4096 / 14336): 16-row tiles for many rows, 8-row tiles for long
  // rows, 8-row whole-K blocks otherwise.
  if (gs == 32 && m == 1 && w4a8_fast_path(cols, gs)) {
    if (rows >= 16384) {
      launch_small_mt<32, 1, 16>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
      return;
    }
    if (cols >= 8192) {
      launch_small_mt<32, 1, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
      return;
    }
    if (8 * groups <= m1_items_per_thread(32) * kThreads) {
      launch_m1_t<32, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
      return;
    }
  }
  // The whole-K kernel wins where few, long rows leave the streaming kernel
  // with too few blocks (measured on 1024..32000 x 2048..14336, g32).
  if (w4a8_fast_path(cols, gs) && m == 1 && cols >= 4096 && rows <= cols) {
    bool done;
    if (gs == 32)
      done = launch_m1<32>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
    else if (gs == 64)
      done = launch_m1<64>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
    else
      done = launch_m1<128>(out, add, nib, params, q_split, scales, sums, rows, cols, groups, s);
    if (done) return;
  }
  if (w4a8_fast_path(cols, gs) && m <= 16) {
    if (gs == 32)
      launch_small_gs<32>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
    else if (gs == 64)
      launch_small_gs<64>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
    else
      launch_small_gs<128>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
    return;
  }
  if (w4a8_fast_path(cols, gs)) {
    if (gs == 32)
      launch_fast_gs<32>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
    else if (gs == 64)
      launch_fast_gs<64>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
    else
      launch_fast_gs<128>(out, add, nib, params, q_split, scales, sums, rows, cols, m, groups, s);
    return;
  }
  dim3 grid((rows + 127) / 128, m);
  hipLaunchKernelGGL(k_w4a8_simple, grid, dim3(128), 0, s, out, add, nib, params, x, q_nat, scales,
                     sums, rows, cols, m, gs, groups);
}

void launch_lane_sums(int32_t *out, const uint8_t *nib, const int8_t *q_nat, int rows, int cols,
                      int m, int gs, hipStream_t s) {
  const int groups = (cols + gs - 1) / gs;
  dim3 grid((rows * groups + 127) / 128, m);
  hipLaunchKernelGGL(k_lane_sums, grid, dim3(128), 0, s, out, nib, q_nat, rows, cols, m, gs,
                     groups);
}

void launch_tied_lm_head(float *logits, const float *hidden, const uint8_t *codes,
                         const uint8_t *params, int vocab, int n, int gs, int m, int8_t *hq,
                         float *hscales, float *hsums, hipStream_t s) {
  const int groups = (n + gs - 1) / gs;
  hipLaunchKernelGGL(k_quantize63, dim3((groups + 63) / 64, m), dim3(64), 0, s, hidden, m, n, gs,
                     groups, hq, hscales, hsums);
  hipLaunchKernelGGL(k_tied_head, dim3((vocab + 127) / 128, m), dim3(128), 0, s, logits, codes,
                     params, hq, hscales, hsums, vocab, n, gs, groups, m);
}

void launch_embed(const uint32_t *tokens, const uint32_t *ctx, int last, int start, int m,
                  const uint8_t *codes, const uint8_t *params, int vocab, int hidden, int egs,
                  float embed_scale, float *out, int *err, hipStream_t s, const int *st) {
  const int egroups = (hidden + egs - 1) / egs;
  hipLaunchKernelGGL(k_embed, dim3(m, (hidden + 255) / 256), dim3(256), 0, s, tokens, ctx, last, start, codes, params,
                     vocab, hidden, egs, egroups, embed_scale, out, err, st);
}

void launch_vec_add(float *h, const float *r, const float *a, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_vec_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, h, r, a, n);
}

void launch_silu_mul(float *gate, const float *up, int m, int n, hipStream_t s) {
  hipLaunchKernelGGL(k_silu_mul, dim3((n + 255) / 256, m), dim3(256), 0, s, gate, up, m, n);
}

void launch_rope_store(float *q, float *k, const float *v, const float *cos_t, const float *sin_t,
                       int pos0, int m, int nh, int nkv, int hd, float *kc, float *vc, int cap,
                       int vstride, int q_ld, int kv_ld, hipStream_t s, const int *st) {
  const int pairs = (nh + nkv) * (hd / 2);
  hipLaunchKernelGGL(k_rope_store, dim3(m, (pairs + 255) / 256), dim3(256), 0, s, q, k, v, cos_t, sin_t, pos0, nh, nkv,
                     hd, kc, vc, cap, vstride, q_ld, kv_ld, st);
}

void launch_rope_apply(float *heads, int nh, int hd, const float *cos_row, const float *sin_row,
                       hipStream_t s) {
  hipLaunchKernelGGL(k_rope_apply, dim3(1), dim3(256), 0, s, heads, nh, hd, cos_row, sin_row);
}

void launch_argmax(const float *logits, int m, int vocab, uint32_t *out, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax, dim3(m), dim3(1024), 0, s, logits, vocab, out);
}

void launch_ngram(const uint32_t *ctx, int len, int min_n, int max_n, int max_draft, int *res,
                  hipStream_t s) {
  hipLaunchKernelGGL(k_ngram, dim3(1), dim3(1024), 0, s, ctx, len, min_n, max_n, max_draft, res);
}

void launch_ngram_next(const uint32_t *ctx, int len, int pos, int min_n, int max_n, int max_draft, int max_ctx,
                       const int *res_acc, int *res, hipStream_t s, const int *st) {
  hipLaunchKernelGGL(k_ngram_next, dim3(1), dim3(1024), 0, s, ctx, len, pos, min_n, max_n, max_draft, max_ctx,
                     res_acc, res, st);
}

void launch_accept(const uint32_t *am, uint32_t *ctx, int len, int start, int nd, int *res2,
                   hipStream_t s, const int *st) {
  hipLaunchKernelGGL(k_accept, dim3(1), dim3(64), 0, s, am, ctx, len, start, nd, res2, st);
}

void launch_router(const float *x, const float *router, int m, int hidden, int experts, int topk,
                   int norm_topk, int *sel, float *wts, float *logits, hipStream_t s) {
  const dim3 g4(m, (experts + 3) / 4);
  if (hidden == 16 * 128)
    hipLaunchKernelGGL(k_router_logits_r<128>, g4, dim3(64), 0, s, x, router, experts, logits);
  else if (hidden == 16 * 64)
    hipLaunchKernelGGL(k_router_logits_r<64>, g4, dim3(64), 0, s, x, router, experts, logits);
  else if (hidden == 16 * 32)
    hipLaunchKernelGGL(k_router_logits_r<32>, g4, dim3(64), 0, s, x, router, experts, logits);
  else
    hipLaunchKernelGGL(k_router_logits, dim3(m, (experts + kRouterEpb - 1) / kRouterEpb), dim3(kRouterThreads), 0,
                       s, x, router, hidden, experts, logits);
  if (experts <= 64)
    hipLaunchKernelGGL(k_router64, dim3(m), dim3(64), 0, s, logits, experts, topk, norm_topk, sel, wts);
  else
    hipLaunchKernelGGL(k_router, dim3(m), dim3(1024), sizeof(float) * ((experts + 3) & ~3), s, logits, experts,
                       topk, norm_topk, sel, wts);
}

void launch_moe_accumulate(float *out, const float *eo, const float *w, int m, int n,
                           hipStream_t s) {
  hipLaunchKernelGGL(k_moe_acc, dim3((n + 255) / 256, m), dim3(256), 0, s, out, eo, w, m, n);
}

void launch_fill(float *p, float v, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_fill, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
}

}  // namespace rai
