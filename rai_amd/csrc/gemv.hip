// W4A8 GEMV for small token counts on the gfx950 matrix cores, group 32.
//
// The integer dot products S[row][token][block] (8 columns of one 32-column
// group, the reference's per-lane int8 x int4 sums, gemm.rs:458-525) come
// from v_mfma_f32_16x16x32_f16 with exact operands: weight codes 0..15 and
// int8 activations are exact in f16, every product and partial sum is an
// integer (or, for codes entered as subnormals, an integer times 2^-24)
// well inside the f32 significand, so the f32 accumulators hold S exactly
// whatever the summation order inside the instruction.
//
// MFMA operand roles (16x16x32): B = weights, column j = row of the weight
// tile (16 rows per wave); A = activations, block-diagonal, so that each of
// the 16 D rows collects one (token, 8-column block) partial sum: lane l
// (j = l % 16, h = l / 16) receives in its 4 accumulators the S values of
// row j and token h for 4 (group, block) pairs.  k_gemv_ms spans one group's
// 4 blocks per instruction, k_gemv_rs block b of 4 consecutive groups.
//
// Each lane then runs the reference epilogue for its (row, token) in group
// order: cs = fl(ws * as); f_b += fl(S_b * cs); zc += fl(wz * xsum), and at
// the end out = hsum8(f0..f3, 0, 0, 0, 0) + zc (gemm.rs:458-537).  The
// chains never leave the lane, so no products go through LDS.  That f32
// epilogue (11 VALU operations per row, token and group) rather than HBM
// bounds these kernels at 9 tokens.
//
// K order inside a block (8 columns c0..c7): f16 element e of the lane's 8
// is column (0, 4, 1, 5, 2, 6, 3, 7)[e].  The weight dword of a block holds
// column c in bits 4c..4c+3; masks 0x000F000F and 0x00F000F0 of the dword
// and of the dword shifted by 8 give columns (0, 4), (1, 5), (2, 6), (3, 7)
// as f16 pairs, the odd columns at 16 times their code.  The activation
// layout holds the odd columns divided by 16 (exact for int8 values), so
// every product is the exact code x activation.
//
// Activations for all three kernels are packed once per GEMV input
// (k_qa_pack4, or the quantizing kernels' matrix-core output) as
// qa4[tg][q][b][i = 4t + r][8] f16: token 4*tg + t, group 4*q + r, block b.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "kernels.h"

namespace rai {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float f16lo(uint32_t w) {
  return __half2float(__ushort_as_half((uint16_t)(w & 0xFFFF)));
}
__device__ __forceinline__ float f16hi(uint32_t w) {
  return __half2float(__ushort_as_half((uint16_t)(w >> 16)));
}

// Eight weight codes of one 8-column block (one dword: byte i = columns
// 2i (low nibble), 2i+1 (high nibble)) as exact f16 values in the K order
// (0, 4, 1, 5, 2, 6, 3, 7), odd columns times 16: 0x6400 | v is the f16
// 1024 + v (v <= 240), minus 1024.
__device__ __forceinline__ h8 unpack_codes(uint32_t w) {
  const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, o = 0x64006400u, t = w >> 8;
  const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2 e0 = __builtin_bit_cast(h2, (w & lo) | o) - bias;
  const h2 e1 = __builtin_bit_cast(h2, (w & hi) | o) - bias;
  const h2 e2 = __builtin_bit_cast(h2, (t & lo) | o) - bias;
  const h2 e3 = __builtin_bit_cast(h2, (t & hi) | o) - bias;
  h8 r;
  r[0] = e0[0];
  r[1] = e0[1];
  r[2] = e1[0];
  r[3] = e1[1];
  r[4] = e2[0];
  r[5] = e2[1];
  r[6] = e3[0];
  r[7] = e3[1];
  return r;
}

}  // namespace

// Block-staged version.  A block of WPB waves owns RB = 16*WPB weight rows
// and TGW token groups (4*TGW tokens); wave w computes rows 16w..16w+15.
// K runs in tiles of P groups.  All threads of the block cooperatively
// fetch the next tiles with 16-byte coalesced loads: weight codes (RB rows x
// P*16 B), params (RB x P dwords), activation A blocks (256 B per (token
// group, group)) and (scale, input sum) pairs.  Pipeline per iteration kt:
// issue the loads of tile kt+2 into one register set, compute tile kt from
// one half of the double-buffered LDS tiles, store tile kt+1 (loaded during
// iteration kt-1, in the other register set) into the other half, barrier.
// Every prefetch is unconditional (clamped to the last tile), so each load
// wait is static.  Requires groups % P == 0.
template <int TGW, int P, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_gemv_ms(
    float *out, const float *add, const uint8_t *__restrict__ nib, const uint8_t *__restrict__ params,
    const _Float16 *__restrict__ qa, const float *__restrict__ scales,
    const float *__restrict__ sums, int rows, int cols, int m) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int NT = 64 * WPB;             // threads
  constexpr int RB = 16 * WPB;             // rows per block
  constexpr int WSTR = 4 * P + 4;          // LDS row stride of the codes (dwords)
  constexpr int PSTR = P + 1;              // LDS row stride of the params (dwords)
  constexpr int NW4 = RB * P / NT;         // code float4 per thread per tile
  constexpr int NP4 = (RB * P / 4 + NT - 1) / NT;   // param float4 per thread
  constexpr int NA4 = (TGW * P * 16 + NT - 1) / NT; // activation float4 per thread
  static_assert(NW4 * NT == RB * P, "code tile must split evenly");
  __shared__ __align__(16) uint32_t lw[2][RB * WSTR];
  __shared__ uint32_t lp[2][RB * PSTR];
  // 17 slots of 8 halves per (tg, group): slots 0..15 hold the A rows,
  // slot 16 stays zero and feeds the lanes whose A block is zero.
  __shared__ __align__(16) _Float16 la[2][TGW][P][17 * 8];
  __shared__ __align__(16) float ls[2][TGW * 4][P][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int tgc = blockIdx.y;
  const int brow0 = blockIdx.x * RB;
  const int groups = cols / 32;
  const int ntiles = groups / P;
  const int last = ntiles - 1;
  const int j = lane & 15, h = lane >> 4;
  const int aslot = ((j & 3) == h) ? j : 16;
  for (int i = tid; i < 2 * TGW * P; i += NT)
    reinterpret_cast<f4 *>(&la[0][0][0][0])[i * 17 + 16] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  // Scale pairs (token, group), NS per thread; entries past TGW*4*P load a
  // clamped duplicate (every load is unconditional) and store nothing.
  constexpr int NSP = TGW * 4 * P;
  constexpr int NS = (NSP + NT - 1) / NT;
  // Raw code/param/activation bits travel as integers (never as floats,
  // which an arithmetic-free move could still canonicalize).
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  struct Stage {
    u4 w[NW4];
    u4 p[NP4];
    u4 a[NA4];
    float s0[NS], s1[NS];
  };
  int st_t[NS], st_g[NS], st_tok[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int i = min(tid + NT * u, NSP - 1);
    st_t[u] = i / P;
    st_g[u] = i % P;
    st_tok[u] = min(tgc * TGW * 4 + st_t[u], m - 1);
  }
  auto load = [&](Stage &S, int kt) {
#pragma unroll
    for (int u = 0; u < NW4; ++u) {
      const int i = tid + NT * u;
      const int r = min(brow0 + i / P, rows - 1), c = i % P;
      S.w[u] = *reinterpret_cast<const u4 *>(nib + (size_t)r * (cols / 2) + (size_t)(kt * P + c) * 16);
    }
#pragma unroll
    for (int u = 0; u < NP4; ++u) {
      const int i = min(tid + NT * u, RB * P / 4 - 1);
      const int r = min(brow0 + i / (P / 4), rows - 1), c4 = i % (P / 4);
      S.p[u] = *reinterpret_cast<const u4 *>(params + ((size_t)r * groups + kt * P + 4 * c4) * 4);
    }
#pragma unroll
    for (int u = 0; u < NA4; ++u) {
      const int i = min(tid + NT * u, TGW * P * 16 - 1);
      const int tg = i / (P * 16), k = i % (P * 16);
      // A row (slot) 4t + b of group p sits at qa4[tg][p / 4][b][4t + p % 4].
      const int p = kt * P + k / 16, t = (k & 15) >> 2, b = k & 3;
      S.a[u] = reinterpret_cast<const u4 *>(qa)[(((size_t)(tgc * TGW + tg) * (groups / 4) + p / 4) * 4 + b) * 16 +
                                                4 * t + (p & 3)];
    }
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      S.s0[u] = scales[(size_t)st_tok[u] * groups + kt * P + st_g[u]];
      S.s1[u] = sums[(size_t)st_tok[u] * groups + kt * P + st_g[u]];
    }
  };
  auto store = [&](const Stage &S, int b) {
#pragma unroll
    for (int u = 0; u < NW4; ++u) {
      const int i = tid + NT * u;
      *reinterpret_cast<u4 *>(&lw[b][(i / P) * WSTR + 4 * (i % P)]) = S.w[u];
    }
#pragma unroll
    for (int u = 0; u < NP4; ++u) {
      const int i = tid + NT * u;
      if (i < RB * P / 4) {
        uint32_t *d = &lp[b][(i / (P / 4)) * PSTR + 4 * (i % (P / 4))];
        d[0] = S.p[u].x;
        d[1] = S.p[u].y;
        d[2] = S.p[u].z;
        d[3] = S.p[u].w;
      }
    }
#pragma unroll
    for (int u = 0; u < NA4; ++u) {
      const int i = tid + NT * u;
      if (i < TGW * P * 16) {
        const int tg = i / (P * 16), k = i % (P * 16);
        reinterpret_cast<u4 *>(&la[b][tg][0][0])[(k / 16) * 17 + k % 16] = S.a[u];
      }
    }
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (tid + NT * u < NSP) {
        ls[b][st_t[u]][st_g[u]][0] = S.s0[u];
        ls[b][st_t[u]][st_g[u]][1] = S.s1[u];
      }
  };

  float f[TGW][4], zc[TGW];
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
    f[tg][0] = f[tg][1] = f[tg][2] = f[tg][3] = 0.0f;
    zc[tg] = 0.0f;
  }
  const int wr = 16 * wave + j;  // this lane's row within the block tile
  auto compute = [&](int b) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint32_t wd = lw[b][wr * WSTR + 4 * p + h];
      const uint32_t pw = lp[b][wr * PSTR + p];
      const h8 bq = unpack_codes(wd);
      const float ws = f16lo(pw), wz = f16hi(pw);
#pragma unroll
      for (int tg = 0; tg < TGW; ++tg) {
        const h8 a = *reinterpret_cast<const h8 *>(&la[b][tg][p][aslot * 8]);
        const float2 sx = *reinterpret_cast<const float2 *>(&ls[b][tg * 4 + h][p][0]);
        const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
        const f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq, zero4, 0, 0, 0);
        const float cs = ws * sx.x;
        f[tg][0] = f[tg][0] + d[0] * cs;
        f[tg][1] = f[tg][1] + d[1] * cs;
        f[tg][2] = f[tg][2] + d[2] * cs;
        f[tg][3] = f[tg][3] + d[3] * cs;
        zc[tg] = zc[tg] + wz * sx.y;
      }
      if (p & 1) __builtin_amdgcn_sched_barrier(0);
    }
  };

  Stage S0, S1;
  load(S0, 0);
  load(S1, min(1, last));
  store(S0, 0);
  __syncthreads();
  int kt = 0;
#define RAI_GEMV_STEP(Snext, Sready)          \
  {                                           \
    load(Snext, min(kt + 2, last));           \
    __builtin_amdgcn_sched_barrier(0);        \
    compute(kt & 1);                          \
    store(Sready, (kt + 1) & 1);              \
    __syncthreads();                          \
    if (++kt >= ntiles) break;                \
  }
  for (;;) {
    RAI_GEMV_STEP(S0, S1)
    RAI_GEMV_STEP(S1, S0)
  }
#undef RAI_GEMV_STEP
  const int row = brow0 + wr;
  if (row < rows) {
#pragma unroll
    for (int tg = 0; tg < TGW; ++tg) {
      const int t = (tgc * TGW + tg) * 4 + h;
      if (t < m) {
        const size_t oi = (size_t)t * rows + row;
        const float v = ((f[tg][0] + f[tg][1]) + (f[tg][2] + f[tg][3])) + zc[tg];
        out[oi] = add ? add[oi] + v : v;
      }
    }
  }
}

// Activations in the matrix-core A layout:
// qa4[tg][q][b][i = 4t + r][8] f16 = token 4*tg + t, group 4*q + r, block b
// in the K order above, odd columns divided by 16 (zeros for tokens past m).
// One thread per (tg, q, b, i).  Requires groups % 4 == 0.
__global__ void k_qa_pack4(const int8_t *__restrict__ q_split, int m, int cols, int ntg,
                           _Float16 *__restrict__ qa) {
  const int groups = cols / 32, nq = groups / 4;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // over ntg*nq*64
  if (idx >= ntg * nq * 64) return;
  const int i = idx & 15, b = (idx >> 4) & 3, qq = (idx >> 6) % nq, tg = (idx >> 6) / nq;
  const int t = 4 * tg + (i >> 2), g = 4 * qq + (i & 3);
  _Float16 *dst = qa + (size_t)idx * 8;
  if (t >= m) {
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e] = (_Float16)0.0f;
    return;
  }
  const int8_t *src = q_split + (size_t)t * cols + g * 32 + 8 * b;
  const int col_of_e[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = col_of_e[e];
    const int sidx = (c & 1) ? 4 + (c >> 1) : (c >> 1);
    const float v = (float)src[sidx];
    dst[e] = (_Float16)((c & 1) ? v * 0.0625f : v);
  }
}

// Register-streamed version.  MFMA K = 32 covers block b of four
// consecutive groups 4q..4q+3: B lane (j, h) = row j's codes of group
// 4q + h, block b (one dword of the 16-byte group it loads); A row
// i = 4t + r is token t's block b of group 4q + r, nonzero only on K block
// r.  Lane (j, h) then holds D[4h + r][j] = S[row j][token h][group 4q+r]
// [block b], so after the four blocks it owns the four lane chains of
// (row j, token h) for four groups, which it accumulates in group order.
//
// Each lane streams its own weight bytes (16 B of codes and 16 B of params
// per step of four groups) through a register ring NQ steps deep; the
// first NQ steps of the loop only fill the ring (through the same code, so
// the loop starts with nothing in flight and every load wait stays
// static).  The block's activations, scales and input sums go through LDS
// in chunks of NQ steps, double-buffered: chunk c + 1 is loaded into
// registers while chunk c is computed and stored behind it, with one barrier
// per chunk.
//
// Codes enter the MFMA either as f16 subnormals v * 2^-24 (SUB: one mask
// per pair, v = n or 16 n; D = S * 2^-24 exactly, products and partial sums
// being multiples of 2^-24 below 2^-10) with the weight scale taken as
// ws * 2^24,
// or as 1024 + n minus 1024 (D = S).  fl(D * fl(ws*2^24 * as)) equals
// fl(S * fl(ws * as)) whenever |ws * as| < 2^104 (power-of-two scaling
// commutes with rounding in the normal range, and ws * as is zero or at
// least 2^-24 * 1e-10 / 127), which holds when every activation scale is
// below 2^88 since |ws| <= 65504.  A chunk whose staged scales include a
// larger finite value is computed in the 1024 + n form.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h8 unpack_codes_sub(uint32_t w) {
  const uint32_t lo = 0x000F000Fu, hi = 0x00F000F0u, t = w >> 8;
  const u32x4 d = {w & lo, w & hi, t & lo, t & hi};
  return __builtin_bit_cast(h8, d);
}

// NQ steps of the main loop on one staged chunk (LDS buffer at la_c, lsc_c,
// lsu_c); steps q < 0 or q >= nq only refill the ring.
template <int TGW, bool SUB>
__device__ __forceinline__ void gemv_rs_step(
    const u32x4 &rc, const u32x4 &rp, int s, int NQ, const u32x4 *__restrict__ la_c,
    const f32x4 *__restrict__ lsc_c, const f32x4 *__restrict__ lsu_c, int h, float (&f)[TGW][4],
    float (&zc)[TGW]) {
  typedef f32x4 f4;
  const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 D[TGW][4], as4[TGW], xs4[TGW];
  float ws[4], wz[4];
  u32x4 av[TGW][4];
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
    const int base = (tg * NQ + s) * 4;
#pragma unroll
    for (int b = 0; b < 4; ++b) av[tg][b] = la_c[(base + b) * 17];
    as4[tg] = lsc_c[base + h];
    xs4[tg] = lsu_c[base + h];
  }
  h8 bq[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) bq[b] = SUB ? unpack_codes_sub(rc[b]) : unpack_codes(rc[b]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    ws[r] = SUB ? f16lo(rp[r]) * 16777216.0f : f16lo(rp[r]);
    wz[r] = f16hi(rp[r]);
  }
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
      D[tg][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, av[tg][b]), bq[b], zero4, 0, 0, 0);
  }
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cs = ws[r] * as4[tg][r];
      f[tg][0] = f[tg][0] + D[tg][0][r] * cs;
      f[tg][1] = f[tg][1] + D[tg][1][r] * cs;
      f[tg][2] = f[tg][2] + D[tg][2][r] * cs;
      f[tg][3] = f[tg][3] + D[tg][3][r] * cs;
      zc[tg] = zc[tg] + wz[r] * xs4[tg][r];
    }
  }
}

// NQ steps of the main loop on one staged chunk (LDS buffer at la_c, lsc_c,
// lsu_c); steps q < 0 or q >= nq only refill the ring.  The compute branch
// holds no memory loads, so every load wait stays static.
template <int TGW, int NQ>
__device__ __forceinline__ void gemv_rs_steps(
    int q0, bool huge, u32x4 (&rc)[NQ], u32x4 (&rp)[NQ], const u32x4 *__restrict__ cptr,
    const u32x4 *__restrict__ pptr, const u32x4 *__restrict__ la_c, const f32x4 *__restrict__ lsc_c,
    const f32x4 *__restrict__ lsu_c, int nq, int h, float (&f)[TGW][4], float (&zc)[TGW]) {
#pragma unroll
  for (int s = 0; s < NQ; ++s) {
    const int q = q0 + s;
    if (q >= 0 && q < nq) {
      if (huge)
        gemv_rs_step<TGW, false>(rc[s], rp[s], s, NQ, la_c, lsc_c, lsu_c, h, f, zc);
      else
        gemv_rs_step<TGW, true>(rc[s], rp[s], s, NQ, la_c, lsc_c, lsu_c, h, f, zc);
    }
    const int qn = min(q + NQ, nq - 1);
    rc[s] = cptr[4 * qn];
    rp[s] = pptr[qn];
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int TGW, int NQ, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_gemv_rs(
    float *out, const float *add, const uint8_t *__restrict__ nib, const uint8_t *__restrict__ params,
    const _Float16 *__restrict__ qa, const float *__restrict__ scales,
    const float *__restrict__ sums, int rows, int cols, int m, int ntg) {
  typedef u32x4 u4;
  typedef f32x4 f4;
  constexpr int NT = 64 * WPB;
  constexpr int AU = TGW * NQ * 64;       // A u4 per chunk
  constexpr int SU = TGW * NQ * 4;        // scale / sum f4 per chunk
  constexpr int NA = (AU + NT - 1) / NT;  // per thread
  constexpr int NS = (SU + NT - 1) / NT;
  constexpr int ABUF = TGW * NQ * 68;     // u4 per A buffer, 17 slots per block
  extern __shared__ __align__(16) unsigned char smem[];
  // LDS: A [2][TGW][NQ][4 blocks][17 slots] u4 (slot 16 zero) | scales,
  // sums [2][TGW][NQ][4 tokens] f4 (groups 4q..4q+3).
  u4 *la = reinterpret_cast<u4 *>(smem);
  f4 *lsc = reinterpret_cast<f4 *>(la + 2 * ABUF);
  f4 *lsu = lsc + 2 * SU;
  const int groups = cols / 32, nq = groups / 4, nch = (nq + NQ - 1) / NQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, h = lane >> 4;
  const int tg0 = blockIdx.y * TGW;
  const int row = blockIdx.x * (16 * WPB) + 16 * wave + j;
  const int rowc = min(row, rows - 1);
  const u4 *cptr = reinterpret_cast<const u4 *>(nib + (size_t)rowc * (cols / 2)) + h;
  const u4 *pptr = reinterpret_cast<const u4 *>(params + (size_t)rowc * groups * 4);
  const u4 *qsrc = reinterpret_cast<const u4 *>(qa);
  for (int i = tid; i < 2 * TGW * NQ * 4; i += NT) la[i * 17 + 16] = u4{0u, 0u, 0u, 0u};

  // Chunk staging.  Token groups past ntg (grid rounding) and steps past nq
  // load clamped duplicates; their results are never stored.
  u4 sa[NA];
  f4 ssc[NS], ssu[NS];
#define RAI_RS_LOAD(C)                                                                          \
  {                                                                                             \
    const int c_ = (C);                                                                         \
    _Pragma("unroll") for (int u = 0; u < NA; ++u) {                                            \
      const int i = min(tid + NT * u, AU - 1);                                                  \
      const int tg = i / (NQ * 64), rem = i - tg * (NQ * 64);                                   \
      const int qq = min(c_ * NQ + rem / 64, nq - 1);                                           \
      sa[u] = qsrc[((size_t)min(tg0 + tg, ntg - 1) * nq + qq) * 64 + (rem & 63)];                \
    }                                                                                           \
    _Pragma("unroll") for (int u = 0; u < NS; ++u) {                                            \
      const int i = min(tid + NT * u, SU - 1);                                                  \
      const int tg = i / (NQ * 4), qq = min(c_ * NQ + (i / 4) % NQ, nq - 1);                     \
      const int tok = min(4 * (tg0 + tg) + (i & 3), m - 1);                                     \
      ssc[u] = reinterpret_cast<const f4 *>(scales + (size_t)tok * groups)[qq];                 \
      ssu[u] = reinterpret_cast<const f4 *>(sums + (size_t)tok * groups)[qq];                   \
    }                                                                                           \
  }
  int huge = 0;
  float f[TGW][4], zc[TGW];
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
    f[tg][0] = f[tg][1] = f[tg][2] = f[tg][3] = 0.0f;
    zc[tg] = 0.0f;
  }
  const int aslot = (h == (j & 3)) ? j : 16;
  u32x4 rc[NQ], rp[NQ];
  for (int c = -1; c < nch; ++c) {
    RAI_RS_LOAD(min(c + 1, nch - 1))
    const int b = c & 1;
    gemv_rs_steps<TGW, NQ>(c * NQ, huge != 0, rc, rp, cptr, pptr, la + b * ABUF + aslot, lsc + b * SU,
                           lsu + b * SU, nq, h, f, zc);
    // Store chunk c + 1 into the other buffer (last read by chunk c - 1,
    // before the previous barrier) and flag huge scales in it.
    const int bn = (c + 1) & 1;
    int big = 0;
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int i = tid + NT * u;
      if (i < AU) la[bn * ABUF + (i >> 4) * 17 + (i & 15)] = sa[u];
    }
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int i = tid + NT * u;
      if (i < SU) {
        lsc[bn * SU + i] = ssc[u];
        lsu[bn * SU + i] = ssu[u];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = fabsf(ssc[u][e]);
          big |= (v >= 0x1p88f && v < INFINITY) ? 1 : 0;
        }
      }
    }
    huge = __syncthreads_or(big);
  }
#undef RAI_RS_LOAD
  if (row < rows) {
#pragma unroll
    for (int tg = 0; tg < TGW; ++tg) {
      const int t = 4 * (tg0 + tg) + h;
      if (t < m) {
        const size_t oi = (size_t)t * rows + row;
        const float v = ((f[tg][0] + f[tg][1]) + (f[tg][2] + f[tg][3])) + zc[tg];
        out[oi] = add ? add[oi] + v : v;
      }
    }
  }
}

// LDS bytes of k_gemv_rs: two chunk buffers of A blocks, scales and sums.
size_t gemv_rs_smem(int tgw, int nq_chunk) {
  return (size_t)2 * tgw * nq_chunk * (68 * 16 + 2 * 4 * 16);
}

// Register-pipelined version for K up to kRpMaxCols (several token groups
// per block) or kRpMaxColsOne (one).  The block stages all of its
// activations in LDS once (no barriers in the main loop).  Each wave
// streams 16 rows as k_gemv_rs does, through a ring of NQ slots (slot s holds
// step q = s mod NQ: 16 B of codes of group 4q + h, 16 B of parameters of
// groups 4q..4q+3), and pipelines by one step: step q unpacks its codes,
// then per token group runs the epilogue of step q - 1 (its MFMA results
// and staged scales, issued a step earlier), requests the scales of step q
// and issues the MFMAs of step q; the A operands of the next token group
// are requested one group ahead.  The slot of step q - 1 is refilled with
// step q - 1 + NQ after its parameters are used.
//
// fl(ws * x) and fl(wz * xsum) come from v_fma_mix with a -0 addend held in
// a register the compiler cannot see through: the fused multiply-add of a
// product and -0 rounds once, like the product, and reads the f16 halves of
// the parameter dword directly.  With subnormal codes the staged activation
// scales carry the 2^24 (as * 2^24 is exact below 2^104): fl(ws * (as *
// 2^24)) = fl((ws * 2^24) * as).
// One 16-byte piece of block-split int8 activations (blocks b and b + 1 of
// one token and group; per block the even columns c0 c2 c4 c6, then the odd
// ones c1 c3 c5 c7) as the two f16 A slots of those blocks: K order (0, 4,
// 1, 5, 2, 6, 3, 7), odd columns divided by 16, as k_qa_pack4 writes them.
// A byte x ^ 0x80 = x + 128 placed under 0x64 is the f16 1152 + x; minus
// 1152 gives x, and times 1/16 then minus 72 gives x / 16, every step exact.
__device__ __forceinline__ void a_slots_from_i8(u32x4 v, u32x4 &a0, u32x4 &a1) {
  const h2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  const h2 sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 off = {(_Float16)-72.0f, (_Float16)-72.0f};
  auto slot = [&](uint32_t ev, uint32_t od) {
    ev ^= 0x80808080u;
    od ^= 0x80808080u;
    const h2 e01 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, ev, 0x04020400u)) + bias;
    const h2 e45 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, ev, 0x04030401u)) + bias;
    const h2 e23 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, od, 0x04020400u)) * sixteenth + off;
    const h2 e67 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, od, 0x04030401u)) * sixteenth + off;
    return u32x4{__builtin_bit_cast(uint32_t, e01), __builtin_bit_cast(uint32_t, e23),
                 __builtin_bit_cast(uint32_t, e45), __builtin_bit_cast(uint32_t, e67)};
  };
  a0 = slot(v[0], v[1]);
  a1 = slot(v[2], v[3]);
}

constexpr int kRpMaxCols = 4096, kRpMaxColsOne = 14336;

template <bool HI>
__device__ __forceinline__ float mul_h16(uint32_t w, float x, float nz) {
  const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(HI ? w >> 16 : w & 0xFFFF));
  return __builtin_fmaf((float)h, x, nz);
}

// NG token groups; la / lsc / lsu point at the lane's slot of token group
// 0: A of (group t, step q, block b) at la[((t * nq + q) * 4 + b) * 17],
// scales / sums of (t, q) at [(t * nq + q) * 4].
//
// L1: the last token group holds a single token, whose four block chains
// then go to the four lane rows instead of four tokens: its MFMA for block b
// takes A row 4b + r = the token's block b of group 4q + r (nonzero on K
// block r only), the four accumulate into one D, and lane (j, h) holds
// S[row j][group 4q + r][block h] for r = 0..3 (every other term an exact
// zero).  The lane runs that token's block-h chain, its cs and its zc chain
// (5 operations per group instead of 11); l1off[b] moves the lane's A slot
// to the one block b needs, hs moves its scale slot to the token's.
template <int NG, int NQ, bool SUB, bool L1, int PSB>
__device__ __forceinline__ void gemv_rp_main(const __amdgpu_buffer_rsrc_t rcs, const __amdgpu_buffer_rsrc_t rps,
                                             uint32_t vc0, uint32_t vp0, const u32x4 *__restrict__ la,
                                             const f32x4 *__restrict__ lsc, const f32x4 *__restrict__ lsu,
                                             int nq, float nz, u32x4 (&rc)[NQ], u32x4 (&rp)[NQ],
                                             float (&f)[NG][4], float (&zc)[NG], const int (&l1off)[4], int hs) {
  typedef u32x4 u4;
  typedef f32x4 f4;
  const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  // MFMA results and staged scales of the previous step (each step runs the
  // epilogue of the one before; step 0 has none, so nothing is zeroed).
  f4 D[NG][4], as4[NG], xs4[NG];
  // Lane offsets of the single-token group's A slots and scale slot.
  auto aoff = [&](int t, int b) { return L1 && t == NG - 1 ? l1off[b] : 0; };
  auto soff = [&](int t) { return L1 && t == NG - 1 ? -hs : 0; };
  u4 avc[4], avn[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) avc[b] = la[b * 17 + aoff(0, b)];
  // One step q in ring slot s; FIRST: step 0, without an epilogue.
  auto step = [&](const int q, const int s, auto first) {
    constexpr bool FIRST = decltype(first)::value;
    const int sp = (s + NQ - 1) % NQ;
    // Refill step, clamped to the last one (a repeated read the cache
    // serves; never used); the uniform part of the offset goes to the
    // SGPR offset.
    const int qr = min(q - 1 + NQ, nq - 1);
    h8 bq[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) bq[b] = SUB ? unpack_codes_sub(rc[s][b]) : unpack_codes(rc[s][b]);
    rc[sp] = __builtin_amdgcn_raw_buffer_load_b128(rcs, (int)vc0, qr * 64, 0);
#pragma unroll
    for (int t = 0; t < NG; ++t) {
      {
        const int tn = t + 1 < NG ? t + 1 : 0;
        const int qn = t + 1 < NG ? q : min(q + 1, nq - 1);
#pragma unroll
        for (int b = 0; b < 4; ++b) avn[b] = la[((tn * nq + qn) * 4 + b) * 17 + aoff(tn, b)];
      }
      const bool one = L1 && t == NG - 1;
      if constexpr (!FIRST) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float cs = mul_h16<false>(rp[sp][r], as4[t][r], nz);
          f[t][0] = f[t][0] + D[t][0][r] * cs;
          if (!one) {
            f[t][1] = f[t][1] + D[t][1][r] * cs;
            f[t][2] = f[t][2] + D[t][2][r] * cs;
            f[t][3] = f[t][3] + D[t][3][r] * cs;
          }
          zc[t] = zc[t] + mul_h16<true>(rp[sp][r], xs4[t][r], nz);
        }
      }
      as4[t] = lsc[(t * nq + q) * 4 + soff(t)];
      xs4[t] = lsu[(t * nq + q) * 4 + soff(t)];
      if (one) {
        D[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, avc[0]), bq[0], zero4, 0, 0, 0);
#pragma unroll
        for (int b = 1; b < 4; ++b)
          D[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, avc[b]), bq[b], D[t][0], 0, 0, 0);
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          D[t][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, avc[b]), bq[b], zero4, 0, 0, 0);
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) avc[b] = avn[b];
    }
    rp[sp] = __builtin_amdgcn_raw_buffer_load_b128(rps, (int)vp0, qr * PSB, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // The first NQ steps (step 0 peeled), then the rest NQ at a time.
  step(0, 0, std::true_type{});
#pragma unroll
  for (int s = 1; s < NQ; ++s) step(s, s, std::false_type{});
  for (int q0 = NQ; q0 < nq; q0 += NQ) {
#pragma unroll
    for (int s = 0; s < NQ; ++s) step(q0 + s, s, std::false_type{});
  }
  // Epilogue of the last step (slot NQ - 1: nq is a multiple of NQ).
#pragma unroll
  for (int t = 0; t < NG; ++t) {
    const bool one = L1 && t == NG - 1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cs = mul_h16<false>(rp[NQ - 1][r], as4[t][r], nz);
      f[t][0] = f[t][0] + D[t][0][r] * cs;
      if (!one) {
        f[t][1] = f[t][1] + D[t][1][r] * cs;
        f[t][2] = f[t][2] + D[t][2][r] * cs;
        f[t][3] = f[t][3] + D[t][3][r] * cs;
      }
      zc[t] = zc[t] + mul_h16<true>(rp[NQ - 1][r], xs4[t][r], nz);
    }
  }
}

// Block of WPB waves = 16 * WPB rows and TGW token groups (blockIdx.y picks
// the token groups); requires K <= 128 * MAXQ and (K / 128) % NQ == 0.
// TMP: the parameters in the 16-row tile layout of k_params_tile16 (rows a
// multiple of 16), where one step's parameters of a wave's 16 rows are 256
// contiguous bytes (two cache lines) instead of 16 bytes in each of 16
// rows: the same values, fewer lines per load.
//
// The A operands are built in the prologue from the block-split int8
// activations (half the bytes of their f16 form, which matters: every CU
// pulls the whole activation block through its L1 before the first step).
template <int TGW, int NQ, int WPB, int MAXQ, bool TMP>
__global__ __launch_bounds__(64 * WPB, 8 / WPB) void k_gemv_rp(
    float *out, const float *add, const uint8_t *__restrict__ nib, const uint8_t *__restrict__ params,
    const int8_t *__restrict__ q_split, const float *__restrict__ scales, const float *__restrict__ sums, int rows,
    int cols, int m, int ntg) {
  typedef u32x4 u4;
  typedef f32x4 f4;
  constexpr int NT = 64 * WPB;
  constexpr int PB = MAXQ * 32 / NT;             // 16-byte int8 pieces per thread and token group
  constexpr int PS = (MAXQ * 4 + NT - 1) / NT;   // scale / sum f4 per thread and token group
  static_assert(PB * NT == MAXQ * 32, "whole activation loads per thread");
  extern __shared__ __align__(16) unsigned char smem[];
  const int groups = cols / 32, nq = groups / 4;
  // LDS: A [TGW][nq][4 blocks][17 slots] u4 (slot 16 zero) | scales, sums
  // [TGW][nq][4 tokens] f4 (groups 4q..4q+3).
  u4 *la = reinterpret_cast<u4 *>(smem);
  f4 *lsc = reinterpret_cast<f4 *>(la + TGW * nq * 68);
  f4 *lsu = lsc + TGW * nq * 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, h = lane >> 4;
  const int tg0 = blockIdx.y * TGW;
  const int row = blockIdx.x * (16 * WPB) + 16 * wave + j;
  const int rowc = min(row, rows - 1);
  // Every weight load is in range (steps clamped to the last one): the
  // lane's row offset in the VGPR offset, the step offset in the SGPR one.
  const __amdgpu_buffer_rsrc_t rcs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(nib), 0, rows * (cols / 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rps =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(params), 0, rows * groups * 4, 0x00020000);
  // Rows of tokens past m read as zeros (past the range).
  const __amdgpu_buffer_rsrc_t rqs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(q_split), 0, m * cols, 0x00020000);
  const uint32_t vc0 = (uint32_t)rowc * (cols / 2) + h * 16;
  constexpr int PSB = TMP ? 256 : 16;  // parameter bytes between steps
  const uint32_t vp0 =
      TMP ? (uint32_t)(rowc >> 4) * groups * 64 + (rowc & 15) * 16 : (uint32_t)rowc * groups * 4;

  // Activations (16-byte int8 pieces), scales and sums first (fixed counts,
  // clamped duplicates past the end, all issued before any wait), then the
  // ring.  Piece i of a token group: its token t = i / (nq * 8), bytes
  // 16 w.. of that token's row (w = i % (nq * 8)), which hold blocks
  // 2 (w & 1) and 2 (w & 1) + 1 of group w / 2.
  const int npr = nq * 8;  // pieces per token row
  auto piece = [&](int i, int &t, int &w) {
    t = (i >= npr) + (i >= 2 * npr) + (i >= 3 * npr);
    w = i - t * npr;
  };
  u4 sq[TGW][PB];
  f4 ssc[TGW][PS], ssu[TGW][PS];
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
    const int tgc = min(tg0 + tg, ntg - 1);
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      int t, w;
      piece(min(tid + NT * u, nq * 32 - 1), t, w);
      sq[tg][u] = __builtin_amdgcn_raw_buffer_load_b128(rqs, (4 * tgc + t) * cols + 16 * w, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < PS; ++u) {
      const int i = min(tid + NT * u, nq * 4 - 1);
      const int tok = min(4 * (tg0 + tg) + (i & 3), m - 1);
      ssc[tg][u] = reinterpret_cast<const f4 *>(scales + (size_t)tok * groups)[i >> 2];
      ssu[tg][u] = reinterpret_cast<const f4 *>(sums + (size_t)tok * groups)[i >> 2];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  u4 rc[NQ], rp[NQ];
  rc[NQ - 1] = rp[NQ - 1] = u4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int s = 0; s < NQ - 1; ++s) {
    rc[s] = __builtin_amdgcn_raw_buffer_load_b128(rcs, (int)vc0, s * 64, 0);
    rp[s] = __builtin_amdgcn_raw_buffer_load_b128(rps, (int)vp0, s * PSB, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Unconditional stores (clamped duplicates write the same values); the
  // codes enter as f16 subnormals unless some activation scale of a real
  // token is at least 2^88.
  int big = 0;
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg) {
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      int t, w;
      piece(min(tid + NT * u, nq * 32 - 1), t, w);
      u4 a0, a1;
      a_slots_from_i8(sq[tg][u], a0, a1);
      u4 *d = la + tg * nq * 68 + ((w >> 3) * 4 + 2 * (w & 1)) * 17 + 4 * t + ((w >> 1) & 3);
      d[0] = a0;
      d[17] = a1;
    }
#pragma unroll
    for (int u = 0; u < PS; ++u) {
      const int i = min(tid + NT * u, nq * 4 - 1);
      lsu[tg * nq * 4 + i] = ssu[tg][u];
      const bool real = tid + NT * u < nq * 4 && 4 * (tg0 + tg) + (i & 3) < m;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = fabsf(ssc[tg][u][e]);
        big |= (real && v >= 0x1p88f && v < INFINITY) ? 1 : 0;
      }
    }
  }
  for (int i = tid; i < TGW * nq * 4; i += NT) la[i * 17 + 16] = u4{0u, 0u, 0u, 0u};
  const bool huge = __syncthreads_or(big) != 0;
  const float sk = huge ? 1.0f : 16777216.0f;
#pragma unroll
  for (int tg = 0; tg < TGW; ++tg)
#pragma unroll
    for (int u = 0; u < PS; ++u) lsc[tg * nq * 4 + min(tid + NT * u, nq * 4 - 1)] = ssc[tg][u] * sk;
  __syncthreads();
  float nz;
  asm volatile("v_mov_b32 %0, 0x80000000" : "=v"(nz));
  float f[TGW][4], zc[TGW];
#pragma unroll
  for (int t = 0; t < TGW; ++t) {
    f[t][0] = f[t][1] = f[t][2] = f[t][3] = 0.0f;
    zc[t] = 0.0f;
  }
  const int aslot = (h == (j & 3)) ? j : 16;
  // The block's last token group is the single token of m = 4k + 1.
  const bool l1 = (m & 3) == 1 && tg0 + TGW == ntg;
  int l1off[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) l1off[b] = ((h == (j & 3) && (j >> 2) == b) ? (j & 3) : 16) - aslot;
  if (huge) {
    // Rare; this path fills a ring of its own (the prologue's loads go
    // unused), which keeps the common path's ring in fixed registers.
    u4 rch[NQ], rph[NQ];
    rch[NQ - 1] = rph[NQ - 1] = u4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < NQ - 1; ++s) {
      rch[s] = __builtin_amdgcn_raw_buffer_load_b128(rcs, (int)vc0, s * 64, 0);
      rph[s] = __builtin_amdgcn_raw_buffer_load_b128(rps, (int)vp0, s * PSB, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    gemv_rp_main<TGW, NQ, false, false, PSB>(rcs, rps, vc0, vp0, la + aslot, lsc + h, lsu + h, nq, nz, rch, rph, f, zc,
                                        l1off, h);
  } else if (l1) {
    gemv_rp_main<TGW, NQ, true, true, PSB>(rcs, rps, vc0, vp0, la + aslot, lsc + h, lsu + h, nq, nz, rc, rp, f, zc,
                                      l1off, h);
  } else {
    gemv_rp_main<TGW, NQ, true, false, PSB>(rcs, rps, vc0, vp0, la + aslot, lsc + h, lsu + h, nq, nz, rc, rp, f, zc,
                                       l1off, h);
  }
  // Single-token group: lane (j, h) holds block chain h; lane (j, 0) sums
  // the four in the reference order.
  float g1 = 0.0f, g2 = 0.0f, g3 = 0.0f;
  if (l1 && !huge) {
    g1 = __shfl(f[TGW - 1][0], j + 16);
    g2 = __shfl(f[TGW - 1][0], j + 32);
    g3 = __shfl(f[TGW - 1][0], j + 48);
  }
  if (row < rows) {
#pragma unroll
    for (int t = 0; t < TGW; ++t) {
      const bool one = l1 && !huge && t == TGW - 1;
      const int tok = 4 * (tg0 + t) + (one ? 0 : h);
      if (tok < m && (!one || h == 0)) {
        const size_t oi = (size_t)tok * rows + row;
        const float v = one ? ((f[t][0] + g1) + (g2 + g3)) + zc[t]
                            : ((f[t][0] + f[t][1]) + (f[t][2] + f[t][3])) + zc[t];
        out[oi] = add ? add[oi] + v : v;
      }
    }
  }
}

namespace {

template <int TGW, int P>
void launch_ms(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const _Float16 *qa,
               const float *scales, const float *sums, int rows, int cols, int m, int ntg,
               hipStream_t s) {
  constexpr int WPB = 4;
  const dim3 grid((rows + 16 * WPB - 1) / (16 * WPB), (ntg + TGW - 1) / TGW);
  hipLaunchKernelGGL((k_gemv_ms<TGW, P, WPB>), grid, dim3(64 * WPB), 0, s, out, add, nib, params, qa,
                     scales, sums, rows, cols, m);
}

}  // namespace

bool w4a8_mfma_path(int rows, int cols, int m, int gs) {
  return gs == 32 && m >= 2 && m <= kMfmaMaxTokens && cols % (32 * 8) == 0 && rows > 0;
}

size_t qa_pack_halves(int m, int cols) {
  return (size_t)((m + 3) / 4) * (cols / 32) * 16 * 8;
}

void launch_qa_pack(const int8_t *q_split, int m, int cols, _Float16 *qa, hipStream_t s) {
  const int ntg = (m + 3) / 4;
  const int n = ntg * (cols / 128) * 64;
  hipLaunchKernelGGL(k_qa_pack4, dim3((n + 255) / 256), dim3(256), 0, s, q_split, m, cols, ntg, qa);
}

namespace {

template <int TGW, int NQ>
void launch_rs(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const _Float16 *qa,
               const float *scales, const float *sums, int rows, int cols, int m, int ntg, hipStream_t s) {
  constexpr int WPB = 4;
  const size_t smem = gemv_rs_smem(TGW, NQ);
  static bool configured = false;
  if (!configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_rs<TGW, NQ, WPB>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = true;
  }
  const dim3 grid((rows + 16 * WPB - 1) / (16 * WPB), (ntg + TGW - 1) / TGW);
  hipLaunchKernelGGL((k_gemv_rs<TGW, NQ, WPB>), grid, dim3(64 * WPB), smem, s, out, add, nib, params, qa,
                     scales, sums, rows, cols, m, ntg);
}

constexpr int kRpRing = 4;

// K the register-pipelined kernel takes with one token group per block
// (longer K only that way: the block's activations must fit in LDS).
bool gemv_rp_ok(int rows, int cols) {
  return cols <= kRpMaxColsOne && (cols / 128) % kRpRing == 0 &&
         (int64_t)rows * (cols / 2) < ((int64_t)1 << 31);
}

template <int TGW, int WPB, int MAXQ, bool TMP, int NQ = kRpRing>
void launch_rp(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
               const float *scales, const float *sums, int rows, int cols, int m, int ntg, hipStream_t s) {
  constexpr size_t kStepBytes = 68 * 16 + 2 * 4 * 16;  // A blocks, scales, sums of one (group, step)
  static bool configured = false;
  if (!configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_rp<TGW, NQ, WPB, MAXQ, TMP>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)(TGW * MAXQ * kStepBytes));
    configured = true;
  }
  const size_t smem = TGW * (size_t)(cols / 128) * kStepBytes;
  const dim3 grid((rows + 16 * WPB - 1) / (16 * WPB), (ntg + TGW - 1) / TGW);
  hipLaunchKernelGGL((k_gemv_rp<TGW, NQ, WPB, MAXQ, TMP>), grid, dim3(64 * WPB), smem, s, out, add, nib, params,
                     q_split, scales, sums, rows, cols, m, ntg);
}

template <bool TMP>
void launch_rp_shape(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                     const float *scales, const float *sums, int rows, int cols, int m, int ntg, hipStream_t s) {
  constexpr int Q = kRpMaxCols / 128, Q1 = kRpMaxColsOne / 128;
  const int rb = (rows + 63) / 64;
  auto blocks = [&](int tgw) { return rb * ((ntg + tgw - 1) / tgw); };
  // Three token groups per wave for 3, 5 or 6 and more groups (the
  // duplicates past an odd count cost less than a third pass over the
  // weights), two for four.  Up to 8192 rows and five token groups, one
  // token group per block with the tiled parameters (qkv 6144x4096 at 9
  // tokens 14.3 -> 13.5 us, at 17 tokens 19.3 -> 14.3; o_proj 4096x4096 at
  // 17 tokens 14.3 -> 13.5).
  const bool three = ntg >= 3 && ntg != 4;
  // Past K = 4096 (one token group per block, 3.5 x the steps) a ring of
  // eight steps where K / 128 allows (down 4096x14336 at 9 tokens 26.9 ->
  // 26.2 us; shorter K is slower with it).
  if (cols > kRpMaxCols && (cols / 128) % 8 == 0)
    launch_rp<1, 4, Q1, TMP, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
  else if (cols > kRpMaxCols)
    launch_rp<1, 4, Q1, TMP>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
  else if (TMP && rows <= 8192 && ntg <= 5)
    launch_rp<1, 4, Q, TMP>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
  else if (three && rows >= 16384)
    launch_rp<3, 8, Q, TMP>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
  else if (three && blocks(3) >= 192)
    launch_rp<3, 4, Q, TMP>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
  else if (ntg >= 2 && blocks(2) >= 192)
    launch_rp<2, 4, Q, TMP>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
  else
    launch_rp<1, 4, Q, TMP>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
}

// One thread per 16 bytes (four groups' parameters of one row).
__global__ void k_params_tile16(const u32x4 *__restrict__ params, int rows, int nq, u32x4 *__restrict__ tiled) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nq) return;
  const int row = i / nq, q = i - row * nq;
  tiled[((size_t)(row >> 4) * nq + q) * 16 + (row & 15)] = params[i];
}

}  // namespace

bool params_tile16_ok(int rows, int cols, int gs) {
  return gs == 32 && rows % 16 == 0 && cols % 128 == 0 && (int64_t)rows * (cols / 32) * 4 < ((int64_t)1 << 31);
}

void launch_params_tile16(const uint8_t *params, int rows, int cols, uint8_t *tiled, hipStream_t s) {
  const int nq = cols / 128;
  const int n = rows * nq;
  hipLaunchKernelGGL(k_params_tile16, dim3((n + 255) / 256), dim3(256), 0, s,
                     reinterpret_cast<const u32x4 *>(params), rows, nq, reinterpret_cast<u32x4 *>(tiled));
}

bool launch_w4a8_mfma(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const _Float16 *qa,
                      const int8_t *q_split, const float *scales, const float *sums, int rows, int cols, int m,
                      int gs, hipStream_t s, const uint8_t *params_tiled) {
  if (!qa || !w4a8_mfma_path(rows, cols, m, gs)) return false;
  const int ntg = (m + 3) / 4;
  const int groups = cols / 32;
  // Kernel and tiling per shape, measured on 4096..32000 x 2048..14336 and
  // M = 2..64 with the weights streamed from HBM.  The register-pipelined
  // kernel: for K <= 4096 three token groups per wave, or two, when that
  // still gives at least 192 blocks of four waves (64 rows), else one (a
  // count of token groups that the wave's groups do not divide runs the
  // last block with clamped duplicate groups whose outputs are not stored);
  // eight waves per block for three groups from 16384 rows.  For longer K (K / 128 a
  // multiple of 4, at most 14336) one token group per block.  With the
  // parameters also in the 16-row tile layout, that copy is read instead
  // (o_proj 4096x4096 at 9 tokens 10.9 -> 9.3 us, down 4096x14336 31.8 ->
  // 26.6, gate|up 28672x4096 27.5 -> 26.6).
  if (q_split && gemv_rp_ok(rows, cols)) {
    if (params_tiled && params_tile16_ok(rows, cols, gs))
      launch_rp_shape<true>(out, add, nib, params_tiled, q_split, scales, sums, rows, cols, m, ntg, s);
    else
      launch_rp_shape<false>(out, add, nib, params, q_split, scales, sums, rows, cols, m, ntg, s);
    return true;
  }
  // Longer K: the register-streamed kernel for many rows (one wave keeps up
  // to four token groups; past 16384 rows a shallower ring lets two blocks
  // share a CU), the block-staged kernel with one token group per wave for
  // fewer rows.
  if (rows >= 16384) {
    if (ntg == 1) launch_rs<1, 4>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else if (ntg == 2) launch_rs<2, 4>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else if (ntg == 3) launch_rs<3, 4>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else launch_rs<4, 4>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  } else if (rows >= 8192) {
    if (ntg == 1) launch_rs<1, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else if (ntg == 3) launch_rs<3, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else launch_rs<2, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  } else if (groups % 16 == 0) {
    launch_ms<1, 16>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  } else {
    launch_ms<1, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  }
  return true;
}

}  // namespace rai
