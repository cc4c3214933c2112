// W4A8 GEMV for small token counts on the gfx950 matrix cores, group 32.
//
// The integer dot products S[row][token][block] (8 columns of one 32-column
// group, the reference's per-lane int8 x int4 sums, gemm.rs:458-525) come
// from v_mfma_f32_16x16x32_f16 with exact operands: weight codes 0..15 and
// int8 activations are exact in f16, every product and partial sum is an
// integer below 2^24, so the f32 accumulators hold S exactly whatever the
// summation order inside the instruction.
//
// MFMA operand roles (16x16x32): B = weights, column j = row of the weight
// tile (16 rows per wave), K = the group's 32 columns in the lane order
// below.  A = activations, block-diagonal: A row i = 4t + b (token t of the
// wave's 4-token group, block b), nonzero only on block b's 8 columns.  So
// D[4t + b][j] = S[row j][token t][block b], and lane l (j = l % 16,
// h = l / 16) receives S for row j, token h, blocks 0..3 in its 4
// accumulators: exactly the 4 reference lane chains of one (row, token).
//
// Each lane then runs the reference epilogue for its (row, token) in group
// order: cs = fl(ws * as); f_b += fl(S_b * cs); zc += fl(wz * xsum), and at
// the end out = hsum8(f0..f3, 0, 0, 0, 0) + zc (gemm.rs:458-537).  The
// chains never leave the lane, so no products go through LDS.
//
// K order inside a block (8 columns c0..c7): f16 element e of the lane's 8
// is column (0, 4, 1, 5, 2, 6, 3, 7)[e], which is what the nibble unpack
// (shifts by 0/4/8/12 of a 0x000F000F mask) produces for the weights.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

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
// (0, 4, 1, 5, 2, 6, 3, 7): 0x6400 | n is the f16 1024 + n, minus 1024.
__device__ __forceinline__ h8 unpack_codes(uint32_t w) {
  const uint32_t m = 0x000F000Fu, o = 0x64006400u;
  const uint32_t d0 = (w & m) | o;
  const uint32_t d1 = ((w >> 4) & m) | o;
  const uint32_t d2 = ((w >> 8) & m) | o;
  const uint32_t d3 = ((w >> 12) & m) | o;
  const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2 e0 = __builtin_bit_cast(h2, d0) - bias;
  const h2 e1 = __builtin_bit_cast(h2, d1) - bias;
  const h2 e2 = __builtin_bit_cast(h2, d2) - bias;
  const h2 e3 = __builtin_bit_cast(h2, d3) - bias;
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

// Activations in the MFMA A-operand layout: qa[tg][g][slot i = 4t + b][8]
// f16, block b of token 4*tg + t in the K order above (zeros for tokens
// past m).  One thread per (token slot, group, block).
__global__ void k_qa_pack(const int8_t *__restrict__ q_split, int m, int cols, int ntg,
                          _Float16 *__restrict__ qa) {
  const int groups = cols / 32;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // over ntg*groups*16
  if (idx >= ntg * groups * 16) return;
  const int i = idx & 15, g = (idx >> 4) % groups, tg = (idx >> 4) / groups;
  const int t = 4 * tg + i / 4, b = i % 4;
  _Float16 *dst = qa + (size_t)idx * 8;
  if (t >= m) {
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[e] = (_Float16)0.0f;
    return;
  }
  // q_split block: bytes 0..3 = even columns 0,2,4,6; bytes 4..7 = odd 1,3,5,7.
  const int8_t *src = q_split + (size_t)t * cols + g * 32 + 8 * b;
  const int col_of_e[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = col_of_e[e];
    const int sidx = (c & 1) ? 4 + (c >> 1) : (c >> 1);
    dst[e] = (_Float16)(float)src[sidx];
  }
}

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
  constexpr int ASLOT = 16 * 8;            // halves per (tg, group) in qa
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
      S.a[u] = reinterpret_cast<const u4 *>(qa + ((size_t)(tgc * TGW + tg) * groups + (size_t)kt * P) * ASLOT)[k];
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
  const int n = ntg * (cols / 32) * 16;
  hipLaunchKernelGGL(k_qa_pack, dim3((n + 255) / 256), dim3(256), 0, s, q_split, m, cols, ntg, qa);
}

bool launch_w4a8_mfma(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const _Float16 *qa,
                      const float *scales, const float *sums, int rows, int cols, int m, int gs,
                      hipStream_t s) {
  if (!qa || !w4a8_mfma_path(rows, cols, m, gs)) return false;
  const int ntg = (m + 3) / 4;
  const int groups = cols / 32;
  // Many rows: one wave keeps every token group (the code unpack and param
  // decode are shared); few rows: one token group per wave for more waves
  // (measured on 4096..32000 x 4096..14336, M = 2..16).
  if (rows >= 8192) {
    if (ntg == 1) launch_ms<1, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else if (ntg == 2) launch_ms<2, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else if (ntg == 3) launch_ms<3, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
    else launch_ms<4, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  } else if (groups % 16 == 0) {
    launch_ms<1, 16>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  } else {
    launch_ms<1, 8>(out, add, nib, params, qa, scales, sums, rows, cols, m, ntg, s);
  }
  return true;
}

}  // namespace rai
