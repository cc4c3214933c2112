// W4A8 GEMM for prefill-sized token counts (M > 64) on the gfx950 matrix
// cores, group 32: the reference's matmul_chunk_i8 / matmul_row_tile
// (gemm.rs:540-784) with the same per-lane integer sums and the same f32
// epilogue order, so the outputs equal the CPU path bit for bit.
//
// Integer part.  v_mfma_f32_32x32x8_f16 with exact operands: one
// instruction takes a K-slice of exactly one 8-column block b of one
// 32-column group, so D[token][row] is the reference's lane sum S_b (the
// PMADDUBSW/PMADDWD sum of 8 code x activation products, gemm.rs:606-614)
// for 32 tokens x 32 rows, with no block-diagonal padding.  Codes 0..15
// enter as f16 subnormals n 2^-24 (odd columns 16 n 2^-24: one mask per
// pair), activations as f16 a (odd columns a / 16); every product and
// partial sum is an integer times 2^-24 below 2^-10, so the f32
// accumulators hold S 2^-24 exactly in any order, and the records carry the
// activation scales times 2^24, so that fl(S 2^-24 * fl(ws * as 2^24)) =
// fl(S * fl(ws * as)) (power-of-two scaling commutes with rounding in the
// normal range; ws * as is zero or above 2^-24 * 1e-10 / 127).  A quad of
// groups whose 32 tokens include a scale of 2^88 or more (where as 2^24
// could overflow the product) keeps its scales as they are, is flagged,
// and runs with the codes as f16 1024 + n minus 1024 (S itself).  The
// f16 instruction is used rather than an int8 one because it returns S
// already as f32: an i32 result would cost one VALU conversion per S, and
// the VALU epilogue, not the matrix core, bounds this kernel.
//
// Lane roles (32x32x8): B = weights, lane l holds row j = l % 32 and the
// K-slice half h = l / 32; A = activations, token i = l % 32, half h; the
// lane's 16 results are tokens 8 (v / 4) + 4 h + v % 4 of row j.  K order
// of a half: columns (2h, 2h + 4, 2h + 1, 2h + 5) of the block.
//
// Epilogue per lane, for its row and 16 tokens, in group order
// (gemm.rs:616-651): cs = fl(ws * as); f_b += fl(S_b * cs) (b = 0..3);
// zc += fl(wz * xsum); at the end out = ((f0 + f1) + (f2 + f3)) + zc (the
// movehdup/movehl sum of gemm.rs:655-662 with lanes 4..7 at +0).
//
// Data: activations are packed once per GEMM input by k_mm_pack into
// 2304-byte records per (32-token tile, group): four 512-byte A operands
// (lane-ordered), then 32 scales (times 2^24 unless flagged) and 32 input
// sums; after the records one int per (token tile, quad of groups), nonzero
// for a flagged quad.  A block of WR waves
// (32 rows each) shares one token tile; the records of P groups are copied
// to LDS by DMA (global_load_lds), double-buffered.  Each lane streams its
// row's codes (16 B per group) and parameters (16 B per four groups)
// through a register ring four groups ahead.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "kernels.h"

namespace rai {

namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kMmRec = 2304;  // bytes per (token tile, group)
constexpr int kMmP = 16;      // groups per LDS stage
constexpr int kMmWR = 4;      // waves (32-row tiles) per block

// One block per (token tile, four consecutive groups), 256 threads.  The
// tile's 32 rows of those 128 columns are read with whole-line loads (eight
// lanes of 16 bytes per row) into LDS; then thread (b, lane) of pass g
// writes the lane's four f16 A values of block b of group g, and one
// thread per (group, token) its scale or input sum.  Tokens past m are
// zero.
__global__ __launch_bounds__(256) void k_mm_pack(const int8_t *__restrict__ q_split,
                                                 const float *__restrict__ scales, const float *__restrict__ sums,
                                                 int m, int cols, int groups, uint8_t *__restrict__ rec) {
  constexpr int QS = 128 + 16;  // LDS row stride (bytes)
  __shared__ __align__(16) int8_t qs[32 * QS];
  const int tid = threadIdx.x, gq = blockIdx.x, tt = blockIdx.y;
  {
    const int row = tid >> 3, seg = tid & 7, t = tt * 32 + row;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (t < m) v = *reinterpret_cast<const uint4 *>(q_split + (size_t)t * cols + 128 * gq + 16 * seg);
    *reinterpret_cast<uint4 *>(qs + row * QS + 16 * seg) = v;
  }
  __syncthreads();
  uint8_t *r0 = rec + ((size_t)tt * groups + 4 * gq) * kMmRec;
  const int l = tid & 63, b = tid >> 6, i = l & 31, h = l >> 5;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    // q_split block: four even columns, then four odd ones.
    const int8_t *e = qs + i * QS + 32 * g + 8 * b;
    h4 a;
    a[0] = (_Float16)(float)e[h];
    a[1] = (_Float16)(float)e[h + 2];
    a[2] = (_Float16)((float)e[4 + h] * 0.0625f);
    a[3] = (_Float16)((float)e[6 + h] * 0.0625f);
    *reinterpret_cast<h4 *>(r0 + g * kMmRec + b * 512 + l * 8) = a;
  }
  {
    const int g = tid >> 6, which = (tid >> 5) & 1, t = tt * 32 + i;
    const float v = t < m ? (which ? sums : scales)[(size_t)t * groups + 4 * gq + g] : 0.0f;
    const float av = fabsf(v);
    const bool huge = __syncthreads_or(which == 0 && av >= 0x1p88f && av < INFINITY) != 0;
    reinterpret_cast<float *>(r0 + g * kMmRec + 2048 + which * 128)[i] = (which == 0 && !huge) ? v * 0x1p24f : v;
    if (tid == 0) reinterpret_cast<int *>(rec + (size_t)gridDim.y * groups * kMmRec)[tt * (groups / 4) + gq] = huge;
  }
}

// fl(x * h) for the f16 half of a parameter dword: a fused multiply-add
// with a -0 addend rounds once, like the product (v_fma_mix reads the half
// directly).
template <bool HI>
__device__ __forceinline__ float mul_half(uint32_t w, float x, float nz) {
  const _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)(HI ? w >> 16 : w & 0xFFFF));
  return __builtin_fmaf((float)hv, x, nz);
}

// The B operand of block dword w for half h (sh = 8 h): the codes as f16
// subnormals (SUB), or as 1024 + n minus 1024.
template <bool SUB>
__device__ __forceinline__ h4 unpack_half(uint32_t w, uint32_t sh) {
  const uint32_t t = w >> sh;
  if constexpr (SUB) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 d = {t & 0x000F000Fu, t & 0x00F000F0u};
    return __builtin_bit_cast(h4, d);
  }
  const h2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2 e0 = __builtin_bit_cast(h2, (t & 0x000F000Fu) | 0x64006400u) - bias;
  const h2 e1 = __builtin_bit_cast(h2, (t & 0x00F000F0u) | 0x64006400u) - bias;
  h4 r;
  r[0] = e0[0];
  r[1] = e0[1];
  r[2] = e1[0];
  r[3] = e1[1];
  return r;
}

struct MmLane {
  float f[4][16];
  float zc[16];
};

// One group: four MFMAs from the LDS record `rc` and the code dword ring
// slot `wq`, then the epilogue with parameter dword `pw`.  Codes as f16
// subnormals (SUB), or as 1024 + n with the record's scales times smul
// (2^-24 for those stored times 2^24: exact).
template <bool SUB>
__device__ __forceinline__ void mm_group(const uint8_t *rc, const u4v &wq, uint32_t pw, uint32_t sh, int lane,
                                         int h, float nz, float smul, MmLane &acc) {
  const f16v zero = {};
  // Blocks 0 and 1 first; their MFMAs run while the zero-point chain and
  // the combined scales are computed.
  f16v D0 = __builtin_amdgcn_mfma_f32_32x32x8f16(*reinterpret_cast<const h4 *>(rc + lane * 8),
                                                 unpack_half<SUB>(wq[0], sh), zero, 0, 0, 0);
  f16v D1 = __builtin_amdgcn_mfma_f32_32x32x8f16(*reinterpret_cast<const h4 *>(rc + 512 + lane * 8),
                                                 unpack_half<SUB>(wq[1], sh), zero, 0, 0, 0);
  float cs[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f4v xs4 = *reinterpret_cast<const f4v *>(rc + 2176 + (8 * q + 4 * h) * 4);
    f4v as4 = *reinterpret_cast<const f4v *>(rc + 2048 + (8 * q + 4 * h) * 4);
    if constexpr (!SUB) as4 = as4 * smul;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc.zc[4 * q + r] = acc.zc[4 * q + r] + mul_half<true>(pw, xs4[r], nz);
      cs[4 * q + r] = mul_half<false>(pw, as4[r], nz);
    }
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    acc.f[0][v] = acc.f[0][v] + D0[v] * cs[v];
    acc.f[1][v] = acc.f[1][v] + D1[v] * cs[v];
  }
  D0 = __builtin_amdgcn_mfma_f32_32x32x8f16(*reinterpret_cast<const h4 *>(rc + 1024 + lane * 8),
                                            unpack_half<SUB>(wq[2], sh), zero, 0, 0, 0);
  D1 = __builtin_amdgcn_mfma_f32_32x32x8f16(*reinterpret_cast<const h4 *>(rc + 1536 + lane * 8),
                                            unpack_half<SUB>(wq[3], sh), zero, 0, 0, 0);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    acc.f[2][v] = acc.f[2][v] + D0[v] * cs[v];
    acc.f[3][v] = acc.f[3][v] + D1[v] * cs[v];
  }
}

// Block: WR waves x 32 rows, one 32-token tile (blockIdx.y).  Requires
// groups % P == 0 and rows * cols / 2 < 2^31.
template <int WR, int P>
__global__ __launch_bounds__(64 * WR, 2) void k_w4a8_mm(float *out, const float *add,
                                                        const uint8_t *__restrict__ nib,
                                                        const uint8_t *__restrict__ params,
                                                        const uint8_t *__restrict__ rec, int rows, int cols, int m) {
  constexpr int NI = P * kMmRec / 1024 / WR;  // DMA instructions per wave and stage
  static_assert(NI * WR * 1024 == P * kMmRec, "stage must split evenly over the waves");
  static_assert(P % 8 == 0, "two parameter quads per unrolled step");
  __shared__ __align__(16) uint8_t bufA[P * kMmRec];
  __shared__ __align__(16) uint8_t bufB[P * kMmRec];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 31, h = lane >> 5;
  const uint32_t sh = 8u * h;
  const int groups = cols >> 5, ntile = groups / P;
  const int row = blockIdx.x * 32 * WR + 32 * wave + j;
  const int rowc = min(row, rows - 1);
  const uint8_t *rtile = rec + (size_t)blockIdx.y * groups * kMmRec;
  const __amdgpu_buffer_rsrc_t rcs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(nib), 0, rows * (cols / 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rps =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(params), 0, rows * groups * 4, 0x00020000);
  const uint32_t vc0 = (uint32_t)rowc * (cols / 2);
  const uint32_t vp0 = (uint32_t)rowc * groups * 4;

  auto dma = [&](uint8_t *buf, int kt) {
    const uint8_t *src = rtile + (size_t)kt * P * kMmRec;
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int c = (u * WR + wave) * 1024;
      __builtin_amdgcn_global_load_lds(src + c + lane * 16, (lds_void *)(buf + c), 16, 0, 0);
    }
  };
  // Ring: codes of groups g..g+3 (slot g % 4), parameters of the current
  // and the next quad of groups; refills clamped to the last group.
  u4v wr[4], pr[2];
#pragma unroll
  for (int s = 0; s < 4; ++s) wr[s] = __builtin_amdgcn_raw_buffer_load_b128(rcs, (int)vc0, min(s, groups - 1) * 16, 0);
  pr[0] = __builtin_amdgcn_raw_buffer_load_b128(rps, (int)vp0, 0, 0);
  pr[1] = __builtin_amdgcn_raw_buffer_load_b128(rps, (int)vp0, min(4, groups - 4) * 4, 0);
  dma(bufA, 0);
  float nz;
  asm volatile("v_mov_b32 %0, 0x80000000" : "=v"(nz));
  MmLane acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    acc.f[0][v] = acc.f[1][v] = acc.f[2][v] = acc.f[3][v] = 0.0f;
    acc.zc[v] = 0.0f;
  }
  __syncthreads();

  // Quad flags of this token tile: any set (rare) runs the whole block with
  // the codes as 1024 + n, and the unflagged quads' scales times 2^-24.
  const int *qflag = reinterpret_cast<const int *>(rec + (size_t)gridDim.y * groups * kMmRec) +
                     (size_t)blockIdx.y * (groups / 4);
  int fl = 0;
  for (int i = lane; i < groups / 4; i += 64) fl |= qflag[i];
  const bool anybig = __builtin_amdgcn_ballot_w64(fl != 0) != 0;

  auto run = [&](auto sub) __attribute__((always_inline)) {
    constexpr bool SUB = decltype(sub)::value;
    // The P groups of stage kt from LDS buffer `buf`, eight at a time (two
    // parameter quads, so the parameter registers alternate statically).
    auto stage = [&](const uint8_t *buf, int kt) __attribute__((always_inline)) {
      for (int g8 = 0; g8 < P; g8 += 8) {
#pragma unroll
        for (int gi = 0; gi < 8; ++gi) {
          const int g = kt * P + g8 + gi;
          const int slot = gi & 3, quad = gi >> 2;
          float smul = 1.0f;
          if constexpr (!SUB) smul = __builtin_amdgcn_readfirstlane(qflag[g >> 2]) ? 1.0f : 0x1p-24f;
          mm_group<SUB>(buf + (g8 + gi) * kMmRec, wr[slot], pr[quad][gi & 3], sh, lane, h, nz, smul, acc);
          wr[slot] = __builtin_amdgcn_raw_buffer_load_b128(rcs, (int)vc0, min(g + 4, groups - 1) * 16, 0);
          if ((gi & 3) == 3)
            pr[quad] = __builtin_amdgcn_raw_buffer_load_b128(rps, (int)vp0, min(g + 5, groups - 4) * 4, 0);
        }
      }
    };
    for (int kt = 0; kt < ntile; kt += 2) {
      if (kt + 1 < ntile) dma(bufB, kt + 1);
      stage(bufA, kt);
      __syncthreads();
      if (kt + 1 < ntile) {
        if (kt + 2 < ntile) dma(bufA, kt + 2);
        stage(bufB, kt + 1);
        __syncthreads();
      }
    }
  };
  if (anybig)
    run(std::false_type{});
  else
    run(std::true_type{});
  if (row < rows) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int t = blockIdx.y * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      if (t < m) {
        const size_t oi = (size_t)t * rows + row;
        const float r = ((acc.f[0][v] + acc.f[1][v]) + (acc.f[2][v] + acc.f[3][v])) + acc.zc[v];
        out[oi] = add ? add[oi] + r : r;
      }
    }
  }
}

}  // namespace

bool w4a8_mm_path(int rows, int cols, int m, int gs) {
  return gs == 32 && m > kMfmaMaxTokens && rows > 0 && cols % (32 * kMmP) == 0 &&
         (int64_t)rows * (cols / 2) < ((int64_t)1 << 31);
}

size_t mm_pack_bytes(int m, int cols) {
  const size_t ntt = (size_t)((m + 31) / 32);
  return ntt * (cols / 32) * kMmRec + ntt * (cols / 128) * sizeof(int);
}

void launch_w4a8_mm(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                    const float *scales, const float *sums, int rows, int cols, int m, uint8_t *pack,
                    hipStream_t s) {
  const int groups = cols / 32, ntt = (m + 31) / 32;
  hipLaunchKernelGGL(k_mm_pack, dim3(groups / 4, ntt), dim3(256), 0, s, q_split, scales, sums, m, cols, groups, pack);
  const dim3 grid((rows + 32 * kMmWR - 1) / (32 * kMmWR), ntt);
  hipLaunchKernelGGL((k_w4a8_mm<kMmWR, kMmP>), grid, dim3(64 * kMmWR), 0, s, out, add, nib, params, pack, rows,
                     cols, m);
}

}  // namespace rai
