// Device helpers shared by the fused quantization kernels (fused.hip) and
// the GEMV kernels that quantize their own input (kernels.hip): per-group
// int8 quantization in the reference's order and the block-wide RMSNorm that
// feeds it.  Same bit-exact contract as the kernels: f32 operations in rai's
// AVX2 order (rai-infer/src/layers.rs, gemm.rs).
#ifndef RAI_QUANT_DEV_H
#define RAI_QUANT_DEV_H

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rai {

// Column c of a block-split row: 8-column block b holds its even columns at
// 8b+0..3 and its odd columns at 8b+4..7 (the q_split layout).
__device__ __forceinline__ int split_col(int c) {
  const int j = c & 7;
  return (c & ~7) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

// Quantize one group held by 8 consecutive lanes (lane j owns the columns
// 8c + j, c = 0..NB-1, of the group) exactly as quantize_input_split_avx2
// and compute_input_sums do (gemm.rs:182-212, 280-374):
//   sum   = ((a0+a4)+(a1+a5))+((a2+a6)+(a3+a7)), a_j = sequential sum of the
//           lane's values in column order;
//   scale = absmax/127 (1 when absmax <= 1e-10); q = clamp(rne(v/scale)).
// qs_grp / qn_grp point at the group's first byte in the block-split and
// natural layouts (qn_grp may be null; either may be in LDS).
// All 64 lanes of the wave must call this together.
// Lanes with ok == false take part in the shuffles and store nothing.
// Matrix-core activation slot of (token t, group g) for group 32 (see
// k_qa_pack4 in gemv.hip): qa4[t/4][g/4][b][4(t%4) + g%4][8] f16; block b of
// the slot is 128 halves further.
__device__ __forceinline__ _Float16 *qa4_slot(_Float16 *qa, int t, int g, int groups) {
  return qa + ((((size_t)(t >> 2) * (groups >> 2) + (g >> 2)) * 64) + 4 * (t & 3) + (g & 3)) * 8;
}

// Lane moves inside 16-lane rows (DPP, no LDS round trip): lane i reads
// lane i + n (0 past the row), lane 7 - i of its 8-lane half, and the
// quad permutations (1,0,3,2) and (2,3,0,1).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppShl1 = 0x101, kDppShl2 = 0x102, kDppShl4 = 0x104, kDppHalfMirror = 0x141, kDppXor1 = 0xB1,
              kDppXor2 = 0x4E;

template <int NB>
__device__ __forceinline__ void quantize_group8_to(const float (&v)[NB], int j, bool ok, int8_t *qs_grp,
                                                   int8_t *qn_grp, float *scale_out, float *sum_out,
                                                   _Float16 *qa_slot = nullptr) {
  float a = 0.0f, amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NB; ++c) {
    a = a + v[c];
    amax = fmaxf(amax, fabsf(v[c]));
  }
  // hsum8 in the reference's order: lanes 0..3 form a_j + a_{j+4}, lanes 0
  // and 2 add their right neighbour, lane 0 adds lane 2.
  const float b = a + dpp_mov<kDppShl4>(a);
  const float c = b + dpp_mov<kDppShl1>(b);
  const float total = c + dpp_mov<kDppShl2>(c);
  // Max over the 8 lanes (order-free), delivered to all of them.
  amax = fmaxf(amax, dpp_mov<kDppHalfMirror>(amax));
  amax = fmaxf(amax, dpp_mov<kDppXor1>(amax));
  amax = fmaxf(amax, dpp_mov<kDppXor2>(amax));
  const float scale = amax > 1e-10f ? amax / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  if (!ok) return;
#pragma unroll
  for (int c8 = 0; c8 < NB; ++c8) {
    float r = rintf(v[c8] * inv);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    const int8_t q = (int8_t)(int)r;
    const int col = 8 * c8 + j;
    qs_grp[split_col(col)] = q;
    if (qn_grp) qn_grp[col] = q;
    // f16 element e of a block is its column (0, 4, 1, 5, 2, 6, 3, 7)[e];
    // odd columns are stored divided by 16 (the codes enter at 16 n).
    if (qa_slot) qa_slot[c8 * 128 + 2 * (j & 3) + (j >> 2)] = (_Float16)((j & 1) ? r * 0.0625f : r);
  }
  if (j == 0) {
    *scale_out = scale;
    *sum_out = total;
  }
}

// inv = 1 / sqrt(sum(x^2) / n + eps) of rms_norm_avx2 (layers.rs:325-376)
// for the row staged in LDS at xs (visible to the whole 256-thread block),
// returned to every thread.  n % 8 == 0.  The sum of squares runs as the
// reference's 16 FMA chains (lane c: j = c & 7 over the elements
// 16i + (c < 8 ? 0 : 8) + j, the trailing 8-block into chains 0..7), then
// lane-wise sq0 + sq1 and hsum8 (no scalar tail when n % 8 == 0).
__device__ __forceinline__ float rmsnorm_inv_block(const float *xs, int n, float eps) {
  __shared__ float chains[16];
  __shared__ float inv_sh;
  const int tid = threadIdx.x;
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
    const float sum = ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
    // Correctly rounded sqrt and divide (the reference's sqrtss / divss).
    inv_sh = 1.0f / __builtin_sqrtf(sum / (float)n + eps);
  }
  __syncthreads();
  return inv_sh;
}

// rms_norm_avx2 of one row followed by the per-group quantization of the
// normalised row (gemm.rs:147-374), by a 256-thread block; out =
// (x * inv) * w.  xs: LDS scratch of n floats; n % 8 == 0, GS | n.
// Group g goes to qs + g * qstr (block-split order), qn + g * GS (natural,
// may be null), scale_out[g], sum_out[g]; nrow (may be null) receives the
// normalised row.  Ends without a barrier: the caller synchronises before
// reading the outputs.
template <int GS>
__device__ __forceinline__ void rmsnorm_quant_block(const float *__restrict__ row, const float *__restrict__ w,
                                                    int n, float eps, float *xs, int8_t *qs, int qstr,
                                                    int8_t *qn, float *scale_out, float *sum_out,
                                                    float *__restrict__ nrow, _Float16 *qa = nullptr,
                                                    int token = 0) {
  const int tid = threadIdx.x;
  for (int i = tid; i < n / 4; i += 256)
    reinterpret_cast<float4 *>(xs)[i] = reinterpret_cast<const float4 *>(row)[i];
  __syncthreads();
  const float inv = rmsnorm_inv_block(xs, n, eps);
  const int groups = n / GS;
  constexpr int NB = GS / 8;
  // 8 lanes per group; every lane of a wave iterates the same number of
  // times so the group shuffles always see all 64 lanes.
  const int passes = (groups + 31) / 32;
  for (int p = 0; p < passes; ++p) {
    const int g = p * 32 + tid / 8;
    const int j = tid & 7;
    const bool ok = g < groups;
    const int col0 = (ok ? g : 0) * GS;
    float v[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      const int col = col0 + 8 * c + j;
      v[c] = ok ? (xs[col] * inv) * w[col] : 0.0f;
      if (ok && nrow) nrow[col] = v[c];
    }
    quantize_group8_to<NB>(v, j, ok, qs + (size_t)(ok ? g : 0) * qstr, qn ? qn + col0 : nullptr,
                           scale_out + (ok ? g : 0), sum_out + (ok ? g : 0),
                           qa ? qa4_slot(qa, token, ok ? g : 0, groups) : nullptr);
  }
}

// The same for a row of at most 32 * P groups whose values a kernel loads
// into registers before anything else (rmsnorm_regs_load), so that waiting
// for them never waits for the loads issued after them: slot (p, c) of the
// thread is column 8c + (tid & 7) of group 32p + tid / 8 (clamped to the
// last group past the row).
template <int GS, int P>
__device__ __forceinline__ void rmsnorm_regs_load(const float *__restrict__ row, const float *__restrict__ w,
                                                  int n, float (&xr)[P][GS / 8], float (&wr)[P][GS / 8]) {
  const int tid = threadIdx.x, groups = n / GS;
  // The row first: the sum of squares waits only for it.
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int g = min(p * 32 + tid / 8, groups - 1);
#pragma unroll
    for (int c = 0; c < GS / 8; ++c) xr[p][c] = row[g * GS + 8 * c + (tid & 7)];
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int g = min(p * 32 + tid / 8, groups - 1);
#pragma unroll
    for (int c = 0; c < GS / 8; ++c) wr[p][c] = w[g * GS + 8 * c + (tid & 7)];
  }
}

// Per-group quantization (as k_quant) of a row of at most 32 * P groups held
// in registers in rmsnorm_regs_load's slots; xr_only loads them.
template <int GS, int P>
__device__ __forceinline__ void xr_only(const float *__restrict__ row, int n, float (&xr)[P][GS / 8]) {
  const int tid = threadIdx.x, groups = n / GS;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int g = min(p * 32 + tid / 8, groups - 1);
#pragma unroll
    for (int c = 0; c < GS / 8; ++c) xr[p][c] = row[g * GS + 8 * c + (tid & 7)];
  }
}

template <int GS, int P>
__device__ __forceinline__ void quant_regs(const float (&xr)[P][GS / 8], int n, int8_t *qs, int qstr,
                                           float *scale_out, float *sum_out) {
  const int tid = threadIdx.x, groups = n / GS, j = tid & 7;
  constexpr int NB = GS / 8;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int g = p * 32 + tid / 8;
    const bool ok = g < groups;
    quantize_group8_to<NB>(xr[p], j, ok, qs + (size_t)(ok ? g : 0) * qstr, nullptr, scale_out + (ok ? g : 0),
                           sum_out + (ok ? g : 0));
  }
}

// Maximum of a wave: DPP moves within rows of 16 lanes (xor 1, xor 2, half
// mirror, mirror), then the four row maxima by lane reads.
template <int CTRL>
__device__ __forceinline__ float max_dpp(float x) {
  const int xi = __float_as_int(x);
  return fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(xi, xi, CTRL, 0xF, 0xF, false)));
}

__device__ __forceinline__ float wave_max_dpp(float x) {
  x = max_dpp<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x = max_dpp<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x = max_dpp<0x141>(x);  // row_half_mirror
  x = max_dpp<0x140>(x);  // row_mirror
  const int xi = __float_as_int(x);
  return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(xi, 0)), __int_as_float(__builtin_amdgcn_readlane(xi, 16))),
               fmaxf(__int_as_float(__builtin_amdgcn_readlane(xi, 32)), __int_as_float(__builtin_amdgcn_readlane(xi, 48))));
}

// Chain-major scratch for rms_norm_avx2's sum of squares: chain c (0..15)
// takes the elements c, c + 16, c + 32, ... (the trailing 8-block of an
// odd n / 8 goes to chains 0..7 as their last element), so row c of the
// scratch holds exactly chain c's elements in order.  The row stride is
// 4 mod 64 floats, so the 16 chain lanes' 16-byte reads hit distinct banks.
__host__ __device__ constexpr int rms_t_stride(int n) { return 64 * ((n / 16 + 1 - 4 + 63) / 64) + 4; }
__host__ __device__ constexpr int rms_scratch_floats(int n) { return 16 * rms_t_stride(n); }

// The 16 sum-of-squares chains of a row of n = 1024 K elements (chains of
// 64 K, no trailing 8-block) from registers, in the first wave: lane 4c + q
// holds segment q (16 K elements) of chain c; phase q runs every lane's
// segment as one FMA chain (only the segment-q lanes carry a live chain),
// then DPP row_shr:1 moves each chain to its next segment's lane, so no LDS
// read sits between the dependent FMAs.  Returns hsum8(sq0 + sq1) on every
// lane of the wave.
template <int K>
__device__ __forceinline__ float rms_sumsq_regs(const float *xt, int stride) {
  constexpr int SEG = 16 * K;
  const int tid = threadIdx.x, c = tid >> 2, q = tid & 3;
  const float4 *src = reinterpret_cast<const float4 *>(xt + c * stride + SEG * q);
  float4 r[SEG / 4];
#pragma unroll
  for (int g = 0; g < SEG / 4; ++g) r[g] = src[g];
  float a = 0.0f;
#pragma unroll
  for (int ph = 0; ph < 4; ++ph) {
#pragma unroll
    for (int g = 0; g < SEG / 4; ++g) {
      a = __fmaf_rn(r[g].x, r[g].x, a);
      a = __fmaf_rn(r[g].y, r[g].y, a);
      a = __fmaf_rn(r[g].z, r[g].z, a);
      a = __fmaf_rn(r[g].w, r[g].w, a);
    }
    if (ph < 3) {
      const int ai = __float_as_int(a);
      const float moved = __int_as_float(__builtin_amdgcn_update_dpp(ai, ai, 0x111, 0xF, 0xF, false));
      a = q == ph + 1 ? moved : a;
    }
  }
  float ch[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) ch[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 4 * k + 3));
  float s[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = ch[j] + ch[8 + j];
  return ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
}

// inv of rms_norm_avx2 from the chain-major scratch (all 256 threads call;
// every thread gets inv).  Rows of 1024 K elements (K <= P) take
// rms_sumsq_regs; otherwise each chain lane streams its row with 16-byte
// reads kept 32 elements ahead of its FMA chain.
template <int P>
__device__ __forceinline__ float rmsnorm_inv_t(const float *xt, int n, float eps) {
  __shared__ float chains[16];
  __shared__ float inv_sh;
  const int tid = threadIdx.x;
  const int c16 = (n / 8) / 2;
  const bool extra8 = 16 * c16 + 8 <= n;
  const int stride = rms_t_stride(n);
  if (n % 1024 == 0 && n <= 1024 * P && n <= 4096) {
    if (tid < 64) {
      const int k = n / 1024;
      const float sum = k == 1 ? rms_sumsq_regs<1>(xt, stride)
                      : k == 2 ? rms_sumsq_regs<2>(xt, stride)
                      : k == 3 ? rms_sumsq_regs<3>(xt, stride)
                               : rms_sumsq_regs<4>(xt, stride);
      // Correctly rounded sqrt and divide (the reference's sqrtss / divss).
      if (tid == 0) inv_sh = 1.0f / __builtin_sqrtf(sum / (float)n + eps);
    }
    __syncthreads();
    return inv_sh;
  }
  if (tid < 16) {
    const float *row = xt + tid * stride;
    const int len = c16 + ((tid < 8 && extra8) ? 1 : 0);
    float a = 0.0f;
    int i = 0;
    if (len >= 32) {
      float4 cur[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = reinterpret_cast<const float4 *>(row)[u];
      for (; i + 32 <= len; i += 32) {
        float4 nxt[8];
        const bool more = i + 64 <= len;
#pragma unroll
        for (int u = 0; u < 8; ++u) nxt[u] = reinterpret_cast<const float4 *>(row + (more ? i + 32 : i))[u];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          a = __fmaf_rn(cur[u].x, cur[u].x, a);
          a = __fmaf_rn(cur[u].y, cur[u].y, a);
          a = __fmaf_rn(cur[u].z, cur[u].z, a);
          a = __fmaf_rn(cur[u].w, cur[u].w, a);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
      }
    }
    for (; i < len; ++i) a = __fmaf_rn(row[i], row[i], a);
    chains[tid] = a;
  }
  __syncthreads();
  if (tid == 0) {
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = chains[j] + chains[8 + j];
    const float sum = ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
    // Correctly rounded sqrt and divide (the reference's sqrtss / divss).
    inv_sh = 1.0f / __builtin_sqrtf(sum / (float)n + eps);
  }
  __syncthreads();
  return inv_sh;
}

// rms_norm_avx2 + quantization of a row held in rmsnorm_regs_load's slots
// (x and the norm weights) by a 256-thread block; xs: LDS scratch of
// rms_scratch_floats(n) floats, 16-byte aligned.  Optional outputs: the
// natural-order codes qn, the normalised row nrow and the matrix-core slots
// of token `token` in qa (group 32).
template <int GS, int P>
__device__ __forceinline__ void rmsnorm_quant_regs(const float (&xr)[P][GS / 8], const float (&wr)[P][GS / 8],
                                                   int n, float eps, float *xs, int8_t *qs, int qstr,
                                                   float *scale_out, float *sum_out, int8_t *qn = nullptr,
                                                   float *nrow = nullptr, _Float16 *qa = nullptr,
                                                   int token = 0) {
  const int tid = threadIdx.x, groups = n / GS, j = tid & 7;
  constexpr int NB = GS / 8;
  const int stride = rms_t_stride(n);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int g = p * 32 + tid / 8;
    if (g < groups) {
#pragma unroll
      for (int c = 0; c < NB; ++c) {
        const int col = g * GS + 8 * c + j;
        xs[(col & 15) * stride + (col >> 4)] = xr[p][c];
      }
    }
  }
  __syncthreads();
  const float inv = rmsnorm_inv_t<P>(xs, n, eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int g = p * 32 + tid / 8;
    const bool ok = g < groups;
    float v[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      v[c] = ok ? (xr[p][c] * inv) * wr[p][c] : 0.0f;
      if (ok && nrow) nrow[g * GS + 8 * c + j] = v[c];
    }
    quantize_group8_to<NB>(v, j, ok, qs + (size_t)(ok ? g : 0) * qstr, qn ? qn + (ok ? g : 0) * GS : nullptr,
                           scale_out + (ok ? g : 0), sum_out + (ok ? g : 0),
                           qa ? qa4_slot(qa, token, ok ? g : 0, groups) : nullptr);
  }
}

}  // namespace rai

#endif
