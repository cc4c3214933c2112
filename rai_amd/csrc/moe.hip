// Sparse-MLP (mixture-of-experts) block on the device: the MoE arm of
// mlp_block (model.rs:208-261) for m tokens with no host round trip, so a
// verify step that crosses a sparse layer stays one stream of launches.
//
//   k_router (kernels.hip)  softmax over all experts, top-k by selection
//                           (route_experts, layers.rs:1808-1870)
//   k_moe_plan              per-expert entry counts and offsets; entry
//                           (token, slot) pairs listed expert by expert
//   k_moe_gather            the token's quantized input row, scales and sums
//                           copied to its entries (the quantization is a
//                           function of the row, so every expert sees the
//                           bytes the reference's per-call quantization gives)
//   k_moe_gemv              one launch per projection over every expert that
//                           has entries: a block's rows of that expert's
//                           matrix against all of its entries (gate and up
//                           share a launch)
//   k_silu_quant (fused.hip) over the entries
//   k_moe_combine           out = sum over slots, in slot order from +0, of
//                           fl(weight * expert value), then hidden += out
//
// Each entry's arithmetic is the one-token W4A8 arithmetic (matmul ==
// matvec, gemm.rs:1774-1919), so the grouping changes no bit.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace rai {

namespace {

__device__ __forceinline__ float half_bits(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// 8-column block dot of the reference (gemm.rs:470-476): low nibbles with
// the even activations, high nibbles with the odd ones.
__device__ __forceinline__ int blk_dot(uint32_t codes, uint32_t q_even, uint32_t q_odd, int acc) {
  const uint32_t lo = codes & 0x0F0F0F0Fu, hi = (codes >> 4) & 0x0F0F0F0Fu;
  acc = __builtin_amdgcn_sdot4((int)lo, (int)q_even, acc, false);
  return __builtin_amdgcn_sdot4((int)hi, (int)q_odd, acc, false);
}

// One block; entries i = t * K + k with sel[i] >= 0.  off[0..E] are the
// exclusive prefix sums of the per-expert counts; ent_of[i] the entry row of
// (t, k) (-1 when the slot is empty); ent_tok[row] its token.
__global__ __launch_bounds__(1024) void k_moe_plan(const int *__restrict__ sel, int n, int K, int E,
                                                   int *__restrict__ off, int *__restrict__ ent_of,
                                                   int *__restrict__ ent_tok) {
  extern __shared__ int cnt[];  // E + 1
  for (int e = threadIdx.x; e <= E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int e = sel[i];
    ent_of[i] = (e >= 0 && e < E) ? atomicAdd(&cnt[e], 1) : -1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      const int c = cnt[e];
      cnt[e] = run;
      off[e] = run;
      run += c;
    }
    off[E] = run;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int e = sel[i];
    if (e >= 0 && e < E) {
      const int row = cnt[e] + ent_of[i];
      ent_of[i] = row;
      ent_tok[row] = i / K;
    }
  }
}

// Entry rows past off[E] are left as they are (never read back).
__global__ void k_moe_gather(const int8_t *__restrict__ q, const float *__restrict__ sc,
                             const float *__restrict__ su, const int *__restrict__ ent_tok,
                             const int *__restrict__ off, int E, int cols, int groups, int8_t *__restrict__ qg,
                             float *__restrict__ scg, float *__restrict__ sug) {
  const int row = blockIdx.y;
  if (row >= off[E]) return;
  const int t = ent_tok[row];
  const int n16 = cols / 16;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n16 + 2 * groups; i += gridDim.x * blockDim.x) {
    if (i < n16) {
      reinterpret_cast<uint4 *>(qg + (size_t)row * cols)[i] = reinterpret_cast<const uint4 *>(q + (size_t)t * cols)[i];
    } else if (i < n16 + groups) {
      scg[(size_t)row * groups + i - n16] = sc[(size_t)t * groups + i - n16];
    } else {
      sug[(size_t)row * groups + i - n16 - groups] = su[(size_t)t * groups + i - n16 - groups];
    }
  }
}

// Grid: x = row blocks of 64 over nmat * rows, y = expert.  Thread = one row
// of matrix `mat` of expert e, against the expert's entries MT at a time.
// Lane sums as the reference's accumulators: group 32 uses 4 lanes (the
// 16-byte block32 path, gemm.rs:616-637), groups 64 and 128 use 8 lanes
// (the 32-byte chunk path, blocks b and b + 8 share lane b % 8).  Codes and
// parameters are read CH groups (128 bytes of codes) at a time, one chunk
// ahead.
template <int GS, int MT>
__global__ __launch_bounds__(64) void k_moe_gemv(float *__restrict__ out, int ld,
                                                 const uint8_t *const *__restrict__ nibp,
                                                 const uint8_t *const *__restrict__ parp, int nmat, int rows,
                                                 int cols, const int8_t *__restrict__ q,
                                                 const float *__restrict__ sc, const float *__restrict__ su,
                                                 const int *__restrict__ off) {
  constexpr int NL = GS == 32 ? 4 : 8;
  constexpr int NW = GS / 8;          // code dwords per group
  constexpr int CH = 128 / (GS / 2);  // groups per 128-byte chunk
  const int e = blockIdx.y;
  const int b0 = off[e], cnt = off[e + 1] - b0;
  if (cnt == 0) return;
  const int rr = blockIdx.x * 64 + threadIdx.x;
  if (rr >= nmat * rows) return;
  const int mat = rr / rows, r = rr - mat * rows;
  const int groups = cols / GS, nch = groups / CH;
  const uint4 *crow = reinterpret_cast<const uint4 *>(nibp[e * nmat + mat] + (size_t)r * (cols / 2));
  const uint32_t *prow = reinterpret_cast<const uint32_t *>(parp[e * nmat + mat] + (size_t)r * groups * 4);
  for (int t0 = 0; t0 < cnt; t0 += MT) {
    const int mt = min(MT, cnt - t0);
    float f[MT][NL], zc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      zc[t] = 0.0f;
#pragma unroll
      for (int l = 0; l < NL; ++l) f[t][l] = 0.0f;
    }
    uint4 cn[8];
    uint32_t pn[CH];
#pragma unroll
    for (int v = 0; v < 8; ++v) cn[v] = crow[v];
#pragma unroll
    for (int g = 0; g < CH; ++g) pn[g] = prow[g];
    for (int c = 0; c < nch; ++c) {
      uint4 cc[8];
      uint32_t pc[CH];
#pragma unroll
      for (int v = 0; v < 8; ++v) cc[v] = cn[v];
#pragma unroll
      for (int g = 0; g < CH; ++g) pc[g] = pn[g];
      const int cnx = min(c + 1, nch - 1);
#pragma unroll
      for (int v = 0; v < 8; ++v) cn[v] = crow[cnx * 8 + v];
#pragma unroll
      for (int g = 0; g < CH; ++g) pn[g] = prow[cnx * CH + g];
      const uint32_t *cw = reinterpret_cast<const uint32_t *>(cc);
#pragma unroll
      for (int gi = 0; gi < CH; ++gi) {
        const int g = c * CH + gi;
        const float ws = half_bits(pc[gi] & 0xFFFFu), wz = half_bits(pc[gi] >> 16);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t < mt) {
            const size_t er = (size_t)(b0 + t0 + t);
            const uint2 *qv = reinterpret_cast<const uint2 *>(q + er * cols + (size_t)g * GS);
            int sl[NL];
#pragma unroll
            for (int l = 0; l < NL; ++l) sl[l] = 0;
#pragma unroll
            for (int b = 0; b < NW; ++b) {
              const uint2 a = qv[b];
              sl[b % NL] = blk_dot(cw[gi * NW + b], a.x, a.y, sl[b % NL]);
            }
            const float cs = ws * sc[er * groups + g];
#pragma unroll
            for (int l = 0; l < NL; ++l) f[t][l] = f[t][l] + (float)sl[l] * cs;
            zc[t] = zc[t] + wz * su[er * groups + g];
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < mt) {
        float d;
        if (NL == 4)
          d = (f[t][0] + f[t][1]) + (f[t][2] + f[t][3]);
        else
          d = ((f[t][0] + f[t][4]) + (f[t][1] + f[t][5])) + ((f[t][2] + f[t][6]) + (f[t][3] + f[t][7]));
        out[(size_t)(b0 + t0 + t) * ld + (size_t)mat * rows + r] = d + zc[t];
      }
    }
  }
}

// hidden[t] += sum over slots k (in order, from +0) of fl(w[t][k] * eo[entry]).
__global__ void k_moe_combine(float *__restrict__ hid, const float *__restrict__ eo, const float *__restrict__ wts,
                              const int *__restrict__ ent_of, int K, int H) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int ent = ent_of[t * K + k];
    if (ent < 0) break;
    acc = acc + wts[t * K + k] * eo[(size_t)ent * H + c];
  }
  hid[(size_t)t * H + c] = hid[(size_t)t * H + c] + acc;
}

}  // namespace

bool moe_device_path(int hidden, int ffn, int gs, int experts) {
  return (gs == 32 || gs == 64 || gs == 128) && experts >= 1 && experts <= 1024 && hidden % 256 == 0 &&
         ffn % 256 == 0;
}

void launch_moe_plan(const int *sel, int m, int K, int E, int *off, int *ent_of, int *ent_tok, hipStream_t s) {
  hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(1024), sizeof(int) * (E + 1), s, sel, m * K, K, E, off, ent_of,
                     ent_tok);
}

void launch_moe_gather(const int8_t *q, const float *sc, const float *su, const int *ent_tok, const int *off, int E,
                       int max_entries, int cols, int groups, int8_t *qg, float *scg, float *sug, hipStream_t s) {
  const int items = cols / 16 + 2 * groups;
  hipLaunchKernelGGL(k_moe_gather, dim3((items + 255) / 256, max_entries), dim3(256), 0, s, q, sc, su, ent_tok, off,
                     E, cols, groups, qg, scg, sug);
}

void launch_moe_gemv(float *out, int ld, const uint8_t *const *nibp, const uint8_t *const *parp, int nmat, int rows,
                     int cols, int gs, int E, const int8_t *q, const float *sc, const float *su, const int *off,
                     hipStream_t s) {
  const dim3 grid((nmat * rows + 63) / 64, E);
  if (gs == 32)
    hipLaunchKernelGGL((k_moe_gemv<32, 8>), grid, dim3(64), 0, s, out, ld, nibp, parp, nmat, rows, cols, q, sc, su,
                       off);
  else if (gs == 64)
    hipLaunchKernelGGL((k_moe_gemv<64, 8>), grid, dim3(64), 0, s, out, ld, nibp, parp, nmat, rows, cols, q, sc, su,
                       off);
  else
    hipLaunchKernelGGL((k_moe_gemv<128, 8>), grid, dim3(64), 0, s, out, ld, nibp, parp, nmat, rows, cols, q, sc, su,
                       off);
}

void launch_moe_combine(float *hid, const float *eo, const float *wts, const int *ent_of, int m, int K, int H,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_moe_combine, dim3((H + 255) / 256, m), dim3(256), 0, s, hid, eo, wts, ent_of, K, H);
}

}  // namespace rai
