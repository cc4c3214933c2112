// Sparse-MLP (mixture-of-experts) block on the device: the MoE arm of
// mlp_block (model.rs:208-261) for m tokens with no host round trip, so a
// verify step that crosses a sparse layer stays one stream of launches.
//
//   k_router_logits_r, k_router64 / k_router (kernels.hip)
//                           router logits, softmax over all experts, top-k
//                           by selection (route_experts, layers.rs:1808-1870)
// Group 32 with the experts' gate|up stored as one matrix: entry t * K + k
// is slot k of token t, with no plan -
//   k_w4a8_dec (decode_gemv.hip), one grid row per entry: the block reads
//                           its expert from the router's picks (an empty
//                           slot leaves), gate|up against the token's row
//   k_silu_quant (fused.hip) over the entries
//   k_w4a8_dec              down, against the entry's row
//   k_moe_combine_sel       out = sum over slots, in slot order from +0, of
//                           fl(weight * expert value), then hidden += out
// Otherwise, entries grouped by expert -
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
//   k_moe_combine           as k_moe_combine_sel through the plan's entry rows
//
// Each entry's arithmetic is the one-token W4A8 arithmetic (matmul ==
// matvec, gemm.rs:1774-1919), so the grouping changes no bit.
#include <hip/hip_runtime.h>

#include <algorithm>
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
                                                   int *__restrict__ ent_tok, int *__restrict__ ent_exp) {
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
      if (ent_exp) ent_exp[row] = e;
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
// of matrix `mat` of expert e, against the expert's entries MT at a time;
// the block stages those entries' quantized rows, scales and sums in LDS
// (dynamic, MT * (cols + 8 * groups) bytes) and reads them as broadcasts.
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
  extern __shared__ __align__(16) unsigned char lact[];
  const int e = blockIdx.y;
  const int b0 = off[e], cnt = off[e + 1] - b0;
  if (cnt == 0) return;
  const int groups = cols / GS, nch = groups / CH;
  int8_t *lq = reinterpret_cast<int8_t *>(lact);
  float *lsc = reinterpret_cast<float *>(lact + (size_t)MT * cols);
  float *lsu = lsc + MT * groups;
  const int rr = min(blockIdx.x * 64 + (int)threadIdx.x, nmat * rows - 1);
  const bool live = blockIdx.x * 64 + (int)threadIdx.x < nmat * rows;
  const int mat = rr / rows, r = rr - mat * rows;
  // Buffer reads (the table's pointers would otherwise become flat reads,
  // whose completion the LDS reads of the staged entries would wait for).
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t rcs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(nibp[e * nmat + mat]), 0, rows * (cols / 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rps = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(parp[e * nmat + mat]), 0, rows * groups * 4, 0x00020000);
  const int vc = r * (cols / 2), vp = r * groups * 4;
  for (int t0 = 0; t0 < cnt; t0 += MT) {
    const int mt = min(MT, cnt - t0);
    __syncthreads();  // the previous chunk's entries are no longer read
    for (int i = threadIdx.x; i < mt * (cols / 16); i += blockDim.x) {
      const int t = i / (cols / 16), c = i % (cols / 16);
      reinterpret_cast<uint4 *>(lq + (size_t)t * cols)[c] =
          reinterpret_cast<const uint4 *>(q + (size_t)(b0 + t0 + t) * cols)[c];
    }
    for (int i = threadIdx.x; i < mt * groups; i += blockDim.x) {
      const int t = i / groups, g = i % groups;
      lsc[i] = sc[(size_t)(b0 + t0 + t) * groups + g];
      lsu[i] = su[(size_t)(b0 + t0 + t) * groups + g];
    }
    __syncthreads();
    float f[MT][NL], zc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      zc[t] = 0.0f;
#pragma unroll
      for (int l = 0; l < NL; ++l) f[t][l] = 0.0f;
    }
    u4 cn[8];
    uint32_t pn[CH];
#pragma unroll
    for (int v = 0; v < 8; ++v) cn[v] = __builtin_amdgcn_raw_buffer_load_b128(rcs, vc, 16 * v, 0);
#pragma unroll
    for (int g = 0; g < CH; ++g) pn[g] = __builtin_amdgcn_raw_buffer_load_b32(rps, vp, 4 * g, 0);
    for (int c = 0; c < nch; ++c) {
      u4 cc[8];
      uint32_t pc[CH];
#pragma unroll
      for (int v = 0; v < 8; ++v) cc[v] = cn[v];
#pragma unroll
      for (int g = 0; g < CH; ++g) pc[g] = pn[g];
      const int cnx = min(c + 1, nch - 1);
#pragma unroll
      for (int v = 0; v < 8; ++v) cn[v] = __builtin_amdgcn_raw_buffer_load_b128(rcs, vc, (cnx * 8 + v) * 16, 0);
#pragma unroll
      for (int g = 0; g < CH; ++g) pn[g] = __builtin_amdgcn_raw_buffer_load_b32(rps, vp, (cnx * CH + g) * 4, 0);
      const uint32_t *cw = reinterpret_cast<const uint32_t *>(cc);
#pragma unroll
      for (int gi = 0; gi < CH; ++gi) {
        const int g = c * CH + gi;
        const float ws = half_bits(pc[gi] & 0xFFFFu), wz = half_bits(pc[gi] >> 16);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t < mt) {
            const uint2 *qv = reinterpret_cast<const uint2 *>(lq + (size_t)t * cols + (size_t)g * GS);
            int sl[NL];
#pragma unroll
            for (int l = 0; l < NL; ++l) sl[l] = 0;
#pragma unroll
            for (int b = 0; b < NW; ++b) {
              const uint2 a = qv[b];
              sl[b % NL] = blk_dot(cw[gi * NW + b], a.x, a.y, sl[b % NL]);
            }
            const float cs = ws * lsc[t * groups + g];
#pragma unroll
            for (int l = 0; l < NL; ++l) f[t][l] = f[t][l] + (float)sl[l] * cs;
            zc[t] = zc[t] + wz * lsu[t * groups + g];
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < mt && live) {
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

// The same sum with the entries in (token, slot) order (entry t * K + k is
// slot k of token t; the slots past the router's last pick hold -1): the
// slots' weights and expert values are loaded eight at a time before the
// sum, which then runs in slot order from +0.
__global__ void k_moe_combine_sel(float *__restrict__ hid, const float *__restrict__ eo,
                                  const float *__restrict__ wts, const int *__restrict__ sel, int K, int H) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  float acc = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 8) {
    const int nk = min(8, K - k0);
    bool ok[8];
    float w[8], v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = t * K + k0 + min(j, nk - 1);
      ok[j] = j < nk && sel[i] >= 0;
      w[j] = wts[i];
      v[j] = eo[(size_t)i * H + c];
    }
    // The slots with a pick come first; the sum stops at the first empty one.
    int run = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (run == j && ok[j]) ++run;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < run) acc = acc + w[j] * v[j];
    if (run < nk) break;
  }
  hid[(size_t)t * H + c] = hid[(size_t)t * H + c] + acc;
}

}  // namespace

bool moe_device_path(int hidden, int ffn, int gs, int experts) {
  // The staged entries (8 rows of int8 plus scales and sums) must fit the
  // 64 KB of LDS a block may use without an opt-in.
  return (gs == 32 || gs == 64 || gs == 128) && experts >= 1 && experts <= 1024 && hidden % 256 == 0 &&
         ffn % 256 == 0 && (size_t)8 * (std::max(hidden, ffn) + 8 * (std::max(hidden, ffn) / gs)) <= 65536;
}

void launch_moe_plan(const int *sel, int m, int K, int E, int *off, int *ent_of, int *ent_tok, int *ent_exp,
                     hipStream_t s) {
  hipLaunchKernelGGL(k_moe_plan, dim3(1), dim3(1024), sizeof(int) * (E + 1), s, sel, m * K, K, E, off, ent_of,
                     ent_tok, ent_exp);
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
  const size_t lds = (size_t)8 * (cols + 8 * (cols / gs));
  if (gs == 32)
    hipLaunchKernelGGL((k_moe_gemv<32, 8>), grid, dim3(64), lds, s, out, ld, nibp, parp, nmat, rows, cols, q, sc, su,
                       off);
  else if (gs == 64)
    hipLaunchKernelGGL((k_moe_gemv<64, 8>), grid, dim3(64), lds, s, out, ld, nibp, parp, nmat, rows, cols, q, sc, su,
                       off);
  else
    hipLaunchKernelGGL((k_moe_gemv<128, 8>), grid, dim3(64), lds, s, out, ld, nibp, parp, nmat, rows, cols, q, sc, su,
                       off);
}

void launch_moe_combine(float *hid, const float *eo, const float *wts, const int *ent_of, int m, int K, int H,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_moe_combine, dim3((H + 255) / 256, m), dim3(256), 0, s, hid, eo, wts, ent_of, K, H);
}

void launch_moe_combine_sel(float *hid, const float *eo, const float *wts, const int *sel, int m, int K, int H,
                            hipStream_t s) {
  hipLaunchKernelGGL(k_moe_combine_sel, dim3((H + 255) / 256, m), dim3(256), 0, s, hid, eo, wts, sel, K, H);
}

}  // namespace rai
