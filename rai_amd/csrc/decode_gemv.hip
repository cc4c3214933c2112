// One-token W4A8 GEMV (decode), group 32, wave-streamed.
//
// Same arithmetic as the reference's AVX2 kernel for one input row
// (gemm.rs:458-537, 1774-1919): per (row, group) the four 8-column block
// sums S_l (exact int32 via v_dot4), cs = fl(ws * as), the lane products
// fl(float(S_l) * cs) and the zero term fl(wz * xsum); per row four lane
// chains and one zero chain accumulated in group order, and at the end
// hsum8(f0..f3, 0, 0, 0, 0) + zc.
//
// Work split.  Every wave owns tiles of R rows and walks them chunk by chunk
// (32 groups = 1024 columns per chunk).  Lane (h = lane / 32, k = lane % 32)
// holds group k of the chunk for the R/2 rows 2i + h, so one load
// instruction reads two 512-byte runs of packed codes and two 128-byte runs
// of group parameters.  Loads stream through a ring of D chunks in
// registers: every load is issued (past the last chunk it points beyond the
// buffer, which a raw buffer load answers with zeros without touching
// memory), so the compiler's wait counts stay exact and D chunks stay in
// flight across tile boundaries.  The lane products go through a
// wave-private LDS area (two buffers) and come back transposed: lane
// c = l * R + r runs chain l of row r over the chunk's 32 products in group
// order, one chunk behind the products, so the chain's dependent adds
// interleave with the next chunk's product instructions.  No block
// barrier is taken after the prologue, which stages the activations
// (int8 codes in the block-split order, scales and sums; ST = 1, 2, 4
// sixteen-byte loads of codes per thread) once per block - or quantizes the
// f32 input row there (ST = 8, quantize_input_split), or, with the fused
// input RMSNorm (ST = 0), normalises and quantizes the hidden row (rms_norm_avx2 then quantize_input_split, layers.rs:325-376,
// gemm.rs:147-374).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "exact_math.h"
#include "kernels.h"
#include "quant_dev.h"

namespace rai {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kDecWaves = 4;       // waves per block
constexpr int kDecChunk = 32;      // groups per chunk
constexpr int kDecRowStride = 36;  // floats per (chain, row) run of 32 products, padded
constexpr int kDecMaxGroups = 448; // K <= 14336 staged in LDS

__device__ __forceinline__ float dec_f16(uint32_t bits) {
  return __half2float(__ushort_as_half((uint16_t)bits));
}

// Integer dot of one 8-column block: low nibbles (even columns) against the
// 4 even activations, high nibbles against the 4 odd ones (the PMADDUBSW
// pairing of gemm.rs:470-476).
__device__ __forceinline__ int dec_block_dot(uint32_t codes, uint32_t q_even, uint32_t q_odd) {
  const uint32_t lo = codes & 0x0F0F0F0Fu;
  const uint32_t hi = (codes >> 4) & 0x0F0F0F0Fu;
  return __builtin_amdgcn_sdot4((int)hi, (int)q_odd, __builtin_amdgcn_sdot4((int)lo, (int)q_even, 0, false),
                                false);
}

template <int R>
struct DecCfg {
  static_assert(R % 2 == 0 && 5 * R <= 64, "one chain per lane");
  static constexpr int IPL = R / 2;                    // (row, group) items per lane and chunk
  static constexpr int LSTR = R * kDecRowStride;       // floats per chain
  static constexpr int WAVE_FLOATS = 10 * LSTR + 64;   // two product buffers + final chain values
};

// LDS bytes of a block: activations (codes, scales, sums) and the waves'
// product areas; with the fused RMSNorm the product areas double as the
// norm's chain-major row scratch.
__host__ __device__ inline int dec_act_bytes(int cols) { return (cols + 8 * (cols / 32) + 15) & ~15; }

template <int R>
size_t dec_smem(int cols, bool fused) {
  const size_t act = dec_act_bytes(cols);
  const size_t waves = sizeof(float) * (size_t)kDecWaves * DecCfg<R>::WAVE_FLOATS;
  return act + std::max(waves, fused ? sizeof(float) * (size_t)rms_scratch_floats(cols) : size_t(0));
}

constexpr int kEpiPlain = 0, kEpiGlu = 1, kEpiRope = 2, kEpiMoe = 3, kEpiMoeGlu = 4;

// rope_store of one rotation pair (x0 at head element i, x1 at i + hd/2)
// as k_rope_store does it (layers.rs:561-726): q and k rotated in the qkv
// output, k also into the K cache row of the position, v unrotated into
// the d-major V cache.  Row index r of the stacked [q; k; v] output.
__device__ __forceinline__ void rope_store_pair(const DecRope &rp, float *out, int r, int pos, float c, float sn,
                                                float x0, float x1) {
  const int hd = rp.hd, half = hd / 2, body = (half / 8) * 8;
  const int head = r / hd, i = r - head * hd;
  float r0 = x0, r1 = x1;
  if (head < rp.nh + rp.nkv) {
    if (i < body) {
      r0 = __fmaf_rn(x0, c, -(x1 * sn));
      r1 = __fmaf_rn(x1, c, x0 * sn);
    } else {
      r0 = x0 * c - x1 * sn;
      r1 = x1 * c + x0 * sn;
    }
  }
  out[r] = r0;
  out[r + half] = r1;
  if (head >= rp.nh && head < rp.nh + rp.nkv) {
    const size_t dst = ((size_t)(head - rp.nh) * rp.cap + pos) * hd;
    rp.kc[dst + i] = r0;
    rp.kc[dst + half + i] = r1;
  } else if (head >= rp.nh + rp.nkv) {
    float *vd = rp.vc + (size_t)(head - rp.nh - rp.nkv) * hd * rp.vstride + pos;
    vd[(size_t)i * rp.vstride] = r0;
    vd[(size_t)(half + i) * rp.vstride] = r1;
  }
}

template <int R, int D, int ST, int EPI>
__global__ __launch_bounds__(256) void k_w4a8_dec(float *out, const float *add, const uint8_t *__restrict__ nib,
                                                  const uint8_t *__restrict__ params,
                                                  const int8_t *__restrict__ q_split,
                                                  const float *__restrict__ scales,
                                                  const float *__restrict__ sums, int rows, int cols,
                                                  int tiles_per_wave, const float *__restrict__ nx,
                                                  const float *__restrict__ nw, float eps, DecRope rope,
                                                  DecMoe moe) {
  using C = DecCfg<R>;
  constexpr int IPL = C::IPL, LSTR = C::LSTR;
  // MOE: one grid row per MoE entry; GLU: the block's gate|up output group
  // through silu_mul and its quantization (both for an entry's experts).
  constexpr bool MOE = EPI == kEpiMoe || EPI == kEpiMoeGlu, GLU = EPI == kEpiGlu || EPI == kEpiMoeGlu;
  constexpr bool ROPE = EPI == kEpiRope;
  static_assert(EPI != kEpiGlu || (R == 8 && ST == 0), "a gate|up block: 4 waves x 8 rows, fused input norm");
  static_assert(EPI != kEpiMoeGlu || R == 8, "an entry's gate|up block: 4 waves x 8 rows");
  static_assert(!ROPE || R == 8, "a rope tile: 4 rows of each half of a head");
  static_assert(!MOE || (ST >= 1 && ST <= 4), "an entry row: quantized activations staged from memory");
  extern __shared__ __align__(16) unsigned char smem[];
  const int groups = cols / 32;
  if constexpr (MOE) {
    // Grid row = MoE entry (token, slot): its expert's matrix, its
    // activation row and its output row (the whole block leaves together
    // for an empty slot).
    const int ent = blockIdx.y;
    const int x = moe.sel[ent];
    if (x < 0 || x >= moe.E) return;
    nib = moe.nib_tab[(size_t)x * moe.tstride];
    params = moe.par_tab[(size_t)x * moe.tstride];
    const int ar = moe.tok_rows ? ent / moe.K : ent;
    q_split += (size_t)ar * cols;
    scales += (size_t)ar * groups;
    sums += (size_t)ar * groups;
    if constexpr (EPI == kEpiMoeGlu) {
      const int fo = rows / 2;  // the entry's silu_mul row: fo values, fo / 32 groups
      moe.qo += (size_t)ent * fo;
      moe.so += (size_t)ent * (fo / 32);
      moe.uo += (size_t)ent * (fo / 32);
    } else {
      out += (size_t)ent * moe.ld;
    }
  }
  const int nchunks = (groups + kDecChunk - 1) / kDecChunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, k = lane & 31;
  // LDS: q [cols] bytes | scales [groups] | sums [groups] | waves' areas.
  int8_t *qsh = reinterpret_cast<int8_t *>(smem);
  float *ash = reinterpret_cast<float *>(smem + cols);
  float *ssh = ash + groups;
  float *wbase = reinterpret_cast<float *>(smem + dec_act_bytes(cols));
  float *pw_lds = wbase + wave * C::WAVE_FLOATS;
  float *fin = pw_lds + 10 * LSTR;

  // Wave w of W walks tiles w, w + W, ...; every wave runs the same number
  // of tiles, those past the matrix read zeros and store nothing.
  const int W = gridDim.x * kDecWaves;
  const int wg = blockIdx.x * kDecWaves + wave;
  const int it_total = tiles_per_wave * nchunks;
  const int rowb = cols / 2;
  // First row of the wave's tile t.  GLU: block b owns output group b of
  // silu(gate) * up, i.e. gate rows 32b.. (tile 0) and up rows
  // rows/2 + 32b.. (tile 1), 8 per wave.  ROPE: tile u of head u / (hd/8)
  // holds the rotation pairs (i, i + hd/2), i = 4 (u % (hd/8)) + 0..3: local
  // rows 0..3 are i, local rows 4..7 are i + hd/2.
  const int rhalf = ROPE ? rope.hd / 2 : 0;
  auto tile_row0 = [&](int t) {
    if constexpr (GLU) {
      return (t ? rows / 2 : 0) + 32 * (int)blockIdx.x + R * wave;
    } else if constexpr (ROPE) {
      const int u = wg + t * W, per = rope.hd / 8;
      return (u / per) * rope.hd + 4 * (u % per);
    } else {
      return (wg + t * W) * R;
    }
  };
  // Row offset of local row r (0..R-1) from tile_row0.
  auto lrow = [&](int r) { return (ROPE && r >= 4) ? rhalf - 4 + r : r; };
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(nib), 0, rows * rowb, 0x00020000);
  const __amdgpu_buffer_rsrc_t rp =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(params), 0, rows * groups * 4, 0x00020000);

  // Activations first (the hidden row and the norm weights, or the
  // quantized row, its scales and sums), then the weight ring: loads
  // complete in issue order, so staging the activations never waits for
  // the ring.
  // Rotation entries of the lane's pair (rope tiles: lanes 0..3, one tile
  // per wave), requested first.
  int rpos = 0;
  float rcos = 0.0f, rsin = 0.0f;
  if constexpr (ROPE) {
    rpos = rope.st ? rope.st[0] : rope.pos0;
    const int r = tile_row0(0) + min(lane, 3);
    const int i = r % rope.hd;
    const bool rot = r < rows && r / rope.hd < rope.nh + rope.nkv;
    const size_t ci = (size_t)rpos * rhalf + (rot ? i : 0);
    rcos = rope.cos_t[ci];
    rsin = rope.sin_t[ci];
  }
  constexpr bool FUSED = ST == 0, QONLY = ST == 8;
  constexpr int NP = (FUSED || QONLY) ? 4 : 1;
  constexpr int QV = (FUSED || QONLY) ? 1 : ST;
  float xr[NP][4], wr[NP][4];
  uint4 qv[QV];
  float av[2], sv[2];
  if constexpr (FUSED) {
    rmsnorm_regs_load<32, NP>(nx, nw, cols, xr, wr);
  } else if constexpr (QONLY) {
    xr_only<32, NP>(nx, cols, xr);
  } else {
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(q_split), 0, cols, 0x00020000);
#pragma unroll
    for (int v = 0; v < QV; ++v) {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rq, 16 * min(tid + v * 256, cols / 16 - 1), 0, 0);
      qv[v] = make_uint4(w.x, w.y, w.z, w.w);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      av[u] = scales[min(tid + u * 256, groups - 1)];
      sv[u] = sums[min(tid + u * 256, groups - 1)];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  u32x4 ring_c[D][IPL];
  uint32_t ring_p[D][IPL];
  // Tile and chunk of the next load; loads are issued in iteration order,
  // one chunk each.
  int lt = 0, lch = 0;
  auto load = [&](u32x4 (&c)[IPL], uint32_t (&p)[IPL]) {
    const int row = tile_row0(lt) + h;  // local row h; item i adds lrow(2i) rows
    const int g = lch * kDecChunk + k;
    uint32_t vc = (uint32_t)row * rowb + g * 16;
    uint32_t vp = ((uint32_t)row * groups + g) * 4;
    // Past the last iteration, and on the lanes past the groups of a
    // partial last chunk: zeros without a memory access.  Zero codes and
    // parameters give +0 or -0 products, which leave a chain unchanged (a
    // chain starts at +0 and a sum of floats is -0 only when both terms
    // are).
    if (lt >= tiles_per_wave || g >= groups) {
      vc = 0x80000000u;  // past num_records
      vp = 0x80000000u;
    }
    // The item offsets go into the VGPR offset: the range check covers the
    // VGPR and instruction offsets, not the SGPR one.
#pragma unroll
    for (int i = 0; i < IPL; ++i)
      c[i] = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)(vc + (uint32_t)(lrow(2 * i) * rowb)), 0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < IPL; ++i)
      p[i] = __builtin_amdgcn_raw_buffer_load_b32(rp, (int)(vp + (uint32_t)(lrow(2 * i) * 4 * groups)), 0, 0);
    if (++lch == nchunks) {
      lch = 0;
      ++lt;
    }
  };
  // Same issue order as the loop's refills (slot by slot), which keeps the
  // compiler's wait counts exact at the loop head.
#pragma unroll
  for (int j = 0; j < D; ++j) {
    load(ring_c[j], ring_p[j]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Stage the activations in LDS while the ring fills.
  if constexpr (FUSED) {
    rmsnorm_quant_regs<32, NP>(xr, wr, cols, eps, wbase, qsh, 32, ash, ssh);
  } else if constexpr (QONLY) {
    quant_regs<32, NP>(xr, cols, qsh, 32, ash, ssh);
  } else {
    // Unconditional stores to the clamped slots (threads past the row
    // rewrite the last slot with the value already there): a conditional
    // store would let the compiler sink the loads behind the ring.
#pragma unroll
    for (int v = 0; v < QV; ++v) reinterpret_cast<uint4 *>(qsh)[min(tid + v * 256, cols / 16 - 1)] = qv[v];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      ash[min(tid + u * 256, groups - 1)] = av[u];
      ssh[min(tid + u * 256, groups - 1)] = sv[u];
    }
  }
  __syncthreads();

  float acc = 0.0f, gate_v = 0.0f, up_v = 0.0f;
  // Chain lane: row crow, chain cl (lanes past the 5R chains re-read chain
  // 4 and their sums are never used).
  const int crow = lane % R, cl = min(lane / R, 4);
  const bool chain_lane = lane < 5 * R;
  const int cbase = cl * LSTR + crow * kDecRowStride;
  // Activations of the iteration's chunk (read one iteration ahead).
  uint4 q0, q1;
  float as, xsum;
  auto read_act = [&](int ch) {
    const int gq = min(ch * kDecChunk + k, groups - 1);
    q0 = *reinterpret_cast<const uint4 *>(qsh + gq * 32);
    q1 = *reinterpret_cast<const uint4 *>(qsh + gq * 32 + 16);
    as = ash[gq];
    xsum = ssh[gq];
  };
  // End of tile t: the row sums from the chain values in acc.
  auto finish = [&](int t) {
    if (chain_lane) fin[lane] = acc;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int row = tile_row0(t) + lrow(lane);
    if (lane < R && row < rows) {
      // hsum8 of (f0, f1, f2, f3, 0, 0, 0, 0) in the _mm256 order.
      const float f0 = fin[lane], f1 = fin[R + lane], f2 = fin[2 * R + lane], f3 = fin[3 * R + lane];
      const float zero = 0.0f;
      const float v = ((f0 + zero) + (f1 + zero)) + ((f2 + zero) + (f3 + zero)) + fin[4 * R + lane];
      if constexpr (GLU) {
        if (t == 0)
          gate_v = v;
        else
          up_v = v;
      } else if constexpr (ROPE) {
        fin[40 + lane] = v;
      } else {
        out[row] = add ? add[row] + v : v;
      }
    }
    if constexpr (ROPE) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (lane < 4 && tile_row0(t) < rows)
        rope_store_pair(rope, out, tile_row0(t) + lane, rpos, rcos, rsin, fin[40 + lane], fin[44 + lane]);
    }
  };

  // Pipelined by one chunk: iteration it computes chunk it's products into
  // LDS buffer it & 1 while the chain lanes add chunk it - 1's (read from
  // LDS at the end of iteration it - 1), so a chain's dependent adds issue
  // between independent product instructions.
  float4 cv[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) cv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  int ct = 0, cch = 0;   // tile and chunk of the iteration
  int pt = 0, pch = -1;  // tile and chunk of the pending chain values (none yet)
  read_act(0);
  for (int it0 = 0; it0 < it_total; it0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int it = it0 + j;
      if (it < it_total) {
        float *pb = pw_lds + (it & 1) * (5 * LSTR);
        acc = pch == 0 ? 0.0f : acc;  // a tile's chains start at its first chunk
        // Products of the lane's items, block-major in 8 slots of IPL / 2
        // block dots each, and in every slot 4 of the pending chain's adds:
        // a dependent add takes several issue slots to complete, and the
        // scheduling barriers keep the independent product work between
        // consecutive adds.
        float cs[IPL];
#pragma unroll
        for (int i = 0; i < IPL; ++i) {
          const uint32_t pw = ring_p[j][i];
          cs[i] = dec_f16(pw & 0xFFFF) * as;
          pb[4 * LSTR + (2 * i + h) * kDecRowStride + k] = dec_f16(pw >> 16) * xsum;
        }
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
#pragma unroll
          for (int e = sl * IPL / 2; e < (sl + 1) * IPL / 2; ++e) {
            const int b = e / IPL, i = e % IPL;  // block b of item i
            const u32x4 cw = ring_c[j][i];
            const uint32_t code = b == 0 ? cw.x : b == 1 ? cw.y : b == 2 ? cw.z : cw.w;
            const uint4 qq = b < 2 ? q0 : q1;
            const int sb = dec_block_dot(code, (b & 1) ? qq.z : qq.x, (b & 1) ? qq.w : qq.y);
            pb[b * LSTR + (2 * i + h) * kDecRowStride + k] = (float)sb * cs[i];
          }
          acc = acc + cv[sl].x;
          acc = acc + cv[sl].y;
          acc = acc + cv[sl].z;
          acc = acc + cv[sl].w;
          __builtin_amdgcn_sched_barrier(0);
        }
        if (pch == nchunks - 1) finish(pt);
        // LDS operations of one wave complete in order; the fences only
        // keep the compiler from moving the chain reads above the writes.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        pt = ct;
        pch = cch;
        if (++cch == nchunks) {
          cch = 0;
          ++ct;
        }
        read_act(cch);
        const float4 *pc = reinterpret_cast<const float4 *>(pb + cbase);
#pragma unroll
        for (int u = 0; u < 8; ++u) cv[u] = pc[u];
      }
      load(ring_c[j], ring_p[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // The last chunk's chain.
  acc = pch == 0 ? 0.0f : acc;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    acc = acc + cv[u].x;
    acc = acc + cv[u].y;
    acc = acc + cv[u].z;
    acc = acc + cv[u].w;
  }
  if (pch == nchunks - 1) finish(pt);
  if constexpr (GLU) {
    // silu_mul_inplace (layers.rs:850-883) of the block's 32 outputs and
    // their quantization (gemm.rs:147-374) as k_silu_quant does; the
    // quantized group goes to q_split / scales / sums, which are outputs
    // here (to the entry's row of moe.qo / so / uo for an expert).
    __syncthreads();  // every wave is done with the staged activations
    float *glu = reinterpret_cast<float *>(smem);
    if (lane < R) {
      glu[R * wave + lane] = gate_v;
      glu[32 + R * wave + lane] = up_v;
    }
    __syncthreads();
    if (wave == 0) {
      const int j = lane & 7, b = blockIdx.x;
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float xv = glu[8 * c + j];
        const float e = rai_exact::schraudolph(xv * -1.0f);
        v[c] = (xv / (1.0f + e)) * glu[32 + 8 * c + j];
      }
      if constexpr (MOE)
        quantize_group8_to<4>(v, j, lane < 8, moe.qo + 32 * b, nullptr, moe.so + b, moe.uo + b);
      else
        quantize_group8_to<4>(v, j, lane < 8, const_cast<int8_t *>(q_split) + 32 * b, nullptr,
                              const_cast<float *>(scales) + b, const_cast<float *>(sums) + b);
    }
  }
}

template <int R, int D, int ST>
void launch_dec_t(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                  const float *scales, const float *sums, int rows, int cols, const float *nx, const float *nw,
                  float eps, int blocks, hipStream_t s) {
  const size_t smem = dec_smem<R>(cols, ST == 0);  // the norm's row scratch
  static size_t configured = 0;
  if (smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_dec<R, D, ST, kEpiPlain>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  const int tiles = (rows + R - 1) / R;
  if (blocks <= 0) blocks = (tiles + kDecWaves - 1) / kDecWaves;
  blocks = std::max(1, std::min(blocks, 1024));
  const int waves = blocks * kDecWaves;
  const int per_wave = (tiles + waves - 1) / waves;
  hipLaunchKernelGGL((k_w4a8_dec<R, D, ST, kEpiPlain>), dim3(blocks), dim3(256), smem, s, out, add, nib, params,
                     q_split, scales, sums, rows, cols, per_wave, nx, nw, eps, DecRope{}, DecMoe{});
}

template <int R, int D>
void launch_dec_rd(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                   const float *scales, const float *sums, int rows, int cols, const float *nx, const float *nw,
                   float eps, int blocks, hipStream_t s) {
  if (nx && nw)
    launch_dec_t<R, D, 0>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s);
  else if (nx)
    launch_dec_t<R, D, 8>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s);
  else if (cols <= 16 * 256)
    launch_dec_t<R, D, 1>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s);
  else if (cols <= 16 * 512)
    launch_dec_t<R, D, 2>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s);
  else
    launch_dec_t<R, D, 4>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s);
}

template <int R, int D, int ST>
void launch_dec_moe_t(float *out, const DecMoe &moe, const int8_t *q_split, const float *scales, const float *sums,
                      int rows, int cols, int blocks, int entries, hipStream_t s) {
  const size_t smem = dec_smem<R>(cols, false);
  static size_t configured = 0;
  if (smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_dec<R, D, ST, kEpiMoe>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  const int tiles = (rows + R - 1) / R, waves = blocks * kDecWaves;
  const int per_wave = (tiles + waves - 1) / waves;
  hipLaunchKernelGGL((k_w4a8_dec<R, D, ST, kEpiMoe>), dim3(blocks, entries), dim3(256), smem, s, out, nullptr,
                     nullptr, nullptr, q_split, scales, sums, rows, cols, per_wave, nullptr, nullptr, 0.0f,
                     DecRope{}, moe);
}

}  // namespace

// Group 32, whole groups, K staged in LDS, byte offsets of every tile the
// waves address (including the zero-reading ones past the matrix) inside
// 31 bits.
bool w4a8_dec_path(int rows, int cols, int gs) {
  if (gs != 32 || rows <= 0 || cols % 32 != 0 || cols / 32 > kDecMaxGroups || cols < 256) return false;
  const long long span = ((long long)rows + 4096LL * 12) * (cols / 2);
  return span < (1LL << 31) - (1LL << 20);
}

bool w4a8_dec_fused_ok(int cols) { return cols / 32 <= 128; }

// Tile height, ring depth and grid per shape, measured on the 7B decode
// shapes (4096..32000 rows, K 4096 / 14336) with the weights streamed from
// HBM: 4-row tiles with a 4-chunk ring, or 8-row tiles with a 3-chunk ring
// where the fused RMSNorm prologue needs fewer blocks; a 512-block grid for
// many rows, one tile per wave otherwise.
static void dec_choice(int rows, bool fused, int &variant, int &blocks) {
  if (!fused) {
    variant = 4;
    blocks = rows >= 16384 ? 512 : 0;
  } else if (rows >= 16384) {
    variant = 2;
    blocks = 512;
  } else if (rows >= 8192) {
    variant = 4;
    blocks = 512;
  } else {
    variant = rows > 4096 ? 2 : 4;
    blocks = 0;
  }
}

bool launch_w4a8_dec(float *out, const float *add, const uint8_t *nib, const uint8_t *params, const int8_t *q_split,
                     const float *scales, const float *sums, int rows, int cols, int gs, const float *nx,
                     const float *nw, float eps, hipStream_t s, int variant, int blocks) {
  if (!w4a8_dec_path(rows, cols, gs)) return false;
  if (nx && !w4a8_dec_fused_ok(cols)) return false;
  if (variant == 0) dec_choice(rows, nw != nullptr, variant, blocks);
  switch (variant) {
    case 1: launch_dec_rd<4, 6>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
    case 2: launch_dec_rd<8, 3>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
    case 3: launch_dec_rd<12, 2>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
    case 4: launch_dec_rd<4, 4>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
    case 5: launch_dec_rd<8, 4>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
    case 6: launch_dec_rd<12, 3>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
    default: launch_dec_rd<8, 3>(out, add, nib, params, q_split, scales, sums, rows, cols, nx, nw, eps, blocks, s); break;
  }
  return true;
}

// 4-row tiles, 4-chunk ring; per entry about 2304 / entries blocks rounded
// up to a multiple of 8 (at least 8, at most one tile per wave): block x of
// every entry then falls on XCD x mod 8, so the entries of one expert read
// each row tile through the same L2.  Measured on the OLMoE expert shapes
// (2048 x 2048 gate|up, 2048 x 1024 down) at 72 entries: 8, 16, 24, 32 and
// 64 blocks per entry gave a 2.29, 2.17, 2.19, 2.14 and 2.21 ms verify step.
bool launch_w4a8_dec_moe(float *out, const DecMoe &moe, const int8_t *q_split, const float *scales,
                         const float *sums, int rows, int cols, int gs, int max_entries, hipStream_t s) {
  if (!w4a8_dec_path(rows, cols, gs) || max_entries <= 0 || max_entries > 65535 || cols > 16 * 1024) return false;
  const int tiles = (rows + 3) / 4, full = (tiles + kDecWaves - 1) / kDecWaves;
  int blocks = std::max(8, (2304 / max_entries + 7) & ~7);
  blocks = std::min(blocks, full);
  // A ring of two chunks (four: 11.0 -> 9.6 us per OLMoE-shaped launch,
  // decode and verify averaged).
  if (cols <= 16 * 256)
    launch_dec_moe_t<4, 2, 1>(out, moe, q_split, scales, sums, rows, cols, blocks, max_entries, s);
  else if (cols <= 16 * 512)
    launch_dec_moe_t<4, 2, 2>(out, moe, q_split, scales, sums, rows, cols, blocks, max_entries, s);
  else
    launch_dec_moe_t<4, 2, 4>(out, moe, q_split, scales, sums, rows, cols, blocks, max_entries, s);
  return true;
}

// The experts' gate|up with silu_mul and the quantization fused: grid
// (F / 32 output groups, entries), the entry's quantized silu_mul row into
// moe.qo / so / uo (F = rows / 2 values per entry).  A ring of two chunks
// (three: 16.4 -> 14.3 us per OLMoE-shaped launch, decode and verify
// averaged).
bool launch_w4a8_dec_moe_glu(const DecMoe &moe, const int8_t *q_split, const float *scales, const float *sums,
                             int rows, int cols, int gs, int max_entries, hipStream_t s) {
  if (!w4a8_dec_path(rows, cols, gs) || rows % 64 != 0 || max_entries <= 0 || max_entries > 65535 ||
      cols > 16 * 1024 || !moe.qo || !moe.so || !moe.uo)
    return false;
  const size_t smem = dec_smem<8>(cols, false);
  auto go = [&](auto st) {
    constexpr int ST = decltype(st)::value;
    static size_t configured = 0;
    if (smem > configured) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_dec<8, 2, ST, kEpiMoeGlu>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      configured = smem;
    }
    hipLaunchKernelGGL((k_w4a8_dec<8, 2, ST, kEpiMoeGlu>), dim3(rows / 64, max_entries), dim3(256), smem, s,
                       nullptr, nullptr, nullptr, nullptr, q_split, scales, sums, rows, cols, 2, nullptr, nullptr,
                       0.0f, DecRope{}, moe);
  };
  if (cols <= 16 * 256)
    go(std::integral_constant<int, 1>{});
  else if (cols <= 16 * 512)
    go(std::integral_constant<int, 2>{});
  else
    go(std::integral_constant<int, 4>{});
  return true;
}

// The fused-norm launches (gate|up + SiLU-mul + quantization, qkv + RoPE +
// KV store) keep a ring of two chunks: their waves run one or two tiles, and
// against three chunks the one-token Mistral-7B step measured gate|up 17.4 ->
// 16.3 us and qkv 10.1 -> 9.2 us (one chunk: 18.4 and 10.4).
bool launch_w4a8_glu1(const uint8_t *nib, const uint8_t *params, const float *x, const float *norm_w, float eps,
                      int rows, int cols, int gs, int8_t *q_out, float *scale_out, float *sum_out, hipStream_t s) {
  if (!w4a8_dec_path(rows, cols, gs) || !w4a8_dec_fused_ok(cols) || rows % 64 != 0) return false;
  const size_t smem = dec_smem<8>(cols, true);
  static size_t configured = 0;
  if (smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_dec<8, 2, 0, kEpiGlu>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  hipLaunchKernelGGL((k_w4a8_dec<8, 2, 0, kEpiGlu>), dim3(rows / 64), dim3(256), smem, s, nullptr, nullptr, nib,
                     params, q_out, scale_out, sum_out, rows, cols, 2, x, norm_w, eps, DecRope{}, DecMoe{});
  return true;
}

bool launch_w4a8_qkv_rope1(float *out, const uint8_t *nib, const uint8_t *params, const float *x,
                           const float *norm_w, float eps, int rows, int cols, int gs, const DecRope &rope,
                           hipStream_t s) {
  if (!w4a8_dec_path(rows, cols, gs) || !w4a8_dec_fused_ok(cols)) return false;
  if (rope.hd % 8 != 0 || rows != (rope.nh + 2 * rope.nkv) * rope.hd) return false;
  const size_t smem = dec_smem<8>(cols, true);
  static size_t configured = 0;
  if (smem > configured) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&k_w4a8_dec<8, 2, 0, kEpiRope>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    configured = smem;
  }
  const int tiles = rows / 8, blocks = (tiles + kDecWaves - 1) / kDecWaves;
  hipLaunchKernelGGL((k_w4a8_dec<8, 2, 0, kEpiRope>), dim3(blocks), dim3(256), smem, s, out, nullptr, nib, params,
                     nullptr, nullptr, nullptr, rows, cols, 1, x, norm_w, eps, rope, DecMoe{});
  return true;
}

}  // namespace rai
