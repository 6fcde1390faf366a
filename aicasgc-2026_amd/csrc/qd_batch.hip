// Batch-8 decode GEMVs on MFMA (gfx950 v_mfma_f32_16x16x32_f16), plus the
// batch step's small kernels (operand images, per-sequence argmax, embedding
// rows, position advance).
//
// y[b][r] = f[b] (W[r] . u[b]) for the (up to) 8 sequences of a decode batch.
// The activation u enters as its operand image (qd_common.h): per K tile of 32
// and lane, one 16-byte load gives the lane's 8 B-operand values, fp16 value
// columns 0..7 and fp16 rounding-residual columns 8..15, so C[r][n] + C[r][n+8]
// = W[r] . u[n] with u carried to ~22 bits.  The producer of an activation
// writes the image in its epilogue, already multiplied by the consumer's
// RMSNorm weight and by a per-sequence scale s that keeps it in fp16 range;
// the consumer's factor f = rstd / s applies the RMSNorm, rstd coming from
// per-row-group partial sums of squares written by the same producer.
//
// A workgroup (8 waves) owns RG rows: 16 (the MFMA M dimension) or 8 (A rows
// 8..15 zero, twice the workgroups without a K split); RG gate + RG up rows
// for the SiLU epilogue.  It covers a K range of KW (1024, 2048, 3072 or 6144);
// wave w owns the slice [w KW/8, (w+1) KW/8) and keeps its image tiles in
// registers.  W is loaded in coalesced 128-byte row pieces and moved into the
// MFMA A layout (row lane % 16, k 8 (lane / 16) .. +8) with ds_bpermute:
// loading the A layout directly would make every lane of a load touch a
// different row.  The 8 K-slice partials are summed through LDS.  When K > KW
// the row group's K ranges run in separate workgroups (grid y); each publishes
// its partial and the last to arrive sums them in a fixed order and runs the
// epilogue.  The lm_head (EPI_ARGMAX) runs one workgroup per CU, each looping
// over row groups with two weight buffers alternating roles (the next group's
// weights in flight while the current one is reduced).
//
// Weights are loaded once per batch step (every weight byte serves all 8
// sequences); the work is bound by HBM (16 flops per 2-byte weight).

#include <float.h>
#include <math.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kB = kBatchMax;     // sequences per batch step (8)
constexpr int kWaves = 8;         // K slices per workgroup
constexpr int kKT = 32;           // K per MFMA

// Lane permutation of a 16-byte register quad: lane d receives lane addr/4's.
__device__ __forceinline__ u32x4 bpermute4(int addr, const u32x4& v) {
  return u32x4{(unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.x), (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.y),
               (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.z), (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.w)};
}

// Partial sums of squares of sequence seq ([parts][8], parts <= 256): four per
// lane, loaded ahead of their use; ss_rstd() finishes the reduction (rstd over
// n elements, the same value in every lane of the calling wave).
constexpr int kMaxSsParts = 4 * kWave;
struct SsPart {
  float v[4] = {0.f, 0.f, 0.f, 0.f};
};
__device__ __forceinline__ SsPart ss_load(const float* ss, int parts, int seq) {
  SsPart r;
  const int p = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (ss != nullptr && p + i * kWave < parts) r.v[i] = ss[(long)(p + i * kWave) * kB + seq];
  return r;
}
__device__ __forceinline__ float ss_rstd(SsPart q, float n, float eps) {
  return rsqrtf(wave_sum((q.v[0] + q.v[1]) + (q.v[2] + q.v[3])) / n + eps);
}

// Sum over groups of R consecutive lanes (R = 8 or 16); every lane of a group
// receives its group's sum.
template <int R>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (R == 16) {
    return row16_sum(v);
  } else {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    return v;
  }
}

// First maximal index per sequence over the nblk workgroup partials that the
// other workgroups of this launch published (agent-coherent loads): the whole
// 512-thread workgroup, wave b for sequence b; the result is the sequence's
// next token.  With a.adv_counter set the workgroup then advances the decode
// state as advance8_kernel does (one launch less per step).
__device__ __forceinline__ void argmax8_finish(const Gemv8Args& a, int nblk) {
  const int seq = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t c = a.adv_counter != nullptr ? a.adv_counter[0] : 0;
  if (seq < a.nseq) {
    float bv = -INFINITY;
    long bi = 0x7fffffffffffL;
    for (int b = lane; b < nblk; b += kWave) {
      const float v = load_coherent(a.part_val + (long)b * kB + seq);
      const long i = load_coherent(a.part_idx + (long)b * kB + seq);
      if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
      }
    }
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const float ov = __shfl_xor(bv, off);
      const long oi = __shfl_xor(bi, off);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      // no finite maximum anywhere (all partials -inf / NaN): token 0
      const int64_t tok = bi >= 0x7fffffffL ? 0 : bi;
      a.token[seq] = tok;
      if (a.adv_counter != nullptr) {
        if (a.adv_out != nullptr && c < a.adv_max_tokens) a.adv_out[c * a.nseq + seq] = tok;
        a.adv_cache_position[seq] += 1;
        a.adv_rope_position[3 * seq + 0] += 1;
        a.adv_rope_position[3 * seq + 1] += 1;
        a.adv_rope_position[3 * seq + 2] += 1;
      }
    }
  }
  __syncthreads();   // every wave read the counter before it moves
  if (threadIdx.x == 0 && a.adv_counter != nullptr) a.adv_counter[0] = c + 1;
}

// RG: rows per workgroup, 16 (the MFMA M dimension) or 8 (rows 8..15 of the
// A operand are zero: twice the workgroups for the same rows, so a shape with
// few row groups fills the CUs without splitting K).
// TILED: W is stored in MFMA tile order, so each 16-byte load of a lane is
// already its A operand and a wave's load is one contiguous 1 KB:
//   RG 16: [rows/16][K/8][16][8], element (g, q, r, e) = W[16 g + r][8 q + e];
//          lane d of K tile kt reads 16 bytes at ((g K/8 + 4 kt) 16 + d) 8;
//   RG 8:  [rows/8][K/64][4][2][8][8], element (g, p, c, h, r, e) =
//          W[8 g + r][64 p + 32 h + 8 c + e]; one load covers the K tile pair
//          (2 p, 2 p + 1): lanes d % 16 < 8 hold rows 0..7 of tile 2 p, the
//          others those of tile 2 p + 1, moved down by a row_ror:8 DPP.
template <int KW, int EPI, int RG, bool TILED = false>
__global__ __launch_bounds__(512) void gemv8_kernel(const Gemv8Args a) {
  constexpr int KS = KW / kWaves;
  constexpr int NT = KS / kKT;
  constexpr bool DUAL = EPI == EPI_SILU;
  constexpr bool ARGMAX = EPI == EPI_ARGMAX;
  constexpr int NA = DUAL ? 2 : 1;
  constexpr int NL = RG / 8;                 // weight loads per tile pair (8 rows each)
  constexpr int NWT = NT / 2 * NL;
  constexpr int NW2 = DUAL ? NWT : 1;
  constexpr int OUT = RG * kB;               // outputs of one row group
  static_assert(RG == 8 || RG == 16, "8 or 16 rows per workgroup");
  static_assert(!ARGMAX || RG == 16, "argmax epilogue: 16 rows per group");
  static_assert(!(TILED && ARGMAX), "tile order: not the looping lm_head (row-major streams faster there)");
  __shared__ float s_fac[kB], s_osc[kB];
  __shared__ float s_part[NA][kWaves][kB][RG];
  __shared__ int s_last;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = lane_id();
  const int m = lane & 15;
  const int t = threadIdx.x;
  const long kb = (long)blockIdx.y * KW + (long)w * KS;
  const long rows = DUAL ? a.up_offset : a.N;
  const int nrg = (int)(rows / RG);

  // Weight loads are coalesced 128-byte row pieces: for the tile pair (2j, 2j+1)
  // (64 K values) load h covers rows 8h..8h+7 with 8 lanes x 16 bytes per row
  // (lane: row 8h + lane / 8, k 8 (lane % 8)).  pair_to_mfma() moves the pair
  // into the MFMA A layout with ds_bpermute (lane d = row r + 16 c of tile 2j+q
  // takes row r, k 32q + 8c: load r / 8, source lane 8 (r % 8) + 4q + c); with
  // RG = 8 the rows 8..15 are zero.
  static_assert(NT % 2 == 0, "tile pairs");
  // (issued in the order the MFMA loop consumes them: gate pair, up pair, ...)
  auto load_w = [&](int rg, u32x4 (&wt)[NWT], u32x4 (&wt2)[NW2]) {
    if constexpr (TILED) {
      // RG 16: tiles 2 j, 2 j + 1 in wt[2 j], wt[2 j + 1]; RG 8: tile pair j in wt[j]
      const uint16_t* p = a.W + ((long)rg * (a.K / 8) + kb / 8) * RG * 8 + lane * 8;
      const uint16_t* p2 = p + (a.up_offset / RG) * (a.K / 8) * RG * 8;
#pragma unroll
      for (int i = 0; i < NWT; ++i) {
        wt[i] = ld_stream(p + (long)i * 512);
        if constexpr (DUAL) wt2[i] = ld_stream(p2 + (long)i * 512);
      }
      return;
    }
    const uint16_t* p = a.W + ((long)rg * RG + (lane >> 3)) * a.ldw + kb + (lane & 7) * 8;
    const uint16_t* p2 = p + a.up_offset * a.ldw;
    const long h8row = 8 * a.ldw;
#pragma unroll
    for (int j = 0; j < NT / 2; ++j) {
#pragma unroll
      for (int h = 0; h < NL; ++h) wt[j * NL + h] = ld_stream(p + h * h8row + 2 * j * kKT);
      if constexpr (DUAL) {
#pragma unroll
        for (int h = 0; h < NL; ++h) wt2[j * NL + h] = ld_stream(p2 + h * h8row + 2 * j * kKT);
      }
    }
  };
  const int src0 = (8 * (m & 7) + (lane >> 4)) * 4;   // byte lane addresses for ds_bpermute
  const int src1 = src0 + 16;
  const bool upper = m >= 8;
  auto pair_to_mfma = [&](const auto& w, int j, u32x4& t0, u32x4& t1) {
    if constexpr (TILED) {
      if constexpr (NL == 2) {
        t0 = w[2 * j];
        t1 = w[2 * j + 1];
      } else {
        const u32x4 z = {0u, 0u, 0u, 0u};
        const u32x4 x = w[j];
        const u32x4 r = {dpp_u<kDppRowRor8>(x.x), dpp_u<kDppRowRor8>(x.y), dpp_u<kDppRowRor8>(x.z),
                         dpp_u<kDppRowRor8>(x.w)};
        t0 = upper ? z : x;
        t1 = upper ? z : r;
      }
      return;
    }
    const u32x4 a0 = bpermute4(src0, w[j * NL]);
    const u32x4 a1 = bpermute4(src1, w[j * NL]);
    if constexpr (NL == 2) {
      const u32x4 b0 = bpermute4(src0, w[j * NL + 1]), b1 = bpermute4(src1, w[j * NL + 1]);
      t0 = upper ? b0 : a0;
      t1 = upper ? b1 : a1;
    } else {
      const u32x4 z = {0u, 0u, 0u, 0u};
      t0 = upper ? z : a0;
      t1 = upper ? z : a1;
    }
  };

  int rg = blockIdx.x;
  const int rl = t % RG;    // epilogue thread: row rl of the group, sequence seq
  const int seq = (t / RG) & (kB - 1);
  const bool live = seq < a.nseq;
  // the epilogue's residual and norm weight, loaded before the weights so the
  // epilogue does not wait for another round trip (one row group per
  // workgroup outside EPI_ARGMAX)
  float res = 0.f, gam = 1.f;
  if constexpr (!ARGMAX) {
    if (t < OUT) {
      const long row = (long)rg * RG + rl;
      if (a.residual != nullptr && live) res = a.residual[(long)seq * a.ldr + row];
      if (a.yb_gamma != nullptr) gam = h2f(a.yb_gamma[row]);
    }
  }
  // Then the wave's image tiles (read once, used for every row group) and the
  // norm partial sums, and only then the weights: loads complete in issue
  // order, so the MFMAs and the norm factors wait only for what they use while
  // the weight stream is still arriving.
  u32x4 bt[NT];
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(a.xb) + (kb / kKT) * kWave + lane;
#pragma unroll
    for (int i = 0; i < NT; ++i) bt[i] = src[i * kWave];
  }
  const SsPart in_q = ss_load(a.in_ss, a.in_parts, w);
  const SsPart pre_q = ss_load(a.pre_ss, a.pre_parts, w);
  u32x4 wt[NWT], wt2[NW2];
  load_w(rg, wt, wt2);
  // wave w: factors of sequence w
  {
    float f = 1.f, o = 1.f;
    if (a.in_ss != nullptr) f = ss_rstd(in_q, (float)a.K, a.eps);
    if (a.in_scale != nullptr) f /= a.in_scale[w];
    if (w >= a.nseq) f = 0.f;
    if (a.pre_ss != nullptr) o = ss_rstd(pre_q, (float)a.N, a.eps);
    if (lane == 0) {
      s_fac[w] = f;
      s_osc[w] = o;
    }
  }
  float best = -INFINITY;
  int best_i = 0x7fffffff;

  // One row group: MFMAs over the weights in wa (wa2: the up rows), the K-slice
  // reduction through LDS, the K-split hand-off and the epilogue.  Returns
  // false when this workgroup's part is done (K split, not the last to arrive).
  auto process = [&](const auto& wa, const auto& wa2, int rg) -> bool {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NT; i += 2) {
      u32x4 t0, t1;
      pair_to_mfma(wa, i / 2, t0, t1);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, t0), __builtin_bit_cast(h8, bt[i]), acc, 0, 0,
                                                   0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, t1), __builtin_bit_cast(h8, bt[i + 1]), acc,
                                                   0, 0, 0);
      if constexpr (DUAL) {
        pair_to_mfma(wa2, i / 2, t0, t1);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, t0), __builtin_bit_cast(h8, bt[i]), acc2,
                                                      0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, t1), __builtin_bit_cast(h8, bt[i + 1]),
                                                      acc2, 0, 0, 0);
      }
    }
    {
      // lanes n < 8 of each 16-lane row: C[r][n] + C[r][n+8], rows 4 (lane / 16) + j
      const int g = lane >> 4;
      const float c[4] = {acc.x, acc.y, acc.z, acc.w};
      const float c2[4] = {acc2.x, acc2.y, acc2.z, acc2.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = c[j] + dpp<kDppRowRor8>(c[j]);
        if (m < kB && 4 * g + j < RG) s_part[0][w][m][4 * g + j] = v;
        if constexpr (DUAL) {
          const float v2 = c2[j] + dpp<kDppRowRor8>(c2[j]);
          if (m < kB && 4 * g + j < RG) s_part[NA - 1][w][m][4 * g + j] = v2;
        }
      }
    }
    __syncthreads();
    float v = 0.f, v2 = 0.f;
    if (t < OUT) {
#pragma unroll
      for (int q = 0; q < kWaves; ++q) v += s_part[0][q][seq][rl];
      if constexpr (DUAL) {
#pragma unroll
        for (int q = 0; q < kWaves; ++q) v2 += s_part[NA - 1][q][seq][rl];
      }
    }
    if constexpr (!ARGMAX) {
      if (a.ksplit > 1) {
        // publish this K range's partials (coherent stores, completed before the
        // arrival count); the last workgroup of the row group sums them in K order
        float* kp = a.kpart + (long)rg * a.ksplit * (NA * OUT);
        if (t < OUT) {
          store_coherent(kp + (long)blockIdx.y * (NA * OUT) + t, v);
          if constexpr (DUAL) store_coherent(kp + (long)blockIdx.y * (NA * OUT) + OUT + t, v2);
        }
        stores_done();
        __syncthreads();
        if (t == 0) s_last = arrive_last(a.kcount + rg, (unsigned)a.ksplit);
        __syncthreads();
        if (!s_last) return false;
        if (t < OUT) {
          // every partial's load issued before the first is used (unconditional,
          // index clamped; a clamped duplicate adds 0): one round trip, not ksplit
          constexpr int kMaxSplit = kBatchMaxKsplit;
          float p[kMaxSplit], p2[kMaxSplit];
#pragma unroll
          for (int q = 0; q < kMaxSplit; ++q) {
            const long o = (long)min(q, a.ksplit - 1) * (NA * OUT) + t;
            p[q] = load_coherent(kp + o);
            if constexpr (DUAL) p2[q] = load_coherent(kp + o + OUT);
          }
          v = 0.f;
          v2 = 0.f;
#pragma unroll
          for (int q = 0; q < kMaxSplit; ++q) {
            v += q < a.ksplit ? p[q] : 0.f;
            if constexpr (DUAL) v2 += q < a.ksplit ? p2[q] : 0.f;
          }
        }
      }
    }
    if (t < OUT) {
      const long row = (long)rg * RG + rl;
      v *= s_fac[seq];
      if constexpr (ARGMAX) {
        if (a.y != nullptr && live) a.y[(long)seq * a.ldy + row] = v;
        // (max, first row) over the group's 16 rows: 16 consecutive lanes
        float bv = v;
        int bi = (int)row;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const float ov = __shfl_xor(bv, off);
          const int oi = __shfl_xor(bi, off);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (bv > best) {   // row groups ascend: ties keep the earlier row
          best = bv;
          best_i = bi;
        }
      } else {
        if constexpr (DUAL) {
          v2 *= s_fac[seq];
          v = (v / (1.0f + __expf(-v))) * v2;
        } else {
          v += res;
        }
        if (!live) v = 0.f;
        if (a.y != nullptr && live) a.y[(long)seq * a.ldy + row] = v;
        if (a.yb != nullptr)
          bimg_store(a.yb, seq, row, v * gam * s_osc[seq]);
        if (a.yss != nullptr) {
          const float q = group_sum<RG>(v * v);
          if (rl == 0) a.yss[(long)rg * kB + seq] = q;
        }
        if (a.out_scale != nullptr && rg == 0 && rl == 0) a.out_scale[seq] = s_osc[seq];
      }
    }
    return true;
  };
  if constexpr (!ARGMAX) {
    if (!process(wt, wt2, rg)) return;
  } else {
    // The lm_head loops over row groups with the next group's weights in
    // flight; the two buffers alternate roles (a register copy would wait for
    // the prefetched loads).  The prefetch is unconditional (past the last
    // group it re-reads the last group) so every path has the same loads in
    // flight and each group waits only for its own.
    u32x4 wn[NWT];
    for (;;) {
      int nxt = rg + (int)gridDim.x;
      load_w(min(nxt, nrg - 1), wn, wt2);
      __builtin_amdgcn_sched_barrier(0);   // keep the prefetch ahead of this group's work
      process(wt, wt2, rg);
      if (nxt >= nrg) break;
      __syncthreads();   // s_part is rewritten by the next group
      rg = nxt;
      nxt = rg + (int)gridDim.x;
      load_w(min(nxt, nrg - 1), wt, wt2);
      __builtin_amdgcn_sched_barrier(0);
      process(wn, wt2, rg);
      if (nxt >= nrg) break;
      __syncthreads();
      rg = nxt;
    }
  }
  if constexpr (ARGMAX) {
    // per-workgroup (max, first index) of each sequence, published with
    // coherent stores; the last workgroup to arrive reduces them (one round
    // of workgroups: none waits for another)
    if (t < OUT && rl == 0) {
      store_coherent(a.part_val + (long)blockIdx.x * kB + seq, best);
      store_coherent(a.part_idx + (long)blockIdx.x * kB + seq, (long)best_i);
      stores_done();
    }
    __syncthreads();
    if (t == 0) s_last = arrive_last(a.argmax_count, gridDim.x);
    __syncthreads();
    if (s_last) argmax8_finish(a, (int)gridDim.x);
  }
}

// Image of 8 consecutive values u[0..7] at K index k0 (k0 % 8 == 0): one
// 16-byte store for the value column, one for the residual column.
__device__ __forceinline__ void bimg_store8(uint16_t* img, int seq, long k0, const float* u) {
  unsigned hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const _Float16 h0 = (_Float16)u[2 * i], h1 = (_Float16)u[2 * i + 1];
    const _Float16 l0 = (_Float16)(u[2 * i] - (float)h0), l1 = (_Float16)(u[2 * i + 1] - (float)h1);
    hi[i] = (unsigned)__builtin_bit_cast(uint16_t, h0) | ((unsigned)__builtin_bit_cast(uint16_t, h1) << 16);
    lo[i] = (unsigned)__builtin_bit_cast(uint16_t, l0) | ((unsigned)__builtin_bit_cast(uint16_t, l1) << 16);
  }
  *reinterpret_cast<u32x4*>(img + bimg_index(seq, k0)) = u32x4{hi[0], hi[1], hi[2], hi[3]};
  *reinterpret_cast<u32x4*>(img + bimg_index(seq + 8, k0)) = u32x4{lo[0], lo[1], lo[2], lo[3]};
}

// Block-wide (256 threads) sum, uniform in every thread.
__device__ __forceinline__ float block256_sum(float v, float* s_red) {
  v = wave_sum(v);
  if (lane_id() == 0) s_red[threadIdx.x / kWave] = v;
  __syncthreads();
  const float r = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  __syncthreads();
  return r;
}

// Image of u = x * gamma * s (s = rstd(x) when norm, else 1), with ss[seq] =
// sum of x^2 and scale[seq] = s; one block per sequence column (zeros beyond
// nseq).  Rows are fp32 x[seq] (TX float) or the fp16 embedding rows of
// token[seq] (TX uint16_t, also copied to x_out as fp32).
template <typename TX>
__global__ __launch_bounds__(256) void bimage8_kernel(const TX* x, long ldx, const int64_t* token, long V,
                                                      const uint16_t* gamma, bool norm, float eps, int K, int nseq,
                                                      float* x_out, uint16_t* img, float* ss, float* scale) {
  __shared__ float s_red[4];
  const int seq = blockIdx.x;
  const bool live = seq < nseq;
  const TX* row = x;
  if constexpr (sizeof(TX) == 2) {
    long tk = live ? token[seq] : 0;
    if (tk < 0 || tk >= V) tk = 0;
    row = x + tk * (long)K;
  } else {
    row = x + (long)seq * ldx;
  }
  float q = 0.f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    float u[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) load_act8<TX>(row, k, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) q = __builtin_fmaf(u[i], u[i], q);
  }
  q = block256_sum(q, s_red);
  const float s = norm ? rsqrtf(q / (float)K + eps) : 1.f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    float u[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) load_act8<TX>(row, k, u);
    if (x_out != nullptr && live) {
      float4* o = reinterpret_cast<float4*>(x_out + (long)seq * K + k);
      o[0] = float4{u[0], u[1], u[2], u[3]};
      o[1] = float4{u[4], u[5], u[6], u[7]};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] *= (gamma != nullptr ? h2f(gamma[k + i]) : 1.f) * s;
    bimg_store8(img, seq, k, u);
  }
  if (threadIdx.x == 0) {
    if (ss != nullptr) ss[seq] = q;
    if (scale != nullptr) scale[seq] = s;
  }
}

// Per sequence: out_tokens[counter][b] = token[b] (while counter < max_tokens),
// ++cache_position[b], ++rope_position[b][0..2]; then ++counter.
__global__ void advance8_kernel(const int64_t* token, int64_t* out_tokens, int64_t* counter,
                                int64_t* cache_position, int64_t* rope_position, int max_tokens, int nseq) {
  const int b = threadIdx.x;
  const int64_t c = counter[0];
  if (b < nseq) {
    if (out_tokens != nullptr && c < max_tokens) out_tokens[c * nseq + b] = token[b];
    cache_position[b] += 1;
    rope_position[3 * b + 0] += 1;
    rope_position[3 * b + 1] += 1;
    rope_position[3 * b + 2] += 1;
  }
  __syncthreads();
  if (b == 0) counter[0] = c + 1;
}

template <int KW, int EPI, int RG>
int launch8(const Gemv8Args& a, unsigned gx, hipStream_t s) {
  if (a.w_tiled)
    hipLaunchKernelGGL((gemv8_kernel<KW, EPI, RG, true>), dim3(gx, (unsigned)a.ksplit), dim3(kWaves * kWave), 0, s,
                       a);
  else
    hipLaunchKernelGGL((gemv8_kernel<KW, EPI, RG>), dim3(gx, (unsigned)a.ksplit), dim3(kWaves * kWave), 0, s, a);
  return qd_host::launch_status("gemv8_kernel");
}

// Only the row-major form for the looping lm_head.
template <>
int launch8<2048, EPI_ARGMAX, 16>(const Gemv8Args& a, unsigned gx, hipStream_t s) {
  if (a.w_tiled) return QD_ERR_SHAPE;
  hipLaunchKernelGGL((gemv8_kernel<2048, EPI_ARGMAX, 16>), dim3(gx, (unsigned)a.ksplit), dim3(kWaves * kWave), 0, s,
                     a);
  return qd_host::launch_status("gemv8_kernel");
}

}  // namespace

int gemv8_launch(const Gemv8Args& a, int epi, hipStream_t s) {
  if (a.nseq < 1 || a.nseq > kB || a.ksplit < 1 || a.ksplit > kBatchMaxKsplit || a.K % a.ksplit != 0 ||
      a.xb == nullptr)
    return QD_ERR_SHAPE;
  if ((a.in_ss != nullptr && (a.in_parts < 1 || a.in_parts > kMaxSsParts)) ||
      (a.pre_ss != nullptr && (a.pre_parts < 1 || a.pre_parts > kMaxSsParts)))
    return QD_ERR_SHAPE;
  const int rg = a.rows_per_group;
  if (rg != 8 && rg != 16) return QD_ERR_SHAPE;
  const long rows = (epi == EPI_SILU) ? a.up_offset : a.N;
  if (rows % rg != 0 || rows <= 0) return QD_ERR_SHAPE;
  const long KW = a.K / a.ksplit;
  const unsigned nrg = (unsigned)(rows / rg);
  if (a.ksplit > 1 && (epi == EPI_ARGMAX || a.kpart == nullptr || a.kcount == nullptr)) return QD_ERR_SHAPE;
  if (epi == EPI_ARGMAX) {
    if (KW != 2048 || rg != 16 || a.part_val == nullptr || a.part_idx == nullptr) return QD_ERR_SHAPE;
    if (a.argmax_count == nullptr || a.token == nullptr) return QD_ERR_ARG;
    const unsigned gx = (a.grid > 0 && (unsigned)a.grid < nrg) ? (unsigned)a.grid : nrg;
    return launch8<2048, EPI_ARGMAX, 16>(a, gx, s);
  }
  if (rg == 8) {
    if (epi == EPI_SILU) return KW == 2048 ? launch8<2048, EPI_SILU, 8>(a, nrg, s) : QD_ERR_SHAPE;
    if (KW == 6144) return launch8<6144, EPI_STORE, 8>(a, nrg, s);
    if (KW == 2048) return launch8<2048, EPI_STORE, 8>(a, nrg, s);
    return QD_ERR_SHAPE;
  }
  if (epi == EPI_SILU) {
    if (KW == 2048) return launch8<2048, EPI_SILU, 16>(a, nrg, s);
    if (KW == 1024) return launch8<1024, EPI_SILU, 16>(a, nrg, s);
    return QD_ERR_SHAPE;
  }
  if (KW == 6144) return launch8<6144, EPI_STORE, 16>(a, nrg, s);
  if (KW == 3072) return launch8<3072, EPI_STORE, 16>(a, nrg, s);
  if (KW == 2048) return launch8<2048, EPI_STORE, 16>(a, nrg, s);
  if (KW == 1024) return launch8<1024, EPI_STORE, 16>(a, nrg, s);
  return QD_ERR_SHAPE;
}

int gemv8_row_groups(long N, int rows_per_group) {
  return (int)((N + rows_per_group - 1) / rows_per_group);
}

int bimage8_launch(const float* x, long ldx, const uint16_t* gamma, bool norm, float eps, int K, int nseq,
                   uint16_t* img, float* ss, float* scale, hipStream_t s) {
  if (K % 32 != 0 || nseq < 1 || nseq > kB) return QD_ERR_SHAPE;
  hipLaunchKernelGGL((bimage8_kernel<float>), dim3(kB), dim3(256), 0, s, x, ldx, nullptr, 0L, gamma, norm, eps, K,
                     nseq, nullptr, img, ss, scale);
  return qd_host::launch_status("bimage8_kernel");
}

int embed8_launch(const uint16_t* table, const int64_t* token, float* out, int H, long V, int nseq,
                  const uint16_t* gamma, float eps, uint16_t* img, float* ss, float* scale, hipStream_t s) {
  if (H % 32 != 0 || nseq < 1 || nseq > kB) return QD_ERR_SHAPE;
  hipLaunchKernelGGL((bimage8_kernel<uint16_t>), dim3(kB), dim3(256), 0, s, table, 0L, token, V, gamma, true, eps,
                     H, nseq, out, img, ss, scale);
  return qd_host::launch_status("embed8_kernel");
}

int advance8_launch(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                    int64_t* rope_position, int max_tokens, int nseq, hipStream_t s) {
  hipLaunchKernelGGL(advance8_kernel, dim3(1), dim3(64), 0, s, token, out_tokens, counter, cache_position,
                     rope_position, max_tokens, nseq);
  return qd_host::launch_status("advance8_kernel");
}

}  // namespace qd
