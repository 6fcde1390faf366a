// Batch-8 decode GEMVs on MFMA (gfx950 v_mfma_f32_16x16x32_f16), plus the
// batch step's small kernels (final RMSNorm, per-sequence argmax, embedding
// rows, position advance).
//
// y[b][r] = W[r] . x[b] for the 8 sequences of a decode batch.  A workgroup
// (8 waves) owns 16 rows (the MFMA M dimension; 16 gate + 16 up rows for the
// SiLU epilogue); wave w owns the K slice [w K/8, (w+1) K/8) and walks it in
// 32-wide K tiles.  Per tile and lane: one 16-byte load of W (row = lane % 16,
// k = 8 (lane / 16) .. +8: exactly the A operand of the MFMA) and the B
// operand for batch column n = lane % 16 built from x in registers:
//   n < 8  : fp16(x[n][k])                      (the value, rounded)
//   n >= 8 : fp16(x[n-8][k] - fp16(x[n-8][k]))  (the rounding residual)
// so C[r][n] + C[r][n+8] = W[r] . x[n] with the activation carried to ~22
// bits: the 16 MFMA columns hold the 8 sequences twice over instead of being
// padding.  The K-slice partials of the 8 waves are summed through LDS.
//
// The weights are loaded once per batch step (every weight byte serves all 8
// sequences), which is what makes batch decoding cheaper per token than batch 1;
// the work stays bound by HBM (16 flops per 2-byte weight).

#include <float.h>
#include <math.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kB = kBatchMax;   // sequences per batch step (8)
constexpr int kRG = 16;         // rows per workgroup (MFMA M)
constexpr int kWaves = 8;       // K slices per workgroup
constexpr int kKT = 32;         // K per MFMA

// row_ror:8 within each 16-lane row: lane i reads lane i ^ 8.
__device__ __forceinline__ float swap8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf,
                                                               false));
}

// B operand of this lane for K offset k: 8 values of x[seq][k..k+8] (optionally
// RMS-normalised), as their fp16 value (lo == false) or fp16 rounding residual.
template <bool NORM>
__device__ __forceinline__ h8 b_operand(const float* xrow, const uint16_t* gamma, float rstd, int k, bool lo) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(xrow + k);
  const f32x4 b = *reinterpret_cast<const f32x4*>(xrow + k + 4);
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  if constexpr (NORM) {
    float g[8];
    unpack8(ld16(gamma + k), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (v[i] * rstd) * g[i];
  }
  h8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 hi = (_Float16)v[i];
    r[i] = lo ? (_Float16)(v[i] - (float)hi) : hi;
  }
  return r;
}

// rsqrt(mean(x[w]^2) + eps) of sequence w into s_rstd[w] (one wave per sequence).
template <int K>
__device__ __forceinline__ void batch_rstd(const float* x, long ldx, float eps, int nseq, float* s_rstd) {
  const int w = threadIdx.x / kWave;
  const int lane = lane_id();
  if (w < nseq) {
    const float* row = x + (long)w * ldx;
    float ss = 0.f;
#pragma unroll 4
    for (int k = lane * 4; k < K; k += kWave * 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + k);
      ss = __builtin_fmaf(v.x, v.x, ss);
      ss = __builtin_fmaf(v.y, v.y, ss);
      ss = __builtin_fmaf(v.z, v.z, ss);
      ss = __builtin_fmaf(v.w, v.w, ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) s_rstd[w] = rsqrtf(ss / (float)K + eps);
  }
}

// One wave: the MFMA sum of its K slice for 16 rows of W (and of W_up).
template <int K, bool NORM, bool DUAL>
__device__ __forceinline__ void slice_mfma(const Gemv8Args& a, const float* s_rstd, long r0, f32x4& acc,
                                           f32x4& acc2) {
  constexpr int KS = K / kWaves;
  constexpr int NT = KS / kKT;
  const int w = threadIdx.x / kWave;
  const int lane = lane_id();
  const int m = lane & 15;
  const int kg = (lane >> 4) * 8;
  const int kb = w * KS;
  const uint16_t* wrow = a.W + (r0 + m) * a.ldw + kb + kg;
  const uint16_t* wrow2 = a.W + (r0 + a.up_offset + m) * a.ldw + kb + kg;
  u32x4 wt[NT], wt2[DUAL ? NT : 1];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    wt[t] = ld_stream(wrow + t * kKT);
    if constexpr (DUAL) wt2[t] = ld_stream(wrow2 + t * kKT);
  }
  const int seq = m & 7;
  const bool lo = m >= 8;
  const bool live = seq < a.nseq;
  const float* xrow = a.x + (long)(live ? seq : 0) * a.ldx;
  const float rstd = NORM ? s_rstd[live ? seq : 0] : 1.f;
  acc = f32x4{0.f, 0.f, 0.f, 0.f};
  acc2 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    h8 bop = b_operand<NORM>(xrow, a.gamma, rstd, kb + kg + t * kKT, lo);
    if (!live) bop = h8{};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, wt[t]), bop, acc, 0, 0, 0);
    if constexpr (DUAL)
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, wt2[t]), bop, acc2, 0, 0, 0);
  }
}

// C[r][n] + C[r][n+8] for the lanes holding n < 8, written as the wave's
// partial into part[w][row][seq].
__device__ __forceinline__ void slice_partial(const f32x4& acc, float (*part)[kRG][kB]) {
  const int w = threadIdx.x / kWave;
  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;
  const float c[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v = c[j] + swap8(c[j]);
    if (n < kB) part[w][4 * g + j][n] = v;
  }
}

template <int K, bool NORM, int EPI>
__global__ __launch_bounds__(512) void gemv8_kernel(const Gemv8Args a) {
  __shared__ float s_rstd[kB];
  __shared__ float s_part[kWaves][kRG][kB];
  __shared__ float s_part2[(EPI == EPI_SILU) ? kWaves : 1][kRG][kB];
  const long r0 = (long)blockIdx.x * kRG;
  if constexpr (NORM) {
    batch_rstd<K>(a.x, a.ldx, a.eps, a.nseq, s_rstd);
    __syncthreads();
  }
  f32x4 acc, acc2;
  slice_mfma<K, NORM, EPI == EPI_SILU>(a, s_rstd, r0, acc, acc2);
  slice_partial(acc, s_part);
  if constexpr (EPI == EPI_SILU) slice_partial(acc2, s_part2);
  __syncthreads();
  const int t = threadIdx.x;
  const int rl = t / kB;
  const int seq = t % kB;
  const long row = r0 + rl;
  float v = 0.f;
  if (t < kRG * kB) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += s_part[w][rl][seq];
  }
  if constexpr (EPI == EPI_SILU) {
    if (t < kRG * kB && seq < a.nseq) {
      float u = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) u += s_part2[w][rl][seq];
      a.y[(long)seq * a.ldy + row] = (v / (1.0f + __expf(-v))) * u;
    }
  } else if constexpr (EPI == EPI_ARGMAX) {
    // per-sequence (max, first index) over the workgroup's 16 rows
    __shared__ float s_v[kRG][kB];
    if (t < kRG * kB) {
      s_v[rl][seq] = v;
      if (a.y != nullptr && seq < a.nseq) a.y[(long)seq * a.ldy + row] = v;
    }
    __syncthreads();
    if (t < kB) {
      float bv = s_v[0][t];
      long bi = r0;
      for (int r = 1; r < kRG; ++r) {
        if (s_v[r][t] > bv) {
          bv = s_v[r][t];
          bi = r0 + r;
        }
      }
      a.part_val[(long)blockIdx.x * kB + t] = bv;
      a.part_idx[(long)blockIdx.x * kB + t] = bi;
    }
  } else {
    if (t < kRG * kB && seq < a.nseq) {
      if (a.residual != nullptr) v += a.residual[(long)seq * a.ldr + row];
      a.y[(long)seq * a.ldy + row] = v;
    }
  }
}

// First maximal index per sequence over the workgroup partials (one block per
// sequence); the result is the sequence's next token.
__global__ __launch_bounds__(256) void argmax8_reduce_kernel(const float* part_val, const long* part_idx, int nblk,
                                                             int64_t* token) {
  __shared__ float r_v[256];
  __shared__ long r_i[256];
  const int seq = blockIdx.x;
  float bv = -INFINITY;
  long bi = 0x7fffffffffffL;
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    const float v = part_val[(long)b * kB + seq];
    const long i = part_idx[(long)b * kB + seq];
    if (v > bv || (v == bv && i < bi)) {
      bv = v;
      bi = i;
    }
  }
  r_v[threadIdx.x] = bv;
  r_i[threadIdx.x] = bi;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      const float v = r_v[threadIdx.x + s];
      const long i = r_i[threadIdx.x + s];
      if (v > r_v[threadIdx.x] || (v == r_v[threadIdx.x] && i < r_i[threadIdx.x])) {
        r_v[threadIdx.x] = v;
        r_i[threadIdx.x] = i;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) token[seq] = r_i[0] == 0x7fffffffffffL ? 0 : r_i[0];
}

// y[b] = rmsnorm(x[b]) * gamma (fp32), one block per sequence.
__global__ __launch_bounds__(256) void rmsnorm8_kernel(const float* x, long ldx, const uint16_t* gamma, float eps,
                                                       int K, float* y, long ldy) {
  __shared__ float s_red[4];
  const float* row = x + (long)blockIdx.x * ldx;
  float ss = 0.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) ss = __builtin_fmaf(row[k], row[k], ss);
  ss = wave_sum(ss);
  if (lane_id() == 0) s_red[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float rstd = rsqrtf((s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)K + eps);
  for (int k = threadIdx.x; k < K; k += blockDim.x)
    y[(long)blockIdx.x * ldy + k] = (row[k] * rstd) * h2f(gamma[k]);
}

// x[b] = embed[token[b]] (fp32), one block per sequence.
__global__ __launch_bounds__(256) void embed8_kernel(const uint16_t* table, const int64_t* token, float* out,
                                                     int H, long V) {
  long t = token[blockIdx.x];
  if (t < 0 || t >= V) t = 0;
  const uint16_t* row = table + t * (long)H;
  for (int i = threadIdx.x; i < H; i += blockDim.x) out[(long)blockIdx.x * H + i] = h2f(row[i]);
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

template <int K, bool NORM, int EPI>
int launch8(const Gemv8Args& a, hipStream_t s) {
  const long rows = (EPI == EPI_SILU) ? a.up_offset : a.N;
  const unsigned grid = (unsigned)((rows + kRG - 1) / kRG);
  hipLaunchKernelGGL((gemv8_kernel<K, NORM, EPI>), dim3(grid), dim3(kWaves * kWave), 0, s, a);
  return qd_host::launch_status("gemv8_kernel");
}

}  // namespace

int gemv8_launch(const Gemv8Args& a, bool norm, int epi, hipStream_t s) {
  if (a.nseq < 1 || a.nseq > kB) return QD_ERR_SHAPE;
  const long rows = (epi == EPI_SILU) ? a.up_offset : a.N;
  if (rows % kRG != 0 || a.ldx % 4 != 0) return QD_ERR_SHAPE;
#define QD_G8(KK)                                                                   \
  if (a.K == KK) {                                                                  \
    if (epi == EPI_SILU) return norm ? launch8<KK, true, EPI_SILU>(a, s) : launch8<KK, false, EPI_SILU>(a, s); \
    if (epi == EPI_ARGMAX) return norm ? launch8<KK, true, EPI_ARGMAX>(a, s) : launch8<KK, false, EPI_ARGMAX>(a, s); \
    return norm ? launch8<KK, true, EPI_STORE>(a, s) : launch8<KK, false, EPI_STORE>(a, s); \
  }
  QD_G8(2048)
  QD_G8(6144)
#undef QD_G8
  return QD_ERR_SHAPE;
}

int gemv8_row_groups(long N) { return (int)((N + kRG - 1) / kRG); }

int argmax8_reduce_launch(const float* part_val, const long* part_idx, int nblk, int64_t* token, int nseq,
                          hipStream_t s) {
  hipLaunchKernelGGL(argmax8_reduce_kernel, dim3((unsigned)nseq), dim3(256), 0, s, part_val, part_idx, nblk, token);
  return qd_host::launch_status("argmax8_reduce_kernel");
}

int rmsnorm8_launch(const float* x, long ldx, const uint16_t* gamma, float eps, int K, float* y, long ldy, int nseq,
                    hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm8_kernel, dim3((unsigned)nseq), dim3(256), 0, s, x, ldx, gamma, eps, K, y, ldy);
  return qd_host::launch_status("rmsnorm8_kernel");
}

int embed8_launch(const uint16_t* table, const int64_t* token, float* out, int H, long V, int nseq, hipStream_t s) {
  hipLaunchKernelGGL(embed8_kernel, dim3((unsigned)nseq), dim3(256), 0, s, table, token, out, H, V);
  return qd_host::launch_status("embed8_kernel");
}

int advance8_launch(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                    int64_t* rope_position, int max_tokens, int nseq, hipStream_t s) {
  hipLaunchKernelGGL(advance8_kernel, dim3(1), dim3(64), 0, s, token, out_tokens, counter, cache_position,
                     rope_position, max_tokens, nseq);
  return qd_host::launch_status("advance8_kernel");
}

}  // namespace qd
