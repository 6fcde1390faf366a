// Batch-1 decode GEMV family for gfx950.
//
// y[N] = W[N, K] . x[K] with fp16 weights, fp32 accumulation and optional
// prologues (RMSNorm, residual-add + RMSNorm) and epilogues (bias/residual
// add, SiLU(gate)*up over row pairs, fused argmax, split-K partials).
//
// Layout: one wave64 owns R whole rows at a time.  Lane l of the wave holds the
// K-slice {c*512 + 8l .. c*512 + 8l + 7 : c < K/512} of x in registers (fp32),
// so every weight load is a 16-byte-per-lane, 1 KiB-per-wave contiguous
// stream and x never goes through LDS.  The row sum is a DPP + readlane wave
// reduction.  The RMSNorm prologue needs sum(x^2) over all K, which each wave
// already holds across its 64 lanes: no LDS, no block barrier.
//
// Reference kernels replaced: decode_gemv_kernel_matvec.cuh:208-347
// (nosplit k2048 / row2), decode_gemv_kernel_fused.cuh:99-185 (rmsnorm+qkv),
// :856-1076 (post-attn MLP phases), decode_gemv_kernel_matvec.cuh:1-205 (split-K).

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

// Loads the R weight rows of output group o0 (rows past N read as zero).
template <int KCH, int R, int RO, int EPI>
__device__ __forceinline__ void load_rows(const GemvArgs& a, long o0, long kofs, int lane, u32x4 (&wv)[R][KCH]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long oi = o0 + (r % RO);
    const long row = (EPI == EPI_SILU && r >= RO) ? oi + a.up_offset : oi;
    if (oi < a.N) {
      const uint16_t* wr = a.W + row * a.ldw + kofs + lane * 8;
#pragma unroll
      for (int c = 0; c < KCH; ++c) wv[r][c] = ld_stream(wr + c * 512);
    } else {
#pragma unroll
      for (int c = 0; c < KCH; ++c) wv[r][c] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// First maximal index over the n per-block partials that the other blocks of
// this launch published (agent-coherent loads; whole block, 256 threads).
// Writes a.token[0] and, when a.adv_counter is set, advances the decode state
// as decode_advance_kernel does (one launch less per decode step).
__device__ __forceinline__ void argmax_finish(const GemvArgs& a, int n) {
  __shared__ float r_v[256];
  __shared__ long r_i[256];
  float bv = -INFINITY;
  long bi = 0x7fffffffffffL;
  for (int b = threadIdx.x; b < n; b += blockDim.x) {
    const float v = load_coherent(a.part_val + b);
    const long i = load_coherent(a.part_idx + b);
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
  if (threadIdx.x == 0) {
    const int64_t tok = r_i[0] == 0x7fffffffffffL ? 0 : (int64_t)r_i[0];
    a.token[0] = tok;
    if (a.adv_counter != nullptr) {
      const int64_t c = a.adv_counter[0];
      if (a.adv_out != nullptr && c < a.adv_max_tokens) a.adv_out[c] = tok;
      a.adv_counter[0] = c + 1;
      a.adv_cache_position[0] += 1;
      a.adv_rope_position[0] += 1;
      a.adv_rope_position[1] += 1;
      a.adv_rope_position[2] += 1;
    }
  }
}

// PIPE: issue the next row group's loads right after the dot products (only
// worth its registers when a wave walks many row groups, i.e. the lm_head).
template <int KCH, int R, int PRO, int EPI, typename TX, typename TY, bool PIPE = (EPI == EPI_ARGMAX)>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
  constexpr int K = KCH * 512;
  constexpr int RO = (EPI == EPI_SILU) ? R / 2 : R;  // outputs per wave iteration
  static_assert(EPI != EPI_SILU || (R % 2) == 0, "SiLU epilogue works on row pairs");
  const int lane = lane_id();
  const int wpb = blockDim.x / kWave;
  const int wib = threadIdx.x / kWave;
  const long kofs = (long)blockIdx.y * K;  // split-K slice (gridDim.y == 1 otherwise)
  const long gw = (long)blockIdx.x * wpb + wib;
  const long nw = (long)gridDim.x * wpb;
  const long stride = nw * RO;
  if constexpr (EPI == EPI_STORE) {
    // read and written by this one thread only, and no other thread of the
    // launch touches either word, so next_src may equal next_dst
    if (a.next_dst != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
      a.next_dst[0] = a.next_src[0] + 1;
  }

  // The weights do not depend on the activation: issue the first row group's
  // loads before the activation prologue so the two latencies overlap.
  u32x4 wv[R][KCH];
  long o0 = gw * RO;
  if (o0 < a.N) load_rows<KCH, R, RO, EPI>(a, o0, kofs, lane, wv);

  // ---- x slice -> registers (+ prologue)
  float xr[KCH][8];
  const TX* x = reinterpret_cast<const TX*>(a.x);
#pragma unroll
  for (int c = 0; c < KCH; ++c) load_act8(x, kofs + c * 512 + lane * 8, xr[c]);
  if constexpr (PRO == PRO_ADD_RMSNORM) {
    const TX* x2 = reinterpret_cast<const TX*>(a.x2);
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      float t[8];
      load_act8(x2, c * 512 + lane * 8, t);
#pragma unroll
      for (int i = 0; i < 8; ++i) xr[c][i] += t[i];
    }
    if (a.r_out != nullptr && blockIdx.x == 0 && wib == 0) {
#pragma unroll
      for (int c = 0; c < KCH; ++c) store_act8(reinterpret_cast<TY*>(a.r_out), c * 512 + lane * 8, xr[c]);
    }
  }
  if constexpr (PRO == PRO_SILU) {
    const TX* x2 = reinterpret_cast<const TX*>(a.x2);
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      float t[8];
      load_act8(x2, kofs + c * 512 + lane * 8, t);
#pragma unroll
      for (int i = 0; i < 8; ++i) xr[c][i] = (xr[c][i] / (1.0f + __expf(-xr[c][i]))) * t[i];
    }
  }
  if constexpr (PRO == PRO_RMSNORM || PRO == PRO_ADD_RMSNORM) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < KCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(xr[c][i], xr[c][i], ss);
    ss = wave_sum(ss);
    const float rstd = rsqrtf(ss / (float)K + a.eps);
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      float g[8];
      unpack8(ld16(a.gamma + c * 512 + lane * 8), g);
#pragma unroll
      for (int i = 0; i < 8; ++i) xr[c][i] = (xr[c][i] * rstd) * g[i];
    }
  }

  float best_v = -INFINITY;
  long best_i = 0x7fffffffffffL;

  // ---- row loop: dot products of the resident rows, then the next group's
  // loads are issued before the cross-lane reductions and the epilogue.
  for (bool first = true; o0 < a.N; o0 += stride, first = false) {
    if constexpr (!PIPE) {
      if (!first) load_rows<KCH, R, RO, EPI>(a, o0, kofs, lane, wv);
    }
    float part[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < KCH; ++c) s = dot8(wv[r][c], xr[c], s);
      part[r] = s;
    }
    if constexpr (PIPE) {
      if (o0 + stride < a.N) load_rows<KCH, R, RO, EPI>(a, o0 + stride, kofs, lane, wv);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(part[r]);

    if constexpr (EPI == EPI_STORE) {
      if (lane == 0) {
        TY* y = reinterpret_cast<TY*>(a.y);
        const TY* bias = reinterpret_cast<const TY*>(a.bias);
        const TY* res = reinterpret_cast<const TY*>(a.residual);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const long o = o0 + r;
          if (o < a.N) {
            float v = acc[r];
            if (bias != nullptr) v += load_act(bias, o);
            if (res != nullptr) v += load_act(res, o);
            store_act(y, o, v);
          }
        }
      }
    } else if constexpr (EPI == EPI_SILU) {
      if (lane == 0) {
        TY* y = reinterpret_cast<TY*>(a.y);
#pragma unroll
        for (int r = 0; r < RO; ++r) {
          const long o = o0 + r;
          if (o < a.N) {
            const float g = acc[r];
            const float u = acc[r + RO];
            store_act(y, o, (g / (1.0f + __expf(-g))) * u);
          }
        }
      }
    } else if constexpr (EPI == EPI_PARTIAL) {
      if (lane == 0) {
        float* pv = a.part_val + (long)blockIdx.y * a.N;
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (o0 + r < a.N) pv[o0 + r] = acc[r];
      }
    } else {  // EPI_ARGMAX
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const long o = o0 + r;
        const float v = a.argmax_f16 ? h2f(f2h(acc[r])) : acc[r];
        if (o < a.N && v > best_v) {  // rows visited in increasing order: first max wins
          best_v = v;
          best_i = o;
        }
      }
      if (a.y != nullptr && lane == 0) {
        TY* y = reinterpret_cast<TY*>(a.y);
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (o0 + r < a.N) store_act(y, o0 + r, acc[r]);
      }
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    // per-block (max, first index), published with coherent stores and
    // reduced by the last block to arrive (a.argmax_count, self-resetting)
    __shared__ float s_v[16];
    __shared__ long s_i[16];
    __shared__ int s_last;
    if (lane == 0) {
      s_v[wib] = best_v;
      s_i[wib] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = s_v[0];
      long bi = s_i[0];
      for (int w = 1; w < wpb; ++w) {
        if (s_v[w] > bv || (s_v[w] == bv && s_i[w] < bi)) {
          bv = s_v[w];
          bi = s_i[w];
        }
      }
      store_coherent(a.part_val + blockIdx.x, bv);
      store_coherent(a.part_idx + blockIdx.x, bi);
      stores_done();
      s_last = arrive_last(a.argmax_count, gridDim.x);
    }
    __syncthreads();
    if (s_last) argmax_finish(a, (int)gridDim.x);
  }
}

// Generic fallback: any K % 8 == 0; one wave per output row, x streamed from
// global memory.  Used by the drop-in entry points for non-model shapes.
template <int PRO, typename TX, typename TY>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const GemvArgs a) {
  const int lane = lane_id();
  const long gw = (long)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const long nw = (long)gridDim.x * (blockDim.x / kWave);
  // the decoder layer's running-length advance, as in gemv_kernel's EPI_STORE
  // (one thread; next_src may equal next_dst)
  if (a.next_dst != nullptr && blockIdx.x == 0 && threadIdx.x == 0) a.next_dst[0] = a.next_src[0] + 1;
  const TX* x = reinterpret_cast<const TX*>(a.x);
  float rstd = 1.f;
  if constexpr (PRO == PRO_RMSNORM) {
    float ss = 0.f;
    for (long k = lane; k < a.K; k += kWave) {
      const float v = load_act(x, k);
      ss = __builtin_fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    rstd = rsqrtf(ss / (float)a.K + a.eps);
  }
  for (long o = gw; o < a.N; o += nw) {
    const uint16_t* wr = a.W + o * a.ldw;
    float s = 0.f;
    for (long k = lane * 8; k < a.K; k += kWave * 8) {
      float xv[8];
      load_act8(x, k, xv);
      if constexpr (PRO == PRO_RMSNORM) {
        float g[8];
        unpack8(ld16(a.gamma + k), g);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = (xv[i] * rstd) * g[i];
      }
      s = dot8(ld_stream(wr + k), xv, s);
    }
    s = wave_sum(s);
    if (lane == 0) {
      const TY* bias = reinterpret_cast<const TY*>(a.bias);
      const TY* res = reinterpret_cast<const TY*>(a.residual);
      if (bias != nullptr) s += load_act(bias, o);
      if (res != nullptr) s += load_act(res, o);
      store_act(reinterpret_cast<TY*>(a.y), o, s);
    }
  }
}

// Split-K reduce: y[o] = sum_s part[s*N + o] (+ bias[o]) in slice order.
template <typename TY>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, const TY* bias, TY* y, long N,
                                                            int splits) {
  for (long o = (long)blockIdx.x * blockDim.x + threadIdx.x; o < N; o += (long)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int p = 0; p < splits; ++p) s += part[(long)p * N + o];
    if (bias != nullptr) s += load_act(bias, o);
    store_act(y, o, s);
  }
}

// ---------------------------------------------------------------- host launchers

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

long ceil_div(long a, long b) { return (a + b - 1) / b; }

template <int KCH, int R, int PRO, int EPI, typename TX, typename TY, bool PIPE = (EPI == EPI_ARGMAX)>
int launch_fixed(const GemvArgs& a, int splits, long max_blocks, hipStream_t s) {
  constexpr int RO = (EPI == EPI_SILU) ? R / 2 : R;
  long blocks = ceil_div(ceil_div(a.N, RO), kWavesPerBlock);
  if (max_blocks > 0 && blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((gemv_kernel<KCH, R, PRO, EPI, TX, TY, PIPE>), dim3((unsigned)blocks, (unsigned)splits),
                     dim3(kThreads), 0, s, a);
  return qd_host::launch_status("gemv_kernel");
}

// Dispatch on K (per split slice) to a register-resident kernel; R rows per wave.
template <int R, int PRO, int EPI, typename TX, typename TY>
int launch_k(const GemvArgs& a, int k_slice, int splits, long max_blocks, hipStream_t s) {
  switch (k_slice) {
    case 512: return launch_fixed<1, R, PRO, EPI, TX, TY>(a, splits, max_blocks, s);
    case 1024: return launch_fixed<2, R, PRO, EPI, TX, TY>(a, splits, max_blocks, s);
    case 2048: return launch_fixed<4, R, PRO, EPI, TX, TY>(a, splits, max_blocks, s);
    case 3072: return launch_fixed<6, (R > 2 ? 2 : R), PRO, EPI, TX, TY>(a, splits, max_blocks, s);
    case 4096: return launch_fixed<8, (R > 2 ? 2 : R), PRO, EPI, TX, TY>(a, splits, max_blocks, s);
    case 6144: return launch_fixed<12, (R > 2 ? 2 : R), PRO, EPI, TX, TY>(a, splits, max_blocks, s);
    default: return 1;  // caller falls back
  }
}

bool has_fixed_k(int k) {
  return k == 512 || k == 1024 || k == 2048 || k == 3072 || k == 4096 || k == 6144;
}

}  // namespace

// Two rows per wave (8 KB of weights in flight per wave) at every N: the
// 151936 x 2048 lm_head takes 88.9-90.2 us (6.9-7.0 TB/s, the part's streaming
// read ceiling) against 94.7-97.2 with 4 rows and 96-98 with 8; qkv (N = 4096)
// 4.9 us against 5.0; 12288 rows within run-to-run spread.  (A looping launch
// for the lm_head-sized GEMV, one 4-wave workgroup per CU over row pairs with
// the next pair in flight as gemv_argmax runs, took 104.6 us.)
template <int PRO, typename TX, typename TY>
int gemv_store(const GemvArgs& a, hipStream_t s) {
  if (has_fixed_k(a.K)) return launch_k<2, PRO, EPI_STORE, TX, TY>(a, a.K, 1, 0, s);
  if constexpr (PRO == PRO_ADD_RMSNORM || PRO == PRO_SILU) return QD_ERR_SHAPE;
  long blocks = ceil_div(a.N, kWavesPerBlock);
  const long cap = (long)qd_host::cu_count() * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL((gemv_generic_kernel<PRO, TX, TY>), dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
  return qd_host::launch_status("gemv_generic_kernel");
}

template <int PRO, typename TX, typename TY>
int gemv_silu(const GemvArgs& a, hipStream_t s) {
  if (!has_fixed_k(a.K)) return QD_ERR_SHAPE;
  return launch_k<4, PRO, EPI_SILU, TX, TY>(a, a.K, 1, 0, s);
}

template <int PRO, typename TX, typename TY>
int gemv_argmax(const GemvArgs& a, hipStream_t s) {
  if (!has_fixed_k(a.K)) return QD_ERR_SHAPE;
  if (a.argmax_count == nullptr) return QD_ERR_ARG;
  // One block of 4 waves per CU, each wave looping over pairs of rows with the
  // next pair in flight: 92.2-92.6 us for the 151936 x 2048 lm_head with its
  // argmax reduction in a second launch, against 95.1-95.5 with 4 blocks per CU
  // and 96.0-96.9 with 2 or 3 (same-box sweep; 4 rows per wave: 101-102 us at
  // 1 block, 97 at 2).  With one round of blocks none waits for another, so the
  // last block to finish reduces the partials: 90.1-90.6 us, one launch.
  // A pure 16-byte streaming read of the same 622 MB peaks at 7.0-7.1 TB/s
  // with ~32 KB in flight per CU (one 4-wave workgroup, 8 loads per lane) and
  // drops to 5.3-6.3 TB/s with 4-16x as many workgroups.
  long max_blocks = (long)qd_host::cu_count();
  if (max_blocks > kMaxArgmaxBlocks) max_blocks = kMaxArgmaxBlocks;
  return launch_k<2, PRO, EPI_ARGMAX, TX, TY>(a, a.K, 1, max_blocks, s);
}

template <typename TX, typename TY>
int gemv_splitk(const GemvArgs& a, int splits, hipStream_t s) {
  const int k_slice = a.K / splits;
  if (a.K % splits != 0 || !has_fixed_k(k_slice)) return QD_ERR_SHAPE;
  int st = launch_k<4, PRO_PLAIN, EPI_PARTIAL, TX, TY>(a, k_slice, splits, 0, s);
  if (st != QD_OK) return st;
  long blocks = ceil_div(a.N, kThreads);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL((splitk_reduce_kernel<TY>), dim3((unsigned)blocks), dim3(kThreads), 0, s, a.part_val,
                     reinterpret_cast<const TY*>(a.bias), reinterpret_cast<TY*>(a.y), (long)a.N, splits);
  return qd_host::launch_status("splitk_reduce_kernel");
}

// Explicit instantiations used by the C ABI and the decode step.
template int gemv_store<PRO_PLAIN, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_store<PRO_RMSNORM, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_store<PRO_ADD_RMSNORM, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_store<PRO_SILU, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_store<PRO_PLAIN, float, float>(const GemvArgs&, hipStream_t);
template int gemv_store<PRO_RMSNORM, float, float>(const GemvArgs&, hipStream_t);
template int gemv_silu<PRO_ADD_RMSNORM, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_silu<PRO_RMSNORM, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_silu<PRO_PLAIN, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_silu<PRO_RMSNORM, float, float>(const GemvArgs&, hipStream_t);
template int gemv_argmax<PRO_RMSNORM, float, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_argmax<PRO_RMSNORM, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_argmax<PRO_PLAIN, uint16_t, uint16_t>(const GemvArgs&, hipStream_t);
template int gemv_splitk<uint16_t, uint16_t>(const GemvArgs&, int, hipStream_t);

}  // namespace qd
