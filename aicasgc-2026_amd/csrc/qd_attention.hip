// Split-KV GQA decode attention for gfx950 (batch 1, head_dim 128, fp16 cache).
//
// Work item = (kv head, split).  A 256-thread workgroup is 16 "slots" of 16
// lanes; slot s walks positions t = chunk_start + s, + 16, ...; within a slot
// lane j owns dims [8j, 8j+8), so one wave reads four consecutive 256-byte
// K (and V) rows per load: 1 KiB contiguous per wave and 16 B per lane.  The
// q.k dot is finished with a 4-step DPP sum inside the 16-lane row.  Every q
// head of the kv group is served from the same K/V registers, so each K/V
// element is read from HBM exactly once (the reference's q-head split-KV kernel
// reads each kv head once per q head, decode_attention_v4_kernel.cu:646-910).
//
// Online softmax per slot in fp32 (one exp per position and head); the 16 slot
// states are merged through LDS into one (normalised output, LSE) pair per
// split.  A second, tiny kernel merges the splits: the partials become visible
// to it at the launch boundary.  With arrival counters (a.done, the batch
// step) the merge runs in the partial kernel instead: each split publishes its
// partials with agent-coherent stores and counts its arrival, and the last
// split of a kv head merges all of them; no workgroup ever waits on another.
//
// The fused variant (native decode step) also performs the decode step's q/k
// head RMSNorm + M-RoPE and the static-cache write in its prologue: every
// workgroup of a kv head recomputes the rotated q, k and v of the new token
// from the raw qkv vector (4 heads x 128 values), the workgroup whose split
// holds cache_position writes K/V to the cache, and the new position is read
// from LDS instead of the cache, so no workgroup depends on another's store.

#include <math.h>

#include <mutex>
#include <vector>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

namespace {
constexpr int kFusedMergeMaxSplits = 64;   // splits per kv head the fused merge accepts
constexpr int kD = 128;
constexpr int kHalf = 64;
constexpr int kSlots = 16;
constexpr int kUnroll = 4;
}  // namespace

// RMSNorm(head) * w then rotate-half RoPE on the pair (j, j + 64) held by lane
// j; w0 / w1 are the norm weights of dims j and j + 64 (fp16 bits).
__device__ __forceinline__ void head_norm_rope(float x0, float x1, unsigned w0, unsigned w1, float eps, float c,
                                               float s, float& o0, float& o1) {
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = rsqrtf(ss / (float)kD + eps);
  const float n0 = (x0 * rstd) * h2f((uint16_t)w0);
  const float n1 = (x1 * rstd) * h2f((uint16_t)w1);
  o0 = n0 * c - n1 * s;
  o1 = n1 * c + n0 * s;
}

// Position stream of frequency slot j under interleaved M-RoPE: 1 (H) for
// j % 3 == 1 (j < 3*sec_h), 2 (W) for j % 3 == 2 (j < 3*sec_w), else 0 (T).
__device__ __forceinline__ int mrope_stream(int j, int sec_h, int sec_w) {
  if (j % 3 == 1 && j < 3 * sec_h) return 1;
  if (j % 3 == 2 && j < 3 * sec_w) return 2;
  return 0;
}

// Online-softmax update of one slot with the kUnroll positions t, t+16, ...
// as one block: the block's scores, one running-max update and one rescale of
// the accumulators per block, then one FMA per dimension and position.  A
// position >= t1 gets weight 0 (its K/V registers hold the finite row t1 - 1,
// see load_kv_batch).  Control flow is uniform across the wave, so the DPP row
// sums never run under divergent execution masks.
template <int G>
__device__ __forceinline__ void online_softmax_batch(const u32x4 (&kk)[kUnroll], const u32x4 (&vv)[kUnroll], int t,
                                                     int t1, const float (&q)[G][8], float scale, float (&m)[G],
                                                     float (&l)[G], float (&acc)[G][8]) {
  float sc[kUnroll][G];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const bool valid = t + u * kSlots < t1;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = row16_sum(dot8(kk[u], q[g], 0.f)) * scale;
      sc[u][g] = valid ? s : -INFINITY;
    }
  }
  float p[kUnroll][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mb = sc[0][g];
#pragma unroll
    for (int u = 1; u < kUnroll; ++u) mb = fmaxf(mb, sc[u][g]);
    const float mn = fmaxf(m[g], mb);
    // mn == -inf: nothing valid yet; keep the (zero) sums as they are
    const float c = mn == -INFINITY ? 1.f : __expf(m[g] - mn);
    float ps = 0.f;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      p[u][g] = sc[u][g] == -INFINITY ? 0.f : __expf(sc[u][g] - mn);
      ps += p[u][g];
    }
    l[g] = __builtin_fmaf(l[g], c, ps);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] *= c;
    m[g] = mn;
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    float vf[8];
    unpack8(vv[u], vf);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(p[u][g], vf[i], acc[g][i]);
  }
}

// K/V rows of positions t, t+16, ... into registers.  The loads are
// unconditional (rows past t1 re-read row t1 - 1, an L1/L2 hit) and the number
// of loads in flight is the same on every path, so a wave waits only for the
// batch it consumes.  The softmax gives positions >= t1 weight 0 and their V
// registers are zeroed before use: in the fused variant row t1 - 1 can be the
// new position, whose cache row still holds stale data when it is loaded (it is
// replaced from LDS only where it is the slot's own position), and a weight of
// 0 times a non-finite value would still be NaN.
__device__ __forceinline__ void load_kv_batch(const uint16_t* kb, const uint16_t* vb, long stride_s, int t, int t1,
                                              u32x4 (&kk)[kUnroll], u32x4 (&vv)[kUnroll]) {
  const int last = t1 > 0 ? t1 - 1 : 0;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int tt = min(t + u * kSlots, last);
    kk[u] = ld_stream(kb + (long)tt * stride_s);
    vv[u] = ld_stream(vb + (long)tt * stride_s);
  }
}

// ---------------------------------------------------------------- batch qkv hand-off
//
// attention_qkv8_launch runs the batch step's qkv GEMV in the attention launch:
// workgroup p < kQkv8Producers computes rows [16 p, 16 p + 16) of every
// sequence's qkv vector and stores each value as a 32-bit word whose mantissa
// LSB carries the parity of the launch (hgen); the workgroups of a (sequence,
// kv head) poll the 512 words they need until every one shows that parity.
// Each word is written once per launch, so consecutive writes alternate their
// parity and a reader can only see the previous write or the awaited one.  The
// producers are the first workgroups of the grid, dispatched first, and wait
// only for each other; the other workgroups wait only for them.  A wait is
// bounded: past its polling budget it records bit 0 in the status word and
// hands NaN on (every output of the launch is then NaN, none looks valid).

constexpr unsigned kQkvSpinLimit = 1u << 16;   // polls per thread and launch (tens of ms)
constexpr int kQkvK = 2048;                    // K of the qkv GEMV
constexpr int kQkvWaves = 4;                   // K slices of a producer (one per wave)
constexpr int kQkvKS = kQkvK / kQkvWaves;      // 512
constexpr int kQkvNT = kQkvKS / 32;            // MFMA K tiles per wave
constexpr unsigned kQkvPoison = 0x7fc00000u;   // quiet NaN, tag bit clear

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

__device__ __forceinline__ u32x4 bperm4(int addr, const u32x4& v) {
  return u32x4{(unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.x), (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.y),
               (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.z), (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)v.w)};
}

__device__ __forceinline__ unsigned tagged_word(float v, unsigned par) {
  return (__builtin_bit_cast(unsigned, v) & ~1u) | par;
}

__device__ __forceinline__ unsigned peek_word(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Values of words p[0] and p[o1] once both show parity `par` (bounded wait;
// `left` is the thread's remaining polling budget for the launch).
__device__ __forceinline__ void take_words(const unsigned* p, long o1, unsigned par, unsigned& left,
                                           unsigned* status, float& v0, float& v1) {
  unsigned w0 = peek_word(p), w1 = peek_word(p + o1);
#pragma clang loop unroll(disable)
  while ((((w0 ^ par) | (w1 ^ par)) & 1u) != 0u) {
    if (left == 0) {
      __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      w0 = w1 = kQkvPoison;
      break;
    }
    --left;
    __builtin_amdgcn_s_sleep(1);
    w0 = peek_word(p);
    w1 = peek_word(p + o1);
  }
  v0 = __builtin_bit_cast(float, w0 & ~1u);
  v1 = __builtin_bit_cast(float, w1 & ~1u);
}

// Inputs of one producer's GEMV, loaded in the order they are used: the image
// tiles of the wave's K slice, the norm partial sums of the wave's two
// sequences, then the weights (16 rows x 512 K per wave as coalesced 128-byte
// row pieces: load 2 j + h covers rows 8 h .. 8 h + 7, K 64 j .. 64 j + 64 of
// the slice, 8 lanes x 16 bytes per row).
struct Qkv8In {
  u32x4 bt[kQkvNT];
  u32x4 wt[kQkvNT];
  float ss[2][4];
};

template <bool TILED>
__device__ __forceinline__ void qkv8_load(const AttnArgs& a, int p, int w, int lane, Qkv8In& in) {
  const long kb = (long)w * kQkvKS;
  const u32x4* src = reinterpret_cast<const u32x4*>(a.xb) + (kb / 32) * 64 + lane;
#pragma unroll
  for (int i = 0; i < kQkvNT; ++i) in.bt[i] = src[i * 64];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int seq = 2 * w + q;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int part = lane + i * kWave;
      in.ss[q][i] = part < a.in_parts ? a.in_ss[(long)part * kBatchMax + seq] : 0.f;
    }
  }
  if constexpr (TILED) {
    // tile order: tile t of the slice is one contiguous 1 KB, already the MFMA operand
    const uint16_t* tp = a.wqkv + ((long)p * (kQkvK / 8) + kb / 8) * 128 + lane * 8;
#pragma unroll
    for (int i = 0; i < kQkvNT; ++i) in.wt[i] = ld_stream(tp + 512L * i);
    return;
  }
  const uint16_t* wp = a.wqkv + ((long)p * 16 + (lane >> 3)) * kQkvK + kb + (lane & 7) * 8;
#pragma unroll
  for (int j = 0; j < kQkvNT / 2; ++j) {
    in.wt[2 * j] = ld_stream(wp + 64 * j);
    in.wt[2 * j + 1] = ld_stream(wp + 8L * kQkvK + 64 * j);
  }
}

// The producer's rows: MFMA over the wave's K slice (C[r][n] + C[r][n + 8] is
// row r of sequence n), the 4 slices summed through LDS, scaled by
// rstd / in_scale of the sequence and stored as tagged words.  Every thread of
// the workgroup calls it (it contains workgroup barriers).
template <bool TILED>
__device__ __forceinline__ void qkv8_produce(const AttnArgs& a, int p, int w, int lane, const Qkv8In& in,
                                             unsigned par, float (&s_part)[kQkvWaves][kBatchMax][16],
                                             float (&s_fac)[kBatchMax]) {
  const int m = lane & 15;
  const int src0 = (8 * (m & 7) + (lane >> 4)) * 4;   // ds_bpermute byte addresses
  const int src1 = src0 + 16;
  const bool upper = m >= 8;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kQkvNT / 2; ++j) {
    u32x4 t0 = in.wt[2 * j], t1 = in.wt[2 * j + 1];
    if constexpr (!TILED) {
      const u32x4 a0 = bperm4(src0, in.wt[2 * j]), a1 = bperm4(src1, in.wt[2 * j]);
      const u32x4 b0 = bperm4(src0, in.wt[2 * j + 1]), b1 = bperm4(src1, in.wt[2 * j + 1]);
      t0 = upper ? b0 : a0;
      t1 = upper ? b1 : a1;
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, t0), __builtin_bit_cast(h8v, in.bt[2 * j]),
                                                 acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, t1),
                                                 __builtin_bit_cast(h8v, in.bt[2 * j + 1]), acc, 0, 0, 0);
  }
  {
    const int g = lane >> 4;
    const float c[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = c[j] + dpp<kDppRowRor8>(c[j]);
      if (m < kBatchMax) s_part[w][m][4 * g + j] = v;
    }
  }
  // factor of sequences 2 w and 2 w + 1: rstd of x / the image's scale (0 past nseq)
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int seq = 2 * w + q;
    const float ss = wave_sum((in.ss[q][0] + in.ss[q][1]) + (in.ss[q][2] + in.ss[q][3]));
    float f = rsqrtf(ss / (float)kQkvK + a.eps);
    if (a.in_scale != nullptr) f /= a.in_scale[seq];
    if (seq >= a.batch) f = 0.f;
    if (lane == 0) s_fac[seq] = f;
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < kBatchMax * 16) {
    const int seq = t >> 4, rl = t & 15;
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < kQkvWaves; ++q) v += s_part[q][seq][rl];
    v *= s_fac[seq];
    // every sequence slot's word, also past the batch (factor 0), so each word
    // is written once per launch whatever batch the launches on this
    // workspace run
    __hip_atomic_store(a.qkv_t + (long)seq * kQkv8Producers * 16 + p * 16 + rl, tagged_word(v, par),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  stores_done();   // polling with a store of the wave still in flight is much slower
}

template <int G, typename TQ, bool FUSED_ROPE, bool XQKV = false, bool WT = false>
__global__ __launch_bounds__(256) void attn_partial_kernel(const AttnArgs a) {
  static_assert(!XQKV || (G == 2 && FUSED_ROPE), "the qkv hand-off serves the fused batch prologue");
  // XQKV: one-dimensional grid in dispatch order, sequence-major
  const int bx = XQKV ? (int)(blockIdx.x % (unsigned)(a.Hkv * a.n_split)) : (int)blockIdx.x;
  const int kvh = bx / a.n_split;
  const int split = bx % a.n_split;
  const int slot = threadIdx.x >> 4;
  const int dl = (threadIdx.x & 15) * 8;
  // sequence of a batch (grid y); every per-sequence pointer is offset here
  const int bq = XQKV ? (int)(blockIdx.x / (unsigned)(a.Hkv * a.n_split)) : (int)blockIdx.y;
  const TQ* q_in = reinterpret_cast<const TQ*>(a.q) + bq * a.bs_q;
  const TQ* qkv = reinterpret_cast<const TQ*>(a.qkv) + bq * a.bs_q;
  const uint16_t* kc = a.k + bq * a.bs_cache;
  const uint16_t* vc = a.v + bq * a.bs_cache;
  uint16_t* kw = a.k_w + bq * a.bs_cache;
  uint16_t* vw = a.v_w + bq * a.bs_cache;
  const int64_t* rope_pos = a.rope_pos + 3 * bq;
  const long part0 = (long)bq * a.Hq * a.n_split;
  float* o_part = a.o_part + part0 * kD;
  float* lse_out = a.lse + part0;
  float* q_rot_out = a.q_rot_out == nullptr ? nullptr : a.q_rot_out + (long)bq * a.Hq * kD;

  // XQKV: the launch's parity, and a producer's GEMV inputs ahead of every
  // other load (a wave's loads complete in issue order)
  unsigned gen = 0u, par = 0u;
  const bool producer = XQKV && blockIdx.x < (unsigned)kQkv8Producers;
  Qkv8In qin;
  if constexpr (XQKV) {
    gen = __hip_atomic_load(a.hgen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    par = (gen + 1u) & 1u;
    if (producer) qkv8_load<WT>(a, (int)blockIdx.x, (int)(threadIdx.x / kWave), lane_id(), qin);
  }

  const long pos = a.cache_position[bq];
  long Ll = pos + 1 < (long)a.T ? pos + 1 : (long)a.T;
  if (Ll < 0) Ll = 0;
  const int L = (int)Ll;
  const int chunk = (L + a.n_split - 1) / a.n_split;
  const int t0 = min(split * chunk, L);
  const int t1 = min(t0 + chunk, L);

  // The cache rows do not depend on the prologue: the first batch of K/V loads
  // is issued before it (the new position, if in this batch, is patched in from
  // LDS afterwards).
  const uint16_t* kb = kc + (long)kvh * a.stride_h + dl;
  const uint16_t* vb = vc + (long)kvh * a.stride_h + dl;
  // The wave's four slots advance together (trip count uniform per wave).
  const int wave_t0 = t0 + (threadIdx.x / kWave) * 4;
  const int row_off = slot - (threadIdx.x / kWave) * 4;

  // The prologue's own inputs are loaded first, then two batches of K/V rows
  // (A: kk/vv, B: kn/vn), which do not depend on the prologue.  Loads complete
  // in issue order, so the prologue waits only for its inputs while the K/V rows
  // are in flight.  A and B alternate roles in the loop below (no register
  // copies, which would wait for the loads).
  constexpr int kPre = (G + 2 + 3) / 4;   // prologue items (q heads, k, v) per wave
  const int w = threadIdx.x / kWave;
  const int j = lane_id();
  float pre[kPre][2] = {};
  unsigned pw[kPre][2] = {};   // fp16 bits, one per register (packing would wait for the loads)
  float ifq = 0.f;
  float q[G][8];
  // (A load issued behind the K/V rows of every workgroup would wait for them in
  // the memory queues, several microseconds at launch.  The rope position of
  // rotary pair j is a per-lane vector load: a scalar load is waited for with
  // every other outstanding scalar load, and the K/V addressing has some.)
  long rpj = 0;
  float cs_c = 0.f, cs_s = 0.f;   // given cos / sin of slot j (a.cos set)
  if constexpr (FUSED_ROPE) {
    if (a.cos != nullptr) {
      cs_c = h2f(a.cos[(long)bq * kD + j]);
      cs_s = h2f(a.sin[(long)bq * kD + j]);
    } else {
      ifq = a.inv_freq[j];
      rpj = rope_pos[mrope_stream(j, a.sec_h, a.sec_w)];
    }
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int item = w + 4 * i;
      if (item < G + 2) {
        if constexpr (!XQKV) {
          const TQ* src = item < G    ? qkv + (long)(kvh * G + item) * kD
                          : item == G ? qkv + (long)a.Hq * kD + (long)kvh * kD
                                      : qkv + (long)(a.Hq + a.Hkv) * kD + (long)kvh * kD;
          pre[i][0] = load_act(src, j);
          pre[i][1] = load_act(src, j + kHalf);
        }
        if (item <= G) {
          const uint16_t* nw = item < G ? a.q_weight : a.k_weight;
          pw[i][0] = nw[j];
          pw[i][1] = nw[j + kHalf];
        }
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) load_act8(q_in, (long)(kvh * G + g) * a.q_stride + dl, q[g]);
  }
  constexpr int kStep = kSlots * kUnroll;
  u32x4 kk[kUnroll], vv[kUnroll], kn[kUnroll], vn[kUnroll];
  // XQKV: only the first batch is requested before the hand-off.  A wave's
  // loads complete in issue order and the memory side serves the chip's
  // requests in order, so every K/V batch requested before the polls delays
  // them by its drain time, while one batch in flight keeps HBM busy as the
  // producers' rows arrive (measured: both batches first, or none, ran slower
  // than the qkv GEMV as a launch of its own; one batch first ran faster).
  __builtin_amdgcn_sched_barrier(0);   // every prologue input is requested before the K/V rows
  load_kv_batch(kb, vb, a.stride_s, wave_t0 + row_off, t1, kk, vv);
  if constexpr (!XQKV) load_kv_batch(kb, vb, a.stride_s, wave_t0 + kStep + row_off, t1, kn, vn);
  __builtin_amdgcn_sched_barrier(0);   // the batches issued before the prologue's math waits

  if constexpr (XQKV) {
    __shared__ float s_part[kQkvWaves][kBatchMax][16];
    __shared__ float s_fac[kBatchMax];
    if (producer) qkv8_produce<WT>(a, (int)blockIdx.x, w, j, qin, par, s_part, s_fac);
    // this sequence's raw q (G heads), k and v of kv head kvh, as the words show them
    unsigned left = a.spin_limit != 0u ? a.spin_limit : kQkvSpinLimit;
    const unsigned* words = a.qkv_t + (long)bq * kQkv8Producers * 16;
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int item = w + 4 * i;
      if (item < G + 2) {
        const long row = item < G    ? (long)(kvh * G + item) * kD
                         : item == G ? (long)a.Hq * kD + (long)kvh * kD
                                     : (long)(a.Hq + a.Hkv) * kD + (long)kvh * kD;
        take_words(words + row + j, kHalf, par, left, a.status, pre[i][0], pre[i][1]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // the second batch behind the polls
    load_kv_batch(kb, vb, a.stride_s, wave_t0 + kStep + row_off, t1, kn, vn);
    __builtin_amdgcn_sched_barrier(0);
  }

  __shared__ float s_q[G][kD];
  __shared__ __align__(16) uint16_t s_kv[2][kD];   // new token's K_rot and V, fp16 as cached
  if constexpr (FUSED_ROPE) {
    float c = cs_c, s = cs_s;
    if (a.cos == nullptr) sincosf((float)rpj * ifq, &s, &c);
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int item = w + 4 * i;
      if (item < G) {
        float o0, o1;
        head_norm_rope(pre[i][0], pre[i][1], pw[i][0], pw[i][1], a.eps, c, s, o0, o1);
        s_q[item][j] = o0;
        s_q[item][j + kHalf] = o1;
      } else if (item == G) {
        float o0, o1;
        head_norm_rope(pre[i][0], pre[i][1], pw[i][0], pw[i][1], a.eps, c, s, o0, o1);
        s_kv[0][j] = f2h(o0);
        s_kv[0][j + kHalf] = f2h(o1);
      } else if (item == G + 1) {
        s_kv[1][j] = f2h(pre[i][0]);
        s_kv[1][j + kHalf] = f2h(pre[i][1]);
      }
    }
    __syncthreads();
    // the split holding the new position stores it into the static cache
    if (pos >= t0 && pos < t1) {
      const int t = threadIdx.x;
      uint16_t* dst = (t < kD ? kw : vw) + (long)kvh * a.stride_h + pos * a.stride_s;
      dst[t & (kD - 1)] = s_kv[t >> 7][t & (kD - 1)];
    }
    // rotated q for inspection by the host (first split of each kv head)
    if (split == 0 && q_rot_out != nullptr) {
      for (int i = threadIdx.x; i < G * kD; i += blockDim.x)
        q_rot_out[(long)kvh * G * kD + i] = s_q[i / kD][i % kD];
    }
  }

  if constexpr (FUSED_ROPE) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) q[g][i] = s_q[g][dl + i];
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }

  // the new position comes from LDS (fp16, as written to the cache); positions
  // past t1 contribute exact zeros (their scores are -inf, their V cleared)
  auto consume = [&](u32x4 (&bk)[kUnroll], u32x4 (&bv)[kUnroll], int t) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (FUSED_ROPE) {
        if (t + u * kSlots == pos && pos < t1) {
          bk[u] = *reinterpret_cast<const u32x4*>(&s_kv[0][dl]);
          bv[u] = *reinterpret_cast<const u32x4*>(&s_kv[1][dl]);
        }
      }
      if (t + u * kSlots >= t1) bv[u] = u32x4{0u, 0u, 0u, 0u};
    }
    online_softmax_batch<G>(bk, bv, t, t1, q, a.scale, m, l, acc);
  };
#pragma unroll 1
  for (int tw = wave_t0; tw < t1; tw += 2 * kStep) {
    consume(kk, vv, tw + row_off);
    load_kv_batch(kb, vb, a.stride_s, tw + 2 * kStep + row_off, t1, kk, vv);
    if (tw + kStep < t1) consume(kn, vn, tw + kStep + row_off);
    load_kv_batch(kb, vb, a.stride_s, tw + 3 * kStep + row_off, t1, kn, vn);
  }

  // ---- merge the 16 slots of this workgroup into one (output, LSE) per q head
  __shared__ float s_acc[kSlots][G][kD];
  __shared__ float s_m[kSlots][G];
  __shared__ float s_l[kSlots][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int i = 0; i < 8; ++i) s_acc[slot][g][dl + i] = acc[g][i];
    if ((threadIdx.x & 15) == 0) {
      s_m[slot][g] = m[g];
      s_l[slot][g] = l[g];
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < G * kD; t += blockDim.x) {
    const int g = t / kD;
    const int d = t % kD;
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) M = fmaxf(M, s_m[s][g]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int s = 0; s < kSlots; ++s) {
        const float w = __expf(s_m[s][g] - M);
        den = __builtin_fmaf(s_l[s][g], w, den);
        num = __builtin_fmaf(s_acc[s][g][d], w, num);
      }
    }
    const int h = kvh * G + g;
    const float o = den > 0.f ? num / den : 0.f;
    const float lse = den > 0.f ? M + __logf(den) : -INFINITY;
    if (a.done == nullptr) {
      o_part[((long)h * a.n_split + split) * kD + d] = o;
      if (d == 0) lse_out[(long)h * a.n_split + split] = lse;
    } else {
      store_coherent(o_part + ((long)h * a.n_split + split) * kD + d, o);
      if (d == 0) store_coherent(lse_out + (long)h * a.n_split + split, lse);
    }
  }
  if (a.done == nullptr) return;

  // ---- fused merge: the last split of this kv head to finish combines all of them
  __shared__ int s_last;
  stores_done();
  __syncthreads();
  if (threadIdx.x == 0) {
    s_last = arrive_last(a.done + (long)bq * a.Hkv + kvh, (unsigned)a.n_split);
    // XQKV: every workgroup read the launch's parity long before; the last to
    // arrive advances it for the next launch
    if (XQKV && arrive_last(a.hdone, gridDim.x))
      __hip_atomic_store(a.hgen, gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  const int S = a.n_split;
  // Thread (g, d) reads the LSEs and partials of kMergeBatch splits at a time,
  // every load of a batch issued before the first is used (unconditional, index
  // clamped to the last split; a clamped duplicate gets weight 0), so a batch
  // costs one round trip to the coherence point.  Weights are exp(lse_s - M)
  // with M the running maximum, rescaled when a later batch raises it (with
  // S <= kMergeBatch: exactly the maximum over all splits); empty splits have
  // lse = -inf and weight 0.
  constexpr int kMergeBatch = 8;
  for (int t = threadIdx.x; t < G * kD; t += blockDim.x) {
    const int g = t / kD;
    const int d = t % kD;
    const int h = kvh * G + g;
    float mrun = -INFINITY, num = 0.f, den = 0.f;
    float* op = o_part + (long)h * S * kD + d;
    float* lp = lse_out + (long)h * S;
    for (int s0 = 0; s0 < S; s0 += kMergeBatch) {
      float lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int s = min(s0 + u, S - 1);
        lv[u] = load_coherent(lp + s);
        ov[u] = load_coherent(op + (long)s * kD);
      }
      float bm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u)
        if (s0 + u < S) bm = fmaxf(bm, lv[u]);
      if (bm > mrun) {
        const float c = __expf(mrun - bm);   // mrun = -inf: c = 0 and num = den = 0 stay 0
        num *= c;
        den *= c;
        mrun = bm;
      }
      if (mrun != -INFINITY) {
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
          const float w = s0 + u < S ? __expf(lv[u] - mrun) : 0.f;
          den += w;
          num = __builtin_fmaf(w, ov[u], num);
        }
      }
    }
    const float o = den > 0.f ? num / den : 0.f;
    if (a.out_img != nullptr)
      bimg_store(a.out_img, bq, (long)h * kD + d, o);
    else
      store_act(reinterpret_cast<TQ*>(a.out) + (long)bq * a.Hq * kD, (long)h * kD + d, o);
  }
}

// out[h, d] = sum_s w_s o_s[d] / sum_s w_s with w_s = exp(lse_s - max lse).
// One wave per (q head, half of the 128 dims): lane s reads the LSE of split s
// and every lane the partials of its dim for 64 splits, every load issued
// before the first is used (unconditional, index clamped to the last split; a
// clamped duplicate gets weight 0), so up to 64 splits cost one round trip.
// Lane s's weight reaches the other lanes by readlane.  More splits run in
// chunks of 64 with a running maximum.  Empty splits (lse = -inf) weigh 0; a
// NaN LSE makes the sum of weights NaN and the output 0, as in the in-kernel
// merge.
constexpr int kMergeMaxSplits = 1024;
constexpr int kMergeChunk = kWave;

template <typename TO>
__global__ __launch_bounds__(kWave) void attn_merge_kernel(const AttnArgs a) {
  const int h = (int)(blockIdx.x >> 1);
  const int lane = lane_id();
  const int d = (int)(blockIdx.x & 1u) * kWave + lane;
  const int S = a.n_split;
  const long bq = blockIdx.y;   // sequence of a batch
  const float* lse = a.lse + (bq * a.Hq + h) * S;
  const float* op = a.o_part + (bq * a.Hq + h) * S * kD + d;
  float M = -INFINITY, num = 0.f, den = 0.f;
  for (int c = 0; c < S; c += kMergeChunk) {
    const int n = min(kMergeChunk, S - c);
    const float l = lane < n ? lse[c + lane] : -INFINITY;
    float v[kMergeChunk];
#pragma unroll
    for (int u = 0; u < kMergeChunk; ++u) v[u] = op[(long)min(c + u, S - 1) * kD];
    const float mn = fmaxf(M, wave_max(l));
    if (mn != -INFINITY) {
      const float r = M == -INFINITY ? 0.f : __expf(M - mn);   // num = den = 0 while M = -inf
      num *= r;
      den *= r;
      const float w = __expf(l - mn);                            // 0 for lanes >= n
      den += wave_sum(w);
#pragma unroll
      for (int u = 0; u < kMergeChunk; ++u) num = __builtin_fmaf(readlane(w, u), v[u], num);
      M = mn;
    }
  }
  const float o = den > 0.f ? num / den : 0.f;
  if (a.out_img != nullptr)
    bimg_store(a.out_img, (int)bq, (long)h * kD + d, o);
  else
    store_act(reinterpret_cast<TO*>(a.out), (bq * a.Hq + h) * kD + d, o);
}

template <typename TQ, bool FUSED>
static int launch_partial_g(const AttnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.Hkv * a.n_split), (unsigned)a.batch);
  switch (a.Hq / a.Hkv) {
    case 1: hipLaunchKernelGGL((attn_partial_kernel<1, TQ, FUSED>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_partial_kernel<2, TQ, FUSED>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_partial_kernel<4, TQ, FUSED>), grid, dim3(256), 0, s, a); break;
    default: return QD_ERR_SHAPE;
  }
  return qd_host::launch_status("attn_partial_kernel");
}

template <typename TQ>
int attention_partial_launch(const AttnArgs& a, hipStream_t s) {
  if (a.done != nullptr && a.n_split > kFusedMergeMaxSplits) return QD_ERR_SHAPE;
  return a.qkv != nullptr ? launch_partial_g<TQ, true>(a, s) : launch_partial_g<TQ, false>(a, s);
}

bool attention_qkv8_device_ok() {
  static std::mutex mu;
  static std::vector<signed char> ok;   // per device: -1 unknown, 0 no, 1 yes
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)ok.size() <= dev) ok.resize(dev + 1, -1);
  if (ok[dev] < 0) {
    int cus = 0, per_cu = 0;
    int per_cu_t = 0;
    const bool q = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                   hipOccupancyMaxActiveBlocksPerMultiprocessor(
                       &per_cu, reinterpret_cast<const void*>(&attn_partial_kernel<2, float, true, true>), 256, 0) ==
                       hipSuccess &&
                   hipOccupancyMaxActiveBlocksPerMultiprocessor(
                       &per_cu_t, reinterpret_cast<const void*>(&attn_partial_kernel<2, float, true, true, true>), 256,
                       0) == hipSuccess;
    if (per_cu_t < per_cu) per_cu = per_cu_t;
    ok[dev] = (q && (long)cus * per_cu >= kQkv8Producers) ? 1 : 0;
    (void)hipGetLastError();
  }
  return ok[dev] == 1;
}

int attention_qkv8_launch(const AttnArgs& a, hipStream_t s) {
  const long grid = (long)a.batch * a.Hkv * a.n_split;
  if (a.Hq != 2 * a.Hkv || (a.Hq + 2 * a.Hkv) * kD != kQkv8Producers * 16 || grid < kQkv8Producers ||
      a.batch < 1 || a.batch > kBatchMax || a.done == nullptr || a.out_img == nullptr || a.n_split > kFusedMergeMaxSplits ||
      a.wqkv == nullptr || a.xb == nullptr || a.in_ss == nullptr || a.in_parts < 1 || a.in_parts > 4 * kWave ||
      a.qkv_t == nullptr || a.hgen == nullptr || a.hdone == nullptr || a.status == nullptr)
    return QD_ERR_SHAPE;
  if (a.wqkv_tiled)
    hipLaunchKernelGGL((attn_partial_kernel<2, float, true, true, true>), dim3((unsigned)grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((attn_partial_kernel<2, float, true, true>), dim3((unsigned)grid), dim3(256), 0, s, a);
  return qd_host::launch_status("attn_partial_kernel<qkv>");
}

template <typename TO>
int attention_merge_launch(const AttnArgs& a, hipStream_t s) {
  if (a.n_split > kMergeMaxSplits) return QD_ERR_SHAPE;
  hipLaunchKernelGGL((attn_merge_kernel<TO>), dim3(2u * (unsigned)a.Hq, (unsigned)a.batch), dim3(kWave), 0, s, a);
  return qd_host::launch_status("attn_merge_kernel");
}

template int attention_partial_launch<uint16_t>(const AttnArgs&, hipStream_t);
template int attention_partial_launch<float>(const AttnArgs&, hipStream_t);
template int attention_merge_launch<uint16_t>(const AttnArgs&, hipStream_t);
template int attention_merge_launch<float>(const AttnArgs&, hipStream_t);

}  // namespace qd
