// Persistent batch-1 decode step for the Qwen3-VL-2B shape on gfx950.
//
// One launch runs all 28 layers.  256 workgroups (one per CU) x 8 waves stay
// resident; every phase of a layer is split statically over the 2048 waves:
//
//   QKV      x -> qkv          2 rows of W_qkv per wave (RMSNorm prologue)
//   ATTN     qkv -> partials    workgroup = (kv head, split of 32); q/k head
//                               RMSNorm + M-RoPE + KV-cache write in the prologue;
//                               32 position slots x 16 lanes; online softmax
//   MERGE    partials -> attn   workgroup = 8 dims of one q head (wave 0)
//   O_PROJ   attn -> r          1 row of W_o per wave, + residual x
//   GATE_UP  r -> hidden        3 (gate, up) row pairs per wave, RMSNorm prologue, SiLU*up
//   DOWN     hidden -> x        1 row of W_d per wave, + residual r
//
// Weights never depend on activations, so each wave issues the register loads
// of its rows for the NEXT phase before it waits for that phase's input: the
// HBM stream of phase p+1 overlaps the hand-off latency of phase p.
//
// Hand-off between workgroups is fence-free: every produced value is written
// as one 64-bit word (fp32 value | 32-bit tag) with a relaxed agent-scope
// atomic store, and consumers poll with relaxed agent-scope 64-bit atomic
// loads until every word they need carries the expected tag.  A word is
// single-copy atomic, so a matching tag implies the matching value; no
// release/acquire (L2 write-back / invalidate) is ever issued.  Tags are
// unique per (step epoch, layer, phase); the epoch advances once per step.
//
// Every wait is bounded: a thread polls at most kSpinLimit times per launch,
// then records an error in the status word and continues, so the grid always
// drains.

#include <math.h>
#include <stdio.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

namespace {

constexpr int H = kPersistHidden, HQ = kPersistHeads, HKV = kPersistKvHeads, D = kPersistHeadDim,
              I = kPersistInter, NQKV = HQ * D + 2 * HKV * D;
constexpr int NB = kPersistBlocks;      // workgroups, one per CU
constexpr int NW = 8;                   // waves per workgroup
constexpr int NTH = NB * NW;            // waves in the grid
constexpr int NS = kPersistSplits;      // attention splits per kv head
constexpr int SLOTS = NW * 4;           // position slots per workgroup (4 rows of 16 lanes per wave)
constexpr int KU = 4;                   // K/V rows per slot per batch
constexpr int MERGE_DIMS = HQ * D / NB; // dims of one head merged per workgroup
constexpr unsigned kSpinLimit = 1u << 16;  // polls per thread and launch (tens of ms)

static_assert(NQKV == 2 * NTH, "QKV: two rows per wave");
static_assert(H == NTH, "o_proj / down: one row per wave");
static_assert(I == 3 * NTH, "gate_up: three row pairs per wave");
static_assert(MERGE_DIMS == 8, "merge: 8 dims per workgroup");

enum Phase { PH_QKV = 0, PH_ATTN = 1, PH_MERGE = 2, PH_OPROJ = 3, PH_GATEUP = 4, PH_DOWN = 5 };

__device__ __forceinline__ unsigned tag_of(unsigned ep, int layer, int phase) {
  return ep * 256u + (unsigned)(layer * 8 + phase) + 1u;
}

__device__ __forceinline__ void put(uint64_t* p, unsigned tag, float v) {
  const uint64_t word = ((uint64_t)tag << 32) | (uint64_t)__builtin_bit_cast(unsigned, v);
  __hip_atomic_store(p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t peek(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A per-lane value the compiler must treat as new at this point: keeps it from
// hoisting per-lane address arithmetic out of the layer loop (where it would
// stay live across all phases and spill).
__device__ __forceinline__ unsigned fresh(unsigned v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Polling budget of one thread for the whole launch.  A legitimate step polls
// a few times per hand-off; once the budget is spent (a workgroup that never
// produces, e.g. a grid that is not co-resident) every later wait of the
// thread gives up after one poll and the status word reports the failure, so
// the grid always drains.
struct Spin {
  unsigned left;
  unsigned* err;
};

// Tagged word at byte offset `off` of a buffer: a uniform base plus a 32-bit
// per-lane offset, so the loads use scalar-base addressing and no 64-bit
// per-lane address has to be kept.
__device__ __forceinline__ const uint64_t* word_at(const uint64_t* base, unsigned off) {
  return reinterpret_cast<const uint64_t*>(reinterpret_cast<const char*>(base) + off);
}

// Waits until every word v[k] (loaded from word_at(base, off0 + k * step))
// carries `tag`.  A lane that is still waiting re-polls all of its words
// (branch-free: one wait per poll instead of one per word).
template <int N>
__device__ __forceinline__ void await_tags(const uint64_t* base, unsigned off0, unsigned step, uint64_t (&v)[N],
                                           unsigned tag, Spin& sp) {
#pragma clang loop unroll(disable)
  while (true) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok &= (unsigned)(v[k] >> 32) == tag;
    if (ok) break;
    if (sp.left == 0) {
      __hip_atomic_fetch_or(sp.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    --sp.left;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = peek(word_at(base, off0 + k * step));
  }
}

__device__ __forceinline__ float value_of(uint64_t v) { return __builtin_bit_cast(float, (unsigned)v); }

// Value of the tagged word base[i] once its tag matches (bounded wait).
__device__ __forceinline__ float take1(const uint64_t* base, unsigned i, unsigned tag, Spin& sp) {
  uint64_t v[1] = {peek(word_at(base, i * 8u))};
  await_tags<1>(base, i * 8u, 0u, v, tag, sp);
  return value_of(v[0]);
}

// THREADS threads (consecutive ids from thread t) gather N * THREADS tagged
// values src[i] into dst[i], i = t + k * THREADS; every load is issued before
// the first wait.
template <int N, int THREADS>
__device__ __forceinline__ void gather_n(const uint64_t* src, float* dst, unsigned t, unsigned tag, Spin& sp) {
  uint64_t v[N];
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = peek(word_at(src, (t + k * THREADS) * 8u));
  await_tags<N>(src, t * 8u, THREADS * 8u, v, tag, sp);
#pragma unroll
  for (int k = 0; k < N; ++k) dst[t + k * THREADS] = value_of(v[k]);
}

// Whole workgroup (512 threads).
template <int N>
__device__ __forceinline__ void gather(const uint64_t* src, float* dst, unsigned tag, Spin& sp) {
  gather_n<N, NW * kWave>(src, dst, fresh(threadIdx.x), tag, sp);
}

template <int KCH>
__device__ __forceinline__ void load_row(const uint16_t* row, int lane, u32x4 (&w)[KCH]) {
#pragma unroll
  for (int c = 0; c < KCH; ++c) w[c] = ld_stream(row + c * 512 + lane * 8);
}

// Chunk c (8 values at c * 512 + lane * 8) of an fp32 vector in LDS.
__device__ __forceinline__ void lds8(const float* s, int c, int lane, float (&x)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(s + c * 512 + lane * 8);
  const f32x4 b = *reinterpret_cast<const f32x4*>(s + c * 512 + lane * 8 + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// rsqrt(mean(s^2) + eps) over the K = 512 * KCH values of s (whole wave).
template <int KCH>
__device__ __forceinline__ float lds_rstd(const float* s, int lane, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    float x[8];
    lds8(s, c, lane, x);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
  }
  return rsqrtf(wave_sum(ss) / (float)(KCH * 512) + eps);
}

// The dot products below read x from LDS one chunk ahead of its use and keep
// the scheduler from hoisting further reads (sched_barrier): left alone it
// issues every chunk's LDS reads up front, and with the prefetched weights of
// the next phases also live the registers run out.

// y[r] = W_r . x for R rows held in registers, x streamed chunk by chunk from LDS.
template <int KCH, int R>
__device__ __forceinline__ void rows_dot(const u32x4 (&w)[R][KCH], const float* s, int lane, float (&y)[R]) {
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  float x[8], xn[8];
  lds8(s, 0, lane, x);
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    if (c + 1 < KCH) lds8(s, c + 1, lane, xn);
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8(w[r][c], x, acc[r]);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = xn[i];
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) y[r] = wave_sum(acc[r]);
}

// y[r] = W_r . (x * rstd * gamma); the lane's gamma chunks already in registers.
template <int KCH, int R>
__device__ __forceinline__ void rows_dot_norm(const u32x4 (&w)[R][KCH], const float* s, const u32x4 (&g)[KCH],
                                              float rstd, int lane, float (&y)[R]) {
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  float x[8], xn[8];
  lds8(s, 0, lane, x);
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    if (c + 1 < KCH) lds8(s, c + 1, lane, xn);
    float gf[8];
    unpack8(g[c], gf);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (x[i] * rstd) * gf[i];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8(w[r][c], x, acc[r]);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = xn[i];
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) y[r] = wave_sum(acc[r]);
}

__device__ __forceinline__ void head_norm_rope_p(float x0, float x1, const uint16_t* w, float eps, float c, float s,
                                                 int j, float& o0, float& o1) {
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = rsqrtf(ss / (float)D + eps);
  const float n0 = (x0 * rstd) * h2f(w[j]);
  const float n1 = (x1 * rstd) * h2f(w[j + 64]);
  o0 = n0 * c - n1 * s;
  o1 = n1 * c + n0 * s;
}

// Weight streaming.  A wave's vector-memory loads complete in issue order, so a
// wave that polls a hand-off must have no load outstanding that the phase after
// the hand-off does not need (it would wait for it first).  The schedule:
//   after DOWN's input      : next layer's W_qkv rows + input-norm gamma   (all waves)
//   after QKV compute       : K/V rows, W_o row, q/k-norm weights          (all waves)
//   after attention compute : W_gate/up rows + post-norm gamma             (waves 1..7)
//   after O_PROJ's input    : the same for wave 0, which polls the split partials
//                             (MERGE) and the merged output (O_PROJ input) alone
//   after GATE_UP's input   : W_down row                                    (all waves)
// so every load is in flight across at least one hand-off and no poll waits for
// a load of a later phase.

}  // namespace

__global__ __launch_bounds__(512) void decode_persistent_kernel(const PersistArgs a) {
  const int b = blockIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: branches on it are scalar
  int lane = lane_id();
  int tid = threadIdx.x;
  const int gw = b * NW + w;
  const bool poller = (w == 0);
  const unsigned ep = a.epoch[0];
  Spin sp{kSpinLimit, a.status};

  const long pos = a.cache_position[0];
  long Ll = pos + 1 < (long)a.T ? pos + 1 : (long)a.T;
  if (Ll < 0) Ll = 0;
  const int L = (int)Ll;
  const int kvh = b % HKV;
  const int split = b / HKV;
  const int chunk = (L + NS - 1) / NS;
  const int t0 = split * chunk;
  const int t1 = min(t0 + chunk, L);
  const int mh = b / (D / MERGE_DIMS);           // merged q head of this workgroup
  const int md0 = (b % (D / MERGE_DIMS)) * MERGE_DIMS;

  __shared__ __align__(16) float s_x[H];         // layer input (residual of o_proj)
  __shared__ __align__(16) float s_att[H];       // merged attention output
  __shared__ __align__(16) float s_r[H];         // post-attention residual
  __shared__ __align__(16) float s_h[I];         // SiLU(gate) * up
  __shared__ __align__(16) float s_raw[4][D];    // raw q0, q1, k, v of this kv head
  __shared__ __align__(16) float s_q[2][D];      // rotated q
  __shared__ __align__(16) uint16_t s_kv[2][D];  // new K_rot / V rows, fp16 as cached
  __shared__ __align__(16) float s_acc[SLOTS][2][D];
  __shared__ float s_m[SLOTS][2];
  __shared__ float s_l[SLOTS][2];
  __shared__ float s_mw[NS][MERGE_DIMS + 1];

  // M-RoPE angle of rotary pair `lane` (the same for every layer of the step)
  float rc, rs;
  {
    int stream = 0;
    if (lane % 3 == 1 && lane < 3 * a.sec_h) stream = 1;
    else if (lane % 3 == 2 && lane < 3 * a.sec_w) stream = 2;
    sincosf((float)a.rope_position[stream] * a.inv_freq[lane], &rs, &rc);
  }

  u32x4 wq[2][4], gq[4];
  {
    const PersistLayer& L0 = a.layers[0];
    load_row<4>(L0.qkv + (long)(2 * gw) * H, lane, wq[0]);
    load_row<4>(L0.qkv + (long)(2 * gw + 1) * H, lane, wq[1]);
#pragma unroll
    for (int c = 0; c < 4; ++c) gq[c] = ld16(L0.input_norm + c * 512 + lane * 8);
  }

  // Lane-derived values are re-derived in every phase: otherwise the compiler
  // hoists the per-lane address arithmetic of all phases out of the layer loop
  // and the registers they occupy run out.
#define QD_FRESH_LANE() \
  do {                  \
    lane = (int)fresh((unsigned)lane); \
    tid = (int)fresh((unsigned)tid);   \
  } while (0)

  for (int l = 0; l < a.num_layers; ++l) {
    const PersistLayer& Lw = a.layers[l];

    // ================================================================ QKV
    QD_FRESH_LANE();
    if (l == 0) {
      long tok = a.token[0];
      if (tok < 0 || tok >= a.vocab) tok = 0;
      const uint16_t* row = a.embed + tok * (long)H;
      for (int i = tid; i < H; i += NW * kWave) s_x[i] = h2f(row[i]);
    } else {
      gather<H / (NW * kWave)>(a.x_t, s_x, tag_of(ep, l - 1, PH_DOWN), sp);
    }
    __syncthreads();
    {
      float y[2];
      rows_dot_norm<4, 2>(wq, s_x, gq, lds_rstd<4>(s_x, lane, a.eps), lane, y);
      if (lane == 0) {
        const unsigned tg = tag_of(ep, l, PH_QKV);
        put(a.qkv_t + 2 * gw, tg, y[0]);
        put(a.qkv_t + 2 * gw + 1, tg, y[1]);
      }
    }

    QD_FRESH_LANE();
    // issue: this workgroup's K/V rows (first batch), this wave's o_proj row,
    // the q/k head-norm weights of the rotary pair `lane`
    int row_off = lane >> 4;  // 16-lane row inside the wave
    int slot = w * 4 + row_off;
    int dl = (lane & 15) * 8;
    const uint16_t* kb = Lw.k_cache + (long)kvh * a.T * D + dl;
    const uint16_t* vb = Lw.v_cache + (long)kvh * a.T * D + dl;
    u32x4 kk[KU], vv[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int tt = t0 + slot + u * SLOTS;
      kk[u] = u32x4{0u, 0u, 0u, 0u};
      vv[u] = u32x4{0u, 0u, 0u, 0u};
      if (tt < t1 && tt != pos) {
        kk[u] = ld_stream(kb + (long)tt * D);
        vv[u] = ld_stream(vb + (long)tt * D);
      }
    }
    u32x4 wo[1][4];
    load_row<4>(Lw.o_proj + (long)gw * H, lane, wo[0]);
    const uint16_t* nw = (w == 2) ? Lw.k_norm : Lw.q_norm;
    const uint16_t nw0 = nw[lane], nw1 = nw[lane + 64];

    // ================================================================ ATTN
    QD_FRESH_LANE();
    {
      // raw q (2 heads), k, v of kv head kvh: 512 tagged values, one per thread
      int src;
      if (tid < 2 * D) src = kvh * 2 * D + tid;
      else if (tid < 3 * D) src = HQ * D + kvh * D + (tid - 2 * D);
      else src = (HQ + HKV) * D + kvh * D + (tid - 3 * D);
      s_raw[tid / D][tid % D] = take1(a.qkv_t, (unsigned)src, tag_of(ep, l, PH_QKV), sp);
    }
    __syncthreads();
    if (w < 4) {
      const int j = lane;
      const float x0 = s_raw[w][j], x1 = s_raw[w][j + 64];
      if (w < 3) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float rstd = rsqrtf(ss / (float)D + a.eps);
        const float n0 = (x0 * rstd) * h2f(nw0);
        const float n1 = (x1 * rstd) * h2f(nw1);
        const float o0 = n0 * rc - n1 * rs;
        const float o1 = n1 * rc + n0 * rs;
        if (w < 2) {
          s_q[w][j] = o0;
          s_q[w][j + 64] = o1;
        } else {
          s_kv[0][j] = f2h(o0);
          s_kv[0][j + 64] = f2h(o1);
        }
      } else {
        s_kv[1][j] = f2h(x0);
        s_kv[1][j + 64] = f2h(x1);
      }
      if (w >= 2 && pos >= t0 && pos < t1) {
        uint16_t* dst = (w == 2 ? Lw.k_cache : Lw.v_cache) + (long)kvh * a.T * D + pos * D;
        dst[j] = s_kv[w - 2][j];
        dst[j + 64] = s_kv[w - 2][j + 64];
      }
    }
    __syncthreads();
    row_off = lane >> 4;
    slot = w * 4 + row_off;
    dl = (lane & 15) * 8;
    {
      float q[2][8];
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) q[g][i] = s_q[g][dl + i];
      float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f}, acc[2][8];
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
      const int wave_t0 = t0 + w * 4;
#pragma unroll 1
      for (int tw = wave_t0; tw < t1; tw += SLOTS * KU) {
        const int t = tw + row_off;
        if (tw != wave_t0) {
#pragma unroll
          for (int u = 0; u < KU; ++u) {
            const int tt = t + u * SLOTS;
            kk[u] = u32x4{0u, 0u, 0u, 0u};
            vv[u] = u32x4{0u, 0u, 0u, 0u};
            if (tt < t1 && tt != pos) {
              kk[u] = ld_stream(kb + (long)tt * D);
              vv[u] = ld_stream(vb + (long)tt * D);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          if (t + u * SLOTS == pos && pos < t1) {
            kk[u] = *reinterpret_cast<const u32x4*>(&s_kv[0][dl]);
            vv[u] = *reinterpret_cast<const u32x4*>(&s_kv[1][dl]);
          }
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const bool valid = t + u * SLOTS < t1;
          float vf[8];
          unpack8(vv[u], vf);
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            const float s = row16_sum(dot8(kk[u], q[g], 0.f)) * a.scale;
            const float dlt = s - m[g];
            const float e = __expf(-fabsf(dlt));
            const bool up = valid && dlt > 0.f;
            const float c = up ? e : 1.f;
            const float p = valid ? (up ? 1.f : e) : 0.f;
            m[g] = up ? s : m[g];
            lsum[g] = __builtin_fmaf(lsum[g], c, p);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(acc[g][i], c, p * vf[i]);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s_acc[slot][g][dl + i] = acc[g][i];
        if ((lane & 15) == 0) {
          s_m[slot][g] = m[g];
          s_l[slot][g] = lsum[g];
        }
      }
    }
    QD_FRESH_LANE();
    __syncthreads();
    if (tid < 2 * D) {
      const int g = tid / D;
      const int d = tid % D;
      float M = -INFINITY;
#pragma unroll
      for (int s = 0; s < SLOTS; ++s) M = fmaxf(M, s_m[s][g]);
      float num = 0.f, den = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
          const float e = __expf(s_m[s][g] - M);
          den = __builtin_fmaf(s_l[s][g], e, den);
          num = __builtin_fmaf(s_acc[s][g][d], e, num);
        }
      }
      const int hq = kvh * 2 + g;
      const unsigned tg = tag_of(ep, l, PH_ATTN);
      put(a.opart_t + ((long)hq * NS + split) * D + d, tg, den > 0.f ? num / den : 0.f);
      if (d == 0) put(a.lse_t + (long)hq * NS + split, tg, den > 0.f ? M + __logf(den) : -INFINITY);
    }

    // ================================================================ MERGE + O_PROJ input (wave 0)
    QD_FRESH_LANE();
    if (poller) {
      const unsigned tg = tag_of(ep, l, PH_ATTN);
      // lanes 0..31: LSE of split `lane`; every lane: dims (lane / 32) * 4 .. +4 of split lane % 32
      const int s = lane % NS;
      const int k0 = (lane / NS) * 4;
      const unsigned lo = fresh((unsigned)((mh * NS + s) * D + md0 + k0)) * 8u;
      uint64_t ov[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) ov[k] = peek(word_at(a.opart_t, lo + k * 8u));
      const float lse = take1(a.lse_t, (unsigned)(mh * NS + s), tg, sp);
      await_tags<4>(a.opart_t, lo, 8u, ov, tg, sp);
      const float M = wave_max(lse);
      const float wgt = (M == -INFINITY) ? 0.f : __expf(lse - M);
#pragma unroll
      for (int k = 0; k < 4; ++k) s_mw[s][k0 + k] = wgt * value_of(ov[k]);
      if (lane < NS) s_mw[s][MERGE_DIMS] = wgt;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      if (lane < MERGE_DIMS) {
        float num = 0.f, den = 0.f;
        for (int t = 0; t < NS; ++t) {
          num += s_mw[t][lane];
          den += s_mw[t][MERGE_DIMS];
        }
        put(a.att_t + mh * D + md0 + lane, tag_of(ep, l, PH_MERGE), den > 0.f ? num / den : 0.f);
      }
      gather_n<H / kWave, kWave>(a.att_t, s_att, (unsigned)lane, tag_of(ep, l, PH_MERGE), sp);
    }
    // issue: this wave's gate/up row pairs and the post-attention norm gamma
    // (waves 1..7 right after the partials, wave 0 after its two polls)
    QD_FRESH_LANE();
    u32x4 wgu[6][4], gp[4];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const long o = (long)gw * 3 + p;
      load_row<4>(Lw.gate_up + o * H, lane, wgu[p]);
      load_row<4>(Lw.gate_up + (o + I) * H, lane, wgu[3 + p]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) gp[c] = ld16(Lw.post_norm + c * 512 + lane * 8);
    __syncthreads();

    // ================================================================ O_PROJ
    QD_FRESH_LANE();
    {
      float y[1];
      rows_dot<4, 1>(wo, s_att, lane, y);
      if (lane == 0) put(a.r_t + gw, tag_of(ep, l, PH_OPROJ), y[0] + s_x[gw]);
    }

    // ================================================================ GATE_UP
    QD_FRESH_LANE();
    gather<H / (NW * kWave)>(a.r_t, s_r, tag_of(ep, l, PH_OPROJ), sp);
    __syncthreads();
    u32x4 wd[1][12];
    load_row<12>(Lw.down + (long)gw * I, lane, wd[0]);
    {
      float gu[6];
      rows_dot_norm<4, 6>(wgu, s_r, gp, lds_rstd<4>(s_r, lane, a.eps), lane, gu);
      if (lane == 0) {
        const unsigned tg = tag_of(ep, l, PH_GATEUP);
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const float g = gu[p];
          put(a.hid_t + (long)gw * 3 + p, tg, (g / (1.0f + __expf(-g))) * gu[3 + p]);
        }
      }
    }

    // ================================================================ DOWN
    QD_FRESH_LANE();
    gather<I / (NW * kWave)>(a.hid_t, s_h, tag_of(ep, l, PH_GATEUP), sp);
    __syncthreads();
    if (l + 1 < a.num_layers) {
      const PersistLayer& Ln = a.layers[l + 1];
      load_row<4>(Ln.qkv + (long)(2 * gw) * H, lane, wq[0]);
      load_row<4>(Ln.qkv + (long)(2 * gw + 1) * H, lane, wq[1]);
#pragma unroll
      for (int c = 0; c < 4; ++c) gq[c] = ld16(Ln.input_norm + c * 512 + lane * 8);
    }
    {
      float y[1];
      rows_dot<12, 1>(wd, s_h, lane, y);
      if (lane == 0) {
        const float v = y[0] + s_r[gw];
        put(a.x_t + gw, tag_of(ep, l, PH_DOWN), v);
        if (l + 1 == a.num_layers) a.x_out[gw] = v;
      }
    }
  }

#undef QD_FRESH_LANE

  // The last workgroup to finish advances the epoch for the next launch.  Every
  // workgroup read the epoch before it produced anything, so none can read the
  // new value in this launch.
  __syncthreads();
  if (tid == 0) {
    const unsigned n = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n == NB - 1) {
      __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.epoch, ep + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

int decode_persistent_launch(const PersistArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(decode_persistent_kernel, dim3(NB), dim3(NW * kWave), 0, s, a);
  return qd_host::launch_status("decode_persistent_kernel");
}

int decode_persistent_check_device(char* why, size_t why_len) {
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_persistent_kernel, NW * kWave, 0);
  if (e != hipSuccess) {
    snprintf(why, why_len, "device query failed: %s", hipGetErrorString(e));
    return 1;
  }
  if ((long)cus * per_cu < NB) {
    snprintf(why, why_len, "persistent step needs %d resident workgroups; device holds %d CUs x %d", NB, cus,
             per_cu);
    return 1;
  }
  return 0;
}

}  // namespace qd
