// Persistent batch-1 decode step for the Qwen3-VL-2B shape on gfx950.
//
// One launch runs all 28 layers.  256 workgroups (one per CU) x 8 waves stay
// resident; every phase of a layer is split statically over the 2048 waves:
//
//   QKV      x -> qkv          2 rows of W_qkv per wave (RMSNorm: the x gather
//                               stores x * gamma and the waves' sums of x^2;
//                               each dot product is scaled by rstd)
//   ATTN     qkv -> partials    workgroup = (kv head, split of 32); q/k head
//                               RMSNorm + M-RoPE + KV-cache write in the prologue;
//                               32 position slots x 16 lanes; online softmax
//   MERGE    partials -> attn   workgroup = 8 dims of one q head (wave 0)
//   O_PROJ   attn -> r          1 row of W_o per wave, + residual x
//   GATE_UP  r -> hidden        3 (gate, up) row pairs per wave, RMSNorm as for QKV, SiLU*up
//   DOWN     hidden -> x        1 row of W_d per wave, + residual r
//
// Weights never depend on activations, so each wave issues the register loads
// of its rows for the NEXT phase before it waits for that phase's input: the
// HBM stream of phase p+1 overlaps the hand-off latency of phase p.
//
// Hand-off between workgroups is fence-free.  Every produced value is one
// 32-bit word: the fp32 value with its mantissa LSB replaced by the parity of
// the write, stored with a relaxed agent-scope atomic store; readers clear
// that bit again, so every reader uses the value with its LSB cleared (a
// change of at most one ulp, the same in every launch).  Consumers read 16
// bytes per lane with device-coherent (sc1)
// buffer loads and poll until every word shows the parity they expect; no
// release/acquire (L2 write-back / invalidate) is ever issued.  Each buffer is
// written once per layer and every reader reads the same words at every layer,
// so the parity alternates between consecutive writes and a reader, having
// seen the previous write, can only see that write (wrong parity) or the one
// it waits for: one bit is a complete tag.  The hidden vector (GATE_UP ->
// DOWN), whose reader takes it as fp16 anyway, moves as 64-bit words of three
// fp16 values and a 16-bit tag (one word per wave, one 64-bit store): 16
// instead of 24 KB per workgroup to gather, no value bit given to the tag.
// A wave waits for its own stores to complete before it polls; polling with a
// store in flight is several times slower on this part.  The words live in one
// uncached area per device, shared by every persistent launch on it; the
// parity follows a per-device layer generation, so launches of different
// layer counts keep the sequence.
//
// Every wait is bounded: a thread polls at most kSpinLimit times per launch,
// then records an error in the status word and continues, so the grid always
// drains.
//
// A second instance of the kernel (LAYER) runs one decoder layer for the
// drop-in layer's forward: its input is the caller's fp16 hidden state
// instead of an embedding row, the rotation uses the caller's cos / sin
// (transformers' rotary embedding), its output is fp16, and the last
// workgroup sets the cache's running length to cache_position + 1.

#include <float.h>
#include <math.h>
#include <stdio.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

// Phase timestamps (library built with -DQD_TRACE only): the first thread of
// wave 0 (a poller, events 0..15) and of wave 4 (a streamer, events 16..31)
// of every workgroup record the 100 MHz real-time clock at fixed points of
// each layer of the last launch; qd_persistent_trace_read copies them out.
constexpr int kTraceLayers = 32, kTraceEvents = 32;
#ifdef QD_TRACE
__device__ unsigned long long qd_trace_stamps[kPersistBlocks * kTraceLayers * kTraceEvents];
#define QD_TRACE_BY(tid0, l, e)                                                                   \
  do {                                                                                           \
    if (threadIdx.x == (tid0))                                                                   \
      qd_trace_stamps[((size_t)blockIdx.x * kTraceLayers + (l)) * kTraceEvents + (e)] =          \
          __builtin_amdgcn_s_memrealtime();                                                      \
  } while (0)
#else
#define QD_TRACE_BY(tid0, l, e) \
  do {                          \
  } while (0)
#endif
#define QD_TRACE_AT(l, e) QD_TRACE_BY(0, l, e)                  // poller wave 0
#define QD_TRACE_ST(l, e) QD_TRACE_BY(4 * kWave, l, 16 + (e))   // streamer wave 4

namespace {

constexpr int H = kPersistHidden, HQ = kPersistHeads, HKV = kPersistKvHeads, D = kPersistHeadDim,
              I = kPersistInter, NQKV = HQ * D + 2 * HKV * D;
constexpr int NB = kPersistBlocks;      // workgroups, one per CU
constexpr int NW = 8;                   // waves per workgroup
constexpr int NTH = NB * NW;            // waves in the grid
constexpr int NA = 4;                   // waves 0..NA-1 poll the hand-offs; the others only stream
constexpr int NS = kPersistSplits;      // attention splits per kv head
constexpr int SLOTS = NW * 4;           // position slots per workgroup (4 rows of 16 lanes per wave)
constexpr int KU = 4;                   // K/V rows per slot per batch
constexpr int MERGE_DIMS = HQ * D / NB; // dims of one head merged per workgroup
constexpr unsigned kSpinLimit = 1u << 16;  // default polls per thread and launch (tens of ms)

static_assert(NQKV == 2 * NTH, "QKV: two rows per wave");
static_assert(H == NTH, "o_proj / down: one row per wave");
static_assert(H == 4 * NW * kWave, "one-layer launch: 4 input values per thread");
static_assert(I == 3 * NTH, "gate_up: three row pairs per wave");
static_assert(MERGE_DIMS == 8, "merge: 8 dims per workgroup");

// Parity of the words written at layer l of the launch that starts at layer
// generation gen.  It alternates from layer to layer and across launches of
// any layer count (the generation advances by the launch's layer count, and
// its wrap at 2^32 keeps the low bit's sequence); the +1 makes the first write
// differ from the zeroed hand-off area.
__device__ __forceinline__ unsigned parity_of(unsigned gen, int l) {
  return (gen + (unsigned)l + 1u) & 1u;
}

__device__ __forceinline__ unsigned word_of(float v, unsigned par) {
  return (__builtin_bit_cast(unsigned, v) & ~1u) | par;
}

__device__ __forceinline__ void put(unsigned* p, unsigned par, float v) {
  __hip_atomic_store(p, word_of(v, par), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two adjacent words (p 8-byte aligned) in one store.
__device__ __forceinline__ void put2(unsigned* p, unsigned par, float v0, float v1) {
  const uint64_t w = (uint64_t)word_of(v0, par) | ((uint64_t)word_of(v1, par) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until this wave's stores have completed (vmcnt(0)).
__device__ __forceinline__ void puts_done() { __builtin_amdgcn_s_waitcnt(0x0f70); }

typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kDeviceCoherent = 16;  // buffer-load cache policy: sc1 (device scope)

__device__ __forceinline__ Rsrc rsrc_of(const unsigned* base, unsigned words) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned*>(base), (short)0, (int)(words * 4u), 0x00020000);
}
__device__ __forceinline__ u32x4 peek4(Rsrc r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kDeviceCoherent);
}
__device__ __forceinline__ unsigned peek1(Rsrc r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kDeviceCoherent);
}
__device__ __forceinline__ bool parity_ok(u32x4 v, unsigned par) {
  return (((v.x ^ par) | (v.y ^ par) | (v.z ^ par) | (v.w ^ par)) & 1u) == 0u;
}
// The values of four words, their tag bit cleared: every reader then uses the
// same value whichever parity the write carried, so a launch's results do not
// depend on the launches before it.  Whole-vector cast: casting the elements
// one by one (bit_cast of v.y, ...) is folded to v.x by this compiler.
__device__ __forceinline__ f32x4 values_of(u32x4 v) { return __builtin_bit_cast(f32x4, v & ~1u); }

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

// Waits until every word of v[k] (16 bytes loaded from byte offset
// off0 + k * step) shows parity `par`.  A lane that is still waiting re-polls
// all of its words (branch-free: one wait per poll instead of one per word).
// Re-issues the N loads of await4 as straight-line code (a loop nested in the
// wait loop below is not unrolled by this compiler).
template <int K, int N>
__device__ __forceinline__ void repoll4(Rsrc r, unsigned off0, unsigned step, u32x4 (&v)[N]) {
  if constexpr (K < N) {
    v[K] = peek4(r, off0 + K * step);
    repoll4<K + 1, N>(r, off0, step, v);
  }
}

// A wait that runs out of its budget records the failure in the status word
// and hands its reader NaN instead of the stale words: NaN then reaches every
// value computed from them (the RMSNorms spread it over whole vectors, the
// attention below carries it through its softmax), so no output of a failed
// launch looks valid.
constexpr unsigned kPoison = 0x7fc00000u;  // quiet NaN; its tag bit is clear

__device__ __forceinline__ void wait_failed(Spin& sp) {
  __hip_atomic_fetch_or(sp.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int N>
__device__ __forceinline__ void await4(Rsrc r, unsigned off0, unsigned step, u32x4 (&v)[N], unsigned par,
                                       Spin& sp) {
#pragma clang loop unroll(disable)
  while (true) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok &= parity_ok(v[k], par);
    if (ok) break;
    if (sp.left == 0) {
      wait_failed(sp);
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = u32x4{kPoison, kPoison, kPoison, kPoison};
      break;
    }
    --sp.left;
    __builtin_amdgcn_s_sleep(1);
    repoll4<0, N>(r, off0, step, v);
  }
}

// Value of word i once it shows parity `par` (bounded wait).
__device__ __forceinline__ float take1(Rsrc r, unsigned i, unsigned par, Spin& sp) {
  unsigned v = peek1(r, i * 4u);
#pragma clang loop unroll(disable)
  while (((v ^ par) & 1u) != 0u) {
    if (sp.left == 0) {
      wait_failed(sp);
      v = kPoison;
      break;
    }
    --sp.left;
    __builtin_amdgcn_s_sleep(1);
    v = peek1(r, i * 4u);
  }
  return __builtin_bit_cast(float, v & ~1u);
}

// The GEMV inputs in LDS (x * gamma, the merged attention output, r * gamma,
// the MLP hidden vector) are fp16, the rounding the reference's fp16 model
// applies to every linear layer's input: a dot product then takes two
// products per instruction (v_dot2_f32_f16, fp32 accumulation) and reads half
// the LDS bytes.  Hand-off words, residuals and sums of squares stay fp32.
typedef uint16_t Act;
typedef _Float16 h2t __attribute__((ext_vector_type(2)));
typedef _Float16 h8t __attribute__((ext_vector_type(8)));

// Four values into an activation vector in LDS at element i (i % 4 == 0).
__device__ __forceinline__ void act_store4(Act* dst, unsigned i, f32x4 v) {
  *reinterpret_cast<uint2*>(dst + i) = uint2{pack2(v.x, v.y), pack2(v.z, v.w)};
}

// THREADS threads (ids t = 0..THREADS-1) gather N * THREADS * 4 words into
// dst: thread t takes words 4 (t + k THREADS) .. +4; every load is issued
// before the first wait.  Each word is read twice, back to back: a lane whose
// first reads do not all show `par` takes the second ones when those do, and
// polls again otherwise.  Measured on the 28-layer launch (same box, A/B):
// 642-647 against 645-655 us at context 1029 and 673-676 against 677-680 us at
// 4096; the same second reads left unused measured the same, so the time is
// not saved by the skipped re-polls (re-polls are rare either way).  Reading
// the x and r gathers (gather4_scaled) twice as well changed nothing.
template <int N, int THREADS>
__device__ __forceinline__ void gather4(Rsrc r, Act* dst, unsigned t, unsigned par, Spin& sp) {
  u32x4 v[N], v2[N];
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = peek4(r, (t + k * THREADS) * 16u);
#pragma unroll
  for (int k = 0; k < N; ++k) v2[k] = peek4(r, (t + k * THREADS) * 16u);
  {
    bool ok = true, ok2 = true;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      ok &= parity_ok(v[k], par);
      ok2 &= parity_ok(v2[k], par);
    }
    if (!ok && ok2) {
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = v2[k];
    }
  }
  await4<N>(r, t * 16u, THREADS * 16u, v, par, sp);
#pragma unroll
  for (int k = 0; k < N; ++k) act_store4(dst, (t + k * THREADS) * 4u, values_of(v[k]));
}

// The hidden vector's hand-off packs the three values a wave produces into one
// 64-bit word: three fp16 values (the rounding the DOWN rows' LDS input takes)
// and a 16-bit tag whose bit 0 is the write parity, stored with one 64-bit
// atomic store, so the tag and the values of a word change together.
__device__ __forceinline__ void put3h(unsigned* p, unsigned par, float v0, float v1, float v2) {
  const uint64_t w = (uint64_t)pack2(v0, v1) | ((uint64_t)((unsigned)f2h(v2) | (par << 16)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tags3h_ok(u32x4 v, unsigned par) {
  return ((((v.y >> 16) ^ par) | ((v.w >> 16) ^ par)) & 1u) == 0u;
}
constexpr unsigned kPoison3h = 0x7e007e00u;   // fp16 quiet NaN in both halves

template <int N>
__device__ __forceinline__ void await3h(Rsrc r, unsigned off0, unsigned step, u32x4 (&v)[N], unsigned par,
                                        Spin& sp) {
#pragma clang loop unroll(disable)
  while (true) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok &= tags3h_ok(v[k], par);
    if (ok) break;
    if (sp.left == 0) {
      wait_failed(sp);
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = u32x4{kPoison3h, kPoison3h, kPoison3h, kPoison3h};
      break;
    }
    --sp.left;
    __builtin_amdgcn_s_sleep(1);
    repoll4<0, N>(r, off0, step, v);
  }
}

// gather4 for the packed words: thread t takes the 16 bytes (two words, six
// values) t + k THREADS and writes values 6 (t + k THREADS) .. +6 to dst.
// Every 16-byte read is issued twice, as in gather4.
template <int N, int THREADS>
__device__ __forceinline__ void gather3h(Rsrc r, Act* dst, unsigned t, unsigned par, Spin& sp) {
  u32x4 v[N], v2[N];
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = peek4(r, (t + k * THREADS) * 16u);
#pragma unroll
  for (int k = 0; k < N; ++k) v2[k] = peek4(r, (t + k * THREADS) * 16u);
  {
    bool ok = true, ok2 = true;
#pragma unroll
    for (int k = 0; k < N; ++k) {
      ok &= tags3h_ok(v[k], par);
      ok2 &= tags3h_ok(v2[k], par);
    }
    if (!ok && ok2) {
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = v2[k];
    }
  }
  await3h<N>(r, t * 16u, THREADS * 16u, v, par, sp);
#pragma unroll
  for (int k = 0; k < N; ++k) {
    unsigned* d = reinterpret_cast<unsigned*>(dst + 6u * (t + k * THREADS));
    d[0] = v[k].x;
    d[1] = (v[k].y & 0xffffu) | (v[k].z << 16);
    d[2] = (v[k].z >> 16) | (v[k].w << 16);
  }
}

// Sum of squares of four values, in the one order every path uses (the
// per-wave partials of a vector must not depend on how it reached LDS).
__device__ __forceinline__ float sumsq4(f32x4 x) {
  return __builtin_fmaf(x.w, x.w, __builtin_fmaf(x.z, x.z, __builtin_fmaf(x.y, x.y, x.x * x.x)));
}

// gather4 with the RMSNorm weight folded in: dst[i] = v[i] * g[i] (g: the fp16
// norm weight in LDS), so the GEMV that reads dst needs only rstd, applied to
// its sums.  Thread t holds words 4 (t + k THREADS) .. +4, as a thread of
// THREADS * k + t would in a layout of 4 words per thread: the sums of squares
// come back per k (ss[k]), so a wave's sums over them equal those of that
// layout's waves.  The raw values of the workgroup's own rows [res0, res0 +
// NW) (the residual of its outputs) go to res.
template <int N, int THREADS>
__device__ __forceinline__ void gather4_scaled(Rsrc r, Act* dst, const uint16_t* g, float* res, unsigned res0,
                                               unsigned t, unsigned par, Spin& sp, float (&ss)[N]) {
  u32x4 v[N];
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = peek4(r, (t + k * THREADS) * 16u);
  await4<N>(r, t * 16u, THREADS * 16u, v, par, sp);
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const unsigned i = (t + k * THREADS) * 4u;
    const f32x4 x = values_of(v[k]);
    const uint2 gw = *reinterpret_cast<const uint2*>(g + i);
    act_store4(dst, i, f32x4{x.x * lo_f(gw.x), x.y * hi_f(gw.x), x.z * lo_f(gw.y), x.w * hi_f(gw.y)});
    ss[k] = sumsq4(x);
    if (i - res0 < (unsigned)NW) *reinterpret_cast<f32x4*>(res + (i - res0)) = x;
  }
}

// rsqrt(mean + eps) from the per-wave partial sums of squares in LDS.
__device__ __forceinline__ float rstd_of(const float (&ss)[NW], float n, float eps) {
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += ss[w];
  return rsqrtf(t / n + eps);
}

template <int KCH>
__device__ __forceinline__ void load_row(const uint16_t* row, int lane, u32x4 (&w)[KCH]) {
#pragma unroll
  for (int c = 0; c < KCH; ++c) w[c] = ld_stream(row + c * 512 + lane * 8);
}

// The dot products below read x from LDS one chunk ahead of its use and keep
// the scheduler from hoisting further reads (sched_barrier): left alone it
// issues every chunk's LDS reads up front, and with the prefetched weights of
// the next phases also live the registers run out.

// acc + sum of the 8 products of fp16 weights and fp16 inputs, two per
// v_dot2_f32_f16 (fp32 accumulation).  The pairs are taken from whole-vector
// bit casts: element-wise casts of an integer ext-vector are folded wrongly by
// this compiler.
__device__ __forceinline__ float dot8h(const u32x4 w, const u32x4 x, float acc) {
  const h8t wh = __builtin_bit_cast(h8t, w);
  const h8t xh = __builtin_bit_cast(h8t, x);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 0, 1), __builtin_shufflevector(xh, xh, 0, 1), acc,
                               false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 2, 3), __builtin_shufflevector(xh, xh, 2, 3), acc,
                               false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 4, 5), __builtin_shufflevector(xh, xh, 4, 5), acc,
                               false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 6, 7), __builtin_shufflevector(xh, xh, 6, 7), acc,
                               false);
  return acc;
}

// y[r] = W_r . x for R rows held in registers, x (fp16) streamed chunk by
// chunk from LDS: 8 values per lane and chunk, one 16-byte read.
template <int KCH, int R>
__device__ __forceinline__ void rows_dot(const u32x4 (&w)[R][KCH], const Act* s, int lane, float (&y)[R]) {
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  u32x4 x = *reinterpret_cast<const u32x4*>(s + lane * 8), xn = x;
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    if (c + 1 < KCH) xn = *reinterpret_cast<const u32x4*>(s + (c + 1) * 512 + lane * 8);
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8h(w[r][c], x, acc[r]);
    x = xn;
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) y[r] = wave_sum(acc[r]);
}

// Weight streaming.  A wave's vector-memory loads complete in issue order, so a
// wave that polls a hand-off waits for every load it issued before the poll.
// The waves therefore split into two groups:
//   pollers (waves 0-3) gather every hand-off into LDS (wave 0 alone gathers
//     the split partials and the merged attention output) and issue each
//     phase's weights only after the poll that precedes the phase;
//   streamers (waves 4-7) never poll, wait only at workgroup barriers and issue
//     weights one phase earlier: W_gate/up after QKV, W_down after attention,
//     the next layer's W_qkv, K/V and W_o after GATE_UP.
// Both groups hold the same number of rows, so a phase ends when the pollers'
// later loads land; the streamers keep HBM busy across the hand-offs.

// LDS of one workgroup.  Buffers whose lifetimes do not overlap share memory
// (a workgroup barrier always separates the last read of one from the first
// write of the other).
struct __align__(16) Smem {
  union {
    Act x[H];                 // layer input times input_norm (QKV phase)
    Act att[H];               // merged attention output (MERGE .. O_PROJ)
  } xa;
  Act r[H];                   // post-attention residual times post_norm
  union {
    Act h[I];                 // SiLU(gate) * up (DOWN)
    float acc[SLOTS][2][D];   // per-slot attention partials (ATTN .. slot merge)
  } ha;
  float raw[4][D];            // raw q0, q1, k, v of this kv head
  float q[2][D];              // rotated q
  uint16_t kv[2][D];          // new K_rot / V rows, fp16 as cached
  float m[SLOTS][2];
  float l[SLOTS][2];
  float mw[NS][MERGE_DIMS + 1];
  uint16_t gin[H];            // input RMSNorm weight of the current / next layer
  uint16_t gpost[H];          // post-attention RMSNorm weight of the current / next layer
  float xres[NW], rres[NW];   // raw x and r of the workgroup's rows (residuals of o_proj / down)
  float ssx[NW], ssr[NW];     // per-wave partial sums of squares of x and r
};

// Rows [t0, t1) of the attended length min(pos + 1, T) that split `split`
// (of NS) of a kv head covers.
__device__ __forceinline__ void split_window(const PersistArgs& a, long pos, int split, int& t0, int& t1) {
  long Ll = pos + 1 < (long)a.T ? pos + 1 : (long)a.T;
  if (Ll < 0) Ll = 0;
  const int L = (int)Ll;
  const int chunk = (L + NS - 1) / NS;
  t0 = split * chunk;
  t1 = min(t0 + chunk, L);
}

// Per-workgroup constants of a launch.
struct Ctx {
  int b, w, gw, kvh, split, t0, t1, mh, md0;
  long pos;
  unsigned gen;
  float rc, rs;               // M-RoPE cos / sin of rotary pair `lane`
};

// The layer loop of one wave group.  Pollers (waves 0..NA-1) and streamers
// run separate instances: their weight loads are issued at different points,
// and in one shared loop the compiler would have to keep each group's
// loop-carried weight registers live on the other group's path as well.
// Both instances execute the same sequence of workgroup barriers.
template <bool STREAM, bool LAYER>
__device__ __forceinline__ void persist_layers(const PersistArgs& a, Ctx& cx, Smem& sm, Spin& sp,
                                               uint2 x_first, uint2 g_first) {
  const int w = cx.w, gw = cx.gw, kvh = cx.kvh, split = cx.split, mh = cx.mh, md0 = cx.md0;
  // (LAYER: read below, once the first weight rows are in flight)
  int t0 = cx.t0, t1 = cx.t1;
  long pos = cx.pos;
  unsigned gen = cx.gen;
  const float rc = cx.rc, rs = cx.rs;
  constexpr bool streamer = STREAM;
  const bool poller = (w == 0);     // polls the split partials (MERGE) and the merged output
  int lane = lane_id();
  int tid = threadIdx.x;
  const Rsrc r_x = rsrc_of(a.x_t, H), r_qkv = rsrc_of(a.qkv_t, NQKV), r_op = rsrc_of(a.opart_t, HQ * NS * D),
             r_lse = rsrc_of(a.lse_t, HQ * NS), r_att = rsrc_of(a.att_t, HQ * D), r_r = rsrc_of(a.r_t, H),
             r_hid = rsrc_of(a.hid_t, I);
  Act(&s_x)[H] = sm.xa.x;
  Act(&s_att)[H] = sm.xa.att;
  Act(&s_r)[H] = sm.r;
  Act(&s_h)[I] = sm.ha.h;
  float(&s_raw)[4][D] = sm.raw;
  float(&s_q)[2][D] = sm.q;
  uint16_t(&s_kv)[2][D] = sm.kv;
  float(&s_acc)[SLOTS][2][D] = sm.ha.acc;
  float(&s_m)[SLOTS][2] = sm.m;
  float(&s_l)[SLOTS][2] = sm.l;
  float(&s_mw)[NS][MERGE_DIMS + 1] = sm.mw;
  uint16_t(&s_gin)[H] = sm.gin;
  uint16_t(&s_gpost)[H] = sm.gpost;

  // Lane-derived values are re-derived in every phase: otherwise the compiler
  // hoists the per-lane address arithmetic of all phases out of the layer loop
  // and the registers they occupy run out.
#define QD_FRESH_LANE() \
  do {                  \
    lane = (int)fresh((unsigned)lane); \
    tid = (int)fresh((unsigned)tid);   \
  } while (0)

  // Per-wave weight registers.  Those a streamer loads one layer ahead live
  // across the layer loop; W_gate/up and W_down are loaded and consumed within
  // one layer on every path, so they are declared in the loop body (a
  // declaration outside would keep the previous layer's values live around
  // the loop on the paths the compiler cannot rule out).
  u32x4 wq[2][4];                 // W_qkv rows 2gw, 2gw+1
  u32x4 kk[KU], vv[KU];           // first batch of K/V rows of the lane's position slot
  u32x4 wo[1][4];                 // W_o row gw
  uint16_t nw0 = 0, nw1 = 0;      // q/k head-norm weights of rotary pair `lane`

  // rs: row stride of the weight loads (H; 0 after the last layer, when every
  // wave re-reads one row that the L2 already holds instead of fetching rows
  // nobody uses); tl: end of this workgroup's K/V rows (t1; t0 after the last
  // layer: none).  The loads stay unconditional, so register liveness and the
  // wait counts are the same on every layer.
  auto issue_qkv = [&](const PersistLayer& Lx, long rs) {
    load_row<4>(Lx.qkv + (long)(2 * gw) * rs, lane, wq[0]);
    load_row<4>(Lx.qkv + (long)(2 * gw + 1) * rs, lane, wq[1]);
  };
  auto issue_kvwo = [&](const PersistLayer& Lx, long rs, int tl) {
    const int slot = w * 4 + (lane >> 4);
    const int dl = (lane & 15) * 8;
    const uint16_t* kb = Lx.k_cache + (long)kvh * a.T * D + dl;
    const uint16_t* vb = Lx.v_cache + (long)kvh * a.T * D + dl;
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int tt = t0 + slot + u * SLOTS;
      kk[u] = u32x4{0u, 0u, 0u, 0u};
      vv[u] = u32x4{0u, 0u, 0u, 0u};
      if (tt < tl && tt != pos) {
        kk[u] = ld_stream(kb + (long)tt * D);
        vv[u] = ld_stream(vb + (long)tt * D);
      }
    }
    load_row<4>(Lx.o_proj + (long)gw * rs, lane, wo[0]);
    const uint16_t* nw = (w == 2) ? Lx.k_norm : Lx.q_norm;
    nw0 = nw[lane];
    nw1 = nw[lane + 64];
  };
  auto issue_gu = [&](const PersistLayer& Lx, u32x4 (&wgu)[6][4]) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const long o = (long)gw * 3 + p;
      load_row<4>(Lx.gate_up + o * H, lane, wgu[p]);
      load_row<4>(Lx.gate_up + (o + I) * H, lane, wgu[3 + p]);
    }
  };
  auto issue_wd = [&](const PersistLayer& Lx, u32x4 (&wd)[1][12]) {
    load_row<12>(Lx.down + (long)gw * I, lane, wd[0]);
  };

  // RMSNorm weights of a layer are staged in LDS by the polling waves: 16 bytes
  // of each vector per thread, loaded in the previous layer and written once
  // that layer has no further use for them (after its gate_up stores).  The
  // gathers of x and r multiply by them (gather4_scaled).
  // (LAYER: stored after the first weight rows are issued, so no wave waits for
  // them before its W_qkv rows are in flight)
  u32x4 gi0 = {0u, 0u, 0u, 0u}, gp0 = {0u, 0u, 0u, 0u};
  if (!streamer) {
    gi0 = ld16(a.layers[0].input_norm + tid * 8);
    gp0 = ld16(a.layers[0].post_norm + tid * 8);
    if constexpr (!LAYER) {
      *reinterpret_cast<u32x4*>(s_gin + tid * 8) = gi0;
      *reinterpret_cast<u32x4*>(s_gpost + tid * 8) = gp0;
    }
  }
  issue_qkv(a.layers[0], H);
  if constexpr (LAYER) {
    // the layer generation and the cache position, by vector loads issued
    // behind the W_qkv rows: only the K/V addressing below waits for them (a
    // scalar load would put a wait for every outstanding scalar load, which
    // return out of order, in front of the first weight rows)
    const Rsrc rg = rsrc_of(a.generation, 1);
    const Rsrc rp = rsrc_of(reinterpret_cast<const unsigned*>(a.cache_position), 2);
    const unsigned g = __builtin_amdgcn_raw_buffer_load_b32(rg, 0u, 0, 0);
    const unsigned p0 = __builtin_amdgcn_raw_buffer_load_b32(rp, 0u, 0, 0);
    const unsigned p1 = __builtin_amdgcn_raw_buffer_load_b32(rp, 4u, 0, 0);
    gen = __builtin_amdgcn_readfirstlane(g);
    pos = (long)(((unsigned long)__builtin_amdgcn_readfirstlane(p1) << 32) | __builtin_amdgcn_readfirstlane(p0));
    split_window(a, pos, split, t0, t1);
    cx.gen = gen;
    cx.pos = pos;
  }
  issue_kvwo(a.layers[0], H, t1);
  if constexpr (LAYER) {
    if (!streamer) {
      *reinterpret_cast<u32x4*>(s_gin + tid * 8) = gi0;
      *reinterpret_cast<u32x4*>(s_gpost + tid * 8) = gp0;
    }
  }

  for (int l = 0; l < a.num_layers; ++l) {
    const PersistLayer& Lw = a.layers[l];
    const unsigned par = parity_of(gen, l);
    // The next layer's weights are issued unconditionally (a conditional issue
    // would leave the previous values live to the end of the iteration on the
    // path that skips it); after the last layer the loads are made cheap
    // instead (row stride 0, no K/V rows).
    const PersistLayer& Ln = a.layers[l + 1 < a.num_layers ? l + 1 : l];
    const bool more = l + 1 < a.num_layers;
    const long rs_n = more ? (long)H : 0L;
    const int tl_n = more ? t1 : t0;
    u32x4 wgu[6][4];              // W_gate/up rows 3gw..3gw+2 (+I)
    u32x4 wd[1][12];              // W_down row gw

    // ================================================================ QKV
    QD_TRACE_AT(l, 0);
    QD_TRACE_ST(l, 0);
    QD_FRESH_LANE();
    // s_x = x * input_norm; the raw x of this workgroup's rows and the waves'
    // partial sums of x^2 beside it
    if (l == 0) {
      // every thread: values 4 tid .. 4 tid + 3 and their norm weights (g_first,
      // loaded at kernel start)
      uint2 xb = x_first;
      if constexpr (!LAYER) {
        long tok = a.token[0];
        if (tok < 0 || tok >= a.vocab) tok = 0;
        xb = *reinterpret_cast<const uint2*>(a.embed + tok * (long)H + tid * 4);
      }
      const f32x4 xv = {lo_f(xb.x), hi_f(xb.x), lo_f(xb.y), hi_f(xb.y)};
      act_store4(s_x, tid * 4u,
                 f32x4{xv.x * lo_f(g_first.x), xv.y * hi_f(g_first.x), xv.z * lo_f(g_first.y), xv.w * hi_f(g_first.y)});
      if ((unsigned)(tid * 4 - cx.b * NW) < (unsigned)NW) *reinterpret_cast<f32x4*>(sm.xres + (tid * 4 - cx.b * NW)) = xv;
      const float ss = wave_sum(sumsq4(xv));
      if (lane == 0) sm.ssx[w] = ss;
    } else if (!streamer) {
      // polling wave w holds the values of waves w and w + NA of the layout above
      float ss[H / (4 * NA * kWave)];
      gather4_scaled<H / (4 * NA * kWave), NA * kWave>(r_x, s_x, s_gin, sm.xres, cx.b * NW, (unsigned)tid, par ^ 1u,
                                                       sp, ss);
      static_assert(H / (4 * NA * kWave) == 2, "x gather: two 4-value groups per polling thread");
      const float s0 = wave_sum(ss[0]), s1 = wave_sum(ss[1]);
      if (lane == 0) {
        sm.ssx[w] = s0;
        sm.ssx[w + NA] = s1;
      }
    }
    __syncthreads();
    QD_TRACE_AT(l, 1);
    QD_TRACE_ST(l, 1);
    QD_FRESH_LANE();
    // o_proj's residual (s_x shares its memory with the merged attention output)
    const float xres = sm.xres[w];
    {
      float y[2];
      rows_dot<4, 2>(wq, s_x, lane, y);
      const float rstd = rstd_of(sm.ssx, (float)H, a.eps);
      if (lane == 0) put2(a.qkv_t + 2 * gw, par, y[0] * rstd, y[1] * rstd);
      if (!streamer) puts_done();
    }
    QD_TRACE_AT(l, 2);
    QD_TRACE_ST(l, 2);
    QD_FRESH_LANE();
    if (streamer) issue_gu(Lw, wgu);
    QD_TRACE_ST(l, 3);

    // ================================================================ ATTN
    QD_FRESH_LANE();
    if (tid < D) {
      // raw q (2 heads), k, v of kv head kvh: 512 words, 4 per thread of waves 0-1
      unsigned src;
      if (tid < D / 2) src = kvh * 2 * D + tid * 4;
      else if (tid < 3 * D / 4) src = HQ * D + kvh * D + (tid - D / 2) * 4;
      else src = (HQ + HKV) * D + kvh * D + (tid - 3 * D / 4) * 4;
      u32x4 v[1] = {peek4(r_qkv, src * 4u)};
      await4<1>(r_qkv, src * 4u, 0u, v, par, sp);
      *reinterpret_cast<f32x4*>(&s_raw[0][0] + tid * 4) = values_of(v[0]);
    }
    __syncthreads();
    QD_TRACE_AT(l, 3);
    QD_TRACE_ST(l, 4);
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
    QD_TRACE_AT(l, 15);
    QD_TRACE_ST(l, 5);
    QD_FRESH_LANE();
    {
      const int row_off = lane >> 4;  // 16-lane row inside the wave
      const int slot = w * 4 + row_off;
      const int dl = (lane & 15) * 8;
      const uint16_t* kb = Lw.k_cache + (long)kvh * a.T * D + dl;
      const uint16_t* vb = Lw.v_cache + (long)kvh * a.T * D + dl;
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
      // One batch: the slot's KU rows t, t + SLOTS, ... in kk / vv.
      auto batch = [&](const int t) {
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          if (t + u * SLOTS == pos && pos < t1) {
            kk[u] = *reinterpret_cast<const u32x4*>(&s_kv[0][dl]);
            vv[u] = *reinterpret_cast<const u32x4*>(&s_kv[1][dl]);
          }
        }
        // online softmax over the batch's KU rows as one block: their scores,
        // one running-maximum update and one rescale per head, then one FMA
        // per dimension and row (rows >= t1 weigh 0; NaN scores stay NaN in
        // the sums, the maximum skips them)
        float sc[KU][2];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const bool valid = t + u * SLOTS < t1;
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            const float s = row16_sum(dot8(kk[u], q[g], 0.f)) * a.scale;
            sc[u][g] = valid ? s : -INFINITY;
          }
        }
        float p[KU][2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float mb = sc[0][g];
#pragma unroll
          for (int u = 1; u < KU; ++u) mb = fmaxf(mb, sc[u][g]);
          const float mn = fmaxf(m[g], mb);
          const float c = mn == -INFINITY ? 1.f : __expf(m[g] - mn);
          float ps = 0.f;
#pragma unroll
          for (int u = 0; u < KU; ++u) {
            p[u][g] = sc[u][g] == -INFINITY ? 0.f : __expf(sc[u][g] - mn);
            ps += p[u][g];
          }
          lsum[g] = __builtin_fmaf(lsum[g], c, ps);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] *= c;
          m[g] = mn;
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          float vf[8];
          unpack8(vv[u], vf);
#pragma unroll
          for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(p[u][g], vf[i], acc[g][i]);
        }
      };
      // The first batch's rows were loaded before this phase's W_gate/up rows
      // (issue_kvwo): processed outside the loop, its wait covers only them.
      // Inside a loop that reloads kk / vv the compiler waits for every load
      // in flight, the streaming waves' whole W_gate/up burst included.
      if (wave_t0 < t1) batch(wave_t0 + row_off);
#pragma unroll 1
      for (int tw = wave_t0 + SLOTS * KU; tw < t1; tw += SLOTS * KU) {
        const int t = tw + row_off;
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
        batch(t);
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
    QD_TRACE_AT(l, 4);
    QD_TRACE_ST(l, 6);
    QD_FRESH_LANE();
    if (streamer) issue_wd(Lw, wd);
    QD_TRACE_ST(l, 7);
    __syncthreads();
    QD_TRACE_ST(l, 8);
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
      } else {
        // no slot raised its maximum: an empty split (every sum 0) or NaN
        // scores (the sums are NaN), which must stay NaN
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) den += s_l[s][g];
        num = den;
      }
      const int hq = kvh * 2 + g;
      const bool live = den > 0.f, empty = den == 0.f;
      // an empty split reports lse = -FLT_MAX (finite: the parity bit must not turn -inf into a NaN)
      put(a.opart_t + ((long)hq * NS + split) * D + d, par, live ? num / den : (empty ? 0.f : den));
      if (d == 0) put(a.lse_t + (long)hq * NS + split, par, live ? M + __logf(den) : (empty ? -FLT_MAX : den));
    }

    // ================================================================ MERGE + O_PROJ input (wave 0)
    QD_FRESH_LANE();
    if (poller) {
      puts_done();
      QD_TRACE_AT(l, 5);
      // lanes 0..31: LSE of split `lane`; every lane: dims (lane / 32) * 4 .. +4 of split lane % 32
      const int s = lane % NS;
      const int k0 = (lane / NS) * 4;
      const unsigned lo = fresh((unsigned)((mh * NS + s) * D + md0 + k0)) * 4u;
      u32x4 ov[1] = {peek4(r_op, lo)};
      const float lse = take1(r_lse, (unsigned)(mh * NS + s), par, sp);
      await4<1>(r_op, lo, 0u, ov, par, sp);
      const f32x4 o4 = values_of(ov[0]);
      const float o[4] = {o4.x, o4.y, o4.z, o4.w};
      const float M = wave_max(lse);
      const float wgt = __expf(lse - M);
#pragma unroll
      for (int k = 0; k < 4; ++k) s_mw[s][k0 + k] = wgt * o[k];
      if (lane < NS) s_mw[s][MERGE_DIMS] = wgt;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      if (lane < MERGE_DIMS) {
        float num = 0.f, den = 0.f;
        for (int t = 0; t < NS; ++t) {
          num += s_mw[t][lane];
          den += s_mw[t][MERGE_DIMS];
        }
        // den >= 1 (the largest split weighs 1) unless an input was NaN
        put(a.att_t + mh * D + md0 + lane, par, den > 0.f ? num / den : __builtin_nanf(""));
      }
      puts_done();
      gather4<H / (4 * kWave), kWave>(r_att, s_att, (unsigned)lane, par, sp);
      QD_TRACE_AT(l, 6);
    }
    // waves 1-3 right after the partials, wave 0 after its two polls
    QD_FRESH_LANE();
    if (!streamer) issue_gu(Lw, wgu);
    QD_TRACE_AT(l, 13);
    __syncthreads();
    QD_TRACE_ST(l, 9);

    // ================================================================ O_PROJ
    QD_TRACE_AT(l, 7);
    QD_FRESH_LANE();
    {
      float y[1];
      rows_dot<4, 1>(wo, s_att, lane, y);
      if (lane == 0) put(a.r_t + gw, par, y[0] + xres);
      if (!streamer) puts_done();
    }
    QD_TRACE_AT(l, 8);
    QD_TRACE_ST(l, 10);

    // ================================================================ GATE_UP
    QD_FRESH_LANE();
    if (!streamer) {
      float ss[H / (4 * NA * kWave)];
      gather4_scaled<H / (4 * NA * kWave), NA * kWave>(r_r, s_r, s_gpost, sm.rres, cx.b * NW, (unsigned)tid, par, sp,
                                                       ss);
      const float s0 = wave_sum(ss[0]), s1 = wave_sum(ss[1]);
      if (lane == 0) {
        sm.ssr[w] = s0;
        sm.ssr[w + NA] = s1;
      }
    }
    __syncthreads();
    QD_TRACE_AT(l, 9);
    QD_TRACE_ST(l, 11);
    QD_FRESH_LANE();
    u32x4 gi_next, gp_next;
    if (!streamer) {
      gi_next = ld16(Ln.input_norm + tid * 8);
      gp_next = ld16(Ln.post_norm + tid * 8);
      issue_wd(Lw, wd);
    }
    QD_TRACE_AT(l, 14);
    {
      float gu[6];
      rows_dot<4, 6>(wgu, s_r, lane, gu);
      const float rstd = rstd_of(sm.ssr, (float)H, a.eps);
      if (lane == 0) {
        float hv[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const float g = gu[p] * rstd;
          hv[p] = (g / (1.0f + __expf(-g))) * (gu[3 + p] * rstd);
        }
        put3h(a.hid_t + 2L * gw, par, hv[0], hv[1], hv[2]);
      }
      if (!streamer) {
        puts_done();
        // this layer's reads of both norms are done (the x and r gathers); the
        // hidden hand-off's barrier below orders these stores before the next
        // layer's gathers
        *reinterpret_cast<u32x4*>(s_gin + tid * 8) = gi_next;
        *reinterpret_cast<u32x4*>(s_gpost + tid * 8) = gp_next;
      }
    }
    QD_TRACE_AT(l, 10);
    QD_TRACE_ST(l, 12);
    QD_FRESH_LANE();
    if (streamer) {
      issue_qkv(Ln, rs_n);
      issue_kvwo(Ln, rs_n, tl_n);
    }
    QD_TRACE_ST(l, 13);

    // ================================================================ DOWN
    QD_FRESH_LANE();
    if (!streamer) gather3h<I / (6 * NA * kWave), NA * kWave>(r_hid, s_h, (unsigned)tid, par, sp);
    __syncthreads();
    QD_TRACE_AT(l, 11);
    QD_TRACE_ST(l, 14);
    QD_FRESH_LANE();
    if (!streamer) issue_qkv(Ln, rs_n);
    {
      float y[1];
      rows_dot<12, 1>(wd, s_h, lane, y);
      if (lane == 0) {
        const float v = y[0] + sm.rres[w];
        if constexpr (LAYER) {
          // every layer's output in fp16; the next layer reads that value, as a
          // launch of its own would (its tag bit lies in the zero low mantissa)
          const uint16_t vh = f2h(v);
          a.x_out16[(long)l * H + gw] = vh;
          put(a.x_t + gw, par, h2f(vh));
        } else {
          put(a.x_t + gw, par, v);
          if (l + 1 == a.num_layers) a.x_out[gw] = v;
        }
      }
      QD_TRACE_ST(l, 15);
      if (!streamer) {
        puts_done();
        QD_TRACE_AT(l, 12);
        // the next layer's K/V rows and W_o row: in flight across the x hand-off
        issue_kvwo(Ln, rs_n, tl_n);
      }
    }
  }

#undef QD_FRESH_LANE
}

}  // namespace

template <bool LAYER>
__global__ __launch_bounds__(512) void decode_persistent_kernel(const PersistArgs a) {
  const int b = blockIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: branches on it are scalar
  const int lane = lane_id();
  const int tid = threadIdx.x;
  Spin sp{a.spin_limit != 0u ? a.spin_limit : kSpinLimit, a.status};
  __shared__ Smem sm;
  // LAYER: the layer input is every thread's first vector load (4 fp16 values),
  // issued before the scalar reads below: loads complete in issue order, so the
  // QKV phase waits for it and not for the weight rows issued later
  uint2 x_first = {0u, 0u};
  if constexpr (LAYER) x_first = *reinterpret_cast<const uint2*>(a.x_in + tid * 4);
  // the first layer's input-norm weights of the same 4 values
  const uint2 g_first = *reinterpret_cast<const uint2*>(a.layers[0].input_norm + tid * 4);
  __builtin_amdgcn_sched_barrier(0);

  Ctx cx;
  cx.b = b;
  cx.w = w;
  cx.gw = b * NW + w;
  cx.kvh = b % HKV;
  cx.split = b / HKV;
  if constexpr (LAYER) {
    // read inside the layer loop's set-up, behind the first weight rows
    cx.gen = 0u;
    cx.pos = 0;
    cx.t0 = cx.t1 = 0;
  } else {
    cx.gen = a.generation[0];
    cx.pos = a.cache_position[0];
    split_window(a, cx.pos, cx.split, cx.t0, cx.t1);
  }
  cx.mh = b / (D / MERGE_DIMS);               // merged q head of this workgroup
  cx.md0 = (b % (D / MERGE_DIMS)) * MERGE_DIMS;
  if constexpr (LAYER) {
    // the caller's rotation of pair `lane` (cos / sin repeat over the two halves)
    cx.rc = h2f(a.rope_cos[lane]);
    cx.rs = h2f(a.rope_sin[lane]);
  } else {
    // M-RoPE angle of rotary pair `lane` (the same for every layer of the step)
    int stream = 0;
    if (lane % 3 == 1 && lane < 3 * a.sec_h) stream = 1;
    else if (lane % 3 == 2 && lane < 3 * a.sec_w) stream = 2;
    sincosf((float)a.rope_position[stream] * a.inv_freq[lane], &cx.rs, &cx.rc);
  }

  if (w >= NA) persist_layers<true, LAYER>(a, cx, sm, sp, x_first, g_first);
  else persist_layers<false, LAYER>(a, cx, sm, sp, x_first, g_first);

  // The last workgroup to finish advances the generation by this launch's
  // layer count.  Every workgroup read the generation before it produced
  // anything, so none can read the new value in this launch.  The same holds
  // for the cache position, which the LAYER instance then advances.
  __syncthreads();
  if (tid == 0) {
    const unsigned n = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n == NB - 1) {
      __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.generation, cx.gen + (unsigned)a.num_layers, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if constexpr (LAYER) {
        for (int l = 0; l < a.num_layers; ++l)
          if (a.layers[l].length_out != nullptr) *a.layers[l].length_out = cx.pos + 1;
      }
    }
  }
}

int decode_persistent_launch(const PersistArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(decode_persistent_kernel<false>, dim3(NB), dim3(NW * kWave), 0, s, a);
  return qd_host::launch_status("decode_persistent_kernel");
}

int decode_persistent_layer_launch(const PersistArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(decode_persistent_kernel<true>, dim3(NB), dim3(NW * kWave), 0, s, a);
  return qd_host::launch_status("decode_persistent_kernel<LAYER>");
}

extern "C" int qd_persistent_trace_read(uint64_t* dst, size_t n, int* dims) {
#ifdef QD_TRACE
  if (dims != nullptr) {
    dims[0] = kPersistBlocks;
    dims[1] = kTraceLayers;
    dims[2] = kTraceEvents;
  }
  const size_t total = (size_t)kPersistBlocks * kTraceLayers * kTraceEvents;
  if (dst == nullptr) return QD_OK;
  const hipError_t e = hipMemcpyFromSymbol(dst, HIP_SYMBOL(qd_trace_stamps),
                                           (n < total ? n : total) * sizeof(uint64_t), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    qd_host::set_error("trace read failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return QD_OK;
#else
  (void)dst;
  (void)n;
  (void)dims;
  qd_host::set_error("this library was built without QD_TRACE (build the traced variant)");
  return QD_ERR_ARG;
#endif
}

int decode_persistent_check_device(char* why, size_t why_len) {
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  int per_cu_layer = 0;
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_persistent_kernel<false>, NW * kWave, 0);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_layer, decode_persistent_kernel<true>, NW * kWave, 0);
  if (per_cu_layer < per_cu) per_cu = per_cu_layer;
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
