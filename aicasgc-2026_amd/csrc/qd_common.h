// Device helpers shared by the gfx950 decode kernels.
//
// Wave64 throughout: a wavefront is 64 lanes; cross-lane sums use DPP row
// operations inside each 16-lane row and v_readlane across the four rows, so a
// full-wave reduction costs 4 DPP adds + 3 scalar-operand adds and leaves the
// (bit-identical) result in every lane.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/qwen3vl_decode.h"

namespace qd {

constexpr int kWave = 64;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float h2f(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}
__device__ __forceinline__ uint16_t f2h(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}
__device__ __forceinline__ float lo_f(unsigned int u) { return h2f((uint16_t)(u & 0xffffu)); }
__device__ __forceinline__ float hi_f(unsigned int u) { return h2f((uint16_t)(u >> 16)); }

// 8 consecutive fp16 values -> fp32.
__device__ __forceinline__ void unpack8(const u32x4 v, float* o) {
  o[0] = lo_f(v.x); o[1] = hi_f(v.x);
  o[2] = lo_f(v.y); o[3] = hi_f(v.y);
  o[4] = lo_f(v.z); o[5] = hi_f(v.z);
  o[6] = lo_f(v.w); o[7] = hi_f(v.w);
}

__device__ __forceinline__ unsigned int pack2(float a, float b) {
  return (unsigned int)f2h(a) | ((unsigned int)f2h(b) << 16);
}

// acc += sum_i w[i] * x[i] for 8 fp16 weights and fp32 x (fp32 products).
__device__ __forceinline__ float dot8(const u32x4 w, const float* x, float acc) {
  acc = __builtin_fmaf(lo_f(w.x), x[0], acc);
  acc = __builtin_fmaf(hi_f(w.x), x[1], acc);
  acc = __builtin_fmaf(lo_f(w.y), x[2], acc);
  acc = __builtin_fmaf(hi_f(w.y), x[3], acc);
  acc = __builtin_fmaf(lo_f(w.z), x[4], acc);
  acc = __builtin_fmaf(hi_f(w.z), x[5], acc);
  acc = __builtin_fmaf(lo_f(w.w), x[6], acc);
  acc = __builtin_fmaf(hi_f(w.w), x[7], acc);
  return acc;
}

// ---------------------------------------------------------------- memory

// Streamed (read-once) 16-byte load: weights and KV rows.
__device__ __forceinline__ u32x4 ld_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Load 8 activation values starting at element i of a fp16 or fp32 vector.
template <typename T>
__device__ __forceinline__ void load_act8(const T* p, long i, float* o);
template <>
__device__ __forceinline__ void load_act8<uint16_t>(const uint16_t* p, long i, float* o) {
  unpack8(ld16(p + i), o);
}
// fp32 activations are moved as float4 vectors.  (Do not bit-cast individual
// elements of an integer ext-vector to float here: clang folds every
// __builtin_bit_cast(float, v.y / v.z / v.w) to element x for this pattern.)
template <>
__device__ __forceinline__ void load_act8<float>(const float* p, long i, float* o) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p + i);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + i + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

template <typename T>
__device__ __forceinline__ float load_act(const T* p, long i);
template <>
__device__ __forceinline__ float load_act<uint16_t>(const uint16_t* p, long i) { return h2f(p[i]); }
template <>
__device__ __forceinline__ float load_act<float>(const float* p, long i) { return p[i]; }

template <typename T>
__device__ __forceinline__ void store_act(T* p, long i, float v);
template <>
__device__ __forceinline__ void store_act<uint16_t>(uint16_t* p, long i, float v) { p[i] = f2h(v); }
template <>
__device__ __forceinline__ void store_act<float>(float* p, long i, float v) { p[i] = v; }

template <typename T>
__device__ __forceinline__ void store_act8(T* p, long i, const float* v);
template <>
__device__ __forceinline__ void store_act8<uint16_t>(uint16_t* p, long i, const float* v) {
  u32x4 o;
  o.x = pack2(v[0], v[1]); o.y = pack2(v[2], v[3]);
  o.z = pack2(v[4], v[5]); o.w = pack2(v[6], v[7]);
  *reinterpret_cast<u32x4*>(p + i) = o;
}
template <>
__device__ __forceinline__ void store_act8<float>(float* p, long i, const float* v) {
  *reinterpret_cast<f32x4*>(p + i) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + i + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// ---------------------------------------------------------------- cross-lane

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;   // row_ror:4
constexpr int kDppRowRor8 = 0x128;   // row_ror:8

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ unsigned dpp_u(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Sum over each 16-lane row; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowRor4>(v);
  v += dpp<kDppRowRor8>(v);
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Full-wave sum, uniform in all lanes, fixed summation order.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppRowRor4>(v));
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// ---------------------------------------------------------------- cross-workgroup hand-off
//
// L2 is private to each XCD, so data handed between workgroups of one launch
// is published with an agent-scope release (write-back of dirty L2 lines) and
// read after an agent-scope acquire (invalidate of stale L2 lines).

__device__ __forceinline__ unsigned atomic_add_release(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_relaxed(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void fence_acquire() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}
__device__ __forceinline__ void fence_release() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

// Fence-free hand-off of a few values: agent-coherent stores (written through
// the XCD-private L2), a wait until this thread's stores have completed, then
// an arrival count; the consumer reads with agent-coherent loads.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(long* p, long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ long load_coherent(long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0x0f70); }   // vmcnt(0)

// Arrival of one workgroup (call from one thread after stores_done() and a
// workgroup barrier): true for the last of `expected` arrivals, which also
// re-arms the counter for the next launch.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected) {
  const unsigned old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool last = old == expected - 1;
  if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// ---------------------------------------------------------------- batch operand images
//
// The B operand of the batch GEMV (v_mfma_f32_16x16x32_f16, 16 columns) for an
// activation u[8][K] of up to 8 sequences, stored in MFMA lane order so one
// 16-byte load per lane and K tile of 32 fetches it:
//   image[((k / 32) * 64 + col + 16 ((k % 32) / 8)) * 8 + k % 8]
// column seq (< 8) holds fp16(u[seq][k]), column seq + 8 the fp16 rounding
// residual u - fp16(u), so the two MFMA columns sum to u with ~22 bits.

__device__ __forceinline__ long bimg_index(int col, long k) {
  return (((k >> 5) * 64 + col + 16 * ((k & 31) >> 3)) << 3) + (k & 7);
}

__device__ __forceinline__ void bimg_store(uint16_t* img, int seq, long k, float u) {
  const _Float16 hi = (_Float16)u;
  const _Float16 lo = (_Float16)(u - (float)hi);
  img[bimg_index(seq, k)] = __builtin_bit_cast(uint16_t, hi);
  img[bimg_index(seq + 8, k)] = __builtin_bit_cast(uint16_t, lo);
}

}  // namespace qd

// Host-side error reporting shared by the C-ABI translation units.
namespace qd_host {
void set_error(const char* fmt, ...);
int launch_status(const char* what);
int cu_count();
}  // namespace qd_host

#define QD_REQUIRE(cond, code, ...)          \
  do {                                       \
    if (!(cond)) {                           \
      qd_host::set_error(__VA_ARGS__);       \
      return (code);                         \
    }                                        \
  } while (0)
