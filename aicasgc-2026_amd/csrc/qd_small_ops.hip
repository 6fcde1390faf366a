// Small fused decode ops for gfx950: per-head QK-RMSNorm + (M-)RoPE with the
// static-KV write, add+RMSNorm, RMSNorm, SiLU*mul, add, embedding gather.
//
// Per-head ops map one 128-element head onto one wave64: lane j holds elements
// j and j + 64, which are exactly the pair rotate-half RoPE mixes, so the
// rotation is lane-local and the head RMSNorm is a single wave reduction.
// Reference kernels replaced: decode_small_ops_kernel.cu:68-182 (qk norm+rope,
// q-rope + KV-cache update), :369-624 (silu_mul, add+rmsnorm, rmsnorm, add).

#include <math.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

namespace {
constexpr int kD = 128;
constexpr int kHalf = 64;
}  // namespace

// cos/sin of frequency slot j (= lane) for this step.
__device__ __forceinline__ void rope_cs(const RopeArgs& a, int row, int j, float& c, float& s) {
  if (a.cos != nullptr) {
    c = h2f(a.cos[(long)row * a.cs_row + j]);
    s = h2f(a.sin[(long)row * a.cs_row + j]);
    return;
  }
  // Interleaved M-RoPE slot assignment: j % 3 == 1 (j < 3*sec_h) -> H stream,
  // j % 3 == 2 (j < 3*sec_w) -> W stream, otherwise T.
  int stream = 0;
  if (j % 3 == 1 && j < 3 * a.sec_h) stream = 1;
  else if (j % 3 == 2 && j < 3 * a.sec_w) stream = 2;
  const float f = (float)a.rope_pos[stream] * a.inv_freq[j];
  sincosf(f, &s, &c);
}

// RMSNorm(head) * w then rotate-half RoPE; x0/x1 = elements j, j+64.
__device__ __forceinline__ void norm_rope(float x0, float x1, const uint16_t* w, float eps, float c, float s,
                                          int j, float& o0, float& o1) {
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = rsqrtf(ss / (float)kD + eps);
  const float n0 = (x0 * rstd) * h2f(w[j]);
  const float n1 = (x1 * rstd) * h2f(w[j + kHalf]);
  o0 = n0 * c - n1 * s;
  o1 = n1 * c + n0 * s;
}

// grid = Hkv, block = 64 * (2 + G): wave 0 = K head (norm, rope, cache write),
// wave 1 = V head (cache write), waves 2.. = the G q heads of the group.
template <typename TI, typename TO>
__global__ __launch_bounds__(384) void q_rope_kv_kernel(const RopeArgs a) {
  const int kvh = blockIdx.x;
  const int w = threadIdx.x / kWave;
  const int j = lane_id();
  const int G = a.Hq / a.Hkv;
  const long pos = a.cache_position[0];
  const bool write = pos >= 0 && pos < (long)a.T;
  float c, s;
  rope_cs(a, 0, j, c, s);
  if (w == 0) {
    const TI* k = reinterpret_cast<const TI*>(a.k) + (long)kvh * a.k_stride;
    float o0, o1;
    norm_rope(load_act(k, j), load_act(k, j + kHalf), a.k_weight, a.eps, c, s, j, o0, o1);
    if (write) {
      uint16_t* dst = a.k_cache + (long)kvh * a.cache_stride_h + pos * a.cache_stride_s;
      dst[j] = f2h(o0);
      dst[j + kHalf] = f2h(o1);
    }
  } else if (w == 1) {
    const TI* v = reinterpret_cast<const TI*>(a.v) + (long)kvh * a.v_stride;
    if (write) {
      uint16_t* dst = a.v_cache + (long)kvh * a.cache_stride_h + pos * a.cache_stride_s;
      dst[j] = f2h(load_act(v, j));
      dst[j + kHalf] = f2h(load_act(v, j + kHalf));
    }
  } else if (w - 2 < G) {
    const int h = kvh * G + (w - 2);
    const TI* q = reinterpret_cast<const TI*>(a.q) + (long)h * a.q_stride;
    float o0, o1;
    norm_rope(load_act(q, j), load_act(q, j + kHalf), a.q_weight, a.eps, c, s, j, o0, o1);
    TO* qo = reinterpret_cast<TO*>(a.q_out) + (long)h * kD;
    store_act(qo, j, o0);
    store_act(qo, j + kHalf, o1);
  }
}

template <typename TI, typename TO>
int q_rope_kv_launch(const RopeArgs& a, hipStream_t s) {
  const int G = a.Hq / a.Hkv;
  hipLaunchKernelGGL((q_rope_kv_kernel<TI, TO>), dim3((unsigned)a.Hkv), dim3(kWave * (2 + G)), 0, s, a);
  return qd_host::launch_status("q_rope_kv_kernel");
}

template int q_rope_kv_launch<uint16_t, uint16_t>(const RopeArgs&, hipStream_t);
template int q_rope_kv_launch<float, float>(const RopeArgs&, hipStream_t);

// grid = (M, Hkv), block = 64 * (1 + G): wave 0 = k head, waves 1.. = q heads.
__global__ __launch_bounds__(320) void qk_norm_rope_kernel(const RopeArgs a) {
  const int m = blockIdx.x;
  const int kvh = blockIdx.y;
  const int w = threadIdx.x / kWave;
  const int j = lane_id();
  const int G = a.Hq / a.Hkv;
  float c, s;
  rope_cs(a, m, j, c, s);
  const uint16_t* src;
  uint16_t* dst;
  const uint16_t* nw;
  if (w == 0) {
    src = reinterpret_cast<const uint16_t*>(a.k) + (long)m * a.k_row + (long)kvh * a.k_stride;
    dst = reinterpret_cast<uint16_t*>(a.k_out) + ((long)m * a.Hkv + kvh) * kD;
    nw = a.k_weight;
  } else if (w - 1 < G) {
    const int h = kvh * G + (w - 1);
    src = reinterpret_cast<const uint16_t*>(a.q) + (long)m * a.q_row + (long)h * a.q_stride;
    dst = reinterpret_cast<uint16_t*>(a.q_out) + ((long)m * a.Hq + h) * kD;
    nw = a.q_weight;
  } else {
    return;
  }
  float o0, o1;
  norm_rope(h2f(src[j]), h2f(src[j + kHalf]), nw, a.eps, c, s, j, o0, o1);
  dst[j] = f2h(o0);
  dst[j + kHalf] = f2h(o1);
}

int qk_norm_rope_f16_launch(const RopeArgs& a, hipStream_t s) {
  const int G = a.Hq / a.Hkv;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)a.M, (unsigned)a.Hkv), dim3(kWave * (1 + G)), 0, s, a);
  return qd_host::launch_status("qk_norm_rope_kernel");
}

// ---------------------------------------------------------------- row norms

__device__ __forceinline__ float block_sum_256(float v, float* sh) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0) sh[w] = v;
  __syncthreads();
  const int nw = blockDim.x / kWave;
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += sh[i];
  return t;
}

// one block per row; residual may be null (plain RMSNorm).
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const uint16_t* res, const uint16_t* x,
                                                          const uint16_t* w, uint16_t* out_sum,
                                                          uint16_t* out_norm, int cols, float eps) {
  __shared__ float sh[4];
  const long base = (long)blockIdx.x * cols;
  float ss = 0.f;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) {
    float v = h2f(x[base + i]);
    if (res != nullptr) v += h2f(res[base + i]);
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = block_sum_256(ss, sh);
  const float rstd = rsqrtf(ss / (float)cols + eps);
  for (int i = threadIdx.x; i < cols; i += blockDim.x) {
    float v = h2f(x[base + i]);
    if (res != nullptr) v += h2f(res[base + i]);
    if (out_sum != nullptr) out_sum[base + i] = f2h(v);
    out_norm[base + i] = f2h((v * rstd) * h2f(w[i]));
  }
}

int add_rmsnorm_f16_launch(const uint16_t* res, const uint16_t* x, const uint16_t* w, uint16_t* out_sum,
                           uint16_t* out_norm, int rows, int cols, float eps, hipStream_t s) {
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, s, res, x, w, out_sum, out_norm,
                     cols, eps);
  return qd_host::launch_status("add_rmsnorm_kernel");
}

// ---------------------------------------------------------------- elementwise

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, const uint16_t* u, uint16_t* out,
                                                       long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const float gv = h2f(g[i]);
    out[i] = f2h((gv / (1.0f + __expf(-gv))) * h2f(u[i]));
  }
}

__global__ __launch_bounds__(256) void add_kernel(const uint16_t* a, const uint16_t* b, uint16_t* out, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    out[i] = f2h(h2f(a[i]) + h2f(b[i]));
}

static unsigned ew_blocks(long n) {
  long b = (n + 255) / 256;
  if (b > 8192) b = 8192;
  return (unsigned)(b < 1 ? 1 : b);
}

int silu_mul_f16_launch(const uint16_t* g, const uint16_t* u, uint16_t* out, long n, hipStream_t s) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3(ew_blocks(n)), dim3(256), 0, s, g, u, out, n);
  return qd_host::launch_status("silu_mul_kernel");
}

int add_f16_launch(const uint16_t* a, const uint16_t* b, uint16_t* out, long n, hipStream_t s) {
  hipLaunchKernelGGL(add_kernel, dim3(ew_blocks(n)), dim3(256), 0, s, a, b, out, n);
  return qd_host::launch_status("add_kernel");
}

// x[i] = table[token, i] as fp32; an out-of-range token id reads row 0.
__global__ __launch_bounds__(256) void embed_gather_kernel(const uint16_t* table, const int64_t* token, float* out,
                                                           int H, long V) {
  long t = token[0];
  if (t < 0 || t >= V) t = 0;
  const uint16_t* row = table + t * (long)H;
  for (int i = (blockIdx.x * blockDim.x + threadIdx.x) * 8; i < H; i += gridDim.x * blockDim.x * 8) {
    float v[8];
    unpack8(ld16(row + i), v);
    store_act8(out, i, v);
  }
}

int embed_gather_launch(const uint16_t* table, const int64_t* token, float* out, int H, long V, hipStream_t s) {
  hipLaunchKernelGGL(embed_gather_kernel, dim3(1), dim3(256), 0, s, table, token, out, H, V);
  return qd_host::launch_status("embed_gather_kernel");
}

__global__ void decode_advance_kernel(const int64_t* token, int64_t* out_tokens, int64_t* counter,
                                      int64_t* cache_position, int64_t* rope_position, int max_tokens) {
  if (threadIdx.x != 0) return;
  const int64_t c = counter[0];
  if (out_tokens != nullptr && c >= 0 && c < max_tokens) out_tokens[c] = token[0];
  counter[0] = c + 1;
  cache_position[0] += 1;
  rope_position[0] += 1;
  rope_position[1] += 1;
  rope_position[2] += 1;
}

int decode_advance_launch(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                          int64_t* rope_position, int max_tokens, hipStream_t s) {
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(64), 0, s, token, out_tokens, counter, cache_position,
                     rope_position, max_tokens);
  return qd_host::launch_status("decode_advance_kernel");
}

}  // namespace qd
