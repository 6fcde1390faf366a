// C ABI of the decode path (see include/qwen3vl_decode.h): argument checks,
// dtype dispatch, and the full batch-1 decode step.

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "qd_common.h"
#include "qd_kernels.h"

// ---------------------------------------------------------------- host helpers

namespace qd_host {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return QD_OK;
}

int cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace qd_host

namespace {

using qd::GemvArgs;
using u16 = uint16_t;

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

// Workspace layout of the lm_head argmax: [header (256 B): the blocks' arrival
// counter] [vals] [idx].
constexpr size_t kArgmaxHeader = 256;
size_t argmax_ws_bytes() {
  return kArgmaxHeader + (size_t)qd::kMaxArgmaxBlocks * (sizeof(float) + sizeof(long));
}
void argmax_ws(void* ws, GemvArgs& a) {
  char* b = reinterpret_cast<char*>(ws);
  a.argmax_count = reinterpret_cast<unsigned*>(b);
  a.part_idx = reinterpret_cast<long*>(b + kArgmaxHeader);
  a.part_val = reinterpret_cast<float*>(b + kArgmaxHeader + (size_t)qd::kMaxArgmaxBlocks * sizeof(long));
}

// Attention workspace: [arrival counters, one per kv head (256 B)] [o_part Hq*S*128 f32] [lse Hq*S f32].
size_t attn_ws_bytes(int Hq, int Hkv, int S_) {
  (void)Hkv;
  return 256 + (size_t)Hq * S_ * 128 * 4 + (size_t)Hq * S_ * 4;
}
void attn_ws(void* ws, qd::AttnArgs& a) {
  char* b = reinterpret_cast<char*>(ws);
  a.o_part = reinterpret_cast<float*>(b + 256);
  a.lse = reinterpret_cast<float*>(b + 256 + (size_t)a.Hq * a.n_split * 128 * 4);
}

// Scratch of the no-allocation attention entry point: one array per GPU
// (each device holds its own copy of a __device__ variable), resolved to its
// device address once per device with hipGetSymbolAddress and kept for the
// process.  Host code never uses the name `scratch` itself: on the host it is
// a stand-in, not a device address.
constexpr size_t kNoallocScratchBytes = QD_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

__global__ void clear_words_kernel(unsigned* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

// Device address of this device's scratch array; on the first call for a
// device the attention arrival counters at its head are cleared on `s` (a
// kernel, not a memset, so the call also works inside stream capture).
int noalloc_scratch(hipStream_t s, void** out) {
  static std::mutex mu;
  static std::vector<void*> addr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    qd_host::set_error("hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  std::lock_guard<std::mutex> lk(mu);
  if ((int)addr.size() <= dev) addr.resize(dev + 1, nullptr);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      qd_host::set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return e != hipSuccess ? (int)e : QD_ERR_WORKSPACE;
    }
    hipLaunchKernelGGL(clear_words_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<unsigned*>(p), 64);
    const int st = qd_host::launch_status("clear_words_kernel");
    if (st != QD_OK) return st;
    addr[dev] = p;
  }
  *out = addr[dev];
  return QD_OK;
}

int check_gemv_ptrs(const void* x, const void* W, const void* y, int N, int K) {
  QD_REQUIRE(x && W && y, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(N > 0 && K > 0 && (K % 8) == 0, QD_ERR_SHAPE, "need N > 0 and K %% 8 == 0 (N=%d K=%d)", N, K);
  QD_REQUIRE(a16(x) && a16(W), QD_ERR_ARG, "x and W must be 16-byte aligned");
  return QD_OK;
}

}  // namespace

// ---------------------------------------------------------------- C ABI

extern "C" {

int qd_version(void) { return 1; }
const char* qd_last_error(void) { return qd_host::g_err; }
int qd_device_cu_count(void) { return qd_host::cu_count(); }

int qd_matvec_f16(const void* x, const void* W, const void* bias, void* y, int N, int K, void* stream) {
  int st = check_gemv_ptrs(x, W, y, N, K);
  if (st) return st;
  GemvArgs a;
  a.x = x; a.W = (const u16*)W; a.bias = bias; a.y = y; a.N = N; a.K = K; a.ldw = K;
  return qd::gemv_store<qd::PRO_PLAIN, u16, u16>(a, S(stream));
}

int qd_splitk_matvec_f16(const void* x, const void* W, const void* bias, float* scratch, void* y, int N, int K,
                         int split_k, void* stream) {
  int st = check_gemv_ptrs(x, W, y, N, K);
  if (st) return st;
  QD_REQUIRE(scratch, QD_ERR_ARG, "null scratch");
  QD_REQUIRE(split_k >= 1 && K % split_k == 0, QD_ERR_SHAPE, "split_k %d must divide K %d", split_k, K);
  GemvArgs a;
  a.x = x; a.W = (const u16*)W; a.bias = bias; a.y = y; a.N = N; a.K = K; a.ldw = K; a.part_val = scratch;
  st = qd::gemv_splitk<u16, u16>(a, split_k, S(stream));
  QD_REQUIRE(st != QD_ERR_SHAPE && st != 1, QD_ERR_SHAPE,
             "split-K slice K/split_k=%d unsupported (need 512/1024/2048/3072/4096/6144)", K / split_k);
  return st;
}

int qd_rmsnorm_matvec_f16(const void* x, const void* gamma, const void* W, const void* bias, void* y, int N, int K,
                          float eps, void* stream) {
  int st = check_gemv_ptrs(x, W, y, N, K);
  if (st) return st;
  QD_REQUIRE(gamma && a16(gamma), QD_ERR_ARG, "gamma null or misaligned");
  GemvArgs a;
  a.x = x; a.gamma = (const u16*)gamma; a.W = (const u16*)W; a.bias = bias; a.y = y;
  a.N = N; a.K = K; a.ldw = K; a.eps = eps;
  return qd::gemv_store<qd::PRO_RMSNORM, u16, u16>(a, S(stream));
}

static int post_attn_mlp(const void* residual, const void* attn, const void* gamma, const void* W_gu,
                         const void* W_d, const void* bias, void* hidden_out, void* out, int H, int I, float eps,
                         const int64_t* position, int64_t* next_position, void* stream) {
  QD_REQUIRE(residual && attn && gamma && W_gu && W_d && hidden_out && out, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(a16(residual) && a16(attn) && a16(gamma) && a16(W_gu) && a16(W_d) && a16(hidden_out) && a16(out),
             QD_ERR_ARG, "pointers must be 16-byte aligned");
  QD_REQUIRE(H > 0 && I > 0 && H % 512 == 0 && I % 512 == 0, QD_ERR_SHAPE, "H, I must be multiples of 512");
  // r = residual + attn is written to `out` first, then used as the residual of down_proj
  // and overwritten element-wise in place (each element read before it is written).
  GemvArgs g;
  g.x = residual; g.x2 = attn; g.gamma = (const u16*)gamma; g.W = (const u16*)W_gu; g.y = hidden_out;
  g.r_out = out; g.N = I; g.K = H; g.ldw = H; g.up_offset = I; g.eps = eps;
  int st = qd::gemv_silu<qd::PRO_ADD_RMSNORM, u16, u16>(g, S(stream));
  QD_REQUIRE(st != QD_ERR_SHAPE && st != 1, QD_ERR_SHAPE, "unsupported H=%d", H);
  if (st) return st;
  GemvArgs d;
  d.x = hidden_out; d.W = (const u16*)W_d; d.bias = bias; d.residual = out; d.y = out;
  d.N = H; d.K = I; d.ldw = I;
  d.next_src = position; d.next_dst = next_position;
  st = qd::gemv_store<qd::PRO_PLAIN, u16, u16>(d, S(stream));
  return st;
}

int qd_post_attn_mlp_f16(const void* residual, const void* attn, const void* gamma, const void* W_gu,
                         const void* W_d, const void* bias, void* hidden_out, void* out, int H, int I, float eps,
                         void* stream) {
  return post_attn_mlp(residual, attn, gamma, W_gu, W_d, bias, hidden_out, out, H, I, eps, nullptr, nullptr,
                       stream);
}

int qd_post_attn_mlp_next_f16(const void* residual, const void* attn, const void* gamma, const void* W_gu,
                              const void* W_d, const void* bias, void* hidden_out, void* out, int H, int I,
                              float eps, const int64_t* position, int64_t* next_position, void* stream) {
  QD_REQUIRE(position && next_position, QD_ERR_ARG, "null position pointer");
  return post_attn_mlp(residual, attn, gamma, W_gu, W_d, bias, hidden_out, out, H, I, eps, position, next_position,
                       stream);
}

int qd_gateup_silu_down_f16(const void* x, const void* W_gu, const void* W_d, const void* bias, void* hidden_out,
                            void* out, int H, int I, void* stream) {
  QD_REQUIRE(x && W_gu && W_d && hidden_out && out, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(a16(x) && a16(W_gu) && a16(W_d) && a16(hidden_out), QD_ERR_ARG, "pointers must be 16-byte aligned");
  QD_REQUIRE(H > 0 && I > 0 && H % 512 == 0 && I % 512 == 0, QD_ERR_SHAPE, "H, I must be multiples of 512");
  GemvArgs g;
  g.x = x; g.W = (const u16*)W_gu; g.y = hidden_out; g.N = I; g.K = H; g.ldw = H; g.up_offset = I;
  int st = qd::gemv_silu<qd::PRO_PLAIN, u16, u16>(g, S(stream));
  QD_REQUIRE(st != QD_ERR_SHAPE && st != 1, QD_ERR_SHAPE, "unsupported H=%d", H);
  if (st) return st;
  GemvArgs d;
  d.x = hidden_out; d.W = (const u16*)W_d; d.bias = bias; d.y = out; d.N = H; d.K = I; d.ldw = I;
  return qd::gemv_store<qd::PRO_PLAIN, u16, u16>(d, S(stream));
}

int qd_add_rmsnorm_matvec_f16(const void* residual, const void* x, const void* gamma, const void* W,
                              const void* bias, void* residual_out, void* y, int N, int K, float eps, void* stream) {
  int st = check_gemv_ptrs(x, W, y, N, K);
  if (st) return st;
  QD_REQUIRE(residual && gamma && a16(residual) && a16(gamma) && (!residual_out || a16(residual_out)), QD_ERR_ARG,
             "residual/gamma null or misaligned");
  QD_REQUIRE(K % 512 == 0, QD_ERR_SHAPE, "K must be a multiple of 512 (K=%d)", K);
  GemvArgs a;
  a.x = residual; a.x2 = x; a.gamma = (const u16*)gamma; a.W = (const u16*)W; a.bias = bias; a.y = y;
  a.r_out = residual_out; a.N = N; a.K = K; a.ldw = K; a.eps = eps;
  st = qd::gemv_store<qd::PRO_ADD_RMSNORM, u16, u16>(a, S(stream));
  QD_REQUIRE(st != QD_ERR_SHAPE && st != 1, QD_ERR_SHAPE, "unsupported K=%d", K);
  return st;
}

int qd_silu_matvec_f16(const void* gate_up, const void* W, const void* bias, void* y, int N, int K, void* stream) {
  int st = check_gemv_ptrs(gate_up, W, y, N, K);
  if (st) return st;
  QD_REQUIRE(K % 512 == 0, QD_ERR_SHAPE, "K must be a multiple of 512 (K=%d)", K);
  GemvArgs a;
  a.x = gate_up; a.x2 = (const u16*)gate_up + K; a.W = (const u16*)W; a.bias = bias; a.y = y;
  a.N = N; a.K = K; a.ldw = K;
  st = qd::gemv_store<qd::PRO_SILU, u16, u16>(a, S(stream));
  QD_REQUIRE(st != QD_ERR_SHAPE && st != 1, QD_ERR_SHAPE, "unsupported K=%d", K);
  return st;
}

size_t qd_lm_head_workspace_bytes(int V) {
  (void)V;
  return argmax_ws_bytes();
}

int qd_lm_head_argmax(const void* h, int h_dtype, const void* gamma, float eps, const void* W, int V, int H,
                      void* logits_out, int64_t* token_out, void* workspace, void* stream) {
  QD_REQUIRE(h && W && token_out && workspace, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(a16(h) && a16(W) && (!gamma || a16(gamma)), QD_ERR_ARG, "pointers must be 16-byte aligned");
  QD_REQUIRE(V > 0 && H > 0 && H % 512 == 0, QD_ERR_SHAPE, "H must be a multiple of 512 (H=%d)", H);
  QD_REQUIRE(h_dtype == QD_F16 || h_dtype == QD_F32, QD_ERR_ARG, "bad h dtype");
  GemvArgs a;
  a.x = h; a.gamma = (const u16*)gamma; a.eps = eps; a.W = (const u16*)W; a.N = V; a.K = H; a.ldw = H;
  a.y = logits_out; a.token = token_out;
  argmax_ws(workspace, a);
  int st;
  if (h_dtype == QD_F32) {
    QD_REQUIRE(gamma, QD_ERR_ARG, "fp32 hidden requires the final-norm gamma");
    st = qd::gemv_argmax<qd::PRO_RMSNORM, float, u16>(a, S(stream));
  } else if (gamma) {
    st = qd::gemv_argmax<qd::PRO_RMSNORM, u16, u16>(a, S(stream));
  } else {
    st = qd::gemv_argmax<qd::PRO_PLAIN, u16, u16>(a, S(stream));
  }
  QD_REQUIRE(st != QD_ERR_SHAPE && st != 1, QD_ERR_SHAPE, "unsupported H=%d", H);
  return st;
}

int qd_q_rope_kv_update(const void* q, const void* k, const void* v, int qkv_dtype, long q_stride, long k_stride,
                        long v_stride, const void* q_weight, const void* k_weight, float eps, const void* cos,
                        const void* sin, const int64_t* rope_pos, const float* inv_freq, int sec_t, int sec_h,
                        int sec_w, void* q_out, int q_out_dtype, void* k_cache, void* v_cache, long cache_stride_h,
                        long cache_stride_s, int T, const int64_t* cache_position, int Hq, int Hkv, void* stream) {
  (void)sec_t;
  QD_REQUIRE(q && k && v && q_weight && k_weight && q_out && k_cache && v_cache && cache_position, QD_ERR_ARG,
             "null pointer");
  QD_REQUIRE((cos && sin) || (rope_pos && inv_freq), QD_ERR_ARG, "need cos/sin or rope_pos + inv_freq");
  QD_REQUIRE(Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && Hq / Hkv <= 4, QD_ERR_SHAPE, "need Hq = G*Hkv with G <= 4");
  QD_REQUIRE(T > 0, QD_ERR_SHAPE, "T must be positive");
  QD_REQUIRE(qkv_dtype == q_out_dtype && (qkv_dtype == QD_F16 || qkv_dtype == QD_F32), QD_ERR_ARG,
             "q/k/v and q_out dtype must match (f16 or f32)");
  qd::RopeArgs a;
  a.q = q; a.k = k; a.v = v; a.q_stride = q_stride; a.k_stride = k_stride; a.v_stride = v_stride;
  a.q_weight = (const u16*)q_weight; a.k_weight = (const u16*)k_weight; a.eps = eps;
  a.cos = (const u16*)cos; a.sin = (const u16*)sin; a.rope_pos = rope_pos; a.inv_freq = inv_freq;
  a.sec_h = sec_h; a.sec_w = sec_w; a.q_out = q_out; a.k_cache = (u16*)k_cache; a.v_cache = (u16*)v_cache;
  a.cache_stride_h = cache_stride_h; a.cache_stride_s = cache_stride_s; a.T = T; a.cache_position = cache_position;
  a.Hq = Hq; a.Hkv = Hkv;
  return qkv_dtype == QD_F16 ? qd::q_rope_kv_launch<u16, u16>(a, S(stream))
                             : qd::q_rope_kv_launch<float, float>(a, S(stream));
}

int qd_qk_norm_rope_f16(const void* q, const void* k, const void* q_weight, const void* k_weight, const void* cos,
                        const void* sin, void* q_out, void* k_out, int M, int Hq, int Hkv, float eps, void* stream) {
  QD_REQUIRE(q && k && q_weight && k_weight && cos && sin && q_out && k_out, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(M > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 4, QD_ERR_SHAPE, "bad head counts");
  qd::RopeArgs a;
  a.q = q; a.k = k; a.q_stride = 128; a.k_stride = 128; a.q_row = (long)Hq * 128; a.k_row = (long)Hkv * 128;
  a.q_weight = (const u16*)q_weight; a.k_weight = (const u16*)k_weight; a.eps = eps;
  a.cos = (const u16*)cos; a.sin = (const u16*)sin; a.cs_row = 128; a.q_out = q_out; a.k_out = k_out;
  a.Hq = Hq; a.Hkv = Hkv; a.M = M;
  return qd::qk_norm_rope_f16_launch(a, S(stream));
}

int qd_add_rmsnorm_f16(const void* residual, const void* x, const void* weight, void* out_sum, void* out_norm,
                       int rows, int cols, float eps, void* stream) {
  QD_REQUIRE(residual && x && weight && out_sum && out_norm, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(rows > 0 && cols > 0, QD_ERR_SHAPE, "empty input");
  return qd::add_rmsnorm_f16_launch((const u16*)residual, (const u16*)x, (const u16*)weight, (u16*)out_sum,
                                    (u16*)out_norm, rows, cols, eps, S(stream));
}

int qd_rmsnorm_f16(const void* x, const void* weight, void* out, int rows, int cols, float eps, void* stream) {
  QD_REQUIRE(x && weight && out, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(rows > 0 && cols > 0, QD_ERR_SHAPE, "empty input");
  return qd::add_rmsnorm_f16_launch(nullptr, (const u16*)x, (const u16*)weight, nullptr, (u16*)out, rows, cols, eps,
                                    S(stream));
}

int qd_silu_mul_f16(const void* gate, const void* up, void* out, long n, void* stream) {
  QD_REQUIRE(gate && up && out, QD_ERR_ARG, "null pointer");
  if (n <= 0) return QD_OK;
  return qd::silu_mul_f16_launch((const u16*)gate, (const u16*)up, (u16*)out, n, S(stream));
}

int qd_add_f16(const void* a, const void* b, void* out, long n, void* stream) {
  QD_REQUIRE(a && b && out, QD_ERR_ARG, "null pointer");
  if (n <= 0) return QD_OK;
  return qd::add_f16_launch((const u16*)a, (const u16*)b, (u16*)out, n, S(stream));
}

size_t qd_attention_workspace_bytes(int Hq, int Hkv, int n_split) { return attn_ws_bytes(Hq, Hkv, n_split); }

int qd_attention_default_splits(int T) {
  // ~128 positions per workgroup, at least 4 and at most 32 splits per kv
  // head.  Up to 16 splits (T <= 2048) the merge runs in the partial kernel (one
  // launch); beyond, the merge kernel (one round trip for up to 64 splits).
  // Measured per call at T = L, cold copies (16 / 24 / 32 splits, us): 8.14 /
  // 8.49 / 8.20 at 2048, 9.05 / 8.72 / 9.00 at 3072, 9.75 / 9.61 / 9.34 at
  // 4096, 11.3 / 10.7 / 10.5 at 6144, 12.8 / 12.4 / 11.6 at 8192, 20.2 / 18.3
  // / 17.4 at 16384; 48 and 64 splits are no faster than 32.
  int s = (T + 127) / 128;
  if (s < 4) s = 4;
  if (s > 32) s = 32;
  return s;
}

static int attn_common(qd::AttnArgs& a, const void* q, int q_dtype, long q_stride, const void* k_cache,
                       const void* v_cache, long cache_stride_h, long cache_stride_s, int T,
                       const int64_t* cache_position, float scale, int Hq, int Hkv, int n_split) {
  QD_REQUIRE(q && k_cache && v_cache && cache_position, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(q_dtype == QD_F16 || q_dtype == QD_F32, QD_ERR_ARG, "bad q dtype");
  QD_REQUIRE(Hkv > 0 && Hq % Hkv == 0 && (Hq / Hkv == 1 || Hq / Hkv == 2 || Hq / Hkv == 4), QD_ERR_SHAPE,
             "need Hq/Hkv in {1,2,4}");
  QD_REQUIRE(T > 0 && n_split >= 1 && n_split <= 1024, QD_ERR_SHAPE, "bad T or n_split");
  QD_REQUIRE(a16(q) && a16(k_cache) && a16(v_cache) && cache_stride_s % 8 == 0 && cache_stride_h % 8 == 0 &&
                 q_stride % 8 == 0,
             QD_ERR_ARG, "q/cache pointers and strides must be 16-byte aligned");
  a.q = q; a.q_stride = q_stride; a.k = (const u16*)k_cache; a.v = (const u16*)v_cache;
  a.stride_h = cache_stride_h; a.stride_s = cache_stride_s; a.T = T; a.cache_position = cache_position;
  a.scale = scale; a.Hq = Hq; a.Hkv = Hkv; a.n_split = n_split;
  return QD_OK;
}

int qd_attention_decode(const void* q, int q_dtype, long q_stride, const void* k_cache, const void* v_cache,
                        long cache_stride_h, long cache_stride_s, int T, const int64_t* cache_position, float scale,
                        void* out, int out_dtype, int Hq, int Hkv, int n_split, void* workspace, void* stream) {
  qd::AttnArgs a;
  int st = attn_common(a, q, q_dtype, q_stride, k_cache, v_cache, cache_stride_h, cache_stride_s, T, cache_position,
                       scale, Hq, Hkv, n_split);
  if (st) return st;
  QD_REQUIRE(out && workspace, QD_ERR_ARG, "null out/workspace");
  QD_REQUIRE(out_dtype == QD_F16 || out_dtype == QD_F32, QD_ERR_ARG, "bad out dtype");
  a.out = out;
  attn_ws(workspace, a);
  if (q_dtype == out_dtype && n_split <= 16 && Hkv <= 64) {
    // one launch: the last split of each kv head to finish merges them all
    // (arrival counters in the workspace header: zeroed once, self-resetting).
    // It reads the partials 8 splits per round trip; with more than 16 splits
    // the merge kernel, which reads them all in parallel, is faster.
    a.done = reinterpret_cast<unsigned*>(workspace);
    return q_dtype == QD_F16 ? qd::attention_partial_launch<u16>(a, S(stream))
                             : qd::attention_partial_launch<float>(a, S(stream));
  }
  st = q_dtype == QD_F16 ? qd::attention_partial_launch<u16>(a, S(stream))
                         : qd::attention_partial_launch<float>(a, S(stream));
  if (st) return st;
  return out_dtype == QD_F16 ? qd::attention_merge_launch<u16>(a, S(stream))
                             : qd::attention_merge_launch<float>(a, S(stream));
}

int qd_attention_qkv_decode_f16(const void* qkv, const void* q_weight, const void* k_weight, float eps,
                                const void* cos, const void* sin, void* k_cache, void* v_cache, long cache_stride_h,
                                long cache_stride_s, int T, const int64_t* cache_position, float scale, void* out,
                                int Hq, int Hkv, int n_split, void* workspace, void* stream) {
  qd::AttnArgs a;
  int st = attn_common(a, qkv, QD_F16, 128, k_cache, v_cache, cache_stride_h, cache_stride_s, T, cache_position,
                       scale, Hq, Hkv, n_split);
  if (st) return st;
  QD_REQUIRE(q_weight && k_weight && cos && sin && out && workspace, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(Hq / Hkv == 2, QD_ERR_SHAPE, "the fused prologue serves 2 q heads per kv head (got %d)", Hq / Hkv);
  QD_REQUIRE(a16(out), QD_ERR_ARG, "out must be 16-byte aligned");
  a.qkv = qkv; a.q_weight = (const u16*)q_weight; a.k_weight = (const u16*)k_weight; a.eps = eps;
  a.cos = (const u16*)cos; a.sin = (const u16*)sin;
  a.k_w = (u16*)k_cache; a.v_w = (u16*)v_cache;
  a.out = out;
  attn_ws(workspace, a);
  if (n_split <= 16 && Hkv <= 64) {
    a.done = reinterpret_cast<unsigned*>(workspace);
    return qd::attention_partial_launch<u16>(a, S(stream));
  }
  if ((st = qd::attention_partial_launch<u16>(a, S(stream)))) return st;
  return qd::attention_merge_launch<u16>(a, S(stream));
}

int qd_attention_decode_noalloc(const void* q, int q_dtype, long q_stride, const void* k_cache,
                                const void* v_cache, long cache_stride_h, long cache_stride_s, int T,
                                const int64_t* cache_position, float scale, void* out, int out_dtype, int Hq, int Hkv,
                                int n_split, void* stream) {
  // the size check comes first: an oversized request launches nothing
  QD_REQUIRE(Hq > 0 && Hkv > 0 && n_split >= 1 && n_split <= 1024, QD_ERR_SHAPE, "bad head or split counts");
  const size_t need = attn_ws_bytes(Hq, Hkv, n_split);
  QD_REQUIRE(need <= kNoallocScratchBytes, QD_ERR_WORKSPACE,
             "qd_attention_decode_noalloc: Hq=%d x n_split=%d needs %zu bytes of scratch, more than the %zu the "
             "library holds per GPU (use qd_attention_decode with a workspace, or fewer splits)",
             Hq, n_split, need, kNoallocScratchBytes);
  void* ws = nullptr;
  const int st = noalloc_scratch(S(stream), &ws);
  if (st) return st;
  return qd_attention_decode(q, q_dtype, q_stride, k_cache, v_cache, cache_stride_h, cache_stride_s, T,
                             cache_position, scale, out, out_dtype, Hq, Hkv, n_split, ws, stream);
}

int qd_attention_partial(const void* q, int q_dtype, long q_stride, const void* k_cache, const void* v_cache,
                         long cache_stride_h, long cache_stride_s, int T, const int64_t* cache_position, float scale,
                         float* o_part, float* lse, int Hq, int Hkv, int n_split, void* stream) {
  qd::AttnArgs a;
  int st = attn_common(a, q, q_dtype, q_stride, k_cache, v_cache, cache_stride_h, cache_stride_s, T, cache_position,
                       scale, Hq, Hkv, n_split);
  if (st) return st;
  QD_REQUIRE(o_part && lse, QD_ERR_ARG, "null partial buffers");
  a.o_part = o_part; a.lse = lse;
  return q_dtype == QD_F16 ? qd::attention_partial_launch<u16>(a, S(stream))
                           : qd::attention_partial_launch<float>(a, S(stream));
}

int qd_attention_merge(const float* o_part, const float* lse, void* out, int out_dtype, int Hq, int n_split,
                       void* stream) {
  QD_REQUIRE(o_part && lse && out, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(Hq > 0 && n_split >= 1, QD_ERR_SHAPE, "bad sizes");
  qd::AttnArgs a;
  a.o_part = const_cast<float*>(o_part); a.lse = const_cast<float*>(lse); a.out = out; a.Hq = Hq;
  a.n_split = n_split;
  return out_dtype == QD_F16 ? qd::attention_merge_launch<u16>(a, S(stream))
                             : qd::attention_merge_launch<float>(a, S(stream));
}

// ---------------------------------------------------------------- decode step

namespace {

struct StepBuffers {
  float* x;        // residual stream [H]
  float* qkv;      // [Hq*D + 2*Hkv*D]
  float* q_rot;    // [Hq*D]
  float* attn;     // [Hq*D]
  float* r;        // [H]
  float* hidden;   // [I]
  char* attn_ws;
  char* argmax_ws;
  unsigned* control;  // persistent step: status word
  // batch step (B > 1): operand images of x (times the next RMSNorm weight),
  // attention output, r (times post_norm) and hidden; per-row-group sums of
  // squares and image scales of x and r; K-split partials; lm_head partials
  u16* xb;
  u16* ab;
  u16* rb;
  u16* hb;
  float* ss_x;
  float* ss_r;
  float* sc_x;
  float* sc_r;
  float* kpart;
  unsigned* kcount;
  unsigned* attn_done;
  float* part_val;
  long* part_idx;
  unsigned* qkv_t;    // batch step, qkv GEMV in the attention launch: tagged words [8][rows]
  unsigned* qkv_ctl;  // its launch count (parity) and finished-workgroup counter
};

using qd::kBatchMaxKsplit;
constexpr int kBatchCounters = 1024;

int batch_of(const qd_model_desc* d) { return d->batch > 1 ? d->batch : 1; }

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Per-sequence buffers are [B][n] (B = batch, 1 for the batch-1 step).
bool step_layout(const qd_model_desc* d, int splits, StepBuffers* b, size_t* total) {
  const size_t B = (size_t)batch_of(d);
  const size_t qkv_rows = (size_t)d->num_heads * d->head_dim + 2 * (size_t)d->num_kv_heads * d->head_dim;
  size_t off = 0;
  size_t o_x = off; off += align256(4 * B * (size_t)d->hidden);
  size_t o_qkv = off; off += align256(4 * B * qkv_rows);
  size_t o_q = off; off += align256(4 * B * (size_t)d->num_heads * d->head_dim);
  size_t o_a = off; off += align256(4 * B * (size_t)d->num_heads * d->head_dim);
  size_t o_r = off; off += align256(4 * B * (size_t)d->hidden);
  size_t o_h = off; off += align256(4 * B * (size_t)d->intermediate);
  size_t o_aw = off; off += align256(256 + B * (attn_ws_bytes(d->num_heads, d->num_kv_heads, splits) - 256));
  size_t o_gw = off; off += align256(argmax_ws_bytes());
  size_t o_ct = off; off += 256;
  size_t o_xb = off, o_ab = off, o_rb = off, o_hb = off, o_ssx = off, o_ssr = off, o_sc = off, o_kp = off,
         o_kc = off, o_ad = off, o_pv = off, o_pi = off, o_qt = off, o_qc = off;
  if (B > 1) {
    // an operand image holds 16 fp16 columns per K index
    const size_t groups = (size_t)qd::gemv8_row_groups(d->vocab);
    const size_t hgroups = (size_t)qd::gemv8_row_groups(d->hidden, 8);   // row groups of o_proj / down
    const size_t max_rows = qkv_rows > (size_t)d->intermediate ? qkv_rows : (size_t)d->intermediate;
    o_xb = off; off += align256(32 * (size_t)d->hidden);
    o_ab = off; off += align256(32 * (size_t)d->num_heads * d->head_dim);
    o_rb = off; off += align256(32 * (size_t)d->hidden);
    o_hb = off; off += align256(32 * (size_t)d->intermediate);
    o_ssx = off; off += align256(4 * hgroups * qd::kBatchMax);
    o_ssr = off; off += align256(4 * hgroups * qd::kBatchMax);
    o_sc = off; off += 256;
    o_kp = off; off += align256(4 * (size_t)qd::gemv8_row_groups((long)max_rows) * kBatchMaxKsplit * 2 * 128);
    o_kc = off; off += align256(4 * (size_t)kBatchCounters);
    o_ad = off; off += align256(4 * B * (size_t)d->num_kv_heads);
    o_pv = off; off += align256(4 * groups * qd::kBatchMax);
    o_pi = off; off += align256(8 * groups * qd::kBatchMax);
    o_qt = off; off += align256(4 * qd::kBatchMax * qkv_rows);
    o_qc = off; off += 256;
  }
  *total = off;
  if (b != nullptr) {
    char* base = reinterpret_cast<char*>(d->workspace);
    b->x = reinterpret_cast<float*>(base + o_x);
    b->qkv = reinterpret_cast<float*>(base + o_qkv);
    b->q_rot = reinterpret_cast<float*>(base + o_q);
    b->attn = reinterpret_cast<float*>(base + o_a);
    b->r = reinterpret_cast<float*>(base + o_r);
    b->hidden = reinterpret_cast<float*>(base + o_h);
    b->attn_ws = base + o_aw;
    b->argmax_ws = base + o_gw;
    b->control = reinterpret_cast<unsigned*>(base + o_ct);
    b->xb = reinterpret_cast<u16*>(base + o_xb);
    b->ab = reinterpret_cast<u16*>(base + o_ab);
    b->rb = reinterpret_cast<u16*>(base + o_rb);
    b->hb = reinterpret_cast<u16*>(base + o_hb);
    b->ss_x = reinterpret_cast<float*>(base + o_ssx);
    b->ss_r = reinterpret_cast<float*>(base + o_ssr);
    b->sc_x = reinterpret_cast<float*>(base + o_sc);
    b->sc_r = b->sc_x + qd::kBatchMax;
    b->kpart = reinterpret_cast<float*>(base + o_kp);
    b->kcount = reinterpret_cast<unsigned*>(base + o_kc);
    b->attn_done = reinterpret_cast<unsigned*>(base + o_ad);
    b->part_val = reinterpret_cast<float*>(base + o_pv);
    b->part_idx = reinterpret_cast<long*>(base + o_pi);
    b->qkv_t = reinterpret_cast<unsigned*>(base + o_qt);
    b->qkv_ctl = reinterpret_cast<unsigned*>(base + o_qc);
  }
  return true;
}

// Splits per kv head: batch-1 default; a batch step already has B x Hkv
// sequence-heads to spread over the CUs, so it takes 1/B as many (at least 4).
int splits_of(const qd_model_desc* d) {
  if (d->attn_splits > 0) return d->attn_splits;
  const int B = batch_of(d);
  if (B > 1) {
    // batch: ~64 positions per workgroup over the B sequences, 4..64 / B splits
    const int s = std::min(64, std::max(4, (d->capacity + 63) / 64));
    return std::max(4, s / B);
  }
  return qd_attention_default_splits(d->capacity);
}

}  // namespace

size_t qd_decode_workspace_bytes(const qd_model_desc* d) {
  if (d == nullptr) return 0;
  size_t total = 0;
  step_layout(d, splits_of(d), nullptr, &total);
  return total;
}

int qd_decode_workspace_layout(const qd_model_desc* d, size_t* offsets, int n) {
  QD_REQUIRE(d && d->workspace, QD_ERR_ARG, "descriptor without workspace");
  StepBuffers b;
  size_t total = 0;
  step_layout(d, splits_of(d), &b, &total);
  const char* base = reinterpret_cast<const char*>(d->workspace);
  const void* bufs[6] = {b.x, b.qkv, b.q_rot, b.attn, b.r, b.hidden};
  for (int i = 0; i < n && i < 6; ++i) offsets[i] = (size_t)(reinterpret_cast<const char*>(bufs[i]) - base);
  return 6;
}

namespace {

bool persistent_device_unsupported(char* why, size_t n);

// Why the persistent step cannot serve this descriptor on the current device
// (empty when it can).
bool persistent_unsupported(const qd_model_desc* d, char* why, size_t n) {
  why[0] = 0;
  if (batch_of(d) > 1) {
    snprintf(why, n, "the persistent step runs batch 1 only (batch %d)", d->batch);
    return true;
  }
  if (d->hidden != qd::kPersistHidden || d->num_heads != qd::kPersistHeads ||
      d->num_kv_heads != qd::kPersistKvHeads || d->head_dim != qd::kPersistHeadDim ||
      d->intermediate != qd::kPersistInter) {
    snprintf(why, n, "persistent step is specialised for H=2048, 16/8 heads of 128, I=6144");
    return true;
  }
  if (d->num_layers < 1 || d->num_layers > qd::kPersistMaxLayers) {
    snprintf(why, n, "persistent step supports 1..%d layers", qd::kPersistMaxLayers);
    return true;
  }
  return persistent_device_unsupported(why, n);
}

// Why the current device cannot keep the persistent grid resident (empty when
// it can); the occupancy query runs once per device.
bool persistent_device_unsupported(char* why, size_t n) {
  why[0] = 0;
  static std::mutex mu;
  static std::vector<int> support;  // per device: 0 unknown, 1 ok, 2 unsupported
  static std::vector<std::string> reason;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    snprintf(why, n, "no current HIP device");
    return true;
  }
  std::lock_guard<std::mutex> lk(mu);
  if ((int)support.size() <= dev) {
    support.resize(dev + 1, 0);
    reason.resize(dev + 1);
  }
  if (support[dev] == 0) {
    char buf[256] = "";
    support[dev] = qd::decode_persistent_check_device(buf, sizeof(buf)) ? 2 : 1;
    reason[dev] = buf;
  }
  if (support[dev] == 2) snprintf(why, n, "%s", reason[dev].c_str());
  return support[dev] == 2;
}

// The persistent step's hand-off words live in one area per device, in
// uncached device memory: the producers' coherent stores and the consumers'
// coherent polls then go straight to memory, which shortens a hand-off under
// full-chip HBM load (about 0.3 us per round trip, measured) and leaves no
// dirty L2 lines for the kernel-boundary cache maintenance.  The area is
// allocated and zeroed at the first persistent step on a device (outside
// stream capture) and kept until the process ends: memory that kernels have
// read through the uncached path is never freed.  Every persistent launch on
// the device shares it (the kernel's per-device layer generation keeps the
// word parities consistent across launches of any layer count), so persistent
// steps on one device must not overlap - they cannot run concurrently anyway,
// each needs every CU.  Beside it, in ordinary device memory: the generation
// and arrival counters (out_ctrl[0], [1]).
int persist_area(hipStream_t s, unsigned** out, unsigned** out_ctrl) {
  static std::mutex mu;
  static std::vector<unsigned*> areas, ctrls;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    qd_host::set_error("no current HIP device: %s", hipGetErrorString(e));
    return (int)e;
  }
  std::lock_guard<std::mutex> lk(mu);
  if ((int)areas.size() <= dev) {
    areas.resize(dev + 1, nullptr);
    ctrls.resize(dev + 1, nullptr);
  }
  if (areas[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(s, &cs);
    if (e != hipSuccess || cs != hipStreamCaptureStatusNone) {
      qd_host::set_error("the persistent step allocates its hand-off area at the first step on a device: run "
                         "one step outside stream capture first");
      return QD_ERR_ARG;
    }
    const size_t bytes = 4 * qd::kPersistTaggedWords;
    unsigned *p = nullptr, *c = nullptr;
    e = hipExtMallocWithFlags(reinterpret_cast<void**>(&p), bytes, hipDeviceMallocUncached);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&c), 256);
    if (e == hipSuccess) e = hipMemset(p, 0, bytes);
    if (e == hipSuccess) e = hipMemset(c, 0, 256);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      qd_host::set_error("persistent step hand-off area (%zu bytes, uncached): %s", bytes, hipGetErrorString(e));
      return (int)e;
    }
    areas[dev] = p;
    ctrls[dev] = c;
  }
  *out = areas[dev];
  *out_ctrl = ctrls[dev];
  return QD_OK;
}

// Polls per thread and launch before a persistent wait gives up (0: the
// kernel's default); set by qd_persistent_set_spin_limit for tests of the
// failure path, read when a launch's arguments are built.
std::atomic<unsigned> g_spin_limit{0};

// The hand-off buffers of a launch, carved from the per-device area.
void set_handoff_words(qd::PersistArgs& p, unsigned* t) {
  p.x_t = t; t += qd::kPersistHidden;
  p.qkv_t = t; t += (qd::kPersistHeads + 2 * qd::kPersistKvHeads) * qd::kPersistHeadDim;
  p.opart_t = t; t += (size_t)qd::kPersistHeads * qd::kPersistSplits * qd::kPersistHeadDim;
  p.lse_t = t; t += qd::kPersistHeads * qd::kPersistSplits;
  p.att_t = t; t += qd::kPersistHeads * qd::kPersistHeadDim;
  p.r_t = t; t += qd::kPersistHidden;
  p.hid_t = t;
}

int launch_persistent(const qd_model_desc* d, const StepBuffers& b, hipStream_t s) {
  qd::PersistArgs p;
  memset(&p, 0, sizeof(p));
  for (int l = 0; l < d->num_layers; ++l) {
    const qd_layer_weights& w = d->layers[l];
    p.layers[l] = qd::PersistLayer{(const u16*)w.qkv,        (const u16*)w.o_proj,    (const u16*)w.gate_up,
                                   (const u16*)w.down,       (const u16*)w.input_norm, (const u16*)w.post_norm,
                                   (const u16*)w.q_norm,     (const u16*)w.k_norm,    (u16*)w.k_cache,
                                   (u16*)w.v_cache,          nullptr};
  }
  p.num_layers = d->num_layers;
  p.T = d->capacity;
  p.vocab = d->vocab;
  p.eps = d->eps;
  p.scale = 1.0f / sqrtf((float)d->head_dim);
  p.sec_h = d->sec_h;
  p.sec_w = d->sec_w;
  p.embed = (const u16*)d->embed;
  p.token = d->token;
  p.cache_position = d->cache_position;
  p.rope_position = d->rope_position;
  p.inv_freq = d->inv_freq;
  unsigned *t = nullptr, *ctrl = nullptr;
  int st = persist_area(s, &t, &ctrl);
  if (st) return st;
  set_handoff_words(p, t);
  p.x_out = b.x;
  p.status = b.control;
  p.generation = ctrl;
  p.done = ctrl + 1;
  p.spin_limit = g_spin_limit.load();
  return qd::decode_persistent_launch(p, s);
}

}  // namespace

int qd_decode_step_mode(const qd_model_desc* d) {
  QD_REQUIRE(d, QD_ERR_ARG, "null descriptor");
  QD_REQUIRE(d->step_mode >= QD_STEP_AUTO && d->step_mode <= QD_STEP_PERSISTENT, QD_ERR_ARG, "bad step_mode %d",
             d->step_mode);
  if (d->step_mode == QD_STEP_CHAIN) return QD_STEP_CHAIN;
  char why[256];
  if (batch_of(d) > 1) {
    if (d->step_mode == QD_STEP_PERSISTENT) {
      qd_host::set_error("the persistent step runs batch 1 only (batch %d requested)", d->batch);
      return QD_ERR_SHAPE;
    }
    return QD_STEP_CHAIN;
  }
  if (persistent_unsupported(d, why, sizeof(why))) {
    if (d->step_mode == QD_STEP_PERSISTENT) {
      qd_host::set_error("%s", why);
      return QD_ERR_SHAPE;
    }
    return QD_STEP_CHAIN;
  }
  return QD_STEP_PERSISTENT;
}

namespace {

// Work split of a batch GEMV with `rows` output rows (gate rows for SiLU):
// rows per workgroup (8 for K = 2048 when 16 would leave fewer row groups than
// CUs (o_proj) and for gate_up: more workgroups and no K split; else 16) and
// workgroups per row group along K (K ranges of 1024, 2048, 3072 or
// 6144): the smallest split whose workgroup count is a multiple of the 256
// CUs, else the smallest that gives at least 256 workgroups.
struct BatchSplit {
  int rows_per_group, ksplit;
};
BatchSplit batch_split(long rows, long K, bool silu) {
  const int rg = ((silu && K == 2048) || (!silu && rows / 16 < 256 && rows % 8 == 0 && K <= 2048)) ? 8 : 16;
  const long groups = rows / rg;
  const int cand[] = {1, 2, 3, 6};
  auto ok = [&](int ks) {
    const long kw = K / ks;
    if (K % ks != 0) return false;
    if (rg == 8) return ks == 1 && (kw == 2048 || kw == 6144);
    return silu ? (kw == 1024 || kw == 2048) : (kw == 1024 || kw == 2048 || kw == 3072 || kw == 6144);
  };
  for (int ks : cand)
    if (ok(ks) && (groups * ks) % 256 == 0) return {rg, ks};
  for (int ks : cand)
    if (ok(ks) && groups * ks >= 256) return {rg, ks};
  for (int ks : cand)
    if (ok(ks)) return {rg, ks};
  return {16, 1};
}

// Batch step (batch 2..8): the kernel chain with MFMA batch GEMVs and the
// split-KV attention run per sequence (grid y), every sequence at its own cache
// position; with QD_STEP_AUTO each layer's qkv GEMV runs inside its attention
// launch (attention_qkv8_launch) where the shape and the device allow it.  Activations move between the GEMVs as operand images: x (times
// the next input_norm, or final_norm after the last layer, scaled by rstd of
// the previous r), the attention output, r (times post_norm, scaled by rstd
// of x) and the MLP hidden; each producer also writes per-row-group sums of
// squares, from which the consumer applies its RMSNorm.
int batch_step(const qd_model_desc* d, hipStream_t s) {
  const int B = batch_of(d);
  QD_REQUIRE(B <= qd::kBatchMax, QD_ERR_SHAPE, "batch %d > %d", B, qd::kBatchMax);
  QD_REQUIRE(d->num_layers >= 1 && d->hidden == 2048 && d->num_heads * d->head_dim == 2048 &&
                 (d->intermediate == 2048 || d->intermediate == 6144) && d->vocab % 16 == 0,
             QD_ERR_SHAPE, "batch step supports H = Hq*D = 2048, I in {2048, 6144}, vocab %% 16 == 0");
  const int splits = splits_of(d);
  QD_REQUIRE(splits <= 64, QD_ERR_SHAPE, "batch step: at most 64 attention splits (got %d)", splits);
  StepBuffers b;
  size_t total = 0;
  step_layout(d, splits, &b, &total);
  const int H = d->hidden, D = d->head_dim, Hq = d->num_heads, Hkv = d->num_kv_heads, I = d->intermediate;
  const long qkv_rows = (long)Hq * D + 2L * Hkv * D;
  // partial sums of squares of x and r: one per row group of their producers
  // (down and o_proj)
  const int x_parts = qd::gemv8_row_groups(H, batch_split(H, I, false).rows_per_group);
  const int r_parts = qd::gemv8_row_groups(H, batch_split(H, (long)Hq * D, false).rows_per_group);
  // QD_STEP_AUTO: each layer's qkv GEMV runs inside its attention launch
  // (attention_qkv8_launch) where the shape and the device allow it; the
  // words it hands over and their counters live in this step's workspace
  const bool fuse_qkv = d->step_mode == QD_STEP_AUTO && H == 2048 && D == 128 && Hq == 2 * Hkv &&
                        qkv_rows == (long)qd::kQkv8Producers * 16 && (long)B * Hkv * splits >= qd::kQkv8Producers &&
                        splits <= 64 && qd::attention_qkv8_device_ok();
  int st = QD_OK;
  if ((st = qd::embed8_launch((const u16*)d->embed, d->token, b.x, H, d->vocab, B,
                              (const u16*)d->layers[0].input_norm, d->eps, b.xb, b.ss_x, b.sc_x, s)))
    return st;
  auto base = [&](qd::Gemv8Args& g, long N, long K, bool silu = false) {
    const BatchSplit sp = batch_split(N, K, silu);
    g.nseq = B; g.eps = d->eps; g.N = N; g.K = K; g.ldw = K; g.ksplit = sp.ksplit; g.rows_per_group = sp.rows_per_group;
    g.kpart = b.kpart; g.kcount = b.kcount;
  };
  // o_proj, gate_up and down in tile order (qd_model_desc.batch_tiled_weights):
  // every row group of the layout the GEMV's row group size implies
  const int gu_tiled = d->batch_tiled_weights ? 1 : 0;
  if (gu_tiled) {
    const struct { long rows, K; bool silu; } m[4] = {
        {qkv_rows, H, false}, {H, (long)Hq * D, false}, {I, H, true}, {H, I, false}};
    for (const auto& x : m) {
      const int rg = batch_split(x.rows, x.K, x.silu).rows_per_group;
      QD_REQUIRE(x.rows % rg == 0 && x.K % (rg == 8 ? 64 : 32) == 0, QD_ERR_SHAPE,
                 "tile-ordered weights need rows %% %d == 0 and K %% %d == 0 (%ld x %ld)", rg, rg == 8 ? 64 : 32, x.rows,
                 x.K);
    }
  }
  for (int li = 0; li < d->num_layers; ++li) {
    const qd_layer_weights& w = d->layers[li];
    const int xparts = li == 0 ? 1 : x_parts;   // the embedding kernel writes one partial
    qd::Gemv8Args g;
    base(g, qkv_rows, H);
    g.xb = b.xb; g.in_ss = b.ss_x; g.in_parts = xparts; g.in_scale = b.sc_x; g.W = (const u16*)w.qkv;
    g.y = b.qkv; g.ldy = qkv_rows; g.w_tiled = gu_tiled;
    if (!fuse_qkv && (st = qd::gemv8_launch(g, qd::EPI_STORE, s))) return st;
    qd::AttnArgs aa;
    aa.k = (const u16*)w.k_cache; aa.v = (const u16*)w.v_cache; aa.k_w = (u16*)w.k_cache; aa.v_w = (u16*)w.v_cache;
    aa.stride_h = (long)d->capacity * D; aa.stride_s = D; aa.T = d->capacity; aa.cache_position = d->cache_position;
    aa.scale = 1.0f / sqrtf((float)D); aa.Hq = Hq; aa.Hkv = Hkv; aa.n_split = splits; aa.out = b.attn;
    aa.qkv = b.qkv; aa.q_weight = (const u16*)w.q_norm; aa.k_weight = (const u16*)w.k_norm; aa.eps = d->eps;
    aa.rope_pos = d->rope_position; aa.inv_freq = d->inv_freq; aa.sec_h = d->sec_h; aa.sec_w = d->sec_w;
    aa.q_rot_out = b.q_rot;
    aa.batch = B; aa.bs_q = qkv_rows; aa.bs_cache = (long)Hkv * d->capacity * D;
    aa.out_img = b.ab; aa.done = b.attn_done;
    attn_ws(b.attn_ws, aa);
    aa.lse = aa.o_part + (size_t)B * Hq * splits * 128;
    if (fuse_qkv) {
      aa.wqkv = (const u16*)w.qkv; aa.wqkv_tiled = gu_tiled; aa.xb = b.xb; aa.in_ss = b.ss_x; aa.in_parts = xparts;
      aa.in_scale = b.sc_x;
      aa.qkv_t = b.qkv_t; aa.hgen = b.qkv_ctl; aa.hdone = b.qkv_ctl + 1; aa.status = b.control;
      aa.spin_limit = g_spin_limit.load();
      if ((st = qd::attention_qkv8_launch(aa, s))) return st;
    } else if ((st = qd::attention_partial_launch<float>(aa, s))) {
      return st;
    }
    // r = x + W_o attn; image of r * post_norm * rstd(x)
    qd::Gemv8Args go;
    base(go, H, (long)Hq * D);
    go.xb = b.ab; go.W = (const u16*)w.o_proj; go.residual = b.x; go.ldr = H; go.y = b.r; go.ldy = H;
    go.w_tiled = gu_tiled;
    go.yb = b.rb; go.yb_gamma = (const u16*)w.post_norm; go.pre_ss = b.ss_x; go.pre_parts = xparts;
    go.out_scale = b.sc_r; go.yss = b.ss_r;
    if ((st = qd::gemv8_launch(go, qd::EPI_STORE, s))) return st;
    qd::Gemv8Args gu;
    base(gu, I, H, true);
    gu.xb = b.rb; gu.in_ss = b.ss_r; gu.in_parts = r_parts; gu.in_scale = b.sc_r; gu.W = (const u16*)w.gate_up;
    gu.up_offset = I; gu.yb = b.hb; gu.w_tiled = gu_tiled;
    if ((st = qd::gemv8_launch(gu, qd::EPI_SILU, s))) return st;
    // x = r + W_down hidden; image of x * (next input_norm | final_norm) * rstd(r)
    const u16* next_gamma =
        (const u16*)(li + 1 < d->num_layers ? d->layers[li + 1].input_norm : d->final_norm);
    qd::Gemv8Args gd;
    base(gd, H, I);
    gd.xb = b.hb; gd.W = (const u16*)w.down; gd.residual = b.r; gd.ldr = H; gd.y = b.x; gd.ldy = H;
    gd.yb = b.xb; gd.yb_gamma = next_gamma; gd.pre_ss = b.ss_r; gd.pre_parts = r_parts; gd.out_scale = b.sc_x;
    gd.yss = b.ss_x; gd.w_tiled = gu_tiled;
    if ((st = qd::gemv8_launch(gd, qd::EPI_STORE, s))) return st;
  }
  // final RMSNorm (applied through the image of x), tied lm_head, per-sequence argmax
  qd::Gemv8Args gl;
  base(gl, d->vocab, H);
  gl.ksplit = 1;
  gl.rows_per_group = 16;
  gl.xb = b.xb; gl.in_ss = b.ss_x; gl.in_parts = x_parts; gl.in_scale = b.sc_x; gl.W = (const u16*)d->embed;
  gl.y = reinterpret_cast<float*>(d->logits_out); gl.ldy = d->vocab; gl.part_val = b.part_val;
  gl.part_idx = b.part_idx;
  const int groups = qd::gemv8_row_groups(d->vocab);
  gl.grid = std::min(groups, qd_host::cu_count());   // one looping workgroup per CU (two buffers of weights in flight)
  // the last workgroup reduces the per-sequence argmax (arrival counter: the
  // header of the batch-1 argmax workspace, which a batch step does not use)
  gl.argmax_count = reinterpret_cast<unsigned*>(b.argmax_ws);
  gl.token = d->token;
  if (d->advance_counter != nullptr) {
    gl.adv_out = d->advance_out_tokens;
    gl.adv_counter = d->advance_counter;
    gl.adv_cache_position = const_cast<int64_t*>(d->cache_position);
    gl.adv_rope_position = const_cast<int64_t*>(d->rope_position);
    gl.adv_max_tokens = d->advance_max_tokens;
  }
  return qd::gemv8_launch(gl, qd::EPI_ARGMAX, s);
}

}  // namespace

static int step_phases(const qd_model_desc* d, int first_layer, int n_layers, unsigned phase_mask, bool advance,
                       void* stream);

int qd_decode_step(const qd_model_desc* d, void* stream) {
  QD_REQUIRE(d, QD_ERR_ARG, "null descriptor");
  const int mode = qd_decode_step_mode(d);
  if (mode < 0) return mode;
  if (batch_of(d) > 1) {
    int st = qd_decode_step_phases(d, 0, 0, 0, stream);  // descriptor checks only
    if (st) return st;
    return batch_step(d, S(stream));
  }
  if (mode == QD_STEP_CHAIN) return step_phases(d, 0, d->num_layers, QD_PHASE_ALL, true, stream);
  int st = qd_decode_step_phases(d, 0, 0, 0, stream);  // descriptor checks only
  if (st) return st;
  StepBuffers b;
  size_t total = 0;
  step_layout(d, splits_of(d), &b, &total);
  if ((st = launch_persistent(d, b, S(stream)))) return st;
  return step_phases(d, 0, 0, QD_PHASE_LM_HEAD, true, stream);
}

int qd_decode_layers_persistent(const qd_model_desc* d, void* stream) {
  QD_REQUIRE(d, QD_ERR_ARG, "null descriptor");
  int st = qd_decode_step_phases(d, 0, 0, 0, stream);
  if (st) return st;
  char why[256];
  QD_REQUIRE(!persistent_unsupported(d, why, sizeof(why)), QD_ERR_SHAPE, "%s", why);
  StepBuffers b;
  size_t total = 0;
  step_layout(d, splits_of(d), &b, &total);
  return launch_persistent(d, b, S(stream));
}

int qd_persistent_prepare(void* stream) {
  char why[256];
  QD_REQUIRE(!persistent_device_unsupported(why, sizeof(why)), QD_ERR_SHAPE, "%s", why);
  unsigned *t = nullptr, *ctrl = nullptr;
  return persist_area(S(stream), &t, &ctrl);
}

static int decoder_layers_persistent(const void* hidden_in, const qd_layer_weights* layers, int n_layers,
                                     int capacity, const int64_t* cache_position, const void* cos, const void* sin,
                                     float eps, float scale, void* hidden_out, int64_t* const* length_out,
                                     unsigned* status, void* stream) {
  QD_REQUIRE(hidden_in && layers && cache_position && cos && sin && hidden_out && status, QD_ERR_ARG,
             "null pointer");
  QD_REQUIRE(n_layers >= 1 && n_layers <= qd::kPersistMaxLayers, QD_ERR_SHAPE, "layer count %d outside 1..%d",
             n_layers, qd::kPersistMaxLayers);
  QD_REQUIRE(capacity >= 1, QD_ERR_SHAPE, "cache capacity %d", capacity);
  // what the kernel reads or writes as vectors: 16-byte weight, norm and cache
  // rows, the 8-byte input slice of each thread, the int64 position words
  for (int l = 0; l < n_layers; ++l) {
    const qd_layer_weights* w = layers + l;
    QD_REQUIRE(w->qkv && w->o_proj && w->gate_up && w->down && w->input_norm && w->post_norm && w->q_norm &&
                   w->k_norm && w->k_cache && w->v_cache,
               QD_ERR_ARG, "null layer weight or cache pointer (layer %d)", l);
    QD_REQUIRE(a16(w->qkv) && a16(w->o_proj) && a16(w->gate_up) && a16(w->down) && a16(w->input_norm) &&
                   a16(w->post_norm) && a16(w->k_cache) && a16(w->v_cache),
               QD_ERR_ARG, "weights, norms and caches must be 16-byte aligned (layer %d)", l);
    QD_REQUIRE(aligned(w->q_norm, 2) && aligned(w->k_norm, 2), QD_ERR_ARG, "q/k norm weights not 2-byte aligned");
    QD_REQUIRE(!length_out || !length_out[l] || aligned(length_out[l], 8), QD_ERR_ARG,
               "length_out must be 8-byte aligned (layer %d)", l);
  }
  QD_REQUIRE(aligned(hidden_in, 8) && aligned(cache_position, 8) && aligned(status, 4) && aligned(hidden_out, 2) &&
                 aligned(cos, 2) && aligned(sin, 2),
             QD_ERR_ARG, "hidden_in, cache_position and length_out must be 8-byte aligned (fp16 vectors 2-byte)");
  char why[256];
  QD_REQUIRE(!persistent_device_unsupported(why, sizeof(why)), QD_ERR_SHAPE, "%s", why);
  qd::PersistArgs p;
  memset(&p, 0, sizeof(p));
  for (int l = 0; l < n_layers; ++l) {
    const qd_layer_weights* w = layers + l;
    p.layers[l] = qd::PersistLayer{(const u16*)w->qkv,        (const u16*)w->o_proj,    (const u16*)w->gate_up,
                                   (const u16*)w->down,       (const u16*)w->input_norm, (const u16*)w->post_norm,
                                   (const u16*)w->q_norm,     (const u16*)w->k_norm,    (u16*)w->k_cache,
                                   (u16*)w->v_cache,          length_out ? length_out[l] : nullptr};
  }
  p.num_layers = n_layers;
  p.T = capacity;
  p.eps = eps;
  p.scale = scale;
  p.cache_position = cache_position;
  p.x_in = (const u16*)hidden_in;
  p.rope_cos = (const u16*)cos;
  p.rope_sin = (const u16*)sin;
  p.x_out16 = (u16*)hidden_out;
  unsigned *t = nullptr, *ctrl = nullptr;
  int st = persist_area(S(stream), &t, &ctrl);
  if (st) return st;
  set_handoff_words(p, t);
  p.status = status;
  p.generation = ctrl;
  p.done = ctrl + 1;
  p.spin_limit = g_spin_limit.load();
  return qd::decode_persistent_layer_launch(p, S(stream));
}

int qd_decoder_layer_persistent_f16(const void* hidden_in, const qd_layer_weights* w, int capacity,
                                    const int64_t* cache_position, const void* cos, const void* sin, float eps,
                                    float scale, void* hidden_out, int64_t* length_out, unsigned* status,
                                    void* stream) {
  QD_REQUIRE(w, QD_ERR_ARG, "null pointer");
  int64_t* lengths[1] = {length_out};
  return decoder_layers_persistent(hidden_in, w, 1, capacity, cache_position, cos, sin, eps, scale, hidden_out,
                                   lengths, status, stream);
}

int qd_decoder_layers_persistent_f16(const void* hidden_in, const qd_layer_weights* layers, int n_layers,
                                     int capacity, const int64_t* cache_position, const void* cos, const void* sin,
                                     float eps, float scale, void* hidden_out, int64_t* const* length_out,
                                     unsigned* status, void* stream) {
  return decoder_layers_persistent(hidden_in, layers, n_layers, capacity, cache_position, cos, sin, eps, scale,
                                   hidden_out, length_out, status, stream);
}

int qd_persistent_set_spin_limit(unsigned polls) {
  g_spin_limit.store(polls);
  return QD_OK;
}

int qd_decode_status(const qd_model_desc* d, unsigned* status, int reset) {
  QD_REQUIRE(d && d->workspace && status, QD_ERR_ARG, "null pointer");
  StepBuffers b;
  size_t total = 0;
  step_layout(d, splits_of(d), &b, &total);
  hipError_t e = hipMemcpy(status, b.control, sizeof(unsigned), hipMemcpyDeviceToHost);
  if (e == hipSuccess && reset) {
    const unsigned zero = 0;
    e = hipMemcpy(b.control, &zero, sizeof(unsigned), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    qd_host::set_error("status read failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return QD_OK;
}

// The kernel chain of a batch-1 step (the phases in phase_mask); `advance`:
// the lm_head's last workgroup also performs the descriptor's end-of-step
// advance (qd_decode_step only, never for phase-wise runs).
static int step_phases(const qd_model_desc* d, int first_layer, int n_layers, unsigned phase_mask, bool advance,
                       void* stream) {
  QD_REQUIRE(d && d->layers && d->embed && d->final_norm && d->token && d->cache_position && d->rope_position &&
                 d->inv_freq && d->workspace,
             QD_ERR_ARG, "incomplete model descriptor");
  QD_REQUIRE(d->head_dim == 128 && d->hidden % 512 == 0 && d->intermediate % 512 == 0 &&
                 d->num_heads % d->num_kv_heads == 0 && d->num_heads * d->head_dim % 512 == 0,
             QD_ERR_SHAPE, "unsupported model shape");
  QD_REQUIRE(first_layer >= 0 && n_layers >= 0 && first_layer + n_layers <= d->num_layers, QD_ERR_ARG,
             "layer range [%d, %d) outside the model", first_layer, first_layer + n_layers);
  QD_REQUIRE(d->batch >= 0 && d->batch <= qd::kBatchMax, QD_ERR_SHAPE, "batch %d outside 0..%d", d->batch,
             qd::kBatchMax);
  QD_REQUIRE(batch_of(d) == 1 || (n_layers == 0 && phase_mask == 0), QD_ERR_ARG,
             "phase-wise execution is batch 1 only (batch %d)", d->batch);
  hipStream_t s = S(stream);
  const int splits = splits_of(d);
  StepBuffers b;
  size_t total = 0;
  step_layout(d, splits, &b, &total);
  const int H = d->hidden, D = d->head_dim, Hq = d->num_heads, Hkv = d->num_kv_heads, I = d->intermediate;
  const long qs = (long)Hq * D, kvs = (long)Hkv * D;
  int st = QD_OK;
  if (phase_mask & QD_PHASE_EMBED) {
    if ((st = qd::embed_gather_launch((const u16*)d->embed, d->token, b.x, H, d->vocab, s))) return st;
  }
  for (int li = first_layer; li < first_layer + n_layers; ++li) {
    const qd_layer_weights& w = d->layers[li];
    // 1. input RMSNorm + fused QKV GEMV
    GemvArgs g1;
    g1.x = b.x; g1.gamma = (const u16*)w.input_norm; g1.W = (const u16*)w.qkv; g1.y = b.qkv;
    g1.N = qs + 2 * kvs; g1.K = H; g1.ldw = H; g1.eps = d->eps;
    if ((phase_mask & QD_PHASE_QKV) && (st = qd::gemv_store<qd::PRO_RMSNORM, float, float>(g1, s))) return st;
    // 2. split-KV attention partials with the q/k head RMSNorm + M-RoPE and the
    //    K/V write of the new token fused into the prologue
    qd::AttnArgs aa;
    aa.k = (const u16*)w.k_cache; aa.v = (const u16*)w.v_cache; aa.k_w = (u16*)w.k_cache; aa.v_w = (u16*)w.v_cache;
    aa.stride_h = (long)d->capacity * D; aa.stride_s = D; aa.T = d->capacity; aa.cache_position = d->cache_position;
    aa.scale = 1.0f / sqrtf((float)D); aa.Hq = Hq; aa.Hkv = Hkv; aa.n_split = splits; aa.out = b.attn;
    aa.qkv = b.qkv; aa.q_weight = (const u16*)w.q_norm; aa.k_weight = (const u16*)w.k_norm; aa.eps = d->eps;
    aa.rope_pos = d->rope_position; aa.inv_freq = d->inv_freq; aa.sec_h = d->sec_h; aa.sec_w = d->sec_w;
    aa.q_rot_out = b.q_rot;
    attn_ws(b.attn_ws, aa);
    // 3. merge of the splits -> attention output [Hq*D]: with both phases and
    //    at most 16 splits in the partial kernel (the last split of each kv
    //    head merges; arrival counters in the workspace header), else the merge
    //    kernel (one phase on its own, e.g. when timing the phases)
    const unsigned attn_both = QD_PHASE_ATTN | QD_PHASE_ATTN_MERGE;
    if ((phase_mask & attn_both) == attn_both && splits <= 16 && Hkv <= 64) {
      aa.done = reinterpret_cast<unsigned*>(b.attn_ws);
      if ((st = qd::attention_partial_launch<float>(aa, s))) return st;
    } else {
      if ((phase_mask & QD_PHASE_ATTN) && (st = qd::attention_partial_launch<float>(aa, s))) return st;
      if ((phase_mask & QD_PHASE_ATTN_MERGE) && (st = qd::attention_merge_launch<float>(aa, s))) return st;
    }
    // 4. o_proj + residual: r = x + W_o attn
    GemvArgs g4;
    g4.x = b.attn; g4.W = (const u16*)w.o_proj; g4.residual = b.x; g4.y = b.r; g4.N = H; g4.K = qs; g4.ldw = qs;
    if ((phase_mask & QD_PHASE_O_PROJ) && (st = qd::gemv_store<qd::PRO_PLAIN, float, float>(g4, s))) return st;
    // 5. post-attn RMSNorm + gate_up + SiLU*up
    GemvArgs g5;
    g5.x = b.r; g5.gamma = (const u16*)w.post_norm; g5.W = (const u16*)w.gate_up; g5.y = b.hidden;
    g5.N = I; g5.K = H; g5.ldw = H; g5.up_offset = I; g5.eps = d->eps;
    if ((phase_mask & QD_PHASE_GATE_UP) && (st = qd::gemv_silu<qd::PRO_RMSNORM, float, float>(g5, s))) return st;
    // 6. down_proj + residual: x = r + W_d hidden
    GemvArgs g6;
    g6.x = b.hidden; g6.W = (const u16*)w.down; g6.residual = b.r; g6.y = b.x; g6.N = H; g6.K = I; g6.ldw = I;
    if ((phase_mask & QD_PHASE_DOWN) && (st = qd::gemv_store<qd::PRO_PLAIN, float, float>(g6, s))) return st;
  }
  // final RMSNorm + tied lm_head + argmax -> token
  GemvArgs gl;
  gl.x = b.x; gl.gamma = (const u16*)d->final_norm; gl.eps = d->eps; gl.W = (const u16*)d->embed;
  gl.N = d->vocab; gl.K = H; gl.ldw = H; gl.y = d->logits_out; gl.token = d->token;
  gl.argmax_f16 = d->argmax_f16_logits != 0;
  argmax_ws(b.argmax_ws, gl);
  if (advance && d->advance_counter != nullptr) {
    gl.adv_out = d->advance_out_tokens; gl.adv_counter = d->advance_counter;
    gl.adv_cache_position = const_cast<int64_t*>(d->cache_position);
    gl.adv_rope_position = const_cast<int64_t*>(d->rope_position); gl.adv_max_tokens = d->advance_max_tokens;
  }
  if (phase_mask & QD_PHASE_LM_HEAD) return qd::gemv_argmax<qd::PRO_RMSNORM, float, u16>(gl, s);
  return QD_OK;
}

int qd_decode_step_phases(const qd_model_desc* d, int first_layer, int n_layers, unsigned phase_mask,
                          void* stream) {
  return step_phases(d, first_layer, n_layers, phase_mask, false, stream);
}

int qd_decode_advance(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                      int64_t* rope_position, int max_tokens, void* stream) {
  QD_REQUIRE(token && counter && cache_position && rope_position, QD_ERR_ARG, "null pointer");
  return qd::decode_advance_launch(token, out_tokens, counter, cache_position, rope_position, max_tokens,
                                   S(stream));
}

int qd_decode_advance_batch(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                            int64_t* rope_position, int max_tokens, int batch, void* stream) {
  QD_REQUIRE(token && counter && cache_position && rope_position, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(batch >= 1 && batch <= qd::kBatchMax, QD_ERR_SHAPE, "batch %d outside 1..%d", batch, qd::kBatchMax);
  return qd::advance8_launch(token, out_tokens, counter, cache_position, rope_position, max_tokens, batch,
                             S(stream));
}

int qd_batch_tile_rows(long rows, long K, int silu) {
  if (rows <= 0 || K <= 0) return 0;
  return batch_split(rows, K, silu != 0).rows_per_group;
}

size_t qd_batch_gemv_workspace_bytes(long N, long K) {
  if (N <= 0 || K <= 0) return 0;
  // image [K][16] fp16, ss + scale [2][8], K-split partials [N/16][<= 6][<= 2][128], counters [N/16]
  return align256(32 * (size_t)K) + 256 + align256(4 * (size_t)qd::gemv8_row_groups(N) * kBatchMaxKsplit * 256) +
         align256(4 * (size_t)qd::gemv8_row_groups(N));
}

int qd_batch_gemv(const float* x, long ldx, const void* gamma, float eps, const void* W, long ldw, long N, long K,
                  long up_offset, const float* residual, long ldr, float* y, long ldy, int nseq, int epilogue,
                  void* workspace, size_t workspace_bytes, void* stream) {
  QD_REQUIRE(x && W && y && workspace, QD_ERR_ARG, "null pointer");
  QD_REQUIRE(nseq >= 1 && nseq <= qd::kBatchMax, QD_ERR_SHAPE, "nseq %d outside 1..%d", nseq, qd::kBatchMax);
  QD_REQUIRE(epilogue == QD_BATCH_EPI_STORE || epilogue == QD_BATCH_EPI_SILU, QD_ERR_ARG, "bad epilogue %d",
             epilogue);
  QD_REQUIRE((K == 2048 || K == 6144) && N % 16 == 0 && N > 0 && ldx % 4 == 0 && a16(x) && a16(W) && ldw % 8 == 0,
             QD_ERR_SHAPE, "need K in {2048, 6144}, N %% 16 == 0 and 16-byte aligned rows");
  QD_REQUIRE(epilogue != QD_BATCH_EPI_SILU || (up_offset == N && K == 2048), QD_ERR_SHAPE,
             "SiLU epilogue: up_offset must equal N and K must be 2048");
  QD_REQUIRE(a16(workspace) && workspace_bytes >= qd_batch_gemv_workspace_bytes(N, K), QD_ERR_ARG,
             "workspace needs %zu bytes (16-byte aligned)", qd_batch_gemv_workspace_bytes(N, K));
  char* ws = reinterpret_cast<char*>(workspace);
  u16* img = reinterpret_cast<u16*>(ws);
  float* ss = reinterpret_cast<float*>(ws + align256(32 * (size_t)K));
  float* scale = ss + qd::kBatchMax;
  float* kpart = reinterpret_cast<float*>(ws + align256(32 * (size_t)K) + 256);
  unsigned* kcount = reinterpret_cast<unsigned*>(
      ws + align256(32 * (size_t)K) + 256 + align256(4 * (size_t)qd::gemv8_row_groups(N) * kBatchMaxKsplit * 256));
  int st = qd::bimage8_launch(x, ldx, (const u16*)gamma, gamma != nullptr, eps, (int)K, nseq, img, ss, scale,
                              S(stream));
  if (st) return st;
  qd::Gemv8Args g;
  g.xb = img; g.in_ss = gamma != nullptr ? ss : nullptr; g.in_parts = 1; g.in_scale = scale; g.eps = eps;
  g.W = (const u16*)W; g.ldw = ldw; g.N = N; g.K = K; g.residual = residual; g.ldr = ldr; g.y = y; g.ldy = ldy;
  g.nseq = nseq; g.kpart = kpart; g.kcount = kcount;
  const BatchSplit sp = batch_split(N, K, epilogue == QD_BATCH_EPI_SILU);
  g.ksplit = sp.ksplit;
  g.rows_per_group = sp.rows_per_group;
  if (epilogue == QD_BATCH_EPI_SILU) {
    g.up_offset = up_offset;
    return qd::gemv8_launch(g, qd::EPI_SILU, S(stream));
  }
  return qd::gemv8_launch(g, qd::EPI_STORE, S(stream));
}

}  // extern "C"
