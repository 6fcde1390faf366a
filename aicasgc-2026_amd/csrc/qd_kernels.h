// Internal (C++) launch interface shared by the kernel translation units and
// the C-ABI layer.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qd {

// PRO_SILU: x[k] = silu(x[k]) * x2[k] (x2 = the 'up' half of a gate_up vector).
enum GemvPrologue { PRO_PLAIN = 0, PRO_RMSNORM = 1, PRO_ADD_RMSNORM = 2, PRO_SILU = 3 };
enum GemvEpilogue { EPI_STORE = 0, EPI_SILU = 1, EPI_ARGMAX = 2, EPI_PARTIAL = 3 };

constexpr int kMaxArgmaxBlocks = 4096;

struct GemvArgs {
  const void* x = nullptr;         // activation [K] (TX)
  const void* x2 = nullptr;        // PRO_ADD_RMSNORM second addend [K] (TX)
  const uint16_t* gamma = nullptr; // RMSNorm weight [K] fp16
  const uint16_t* W = nullptr;     // fp16 [rows, ldw]
  const void* bias = nullptr;      // [N] (TY) or null
  const void* residual = nullptr;  // [N] (TY) added after the dot, or null
  void* y = nullptr;               // output [N] (TY); EPI_ARGMAX: optional logits
  void* r_out = nullptr;           // PRO_ADD_RMSNORM: pre-norm sum [K] (TY) or null
  long N = 0;                      // outputs (EPI_SILU: gate rows == up rows == N)
  long K = 0;
  long ldw = 0;
  long up_offset = 0;              // EPI_SILU: row offset of the up half
  float eps = 1e-6f;
  float* part_val = nullptr;       // EPI_ARGMAX per-block max / EPI_PARTIAL [splits, N]
  long* part_idx = nullptr;        // EPI_ARGMAX per-block argmax
  unsigned* argmax_count = nullptr; // EPI_ARGMAX (required): arrival counter, zeroed once and
                                    // self-resetting; the last block to arrive reduces the partials
  int64_t* token = nullptr;        // EPI_ARGMAX result
  // EPI_ARGMAX: the argmax reduction also advances the decode state
  // (qd_decode_advance semantics) when adv_counter is set
  int64_t* adv_out = nullptr;
  int64_t* adv_counter = nullptr;
  int64_t* adv_cache_position = nullptr;
  int64_t* adv_rope_position = nullptr;
  int adv_max_tokens = 0;
  // EPI_ARGMAX: compare the logits rounded to fp16 (the reference's fp16
  // logits + torch.argmax: among logits equal in fp16 the first index wins)
  // instead of the fp32 accumulators
  int argmax_f16 = 0;
  // EPI_STORE: one thread also writes next_dst[0] = next_src[0] + 1 (a decoder
  // layer's last kernel advancing its cache's running length); null = none
  const int64_t* next_src = nullptr;
  int64_t* next_dst = nullptr;
};

template <int PRO, typename TX, typename TY>
int gemv_store(const GemvArgs& a, hipStream_t s);
template <int PRO, typename TX, typename TY>
int gemv_silu(const GemvArgs& a, hipStream_t s);
template <int PRO, typename TX, typename TY>
int gemv_argmax(const GemvArgs& a, hipStream_t s);
template <typename TX, typename TY>
int gemv_splitk(const GemvArgs& a, int splits, hipStream_t s);

// ---------------------------------------------------------------- attention

struct AttnArgs {
  const void* q = nullptr;         // [Hq, 128] rows of stride q_stride (TQ), already rotated
  long q_stride = 128;
  const uint16_t* k = nullptr;     // fp16 cache [Hkv, T, 128]
  const uint16_t* v = nullptr;
  long stride_h = 0, stride_s = 128;
  int T = 0;
  const int64_t* cache_position = nullptr;
  float scale = 0.f;
  int Hq = 16, Hkv = 8, n_split = 1;
  float* o_part = nullptr;         // [Hq, n_split, 128]
  float* lse = nullptr;            // [Hq, n_split]
  void* out = nullptr;             // [Hq, 128] (TO), merge kernel
  // fused prologue (native step): raw qkv [Hq*D + 2*Hkv*D] (TQ) instead of q
  const void* qkv = nullptr;
  const uint16_t* q_weight = nullptr;
  const uint16_t* k_weight = nullptr;
  float eps = 1e-6f;
  const int64_t* rope_pos = nullptr;  // int64 [3]
  const float* inv_freq = nullptr;    // fp32 [64]
  // instead of rope_pos / inv_freq: the rotation's cos / sin (fp16 [batch][128],
  // slot j at j; the caller's rotary embedding, e.g. transformers')
  const uint16_t* cos = nullptr;
  const uint16_t* sin = nullptr;
  int sec_h = 20, sec_w = 20;
  uint16_t* k_w = nullptr;            // writable aliases of k / v for the new row
  uint16_t* v_w = nullptr;
  float* q_rot_out = nullptr;         // optional fp32 [Hq, 128] copy of the rotated q
  // batch (grid y = sequence): per-sequence element strides of q / qkv, of the
  // caches, of o_part / lse / out / q_rot_out; cache_position[b], rope_pos[3b..]
  int batch = 1;
  long bs_q = 0, bs_cache = 0;
  uint16_t* out_img = nullptr;        // merge: batch operand image of the output (instead of out)
  unsigned* done = nullptr;           // [batch][Hkv] arrival counters: the last split of a kv head
                                      // merges in the partial kernel (no merge launch), or null
  // batch step with the qkv GEMV in the same launch (attention_qkv8_launch):
  // the first kQkv8Producers workgroups compute 16 rows of
  // qkv[b] = rstd_b / in_scale[b] * (W_qkv . image(x)[b]) each and hand them
  // to every workgroup through parity-tagged words in the uncached hand-off
  // area (qkv_t [kBatchMax][rows]); `qkv` is then unused
  const uint16_t* wqkv = nullptr;     // fp16 [rows][2048], or in tile order (wqkv_tiled)
  int wqkv_tiled = 0;                 // wqkv in the batch GEMVs' tile order for 16-row groups
  const uint16_t* xb = nullptr;       // operand image of x [2048/32][64][8]
  const float* in_ss = nullptr;       // [in_parts][8] partial sums of squares of x
  int in_parts = 0;
  const float* in_scale = nullptr;    // [8] scale of the image
  unsigned* qkv_t = nullptr;
  unsigned* hgen = nullptr;           // launches so far (the words' parity), advanced by the last workgroup
  unsigned* hdone = nullptr;          // workgroups finished in this launch (self-resetting)
  unsigned* status = nullptr;         // bit 0: a hand-off wait ran out of its polling budget
  unsigned spin_limit = 0;            // polls per thread and launch (0: the default)
};

// Partials of every (kv head, split); fused prologue when a.qkv != nullptr.
template <typename TQ>
int attention_partial_launch(const AttnArgs& a, hipStream_t s);
template <typename TO>
int attention_merge_launch(const AttnArgs& a, hipStream_t s);
// Batch step: the qkv GEMV and the fused attention (q/k norm + RoPE + K/V
// write + split-KV + merge into out_img) in one launch of batch * Hkv * n_split
// workgroups, the first kQkv8Producers of which produce the qkv rows (the
// launch needs them resident together: one per CU on 256 CUs).  Hq = 2 Hkv,
// head dim 128, qkv rows = kQkv8Producers * 16, K = 2048, a.done set.
constexpr int kQkv8Producers = 256;
int attention_qkv8_launch(const AttnArgs& a, hipStream_t s);
// True when the current device keeps kQkv8Producers workgroups of that launch
// resident at once (queried once per device).
bool attention_qkv8_device_ok();

// ---------------------------------------------------------------- small ops

struct RopeArgs {
  const void* q = nullptr;
  const void* k = nullptr;
  const void* v = nullptr;
  long q_stride = 128, k_stride = 128, v_stride = 128;   // per head (elements)
  long q_row = 0, k_row = 0;                              // per token row (qk-norm op)
  const uint16_t* q_weight = nullptr;
  const uint16_t* k_weight = nullptr;
  float eps = 1e-6f;
  const uint16_t* cos = nullptr;   // fp16 [M, 128] or null
  const uint16_t* sin = nullptr;
  long cs_row = 128;
  const int64_t* rope_pos = nullptr;  // int64 [3]
  const float* inv_freq = nullptr;    // fp32 [64]
  int sec_h = 20, sec_w = 20;
  void* q_out = nullptr;           // [M, Hq, 128]
  void* k_out = nullptr;           // [M, Hkv, 128] (qk-norm op) or null
  uint16_t* k_cache = nullptr;     // cache-write op
  uint16_t* v_cache = nullptr;
  long cache_stride_h = 0, cache_stride_s = 128;
  int T = 0;
  const int64_t* cache_position = nullptr;
  int Hq = 16, Hkv = 8, M = 1;
};

template <typename TI, typename TO>
int q_rope_kv_launch(const RopeArgs& a, hipStream_t s);
int qk_norm_rope_f16_launch(const RopeArgs& a, hipStream_t s);

int add_rmsnorm_f16_launch(const uint16_t* res, const uint16_t* x, const uint16_t* w, uint16_t* out_sum,
                           uint16_t* out_norm, int rows, int cols, float eps, hipStream_t s);
int silu_mul_f16_launch(const uint16_t* g, const uint16_t* u, uint16_t* out, long n, hipStream_t s);
int add_f16_launch(const uint16_t* a, const uint16_t* b, uint16_t* out, long n, hipStream_t s);
int embed_gather_launch(const uint16_t* table, const int64_t* token, float* out, int H, long V, hipStream_t s);
int decode_advance_launch(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                          int64_t* rope_position, int max_tokens, hipStream_t s);

// ---------------------------------------------------------------- persistent step

constexpr int kPersistMaxLayers = 32;

struct PersistLayer {
  const uint16_t* qkv;
  const uint16_t* o_proj;
  const uint16_t* gate_up;
  const uint16_t* down;
  const uint16_t* input_norm;
  const uint16_t* post_norm;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t* length_out;            // LAYER instance: the cache's running length, set to
                                  // cache_position + 1 after the launch (nullable)
};

// Everything one persistent launch reads: passed by value, so the layer
// table travels in the kernel arguments (no device copy of it is needed).
struct PersistArgs {
  PersistLayer layers[kPersistMaxLayers];
  int num_layers;
  int T;                          // cache rows per layer
  long vocab;
  float eps, scale;
  int sec_h, sec_w;
  const uint16_t* embed;          // fp16 [V, H]
  const int64_t* token;           // int64 [1]
  const int64_t* cache_position;  // int64 [1]
  const int64_t* rope_position;   // int64 [3]
  const float* inv_freq;          // fp32 [64]
  // hand-off buffers (the per-device uncached hand-off area): fp32 words
  // whose mantissa LSB carries the write parity
  unsigned* x_t;                  // [H]
  unsigned* qkv_t;                // [Hq*D + 2*Hkv*D]
  unsigned* opart_t;              // [Hq, splits, D]
  unsigned* lse_t;                // [Hq, splits]
  unsigned* att_t;                // [Hq*D]
  unsigned* r_t;                  // [H]
  unsigned* hid_t;                // [I]
  float* x_out;                   // fp32 [H]: last layer's output (lm_head input)
  unsigned* status;               // bit 0: a hand-off wait ran out of its spin budget
  // per-device state shared by every persistent launch on the device, like the
  // hand-off words: the layer generation (layers run so far; the words' write
  // parity follows it) and the workgroups finished in this launch (self-resetting)
  unsigned* generation;
  unsigned* done;
  // drop-in decoder layers (the kernel's LAYER instance, one or more layers
  // of the swapped model): the first layer's input instead of the embedding
  // row, transformers' cos / sin instead of the M-RoPE positions, every
  // layer's output in fp16 (the next layer reads that fp16 value, as it would
  // from a launch of its own), and each cache's running length set to
  // cache_position + 1 after the launch
  const uint16_t* x_in;           // fp16 [H]
  const uint16_t* rope_cos;       // fp16 [D] (two equal halves)
  const uint16_t* rope_sin;       // fp16 [D]
  uint16_t* x_out16;              // fp16 [num_layers][H]
  unsigned spin_limit;            // polls per thread and launch before a wait gives up (0: the default)
};

// Model shape the persistent kernel is specialised for, and its grid.
constexpr int kPersistHidden = 2048, kPersistHeads = 16, kPersistKvHeads = 8, kPersistHeadDim = 128,
              kPersistInter = 6144, kPersistBlocks = 256, kPersistSplits = kPersistBlocks / kPersistKvHeads;
constexpr size_t kPersistTaggedWords = kPersistHidden                                              // x
                                       + (size_t)(kPersistHeads + 2 * kPersistKvHeads) * kPersistHeadDim  // qkv
                                       + (size_t)kPersistHeads * kPersistSplits * kPersistHeadDim    // o_part
                                       + (size_t)kPersistHeads * kPersistSplits                      // lse
                                       + (size_t)kPersistHeads * kPersistHeadDim                     // att
                                       + kPersistHidden + kPersistInter;                              // r, hid

int decode_persistent_launch(const PersistArgs& a, hipStream_t s);
// The same kernel's one-layer instance for the drop-in decoder layer (x_in,
// rope_cos / rope_sin, x_out16 and length_out set; num_layers 1).
int decode_persistent_layer_launch(const PersistArgs& a, hipStream_t s);

// ---------------------------------------------------------------- batch step

constexpr int kBatchMax = 8;
constexpr int kBatchMaxKsplit = 6;   // K ranges of one batch-GEMV row group

// Batch GEMV on MFMA: y[b][r] = f[b] * (W[r] . u[b]) for b < nseq, where u is
// the input's operand image (u = x * gamma * s, written by the producer with
// scale s = in_scale[b]) and f = rstd(in_ss) / s (1 / s without in_ss), so
// y = W . (RMSNorm(x) * gamma).  K in {2048, 6144}; rows a multiple of rows_per_group.
// The epilogue adds the residual (EPI_STORE) or forms silu(gate) * up
// (EPI_SILU), stores y, and writes the output's own operand image (times
// yb_gamma and out scale rstd(pre_ss), stored to out_scale) with per-row-group
// partial sums of y^2 (yss).
struct Gemv8Args {
  const uint16_t* xb = nullptr;    // input operand image [K/32][64][8] fp16
  const float* in_ss = nullptr;    // [in_parts][8] partial sums of squares of x, or null (no RMSNorm)
  int in_parts = 0;
  const float* in_scale = nullptr; // [8] scale of the input image, or null (1)
  float eps = 1e-6f;
  const uint16_t* W = nullptr;     // fp16 [rows][ldw], or in tile order (w_tiled)
  long ldw = 0;
  int w_tiled = 0;                 // W in MFMA tile order (gemv8_tile_order; not EPI_ARGMAX)
  long N = 0;                      // output rows (EPI_SILU: gate rows == up rows == up_offset)
  long K = 0;
  long up_offset = 0;
  const float* residual = nullptr; // fp32 [nseq][ldr] added in EPI_STORE, or null
  long ldr = 0;
  float* y = nullptr;              // fp32 [nseq][ldy] or null (EPI_ARGMAX: optional logits)
  long ldy = 0;
  uint16_t* yb = nullptr;          // output operand image [N/32][64][8], or null
  const uint16_t* yb_gamma = nullptr;
  const float* pre_ss = nullptr;   // [pre_parts][8]: output image scale rstd over N, or null (1)
  int pre_parts = 0;
  float* out_scale = nullptr;      // [8] the output image's scale, or null
  float* yss = nullptr;            // [N/rows][8] partial sums of squares of y, or null
  int nseq = 0;
  int rows_per_group = 16;         // 16 or 8 (not EPI_ARGMAX): rows of W per workgroup
  int ksplit = 1;                  // workgroups per row group along K (not EPI_ARGMAX)
  float* kpart = nullptr;          // ksplit > 1: [N/rows][ksplit][1 or 2 (EPI_SILU)][rows * 8] partials
  unsigned* kcount = nullptr;      // ksplit > 1: [N/rows] arrival counters (zero, self-resetting)
  int grid = 0;                    // EPI_ARGMAX: workgroups (each loops over row groups); 0: one per group
  float* part_val = nullptr;       // EPI_ARGMAX: [grid][8]
  long* part_idx = nullptr;
  // EPI_ARGMAX: the last workgroup to arrive (argmax_count: zeroed once,
  // self-resetting) reduces the partials to token[nseq] and, with adv_counter
  // set, advances the decode state as advance8_launch does
  unsigned* argmax_count = nullptr;
  int64_t* token = nullptr;
  int64_t* adv_out = nullptr;
  int64_t* adv_counter = nullptr;
  int64_t* adv_cache_position = nullptr;
  int64_t* adv_rope_position = nullptr;
  int adv_max_tokens = 0;
};

int gemv8_launch(const Gemv8Args& a, int epi, hipStream_t s);
int gemv8_row_groups(long N, int rows_per_group = 16);
// Image of u = x * gamma * s (gamma null: 1), s = rstd(x) when norm else 1,
// sum of squares of x as one partial ss[8], s to scale[8].
int bimage8_launch(const float* x, long ldx, const uint16_t* gamma, bool norm, float eps, int K, int nseq,
                   uint16_t* img, float* ss, float* scale, hipStream_t s);
// x[b] = embed[token[b]] and its image (gamma, scale rstd(x)), ss, scale.
int embed8_launch(const uint16_t* table, const int64_t* token, float* out, int H, long V, int nseq,
                  const uint16_t* gamma, float eps, uint16_t* img, float* ss, float* scale, hipStream_t s);
int advance8_launch(const int64_t* token, int64_t* out_tokens, int64_t* counter, int64_t* cache_position,
                    int64_t* rope_position, int max_tokens, int nseq, hipStream_t s);
// 0 when the device can keep the whole persistent grid resident at once.
int decode_persistent_check_device(char* why, size_t why_len);

}  // namespace qd
