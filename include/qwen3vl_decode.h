/*
 * qwen3vl_decode.h — C ABI of the MI355X (gfx950) batch-1 decode path for the
 * Qwen3-VL-2B text decoder.
 *
 * Every entry point:
 *   - takes raw device pointers, sizes, scalars and a hipStream_t (passed as
 *     void*; NULL = the null stream), never framework types;
 *   - only borrows the pointers for the duration of the (asynchronous) launch
 *     and allocates nothing on the hot path;
 *   - returns an int status: QD_OK, a negative QD_ERR_* for a rejected
 *     argument (nothing was launched), or a positive hipError_t from the
 *     launch; qd_last_error() returns a message for the last failure on the
 *     calling thread;
 *   - launches on the given stream, never synchronises, and is safe inside HIP
 *     stream capture (counters used for cross-workgroup hand-off are reset by
 *     the kernels themselves, and no memset nodes are issued).
 *
 * Activation dtype codes (QD_F16 / QD_F32) select the storage type of
 * activation vectors; weights and the KV cache are always fp16.  All
 * arithmetic is fp32 (fp16 products accumulated in fp32).
 *
 * Each function cites the reference interface it replaces
 * (/root/reference = wangxiyu191/AICASGC-2026).
 */
#ifndef QWEN3VL_DECODE_H
#define QWEN3VL_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QD_OK 0
#define QD_ERR_ARG (-1)          /* null pointer / bad scalar */
#define QD_ERR_SHAPE (-2)        /* unsupported or inconsistent size */
#define QD_ERR_WORKSPACE (-3)    /* workspace too small */

#define QD_F16 0
#define QD_F32 1

/* Library version and last error message on this thread ("" if none). */
int qd_version(void);
const char* qd_last_error(void);

/* Number of compute units of the current device (cached per device). */
int qd_device_cu_count(void);

/* ------------------------------------------------------------------ GEMV family */

/* y[N] = W[N,K] x[K] (+ bias[N]).  fp16 x/bias/y.  Replaces
 * nosplit_matvec_half (cuda_decode_gemv_ops/matvec.py:274-321 ->
 * decode_gemv_kernel_launchers.cuh:367-445). bias may be NULL.  K % 8 == 0. */
int qd_matvec_f16(const void* x, const void* W, const void* bias, void* y,
                  int N, int K, void* stream);

/* Split-K form of the same product: the K dimension is cut into split_k
 * slices, each writes fp32 partials to scratch[split_k * N], and a reduce pass
 * adds them in slice order (deterministic) + bias.  Replaces splitk_matvec
 * (cuda_decode_gemv_ops/matvec.py:10-51).  scratch needs split_k*N floats. */
int qd_splitk_matvec_f16(const void* x, const void* W, const void* bias,
                         float* scratch, void* y, int N, int K, int split_k,
                         void* stream);

/* y = W (rmsnorm(x) * gamma) (+ bias), rmsnorm over K with eps.  fp16 I/O.
 * Replaces fused_rmsnorm_qkv_half (cuda_decode_gemv_ops/fused.py:71-105 ->
 * decode_gemv_kernel_fused.cuh:99-185). */
int qd_rmsnorm_matvec_f16(const void* x, const void* gamma, const void* W,
                          const void* bias, void* y, int N, int K, float eps,
                          void* stream);

/* Post-attention MLP of one layer, fp16 I/O:
 *   r = residual + attn; xn = rmsnorm(r) * gamma;
 *   hidden[j] = silu(W_gu[j] xn) * W_gu[I + j] xn   (j < I);
 *   out = W_d hidden + r (+ bias).
 * W_gu is [2I, H], W_d is [H, I].  Replaces fused_post_attn_mlp_softsync_half
 * (cuda_decode_gemv_ops/fused.py:261-337 -> decode_gemv_kernel_fused.cuh:856-1076)
 * and fused_post_attn_mlp_persistent_half (fused.py:198-259).  bias may be NULL. */
int qd_post_attn_mlp_f16(const void* residual, const void* attn, const void* gamma,
                         const void* W_gu, const void* W_d, const void* bias,
                         void* hidden_out, void* out, int H, int I, float eps,
                         void* stream);

/* qd_post_attn_mlp_f16 that also sets next_position[0] = position[0] + 1
 * (int64 device words; they may be the same word) from its last kernel, after
 * every earlier launch of the layer has read the position.  For a decoder
 * layer that is the last user of its cache's write row: the swapped
 * OptimizedDecoderLayer advances its StaticLayer's cumulative_length this way,
 * as transformers' StaticLayer.update (cache_utils.py) does on the reference
 * path (OptimizedDecoderLayer.forward, optimized_layer.py:108-469, then the
 * cache update), without two extra launches per layer. */
int qd_post_attn_mlp_next_f16(const void* residual, const void* attn, const void* gamma,
                              const void* W_gu, const void* W_d, const void* bias,
                              void* hidden_out, void* out, int H, int I, float eps,
                              const int64_t* position, int64_t* next_position,
                              void* stream);

/* hidden = silu(W_gu[:I] x) * (W_gu[I:] x); out = W_d hidden (+ bias).  fp16
 * I/O, bias may be NULL.  Replaces fused_gateup_silu_downproj_half and its
 * persistent / softsync / gridsync / mega variants
 * (cuda_decode_gemv_ops/fused.py:148-197, :668-892). */
int qd_gateup_silu_down_f16(const void* x, const void* W_gu, const void* W_d,
                            const void* bias, void* hidden_out, void* out, int H, int I,
                            void* stream);

/* residual_out = residual + x; y = W (rmsnorm(residual_out) * gamma) (+ bias).
 * fp16 I/O, K % 512 == 0.  Replaces fused_add_rmsnorm_gateup_half
 * (cuda_decode_gemv_ops/fused.py:12-68). */
int qd_add_rmsnorm_matvec_f16(const void* residual, const void* x, const void* gamma,
                              const void* W, const void* bias, void* residual_out, void* y,
                              int N, int K, float eps, void* stream);

/* y = W (silu(gate_up[:K]) * gate_up[K:]) (+ bias).  fp16 I/O, K % 512 == 0.
 * Replaces fused_silu_downproj_half (cuda_decode_gemv_ops/fused.py:108-145). */
int qd_silu_matvec_f16(const void* gate_up, const void* W, const void* bias, void* y,
                       int N, int K, void* stream);

/* Tied lm_head with fused argmax:
 *   logits = W[V,H] (rmsnorm(h) * gamma)   (gamma == NULL: no norm)
 *   token  = first index of max(logits)      (fp32 logits, torch.argmax order)
 * h dtype h_dtype; logits_out (fp16, may be NULL); token_out int64[1].
 * partial: workspace of qd_lm_head_workspace_bytes(V) bytes; its counter is
 * self-resetting (zero it once at allocation).  The last workgroup to finish
 * reduces the partials in the same launch, so calls that share a workspace
 * must not overlap (order them on one stream).  Replaces FastLmHead.forward +
 * torch.argmax (evaluation_wrapper.py:1227-1238, :952). */
size_t qd_lm_head_workspace_bytes(int V);
int qd_lm_head_argmax(const void* h, int h_dtype, const void* gamma, float eps,
                      const void* W, int V, int H, void* logits_out,
                      int64_t* token_out, void* workspace, void* stream);

/* ------------------------------------------------------------------ small ops */

/* Per-head RMSNorm (head_dim 128) + rotate-half RoPE on q and k, K_rot and V
 * written into the static cache at row cache_position[0] (rows outside [0,T)
 * are not written).  qkv_dtype is the dtype of q/k/v; q_out has q_out_dtype.
 * q: [Hq,128] (row stride q_stride), k/v: [Hkv,128] (strides k_stride,
 * v_stride).  Caches fp16 [Hkv, T, 128] with head stride cache_stride_h and
 * row stride cache_stride_s (elements).
 * RoPE source: cos/sin fp16 [128] when non-NULL (the reference's form);
 * otherwise computed in fp32 from rope_pos[0..2] (int64 T/H/W positions, all
 * three read) + the fp32 inv_freq[64] table and the mrope section triple.
 * Replaces fused_q_rope_kv_cache_update (cuda_decode_small_ops.py:136-225 ->
 * decode_small_ops_kernel.cu:115-182). */
int qd_q_rope_kv_update(const void* q, const void* k, const void* v, int qkv_dtype,
                        long q_stride, long k_stride, long v_stride,
                        const void* q_weight, const void* k_weight, float eps,
                        const void* cos, const void* sin,
                        const int64_t* rope_pos, const float* inv_freq,
                        int sec_t, int sec_h, int sec_w,
                        void* q_out, int q_out_dtype,
                        void* k_cache, void* v_cache, long cache_stride_h,
                        long cache_stride_s, int T, const int64_t* cache_position,
                        int Hq, int Hkv, void* stream);

/* q/k per-head RMSNorm + RoPE without cache write, fp16 [M, H, 128] rows
 * (cos/sin fp16 [M, 128]).  Replaces fused_qk_rms_norm_rope
 * (cuda_decode_small_ops.py:70-133). */
int qd_qk_norm_rope_f16(const void* q, const void* k, const void* q_weight,
                        const void* k_weight, const void* cos, const void* sin,
                        void* q_out, void* k_out, int M, int Hq, int Hkv,
                        float eps, void* stream);

/* out_sum = residual + x; out_norm = rmsnorm(out_sum) * weight; rows x cols fp16.
 * Replaces fused_add_rms_norm (cuda_decode_small_ops.py:250-287). */
int qd_add_rmsnorm_f16(const void* residual, const void* x, const void* weight,
                       void* out_sum, void* out_norm, int rows, int cols,
                       float eps, void* stream);

/* out = rmsnorm(x) * weight; rows x cols fp16.  Replaces rms_norm
 * (cuda_decode_small_ops.py:290-317). */
int qd_rmsnorm_f16(const void* x, const void* weight, void* out, int rows, int cols,
                   float eps, void* stream);

/* out = silu(gate) * up, n fp16 elements.  Replaces fused_silu_mul
 * (cuda_decode_small_ops.py:228-247). */
int qd_silu_mul_f16(const void* gate, const void* up, void* out, long n, void* stream);

/* out = a + b, n fp16 elements.  Replaces add (cuda_decode_small_ops.py:320-339). */
int qd_add_f16(const void* a, const void* b, void* out, long n, void* stream);

/* ------------------------------------------------------------------ attention */

/* Split-KV GQA decode attention at batch 1, fused merge:
 *   L = min(cache_position[0] + 1, T); out[h] = softmax(q_h K[:L]^T * scale) V[:L]
 * for q head h on kv head h / (Hq/Hkv).  head_dim 128.  Each workgroup owns
 * one (kv head, split) and serves every q head of the group, so K/V is read
 * once.  Partials (normalised output + LSE) go to the workspace; the last
 * split of each kv head to finish merges them (an arrival counter per kv head
 * in the workspace, which resets itself; no workgroup waits on another).
 * When q_dtype != out_dtype, n_split > 16 or Hkv > 64 a second launch merges
 * instead (faster for many splits: it reads all partials in parallel).
 * q: [Hq,128] with row stride q_stride (q_dtype); caches fp16 with head
 * stride cache_stride_h and row stride cache_stride_s; out [Hq,128] out_dtype.
 * Workspace: qd_attention_workspace_bytes(Hq, Hkv, n_split) bytes, zeroed
 * once at allocation; calls that share a workspace must be ordered (one
 * stream), since its counters and partials are reused by every call.  Replaces decode_attn_v4_cta_qhead_splitkv_fused
 * (cuda_decode_attention.py:489-558 -> decode_attention_v4_kernel.cu:646-910)
 * and decode_attn_v4_fused (cuda_decode_attention.py:305-392). */
size_t qd_attention_workspace_bytes(int Hq, int Hkv, int n_split);
int qd_attention_decode(const void* q, int q_dtype, long q_stride,
                        const void* k_cache, const void* v_cache,
                        long cache_stride_h, long cache_stride_s, int T,
                        const int64_t* cache_position, float scale,
                        void* out, int out_dtype, int Hq, int Hkv, int n_split,
                        void* workspace, void* stream);

/* One decoder layer's attention from its raw qkv projection, in one launch
 * (two when n_split > 16): per-head RMSNorm of q and k (q_weight / k_weight,
 * 128 fp16 each, eps) and rotate-half RoPE with the caller's cos / sin (fp16
 * [128]: transformers' rotary embedding for the new token), the new K_rot and
 * V row written to the fp16 caches at cache_position[0], then qd_attention_decode
 * with the rotated q kept in fp32 (the new row comes from registers, not from
 * the cache).  qkv: fp16 [Hq*128 | Hkv*128 | Hkv*128]; Hq = 2 Hkv; out fp16
 * [Hq,128]; workspace as for qd_attention_decode.  Replaces the pair
 * fused_q_rope_kv_cache_update (cuda_decode_small_ops.py:136-225) +
 * decode_attn_v4_cta_qhead_splitkv_fused (cuda_decode_attention.py:489-558)
 * that OptimizedDecoderLayer.forward calls back to back
 * (optimized_layer.py:108-469). */
int qd_attention_qkv_decode_f16(const void* qkv, const void* q_weight, const void* k_weight,
                                float eps, const void* cos, const void* sin,
                                void* k_cache, void* v_cache,
                                long cache_stride_h, long cache_stride_s, int T,
                                const int64_t* cache_position, float scale, void* out,
                                int Hq, int Hkv, int n_split, void* workspace, void* stream);

/* qd_attention_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, which
 * always takes a caller-allocated workspace.  The partials and the arrival
 * counters live in a library-owned static device array of
 * QD_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; the call
 * allocates nothing.  It accepts qd_attention_workspace_bytes(Hq, Hkv, n_split)
 * <= QD_NOALLOC_SCRATCH_BYTES (Hq = 16: up to 126 splits) and otherwise
 * returns QD_ERR_WORKSPACE without launching.  Every call on one GPU uses
 * that GPU's array: calls that overlap in time on one GPU (two streams, two
 * host threads) race and must be ordered by the caller.  The first call on a
 * device also enqueues a small kernel that clears the counters. */
#define QD_NOALLOC_SCRATCH_BYTES (1u << 20)
int qd_attention_decode_noalloc(const void* q, int q_dtype, long q_stride,
                                const void* k_cache, const void* v_cache,
                                long cache_stride_h, long cache_stride_s, int T,
                                const int64_t* cache_position, float scale,
                                void* out, int out_dtype, int Hq, int Hkv, int n_split,
                                void* stream);

/* The same computation as two launches: partials only (o_part fp32
 * [Hq, n_split, 128], lse fp32 [Hq, n_split]), then the merge.  Replaces
 * decode_attn_v4_splitkv (cuda_decode_attention.py:226-302). */
int qd_attention_partial(const void* q, int q_dtype, long q_stride,
                         const void* k_cache, const void* v_cache,
                         long cache_stride_h, long cache_stride_s, int T,
                         const int64_t* cache_position, float scale,
                         float* o_part, float* lse, int Hq, int Hkv, int n_split,
                         void* stream);
int qd_attention_merge(const float* o_part, const float* lse, void* out, int out_dtype,
                       int Hq, int n_split, void* stream);

/* Default split count for a cache of capacity T (fixed per captured graph):
 * about 128 rows per split, 4..32 splits; up to 16 (T <= 2048) the merge runs
 * in the partial kernel, beyond it the merge kernel follows the partial kernel
 * (32 splits from T = 3969 on: 256 workgroups at 8 kv heads). */
int qd_attention_default_splits(int T);

/* ------------------------------------------------------------------ decode step */

/* One decoder layer's weights (fused layout of optimized_layer.py:60-84). */
typedef struct qd_layer_weights {
  const void* qkv;             /* fp16 [Hq*D + 2*Hkv*D, H] */
  const void* o_proj;          /* fp16 [H, Hq*D] */
  const void* gate_up;         /* fp16 [2I, H] */
  const void* down;            /* fp16 [H, I] */
  const void* input_norm;      /* fp16 [H] */
  const void* post_norm;       /* fp16 [H] */
  const void* q_norm;          /* fp16 [D] */
  const void* k_norm;          /* fp16 [D] */
  void* k_cache;               /* fp16 [Hkv, T, D] */
  void* v_cache;               /* fp16 [Hkv, T, D] */
} qd_layer_weights;

typedef struct qd_model_desc {
  int num_layers, hidden, num_heads, num_kv_heads, head_dim, intermediate, vocab;
  int capacity;                /* T: static-cache rows per layer */
  float eps;
  int sec_t, sec_h, sec_w;     /* M-RoPE sections */
  const float* inv_freq;       /* device fp32 [D/2] */
  const qd_layer_weights* layers;  /* host array [num_layers] */
  const void* embed;           /* fp16 [V, H] (also the tied lm_head) */
  const void* final_norm;      /* fp16 [H] */
  /* step state (device) */
  int64_t* token;              /* int64 [1]: input token, overwritten with the next token */
  const int64_t* cache_position;   /* int64 [1] */
  const int64_t* rope_position;    /* int64 [3]: T/H/W rope positions of this step */
  void* logits_out;            /* fp16 [V] or NULL */
  void* workspace;             /* qd_decode_workspace_bytes() bytes, zeroed once; its layout
                                  and self-resetting counters follow this descriptor's batch,
                                  capacity and attn_splits: a descriptor that changes any of
                                  them needs a workspace of its own, zeroed */
  int attn_splits;             /* 0 = qd_attention_default_splits(capacity) */
  int step_mode;               /* QD_STEP_AUTO / QD_STEP_CHAIN / QD_STEP_PERSISTENT */
  int batch;                   /* sequences per step: 0 or 1 = batch 1; 2..8 = batch step, then
                                  token [B], cache_position [B], rope_position [B][3], each layer's
                                  k_cache / v_cache [B, Hkv, T, D] and logits_out fp32 [B][V] */
  /* Optional end-of-step advance.  When advance_counter != NULL the step
   * finishes with qd_decode_advance (batch step: qd_decode_advance_batch,
   * out_tokens [max][B]) on (token, advance_out_tokens, advance_counter,
   * cache_position, rope_position, advance_max_tokens), done by the argmax
   * reduction instead of a separate launch; the
   * cache_position / rope_position buffers are then written by the step. */
  int64_t* advance_out_tokens;
  int64_t* advance_counter;
  int advance_max_tokens;
  /* Batch-1 argmax over the logits rounded to fp16, the first index winning
   * among equal fp16 values: the reference's FastLmHead returns fp16 logits
   * and takes torch.argmax over them (evaluation_wrapper.py:952, :1233-1238).
   * 0 (default) compares the fp32 logits, the fp32 math the parity criterion
   * is stated in; the two differ only where the top logits round to one fp16
   * value. */
  int argmax_f16_logits;
  /* Batch step only: when nonzero, every layer's qkv, o_proj, gate_up and
   * down point to copies of those matrices in MFMA tile order (the reference
   * keeps row-major weights; this layout is the batch GEMVs' own, no
   * counterpart there).  With R = qd_batch_tile_rows(rows, K, silu) for the
   * matrix (qkv: (Hq + 2 Hkv) D x H, silu 0; o_proj: H x Hq*D, silu 0;
   * gate_up: I x H, silu 1, both halves tiled as one [2I, H] matrix; down:
   * H x I, silu 0), element W[row][k] sits at
   *   R = 16: ((row / 16) * (K / 8) + k / 8) * 128 + (row % 16) * 8 + k % 8;
   *   R = 8:  ((row / 8) * (K / 64) + k / 64) * 512 + ((k % 64) / 8 % 4) * 128
   *           + ((k % 64) / 32) * 64 + (row % 8) * 8 + k % 8,
   * so one wave load is one contiguous 1 KB that is already the MFMA operand
   * (no lane permutation).  Results equal the row-major step's bit for bit. */
  int batch_tiled_weights;
} qd_model_desc;

/* How qd_decode_step runs the 28 layers.
 *   QD_STEP_CHAIN       one kernel per phase (6 per layer), any supported shape;
 *   QD_STEP_PERSISTENT  one persistent kernel for all layers (Qwen3-VL-2B text
 *                       shape, needs 256 resident workgroups of 512 threads);
 *   QD_STEP_AUTO        persistent when possible, else the chain.
 * The attention of the persistent kernel always uses 32 splits per kv head;
 * attn_splits applies to the chain.  Batch step (batch 2..8): QD_STEP_AUTO
 * runs each layer's qkv GEMV inside its attention launch, the first 256
 * workgroups computing 16 qkv rows each and handing them to the attention
 * workgroups through parity-tagged words in the workspace (bounded waits,
 * reported by qd_decode_status), when the shape allows it (H = 2048, Hq = 2 Hkv,
 * head dim 128, 4096 qkv rows, batch x Hkv x splits >= 256) and the device keeps
 * 256 of its workgroups resident; QD_STEP_CHAIN keeps the two launches;
 * QD_STEP_PERSISTENT is rejected. */
#define QD_STEP_AUTO 0
#define QD_STEP_CHAIN 1
#define QD_STEP_PERSISTENT 2

size_t qd_decode_workspace_bytes(const qd_model_desc* d);

/* Byte offsets inside the step workspace of the fp32 activation vectors the
 * step hands between kernels, in this order: residual stream x [H], qkv,
 * rotated q [Hq*D], attention output [Hq*D], post-attention residual r [H],
 * SiLU(gate)*up [I].  Writes min(n, 6) offsets; returns how many exist (6).
 * For inspection and parity tests of individual phases. */
int qd_decode_workspace_layout(const qd_model_desc* d, size_t* offsets, int n);

/* Enqueue one full batch-1 decode step: embedding row of *token, 28 layers,
 * final norm, lm_head, argmax -> *token.  The K/V of the new token are written
 * at *cache_position.  Capturable into a hipGraph (in persistent mode after a
 * first step on the device outside capture: see qd_decode_layers_persistent).
 * Replaces the captured step
 * DecodeCudaGraphRunner._run_step (evaluation_wrapper.py:941-952) driving
 * OptimizedDecoderLayer.forward (optimized_layer.py:108-469) x 28 and
 * FastLmHead (evaluation_wrapper.py:1227-1238). */
int qd_decode_step(const qd_model_desc* d, void* stream);

/* The same step restricted to layers [first_layer, first_layer + n_layers)
 * and to the phases in phase_mask (QD_PHASE_* bits); qd_decode_step is
 * (0, num_layers, QD_PHASE_ALL).  Used to time or profile one phase of the
 * chain in isolation, the role of the reference's *_profile entry points
 * (cuda_decode_gemv_ops/profile.py). */
#define QD_PHASE_EMBED 0x01u
#define QD_PHASE_QKV 0x02u
/* attention partials; the q/k head RMSNorm + M-RoPE and the K/V write of the
 * new token run in this phase's prologue */
#define QD_PHASE_ATTN 0x04u
#define QD_PHASE_ATTN_MERGE 0x08u
#define QD_PHASE_O_PROJ 0x10u
#define QD_PHASE_GATE_UP 0x20u
#define QD_PHASE_DOWN 0x40u
#define QD_PHASE_LM_HEAD 0x80u
#define QD_PHASE_ALL 0xFFu
int qd_decode_step_phases(const qd_model_desc* d, int first_layer, int n_layers,
                          unsigned phase_mask, void* stream);

/* The mode qd_decode_step will use for this descriptor on the current device
 * (QD_STEP_CHAIN or QD_STEP_PERSISTENT), or a negative status when
 * step_mode == QD_STEP_PERSISTENT cannot be honoured (the message says why). */
int qd_decode_step_mode(const qd_model_desc* d);

/* Embedding + all layers as ONE persistent launch: 256 workgroups stay
 * resident and hand activations to each other through parity-tagged words (no
 * grid barrier, no kernel boundary between layers).  The words live in one
 * area per device that the library allocates (uncached device memory, about
 * 330 KB, plus a 256-byte counter block), zeroes at the first persistent step
 * on the device and keeps until the process ends; that first step must run
 * outside stream capture (QD_ERR_ARG otherwise).  Every persistent launch on
 * the device shares the area, so persistent launches on one device must not
 * overlap in time: issue them on one stream, or order their streams with
 * events.  A launch's workgroups fill every CU, but a launch on another stream
 * can still start on the CUs that the previous launch's finished workgroups
 * free; such overlap is not detected, and the hand-offs of the launches
 * involved and of later ones on the device are then undefined.  Leaves the
 * final hidden state (before the final norm) in the workspace's residual vector
 * x (first offset of qd_decode_workspace_layout); the lm_head phase of
 * qd_decode_step_phases continues from there.  Replaces the same span of the
 * reference's captured step as qd_decode_step (OptimizedDecoderLayer.forward x
 * 28, optimized_layer.py:108-469). */
int qd_decode_layers_persistent(const qd_model_desc* d, void* stream);

/* One Qwen3-VL-2B decoder layer for one token as one persistent launch (the
 * kernel of qd_decode_layers_persistent, one layer): hidden_in fp16 [2048] ->
 * hidden_out fp16 [2048], with RMSNorm + QKV, q/k head RMSNorm + RoPE by the
 * caller's cos / sin (fp16 [128] each, two equal halves as transformers'
 * rotary embedding makes them), the new K/V row written into w->k_cache /
 * w->v_cache ([8, capacity, 128]) at *cache_position, attention over rows
 * 0..min(*cache_position, capacity - 1) scaled by `scale`, o_proj + residual,
 * RMSNorm + gate_up + SiLU*up, down + residual; each linear layer's input is
 * rounded to fp16 (as the reference's fp16 modules take it), while the
 * residual stream, the sums of squares and the values handed between the
 * phases stay fp32.  length_out (nullable): set to *cache_position + 1 after every
 * workgroup has read *cache_position (a static cache's running length; it may
 * be the same word as cache_position).  status: a device word the caller
 * zeroes; bit 0 is set when a hand-off wait ran out of its polling budget
 * (the output is then invalid).  Shares the per-device hand-off area and its
 * rules with qd_decode_layers_persistent (the first persistent launch on a
 * device must not be under stream capture: qd_persistent_prepare).
 * QD_ERR_SHAPE when the device cannot keep the grid resident.  Replaces
 * cuda_decode_gemv.fused_decode_full_layer_softsync_half
 * (cuda_decode_gemv_ops/fused.py:498-665), the one-launch decoder layer that
 * OptimizedDecoderLayer.forward tries first (optimized_layer.py:127-154,
 * :1490-1610). */
int qd_decoder_layer_persistent_f16(const void* hidden_in, const qd_layer_weights* w, int capacity,
                                    const int64_t* cache_position, const void* cos, const void* sin, float eps,
                                    float scale, void* hidden_out, int64_t* length_out, unsigned* status,
                                    void* stream);

/* Several consecutive decoder layers of the swapped model in one persistent
 * launch: layer l reads layer l - 1's output rounded to fp16, exactly what a
 * launch of qd_decoder_layer_persistent_f16 for layer l would read, so every
 * output equals (bit for bit) that of n_layers one-layer launches in a row.
 * hidden_out: fp16 [n_layers][2048], layer l's output in row l.  length_out:
 * nullable array of n_layers nullable words, each set to *cache_position + 1
 * after the launch.  All layers decode the same cache position with the same
 * cos / sin (transformers passes one rotary embedding to every layer).  Other
 * arguments, the status word and the hand-off area's rules as for
 * qd_decoder_layer_persistent_f16.  Used by the swapped layers' opt-in
 * look-ahead: the first swapped layer of a step launches the whole stack when
 * every layer after it is swapped and hook-free, and the later layers return
 * their rows (optimized_layer.set_decode_layer_lookahead).  No counterpart in
 * the reference, whose OptimizedDecoderLayer.forward launches one layer per
 * call (optimized_layer.py:108-154); it serves that forward's callers. */
int qd_decoder_layers_persistent_f16(const void* hidden_in, const qd_layer_weights* layers, int n_layers,
                                     int capacity, const int64_t* cache_position, const void* cos, const void* sin,
                                     float eps, float scale, void* hidden_out, int64_t* const* length_out,
                                     unsigned* status, void* stream);

/* Allocates and zeroes the current device's persistent hand-off area if it is
 * not there yet (outside stream capture; synchronous the first time), so that
 * later persistent launches may be captured.  QD_ERR_SHAPE when the device
 * cannot keep the persistent grid resident.  No counterpart in the reference
 * (its soft-sync kernels take their counters from the caller's workspace). */
int qd_persistent_prepare(void* stream);

/* Diagnostic: every later persistent launch of the process (qd_decode_step in
 * persistent mode, qd_decode_layers_persistent, qd_decoder_layer_persistent_f16)
 * and every later batch step's qkv hand-off lets each thread poll at most
 * `polls` times over the whole launch before its hand-off waits give up (0
 * restores the default, tens of milliseconds of polling).  A launch whose
 * budget runs out sets bit 0 of its status word, finishes every wave and
 * writes every hand-off word once per layer, so the next launch is
 * unaffected; its own results are invalid.  Launches already
 * captured in a graph keep the limit they were captured with.  For tests of
 * the failure path; no counterpart in the reference (its soft-sync waits are
 * unbounded). */
int qd_persistent_set_spin_limit(unsigned polls);

/* Phase timeline of the persistent step, for profiling.  A library built with
 * -DQD_TRACE (libqwen3vl_decode_trace.so, made by the package's build step
 * next to the main library) has the first thread of wave 0 (a polling wave)
 * and of wave 4 (a streaming wave) of every workgroup record the 100 MHz
 * real-time clock at fixed points of every layer of each launch: events 0..12
 * (wave 0) layer start, x gathered, qkv rows stored, qkv gathered, attention
 * loop done, split partials stored, merged output gathered, o_proj start, r
 * rows stored, r gathered, hidden rows stored, hidden gathered, x rows stored;
 * 13..15 further wave-0 points; 16..31 wave 4's points (the names are listed
 * in qwen3vl_hip/phase_trace.py).  Writes
 * dims[3] = {workgroups, layer slots, event slots} and copies
 * min(n, product of dims) stamps of the last launch, indexed
 * [(workgroup * layer slots + layer) * event slots + event], to host dst
 * (synchronous).  The regular library returns QD_ERR_ARG and copies nothing.
 * No counterpart in the reference (its NVIDIA profiling hooks,
 * cuda_decode_gemv_ops/profile.py, are out of scope). */
int qd_persistent_trace_read(uint64_t* dst, size_t n, int* dims);

/* Synchronously reads the status word of the persistent step, or of the
 * batch step's qkv hand-off (0 = every hand-off completed; bit 0 = a wait
 * exhausted its spin budget, results of that step are invalid) and clears it
 * when reset != 0. */
int qd_decode_status(const qd_model_desc* d, unsigned* status, int reset);

/* Batch decoding (batch 2..8 in qd_model_desc.batch).  qd_decode_step runs
 * the batch step: per layer an MFMA batch GEMV (v_mfma_f32_16x16x32_f16; the
 * activation enters as fp16 value + fp16 rounding residual, so the product is
 * fp32-accurate) for RMSNorm+QKV, o_proj+residual, RMSNorm+gate_up+SiLU*up and
 * down+residual, and the split-KV attention with each sequence at its own cache
 * position; then final RMSNorm, lm_head and an argmax per sequence.  The
 * reference has no batch path: it rejects batch != 1 in its decode runner
 * (evaluation_wrapper.py:110-111) and falls back to HF generate; this is the
 * batch-8 workload of the benchmark configurations (config 4). */
#define QD_BATCH_EPI_STORE 0   /* y = W x' (+ residual) */
#define QD_BATCH_EPI_SILU 1    /* y = silu(W_gate x') * (W_up x'), W_up = rows [N, 2N) */

/* Batch GEMV for up to 8 sequences: y[b][r] = W[r] . x'[b] for b < nseq, with
 * x' = RMSNorm(x[b]) * gamma when gamma != NULL (eps), else x.  x, residual, y
 * fp32 with row strides ldx / ldr / ldy; W fp16 [rows, ldw]; K in {2048, 6144};
 * N a multiple of 16; for QD_BATCH_EPI_SILU up_offset == N and K == 2048.
 * workspace: device memory of qd_batch_gemv_workspace_bytes(N, K) bytes,
 * zeroed before its first use (it holds self-resetting counters) and not
 * shared by two calls in flight. */
size_t qd_batch_gemv_workspace_bytes(long N, long K);
int qd_batch_gemv(const float* x, long ldx, const void* gamma, float eps, const void* W, long ldw, long N,
                  long K, long up_offset, const float* residual, long ldr, float* y, long ldy, int nseq,
                  int epilogue, void* workspace, size_t workspace_bytes, void* stream);

/* Rows per row group (8 or 16) of the batch step's GEMV over a rows x K
 * matrix (silu: the gate_up GEMV, rows = I), which fixes its tile-order
 * layout (qd_model_desc.batch_tiled_weights); 0 for sizes <= 0. */
int qd_batch_tile_rows(long rows, long K, int silu);

/* qd_decode_advance for a batch: out_tokens [max_tokens][batch]. */
int qd_decode_advance_batch(const int64_t* token, int64_t* out_tokens, int64_t* counter,
                            int64_t* cache_position, int64_t* rope_position, int max_tokens, int batch,
                            void* stream);

/* Device-side end of a generation step (single thread):
 *   out_tokens[*counter] = *token (when *counter < max_tokens); ++*counter;
 *   ++*cache_position; ++rope_position[0..2].
 * Captured after qd_decode_step it lets a hipGraph replay loop generate with
 * no host writes; it replaces the host-side input staging of
 * DecodeCudaGraphRunner._write_inputs (evaluation_wrapper.py:954-960). */
int qd_decode_advance(const int64_t* token, int64_t* out_tokens, int64_t* counter,
                      int64_t* cache_position, int64_t* rope_position, int max_tokens,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN3VL_DECODE_H */
