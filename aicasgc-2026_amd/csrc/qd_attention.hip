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
// Online softmax per slot in fp32 (one exp per position and head), slot
// partials merged through LDS into a per-split (normalised output, LSE) pair;
// splits are merged either by the last workgroup of the kv head to arrive
// (self-resetting arrival counter) or by a separate merge kernel.

#include <math.h>

#include "qd_common.h"
#include "qd_kernels.h"

namespace qd {

namespace {
constexpr int kD = 128;
constexpr int kSlots = 16;
constexpr int kUnroll = 4;
}  // namespace

template <int G, typename TO>
__device__ __forceinline__ void merge_splits(const AttnArgs& a, int kvh) {
  TO* out = reinterpret_cast<TO*>(a.out);
  for (int t = threadIdx.x; t < G * kD; t += blockDim.x) {
    const int h = kvh * G + t / kD;
    const int d = t % kD;
    const float* lse = a.lse + (long)h * a.n_split;
    float M = -INFINITY;
    for (int s = 0; s < a.n_split; ++s) M = fmaxf(M, lse[s]);
    float num = 0.f, den = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < a.n_split; ++s) {
        const float w = __expf(lse[s] - M);
        den += w;
        num = __builtin_fmaf(w, a.o_part[((long)h * a.n_split + s) * kD + d], num);
      }
    }
    store_act(out, (long)h * kD + d, den > 0.f ? num / den : 0.f);
  }
}

template <int G, typename TQ, typename TO>
__global__ __launch_bounds__(256) void attn_split_kernel(const AttnArgs a, const int fused_merge) {
  const int kvh = blockIdx.x / a.n_split;
  const int split = blockIdx.x % a.n_split;
  const int slot = threadIdx.x >> 4;
  const int dl = (threadIdx.x & 15) * 8;

  const long pos = a.cache_position[0];
  long Ll = pos + 1 < (long)a.T ? pos + 1 : (long)a.T;
  if (Ll < 0) Ll = 0;
  const int L = (int)Ll;
  const int chunk = (L + a.n_split - 1) / a.n_split;
  const int t0 = split * chunk;
  const int t1 = min(t0 + chunk, L);

  float q[G][8];
  const TQ* qp = reinterpret_cast<const TQ*>(a.q);
#pragma unroll
  for (int g = 0; g < G; ++g) load_act8(qp, (long)(kvh * G + g) * a.q_stride + dl, q[g]);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }

  const uint16_t* kb = a.k + (long)kvh * a.stride_h + dl;
  const uint16_t* vb = a.v + (long)kvh * a.stride_h + dl;
  for (int t = t0 + slot; t < t1; t += kSlots * kUnroll) {
    u32x4 kk[kUnroll], vv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int tt = t + u * kSlots;
      if (tt < t1) {
        kk[u] = ld_stream(kb + (long)tt * a.stride_s);
        vv[u] = ld_stream(vb + (long)tt * a.stride_s);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int tt = t + u * kSlots;
      if (tt < t1) {
        float vf[8];
        unpack8(vv[u], vf);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float s = row16_sum(dot8(kk[u], q[g], 0.f)) * a.scale;
          const float dlt = s - m[g];
          const float e = __expf(-fabsf(dlt));
          const bool up = dlt > 0.f;
          const float c = up ? e : 1.f;   // rescale of the running sums
          const float p = up ? 1.f : e;   // weight of this position
          m[g] = up ? s : m[g];
          l[g] = __builtin_fmaf(l[g], c, p);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(acc[g][i], c, p * vf[i]);
        }
      }
    }
  }

  // ---- merge the 16 slots of this workgroup
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
    a.o_part[((long)h * a.n_split + split) * kD + d] = den > 0.f ? num / den : 0.f;
    if (d == 0) a.lse[(long)h * a.n_split + split] = den > 0.f ? M + __logf(den) : -INFINITY;
  }

  if (!fused_merge) return;
  __shared__ int s_last;
  fence_release();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomic_add_release(a.counters + kvh, 1u);
    s_last = (prev == (unsigned)a.n_split - 1u);
  }
  __syncthreads();
  if (!s_last) return;
  fence_acquire();
  merge_splits<G, TO>(a, kvh);
  if (threadIdx.x == 0) store_relaxed(a.counters + kvh, 0u);
}

template <typename TO>
__global__ __launch_bounds__(128) void attn_merge_kernel(const AttnArgs a) {
  // one block per q head; merge_splits with G = 1 treats blockIdx.x as the head.
  merge_splits<1, TO>(a, blockIdx.x);
}

template <typename TQ, typename TO>
int attention_launch(const AttnArgs& a, bool fused_merge, hipStream_t s) {
  const int G = a.Hq / a.Hkv;
  const dim3 grid((unsigned)(a.Hkv * a.n_split));
  const int fm = fused_merge ? 1 : 0;
  switch (G) {
    case 1: hipLaunchKernelGGL((attn_split_kernel<1, TQ, TO>), grid, dim3(256), 0, s, a, fm); break;
    case 2: hipLaunchKernelGGL((attn_split_kernel<2, TQ, TO>), grid, dim3(256), 0, s, a, fm); break;
    case 4: hipLaunchKernelGGL((attn_split_kernel<4, TQ, TO>), grid, dim3(256), 0, s, a, fm); break;
    default: return QD_ERR_SHAPE;
  }
  return qd_host::launch_status("attn_split_kernel");
}

template <typename TO>
int attention_merge_launch(const AttnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((attn_merge_kernel<TO>), dim3((unsigned)a.Hq), dim3(128), 0, s, a);
  return qd_host::launch_status("attn_merge_kernel");
}

template int attention_launch<uint16_t, uint16_t>(const AttnArgs&, bool, hipStream_t);
template int attention_launch<float, float>(const AttnArgs&, bool, hipStream_t);
template int attention_launch<uint16_t, float>(const AttnArgs&, bool, hipStream_t);
template int attention_launch<float, uint16_t>(const AttnArgs&, bool, hipStream_t);
template int attention_merge_launch<uint16_t>(const AttnArgs&, hipStream_t);
template int attention_merge_launch<float>(const AttnArgs&, hipStream_t);

}  // namespace qd
