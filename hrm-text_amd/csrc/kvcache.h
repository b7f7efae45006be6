// KV-cache attention: the inference path of the reference's attention layer
// (flash_attn_with_kvcache at models/layers.py:147-151, driven by
// simple_inference_engine.py:105-112, :131, :179-180).
//
// Semantics (FlashAttention's documented kv-cache call, as the reference uses it):
// the new rows k, v [B, S, H, D] are written into the caches [B, Smax, H, D] at
// rows len_b .. len_b + S - 1 (len_b = cache_seqlens[b]); query i of batch row b
// then attends the lk = len_b + S cache keys (lk = len_b when no new rows are
// given), and with `causal` only keys j <= lk - S + i (bottom-right alignment). No
// segment structure: a cache row is one sequence.
//
// Kernels:
//   append  : copies the new k, v rows into the caches (rows past Smax are dropped);
//   decode  : split-K over the keys. A workgroup = (b, h, split of kChunk keys); each
//             16-lane group owns one key at a time (16 x 16-byte chunks of a 256-byte
//             row), four keys per step, with an online softmax in fp32; the 16
//             groups are merged through LDS and the split writes (max, sum, o[D])
//             unnormalised to the workspace. HBM-bound: 2 * D * 2 bytes per key.
//   combine : merges the splits of each (b, i, h) and writes bf16 out.
#pragma once
#include "common.h"

namespace prefixlm {
namespace kvc {

constexpr int D = 128;
constexpr int NT = 256;
constexpr int GROUPS = NT / 16;      // keys in flight per workgroup step (x kUnroll)
constexpr int kUnroll = 4;
constexpr int kChunk = 512;          // keys per split
constexpr int kPart = D + 4;         // floats per partial: max (log2 units), sum, 2 unused, o[D]
static_assert(kPart % 4 == 0, "partials keep o 16-byte aligned");

struct Params {
  const bf16* q;
  const bf16* k;          // new rows (may be null)
  const bf16* v;
  bf16* kc;
  bf16* vc;
  bf16* out;
  float* part;            // [B, S, H, nsplit, kPart]
  const int32_t* seqlens; // device [B]; null: every row has seqlen_const
  int64_t q_sb, q_ss, q_sh, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh;
  int64_t kc_sb, kc_ss, kc_sh, vc_sb, vc_ss, vc_sh, o_sb, o_ss, o_sh;
  int B, S, H, Smax, nsplit, causal, seqlen_const;
  int s_new;              // rows appended by this call: S, or 0 without new k, v
  float scale_log2;
};

__device__ __forceinline__ int cache_len(const Params& P, int b) {
  return P.seqlens ? P.seqlens[b] : P.seqlen_const;
}

// thread = 16-byte chunk of one (b, i, h) row of k and of v
__global__ __launch_bounds__(256) void append_kernel(Params P) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int c = (int)(gid & 15);
  const int64_t r = gid >> 4;
  if (r >= (int64_t)P.B * P.S * P.H) return;
  const int h = (int)(r % P.H);
  const int i = (int)((r / P.H) % P.S);
  const int b = (int)(r / ((int64_t)P.H * P.S));
  const int row = cache_len(P, b) + i;
  if (row < 0 || row >= P.Smax) return;
  const u32x4 kv = *reinterpret_cast<const u32x4*>(P.k + b * P.k_sb + i * P.k_ss + h * P.k_sh + 8 * c);
  const u32x4 vv = *reinterpret_cast<const u32x4*>(P.v + b * P.v_sb + i * P.v_ss + h * P.v_sh + 8 * c);
  *reinterpret_cast<u32x4*>(P.kc + b * P.kc_sb + row * P.kc_ss + h * P.kc_sh + 8 * c) = kv;
  *reinterpret_cast<u32x4*>(P.vc + b * P.vc_sb + row * P.vc_ss + h * P.vc_sh + 8 * c) = vv;
}

__device__ __forceinline__ float sum16(float x) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

// blockIdx.x = ((b * H + h) * nsplit + split); queries i = 0 .. S-1 one after another
__global__ __launch_bounds__(NT) void decode_kernel(Params P) {
  __shared__ float s_m[GROUPS], s_l[GROUPS];
  __shared__ f32x4 s_o[GROUPS][D / 4];
  const int split = blockIdx.x % P.nsplit;
  const int bh = blockIdx.x / P.nsplit;
  const int h = bh % P.H, b = bh / P.H;
  const int tid = threadIdx.x, grp = tid >> 4, g16 = tid & 15;
  const int len = cache_len(P, b);
  const int lk = min(P.Smax, len + P.s_new);   // keys in the cache after the append
  const bf16* kbase = P.kc + b * P.kc_sb + h * P.kc_sh + 8 * g16;
  const bf16* vbase = P.vc + b * P.vc_sb + h * P.vc_sh + 8 * g16;
  for (int i = 0; i < P.S; ++i) {
    // keys [k0, k1) of this split that query i sees
    const int kmax = P.causal ? min(lk, len + P.s_new - P.S + i + 1) : lk;
    const int k0 = split * kChunk;
    const int k1 = min(kmax, k0 + kChunk);
    float q[8];
    {
      const u32x4 w = *reinterpret_cast<const u32x4*>(P.q + b * P.q_sb + i * P.q_ss + h * P.q_sh + 8 * g16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        q[2 * e] = bf16lo(w[e]) * P.scale_log2;
        q[2 * e + 1] = bf16hi(w[e]) * P.scale_log2;
      }
    }
    float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
    for (int j0 = k0 + grp; j0 < k1; j0 += GROUPS * kUnroll) {
      u32x4 kw[kUnroll], vw[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int j = min(j0 + u * GROUPS, k1 - 1);   // clamped rows are masked below
        kw[u] = *reinterpret_cast<const u32x4*>(kbase + j * P.kc_ss);
        vw[u] = *reinterpret_cast<const u32x4*>(vbase + j * P.vc_ss);
      }
      float s[kUnroll], mx = m;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) d += q[2 * e] * bf16lo(kw[u][e]) + q[2 * e + 1] * bf16hi(kw[u][e]);
        d = sum16(d);
        s[u] = (j0 + u * GROUPS < k1) ? d : -INFINITY;
        mx = fmaxf(mx, s[u]);
      }
      const float alpha = __builtin_amdgcn_exp2f(m - mx);   // m = -inf at first: 0
      l *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float p = __builtin_amdgcn_exp2f(s[u] - mx);
        l += p;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[2 * e] += p * bf16lo(vw[u][e]);
          o[2 * e + 1] += p * bf16hi(vw[u][e]);
        }
      }
      m = mx;
    }
    // merge the 16 groups
    if (g16 == 0) {
      s_m[grp] = m;
      s_l[grp] = l;
    }
    s_o[grp][2 * g16] = f32x4{o[0], o[1], o[2], o[3]};
    s_o[grp][2 * g16 + 1] = f32x4{o[4], o[5], o[6], o[7]};
    __syncthreads();
    if (tid < D / 4) {
      float M = -INFINITY;
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) M = fmaxf(M, s_m[g]);
      float L = 0.f;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) {
        const float w = s_m[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[g] - M);
        L += w * s_l[g];
        acc += w * s_o[g][tid];
      }
      float* dst = P.part + ((((int64_t)b * P.S + i) * P.H + h) * P.nsplit + split) * kPart;
      if (tid == 0) {
        dst[0] = M;
        dst[1] = L;
      }
      *reinterpret_cast<f32x4*>(dst + 4 + 4 * tid) = acc;   // kPart keeps o 16-byte aligned
    }
    __syncthreads();
  }
}

// one wave per (b, i, h); lane covers d = 2 * lane, 2 * lane + 1
__global__ __launch_bounds__(256) void combine_kernel(Params P) {
  const int64_t w = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (w >= (int64_t)P.B * P.S * P.H) return;
  const int h = (int)(w % P.H);
  const int i = (int)((w / P.H) % P.S);
  const int b = (int)(w / ((int64_t)P.H * P.S));
  const float* src = P.part + w * P.nsplit * kPart;
  float M = -INFINITY;
  for (int s = 0; s < P.nsplit; ++s) M = fmaxf(M, src[s * kPart]);
  float L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int s = 0; s < P.nsplit; ++s) {
    const float ms = src[s * kPart];
    if (ms == -INFINITY) continue;
    const float wgt = __builtin_amdgcn_exp2f(ms - M);
    L += wgt * src[s * kPart + 1];
    o0 += wgt * src[s * kPart + 4 + 2 * lane];
    o1 += wgt * src[s * kPart + 5 + 2 * lane];
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  f32x4 pr = {o0 * inv, o1 * inv, 0.f, 0.f};
  const bf16x4 ob = __builtin_convertvector(pr, bf16x4);
  bf16* op = P.out + b * P.o_sb + i * P.o_ss + h * P.o_sh + 2 * lane;
  op[0] = ob[0];
  op[1] = ob[1];
}

// metadata of a batched prefill (cache_seqlen 0): batch row b is segment b of S
// rows, a whole prefix (bidirectional) or, with causal, a whole suffix
__global__ void prefill_meta_kernel(int32_t* prefix, int32_t* causal_lens, int32_t* cu, int B, int S, int causal) {
  for (int b = threadIdx.x; b <= B; b += blockDim.x) {
    if (b < B) {
      prefix[b] = causal ? 0 : S;
      causal_lens[b] = causal ? S : 0;
    }
    cu[b] = b * S;
  }
}

}  // namespace kvc
}  // namespace prefixlm
