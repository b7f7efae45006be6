// Forward kernel: one workgroup = one (segment, 128-row query tile, head).
//
// Computes O and the LSE for the prefix rows (reference pass 1,
// models/flash_attention_prefixlm_v2.py:115-121) and the suffix rows (pass 2,
// :122-128) of a tile in one launch: rows below the prefix boundary see the whole
// prefix, rows at or past it see keys <= themselves.
//
// Layout (D = 128, 4 waves, each wave owns 32 query rows):
//   * the wave computes S^T = K Q^T so that each lane owns one query (column) and
//     the softmax max/sum need one cross-lane step (lane l <-> l^32);
//   * Q^T stays in registers as the MFMA B operand for the whole key loop;
//   * K tiles (64 keys) are staged in LDS row-major, V tiles transposed (d-major),
//     both double-buffered, loaded with 128-bit buffer loads one tile ahead;
//   * O^T accumulates in 4 32x32 fp32 tiles; every lane rescales only its own column.
#pragma once
#include "common.h"

namespace prefixlm {
namespace fwd {

constexpr int D = 128;
constexpr int BM = 128;          // query rows per workgroup
constexpr int BN = 64;           // keys per inner iteration
constexpr int NT = 256;          // threads
constexpr int KS = D + 8;        // LDS row stride of K tile (elements): 272 B
constexpr int VS = BN + 8;       // LDS row stride of V^T tile (elements): 144 B
constexpr int K_TILE = BN * KS;  // elements
constexpr int V_TILE = D * VS;
constexpr int STAGE = K_TILE + V_TILE;
constexpr int LDS_BYTES = 2 * STAGE * 2;

struct Params {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  bf16* o_lo;        // optional: bf16(O - bf16(O)), the rounding residual of o
  float* lse;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lo_st, lo_sh;
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  const int2* items;
  const WsHeader* hdr;
  int T, H, is_causal;
  float scale_log2;  // softmax_scale * log2(e)
};

__global__ __launch_bounds__(NT, 2) void prefixlm_fwd_kernel(Params P) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];

  const int item = blockIdx.x / P.H;
  const int h = blockIdx.x - item * P.H;
  if (item >= P.hdr->n_items) return;
  const int2 it = P.items[item];
  const int seg = it.x, qt = it.y;
  const int cs = P.cu[seg];
  const int L = P.prefix[seg] + P.causal[seg];
  const int p = P.is_causal ? 0 : P.prefix[seg];

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int q0 = qt * BM;
  const int qw0 = q0 + w * 32;
  const int kend = min(L, max(p, min(q0 + BM, L)));
  const int nk = (kend + BN - 1) / BN;
  const bool wave_active = qw0 < L;
  const int kend_w = wave_active ? min(L, max(p, min(qw0 + 32, L))) : 0;

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(P.q + cs * P.q_st + h * P.q_sh, rows_bytes(L, P.q_st, D));
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(P.k + cs * P.k_st + h * P.k_sh, rows_bytes(L, P.k_st, D));
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(P.v + cs * P.v_st + h * P.v_sh, rows_bytes(L, P.v_st, D));
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(P.o + cs * P.o_st + h * P.o_sh, rows_bytes(L, P.o_st, D));
  const bool has_lo = P.o_lo != nullptr;
  const __amdgpu_buffer_rsrc_t lor =
      make_rsrc(has_lo ? P.o_lo + cs * P.lo_st + h * P.lo_sh : P.o, has_lo ? rows_bytes(L, P.lo_st, D) : 0u);
  const uint32_t kst2 = (uint32_t)P.k_st * 2, vst2 = (uint32_t)P.v_st * 2;

  // Q^T fragments: lane holds query qw0+l32, d = 16*s + 8*hh + 0..7
  bf16x8 qf[8];
  {
    const uint32_t off = (uint32_t)(qw0 + l32) * (uint32_t)P.q_st * 2 + hh * 16;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(bf16x8, buf_load16(qr, off + s * 32));
  }
  // Wait for Q here: otherwise the first MFMAs of every loop iteration carry a
  // conservative vmcnt wait that also covers the next tile's prefetch loads.
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)

  // global -> register staging of one K/V tile
  const int kr_row = tid >> 4, kr_chunk = tid & 15;   // K: 4 passes of 16 rows x 16 chunks
  const int vg = tid & 15, vdc = tid >> 4;            // V: 4 tokens (4*vg..) x 8 dims (8*vdc..)
  u32x4 ks[4], vs[4];
  auto load_kv = [&](int k0) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      ks[r] = buf_load16(kr, (uint32_t)(k0 + r * 16 + kr_row) * kst2 + kr_chunk * 16);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      vs[j] = buf_load16(vr, (uint32_t)(k0 + 4 * vg + j) * vst2 + vdc * 16);
  };
  auto store_kv = [&](int stage) {
    bf16* Ks = smem + stage * STAGE;
    bf16* Vt = Ks + K_TILE;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<u32x4*>(Ks + (r * 16 + kr_row) * KS + kr_chunk * 8) = ks[r];
    const int pos = swz23(4 * vg);
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      const uint32_t w0 = vs[0][e2], w1 = vs[1][e2], w2 = vs[2][e2], w3 = vs[3][e2];
      u32x2 lo = {pack_lo(w0, w1), pack_lo(w2, w3)};
      u32x2 hi = {pack_hi(w0, w1), pack_hi(w2, w3)};
      *reinterpret_cast<u32x2*>(Vt + (8 * vdc + 2 * e2) * VS + pos) = lo;
      *reinterpret_cast<u32x2*>(Vt + (8 * vdc + 2 * e2 + 1) * VS + pos) = hi;
    }
  };

  f32x16 oacc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float c = P.scale_log2;
  const int qi = qw0 + l32;   // this lane's query (local index)

  if (nk > 0) {
    load_kv(0);
    store_kv(0);
  }
  __syncthreads();

  for (int j = 0; j < nk; ++j) {
    const int stage = j & 1;
    const int k0 = j * BN;
    if (j + 1 < nk) load_kv(k0 + BN);
    if (wave_active && k0 < kend_w) {
      const bf16* Ks = smem + stage * STAGE;
      const bf16* Vt = Ks + K_TILE;
      f32x16 sacc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[t][r] = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(Ks + (t * 32 + l32) * KS + s * 16 + hh * 8);
          sacc[t] = mfma32x32x16(a, qf[s], sacc[t]);
        }
      }
      // per-element mask only on tiles that touch the diagonal band, the prefix
      // boundary or the segment end
      const bool full = (k0 + BN <= L) && (k0 + BN <= max(p, qw0 + 1));
      if (!full) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kj = k0 + t * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
            const bool ok = (kj < L) && (kj <= qi || kj < p);
            if (!ok) sacc[t][r] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
      mx = fmaxf(mx, wave_xor32(mx));
      const float m_new = fmaxf(m_run, mx * c);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
      bf16x8 pb[4];
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            e[i] = __builtin_amdgcn_exp2f(sacc[t][8 * half + i] * c - m_use);
            ps += e[i];
          }
          pb[2 * t + half] = cvt8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
        }
      l_run += ps;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(Vt + (t * 32 + l32) * VS + s * 16 + hh * 8);
          oacc[t] = mfma32x32x16(a, pb[s], oacc[t]);
        }
      }
    }
    if (j + 1 < nk) store_kv(stage ^ 1);
    __syncthreads();
  }

  if (wave_active) {
    const float lt = l_run + wave_xor32(l_run);
    const float inv = 1.f / lt;
    const uint32_t obase = (uint32_t)qi * (uint32_t)P.o_st * 2;
    const uint32_t lobase = (uint32_t)qi * (uint32_t)P.lo_st * 2;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float o0 = oacc[t][4 * g] * inv, o1 = oacc[t][4 * g + 1] * inv;
        const float o2 = oacc[t][4 * g + 2] * inv, o3 = oacc[t][4 * g + 3] * inv;
        const bf16x4 v4 = cvt4(o0, o1, o2, o3);
        const int dcol = t * 32 + 8 * g + 4 * hh;
        buf_store8(__builtin_bit_cast(u32x2, v4), orr, obase + dcol * 2);
        if (has_lo) {
          const bf16x4 r4 = cvt4(o0 - (float)v4[0], o1 - (float)v4[1], o2 - (float)v4[2], o3 - (float)v4[3]);
          buf_store8(__builtin_bit_cast(u32x2, r4), lor, lobase + dcol * 2);
        }
      }
    if (hh == 0 && qi < L) P.lse[(int64_t)h * P.T + cs + qi] = (m_run + __builtin_log2f(lt)) * kLn2;
  }
}

// Rows >= total_seqlen: out = 0 (and its residual) and lse = -inf (reference :130;
// FA3 leaves its LSE there unspecified). One 16-thread group per (row, head), 16 B
// per thread.
__global__ __launch_bounds__(256) void prefixlm_fwd_pad_kernel(bf16* o, bf16* o_lo, float* lse,
                                                                int64_t o_st, int64_t o_sh,
                                                                int64_t lo_st, int64_t lo_sh, int T,
                                                                int H, int total) {
  const int64_t gidx = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int64_t rows = (int64_t)(T - total) * H;
  if (gidx >= rows) return;
  const int t = total + (int)(gidx / H);
  const int h = (int)(gidx % H);
  const int chunk = threadIdx.x & 15;
  u32x4 z = {0u, 0u, 0u, 0u};
  *reinterpret_cast<u32x4*>(o + t * o_st + h * o_sh + chunk * 8) = z;
  if (o_lo) *reinterpret_cast<u32x4*>(o_lo + t * lo_st + h * lo_sh + chunk * 8) = z;
  if (chunk == 0) lse[(int64_t)h * T + t] = -INFINITY;
}

}  // namespace fwd
}  // namespace prefixlm
