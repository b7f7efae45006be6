// Backward kernels.
//
// Replaces the two FA3 backward calls and the elementwise epilogue of
// models/flash_attention_prefixlm_v2.py:152-212 (reference):
//   pre  : delta[h,t] = sum_d dO*O (fp32; O = out + its rounding residual when the
//          forward kept one) and per-head maxima of |dO|, ||dO_t|| and |delta_t|;
//   dkdv : one workgroup = one (segment, 128-key tile, head) in four wave pairs of 32
//          keys. Per 32-row query tile, wave A of a pair recomputes S = Q K^T and
//          P = exp(S*scale - lse), hands P to wave B through LDS and accumulates
//          dV^T += dO^T P; wave B computes dP = dO V^T, dS = P (dP - delta) and
//          accumulates dK^T += Q^T dS. Each key row is owned by one workgroup, which
//          sees both the prefix rows and the suffix rows, so the reference's
//          dk1 + dk2 / dv1 + dv2 (:212) disappears;
//   dq   : one workgroup = one (segment, 128-query tile, head); each wave holds Q and
//          dO of 32 queries in registers, streams 32-key tiles of K and V through
//          LDS, recomputes S, P, dP, dS and accumulates dQ^T += K^T dS^T, then
//          writes bf16 dQ. No atomics: dQ is bitwise deterministic;
//   pad  : dq, dk, dv rows >= total_seqlen are zeroed (:209-211).
//
// Precision: S and dP contract 16-bit inputs over D whose products are exact in
// fp32. The dV product uses fp16 P (P lies in [0, 1]) and fp16 dO scaled by a
// per-head power of two; the dQ product uses fp16 dS and fp16 K, each scaled by a
// power of two chosen from a bound on its magnitude. fp16 keeps 3 more mantissa
// bits than bf16 and the power-of-two scales are undone exactly in fp32. dK uses
// bf16 dS and Q (its error budget is met without it).
#pragma once
#include <type_traits>

#include "common.h"

namespace prefixlm {
namespace bwd {

constexpr int D = 128;
constexpr int kStats = 4;        // per head: max|dO|, max ||dO_t||_2, max |delta_t|, unused
constexpr int kSegStats = 2;     // per (segment, head): max |K|, max ||V_k||_2

__device__ __forceinline__ void atomic_max_nonneg(float* p, float v) {
  atomicMax(reinterpret_cast<int*>(p), __builtin_bit_cast(int, v));
}

// =====================================================================================
// dK / dV
// =====================================================================================
namespace kv {
constexpr int BK = 128;                // keys per workgroup
constexpr int KP = 32;                 // keys per wave pair
constexpr int NPAIR = BK / KP;
constexpr int BQ = 32;                 // query rows per iteration
constexpr int NT = 2 * NPAIR * 64;     // waves 0..NPAIR-1: role A, NPAIR..: role B
constexpr int TILE = BQ * RS;          // one 32 x 128 16-bit tile
constexpr int OFF_QS = 0;              // [3] tiles: bf16 Q (tiles i-1, i, i+1)
constexpr int OFF_DOS = 3 * TILE;      // [3] tiles: fp16 dO * s_do
constexpr int PEX_BUF = NPAIR * 2048;  // [NPAIR][2][64 lanes][8] fp16 P, A -> B
constexpr int OFF_PEX = 6 * TILE;      // [2] P buffers (tiles i-1, i)
constexpr int OFF_LSE = OFF_PEX + 2 * PEX_BUF;    // [2][BQ] lse * log2(e)
constexpr int OFF_DLT = OFF_LSE + 2 * BQ * 4;     // [2][BQ] -delta * s_do * s_v
constexpr int OFF_RED = OFF_DLT + 2 * BQ * 4;     // [NPAIR] max ||V_k|| of each pair
constexpr int LDS_BYTES = OFF_RED + 16;
}  // namespace kv

struct KvParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* dout;
  const float* lse;       // [H, T]
  const float* delta;     // [H, T]
  const float* stats;     // [H, kStats]
  float* segstats;        // [numseqs, H, kSegStats], atomic max
  bf16* dk;
  bf16* dv;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, do_st, do_sh, dk_st, dk_sh, dv_st, dv_sh;
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  const int2* items;
  const WsHeader* hdr;
  int T, H, is_causal;
  int numseqs;            // items naming a segment >= numseqs (a stale plan) are skipped
  float scale_log2;       // softmax_scale * log2(e)
  float scale;            // softmax_scale
};

// One wave of a pair. ROLE 0 (A): K rows in registers, S -> P, P to LDS, dV^T.
// ROLE 1 (B): V rows in registers (fp16, scaled), dP, P from LDS -> dS, dK^T.
// Both roles execute the same sequence of workgroup barriers.
template <int ROLE>
__device__ __forceinline__ void kv_wave(const KvParams& P, char* smem, int seg, int h, int cs, int L,
                                        int p, int k0) {
  using namespace kv;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = w & (NPAIR - 1);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int kA = k0 + KP * j;          // first key (local index) of this pair
  const int key = kA + l32;            // this lane's key

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(P.q + cs * P.q_st + h * P.q_sh, rows_bytes(L, P.q_st, D));
  const __amdgpu_buffer_rsrc_t dor = make_rsrc(P.dout + cs * P.do_st + h * P.do_sh, rows_bytes(L, P.do_st, D));
  const __amdgpu_buffer_rsrc_t lser = make_rsrc(P.lse + (int64_t)h * P.T + cs, (uint32_t)L * 4);
  const __amdgpu_buffer_rsrc_t dltr = make_rsrc(P.delta + (int64_t)h * P.T + cs, (uint32_t)L * 4);
  const uint32_t qst2 = (uint32_t)P.q_st * 2, dost2 = (uint32_t)P.do_st * 2;
  const float s_do = pow2_scale(P.stats[h * kStats + 0]);   // max |dO|
  float* segst = P.segstats + ((int64_t)seg * P.H + h) * kSegStats;
  float* red = reinterpret_cast<float*>(smem + OFF_RED);

  const int qstart = (k0 < p) ? 0 : k0;
  const int nq = (L - qstart + BQ - 1) / BQ;

  // staging of a query tile: thread = 16-byte chunk sch of rows srow + SROWS*k;
  // tile i+1 is loaded at the start of iteration i and stored at its end
  constexpr int SROWS = NT / 16, SPASS = BQ / SROWS;
  static_assert(SPASS >= 1 && SPASS * SROWS == BQ, "staging covers the query tile exactly");
  const int srow = tid >> 4, sch = tid & 15;
  char* stage_base = smem + srow * RS + sch * 16;
  u32x4 sq[SPASS], sd[SPASS];
  float s_lse = 0.f, s_dlt = 0.f;
  auto load_tile = [&](int qi) {
#pragma unroll
    for (int k = 0; k < SPASS; ++k) {
      sq[k] = buf_load16(qr, (uint32_t)(qi + srow + SROWS * k) * qst2 + sch * 16);
      sd[k] = buf_load16(dor, (uint32_t)(qi + srow + SROWS * k) * dost2 + sch * 16);
    }
    s_lse = buf_loadf(lser, (uint32_t)(qi + (tid & (BQ - 1))) * 4);
    s_dlt = buf_loadf(dltr, (uint32_t)(qi + (tid & (BQ - 1))) * 4);
  };
  // the first query tile's loads overlap the K/V row loads and the maxima below
  load_tile(qstart);

  // stationary operand: B[k = d 16s+8hh+i][col = key l32] of S = Q K^T (role A) or
  // of dP = dO V^T (role B, fp16 scaled by a per-workgroup power of two)
  u32x4 kv_op[8];
  {
    const __amdgpu_buffer_rsrc_t r =
        ROLE == 0 ? make_rsrc(P.k + cs * P.k_st + h * P.k_sh, rows_bytes(L, P.k_st, D))
                  : make_rsrc(P.v + cs * P.v_st + h * P.v_sh, rows_bytes(L, P.v_st, D));
    const uint32_t st2 = (uint32_t)(ROLE == 0 ? P.k_st : P.v_st) * 2;
#pragma unroll
    for (int s = 0; s < 8; ++s) kv_op[s] = buf_load16(r, (uint32_t)key * st2 + (16 * s + 8 * hh) * 2);
    float m = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16lo(kv_op[s][e]), x1 = bf16hi(kv_op[s][e]);
        if (ROLE == 0)
          m = fmaxf(m, fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1)));
        else
          m += x0 * x0 + x1 * x1;
      }
    if (ROLE == 1) m = __builtin_sqrtf(m + __shfl_xor(m, 32));   // ||V_key||
    m = wave_max(m);
    if (lane == 0) {
      atomic_max_nonneg(segst + ROLE, m);
      if (ROLE == 1) red[j] = m;
    }
  }
  __syncthreads();   // per-pair maxima of ||V|| visible
  float vmax = 0.f;
#pragma unroll
  for (int i = 0; i < NPAIR; ++i) vmax = fmaxf(vmax, red[i]);
  const float s_v = pow2_scale(vmax);
  // dP is accumulated scaled by s_dp = s_do * s_v, starting from -delta * s_dp
  const float s_dp = s_do * s_v;
  if (ROLE == 1) {
#pragma unroll
    for (int s = 0; s < 8; ++s) kv_op[s] = __builtin_bit_cast(u32x4, bf16x8_to_f16_scaled(kv_op[s], s_v));
  }

  f32x16 acc[4];   // dV^T (role A) or s_dp * dK^T (role B): [d 32dt + row][key l32]
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

  auto store_tile = [&](int tb, int lb) {   // tb: tile buffer 0..2, lb: lse/delta buffer 0..1
#pragma unroll
    for (int k = 0; k < SPASS; ++k) {
      *reinterpret_cast<u32x4*>(stage_base + OFF_QS + tb * TILE + SROWS * k * RS) = sq[k];
      *reinterpret_cast<f16x8*>(stage_base + OFF_DOS + tb * TILE + SROWS * k * RS) = bf16x8_to_f16_scaled(sd[k], s_do);
    }
    if (tid < BQ)
      reinterpret_cast<float*>(smem + OFF_LSE)[lb * BQ + tid] = s_lse * kLog2e;
    else if (tid < 2 * BQ)
      reinterpret_cast<float*>(smem + OFF_DLT)[lb * BQ + tid - BQ] = -s_dlt * s_dp;
  };

  // query row qrow sees this lane's key iff qrow >= thr. Rows at or past L need no
  // mask: their Q, dO, lse and delta read as 0, so P = 1, dP = 0, dS = 0 and
  // dO^T P adds 0 to dV.
  const int thr = key < p ? -(1 << 30) : (key < L ? key : (1 << 30));
  const float c = P.scale_log2;
  const int pex_lane = OFF_PEX + j * 2048 + lane * 16;
  const char* row_base = smem + l32 * RS + hh * 16;   // A operand rows: row l32, d 16s + 8hh
  const char* xt_base = smem + xt_lane_off(lane);
  const float* lse_base = reinterpret_cast<const float*>(smem + OFF_LSE) + 4 * hh;
  const float* dlt_base = reinterpret_cast<const float*>(smem + OFF_DLT) + 4 * hh;

  // The pair is software-pipelined by one query tile, with one workgroup barrier per
  // iteration. In iteration i, wave A issues dV(i-1) interleaved with S(i), then
  // forms P(i) and publishes it; wave B forms dS(i-1) from P(i-1) and its dP(i-1)
  // accumulator, then issues dK(i-1) interleaved with dP(i). Tiles i-1, i, i+1 live
  // in three LDS buffers; iteration nq only drains tile nq-1.
  f16x8 pb_prev[2];    // role A: P of tile i-1 (B operand of dV)
  f32x16 x_prev;       // role B: s_dp (dP - delta) of tile i-1
  bool seen_prev = false;
  int b_cur = 0, b_prev = 2, b_next = 1;   // tile buffers of tiles i, i-1, i+1

  store_tile(0, 0);
  for (int iq = 0; iq <= nq; ++iq) {
    const int qi = qstart + iq * BQ;
    const int lb = iq & 1;
    __syncthreads();   // tile iq and P(iq-1) visible; buffers of tile iq-2 and P(iq-2) free
    if (iq + 1 < nq) load_tile(qi + BQ);
    // some (query, key) pair of tile iq is allowed for this pair's keys
    const bool seen = iq < nq && kA < L && (kA < p || qi + BQ > kA);
    const int q_cur = OFF_QS + b_cur * TILE, q_prev = OFF_QS + b_prev * TILE;
    const int o_cur = OFF_DOS + b_cur * TILE, o_prev = OFF_DOS + b_prev * TILE;
    if (ROLE == 0) {
      // ---- dV(i-1) MFMAs interleaved with S(i) = Q K^T ------------------------------
      // (CUR: tile i is seen, PRV: tile i-1 was; chosen once per iteration so the
      // MFMA sequence itself has no branches)
      f32x16 xacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) xacc[r] = 0.f;
      auto mfma_phase = [&](auto cur, auto prv) {
        constexpr bool CUR = decltype(cur)::value, PRV = decltype(prv)::value;
        bf16x8 qa[8];
        u32x4 xt[4][2];
        if constexpr (CUR) {
#pragma unroll
          for (int s = 0; s < 3; ++s) qa[s] = *reinterpret_cast<const bf16x8*>(row_base + q_cur + 32 * s);
        }
        if constexpr (PRV) {
#pragma unroll
          for (int i = 0; i < 2; ++i) xt[i >> 1][i & 1] = lds_read_xt(xt_base + o_prev, i & 1, i >> 1);
        }
        sched_fence();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if constexpr (CUR) {
            if (s + 3 < 8) qa[s + 3] = *reinterpret_cast<const bf16x8*>(row_base + q_cur + 32 * (s + 3));
          }
          if constexpr (PRV) {
            if (s + 2 < 8) xt[(s + 2) >> 1][(s + 2) & 1] = lds_read_xt(xt_base + o_prev, (s + 2) & 1, (s + 2) >> 1);
          }
          sched_fence();
          if constexpr (CUR) xacc = mfma32x32x16(qa[s], __builtin_bit_cast(bf16x8, kv_op[s]), xacc);
          if constexpr (PRV)   // dV^T[d][key] += dO^T[d][q] P[q][key]
            acc[s >> 1] = mfma32x32x16_f16(__builtin_bit_cast(f16x8, xt[s >> 1][s & 1]), pb_prev[s & 1], acc[s >> 1]);
          sched_fence();
        }
      };
      if (seen) {
        if (seen_prev)
          mfma_phase(std::true_type(), std::true_type());
        else
          mfma_phase(std::true_type(), std::false_type());
      } else if (seen_prev) {
        mfma_phase(std::false_type(), std::true_type());
      }
      // ---- P(i) = exp2(S c - lse2), published for wave B ------------------------------
      if (seen) {
        f32x4 l4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) l4[m] = *reinterpret_cast<const f32x4*>(lse_base + lb * BQ + 8 * m);
        float pv[16];
        if (kA + KP <= L && (kA + KP <= p || kA + KP - 1 <= qi)) {   // every pair allowed
#pragma unroll
          for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(xacc[r], c, -l4[r >> 2][r & 3]));
        } else {
          const int tq = thr - qi - 4 * hh;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(xacc[r], c, -l4[r >> 2][r & 3]));
            pv[r] = (8 * (r >> 2) + (r & 3) >= tq) ? e : 0.f;
          }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          pb_prev[t] = cvt8h(pv[8 * t], pv[8 * t + 1], pv[8 * t + 2], pv[8 * t + 3], pv[8 * t + 4], pv[8 * t + 5],
                             pv[8 * t + 6], pv[8 * t + 7]);
          *reinterpret_cast<f16x8*>(smem + pex_lane + lb * PEX_BUF + t * 1024) = pb_prev[t];
        }
      }
    } else {
      // ---- dS(i-1) = P(i-1) * x_prev, then dK(i-1) interleaved with dP(i) -------------
      auto mfma_phase = [&](auto cur, auto prv) {
        constexpr bool CUR = decltype(cur)::value, PRV = decltype(prv)::value;
        f32x16 xnew;     // s_dp (dP - delta) of tile i, starting at -delta * s_dp
        f16x8 oa[8];
        u32x4 xt[4][2];
        bf16x8 db[2];
        if constexpr (CUR) {
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dlt_base + lb * BQ + 8 * m);
#pragma unroll
            for (int i = 0; i < 4; ++i) xnew[4 * m + i] = d4[i];
          }
#pragma unroll
          for (int s = 0; s < 3; ++s) oa[s] = *reinterpret_cast<const f16x8*>(row_base + o_cur + 32 * s);
        }
        if constexpr (PRV) {
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const f16x8 pe = *reinterpret_cast<const f16x8*>(smem + pex_lane + (lb ^ 1) * PEX_BUF + t * 1024);
            float ds[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) ds[i] = __builtin_fmaf((float)pe[i], x_prev[8 * t + i], 0.f);
            db[t] = cvt8(ds[0], ds[1], ds[2], ds[3], ds[4], ds[5], ds[6], ds[7]);
          }
#pragma unroll
          for (int i = 0; i < 2; ++i) xt[i >> 1][i & 1] = lds_read_xt(xt_base + q_prev, i & 1, i >> 1);
        }
        sched_fence();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if constexpr (CUR) {
            if (s + 3 < 8) oa[s + 3] = *reinterpret_cast<const f16x8*>(row_base + o_cur + 32 * (s + 3));
          }
          if constexpr (PRV) {
            if (s + 2 < 8) xt[(s + 2) >> 1][(s + 2) & 1] = lds_read_xt(xt_base + q_prev, (s + 2) & 1, (s + 2) >> 1);
          }
          sched_fence();
          if constexpr (CUR) xnew = mfma32x32x16_f16(oa[s], __builtin_bit_cast(f16x8, kv_op[s]), xnew);
          if constexpr (PRV)   // s_dp dK^T[d][key] += Q^T[d][q] (s_dp dS)[q][key]
            acc[s >> 1] = mfma32x32x16(__builtin_bit_cast(bf16x8, xt[s >> 1][s & 1]), db[s & 1], acc[s >> 1]);
          sched_fence();
        }
        if constexpr (CUR) x_prev = xnew;
      };
      if (seen) {
        if (seen_prev)
          mfma_phase(std::true_type(), std::true_type());
        else
          mfma_phase(std::true_type(), std::false_type());
      } else if (seen_prev) {
        mfma_phase(std::false_type(), std::true_type());
      }
    }
    seen_prev = seen;
    // tile iq+1 into buffer b_next: it held tile iq-2, last read before this barrier
    if (iq + 1 < nq) store_tile(b_next, lb ^ 1);
    b_prev = b_cur;
    b_cur = b_next;
    b_next = b_next == 2 ? 0 : b_next + 1;
  }

  // dV = acc / s_do, dK = scale * acc / s_dp, rows staged through LDS (free after this
  // barrier)
  __syncthreads();
  {
    static_assert(NT / 64 * OUT_WAVE_BYTES <= LDS_BYTES, "output staging fits in LDS");
    const __amdgpu_buffer_rsrc_t outr =
        ROLE == 0 ? make_rsrc(P.dv + cs * P.dv_st + h * P.dv_sh, rows_bytes(L, P.dv_st, D))
                  : make_rsrc(P.dk + cs * P.dk_st + h * P.dk_sh, rows_bytes(L, P.dk_st, D));
    const uint32_t st2 = (uint32_t)(ROLE == 0 ? P.dv_st : P.dk_st) * 2;
    store_rows_via_lds(acc, ROLE == 0 ? 1.f / s_do : P.scale / s_dp, smem + w * OUT_WAVE_BYTES, outr, kA, st2,
                       lane);
  }
}

// Work item = (segment, 128-key tile, head).
__global__ __launch_bounds__(kv::NT, 1) void prefixlm_bwd_dkdv_kernel(KvParams P) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int item = blockIdx.x / P.H;
  const int h = blockIdx.x - item * P.H;
  if (item >= P.hdr->n_items) return;
  const int2 it = P.items[item];
  const int seg = it.x;
  if (seg < 0 || seg >= P.numseqs) return;
  const int cs = P.cu[seg];
  const int L = P.prefix[seg] + P.causal[seg];
  const int p = P.is_causal ? 0 : P.prefix[seg];
  const int k0 = it.y * kv::BK;
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < kv::NPAIR)
    kv_wave<0>(P, smem, seg, h, cs, L, p, k0);
  else
    kv_wave<1>(P, smem, seg, h, cs, L, p, k0);
}

// =====================================================================================
// dQ
// =====================================================================================
namespace qk {
constexpr int BQ = 128;                // queries per workgroup (32 per wave)
constexpr int BKT = 32;                // keys per tile
constexpr int NT = (BQ / 32) * 64;
constexpr int TILE = BKT * RS;
constexpr int OFF_KS = 0;              // [2] tiles: fp16 K * s_k
constexpr int OFF_VS = 2 * TILE;       // [2] tiles: bf16 V
constexpr int LDS_BYTES = 4 * TILE;
}  // namespace qk

struct QParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* dout;
  const float* lse;
  const float* delta;
  const float* segstats;   // [numseqs, H, kSegStats] from the dK/dV kernel
  bf16* dq;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, do_st, do_sh, dq_st, dq_sh;
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  const int2* items;
  const WsHeader* hdr;
  int T, H, is_causal;
  int numseqs;
  float scale_log2;
  float scale;
};

// Work item = (segment, 128-query tile, head). Wave w owns queries q0+32w..+31:
// Q (fp16, scaled) and dO (bf16) stay in registers as B operands of S^T = K Q^T and
// dP^T = V dO^T (key = accumulator row, query = lane column), so each lane's query
// needs one lse and one delta. dS^T goes straight from the accumulator registers
// into the B operand of dQ^T += K^T dS^T, whose A operand is read transposed from
// the K tile.
__global__ __launch_bounds__(qk::NT, 2) void prefixlm_bwd_dq_kernel(QParams P) {
  using namespace qk;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int item = blockIdx.x / P.H;
  const int h = blockIdx.x - item * P.H;
  if (item >= P.hdr->n_items) return;
  const int2 it = P.items[item];
  const int seg = it.x;
  if (seg < 0 || seg >= P.numseqs) return;
  const int cs = P.cu[seg];
  const int L = P.prefix[seg] + P.causal[seg];
  const int p = P.is_causal ? 0 : P.prefix[seg];
  const int q0 = it.y * BQ;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int qA = q0 + 32 * w;
  const int qrow = qA + l32;

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(P.q + cs * P.q_st + h * P.q_sh, rows_bytes(L, P.q_st, D));
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(P.k + cs * P.k_st + h * P.k_sh, rows_bytes(L, P.k_st, D));
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(P.v + cs * P.v_st + h * P.v_sh, rows_bytes(L, P.v_st, D));
  const __amdgpu_buffer_rsrc_t dor = make_rsrc(P.dout + cs * P.do_st + h * P.do_sh, rows_bytes(L, P.do_st, D));
  const __amdgpu_buffer_rsrc_t lser = make_rsrc(P.lse + (int64_t)h * P.T + cs, (uint32_t)L * 4);
  const __amdgpu_buffer_rsrc_t dltr = make_rsrc(P.delta + (int64_t)h * P.T + cs, (uint32_t)L * 4);
  const uint32_t kst2 = (uint32_t)P.k_st * 2, vst2 = (uint32_t)P.v_st * 2;

  // per-lane query operands: B[k = d 16s+8hh+i][col = query l32]
  u32x4 qf[8], dof[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    qf[s] = buf_load16(qr, (uint32_t)qrow * (uint32_t)P.q_st * 2 + (16 * s + 8 * hh) * 2);
    dof[s] = buf_load16(dor, (uint32_t)qrow * (uint32_t)P.do_st * 2 + (16 * s + 8 * hh) * 2);
  }
  const float lse2 = buf_loadf(lser, (uint32_t)qrow * 4) * kLog2e;
  const float dlt = buf_loadf(dltr, (uint32_t)qrow * 4);
  const float* segst = P.segstats + ((int64_t)seg * P.H + h) * kSegStats;
  const float s_k = pow2_scale(segst[0]);
  float s_q, s_ds;
  {
    float qm = 0.f, dss = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qm = fmaxf(qm, fmaxf(__builtin_fabsf(bf16lo(qf[s][e])), __builtin_fabsf(bf16hi(qf[s][e]))));
        const float d0 = bf16lo(dof[s][e]), d1 = bf16hi(dof[s][e]);
        dss += d0 * d0 + d1 * d1;
      }
    const float dnorm = __builtin_sqrtf(dss + __shfl_xor(dss, 32));
    s_q = pow2_scale(wave_max(qm));
    // |dS| <= P (||dO_q|| ||V_k|| + |delta_q|) <= ||dO_q|| max||V|| + |delta_q|
    s_ds = pow2_scale(wave_max(dnorm * segst[1] + __builtin_fabsf(dlt)));
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(u32x4, bf16x8_to_f16_scaled(qf[s], s_q));
  const float cq = P.scale_log2 / (s_q * s_k);
  // P * s_ds = exp2(S c - lse2 + log2 s_ds); s_ds is a power of two
  const float lse2s = lse2 - __builtin_log2f(s_ds);

  f32x16 acc[4];   // s_ds s_k dQ^T: [d 32dt + 8(r/4)+4hh+r%4][query l32]
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

  // keys [0, kend) are seen by some query of the workgroup; [0, kw) by this wave
  const int kend = max(p, min(L, q0 + BQ));
  const int kw = max(p, min(L, qA + 32));
  const int nk = (kend + BKT - 1) / BKT;
  // this lane's query sees keys [0, kq); every query of the wave sees [0, kfull)
  const int kq = min(L, max(p, qrow + 1));
  const int kfull = min(L, max(p, qA + 1));

  // staging: thread = 16-byte chunk sch of rows srow + SROWS*k of the K and V tiles
  constexpr int SROWS = NT / 16, SPASS = BKT / SROWS;
  static_assert(SPASS >= 1 && SPASS * SROWS == BKT, "staging covers the key tile exactly");
  const int srow = tid >> 4, sch = tid & 15;
  char* stage_base = smem + srow * RS + sch * 16;
  u32x4 sk[SPASS], sv[SPASS];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int k = 0; k < SPASS; ++k) {
      sk[k] = buf_load16(kr, (uint32_t)(k0 + srow + SROWS * k) * kst2 + sch * 16);
      sv[k] = buf_load16(vr, (uint32_t)(k0 + srow + SROWS * k) * vst2 + sch * 16);
    }
  };
  auto store_tile = [&](int b) {
#pragma unroll
    for (int k = 0; k < SPASS; ++k) {
      *reinterpret_cast<f16x8*>(stage_base + OFF_KS + b * TILE + SROWS * k * RS) = bf16x8_to_f16_scaled(sk[k], s_k);
      *reinterpret_cast<u32x4*>(stage_base + OFF_VS + b * TILE + SROWS * k * RS) = sv[k];
    }
  };
  const char* row_base = smem + l32 * RS + hh * 16;   // A operand rows: key row l32, d 16s + 8hh
  const char* xt_base = smem + xt_lane_off(lane);

  load_tile(0);
  store_tile(0);
  for (int ik = 0; ik < nk; ++ik) {
    const int B = ik & 1;
    const int kt0 = ik * BKT;
    __syncthreads();   // K/V tile ik visible in buffer B
    if (ik + 1 < nk) load_tile(kt0 + BKT);
    if (kt0 < kw) {
      f32x16 sacc, pacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[r] = 0.f;
        pacc[r] = 0.f;
      }
      // S^T = K Q^T (fp16, scaled by s_k s_q), dP^T = V dO^T (bf16); K and V rows two
      // steps ahead of the MFMAs that use them
      f16x8 ka[8];
      bf16x8 va[8];
      auto rd = [&](int s) {
        ka[s] = *reinterpret_cast<const f16x8*>(row_base + OFF_KS + B * TILE + 32 * s);
        va[s] = *reinterpret_cast<const bf16x8*>(row_base + OFF_VS + B * TILE + 32 * s);
      };
      rd(0);
      rd(1);
      sched_fence();
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (s + 2 < 8) rd(s + 2);
        sched_fence();
        sacc = mfma32x32x16_f16(ka[s], __builtin_bit_cast(f16x8, qf[s]), sacc);
        pacc = mfma32x32x16(va[s], __builtin_bit_cast(bf16x8, dof[s]), pacc);
        sched_fence();
      }
      // transposed K operands of the dQ step, in flight during the elementwise math
      u32x4 xt[4][2];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int t = 0; t < 2; ++t) xt[dt][t] = lds_read_xt(xt_base + OFF_KS + B * TILE, t, dt);
      sched_fence();
      // s_ds dS^T[key][q] = s_ds P (dP - delta), key = kt0 + 8(r/4) + 4hh + r%4
      float ds[16];
      if (kt0 + BKT <= kfull) {   // every key of the tile is seen by every query
#pragma unroll
        for (int r = 0; r < 16; ++r)
          ds[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], cq, -lse2s)) * (pacc[r] - dlt);
      } else {
        const int tk = kq - kt0 - 4 * hh;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], cq, -lse2s));
          ds[r] = (8 * (r >> 2) + (r & 3) < tk) ? e * (pacc[r] - dlt) : 0.f;
        }
      }
      f16x8 db[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        db[t] = cvt8h(ds[8 * t], ds[8 * t + 1], ds[8 * t + 2], ds[8 * t + 3], ds[8 * t + 4], ds[8 * t + 5],
                      ds[8 * t + 6], ds[8 * t + 7]);
      sched_fence();
      // dQ^T[d][q] += K^T[d][key] dS^T[key][q]
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          acc[dt] = mfma32x32x16_f16(__builtin_bit_cast(f16x8, xt[dt][t]), db[t], acc[dt]);
    }
    // tile ik+1 into the other buffer: tile ik-1 there was last read before this
    // iteration's barrier
    if (ik + 1 < nk) store_tile(B ^ 1);
  }

  // dq = scale * acc / (s_ds s_k), rows staged through LDS (free after this barrier)
  __syncthreads();
  {
    static_assert(NT / 64 * OUT_WAVE_BYTES <= LDS_BYTES, "output staging fits in LDS");
    const __amdgpu_buffer_rsrc_t dqr = make_rsrc(P.dq + cs * P.dq_st + h * P.dq_sh, rows_bytes(L, P.dq_st, D));
    store_rows_via_lds(acc, P.scale / (s_ds * s_k), smem + w * OUT_WAVE_BYTES, dqr, qA, (uint32_t)P.dq_st * 2,
                       lane);
  }
}

// =====================================================================================
// pre-pass and padding rows
// =====================================================================================
constexpr int kPreRows = 32;     // token rows per pre-pass workgroup
constexpr int kPreBatch = 8;     // row-heads per 16-lane group whose loads are in flight together
constexpr int kPreMaxHeads = 64; // per-head maxima kept in LDS

// delta[h, t] = sum_d dO[t,h,d] * (O + O_lo)[t,h,d] for t < total (0 for the other
// rows of the workgroup's range) and the per-head maxima max|dO|, max ||dO_t||_2
// and max |delta_t| (atomicMax on the bit patterns of non-negative floats; `stats`
// must be zero on entry). A 16-lane group reduces one (row, head) at a time; the
// maxima are combined in LDS first so each workgroup issues 3 global atomics per
// head. Rows past total read as zero through the buffer bounds.
//
// Optional output gate of the attention layer (models/layers.py:154), whose
// backward runs here: with y = sigmoid(gate) * o the kernel reads dy (passed as
// dout) and the gate, and writes dO = dy * s and dgate = (dy * o) * (1 - s) * s,
// s = sigmoid(gate) in bf16, each rounded to bf16 as autograd rounds them for bf16
// tensors. dO goes to dout_attn, which the dK/dV and dQ kernels then read as dout.
struct GateBwd {
  const bf16* gate;
  bf16* dgate;
  bf16* dout_attn;
  int64_t g_st, g_sh, dg_st, dg_sh, da_st, da_sh;
};

template <bool GATED>
__global__ __launch_bounds__(256) void prefixlm_bwd_pre_kernel(
    const bf16* o, const bf16* o_lo, const bf16* dout, int64_t o_st, int64_t o_sh, int64_t lo_st,
    int64_t lo_sh, int64_t do_st, int64_t do_sh, float* delta, float* stats, int T, int H, int total,
    GateBwd G) {
  __shared__ int smax[kPreMaxHeads * 3];
  const int t0 = blockIdx.x * kPreRows;
  const int rows = min(kPreRows, T - t0);
  const int tid = threadIdx.x;
  const int grp = tid >> 4, chunk = tid & 15;
  for (int i = tid; i < H * 3; i += 256) smax[i] = 0;
  __syncthreads();
  const int vrows = max(0, min(rows, total - t0));   // rows of this range below total
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(o + t0 * o_st, rows_bytes(vrows, o_st, (int)((H - 1) * o_sh + D)));
  const __amdgpu_buffer_rsrc_t lor =
      make_rsrc(o_lo ? o_lo + t0 * lo_st : o, o_lo ? rows_bytes(vrows, lo_st, (int)((H - 1) * lo_sh + D)) : 0u);
  const __amdgpu_buffer_rsrc_t dor = make_rsrc(dout + t0 * do_st, rows_bytes(vrows, do_st, (int)((H - 1) * do_sh + D)));
  __amdgpu_buffer_rsrc_t gr = orr, dgr = orr, dar = orr;
  if constexpr (GATED) {
    gr = make_rsrc(G.gate + t0 * G.g_st, rows_bytes(vrows, G.g_st, (int)((H - 1) * G.g_sh + D)));
    // dgate and dO are written for every row of the range: 0 at rows >= total
    dgr = make_rsrc(G.dgate + t0 * G.dg_st, rows_bytes(rows, G.dg_st, (int)((H - 1) * G.dg_sh + D)));
    dar = make_rsrc(G.dout_attn + t0 * G.da_st, rows_bytes(rows, G.da_st, (int)((H - 1) * G.da_sh + D)));
  }
  const int n = rows * H;   // (row, head) pairs of this workgroup, head fastest
  for (int base = grp; base < n; base += 16 * kPreBatch) {
    u32x4 a[kPreBatch], b[kPreBatch], r[kPreBatch], gg[kPreBatch];
#pragma unroll
    for (int j = 0; j < kPreBatch; ++j) {
      const int idx = min(base + 16 * j, n - 1);
      const int t = idx / H, h = idx - t * H;
      a[j] = buf_load16(orr, (uint32_t)((t * o_st + h * o_sh + chunk * 8) * 2));
      b[j] = buf_load16(dor, (uint32_t)((t * do_st + h * do_sh + chunk * 8) * 2));
      r[j] = buf_load16(lor, (uint32_t)((t * lo_st + h * lo_sh + chunk * 8) * 2));
      if constexpr (GATED) gg[j] = buf_load16(gr, (uint32_t)((t * G.g_st + h * G.g_sh + chunk * 8) * 2));
    }
#pragma unroll
    for (int j = 0; j < kPreBatch; ++j) {
      const int idx = base + 16 * j;
      if constexpr (GATED) {
        // b[j] holds dy; replace it by dO = bf16(dy * s) and write dgate
        float dov[8], dgv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const float dy = half ? bf16hi(b[j][i]) : bf16lo(b[j][i]);
            const float ov = half ? bf16hi(a[j][i]) : bf16lo(a[j][i]);
            const float s = sigmoid_bf16(half ? bf16hi(gg[j][i]) : bf16lo(gg[j][i]));
            dov[2 * i + half] = dy * s;
            const float ds = (float)(bf16)(dy * ov);
            dgv[2 * i + half] = ds * (1.f - s) * s;
          }
        }
        b[j] = __builtin_bit_cast(u32x4, cvt8(dov[0], dov[1], dov[2], dov[3], dov[4], dov[5], dov[6], dov[7]));
        if (idx < n) {
          const int t = idx / H, h = idx - t * H;
          buf_store16(b[j], dar, (uint32_t)((t * G.da_st + h * G.da_sh + chunk * 8) * 2));
          buf_store16(__builtin_bit_cast(u32x4, cvt8(dgv[0], dgv[1], dgv[2], dgv[3], dgv[4], dgv[5], dgv[6], dgv[7])),
                      dgr, (uint32_t)((t * G.dg_st + h * G.dg_sh + chunk * 8) * 2));
        }
      }
      float dot = 0.f, ss = 0.f, ma = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float o0 = bf16lo(a[j][i]) + bf16lo(r[j][i]), o1 = bf16hi(a[j][i]) + bf16hi(r[j][i]);
        const float d0 = bf16lo(b[j][i]), d1 = bf16hi(b[j][i]);
        dot += o0 * d0 + o1 * d1;
        ss += d0 * d0 + d1 * d1;
        ma = fmaxf(ma, fmaxf(__builtin_fabsf(d0), __builtin_fabsf(d1)));
      }
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) {
        dot += __shfl_xor(dot, m);
        ss += __shfl_xor(ss, m);
        ma = fmaxf(ma, __shfl_xor(ma, m));
      }
      if (chunk == 0 && idx < n) {
        const int t = idx / H, h = idx - t * H;
        delta[(int64_t)h * T + t0 + t] = dot;
        atomicMax(&smax[h * 3 + 0], __builtin_bit_cast(int, ma));
        atomicMax(&smax[h * 3 + 1], __builtin_bit_cast(int, __builtin_sqrtf(ss)));
        atomicMax(&smax[h * 3 + 2], __builtin_bit_cast(int, __builtin_fabsf(dot)));
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < H * 3; i += 256) {
    const int h = i / 3, k = i - h * 3;
    if (smax[i] != 0) atomicMax(reinterpret_cast<int*>(stats + h * kStats + k), smax[i]);
  }
}

// dq = dk = dv = 0 on rows total .. T-1 (one workgroup per row)
__global__ __launch_bounds__(256) void prefixlm_bwd_pad_kernel(bf16* dq, bf16* dk, bf16* dv, int64_t dq_st,
                                                               int64_t dq_sh, int64_t dk_st, int64_t dk_sh,
                                                               int64_t dv_st, int64_t dv_sh, int H, int total) {
  const int64_t t = total + (int64_t)blockIdx.x;
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int idx = threadIdx.x; idx < H * 16; idx += 256) {
    const int h = idx >> 4, chunk = idx & 15;
    *reinterpret_cast<u32x4*>(dq + t * dq_st + h * dq_sh + chunk * 8) = z;
    *reinterpret_cast<u32x4*>(dk + t * dk_st + h * dk_sh + chunk * 8) = z;
    *reinterpret_cast<u32x4*>(dv + t * dv_st + h * dv_sh + chunk * 8) = z;
  }
}

// Zeroes the backward statistics when a host plan replaces the work-list kernel
// (which clears them otherwise).
__global__ __launch_bounds__(256) void zero_floats_kernel(float* p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0.f;
}

}  // namespace bwd
}  // namespace prefixlm
