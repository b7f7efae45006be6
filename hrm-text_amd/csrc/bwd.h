// Backward kernels.
//
// Replaces the two FA3 backward calls and the elementwise epilogue of
// models/flash_attention_prefixlm_v2.py:152-212 (reference):
//   pre  : delta[h,t] = sum_d dO*O (fp32; O = out + its rounding residual when the
//          forward kept one), per-head maxima used to pick exact power-of-two
//          scales, and zeroing of the fp32 dQ accumulator;
//   main : one workgroup = one (segment, 128-key tile, head); each of the 4 waves
//          owns 32 keys, keeps K and V rows in registers and accumulates dK^T / dV^T
//          in fp32 while it walks the 32-row query tiles that see its keys. Per query
//          tile it recomputes S = Q K^T and dP = dO V^T (lane = key column), forms
//          P = exp(S*scale - lse) and dS = P (dP - delta), and issues dV^T += dO^T P and
//          dK^T += Q^T dS. dS goes through LDS so that each wave can then form the dQ
//          columns [32w, 32w+32) over all 128 keys of the workgroup, which are added
//          to the fp32 accumulator with one atomic per element;
//   post : dq = bf16(scale * acc); dk, dv rows >= total_seqlen are zeroed.
// The reference's dk1 + dk2 / dv1 + dv2 (:212) disappears: each key row is owned by
// exactly one workgroup, which sees both the prefix rows and the suffix rows.
//
// Precision: S and dP contract bf16 inputs over D (exact products, fp32 sums). The
// dV product uses fp16 P (P lies in [0, 1]) and fp16 dO scaled by a per-head power
// of two; the dQ product uses fp16 dS and fp16 K, each scaled by a per-workgroup
// power of two chosen from a bound on its magnitude. fp16 keeps 3 more mantissa bits
// than bf16 and the power-of-two scales are undone exactly in fp32. dK uses bf16 dS
// and Q (its error budget is met without it).
#pragma once
#include "common.h"

namespace prefixlm {
namespace bwd {

constexpr int D = 128;
constexpr int BK = 128;          // keys per workgroup
constexpr int BQ = 32;           // query rows per inner iteration
constexpr int NT = 256;
constexpr int QS = D + 8;        // Qs / dOs row stride (elements): 272 B
constexpr int QTS = BQ + 8;      // Qt / dOt row stride (elements): 80 B
constexpr int SS = BK + 8;       // dS row stride (elements): 272 B
constexpr int OFF_QS = 0;
constexpr int OFF_DOS = OFF_QS + BQ * QS * 2;
constexpr int OFF_QT = OFF_DOS + BQ * QS * 2;
constexpr int OFF_DOT = OFF_QT + D * QTS * 2;
constexpr int OFF_DS = OFF_DOT + D * QTS * 2;
constexpr int OFF_LSE = OFF_DS + BQ * SS * 2;
constexpr int OFF_DLT = OFF_LSE + BQ * 4;
constexpr int OFF_RED = OFF_DLT + BQ * 4;
constexpr int KTS = BK + 8;      // K^T row stride (elements): 272 B
constexpr int OFF_KT = OFF_RED + 8 * 4;
constexpr int LDS_BYTES = OFF_KT + D * KTS * 2;

constexpr int kStats = 4;   // per head: max|dO|, max ||dO_row||_2, max |delta|, unused

struct Params {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* dout;
  const float* lse;     // [H, T]
  const float* delta;   // [H, T]
  const float* stats;   // [H, kStats]
  float* dq_acc;        // [T, H, D]
  bf16* dk;
  bf16* dv;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, do_st, do_sh, dk_st, dk_sh, dv_st, dv_sh;
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  const int2* items;
  const WsHeader* hdr;
  int T, H, is_causal;
  float scale_log2;     // softmax_scale * log2(e)
  float scale;          // softmax_scale
};

__device__ __forceinline__ bool wave_sees_tile(int kw0, int L, int p, int qi) {
  // keys [kw0, kw0+32) have a query in [qi, qi+BQ) that attends one of them
  return kw0 < L && (kw0 < p || qi + BQ > kw0);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}

__global__ __launch_bounds__(NT, 1) void prefixlm_bwd_kernel(Params P) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  bf16* Qs = reinterpret_cast<bf16*>(smem_raw + OFF_QS);
  bf16* dOs = reinterpret_cast<bf16*>(smem_raw + OFF_DOS);
  bf16* Qt = reinterpret_cast<bf16*>(smem_raw + OFF_QT);
  uint16_t* dOt = reinterpret_cast<uint16_t*>(smem_raw + OFF_DOT);   // fp16, scaled
  uint16_t* dSs = reinterpret_cast<uint16_t*>(smem_raw + OFF_DS);    // fp16, scaled
  float* lse2s = reinterpret_cast<float*>(smem_raw + OFF_LSE);
  float* dlts = reinterpret_cast<float*>(smem_raw + OFF_DLT);
  float* red = reinterpret_cast<float*>(smem_raw + OFF_RED);
  uint16_t* Kt = reinterpret_cast<uint16_t*>(smem_raw + OFF_KT);     // fp16, scaled

  const int item = blockIdx.x / P.H;
  const int h = blockIdx.x - item * P.H;
  if (item >= P.hdr->n_items) return;
  const int2 it = P.items[item];
  const int seg = it.x, kt = it.y;
  const int cs = P.cu[seg];
  const int L = P.prefix[seg] + P.causal[seg];
  const int p = P.is_causal ? 0 : P.prefix[seg];

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int k0 = kt * BK;
  const int kw0 = k0 + 32 * w;
  const bool wave_has_keys = kw0 < L;

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(P.q + cs * P.q_st + h * P.q_sh, rows_bytes(L, P.q_st, D));
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(P.k + cs * P.k_st + h * P.k_sh, rows_bytes(L, P.k_st, D));
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(P.v + cs * P.v_st + h * P.v_sh, rows_bytes(L, P.v_st, D));
  const __amdgpu_buffer_rsrc_t dor = make_rsrc(P.dout + cs * P.do_st + h * P.do_sh, rows_bytes(L, P.do_st, D));
  const __amdgpu_buffer_rsrc_t dkr = make_rsrc(P.dk + cs * P.dk_st + h * P.dk_sh, rows_bytes(L, P.dk_st, D));
  const __amdgpu_buffer_rsrc_t dvr = make_rsrc(P.dv + cs * P.dv_st + h * P.dv_sh, rows_bytes(L, P.dv_st, D));
  const __amdgpu_buffer_rsrc_t lser = make_rsrc(P.lse + (int64_t)h * P.T + cs, (uint32_t)L * 4);
  const __amdgpu_buffer_rsrc_t dltr = make_rsrc(P.delta + (int64_t)h * P.T + cs, (uint32_t)L * 4);
  // fp32 dQ accumulator rows of this segment and head: [L, H, D] with row stride H*D
  const __amdgpu_buffer_rsrc_t dqr =
      make_rsrc(P.dq_acc + ((int64_t)cs * P.H + h) * D,
                L <= 0 ? 0u : (uint32_t)((((int64_t)L - 1) * P.H * D + D) * 4));
  const uint32_t qst2 = (uint32_t)P.q_st * 2, dost2 = (uint32_t)P.do_st * 2, kst2 = (uint32_t)P.k_st * 2;

  // K, V rows of this wave's keys as MFMA B operands: lane = key kw0+l32, d = 16s+8hh+0..7
  bf16x8 kf[8], vf[8];
  {
    const uint32_t koff = (uint32_t)(kw0 + l32) * kst2 + hh * 16;
    const uint32_t voff = (uint32_t)(kw0 + l32) * (uint32_t)P.v_st * 2 + hh * 16;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      kf[s] = __builtin_bit_cast(bf16x8, buf_load16(kr, koff + s * 32));
      vf[s] = __builtin_bit_cast(bf16x8, buf_load16(vr, voff + s * 32));
    }
  }
  // block maxima: ||V_k||_2 and |K| over the workgroup's keys
  {
    float vss = 0.f, kmax = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float vv = (float)vf[s][e];
        vss += vv * vv;
        kmax = fmaxf(kmax, __builtin_fabsf((float)kf[s][e]));
      }
    vss += __shfl_xor(vss, 32);
    const float vn = wave_max(__builtin_sqrtf(vss));
    kmax = wave_max(kmax);
    if (lane == 0) {
      red[w] = vn;
      red[4 + w] = kmax;
    }
  }
  __syncthreads();
  const float vn_blk = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float km_blk = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
  const float st_abs = P.stats[h * kStats + 0];    // max |dO|
  const float st_nrm = P.stats[h * kStats + 1];    // max ||dO_q||_2
  const float st_dlt = P.stats[h * kStats + 2];    // max |delta_q|
  // |dS| = P |dP - delta| <= ||dO_q|| ||V_k|| + |delta_q|
  const float s_do = pow2_scale(st_abs);
  const float s_ds = pow2_scale(st_nrm * vn_blk + st_dlt);
  const float s_k = pow2_scale(km_blk);
  const float dq_unscale = 1.f / (s_ds * s_k);
  // K^T of the workgroup's keys into LDS as fp16 scaled by s_k (read by every
  // wave as the dQ B operand): thread = 4 keys x 8 dims per pass, transposed in
  // registers, 8-byte LDS writes along the key axis
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int g = (tid & 15) + 16 * pass, dc = tid >> 4;
    u32x4 kk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) kk[j] = buf_load16(kr, (uint32_t)(k0 + 4 * g + j) * kst2 + dc * 16);
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      u32x2 lo = {cvt2h_bits(bf16lo(kk[0][e2]) * s_k, bf16lo(kk[1][e2]) * s_k),
                  cvt2h_bits(bf16lo(kk[2][e2]) * s_k, bf16lo(kk[3][e2]) * s_k)};
      u32x2 hi = {cvt2h_bits(bf16hi(kk[0][e2]) * s_k, bf16hi(kk[1][e2]) * s_k),
                  cvt2h_bits(bf16hi(kk[2][e2]) * s_k, bf16hi(kk[3][e2]) * s_k)};
      *reinterpret_cast<u32x2*>(Kt + (8 * dc + 2 * e2) * KTS + 4 * g) = lo;
      *reinterpret_cast<u32x2*>(Kt + (8 * dc + 2 * e2 + 1) * KTS + 4 * g) = hi;
    }
  }

  f32x16 dkacc[4], dvacc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dkacc[t][r] = 0.f;
      dvacc[t][r] = 0.f;
    }

  const int qstart = (k0 < p) ? 0 : (k0 / BQ) * BQ;
  const int nq = (L - qstart + BQ - 1) / BQ;

  // staging of one query tile: thread = rows 4*sg..4*sg+3, dims 4*sdc..4*sdc+3
  const int sg = tid & 7, sdc = tid >> 3;
  u32x2 qstg[4], dostg[4];
  float lse_stg = 0.f, dlt_stg = 0.f;
  auto load_q = [&](int qi) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qstg[j] = buf_load8(qr, (uint32_t)(qi + 4 * sg + j) * qst2 + sdc * 8);
      dostg[j] = buf_load8(dor, (uint32_t)(qi + 4 * sg + j) * dost2 + sdc * 8);
    }
    // every thread loads (rows past the segment read 0); a branch here would make
    // the compiler's vmcnt waits cover the dQ atomics of the previous tile
    lse_stg = buf_loadf(lser, (uint32_t)(qi + (tid & (BQ - 1))) * 4);
    dlt_stg = buf_loadf(dltr, (uint32_t)(qi + (tid & (BQ - 1))) * 4);
  };
  auto store_q = [&]() {
    const int pos = swz23(4 * sg);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<u32x2*>(Qs + (4 * sg + j) * QS + 4 * sdc) = qstg[j];
      *reinterpret_cast<u32x2*>(dOs + (4 * sg + j) * QS + 4 * sdc) = dostg[j];
    }
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2) {
      {
        const uint32_t w0 = qstg[0][e2], w1 = qstg[1][e2], w2 = qstg[2][e2], w3 = qstg[3][e2];
        u32x2 lo = {pack_lo(w0, w1), pack_lo(w2, w3)};
        u32x2 hi = {pack_hi(w0, w1), pack_hi(w2, w3)};
        *reinterpret_cast<u32x2*>(Qt + (4 * sdc + 2 * e2) * QTS + pos) = lo;
        *reinterpret_cast<u32x2*>(Qt + (4 * sdc + 2 * e2 + 1) * QTS + pos) = hi;
      }
      {
        // dO^T as fp16, scaled by s_do
        const uint32_t w0 = dostg[0][e2], w1 = dostg[1][e2], w2 = dostg[2][e2], w3 = dostg[3][e2];
        u32x2 lo = {cvt2h_bits(bf16lo(w0) * s_do, bf16lo(w1) * s_do),
                    cvt2h_bits(bf16lo(w2) * s_do, bf16lo(w3) * s_do)};
        u32x2 hi = {cvt2h_bits(bf16hi(w0) * s_do, bf16hi(w1) * s_do),
                    cvt2h_bits(bf16hi(w2) * s_do, bf16hi(w3) * s_do)};
        *reinterpret_cast<u32x2*>(dOt + (4 * sdc + 2 * e2) * QTS + pos) = lo;
        *reinterpret_cast<u32x2*>(dOt + (4 * sdc + 2 * e2 + 1) * QTS + pos) = hi;
      }
    }
    if (tid < BQ) {
      lse2s[tid] = lse_stg * kLog2e;
      dlts[tid] = dlt_stg;
    }
  };

  const float c = P.scale_log2;
  const int key = kw0 + l32;   // this lane's key (local index)

  // Loop order: barrier A | load tile i+1 | S, dP, P, dS, dV, dK of tile i | dS to LDS |
  // barrier B | dQ MFMAs | tile i+1 into LDS | dQ atomics. gfx9 counts loads and
  // atomics on one counter and the compiler then waits for zero, so the staged loads
  // are consumed before this tile's atomics are issued: the only atomics still in
  // flight at that wait are the previous tile's, issued a full iteration earlier.
  if (nq > 0) {
    load_q(qstart);
    store_q();
  }
  for (int iq = 0; iq < nq; ++iq) {
    const int qi = qstart + iq * BQ;
    __syncthreads();
    if (iq + 1 < nq) load_q(qi + BQ);

    // No branch around the MFMAs: a wave whose keys this query tile does not see
    // masks every element instead (a branch here makes the compiler carry the dK/dV
    // accumulators through PHI nodes in VGPRs and copy them into AGPRs per MFMA).
    // Each phase first issues all of its LDS operand reads into registers, so the
    // MFMAs stream instead of waiting for one read at a time.
    const bool seen = wave_sees_tile(kw0, L, p, qi);
    bf16x8 qa[8], da[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      qa[s] = *reinterpret_cast<const bf16x8*>(Qs + l32 * QS + s * 16 + hh * 8);
      da[s] = *reinterpret_cast<const bf16x8*>(dOs + l32 * QS + s * 16 + hh * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x16 sacc, pacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = 0.f;
      pacc[r] = 0.f;
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      sacc = mfma32x32x16(qa[s], kf[s], sacc);
      pacc = mfma32x32x16(da[s], vf[s], pacc);
    }
    // operands of dV^T += dO^T P and dK^T += Q^T dS, in flight during the softmax math
    f16x8 oa[8];
    bf16x8 ka[8];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        oa[4 * s + t] = *reinterpret_cast<const f16x8*>(dOt + (t * 32 + l32) * QTS + s * 16 + hh * 8);
        ka[4 * s + t] = *reinterpret_cast<const bf16x8*>(Qt + (t * 32 + l32) * QTS + s * 16 + hh * 8);
      }
    f32x4 l4[4], d4[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      l4[g] = *reinterpret_cast<const f32x4*>(lse2s + 8 * g + 4 * hh);
      d4[g] = *reinterpret_cast<const f32x4*>(dlts + 8 * g + 4 * hh);
    }
    const bool full = seen && (qi + BQ <= L) && (kw0 + 32 <= L) && (kw0 + 32 <= max(p, qi + 1));
    float pv[16], dsv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * g + i;
        float pr = __builtin_amdgcn_exp2f(sacc[r] * c - l4[g][i]);
        if (!full) {
          const int qrow = qi + 8 * g + 4 * hh + i;
          const bool ok = seen && (qrow < L) && (key < L) && (key <= qrow || key < p);
          pr = ok ? pr : 0.f;
        }
        pv[r] = pr;
        dsv[r] = pr * (pacc[r] - d4[g][i]);
      }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const f16x8 pb = cvt8h(pv[8 * s], pv[8 * s + 1], pv[8 * s + 2], pv[8 * s + 3], pv[8 * s + 4],
                             pv[8 * s + 5], pv[8 * s + 6], pv[8 * s + 7]);
      const bf16x8 db = cvt8(dsv[8 * s], dsv[8 * s + 1], dsv[8 * s + 2], dsv[8 * s + 3],
                             dsv[8 * s + 4], dsv[8 * s + 5], dsv[8 * s + 6], dsv[8 * s + 7]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        dvacc[t] = mfma32x32x16_f16(oa[4 * s + t], pb, dvacc[t]);
        dkacc[t] = mfma32x32x16(ka[4 * s + t], db, dkacc[t]);
      }
    }
    // dS (fp16, scaled by s_ds) -> LDS as [q][key] (key-contiguous) for the dQ product
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qrow = 8 * (r >> 2) + 4 * hh + (r & 3);
      dSs[qrow * SS + 32 * w + l32] = __builtin_bit_cast(uint16_t, (_Float16)(dsv[r] * s_ds));
    }
    __syncthreads();

    // dQ[:, 32w .. 32w+32) over the workgroup's 128 keys; waves whose keys this tile
    // does not see wrote dS = 0, so no key step needs skipping
    {
      f16x8 sa[8], kb[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        sa[s] = *reinterpret_cast<const f16x8*>(dSs + l32 * SS + s * 16 + hh * 8);
        kb[s] = *reinterpret_cast<const f16x8*>(Kt + (32 * w + l32) * KTS + s * 16 + hh * 8);
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x16 qacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) qacc[r] = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) qacc = mfma32x32x16_f16(sa[s], kb[s], qacc);
      // Q/dO of the next tile can overwrite LDS now: every wave is past barrier B
      if (iq + 1 < nq) store_q();
      // unconditional: wave 0's keys always see the tile (qstart is chosen so), and a
      // branch would make later vmcnt waits conservative. Rows past the segment fall
      // outside the buffer and are dropped.
      {
        const uint32_t rowb = (uint32_t)P.H * D * 4;
        const uint32_t voff = (uint32_t)(qi + 4 * hh) * rowb + (32 * w + l32) * 4;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t roff = (uint32_t)(8 * (r >> 2) + (r & 3)) * rowb;
          __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(qacc[r] * dq_unscale, dqr, voff + roff, 0, 0);
        }
      }
    }
  }

  if (wave_has_keys) {
    const uint32_t kb = (uint32_t)key * (uint32_t)P.dk_st * 2;
    const uint32_t vb = (uint32_t)key * (uint32_t)P.dv_st * 2;
    const float dv_unscale = 1.f / s_do;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = t * 32 + 8 * g + 4 * hh;
        const bf16x4 k4 = cvt4(dkacc[t][4 * g] * P.scale, dkacc[t][4 * g + 1] * P.scale,
                               dkacc[t][4 * g + 2] * P.scale, dkacc[t][4 * g + 3] * P.scale);
        const bf16x4 v4 = cvt4(dvacc[t][4 * g] * dv_unscale, dvacc[t][4 * g + 1] * dv_unscale,
                               dvacc[t][4 * g + 2] * dv_unscale, dvacc[t][4 * g + 3] * dv_unscale);
        buf_store8(__builtin_bit_cast(u32x2, k4), dkr, kb + d0 * 2);
        buf_store8(__builtin_bit_cast(u32x2, v4), dvr, vb + d0 * 2);
      }
  }
}

constexpr int kPreRows = 16;   // token rows per pre-pass workgroup
constexpr int kPreBatch = 4;   // rows whose loads are issued together

// delta[h, t] = sum_d dO[t,h,d] * (O + O_lo)[t,h,d] for t < total (0 past it), the
// per-head maxima max|dO|, max ||dO_t||_2 and max |delta_t| (atomicMax on the bit
// patterns of non-negative floats; `stats` must be zero on entry), and
// dq_acc[t, :, :] = 0. 16 threads per (row, head), one head per 16-thread group;
// the loads of kPreBatch rows are in flight together.
__global__ __launch_bounds__(256) void prefixlm_bwd_pre_kernel(
    const bf16* o, const bf16* o_lo, const bf16* dout, int64_t o_st, int64_t o_sh, int64_t lo_st,
    int64_t lo_sh, int64_t do_st, int64_t do_sh, float* delta, float* stats, float* dq_acc, int T,
    int H, int total) {
  const int t0 = blockIdx.x * kPreRows;
  const int tid = threadIdx.x;
  const int grp = tid >> 4, chunk = tid & 15;
  for (int h = grp; h < H; h += 16) {
    float m_abs = 0.f, m_nrm = 0.f, m_dlt = 0.f;
    for (int tb = t0; tb < t0 + kPreRows; tb += kPreBatch) {
      u32x4 a[kPreBatch], b[kPreBatch], r[kPreBatch];
#pragma unroll
      for (int j = 0; j < kPreBatch; ++j) {
        const int t = tb + j;
        const u32x4 z = {0u, 0u, 0u, 0u};
        a[j] = z;
        b[j] = z;
        r[j] = z;
        if (t < total) {
          a[j] = *reinterpret_cast<const u32x4*>(o + t * o_st + h * o_sh + chunk * 8);
          b[j] = *reinterpret_cast<const u32x4*>(dout + t * do_st + h * do_sh + chunk * 8);
          if (o_lo) r[j] = *reinterpret_cast<const u32x4*>(o_lo + t * lo_st + h * lo_sh + chunk * 8);
        }
      }
#pragma unroll
      for (int j = 0; j < kPreBatch; ++j) {
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
        const int t = tb + j;
        if (chunk == 0 && t < T) delta[(int64_t)h * T + t] = dot;
        m_abs = fmaxf(m_abs, ma);
        m_nrm = fmaxf(m_nrm, ss);
        m_dlt = fmaxf(m_dlt, __builtin_fabsf(dot));
      }
    }
    if (chunk == 0) {
      atomicMax(reinterpret_cast<int*>(stats + h * kStats + 0), __builtin_bit_cast(int, m_abs));
      atomicMax(reinterpret_cast<int*>(stats + h * kStats + 1), __builtin_bit_cast(int, __builtin_sqrtf(m_nrm)));
      atomicMax(reinterpret_cast<int*>(stats + h * kStats + 2), __builtin_bit_cast(int, m_dlt));
    }
  }
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  const int t1 = min(t0 + kPreRows, T);
  f32x4* rows = reinterpret_cast<f32x4*>(dq_acc + (int64_t)t0 * H * D);
  const int n4 = (t1 - t0) * H * D / 4;
  for (int i = tid; i < n4; i += 256) rows[i] = z;
}

// dq = bf16(scale * dq_acc) for every row; dk = dv = 0 on rows >= total.
__global__ __launch_bounds__(256) void prefixlm_bwd_post_kernel(
    const float* dq_acc, bf16* dq, bf16* dk, bf16* dv, int64_t dq_st, int64_t dq_sh, int64_t dk_st,
    int64_t dk_sh, int64_t dv_st, int64_t dv_sh, int T, int H, int total, float scale) {
  const int t = blockIdx.x;
  for (int idx = threadIdx.x; idx < H * 16; idx += 256) {
    const int h = idx >> 4, chunk = idx & 15;
    const f32x4* a = reinterpret_cast<const f32x4*>(dq_acc + ((int64_t)t * H + h) * D + chunk * 8);
    const f32x4 a0 = a[0], a1 = a[1];
    const bf16x8 r = cvt8(a0[0] * scale, a0[1] * scale, a0[2] * scale, a0[3] * scale,
                          a1[0] * scale, a1[1] * scale, a1[2] * scale, a1[3] * scale);
    *reinterpret_cast<bf16x8*>(dq + t * dq_st + h * dq_sh + chunk * 8) = r;
    if (t >= total) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(dk + t * dk_st + h * dk_sh + chunk * 8) = z;
      *reinterpret_cast<u32x4*>(dv + t * dv_st + h * dv_sh + chunk * 8) = z;
    }
  }
}

}  // namespace bwd
}  // namespace prefixlm
