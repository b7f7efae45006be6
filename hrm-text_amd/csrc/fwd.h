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
//   * K and V tiles (32 keys) are staged row-major in LDS (padded rows, V's
//     permuted within 16-row blocks for conflict-free transposing reads; double
//     buffered, 128-bit buffer loads one tile ahead); V^T, the A operand of
//     O^T += V^T P^T, is read with transposing LDS reads whose key order matches the
//     row order of the S^T accumulator, so P^T goes from accumulator to operand in
//     place;
//   * O^T accumulates in 4 32x32 fp32 tiles. O is rescaled only on tiles where some
//     lane's running max rises (decided per wave); the max stays exact, so the largest
//     P of a row is exactly 1 and survives the bf16 rounding of P;
//   * O and its rounding residual leave through LDS as whole 256-byte rows.
#pragma once
#include <type_traits>

#include "common.h"

namespace prefixlm {
namespace fwd {

#ifndef PREFIXLM_FWD_BM
#define PREFIXLM_FWD_BM 128
#endif
constexpr int BM = PREFIXLM_FWD_BM;   // query rows per workgroup (32 per wave)
constexpr int BN = 32;           // keys per inner iteration
constexpr int NT = BM / 32 * 64;   // threads

// Tile geometry for head dim HD (128 or 64).
template <int HD>
struct Geo {
  // LDS row stride: the row's bytes + 48, so consecutive rows start 12 banks apart
  // (304 bytes for 128 columns, 176 for 64): the 16 rows of a ds_read_b128 cycle cover
  // all 64 banks, and the permuted V rows a transposing cycle reads (4 rows apart)
  // start 48 banks apart
  static constexpr int RS = 2 * HD + 48;
  static constexpr int CPR = HD / 8;          // 16-byte chunks per row
  static constexpr int SROWS = NT / CPR;      // staging: rows per pass
  static constexpr int SPASS = BN / SROWS;
  static constexpr int TILE = BN * RS;        // one BN x HD 16-bit tile
  static constexpr int OFF_K = 0;             // [2] K tiles
  static constexpr int OFF_V = 2 * TILE;      // [2] V tiles
  static constexpr int LDS_BYTES = 4 * TILE;
  static constexpr int NS = HD / 16;          // k-steps of S = K Q^T
  static constexpr int NDT = HD / 32;         // 32-column tiles of O^T
  static_assert(SPASS >= 1 && SPASS * SROWS == BN, "staging covers the key tile exactly");
  static_assert(SROWS % 16 == 0, "staging rows srow + SROWS k keep perm_row's block");
  static_assert(NT / 64 * out_wave_bytes<NDT>() <= LDS_BYTES, "output staging fits in the tiles' LDS");
};

struct Params {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  int8_t* o_lo;      // optional: the rounding residual of o as int8 codes (lo_code)
  float* lse;
  const bf16* gate;  // optional: with y, also write y = sigmoid(gate) * o
  bf16* y;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lo_st, lo_sh, g_st, g_sh, y_st, y_sh;
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  const int2* items;
  const WsHeader* hdr;
  float* q_amax;     // optional: max |Q| of each wave's rows, at slot NT / 64 * blockIdx.x + wave (0: none)
  int T, H, is_causal;
  int numseqs;       // items naming a segment >= numseqs (a stale plan) are skipped
  float scale_log2;  // softmax_scale * log2(e)
};

// Three workgroups per CU at HD = 128 (12 waves, at most 168 VGPRs each): 32-key tiles
// keep the registers and the LDS (4 tiles of 9.5 KB per workgroup) within that budget,
// and the third workgroup hides more of each wave's MFMA -> softmax -> MFMA latency
// than the larger tiles of two workgroups did. HD = 64 halves the Q and O registers
// and the tiles, and runs four workgroups per CU.
template <int HD>
__global__ __launch_bounds__(NT, HD == 64 ? 4 : 3) void prefixlm_fwd_kernel(Params P) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  using G = Geo<HD>;
  constexpr int RS = G::RS, TILE = G::TILE, SROWS = G::SROWS, SPASS = G::SPASS, OFF_K = G::OFF_K,
                OFF_V = G::OFF_V, NS = G::NS, NDT = G::NDT, D = HD;

  int item, h;
  // a workgroup without work still writes its max |Q| slots (0), so that every slot of
  // the grid holds a value
  if (!unit_of(blockIdx.x, P.hdr->n_items, P.H, &item, &h)) {
    if (P.q_amax != nullptr && threadIdx.x < NT / 64) P.q_amax[NT / 64 * blockIdx.x + threadIdx.x] = 0.f;
    return;
  }
  const int2 it = P.items[item];
  const int seg = it.x, qt = it.y;
  if (seg < 0 || seg >= P.numseqs) {
    if (P.q_amax != nullptr && threadIdx.x < NT / 64) P.q_amax[NT / 64 * blockIdx.x + threadIdx.x] = 0.f;
    return;
  }
  const int cs = P.cu[seg];
  const int L = P.prefix[seg] + P.causal[seg];
  const int p = P.is_causal ? 0 : P.prefix[seg];

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int q0 = qt * BM;
  const int qw0 = q0 + w * 32;
  const int kend = min(L, max(p, min(q0 + BM, L)));
  const int nk = (kend + BN - 1) / BN;
  const bool wave_active = qw0 < L;
  const int kend_w = wave_active ? min(L, max(p, min(qw0 + 32, L))) : 0;
  // every query of the wave sees keys [0, kfull)
  const int kfull = min(L, max(p, qw0 + 1));

  const __amdgpu_buffer_rsrc_t qr = make_rsrc(P.q + cs * P.q_st + h * P.q_sh, rows_bytes(L, P.q_st, D));
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(P.k + cs * P.k_st + h * P.k_sh, rows_bytes(L, P.k_st, D));
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(P.v + cs * P.v_st + h * P.v_sh, rows_bytes(L, P.v_st, D));
  const uint32_t kst2 = (uint32_t)P.k_st * 2, vst2 = (uint32_t)P.v_st * 2;

  // staging of one K/V tile: thread = 16-byte chunk sch of rows srow + SROWS k; the V
  // thread loads the key row that goes to stored row srow (perm_row is its own inverse)
  const int srow = tid / G::CPR, sch = tid % G::CPR;
  const int vrow = perm_row(srow);
  char* stage_base = smem + srow * RS + sch * 16;
  u32x4 ks[SPASS], vs[SPASS];
  auto load_kv = [&](int k0) {
#pragma unroll
    for (int r = 0; r < SPASS; ++r) {
      ks[r] = buf_load16(kr, (uint32_t)(k0 + SROWS * r + srow) * kst2 + sch * 16);
      vs[r] = buf_load16(vr, (uint32_t)(k0 + SROWS * r + vrow) * vst2 + sch * 16);
    }
  };
  auto store_kv = [&](int b) {
#pragma unroll
    for (int r = 0; r < SPASS; ++r) {
      *reinterpret_cast<u32x4*>(stage_base + OFF_K + b * TILE + SROWS * r * RS) = ks[r];
      *reinterpret_cast<u32x4*>(stage_base + OFF_V + b * TILE + SROWS * r * RS) = vs[r];
    }
  };
  if (nk > 0) load_kv(0);

  // Q^T fragments: lane holds query qw0+l32, d = 16*s + 8*hh + 0..7
  bf16x8 qf[NS];
  {
    const uint32_t off = (uint32_t)(qw0 + l32) * (uint32_t)P.q_st * 2 + hh * 16;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = __builtin_bit_cast(bf16x8, buf_load16(qr, off + s * 32));
  }

  f32x16 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float c = P.scale_log2;
  const int qi = qw0 + l32;   // this lane's query (local index)
  const int kq = min(L, max(p, qi + 1));   // this lane's query sees keys [0, kq)
  const char* row_base = smem + l32 * RS + hh * 16;   // K rows: key l32 (+32t), d 16s + 8hh
  const char* xt_base = smem + xt_lane_off<RS>(lane);

  if (nk > 0) store_kv(0);
  // Q has arrived before the loop: the loop's only memory wait is the one for the
  // next K/V tile, before it goes to LDS
#pragma unroll
  for (int s = 0; s < NS; ++s) settle(__builtin_bit_cast(u32x4, qf[s]));
  // max |Q| of the wave's rows, for the backward's fp16 scale of Q (rows past the segment
  // read as 0): bf16 magnitudes compare as 16-bit integers, two per word
  if (P.q_amax != nullptr) {
    u16x2 m = {0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, __builtin_bit_cast(u32x4, qf[s])[e] & 0x7fff7fffu));
    // the wave's max: DPP within each 16-lane row, then the four rows' results (no LDS
    // round trips)
    const int mi = __builtin_bit_cast(
        int, row16_max(__builtin_bit_cast(float, (uint32_t)(m[0] > m[1] ? m[0] : m[1]) << 16)));
    auto row = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(mi, l)); };
    const float wm = fmaxf(fmaxf(row(0), row(16)), fmaxf(row(32), row(48)));
    if (lane == 0) P.q_amax[NT / 64 * blockIdx.x + w] = wm;
  }
  __syncthreads();

  for (int j = 0; j < nk; ++j) {
    const int B = j & 1;
    const int k0 = j * BN;
    load_kv(k0 + BN);   // unconditional: the tile past the end goes to a buffer no wave reads again
    if (wave_active && k0 < kend_w) {
      // ---- S^T = K Q^T, K rows two steps ahead of the MFMAs -------------------------
      f32x16 sacc[BN / 32];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[t][r] = 0.f;
      bf16x8 ka[NS][BN / 32];
      auto rd = [&](int s) {
#pragma unroll
        for (int t = 0; t < BN / 32; ++t)
          ka[s][t] = *reinterpret_cast<const bf16x8*>(row_base + OFF_K + B * TILE + 32 * t * RS + 32 * s);
      };
      rd(0);
      rd(1);
      sched_fence();
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (s + 2 < NS) rd(s + 2);
        sched_fence();
#pragma unroll
        for (int t = 0; t < BN / 32; ++t) sacc[t] = mfma32x32x16(ka[s][t], qf[s], sacc[t]);
        sched_fence();
      }
      // first V^T operands in flight during the softmax
      constexpr int NPV = BN / 16 * NDT;   // P.V MFMAs: key steps x d tiles
      u32x4 xt[NPV];   // operand of P.V step i: k-step i / NDT, d tile i % NDT
      xt[0] = lds_read_xt<RS>(xt_base + OFF_V + B * TILE, 0, 0);
      xt[1] = lds_read_xt<RS>(xt_base + OFF_V + B * TILE, 1 / NDT, 1 % NDT);
      sched_fence();
      // ---- softmax: mask only on tiles that are not fully visible ---------------------
      if (k0 + BN > kfull) {
        // key k0 + 32t + 8(r/4) + 4hh + r%4 is seen iff it is below kq
        const int tk = kq - k0 - 4 * hh;
#pragma unroll
        for (int t = 0; t < BN / 32; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            sacc[t][r] = (32 * t + 8 * (r >> 2) + (r & 3) < tk) ? sacc[t][r] : -INFINITY;
      }
      float mx = sacc[0][0];
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int r = (t == 0 ? 1 : 0); r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
      mx = halves_max(mx) * c;
      // rescale only when some lane's running max rises (the decision is per wave)
      if (__builtin_amdgcn_ballot_w64(mx > m_run) != 0) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
      }
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
      bf16x8 pb[BN / 16];
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t][8 * half + i], c, -m_use));
            ps += e[i];
          }
          pb[2 * t + half] = cvt8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
        }
      l_run += ps;
      sched_fence();
      // ---- O^T += V^T P^T, V^T operands read two MFMAs ahead ------------------------
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        if (i + 2 < NPV) xt[i + 2] = lds_read_xt<RS>(xt_base + OFF_V + B * TILE, (i + 2) / NDT, (i + 2) % NDT);
        sched_fence();
        oacc[i % NDT] = mfma32x32x16(__builtin_bit_cast(bf16x8, xt[i]), pb[i / NDT], oacc[i % NDT]);
        sched_fence();
      }
    }
    store_kv(B ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O and its residual as whole rows through LDS, then the LSE ------------
  if (nk == 0) __syncthreads();
  const float lt = halves_sum(l_run);
  const float inv = wave_active ? 1.f / lt : 0.f;
  {
    char* wl = smem + w * out_wave_bytes<NDT>();
    const __amdgpu_buffer_rsrc_t orr = make_rsrc(P.o + cs * P.o_st + h * P.o_sh, rows_bytes(L, P.o_st, D));
    bool gated = false;
    if constexpr (HD == 128) {
      if (P.gate != nullptr) {
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(P.gate + cs * P.g_st + h * P.g_sh, rows_bytes(L, P.g_st, D));
        const __amdgpu_buffer_rsrc_t yr = make_rsrc(P.y + cs * P.y_st + h * P.y_sh, rows_bytes(L, P.y_st, D));
        store_rows_gated_via_lds(oacc, inv, wl, orr, gr, yr, qw0, (uint32_t)P.o_st * 2, (uint32_t)P.g_st * 2,
                                 (uint32_t)P.y_st * 2, lane);
        gated = true;
      }
    }
    // O and its residual are read again only by the backward: non-temporal stores
    if (!gated) store_rows_via_lds<NDT, 2>(oacc, inv, wl, orr, qw0, (uint32_t)P.o_st * 2, lane);
    if (P.o_lo != nullptr) {
      // the residual of the rounding above, from the same fp32 values, as int8 codes
      const __amdgpu_buffer_rsrc_t lor =
          make_rsrc(P.o_lo + cs * P.lo_st + h * P.lo_sh, rows_bytes(L, P.lo_st, D, 1));
      store_lo_rows_via_lds<NDT, 2>(oacc, inv, wl, lor, qw0, (uint32_t)P.lo_st, lane);
    }
  }
  if (wave_active && hh == 0 && qi < L) P.lse[(int64_t)h * P.T + cs + qi] = (m_run + __builtin_log2f(lt)) * kLn2;
}

// Rows >= total_seqlen: out = 0 (and its residual) and lse = -inf (reference :130;
// FA3 leaves its LSE there unspecified). One HD/8-thread group per (row, head), 16 B
// of O (8 elements, and their 8 residual bytes) per thread.
template <int HD>
__global__ __launch_bounds__(256) void prefixlm_fwd_pad_kernel(bf16* o, int8_t* o_lo, bf16* y, float* lse,
                                                                int64_t o_st, int64_t o_sh,
                                                                int64_t lo_st, int64_t lo_sh, int64_t y_st,
                                                                int64_t y_sh, int T, int H, int total) {
  constexpr int CPR = HD / 8, GROUPS = 256 / CPR;
  const int64_t gidx = (int64_t)blockIdx.x * GROUPS + (threadIdx.x / CPR);
  const int64_t rows = (int64_t)(T - total) * H;
  if (gidx >= rows) return;
  const int t = total + (int)(gidx / H);
  const int h = (int)(gidx % H);
  const int chunk = threadIdx.x % CPR;
  u32x4 z = {0u, 0u, 0u, 0u};
  *reinterpret_cast<u32x4*>(o + t * o_st + h * o_sh + chunk * 8) = z;
  if (o_lo) *reinterpret_cast<u32x2*>(o_lo + t * lo_st + h * lo_sh + chunk * 8) = u32x2{0u, 0u};
  if (y) *reinterpret_cast<u32x4*>(y + t * y_st + h * y_sh + chunk * 8) = z;
  if (chunk == 0) lse[(int64_t)h * T + t] = -INFINITY;
}

}  // namespace fwd
}  // namespace prefixlm
