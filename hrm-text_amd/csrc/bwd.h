// Backward kernels.
//
// Replaces the two FA3 backward calls and the elementwise epilogue of
// models/flash_attention_prefixlm_v2.py:152-212 (reference):
//   pre  : delta[h,t] = sum_d dO*O (fp32; O = out + its rounding residual when the
//          forward kept one) and per-head maxima of |dO|, ||dO_t|| and |delta_t|;
//   dkdv : one workgroup = one (segment, 128-key tile, head) in two groups of 64
//          keys, each group with four jobs (S and P; dV; dP and dS; dK; the dV and dK
//          jobs on two waves each, one per half of head_dim),
//          pipelined over 32-row query tiles with P and dS passed through LDS.
//          Each key row is owned by one workgroup, which sees both the prefix rows
//          and the suffix rows, so the reference's dk1 + dk2 / dv1 + dv2 (:212)
//          disappears;
//   dq   : one workgroup = one (segment, 128-query tile, head); each wave holds Q and
//          dO of 32 queries in registers, streams 32-key tiles of K and V through
//          LDS, recomputes S, P, dP, dS and accumulates dQ^T += K^T dS^T, then
//          writes bf16 dQ. No atomics: dQ is bitwise deterministic;
//   pad  : dq, dk, dv rows >= total_seqlen are zeroed (:209-211).
//
// Precision: S and dP contract 16-bit inputs over D whose products are exact in
// fp32. Every product runs in fp16 with power-of-two scales: the dV product uses fp16
// P (P lies in [0, 1]) and fp16 dO scaled per head; the dQ and dK products use fp16 dS
// scaled from a bound on its magnitude, with fp16 K (scaled per segment and head) or
// fp16 Q (scaled per head from the forward's max |Q|); S uses the same scaled Q and
// K. fp16 keeps 3 more mantissa bits than bf16, bf16 -> fp16 with such a scale is
// exact, and the scales are undone exactly in fp32.
#pragma once
#include <type_traits>

#include "common.h"
#include "fwd.h"
#include "worklist.h"

namespace prefixlm {
namespace bwd {

constexpr int kStats = 4;        // per head: max|dO|, max ||dO_t||_2, max |delta_t|, max |Q|
constexpr int kSegStats = 2;     // per (segment, head): max |K|, max ||V_k||_2
constexpr int kCounters = 16;    // work-item counters after the statistics (8 per persistent kernel)

__device__ __forceinline__ void atomic_max_nonneg(float* p, float v) {
  atomicMax(reinterpret_cast<int*>(p), __builtin_bit_cast(int, v));
}

// =====================================================================================
// dK / dV
// =====================================================================================
struct KvParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* dout;
  const float* lse;       // [H, T]
  const float* delta;     // [H, T]
  const float* stats;     // [H, kStats]
  float* segstats;        // [numseqs, H, kSegStats], atomic max
  int* counters;          // [8] work-item counters of the persistent grid, zero on entry
  // optional (ds null: none): dS stored for the dQ-from-dS kernel, as fp16 blocks of 32
  // queries x 64 keys, one per attended (key group, query tile) in the layout of
  // ds_blk_off (worklist.h), and one scale per 128-key tile
  char* ds;
  float* ds_scale;        // [H, ds_nkslot]
  const int32_t* ds_base; // [numseqs + 1] first block of each segment
  uint32_t ds_hbytes;     // bytes of one head's blocks
  int ds_nkslot;          // key-tile slots per head
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

// One workgroup = one (segment, 128-key tile, head) in two groups of 64 keys; each
// group has four jobs, pipelined over 32-row query tiles t:
//   S  : S(t) = Q(t) K^T for its 64 keys (Q and K fp16, scaled; K in registers),
//        P(t) = exp2(S c - lse2) (fp16, masked) into an exchange buffer;
//   dV : dV^T += dO(t-1)^T P(t-1)            (accumulator only: MFMA and LDS reads);
//   dP : dS(t-1) = P(t-1) x(t-1) (fp16, scaled) into an exchange buffer (and the
//        stored dS), then x(t) = s_dp (dO(t) V^T - delta) with V in registers (fp16,
//        scaled);
//   dK : dK^T += Q(t-2)^T dS(t-2)            (accumulator only).
// S and dP run on one wave each; dV and dK on two waves each, one per half of
// head_dim (12 waves). Waves w, w+4 and w+8 share a SIMD, so every SIMD runs a wave
// with softmax or dS work (S, dP) beside two MFMA-only waves (dV, dK halves), three
// waves per SIMD in all; the dV and dK waves also stage the query tiles (loads, dO
// conversion, LDS stores), which keeps that work off the S and dP waves' longer
// chains. Each LDS operand fragment of S and dP feeds the MFMAs of both 32-key blocks.
// One workgroup barrier per query tile; Q tiles live four iterations, dO tiles three.
namespace kv {
constexpr int BK = 128;                // keys per workgroup
constexpr int KG = 64;                 // keys per group
constexpr int BQ = 32;                 // query rows per tile
// Waves per dV / dK job, each owning 1 / NSPLIT of head_dim. Two (12 waves, at most 168
// VGPRs each) measured 1.6% faster than one (8 waves of 256 VGPRs) on config 2, 0.5% on
// configs 3 and 4; 1 still builds.
constexpr int NSPLIT = 2;
constexpr int NT = (4 + 4 * NSPLIT) * 64;
constexpr int NQB = 4, NOB = 3;        // Q and dO tile buffers
constexpr int XG = 4096;               // exchange bytes per group: [key block][k-step][64 lanes][16 B]
constexpr int XBUF = 2 * XG;           // one exchange buffer (both groups)
static_assert(BK == 2 * KG && (NSPLIT == 1 || NSPLIT == 2), "two groups of four jobs");
enum Role { R_S = 0, R_DV = 1, R_DP = 2, R_DK = 3 };
// LDS map for head dim HD (128 or 64); P and dS are [query][key] and independent of HD
template <int HD>
struct Geo {
  static constexpr int W = rsw_of<HD>();            // wide rows: conflict-free row and transposing reads
  static constexpr int TILE = BQ * W;
  static constexpr int NS = HD / 16;                // k-steps of S and dP (contraction over d)
  static constexpr int NDT = HD / 32;               // 32-column d tiles of dV and dK
  static constexpr int DT = NDT / NSPLIT;           // d tiles of one dV or dK wave
  static constexpr int PIECE = HD / 8;              // staging bytes per thread: 32 rows x 16 pieces
  static constexpr int OFF_QS = 0;
  static constexpr int OFF_DOS = NQB * TILE;
  static constexpr int OFF_PX = OFF_DOS + NOB * TILE;     // [2] P buffers
  static constexpr int OFF_SX = OFF_PX + 2 * XBUF;        // [2] dS buffers
  static constexpr int OFF_LSE = OFF_SX + 2 * XBUF;       // [2][BQ] lse * log2(e)
  static constexpr int OFF_DLT = OFF_LSE + 2 * BQ * 4;    // [2][BQ] -delta * s_dp
  static constexpr int OFF_RED = OFF_DLT + 2 * BQ * 4;    // [2] max ||V_k|| of each group
  static constexpr int OFF_NEXT = OFF_RED + 16;           // the next work index
  static constexpr int LDS_BYTES = OFF_NEXT + 16;
  static_assert(2 * 16 == BQ && 16 * PIECE == 2 * HD, "staging: two waves per tile x 16 rows x 16 pieces");
  static_assert(NT / 64 * out_wave_bytes<DT>() <= OFF_RED, "output staging fits below the scalars");
};
}  // namespace kv

// A work item of the persistent dK/dV kernel: (segment, 128-key tile, head) and the
// segment's geometry. An index past the list, or naming a segment >= numseqs (a stale
// plan), gives an empty item (L = 0) that runs no tiles and writes nothing.
struct KvItem {
  int valid, seg, h, cs, L, p, k0;
};
__device__ __forceinline__ KvItem kv_item(const KvParams& P, int idx, int n_items) {
  KvItem d{0, 0, 0, 0, 0, 0, 0};
  int item, h;
  if (!unit_of(idx, n_items, P.H, &item, &h)) return d;
  d.h = h;
  const int2 it = P.items[item];
  d.valid = 1;
  if (it.x < 0 || it.x >= P.numseqs) return d;
  // every field is the same in all lanes: kept as scalars, so that the buffer resources
  // built from them need no readfirstlane loop around each load
  d.seg = __builtin_amdgcn_readfirstlane(it.x);
  d.cs = __builtin_amdgcn_readfirstlane(P.cu[d.seg]);
  d.L = __builtin_amdgcn_readfirstlane(P.prefix[d.seg] + P.causal[d.seg]);
  d.p = P.is_causal ? 0 : __builtin_amdgcn_readfirstlane(P.prefix[d.seg]);
  d.k0 = __builtin_amdgcn_readfirstlane(it.y) * kv::BK;
  return d;
}

// 16 (head dim 128) or 8 (head dim 64) bytes of a staged row
template <int HD>
using Piece = std::conditional_t<HD == 128, u32x4, u32x2>;
template <int HD, int AUX = 0>
__device__ __forceinline__ Piece<HD> load_piece(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (HD == 128)
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
  else
    return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, AUX);
}

template <int ROLE, int HD>
__device__ __forceinline__ void kv_wave(const KvParams& P, char* smem) {
  using namespace kv;
  using G = Geo<HD>;
  constexpr int D = HD, W = G::W, TILE = G::TILE, NS = G::NS, DT = G::DT;
  constexpr int OFF_QS = G::OFF_QS, OFF_DOS = G::OFF_DOS, OFF_PX = G::OFF_PX, OFF_SX = G::OFF_SX,
                OFF_LSE = G::OFF_LSE, OFF_DLT = G::OFF_DLT, OFF_RED = G::OFF_RED, OFF_NEXT = G::OFF_NEXT;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = (w >> 1) & 1;
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  float* red = reinterpret_cast<float*>(smem + OFF_RED);
  int* next_slot = reinterpret_cast<int*>(smem + OFF_NEXT);
  const uint32_t qst2 = (uint32_t)P.q_st * 2, dost2 = (uint32_t)P.do_st * 2;

  // Work units: this workgroup's first index is its blockIdx; every later one comes from
  // the counter of its XCD (blockIdx % 8: the hardware deals workgroups to the 8 XCDs
  // round robin), so an XCD only ever takes indices of its own residue mod 8, which
  // unit_of maps to the XCD's own heads, as for a non-persistent grid.
  const int n_items = P.hdr->n_items;
  const int xcd = blockIdx.x & 7;
  KvItem cur = kv_item(P, blockIdx.x, n_items);

  __amdgpu_buffer_rsrc_t qr, dor, lser, dltr;
  auto set_rsrc = [&](const KvItem& d) {
    qr = make_rsrc(P.q + d.cs * P.q_st + d.h * P.q_sh, rows_bytes(d.L, P.q_st, D));
    dor = make_rsrc(P.dout + d.cs * P.do_st + d.h * P.do_sh, rows_bytes(d.L, P.do_st, D));
    lser = make_rsrc(P.lse + (int64_t)d.h * P.T + d.cs, (uint32_t)d.L * 4);
    dltr = make_rsrc(P.delta + (int64_t)d.h * P.T + d.cs, (uint32_t)d.L * 4);
  };

  // Staging of a query tile (32 rows x 16 pieces of HD / 8 bytes) by the MFMA-only
  // waves, so the S and dP waves, whose softmax and dS work is the longer chain of a
  // trip, issue no tile loads and no staging stores: the dV waves (4, 6, 8, 10) stage the
  // Q tile, the dK waves (5, 7, 9, 11) the dO tile, each converted to scaled fp16, rows
  // 4 SPW u + lane / 16 + 4 j (j < SPW) of its tile, u = ((w - 4) / 2) % 4. The rows of
  // one wave keep row % 4 and have (row / 4) % 4 = 2 (u % 2) + j (no wrap), so row
  // srow + 4 j sits at stage_base + wrow_off(4 j) - wrow_off(0).
  constexpr bool STAGER = ROLE == R_DV || ROLE == R_DK;
  constexpr int SPW = 4 / NSPLIT;   // pieces per lane of a staging wave: rows srow + 4 j, j < SPW
  const int sv = ((w - 4) >> 1) & (2 * NSPLIT - 1);
  const int srow = 4 * SPW * sv + (lane >> 4), sch = lane & 15;
  // dV / dK waves: d tiles [DT dh, DT dh + DT) of the group's keys
  const int dh = (w >= 4) ? (w - 4) >> 2 : 0;
  char* stage_base = smem + wrow_off<W>(srow) + sch * G::PIECE;
  // Loads run two tiles ahead of their LDS stores through two register sets. Rows past
  // the segment load as zeros (buffer bounds); offsets stay below the host's 2 GiB
  // check of (max_seqlen_all + 256) rows.
  struct Stage {
    Piece<HD> x[SPW];
    float lse, dlt;
  };
  Stage sa, sb;
  auto load_tile = [&](Stage& st, int qi) {
    if constexpr (STAGER) {
      const __amdgpu_buffer_rsrc_t r = ROLE == R_DV ? qr : dor;
      const uint32_t st2 = ROLE == R_DV ? qst2 : dost2;
#pragma unroll
      for (int j = 0; j < SPW; ++j) st.x[j] = load_piece<HD>(r, (uint32_t)(qi + srow + 4 * j) * st2 + sch * G::PIECE);
      // lse and delta go to LDS from wave 5 (a dK wave)
      if constexpr (ROLE == R_DK) {
        if (w == 5) {
          st.lse = buf_loadf(lser, (uint32_t)(qi + (lane & (BQ - 1))) * 4);
          st.dlt = buf_loadf(dltr, (uint32_t)(qi + (lane & (BQ - 1))) * 4);
        }
      }
    }
  };
  // stationary operand (S: K, dP: V fp16 scaled): B[k = d 16s+8hh+i][col = key] of
  // key block kb = keys kA + 32 kb + l32
  u32x4 kv_op[2][NS];
  auto load_kv = [&](const KvItem& d) {
    if constexpr (ROLE == R_S || ROLE == R_DP) {
      const __amdgpu_buffer_rsrc_t r =
          ROLE == R_S ? make_rsrc(P.k + d.cs * P.k_st + d.h * P.k_sh, rows_bytes(d.L, P.k_st, D))
                      : make_rsrc(P.v + d.cs * P.v_st + d.h * P.v_sh, rows_bytes(d.L, P.v_st, D));
      const uint32_t st2 = (uint32_t)(ROLE == R_S ? P.k_st : P.v_st) * 2;
      const int ka = d.k0 + KG * g;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < NS; ++s)
          kv_op[kb][s] = buf_load16(r, (uint32_t)(ka + 32 * kb + l32) * st2 + (16 * s + 8 * hh) * 2);
    }
  };
  set_rsrc(cur);
  load_tile(sa, (cur.k0 < cur.p) ? 0 : cur.k0);
  load_kv(cur);

  while (cur.valid) {
    const int seg = cur.seg, h = cur.h, cs = cur.cs, L = cur.L, p = cur.p, k0 = cur.k0;
    const int kA = k0 + KG * g;          // first key of this group
    const float s_do = pow2_scale(P.stats[h * kStats + 0]);   // max |dO|
    float* segst = P.segstats + ((int64_t)seg * P.H + h) * kSegStats;
    // fp16 scale of Q: none (a plain conversion, exact) when max |Q| lies in [2^-4, 2^14],
    // as query activations do, else a power of two that puts it in (2^13, 2^14]
    const float q_max = P.stats[h * kStats + 3];
    const float s_q = (q_max >= 0x1p-4f && q_max <= 0x1p14f) ? 1.f : pow2_scale(q_max);
    const int qstart = (k0 < p) ? 0 : k0;
    const int nq = (L - qstart + BQ - 1) / BQ;
    // the next index, claimed now and read at the end of this item
    int claimed = 0;
    if (tid == 0) claimed = atomicAdd(P.counters + xcd, 1);

    float kmax = 0.f;   // role S: max |K| over this wave's keys
    if constexpr (ROLE == R_S || ROLE == R_DP) {
      float m = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float mk = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x0 = bf16lo(kv_op[kb][s][e]), x1 = bf16hi(kv_op[kb][s][e]);
            if (ROLE == R_S)
              mk = fmaxf(mk, fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1)));
            else
              mk += x0 * x0 + x1 * x1;
          }
        if (ROLE == R_DP) mk = __builtin_sqrtf(mk + __shfl_xor(mk, 32));   // ||V_key||
        m = fmaxf(m, mk);
      }
      m = wave_max(m);
      if (lane == 0) {
        if (L > 0) atomic_max_nonneg(segst + (ROLE == R_S ? 0 : 1), m);
        if (ROLE == R_DP) red[g] = m;
      }
      kmax = m;
    }
    __syncthreads();   // per-group maxima of ||V|| visible; the last item's outputs are out
    // Stored dS is s_st dS in fp16, s_st a power of two with s_st |dS| <= 2^14 from
    // |dS| <= P |dP - delta| <= max ||dO_t|| max ||V_k|| + max |delta_t| (this tile's keys)
    const bool ds_on = P.ds != nullptr;
    const float s_st = pow2_scale(P.stats[h * kStats + 1] * fmaxf(red[0], red[1]) + P.stats[h * kStats + 2]);
    if (ds_on && tid == 0 && L > 0) P.ds_scale[(int64_t)h * P.ds_nkslot + ((cs + k0) >> 7) + seg] = s_st;
    // V's fp16 scale (a power of two): s_st / s_do, so that dP comes out carrying s_st and
    // the dS values need no rescaling before their store. It keeps s_v |V| < 2: s_do >
    // 2^13 / max |dO| and s_st <= 2^14 / (max |dO| max ||V||). Where that ratio leaves
    // [2^-100, s_vmax] (dO = 0, say, makes it 1 whatever V is), the largest safe scale
    // s_vmax (s_vmax max ||V|| < 2^14) is taken and the dS values are rescaled by ds_f.
    const float s_vmax = pow2_scale(fmaxf(red[0], red[1]));
    const float s_want = s_st / s_do;
    const float s_v = (s_want <= s_vmax && s_want >= 0x1p-100f) ? s_want : s_vmax;
    const float s_dp = s_do * s_v;   // dP is accumulated scaled by s_dp, from -delta * s_dp
    const float ds_f = s_st / s_dp;  // 1 unless s_v fell back to s_vmax
    const __amdgpu_buffer_rsrc_t dsr =
        make_rsrc(ds_on ? P.ds + (int64_t)h * P.ds_hbytes : reinterpret_cast<char*>(P.dk), ds_on ? P.ds_hbytes : 0u);
    // block of (this group's key group, query tile 0); the layout uses prefix_lens
    // whatever is_causal
    int ds_blk0 = 0;
    if (ROLE == R_DP && ds_on) {
      const int pl = P.prefix[seg];
      ds_blk0 = P.ds_base[seg] + ds_blk_off(kA >> 6, (L + 31) >> 5, ds_kp(pl, L));
    }
    // K (role S) as fp16 scaled by a power of two from this wave's max |K|; S then comes
    // out scaled by s_q s_k, which the softmax's multiplier undoes
    const float s_k = pow2_scale(kmax);
    if constexpr (ROLE == R_DP || ROLE == R_S) {
      // the operands are unpacked again here rather than kept unpacked (twice the
      // registers) from the statistics above
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < NS; ++s) renew(kv_op[kb][s]);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s = 0; s < NS; ++s)
          kv_op[kb][s] = __builtin_bit_cast(u32x4, bf16x8_to_f16_scaled(kv_op[kb][s], ROLE == R_DP ? s_v : s_k));
    }

    f32x16 acc[2][DT];   // dV (role dV) or s_dp dK (role dK): [key block][d tile DT dh + ..]
    if constexpr (ROLE == R_DV || ROLE == R_DK) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[kb][t][r] = 0.f;
    }

    // row srow + 4 j sits at stage_base + wrow_off(4 j) - wrow_off(0) (see the staging
    // above). The tile buffer's offset goes through readfirstlane (an SGPR the compiler cannot
    // fold), so each trip adds it to the one lane base in a VGPR instead of the compiler
    // keeping an address per (buffer, row) in registers, which spilled them
    auto store_tile = [&](const Stage& st, int qb, int ob, int lb) {
      if constexpr (ROLE == R_DV) {
        char* base = stage_base + __builtin_amdgcn_readfirstlane(OFF_QS + qb * TILE);
        if (s_q == 1.f) {   // wave-uniform: the usual case, no multiplies
#pragma unroll
          for (int j = 0; j < SPW; ++j) {
            char* dst = base + wrow_off<W>(4 * j) - wrow_off<W>(0);
            if constexpr (HD == 128)
              *reinterpret_cast<f16x8*>(dst) = bf16x8_to_f16(st.x[j]);
            else
              *reinterpret_cast<u32x2*>(dst) = bf16x4_to_f16(st.x[j]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < SPW; ++j) {
            char* dst = base + wrow_off<W>(4 * j) - wrow_off<W>(0);
            if constexpr (HD == 128)
              *reinterpret_cast<f16x8*>(dst) = bf16x8_to_f16_scaled(st.x[j], s_q);
            else
              *reinterpret_cast<u32x2*>(dst) = bf16x4_to_f16_scaled(st.x[j], s_q);
          }
        }
      } else if constexpr (ROLE == R_DK) {
        char* base = stage_base + __builtin_amdgcn_readfirstlane(OFF_DOS + ob * TILE);
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
          char* dst = base + wrow_off<W>(4 * j) - wrow_off<W>(0);
          if constexpr (HD == 128)
            *reinterpret_cast<f16x8*>(dst) = bf16x8_to_f16_scaled(st.x[j], s_do);
          else
            *reinterpret_cast<u32x2*>(dst) = bf16x4_to_f16_scaled(st.x[j], s_do);
        }
        if (w == 5) {
          if (lane < BQ)
            reinterpret_cast<float*>(smem + OFF_LSE)[lb * BQ + lane] = st.lse * kLog2e;
          else
            reinterpret_cast<float*>(smem + OFF_DLT)[lb * BQ + lane - BQ] = -st.dlt * s_dp;
        }
      }
    };

    const float c = P.scale_log2 / s_q / s_k;   // role S: S is scaled by s_q s_k
    const int x_lane = g * XG + lane * 16;   // + kb * 2048 + kstep * 1024 in an exchange buffer
    const char* row_base = smem + wrow_off<W>(l32) + hh * 16;   // A operand rows: row l32, d 16s + 8hh
    const char* xt_base = smem + xtw_lane_off<W>(lane);
    const float* lse_base = reinterpret_cast<const float*>(smem + OFF_LSE) + 4 * hh;
    const float* dlt_base = reinterpret_cast<const float*>(smem + OFF_DLT) + 4 * hh;

    f32x16 x_prev[2];   // role dP: s_dp (dP - delta) of tile t-1
    int ob_cur = 0, ob_prev = 2, ob_next = 1;   // dO buffers of tiles t, t-1, t+1

    // some (query, key) pair of tile t is allowed for this group's keys
    auto seen_tile = [&](int t) {
      const int qi = qstart + t * BQ;
      return t >= 0 && t < nq && kA < L && (kA < p || qi + BQ > kA);
    };

    store_tile(sa, 0, 0, 0);
    load_tile(sb, qstart + BQ);
    // One query tile t: tile t+2 is loaded into `ld` (the set of tile t, stored already)
    // and tile t+1 goes from `st` into the buffers freed in t-1. Both run unconditionally:
    // tiles past nq land in buffers that no wave reads again.
    auto trip = [&](int t, Stage& ld, const Stage& st) __attribute__((always_inline)) {
      const int qi = qstart + t * BQ;
      __syncthreads();   // tile t, P(t-1), dS(t-2) visible; buffers read in t-1 are free
      load_tile(ld, qi + 2 * BQ);
      if constexpr (ROLE == R_S) {
        if (seen_tile(t)) {
          f32x16 xacc[2];
  #pragma unroll
          for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
            for (int r = 0; r < 16; ++r) xacc[kb][r] = 0.f;
          const char* qb = row_base + OFF_QS + (t & 3) * TILE;
          f16x8 qa[NS];
  #pragma unroll
          for (int s = 0; s < 3; ++s) qa[s] = *reinterpret_cast<const f16x8*>(qb + 32 * s);
          sched_fence();
  #pragma unroll
          for (int s = 0; s < NS; ++s) {
            if (s + 3 < NS) qa[s + 3] = *reinterpret_cast<const f16x8*>(qb + 32 * (s + 3));
            sched_fence();
  #pragma unroll
            for (int kb = 0; kb < 2; ++kb)
              xacc[kb] = mfma32x32x16_f16(qa[s], __builtin_bit_cast(f16x8, kv_op[kb][s]), xacc[kb]);
            sched_fence();
          }
          f32x4 l4[4];
  #pragma unroll
          for (int m = 0; m < 4; ++m) l4[m] = *reinterpret_cast<const f32x4*>(lse_base + (t & 1) * BQ + 8 * m);
          const bool all = kA + KG <= L && (kA + KG <= p || kA + KG - 1 <= qi);
          char* px = smem + OFF_PX + (t & 1) * XBUF + x_lane;
  #pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            float pv[16];
            if (all) {
  #pragma unroll
              for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(xacc[kb][r], c, -l4[r >> 2][r & 3]));
            } else {
              // query row qrow sees key kA + 32 kb + l32 iff qrow >= thr
              const int key = kA + 32 * kb + l32;
              const int thr = key < p ? -(1 << 30) : (key < L ? key : (1 << 30));
              const int tq = thr - qi - 4 * hh;
  #pragma unroll
              for (int r = 0; r < 16; ++r) {
                const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(xacc[kb][r], c, -l4[r >> 2][r & 3]));
                pv[r] = (8 * (r >> 2) + (r & 3) >= tq) ? e : 0.f;
              }
            }
  #pragma unroll
            for (int ks = 0; ks < 2; ++ks)
              *reinterpret_cast<f16x8*>(px + kb * 2048 + ks * 1024) =
                  cvt8h(pv[8 * ks], pv[8 * ks + 1], pv[8 * ks + 2], pv[8 * ks + 3], pv[8 * ks + 4], pv[8 * ks + 5],
                        pv[8 * ks + 6], pv[8 * ks + 7]);
          }
        }
      } else if constexpr (ROLE == R_DV || ROLE == R_DK) {
        // dV^T[d][key] += dO^T[d][q] P[q][key] (tile t-1) or s_q s_st dK^T += Q^T dS (tile t-2)
        const int tt = ROLE == R_DV ? t - 1 : t - 2;
        if (seen_tile(tt)) {
          const char* xb = smem + (ROLE == R_DV ? OFF_PX : OFF_SX) + (tt & 1) * XBUF + x_lane;
          const char* ab =
              xt_base + (ROLE == R_DV ? OFF_DOS + ob_prev * TILE : OFF_QS + (tt & 3) * TILE) + 64 * DT * dh;
          u32x4 bx[2][2];
  #pragma unroll
          for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
            for (int ks = 0; ks < 2; ++ks) bx[kb][ks] = *reinterpret_cast<const u32x4*>(xb + kb * 2048 + ks * 1024);
          u32x4 xt[2 * DT];   // A operand of MFMA step i: d tile DT dh + i >> 1, k-step i & 1
          constexpr int XA = 2 * DT < 3 ? 2 * DT : 3;   // operands read ahead
  #pragma unroll
          for (int i = 0; i < XA; ++i) xt[i] = lds_read_xtw<W>(ab, i & 1, i >> 1);
          sched_fence();
  #pragma unroll
          for (int i = 0; i < 2 * DT; ++i) {
            if (i + XA < 2 * DT) xt[i + XA] = lds_read_xtw<W>(ab, (i + XA) & 1, (i + XA) >> 1);
            sched_fence();
  #pragma unroll
            for (int kb = 0; kb < 2; ++kb)
              acc[kb][i >> 1] = mfma32x32x16_f16(__builtin_bit_cast(f16x8, xt[i]),
                                                 __builtin_bit_cast(f16x8, bx[kb][i & 1]), acc[kb][i >> 1]);
            sched_fence();
          }
        }
      } else {   // R_DP
        // s_st dS(t-1) = P(t-1) * x(t-1) (* ds_f) in fp16, published for the dK wave (and
        // stored for dQ)
        if (seen_tile(t - 1)) {
          const char* px = smem + OFF_PX + ((t - 1) & 1) * XBUF + x_lane;
          char* sx = smem + OFF_SX + ((t - 1) & 1) * XBUF + x_lane;
          // block (key group kA / 64, 32-row query tile of tile t-1) in the segment's
          // key-group-major layout, so that consecutive query tiles (this loop, and the four
          // waves of a dQ workgroup) touch consecutive blocks; the 16 bytes of (key block
          // kb, k-step ks) of lane (l32, hh) go to 16-byte slot
          // 64 (2 kb + ks) + 8 ((l32 / 4) ^ ks) + 2 (l32 % 4) + hh, so that each store
          // instruction fills one 1 KB quarter and the dQ kernel's transposing reads of the
          // block are free of bank conflicts
          const uint32_t blk = (uint32_t)(ds_blk0 + ((qstart + (t - 1) * BQ) >> 5)) * 4096u;
          // the published and stored values are s_st dS: the dS values themselves when
          // ds_f is 1 (the usual case, a wave-uniform branch), else rescaled first
          auto ds_block = [&](auto rescale) __attribute__((always_inline)) {
  #pragma unroll
            for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
              for (int ks = 0; ks < 2; ++ks) {
                const f16x8 pe = *reinterpret_cast<const f16x8*>(px + kb * 2048 + ks * 1024);
                float ds[8];
  #pragma unroll
                for (int i = 0; i < 8; ++i) ds[i] = __builtin_fmaf((float)pe[i], x_prev[kb][8 * ks + i], 0.f);
                if constexpr (decltype(rescale)::value) {
  #pragma unroll
                  for (int i = 0; i < 8; ++i) ds[i] *= ds_f;
                }
                const f16x8 dh = cvt8h(ds[0], ds[1], ds[2], ds[3], ds[4], ds[5], ds[6], ds[7]);
                *reinterpret_cast<f16x8*>(sx + kb * 2048 + ks * 1024) = dh;
                if (ds_on) {
                  const int sl = 64 * (2 * kb + ks) + 8 * ((l32 >> 2) ^ ks) + 2 * (l32 & 3) + hh;
                  // non-temporal (aux 2 = nt): the dQ kernel reads it once, after this kernel
                  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dh), dsr, (int)(blk + 16 * sl), 0, 2);
                }
              }
          };
          if (ds_f == 1.f)
            ds_block(std::false_type{});
          else
            ds_block(std::true_type{});
        }
        // x(t) = s_dp (dO(t) V^T - delta), from -delta * s_dp
        if (seen_tile(t)) {
          f32x16 xnew[2];
  #pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(dlt_base + (t & 1) * BQ + 8 * m);
  #pragma unroll
            for (int i = 0; i < 4; ++i) xnew[0][4 * m + i] = xnew[1][4 * m + i] = d4[i];
          }
          const char* ob = row_base + OFF_DOS + ob_cur * TILE;
          f16x8 oa[NS];
  #pragma unroll
          for (int s = 0; s < 3; ++s) oa[s] = *reinterpret_cast<const f16x8*>(ob + 32 * s);
          sched_fence();
  #pragma unroll
          for (int s = 0; s < NS; ++s) {
            if (s + 3 < NS) oa[s + 3] = *reinterpret_cast<const f16x8*>(ob + 32 * (s + 3));
            sched_fence();
  #pragma unroll
            for (int kb = 0; kb < 2; ++kb)
              xnew[kb] = mfma32x32x16_f16(oa[s], __builtin_bit_cast(f16x8, kv_op[kb][s]), xnew[kb]);
            sched_fence();
          }
          x_prev[0] = xnew[0];
          x_prev[1] = xnew[1];
        }
      }
      // tile t+1 into the buffers of tiles t-3 (Q) and t-2 (dO), last read in t-1
      store_tile(st, (t + 1) & 3, ob_next, (t + 1) & 1);
      ob_prev = ob_cur;
      ob_cur = ob_next;
      ob_next = ob_next == 2 ? 0 : ob_next + 1;
    };
    // unrolled by two so that each register set has a fixed name
    for (int t = 0; t <= nq + 1; t += 2) {
      trip(t, sa, sb);
      if (t + 1 <= nq + 1) trip(t + 1, sb, sa);
    }
    if (tid == 0) next_slot[0] = (int)gridDim.x + 8 * claimed + xcd;
    // all tiles done, the next index visible; the LDS tiles are free for the output
    // staging below
    __syncthreads();
    const KvItem nxt = kv_item(P, __builtin_amdgcn_readfirstlane(next_slot[0]), n_items);
    // the next item's first loads, in flight while this item's dK and dV leave
    set_rsrc(nxt);
    load_tile(sa, (nxt.k0 < nxt.p) ? 0 : nxt.k0);
    load_kv(nxt);
    // dV = acc / s_do, dK = scale * acc / (s_q s_st), rows staged through LDS
    if constexpr (ROLE == R_DV || ROLE == R_DK) {
      const __amdgpu_buffer_rsrc_t outr =
          ROLE == R_DV ? make_rsrc(P.dv + cs * P.dv_st + h * P.dv_sh + 32 * DT * dh, rows_bytes(L, P.dv_st, 32 * DT))
                       : make_rsrc(P.dk + cs * P.dk_st + h * P.dk_sh + 32 * DT * dh, rows_bytes(L, P.dk_st, 32 * DT));
      const uint32_t st2 = (uint32_t)(ROLE == R_DV ? P.dv_st : P.dk_st) * 2;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        store_rows_via_lds<DT, 2>(acc[kb], ROLE == R_DV ? 1.f / s_do : P.scale / s_q / s_st,
                                  smem + w * out_wave_bytes<DT>(), outr, kA + 32 * kb, st2, lane);
    }
    cur = nxt;
  }
}

// Persistent: gridDim.x workgroups (at most one per CU, a multiple of 8 when the list
// is longer than the grid), each running work items (segment, 128-key tile, head) until
// its XCD's share of the list is done. `counters` (8 ints) must be zero on entry.
template <int HD>
__global__ __launch_bounds__(kv::NT, 1) void prefixlm_bwd_dkdv_kernel(KvParams P) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // waves 0..3: S, dP, S, dP; waves 4..11: dV, dK, dV, dK (first half of head_dim), then
  // the same for the second half (waves w, w+4 and w+8 share a SIMD)
  if (w < 4) {
    if (w & 1)
      kv_wave<kv::R_DP, HD>(P, smem);
    else
      kv_wave<kv::R_S, HD>(P, smem);
  } else {
    if (w & 1)
      kv_wave<kv::R_DK, HD>(P, smem);
    else
      kv_wave<kv::R_DV, HD>(P, smem);
  }
}

// =====================================================================================
// dQ
// =====================================================================================
namespace qk {
constexpr int BQ = 128;                // queries per workgroup (32 per wave)
constexpr int BKT = 32;                // keys per tile
constexpr int NT = (BQ / 32) * 64;
template <int HD>
struct Geo {
  static constexpr int W = rsw_of<HD>();        // wide rows: conflict-free row and transposing reads
  static constexpr int TILE = BKT * W;
  static constexpr int OFF_KS = 0;              // [2] tiles: fp16 K * s_k
  static constexpr int OFF_VS = 2 * TILE;       // [2] tiles: bf16 V
  static constexpr int LDS_BYTES = 4 * TILE;
  static constexpr int NS = HD / 16;            // k-steps of S and dP
  static constexpr int NDT = HD / 32;           // 32-column d tiles of dQ
  static constexpr int CPR = HD / 8;            // 16-byte chunks per row
  static_assert(NT / 64 * out_wave_bytes<NDT>() <= LDS_BYTES, "output staging fits in LDS");
};
// Two workgroups per CU at head dim 128 (248 VGPRs); head dim 64 halves the Q, dO and
// dQ registers and the tiles and runs three.
template <int HD>
constexpr int occupancy() { return HD == 128 ? 2 : 3; }
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
template <int HD>
__global__ __launch_bounds__(qk::NT, qk::occupancy<HD>()) void prefixlm_bwd_dq_kernel(QParams P) {
  using namespace qk;
  using G = Geo<HD>;
  constexpr int D = HD, W = G::W, TILE = G::TILE, NS = G::NS, NDT = G::NDT, OFF_KS = G::OFF_KS,
                OFF_VS = G::OFF_VS;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int item, h;
  if (!unit_of(blockIdx.x, P.hdr->n_items, P.H, &item, &h)) return;
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
  u32x4 qf[NS], dof[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
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
    for (int s = 0; s < NS; ++s)
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
  for (int s = 0; s < NS; ++s) qf[s] = __builtin_bit_cast(u32x4, bf16x8_to_f16_scaled(qf[s], s_q));
  const float cq = P.scale_log2 / (s_q * s_k);
  // P * s_ds = exp2(S c - lse2 + log2 s_ds); s_ds is a power of two
  const float lse2s = lse2 - __builtin_log2f(s_ds);

  f32x16 acc[NDT];   // s_ds s_k dQ^T: [d 32dt + 8(r/4)+4hh+r%4][query l32]
#pragma unroll
  for (int t = 0; t < NDT; ++t)
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
  constexpr int SROWS = NT / G::CPR, SPASS = BKT / SROWS;
  static_assert(SROWS % 16 == 0, "staging rows srow + SROWS k keep the wide-row chunk offset");
  static_assert(SPASS >= 1 && SPASS * SROWS == BKT, "staging covers the key tile exactly");
  const int srow = tid / G::CPR, sch = tid % G::CPR;
  char* stage_base = smem + wrow_off<W>(srow) + sch * 16;
  // Loads run two tiles ahead of their LDS stores through two register sets, both
  // unconditional (rows past the segment read as zeros into buffers no wave reads
  // again); offsets stay below the host's 2 GiB check of (max_seqlen_all + 256) rows.
  struct Stage {
    u32x4 k[SPASS], v[SPASS];
  };
  auto load_tile = [&](Stage& st, int k0) {
#pragma unroll
    for (int k = 0; k < SPASS; ++k) {
      st.k[k] = buf_load16(kr, (uint32_t)(k0 + srow + SROWS * k) * kst2 + sch * 16);
      st.v[k] = buf_load16(vr, (uint32_t)(k0 + srow + SROWS * k) * vst2 + sch * 16);
    }
  };
  auto store_tile = [&](const Stage& st, int b) {
#pragma unroll
    for (int k = 0; k < SPASS; ++k) {
      // rows srow + SROWS k share wrow_off's chunk offset (SROWS is a multiple of 16)
      *reinterpret_cast<f16x8*>(stage_base + OFF_KS + b * TILE + SROWS * k * W) = bf16x8_to_f16_scaled(st.k[k], s_k);
      *reinterpret_cast<u32x4*>(stage_base + OFF_VS + b * TILE + SROWS * k * W) = st.v[k];
    }
  };
  const char* row_base = smem + wrow_off<W>(l32) + hh * 16;   // A operand rows: key row l32, d 16s + 8hh
  const char* xt_base = smem + xtw_lane_off<W>(lane);

  Stage sa, sb;
  load_tile(sa, 0);
  store_tile(sa, 0);
  load_tile(sb, BKT);
  // tile ik+2 into `ld` (the set of tile ik, stored already); tile ik+1 from `st` into
  // the other buffer, whose tile ik-1 was last read before this trip's barrier
  auto trip = [&](int ik, Stage& ld, const Stage& st) __attribute__((always_inline)) {
    const int B = ik & 1;
    const int kt0 = ik * BKT;
    __syncthreads();   // K/V tile ik visible in buffer B
    load_tile(ld, kt0 + 2 * BKT);
    if (kt0 < kw) {
      f32x16 sacc, pacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[r] = 0.f;
        pacc[r] = 0.f;
      }
      // S^T = K Q^T (fp16, scaled by s_k s_q), dP^T = V dO^T (bf16); K and V rows two
      // steps ahead of the MFMAs that use them
      f16x8 ka[NS];
      bf16x8 va[NS];
      auto rd = [&](int s) {
        ka[s] = *reinterpret_cast<const f16x8*>(row_base + OFF_KS + B * TILE + 32 * s);
        va[s] = *reinterpret_cast<const bf16x8*>(row_base + OFF_VS + B * TILE + 32 * s);
      };
      rd(0);
      rd(1);
      sched_fence();
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (s + 2 < NS) rd(s + 2);
        sched_fence();
        sacc = mfma32x32x16_f16(ka[s], __builtin_bit_cast(f16x8, qf[s]), sacc);
        pacc = mfma32x32x16(va[s], __builtin_bit_cast(bf16x8, dof[s]), pacc);
        sched_fence();
      }
      // transposed K operands of the dQ step (MFMA i: d tile i >> 1, k-step i & 1), the
      // first four in flight during the elementwise math
      u32x4 xt[2 * NDT];
#pragma unroll
      for (int i = 0; i < 4; ++i) xt[i] = lds_read_xtw<W>(xt_base + OFF_KS + B * TILE, i & 1, i >> 1);
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
      for (int i = 0; i < 2 * NDT; ++i) {
        if (i + 4 < 2 * NDT) xt[i + 4] = lds_read_xtw<W>(xt_base + OFF_KS + B * TILE, (i + 4) & 1, (i + 4) >> 1);
        sched_fence();
        acc[i >> 1] = mfma32x32x16_f16(__builtin_bit_cast(f16x8, xt[i]), db[i & 1], acc[i >> 1]);
        sched_fence();
      }
    }
    store_tile(st, B ^ 1);
  };
  for (int ik = 0; ik < nk; ik += 2) {
    trip(ik, sa, sb);
    if (ik + 1 < nk) trip(ik + 1, sb, sa);
  }

  // dq = scale * acc / (s_ds s_k), rows staged through LDS (free after this barrier)
  __syncthreads();
  {
    const __amdgpu_buffer_rsrc_t dqr = make_rsrc(P.dq + cs * P.dq_st + h * P.dq_sh, rows_bytes(L, P.dq_st, D));
    store_rows_via_lds<NDT, 2>(acc, P.scale / (s_ds * s_k), smem + w * out_wave_bytes<NDT>(), dqr, qA,
                            (uint32_t)P.dq_st * 2, lane);
  }
}

// =====================================================================================
// dQ from the stored dS
// =====================================================================================
// With a dS buffer the dK/dV kernel's dP waves also store dS (fp16, scaled per 128-key
// tile), and dQ = scale * dS K becomes a streaming product: no recomputation of S, P and
// dP, so the dQ kernel reads dS and K instead of Q, dO, K and V and runs a third of the
// MFMAs. Work item = (segment, 128-query tile, head), the dQ list; wave w owns queries
// q0 + 32w .. +31 and, per 64-key group, reads its own 4 KB dS block straight into LDS
// and the shared K tile (fp16 K * s_k, staged by all waves).
namespace q2 {
constexpr int BQ = 128;          // queries per workgroup (32 per wave)
constexpr int KG = 32;           // keys per step: half a stored block per wave
constexpr int NT = 256;
constexpr int BLK = 4096;        // one stored block: 32 queries x 64 keys fp16
constexpr int SBLK = KG * 64;    // bytes of a step's part of a block (keys 32 kb.. are bytes 2048 kb..)
constexpr int NDS = SBLK / 1024;    // direct loads (1 KB) of a step's dS per wave
constexpr int DS_AHEAD = 3;          // a step's dS is loaded this many steps ahead
constexpr int NDSB = DS_AHEAD + 1;   // dS buffers per wave
constexpr int MAX_KT = 256;      // 128-key tiles of a segment (the dS path needs max_seqlen_all <= 32768)
static_assert(KG == 32 || KG == 64, "a step is half a stored block or a whole one");
template <int HD>
struct Geo {
  static constexpr int RS = 2 * HD + 48;   // padded K rows, permuted (perm_row) for the transposing reads
  static constexpr int TILE = KG * RS;
  static constexpr int OFF_K = 0;          // [2] K tiles
  static constexpr int OFF_DS = 2 * TILE;  // [NDSB buffers][4 waves] a step's dS
  static constexpr int OFF_SC = OFF_DS + NDSB * 4 * SBLK;   // [MAX_KT] scales of the segment's key tiles
  static constexpr int LDS_BYTES = OFF_SC + MAX_KT * 4;
  static constexpr int NDT = HD / 32;      // 32-column d tiles of dQ
  static constexpr int CPR = HD / 8;       // 16-byte chunks per K row
  static constexpr int SROWS = NT / CPR;   // K rows per staging pass
  static constexpr int SPASS = KG / SROWS;
  static_assert(SROWS % 16 == 0 && SPASS * SROWS == KG, "staging rows keep perm_row's blocks");
  // the output staging reuses the tiles once every load has landed
  static_assert(NT / 64 * out_wave_bytes<NDT>() <= LDS_BYTES, "output staging fits in LDS");
};
// Lane part of the transposing read of B = dS^T (slot 8h + i of k-step s = key
// 16s + 8(i/4) + 4h + i%4, column = query l32) from a block in the layout the dK/dV
// kernel stores; ds_off adds k-step s and read half rd (keys +0..3 / +8..11).
__device__ __forceinline__ int ds_lane_off(int lane) {
  const int g = lane >> 4, j = lane & 15;
  const int key = 4 * (g >> 1) + (j >> 2), ks = g & 1;
  return 16 * (64 * ks + 8 * ((key >> 2) ^ ks) + 2 * (key & 3) + (j & 1)) + 8 * ((j & 3) >> 1);
}
__host__ __device__ constexpr int ds_off(int s, int rd) { return 2048 * (s >> 1) + 512 * (s & 1) + 256 * rd; }
}  // namespace q2

struct Q2Params {
  const bf16* k;
  const float* segstats;    // [numseqs, H, kSegStats] from the dK/dV kernel
  const char* ds;
  const float* ds_scale;
  const int32_t* ds_base;   // [numseqs + 1] first block of each segment
  bf16* dq;
  int64_t k_st, k_sh, dq_st, dq_sh;
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  const int2* items;
  const WsHeader* hdr;
  int T, H, is_causal;
  int numseqs;
  uint32_t ds_hbytes;
  int ds_nkslot;
  float scale;
};

template <int HD>
__global__ __launch_bounds__(q2::NT, 3) void prefixlm_bwd_dq_ds_kernel(Q2Params P) {
  using namespace q2;
  using G = Geo<HD>;
  constexpr int D = HD, RS = G::RS, TILE = G::TILE, NDT = G::NDT, SROWS = G::SROWS, SPASS = G::SPASS;
  static_assert(SPASS == 4 || SPASS == 2 || SPASS == 1, "K staging of 1, 2 or 4 loads per thread");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int item, h;
  if (!unit_of(blockIdx.x, P.hdr->n_items, P.H, &item, &h)) return;
  const int2 it = P.items[item];
  const int seg = it.x;
  if (seg < 0 || seg >= P.numseqs) return;
  const int cs = P.cu[seg];
  const int L = P.prefix[seg] + P.causal[seg];
  const int p = P.is_causal ? 0 : P.prefix[seg];
  const int q0 = it.y * BQ;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int qA = q0 + 32 * w;
  // keys [0, kend) are seen by some query of the workgroup, [0, kw) by this wave (none
  // when its rows are past the segment: their blocks were never stored)
  const int kend = max(p, min(L, q0 + BQ));
  const int kw = qA < L ? max(p, min(L, qA + 32)) : 0;
  const int nkg = (kend + KG - 1) / KG;

  const float s_k = pow2_scale(P.segstats[((int64_t)seg * P.H + h) * kSegStats]);
  // the scales of this segment's 128-key tiles (slots (cs >> 7) + seg + j), into LDS
  float* sc_lds = reinterpret_cast<float*>(smem + G::OFF_SC);
  {
    const int nkt = (kend + 127) >> 7;
    const float* scl = P.ds_scale + (int64_t)h * P.ds_nkslot + (cs >> 7) + seg;
    if (tid < nkt) sc_lds[tid] = scl[tid];
  }
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(P.k + cs * P.k_st + h * P.k_sh, rows_bytes(L, P.k_st, D));
  const uint32_t kst2 = (uint32_t)P.k_st * 2;
  const __amdgpu_buffer_rsrc_t dsr = make_rsrc(P.ds + (int64_t)h * P.ds_hbytes, P.ds_hbytes);
  // this wave's blocks: query tile qA / 32 of every key group (ds_blk_off; the layout
  // uses prefix_lens whatever is_causal); lane j moves bytes 16 j..
  const int ds_n32 = (L + 31) >> 5, ds_kpl = ds_kp(P.prefix[seg], L);
  const int ds_row = P.ds_base[seg] + (qA >> 5);
  const uint32_t lane_off = lane * 16;
  // K staging: thread = 16-byte chunk sch of stored rows srow + SROWS r, which hold keys
  // perm_row(srow) + SROWS r (perm_row is its own inverse)
  const int srow = tid / G::CPR, sch = tid % G::CPR;
  const uint32_t koff = (uint32_t)perm_row(srow) * kst2 + sch * 16;
  char* stage_base = smem + G::OFF_K + srow * RS + sch * 16;
  // All loads of the key loop are inline asm (the compiler tracks none of them), in one
  // order per step: K tile kg+2 (SPASS loads into registers), then the dS of step kg+3
  // (NDS direct loads into this wave's buffer (kg+3) % NDSB). A wait counts the loads
  // issued after the group it waits for; loads complete in order.
  struct Stage {
    u32x4 k[4];
  };
  // Steps past the last one re-read the last step's data (cache hits, no HBM traffic),
  // so every step issues the same loads.
  const int last_k = max(nkg - 1, 0), last_ds = max((kw + KG - 1) / KG - 1, 0);
  auto load_k = [&](Stage& st, int kg) {
    kg = min(kg, last_k);
#pragma unroll
    for (int r = 0; r < SPASS; ++r) st.k[r] = asm_load16(kr, (uint32_t)(KG * kg + SROWS * r) * kst2 + koff);
  };
  const uint32_t ds_lds = lds_addr(smem) + G::OFF_DS + w * SBLK;
  auto load_ds = [&](int kg) {
    const uint32_t lb = ds_lds + (uint32_t)(kg % NDSB) * 4 * SBLK;
    kg = min(kg, last_ds);
    const uint32_t go = (uint32_t)(ds_row + ds_blk_off(KG * kg / 64, ds_n32, ds_kpl)) * BLK +
                        (uint32_t)(KG * kg % 64) * 64 + lane_off;
#pragma unroll
    for (int n = 0; n < NDS; ++n) dma16_nt(dsr, __builtin_amdgcn_readfirstlane(lb + n * 1024), go + n * 1024);
  };
  // registers of a K tile, with N loads issued after everything the wait must cover
  auto wait_k = [&](Stage& st, auto n) {
    constexpr int N = decltype(n)::value;
    if constexpr (SPASS == 4)
      vm_wait<N>(st.k[0], st.k[1], st.k[2], st.k[3]);
    else if constexpr (SPASS == 2)
      vm_wait<N>(st.k[0], st.k[1]);
    else
      vm_wait<N>(st.k[0]);
  };
  auto store_k = [&](const Stage& st, int b) {
#pragma unroll
    for (int r = 0; r < SPASS; ++r)
      *reinterpret_cast<f16x8*>(stage_base + b * TILE + SROWS * r * RS) = bf16x8_to_f16_scaled(st.k[r], s_k);
  };

  f32x16 acc[NDT];   // c s_k dQ^T: [d 32dt + 8(r/4)+4hh+r%4][query l32], c the blocks' scale
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
  float c_cur = 0.f;

  const char* xt_base = smem + G::OFF_K + xt_lane_off<RS>(lane);
  const char* ds_base = smem + G::OFF_DS + w * SBLK + ds_lane_off(lane);

  Stage sa, sb;
  sched_fence();
  // prologue: K 0, dS 0, dS 1, K 1, dS 2; K 0 and the dS of steps 0 and 1 are waited
  // for here (K 1 and dS 2 follow them), the later steps' by the end-of-step waits
  load_k(sa, 0);
  load_ds(0);
  load_ds(1);
  load_k(sb, 1);
  load_ds(2);
  wait_k(sa, std::integral_constant<int, SPASS + NDS>{});
  store_k(sa, 0);
  // Step kg: K tile kg+2 and the dS of step kg+3 are issued, step kg's tiles (complete
  // since the end of step kg-1) are read, and K tile kg+1 goes from `st` to LDS.
  auto trip = [&](int kg, Stage& ld, Stage& st) __attribute__((always_inline)) {
    const int B = kg & 1;
    // step kg's K tile visible, every wave's reads of step kg-1 done (LDS-only barrier:
    // the loads in flight stay in flight)
    sched_fence();
    waitcnt<63, 0>();
    __builtin_amdgcn_s_barrier();
    sched_fence();
    load_k(ld, kg + 2);
    load_ds(kg + 3);
    sched_fence();
    if (kg * KG < kw) {
      // blocks of another 128-key tile may carry another scale: bring acc to it (powers
      // of two, exact)
      const float sc = sc_lds[(KG * kg) >> 7];
      if (sc != c_cur) {
        const float f = c_cur > 0.f ? sc / c_cur : 0.f;
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[t][r] *= f;
        c_cur = sc;
      }
      const char* db = ds_base + (kg % NDSB) * 4 * SBLK;
      constexpr int NKS = KG / 16;   // k-steps of the step
      u32x4 bq[NKS];
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const u32x2 x0 = lds_read_tr(db, ds_off(s, 0));
        const u32x2 x1 = lds_read_tr(db, ds_off(s, 1));
        bq[s] = u32x4{x0[0], x0[1], x1[0], x1[1]};
      }
      // dQ^T[d][q] += K^T[d][key] dS^T[key][q]: MFMA i = k-step i / NDT, d tile i % NDT,
      // K^T operands read three ahead
      constexpr int NM = NKS * NDT;
      const char* kb = xt_base + B * TILE;
      u32x4 xt[NM];
#pragma unroll
      for (int i = 0; i < 3; ++i) xt[i] = lds_read_xt<RS>(kb, i / NDT, i % NDT);
      sched_fence();
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        if (i + 3 < NM) xt[i + 3] = lds_read_xt<RS>(kb, (i + 3) / NDT, (i + 3) % NDT);
        sched_fence();
        acc[i % NDT] = mfma32x32x16_f16(__builtin_bit_cast(f16x8, xt[i]), __builtin_bit_cast(f16x8, bq[i / NDT]),
                                        acc[i % NDT]);
        sched_fence();
      }
    }
    // K tile kg+1 and everything issued before it (the dS of steps up to kg+1); issued
    // after it: the dS of step kg+2, K tile kg+2 and the dS of step kg+3
    wait_k(st, std::integral_constant<int, SPASS + 2 * NDS>{});
    store_k(st, B ^ 1);
  };
  for (int kg = 0; kg < nkg; kg += 2) {
    trip(kg, sa, sb);
    if (kg + 1 < nkg) trip(kg + 1, sb, sa);
  }

  // every load landed and every wave's reads done before the output staging; the K
  // registers are marked as written here, so that the compiler reuses none of them while
  // a load into them may still be in flight
  sched_fence();
  vm_wait<0>(sa.k[0], sa.k[1], sa.k[2], sa.k[3]);
  vm_wait<0>(sb.k[0], sb.k[1], sb.k[2], sb.k[3]);
  waitcnt<0, 0>();
  __syncthreads();
  {
    const __amdgpu_buffer_rsrc_t dqr = make_rsrc(P.dq + cs * P.dq_st + h * P.dq_sh, rows_bytes(L, P.dq_st, D));
    const float f = c_cur > 0.f ? P.scale / (c_cur * s_k) : 0.f;
    store_rows_via_lds<NDT, 2>(acc, f, smem + w * out_wave_bytes<NDT>(), dqr, qA, (uint32_t)P.dq_st * 2, lane);
  }
}

// =====================================================================================
// pre-pass and padding rows
// =====================================================================================
constexpr int kPreRows = 32;     // token rows per pre-pass workgroup
constexpr int kPreBatch = 8;     // row-heads per 16-lane group whose loads are in flight together
constexpr int kPreMaxHeads = 64; // per-head maxima kept in LDS

// delta[h, t] = sum_d dO[t,h,d] * (O + O_lo)[t,h,d] for t < total (0 for the other
// rows of the workgroup's range) and the per-head maxima max|dO|, max ||dO_t||_2,
// max |delta_t| and max |Q| (atomicMax on the bit patterns of non-negative floats;
// `stats` must be zero on entry). max |Q| comes from the forward's per-wave slots
// q_amax[0, q_slots) (slot b: wave b % 4 of the forward's grid index b / 4, head
// unit_head(b / 4, H); 0 for no rows), spread over the pre-pass's workgroups. A 16-lane group reduces one (row, head) at a time, HD / 8
// bytes per lane; the maxima are combined in LDS first so each workgroup issues 3
// global atomics per head. Rows past total read as zero through the buffer bounds.
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

template <int HD, bool GATED>
__global__ __launch_bounds__(256) void prefixlm_bwd_pre_kernel(
    const bf16* o, const int8_t* o_lo, const bf16* dout, int64_t o_st, int64_t o_sh, int64_t lo_st,
    int64_t lo_sh, int64_t do_st, int64_t do_sh, float* delta, float* stats, int T, int H, int total,
    GateBwd G, const float* q_amax, int q_slots) {
  static_assert(HD == 128 || !GATED, "the output gate is applied at head dim 128");
  constexpr int D = HD, NW = HD / 32;   // 32-bit words (bf16 pairs) per lane
  __shared__ int smax[kPreMaxHeads * kStats];
  const int t0 = blockIdx.x * kPreRows;
  const int rows = min(kPreRows, T - t0);
  const int tid = threadIdx.x;
  const int grp = tid >> 4, chunk = tid & 15;
  for (int i = tid; i < H * kStats; i += 256) smax[i] = 0;
  // this workgroup's share of the forward's max |Q| slots (at most one per thread when the
  // grid has at least q_slots / 256 workgroups), loaded now and folded in at the end
  const int q_per = (q_slots + (int)gridDim.x - 1) / (int)gridDim.x;
  const int qb = blockIdx.x * q_per + tid;
  const bool q_own = tid < q_per && qb < q_slots;
  const float qv = q_own ? q_amax[qb] : 0.f;
  __syncthreads();
  const int vrows = max(0, min(rows, total - t0));   // rows of this range below total
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(o + t0 * o_st, rows_bytes(vrows, o_st, (int)((H - 1) * o_sh + D)));
  const __amdgpu_buffer_rsrc_t lor =
      make_rsrc(o_lo ? static_cast<const void*>(o_lo + t0 * lo_st) : o,
                o_lo ? rows_bytes(vrows, lo_st, (int)((H - 1) * lo_sh + D), 1) : 0u);
  const __amdgpu_buffer_rsrc_t dor = make_rsrc(dout + t0 * do_st, rows_bytes(vrows, do_st, (int)((H - 1) * do_sh + D)));
  __amdgpu_buffer_rsrc_t gr = orr, dgr = orr, dar = orr;
  if constexpr (GATED) {
    gr = make_rsrc(G.gate + t0 * G.g_st, rows_bytes(vrows, G.g_st, (int)((H - 1) * G.g_sh + D)));
    // dgate and dO are written for every row of the range: 0 at rows >= total
    dgr = make_rsrc(G.dgate + t0 * G.dg_st, rows_bytes(rows, G.dg_st, (int)((H - 1) * G.dg_sh + D)));
    dar = make_rsrc(G.dout_attn + t0 * G.da_st, rows_bytes(rows, G.da_st, (int)((H - 1) * G.da_sh + D)));
  }
  const int n = rows * H;   // (row, head) pairs of this workgroup, head fastest
  // The group's pairs are grp, grp + 16, ...: its row t, head h and element offsets
  // (relative to row t0, which fit 32 bits by the host's check) advance by 16 pairs per
  // step, q16 rows and r16 heads with a carry when the head wraps, instead of a division
  // by H and 64-bit multiplies per pair.
  const int q16 = 16 / H, r16 = 16 - q16 * H;
  auto adv = [&](int64_t st, int64_t sh) { return (int)(q16 * st + r16 * sh); };
  auto wrap = [&](int64_t st, int64_t sh) { return (int)(st - (int64_t)H * sh); };
  const int dA_o = adv(o_st, o_sh), dW_o = wrap(o_st, o_sh);
  const int dA_do = adv(do_st, do_sh), dW_do = wrap(do_st, do_sh);
  const int dA_lo = adv(lo_st, lo_sh), dW_lo = wrap(lo_st, lo_sh);
  int pt = grp / H, ph = grp - (grp / H) * H;
  int off_o = (int)(pt * o_st + ph * o_sh), off_do = (int)(pt * do_st + ph * do_sh),
      off_lo = (int)(pt * lo_st + ph * lo_sh);
  // the last pair, whose data the steps past the range load again (as before: in range)
  const int last_o = (int)((rows - 1) * o_st + (H - 1) * o_sh), last_do = (int)((rows - 1) * do_st + (H - 1) * do_sh),
            last_lo = (int)((rows - 1) * lo_st + (H - 1) * lo_sh);
  for (int base = grp; base < n; base += 16 * kPreBatch) {
    // the residual codes of the lane's 2 NW elements: one byte each
    using LoPiece = std::conditional_t<HD == 128, u32x2, uint32_t>;
    Piece<HD> a[kPreBatch], b[kPreBatch];
    LoPiece r[kPreBatch];
    u32x4 gg[kPreBatch];
    int tj[kPreBatch], hj[kPreBatch];
#pragma unroll
    for (int j = 0; j < kPreBatch; ++j) {
      tj[j] = pt;
      hj[j] = ph;
      const bool in = pt < rows;   // pair base + 16 j < n
      const int oo = in ? off_o : last_o, od = in ? off_do : last_do, ol = in ? off_lo : last_lo;
      // O and its residual are read only here: non-temporal loads
      a[j] = load_piece<HD, 2>(orr, (uint32_t)((oo + chunk * 2 * NW) * 2));
      b[j] = load_piece<HD>(dor, (uint32_t)((od + chunk * 2 * NW) * 2));
      const int lo_off = ol + chunk * 2 * NW;
      if constexpr (HD == 128)
        r[j] = __builtin_amdgcn_raw_buffer_load_b64(lor, lo_off, 0, 2);
      else
        r[j] = __builtin_amdgcn_raw_buffer_load_b32(lor, lo_off, 0, 2);
      if constexpr (GATED) {
        const int t = in ? pt : rows - 1, h = in ? ph : H - 1;
        gg[j] = buf_load16(gr, (uint32_t)((t * G.g_st + h * G.g_sh + chunk * 8) * 2));
      }
      // step to pair base + 16 (j + 1)
      ph += r16;
      const bool w = ph >= H;
      ph -= w ? H : 0;
      pt += q16 + (w ? 1 : 0);
      off_o += dA_o + (w ? dW_o : 0);
      off_do += dA_do + (w ? dW_do : 0);
      off_lo += dA_lo + (w ? dW_lo : 0);
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
          const int t = tj[j], h = hj[j];
          buf_store16(b[j], dar, (uint32_t)((t * G.da_st + h * G.da_sh + chunk * 8) * 2));
          buf_store16(__builtin_bit_cast(u32x4, cvt8(dgv[0], dgv[1], dgv[2], dgv[3], dgv[4], dgv[5], dgv[6], dgv[7])),
                      dgr, (uint32_t)((t * G.dg_st + h * G.dg_sh + chunk * 8) * 2));
        }
      }
      float dot = 0.f, ss = 0.f, ma = 0.f;
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        // elements 2i and 2i + 1: bytes 2i and 2i + 1 of the codes
        uint32_t rw;
        if constexpr (HD == 128)
          rw = r[j][i >> 1];
        else
          rw = r[j];
        const int k0 = HD == 128 ? 2 * (i & 1) : 2 * i;
        const float o0 = lo_decode(bf16lo(a[j][i]), lo_byte(rw, k0));
        const float o1 = lo_decode(bf16hi(a[j][i]), lo_byte(rw, k0 + 1));
        const float d0 = bf16lo(b[j][i]), d1 = bf16hi(b[j][i]);
        dot += o0 * d0 + o1 * d1;
        ss += d0 * d0 + d1 * d1;
        ma = fmaxf(ma, fmaxf(__builtin_fabsf(d0), __builtin_fabsf(d1)));
      }
      dot = row16_sum(dot);
      ss = row16_sum(ss);
      ma = row16_max(ma);
      if (chunk == 0 && idx < n) {
        const int t = tj[j], h = hj[j];
        delta[(int64_t)h * T + t0 + t] = dot;
        atomicMax(&smax[h * kStats + 0], __builtin_bit_cast(int, ma));
        atomicMax(&smax[h * kStats + 1], __builtin_bit_cast(int, __builtin_sqrtf(ss)));
        atomicMax(&smax[h * kStats + 2], __builtin_bit_cast(int, __builtin_fabsf(dot)));
      }
    }
  }
  constexpr int QW = fwd::NT / 64;   // slots per forward workgroup
  if (qv > 0.f) atomicMax(&smax[unit_head(qb / QW, H) * kStats + 3], __builtin_bit_cast(int, qv));   // NaN: skipped
  // the rest of a larger share (fewer workgroups than q_slots / 256)
  for (int b = blockIdx.x * q_per + 256 + tid; b < min(q_slots, (blockIdx.x + 1) * q_per); b += 256) {
    const float v = q_amax[b];
    if (v > 0.f) atomicMax(&smax[unit_head(b / QW, H) * kStats + 3], __builtin_bit_cast(int, v));
  }
  __syncthreads();
  for (int i = tid; i < H * kStats; i += 256) {
    if (smax[i] != 0) atomicMax(reinterpret_cast<int*>(stats + i), smax[i]);
  }
}

// dq = dk = dv = 0 on rows total .. T-1 (one workgroup per row)
template <int HD>
__global__ __launch_bounds__(256) void prefixlm_bwd_pad_kernel(bf16* dq, bf16* dk, bf16* dv, int64_t dq_st,
                                                               int64_t dq_sh, int64_t dk_st, int64_t dk_sh,
                                                               int64_t dv_st, int64_t dv_sh, int H, int total) {
  constexpr int CPR = HD / 8;   // 16-byte chunks per (row, head)
  const int64_t t = total + (int64_t)blockIdx.x;
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int idx = threadIdx.x; idx < H * CPR; idx += 256) {
    const int h = idx / CPR, chunk = idx % CPR;
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
