// Projection GEMMs of the HRM block with the RMSNorm before them and the SwiGLU after
// them fused in (models/transformer.py:87-92 pre-norm, models/layers.py:124-135 gqkv
// projection, :158-168 gate_up projection and SwiGLU).
//
//   y = rmsnorm(x) W^T                         (PLAIN: the attention's gqkv projection)
//   y = silu(rmsnorm(x) Wg^T) * (rmsnorm(x) Wu^T)   (SWIGLU: the MLP's gate_up + SwiGLU)
//
// x: bf16 [M, K] (row stride ldx), W: bf16 [N, K] (row stride ldw; for SWIGLU the first
// F rows are the gate, the next F rows the up projection, N = 2F), y: bf16 [M, Nout]
// (Nout = N, or F for SWIGLU). The weightless RMSNorm is a per-row scale,
// rmsnorm(x) W^T = diag(r) (x W^T) with r = (mean(x^2) + eps)^(-1/2), so the kernel
// multiplies x's raw rows (never writing the normalized x) and applies r, read from
// `rstd` (one fp32 per row, from a row pass before the GEMM), to the fp32 products.
// With norm off, r = 1. Each output is rounded to bf16 once.
//
// Workgroup: 256 x rows by 256 W rows, 8 waves (two per SIMD) of 128 x rows by 64 W rows,
// K in stages of 64 staged by direct global->LDS loads (two stages: the next one lands
// while this one is read). Every wave computes Y^T tiles (A = W rows, B = x rows; lane =
// output row, registers = output columns), so a gate tile and its up tile meet in the
// same lanes and the epilogue stores whole rows.
#pragma once
#include "common.h"

namespace prefixlm {
namespace mlp {

constexpr int MT = 256;              // x rows per workgroup
constexpr int WT = 256;              // W rows per workgroup
constexpr int KT = 64;               // K per stage (four MFMA k steps between barriers)
constexpr int NSTAGE = 128 / KT;     // LDS stages (128 KB in all): one in flight while one is read
constexpr int KS = KT / 16;          // MFMA k steps per stage
constexpr int NTH = 512;             // 8 waves, two per SIMD
constexpr int ROWB = KT * 2;         // bytes of one staged row
constexpr int CPR = ROWB / 16;       // 16-byte chunks per staged row
constexpr int RPW = 256 / ROWB;      // staged rows per 256-byte bank window
constexpr int RPB = 1024 / ROWB;     // staged rows per 1 KB direct load
constexpr int NDMA = 32 / RPB;       // direct loads per wave, operand and stage (32 rows)
constexpr int A_BYTES = MT * ROWB;   // x tile
constexpr int B_BYTES = WT * ROWB;   // W tile
constexpr int STAGE = A_BYTES + B_BYTES;
constexpr int LDS_BYTES = NSTAGE * STAGE;   // the output staging reuses it
constexpr int OUT_RS = 64 * 2 + 16;         // output staging row: 64 bf16 + 16 B pad
static_assert(KS % 2 == 0 && CPR * RPW == 16 && NSTAGE >= 2, "stage geometry");
static_assert(8 * 32 * OUT_RS <= LDS_BYTES && NDMA >= 1, "output staging fits in LDS");

// Staged row r, logical 16-byte chunk c lives at r * ROWB + 16 (c ^ f(r)),
// f(r) = (r / RPW) % CPR: the 16 rows of one quarter-wave operand read (a fixed chunk)
// land on 16 different 16-byte positions of the 256-byte bank window, so the operand
// reads are free of bank conflicts.
__device__ __forceinline__ int swz_f(int r) { return (r / RPW) % CPR; }

struct Params {
  const bf16* x;
  const bf16* w;
  bf16* y;
  const float* rstd;   // [M] row scales (NORM)
  int64_t ldx, ldw, ldy;
  int M, K, N;       // N: W rows (2F for SWIGLU)
  int m_tiles, n_tiles;
};

template <bool SWIGLU, bool NORM>
__global__ __launch_bounds__(NTH, 1) void proj_gemm_kernel(Params P) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // XCD-aware order: XCD b % 8 runs the m tiles congruent to it mod 8. Its workgroups
  // take them in groups of 8 m tiles; within a group, 32 consecutive workgroups (one per
  // CU of the XCD, running together) cover 8 m tiles x 4 n tiles, so each x slice is
  // shared by 4 of them and each W slice by 8 in the XCD's L2.
  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int per_group = 8 * ((P.n_tiles + 3) / 4 * 4);
  const int grp = j / per_group, r = j - grp * per_group;
  const int nt = 4 * (r >> 5) + (r & 3);
  const int mt = xcd + 8 * (8 * grp + ((r & 31) >> 2));
  if (mt >= P.m_tiles || nt >= P.n_tiles) return;
  const int m0 = mt * MT;
  const int F = P.N >> 1;
  // W rows of this tile: SWIGLU: gate rows n0..n0+127 then up rows F+n0..; PLAIN: n0..n0+255
  const int n0 = nt * (SWIGLU ? WT / 2 : WT);

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wm = w >> 2, wn = w & 3;   // 2 x 4 waves of 128 x rows by 64 W rows

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(P.x + (int64_t)m0 * P.ldx,
                                              rows_bytes(min(MT, P.M - m0), P.ldx, P.K));
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(P.w, rows_bytes(P.N, P.ldw, P.K));

  // Direct global -> LDS loads: one instruction moves RPB rows (1 KB); lane L writes
  // slot L % CPR of row RPB i + L / CPR, which holds logical chunk (L % CPR) ^ f(row).
  // Wave w loads rows 32 w .. 32 w + 31 of both tiles (NDMA instructions each).
  uint32_t xoff[NDMA], woff[NDMA];
  {
    // W rows of the wave's 32: SWIGLU waves 0-3 the gate rows, 4-7 the up rows
    const int wbase = SWIGLU ? (w < 4 ? n0 + 32 * w : F + n0 + 32 * (w - 4)) : n0 + 32 * w;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int tr = 32 * w + RPB * i + lane / CPR;   // tile row
      const int ch = (lane % CPR) ^ swz_f(tr);
      xoff[i] = (uint32_t)((int64_t)tr * P.ldx * 2) + ch * 16;
      woff[i] = (uint32_t)((int64_t)(wbase + RPB * i + lane / CPR) * P.ldw * 2) + ch * 16;
    }
  }
  typedef __attribute__((address_space(3))) char lds_char;
  auto issue_stage_at = [&](int buf, int kk) {
    lds_char* base = (lds_char*)smem + buf * STAGE + 32 * w * ROWB;
    const uint32_t k2 = (uint32_t)(kk * ROWB);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(base + 1024 * i), 16,
                                               xoff[i] + k2, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (__attribute__((address_space(3))) void*)(base + A_BYTES + 1024 * i),
                                               16, woff[i] + k2, 0, 0, 0);
    }
  };

  // operand reads: A = W rows (lane = W row of the tile), B = x rows (lane = x row);
  // logical chunk 2 ks + hh of k step ks, at 16 ((2 ks + hh) ^ f(l32)) of the row (the
  // operand row bases are multiples of 32)
  int coff[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) coff[ks] = 16 * ((2 * ks + hh) ^ swz_f(l32));
  // W tile rows of A operand bi: SWIGLU: bi = 0 the gate rows 32 wn, bi = 1 the up rows
  // 128 + 32 wn of the same output columns; PLAIN: 64 wn + 32 bi
  auto a_row = [&](int bi) { return SWIGLU ? bi * (WT / 2) + 32 * wn : 64 * wn + 32 * bi; };
  const int brow0 = 128 * wm;   // x rows of B operand mi: brow0 + 32 mi

  f32x16 acc[4][2];   // [mi: x rows][bi: W rows]; Y^T tiles (register = W row, lane = x row)
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][bi][r] = 0.f;

  const int nk = P.K / KT;
  // LDS reads of k step ks of stage kk into fragment set `set`
  bf16x8 af[2][2], bfr[2][4];
  auto rd = [&](int kk, int ks, int set) {
    const char* abase = smem + (kk % NSTAGE) * STAGE + A_BYTES + l32 * ROWB + coff[ks];
    const char* bbase = smem + (kk % NSTAGE) * STAGE + l32 * ROWB + coff[ks];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[set][i] = *reinterpret_cast<const bf16x8*>(abase + a_row(i) * ROWB);
#pragma unroll
    for (int i = 0; i < 4; ++i) bfr[set][i] = *reinterpret_cast<const bf16x8*>(bbase + (brow0 + 32 * i) * ROWB);
  };
  // MFMAs of x operands mi in [m_lo, m_hi) of fragment set `set`
  auto mm_part = [&](int set, int m_lo, int m_hi) {
#pragma unroll
    for (int mi = m_lo; mi < m_hi; ++mi)
#pragma unroll
      for (int bi = 0; bi < 2; ++bi) acc[mi][bi] = mfma32x32x16(af[set][bi], bfr[set][mi], acc[mi][bi]);
  };
  // Stage loads past the last stage re-read the last one into a buffer nobody reads
  // again, so every stage has the same loads in flight and the loop body has no branch
  // (a branch would let the compiler sink the reads below the MFMAs they should overlap
  // and make it wait for all of them).
  auto issue = [&](int kk) { issue_stage_at(kk % NSTAGE, min(kk, nk - 1)); };
  // waits until this wave's loads of the oldest stage in flight are in LDS (the
  // NSTAGE - 2 younger stages stay in flight), then a plain barrier (no memory fence:
  // it would also wait for the younger stages)
  auto stage_barrier = [&]() {
    sched_fence();
    waitcnt<2 * NDMA * (NSTAGE - 2), 0>();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    sched_fence();
  };
#pragma unroll
  for (int s = 0; s < NSTAGE - 1; ++s) issue(s);
  stage_barrier();   // stage 0 in LDS
  issue(NSTAGE - 1);
  rd(0, 0, 0);
  // Stage kk: k steps 0 .. KS-1, each step's MFMAs running over the next step's reads.
  // In the last step, after the first MFMAs, stage kk + 1 is waited for, the workgroup
  // syncs, stage kk + NSTAGE is issued into the buffer of stage kk (every wave's reads of
  // it are done), and the reads of stage kk + 1's first step run under the remaining
  // MFMAs. (Each step's first MFMAs come before the next reads are issued, so the wait
  // for their operands does not also wait for the reads issued after them.)
  for (int kk = 0; kk < nk; ++kk) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int set = ks & 1;
      sched_fence();
      mm_part(set, 0, 1);
      sched_fence();
      if (ks + 1 < KS) {
        rd(kk, ks + 1, set ^ 1);
      } else if (kk + 1 < nk) {
        stage_barrier();
        issue(kk + NSTAGE);
        rd(kk + 1, 0, set ^ 1);
      }
      sched_fence();
      mm_part(set, 1, 4);
    }
  }
  waitcnt<0, 15>();   // no stage load left in flight
  __syncthreads();

  // ---- epilogue ------------------------------------------------------------------
  float r4[4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int row = min(m0 + brow0 + 32 * mi + l32, P.M - 1);
    r4[mi] = NORM ? P.rstd[row] : 1.f;
  }
  char* wl = smem + w * 32 * OUT_RS;
  constexpr int NOT = SWIGLU ? 1 : 2;                      // output 32-column tiles of the wave
  const int ycol0 = SWIGLU ? nt * (WT / 2) + 32 * wn : n0 + 64 * wn;
  const __amdgpu_buffer_rsrc_t yr = make_rsrc(P.y + (int64_t)m0 * P.ldy,
                                              rows_bytes(min(MT, P.M - m0), P.ldy, SWIGLU ? F : P.N));
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const float r = r4[mi];
    // lane holds columns 8 (reg / 4) + 4 hh + reg % 4 of each 32-column tile
#pragma unroll
    for (int ti = 0; ti < NOT; ++ti)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (SWIGLU) {
            const float g = acc[mi][0][4 * q + e] * r, u = acc[mi][1][4 * q + e] * r;
            o[e] = g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e)) * u;
          } else {
            o[e] = acc[mi][ti][4 * q + e] * r;
          }
        }
        *reinterpret_cast<bf16x4*>(wl + l32 * OUT_RS + (32 * ti + 8 * q + 4 * hh) * 2) = cvt4(o[0], o[1], o[2], o[3]);
      }
    // 32 rows x 32 NOT columns: chunk (lane % CPO) of row (lane / CPO) + RPP k
    constexpr int CPO = 32 * NOT / 8;                      // 16-byte chunks per output row
    constexpr int RPP = 64 / CPO;                          // rows per pass
#pragma unroll
    for (int k = 0; k < 32 / RPP; ++k) {
      const int rr = lane / CPO + RPP * k, ch = lane % CPO;
      const u32x4 v = *reinterpret_cast<const u32x4*>(wl + rr * OUT_RS + ch * 16);
      buf_store16(v, yr, (uint32_t)((int64_t)(brow0 + 32 * mi + rr) * P.ldy * 2) + (uint32_t)(ycol0 * 2 + ch * 16));
    }
  }
}

}  // namespace mlp
}  // namespace prefixlm
