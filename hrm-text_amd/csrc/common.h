// Shared device-side helpers for the gfx950 PrefixLM attention kernels.
//
// Conventions used by every kernel in this directory:
//   * q/k/v/out/dq/dk/dv are packed [T, H, D] bf16 with unit stride over D and
//     arbitrary (element) strides over tokens and heads;
//   * a segment s occupies token rows [cu[s], cu[s] + L) with L = prefix + causal;
//     local query i sees local key j iff j <= i or j < prefix (j <= i only when
//     is_causal), which is the union of the two FlashAttention passes of
//     models/flash_attention_prefixlm_v2.py:115-128 (reference);
//   * all global loads/stores of token rows go through raw buffer resources
//     whose size ends at the segment's last row, so rows past the segment read
//     as zero and writes past it are dropped by the hardware.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prefixlm {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Work-list header written by the prep kernel into the caller's workspace.
struct WsHeader {
  int32_t n_items;   // number of valid entries in the item array
  int32_t error;     // nonzero: inconsistent metadata was seen (bit flags)
  int32_t pad[14];
};
static_assert(sizeof(WsHeader) == 64, "header is one 64-byte line");

enum : int32_t {
  kErrBadSegment = 1,     // negative length / segment past total_seqlen / cu mismatch /
                          // longer than max_seqlen_all
  kErrCuStart = 2,        // cu_seqlens[0] != 0
  kErrDsCapacity = 4,     // the segments' stored-dS blocks exceed the buffer's capacity
};

// ---- grid index -> work unit ------------------------------------------------------
// The hardware deals the workgroups of a grid to the 8 XCDs round robin, so grid index b
// runs on XCD b % 8, as the j = b / 8-th workgroup of that XCD. A work unit is one
// (item, head); items are cost-ordered. XCD x owns heads x, x + 8, ... (F = H / 8 of
// them) for every item, and the r = H % 8 remaining heads are cut into q = 8 / gcd(r, 8)
// parts by item index mod q, r / gcd(r, 8) parts per XCD. Each XCD thus takes the same
// number of units per q items, in item (cost) order, and keeps its heads' rows in its own
// L2; with H % 8 == 0 this is the plain order b = item * H + head. Returns false for a
// unit past the n items (the valid units of an XCD are a prefix of its sequence).
__host__ __device__ inline int gcd8(int r) { return (r & 1) ? 1 : (r & 2) ? 2 : (r & 4) ? 4 : 8; }
__host__ __device__ inline bool unit_of(int b, int n, int H, int* item, int* head) {
  const int x = b & 7, j = b >> 3;
  const int F = H >> 3, r = H & 7;
  if (r == 0) {
    *item = j / F;
    *head = x + 8 * (j - *item * F);
    return *item < n;
  }
  const int g = gcd8(r), q = 8 / g, pr = r / g;
  const int per = F * q + pr;                 // units of XCD x per q consecutive items
  const int blk = j / per;
  int rem = j - blk * per;
  for (int c = 0; c < q; ++c) {
    const int i = blk * q + c;
    if (rem < F) {
      *item = i;
      *head = x + 8 * rem;
      return i < n;
    }
    rem -= F;
    for (int k = 0; k < pr; ++k) {
      const int part = x * pr + k;            // remainder head part / q, residue part % q
      if (part % q == c) {
        if (rem == 0) {
          *item = i;
          *head = 8 * F + part / q;
          return i < n;
        }
        --rem;
      }
    }
  }
  return false;
}
// Head of grid index b (the same for every item count n).
__host__ __device__ inline int unit_head(int b, int H) {
  int item = 0, head = 0;
  (void)unit_of(b, 0x7fffffff, H, &item, &head);
  return head;
}
// Grid indices that cover every unit of n items.
__host__ __device__ inline int64_t unit_grid(int64_t n, int H) {
  const int F = H >> 3, r = H & 7;
  if (r == 0) return n * H;
  const int g = gcd8(r), q = 8 / g, pr = r / g;
  return 8 * ((n + q - 1) / q) * (int64_t)(F * q + pr);
}

// ---- MFMA -------------------------------------------------------------------
// D(32x32 f32) += A(32x16 bf16) * B(16x32 bf16).
// Lane l holds A[l%32][8*(l/32) + 0..7] and B[8*(l/32) + 0..7][l%32]; the
// accumulator register r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Same shape and lane layout with fp16 operands.
__device__ __forceinline__ f32x16 mfma32x32x16_f16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ---- buffer resources ----------------------------------------------------------
// Raw (unstructured) buffer: byte offsets, reads past num_bytes return 0 and
// writes past it are discarded. Word 3 = 0x00020000 is the gfx9 raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ float buf_loadf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ void buf_store8(u32x2 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, 0);
}
__device__ __forceinline__ void buf_store16(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, 0);
}

// Bytes spanned by rows [0, L) of a [rows, ., D] bf16 view with token stride st
// (elements): the last row ends at ((L-1)*st + D) * 2.
__device__ __forceinline__ uint32_t rows_bytes(int L, int64_t st, int D, int elem_bytes = 2) {
  return L <= 0 ? 0u : (uint32_t)(((int64_t)(L - 1) * st + D) * elem_bytes);
}

// ---- out_lo: the rounding residual of O as int8 codes ------------------------------
// For o (fp32) and b = bf16(o) = m 2^e (m in [0.5, 1), e from frexp), the code is
// q = clamp(rint((o - b) 2^(16 - e)), -128, 127): the residual in units of 2^(e - 16), 1/256
// of b's bf16 ulp 2^(e - 8). |o - b| <= ulp / 2 keeps |q| <= 128 (128 saturates to 127),
// and b + q 2^(e - 16) recovers o to about 16 significant bits. b = 0 (|o| below half the
// smallest bf16 subnormal) gives q = 0; non-finite b decodes to itself or NaN.
__device__ __forceinline__ int lo_code(float o, float b) {
  // x >= -128 always (|o - b| <= ulp / 2); only +128 needs the clamp
  const float x = __builtin_rintf(__builtin_amdgcn_ldexpf(o - b, 16 - __builtin_amdgcn_frexp_expf(b)));
  return (int)__builtin_fminf(x, 127.f);
}
__device__ __forceinline__ float lo_decode(float b, int q) {
  // 2^(e - 16) from b's exponent bits: 2^(E - 127) * 2^-15 for biased exponent E = e + 126
  // (normal b; 0 for a subnormal b, whose residual is below 2^-133)
  const float s = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, b) & 0x7f800000u) * 0x1p-15f;
  return __builtin_fmaf((float)q, s, b);
}
// byte k (0..3) of w as a signed code
__device__ __forceinline__ int lo_byte(uint32_t w, int k) { return __builtin_amdgcn_sbfe((int)w, 8 * k, 8); }

// ---- packing ---------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack_lo(uint32_t a_lo_src, uint32_t b_hi_src) {
  // low 16 bits of a -> low half, low 16 bits of b -> high half
  return __builtin_amdgcn_perm(b_hi_src, a_lo_src, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a_lo_src, uint32_t b_hi_src) {
  // high 16 bits of a -> low half, high 16 bits of b -> high half
  return __builtin_amdgcn_perm(b_hi_src, a_lo_src, 0x07060302u);
}

__device__ __forceinline__ bf16x8 cvt8(float a0, float a1, float a2, float a3,
                                       float a4, float a5, float a6, float a7) {
  f32x8 v = {a0, a1, a2, a3, a4, a5, a6, a7};
  return __builtin_convertvector(v, bf16x8);
}
__device__ __forceinline__ f16x8 cvt8h(float a0, float a1, float a2, float a3,
                                       float a4, float a5, float a6, float a7) {
  f32x8 v = {a0, a1, a2, a3, a4, a5, a6, a7};
  return __builtin_convertvector(v, f16x8);
}
__device__ __forceinline__ uint32_t cvt2h_bits(float a0, float a1) {
  f32x4 v = {a0, a1, 0.f, 0.f};
  const f16x4 h = __builtin_convertvector(v, f16x4);
  return __builtin_bit_cast(u32x2, h)[0];
}
// bf16 held in the low / high half of a 32-bit word, as float
__device__ __forceinline__ float bf16lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Power of two s with x * s <= 2^14 and x * s > 2^13 (x > 0); 1 for x == 0 or
// non-finite x. Scaling by s is exact, and 2^14 leaves fp16 (max 65504) a 4x margin.
__device__ __forceinline__ float pow2_scale(float x) {
  if (!(x > 0.f) || !__builtin_isfinite(x)) return 1.f;
  int e;
  (void)frexpf(x, &e);   // x = m * 2^e with m in [0.5, 1)
  e = min(max(14 - e, -120), 120);
  return ldexpf(1.f, e);
}

__device__ __forceinline__ bf16x4 cvt4(float a0, float a1, float a2, float a3) {
  f32x4 v = {a0, a1, a2, a3};
  return __builtin_convertvector(v, bf16x4);
}

// Position of key (or query) u inside a 16-aligned group once bits 2 and 3 are
// swapped. Storing transposed tiles in this order makes the 8 contraction
// elements a lane needs for an MFMA step contiguous: with the accumulator
// layout above, lane half h holds rows {4h..4h+3} and {8+4h..8+4h+3} of each
// 16-row group, which this map sends to positions 8h..8h+7.
__device__ __forceinline__ int swz23(int u) {
  return (u & ~12) | ((u & 4) << 1) | ((u & 8) >> 1);
}

__device__ __forceinline__ float wave_xor32(float x) { return __shfl_xor(x, 32); }

// max / sum of x over lanes l and l ^ 32 through v_permlane32_swap (a VALU op; the
// shuffle above goes through LDS). Swapping two copies of x leaves lanes 0-31 holding
// (x[l], x[l+32]) and lanes 32-63 holding (x[l-32], x[l]), so every lane combines the
// same two operands as `x op wave_xor32(x)`, bitwise. Written as inline asm with the
// s_nop hazard waits the instruction needs around it (VALU write before, VALU read
// after), since the builtin's two results fold to one when both operands are equal.
__device__ __forceinline__ float halves_max(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 0\n\tv_max_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
}
__device__ __forceinline__ float halves_sum(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 0\n\tv_add_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
}

// ---- LDS tiles and MFMA operand movement -----------------------------------------
// LDS tiles hold rows of 128 16-bit values at a stride of RS = 304 bytes (256 data +
// 48 pad): consecutive rows start 12 banks apart, so the 16 lanes of one
// ds_read_b128 cycle reading 16 consecutive rows at one column cover all 64 banks.
// Every LDS address is a per-lane base plus a compile-time offset.
constexpr int RS = 304;

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4 of the
// 4-element vectors addressed by lanes i/4, 4+i/4, 8+i/4, 12+i/4 of its group.
__device__ __forceinline__ u32x2 lds_read_tr(const char* lds, int byte_off) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(
          (__attribute__((address_space(3))) char*)(lds) + byte_off));
  return __builtin_bit_cast(u32x2, v);
}

// Tiles read transposed permute their rows within each 16-row block: row
// 16b + 4a + m (a, m < 4) is stored at row 16b + 4m + a. One 32-lane cycle of
// ds_read_b64_tr_b16 reads 64-byte pieces of 4 consecutive rows 4a..4a+3; stored 4
// rows (48 banks) apart, the 4 pieces cover all 64 banks (unpermuted rows 12 banks
// apart overlap, a 2-way conflict).
__host__ __device__ __forceinline__ int perm_row(int r) { return (r & ~15) | ((r & 3) << 2) | ((r >> 2) & 3); }

// A operand X^T (32 rows of dimension d x 16 contraction slots) of a 32x32x16 MFMA,
// read from a row-major [row][d] tile with permuted rows (perm_row). Contraction slot
// 8h+i (h = lane/32) maps to tile row 16t + 8(i/4) + 4h + i%4, the row order of the
// accumulator registers 8t..8t+7 of a 32x32 MFMA result (see mfma32x32x16), so a
// result tile converts into the matching B operand without moving data between
// lanes. Lane l reads column 32*dt + l%32. `xt_base` = tile + xt_lane_off(lane); the
// stored row of tile row 16t + 8k + 4h + m is 16t + 4m + 2k + h.
// STRIDE: the tile's row stride in bytes.
template <int STRIDE = RS>
__device__ __forceinline__ int xt_lane_off(int lane) {
  const int a16 = (lane >> 4) & 3, r16 = lane & 15, h = a16 >> 1;
  return (4 * (r16 >> 2) + h) * STRIDE + (16 * (a16 & 1) + 4 * (r16 & 3)) * 2;
}
template <int STRIDE = RS>
__device__ __forceinline__ u32x4 lds_read_xt(const char* xt_base, int t, int dt) {
  const u32x2 x0 = lds_read_tr(xt_base, 16 * t * STRIDE + 64 * dt);
  const u32x2 x1 = lds_read_tr(xt_base, (16 * t + 2) * STRIDE + 64 * dt);
  const u32x4 r = {x0[0], x0[1], x1[0], x1[1]};
  return r;
}

// Keeps the compiler's scheduler from moving instructions across this point: LDS
// reads issued ahead of the MFMAs that consume them stay ahead.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// s_waitcnt for vmcnt <= VM and lgkmcnt <= LGKM (gfx9 encoding: vmcnt in bits 0-3 and
// 14-15, expcnt 4-6, lgkmcnt 8-11); VM = 63 or LGKM = 15 leaves that counter alone.
template <int VM, int LGKM>
__device__ __forceinline__ void waitcnt() {
  static_assert(VM >= 0 && VM <= 63 && LGKM >= 0 && LGKM <= 15, "counter range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | 0x70 | (LGKM << 8));
}

// Direct global -> LDS load of 16 bytes per lane: lane j writes bytes [16 j, 16 j + 16)
// after the wave-uniform LDS byte address `lds_addr` (M0). Inline asm, so the compiler's
// wait counters do not track it: the caller waits for it (vmcnt) before reading the LDS
// it writes; the compiler, not counting it, only ever waits longer than it needs to.
// Non-temporal (nt): for data read once.
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_addr, uint32_t voffset) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(voffset), "s"(rsrc)
      : "memory");
}
// 16-byte buffer load through inline asm, for loops whose loads the compiler must not
// track (its waits, counting only the loads it sees, would also wait for the direct
// loads above): the value is not there until the caller's vm_wait on it.
__device__ __forceinline__ u32x4 asm_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voffset), "s"(rsrc) : "memory");
  return v;
}
// s_waitcnt vmcnt(N) that also marks the given registers as written here, so that the
// compiler reads the asm_load16 results only after the wait.
template <int N>
__device__ __forceinline__ void vm_wait(u32x4& a) {
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(a) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}

// LDS byte address of a pointer into the kernel's LDS
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Marks a register value as used here, so the memory wait for the load that wrote it
// is placed here. Loads issued before a loop and first read inside it otherwise leave
// the loop's wait counters looking pending on every trip, and the compiler then waits
// for everything in flight, prefetches issued in the same trip included, before the
// first read.
__device__ __forceinline__ void settle(const u32x4& x) { asm volatile("" ::"v"(x)); }
// The same for arithmetic results: the value is computed before this point, which keeps
// VALU work placed between the MFMAs it is meant to run under (without it, instruction
// selection moves pure arithmetic next to its last use, across scheduling fences).
__device__ __forceinline__ void settle(float x) { asm volatile("" ::"v"(x)); }
// Marks x as rewritten (an empty asm that reads and writes it), so values the compiler
// derived from it before this point are not carried past it: they are derived again
// from x afterwards instead of holding registers in between.
__device__ __forceinline__ void renew(u32x4& x) { asm volatile("" : "+v"(x)); }

// Wide tile rows: LDS rows holding a row of data from 16-byte chunk
// f(r) = 4 (r & 3) + ((r >> 2) & 3) on. With 64 banks of 4 bytes, 16 rows read at one
// logical chunk (a b128 row read) land on 16 different chunk positions, and the
// transposing reads (4 rows x 16 consecutive bytes per row pair, 32 lanes) cover 16
// different chunks as well, so both are free of bank conflicts; the 304-byte rows
// above serve the first pattern only. Row r, logical chunk c sits at
// wrow_off(r) + 16 c. The stride is 512 bytes for 256-byte rows of data (head dim
// 128). 128-byte rows (head dim 64) use 384: rows 24 chunks apart shift the bank
// position by 8 chunks per odd row, which with f still sends the 16 rows of a row read
// and the 4 rows x 4 chunks of a transposing read to 16 different chunk positions.
constexpr int RSW = 512;
template <int HD>
constexpr int rsw_of() { return HD == 128 ? 512 : 384; }
template <int W = RSW>
__device__ __forceinline__ int wrow_off(int r) { return r * W + 16 * (4 * (r & 3) + ((r >> 2) & 3)); }
// lds_read_xt for wide rows: the row f(r) of the transposing read at tile row
// 16t + 8 half + 4h + m is 4m + h + 2 half, so the lane part and the (t, half, dt)
// part of the address still add.
template <int W = RSW>
__device__ __forceinline__ int xtw_lane_off(int lane) {
  const int a16 = (lane >> 4) & 3, r16 = lane & 15, h = a16 >> 1, m = r16 >> 2;
  return (4 * h + m) * W + 16 * (2 * (a16 & 1) + ((r16 & 3) >> 1) + 4 * m + h) + 8 * (r16 & 1);
}
template <int W = RSW>
__device__ __forceinline__ u32x4 lds_read_xtw(const char* xt_base, int t, int dt) {
  const u32x2 x0 = lds_read_tr(xt_base, 16 * t * W + 64 * dt);
  const u32x2 x1 = lds_read_tr(xt_base, (16 * t + 8) * W + 64 * dt + 32);
  const u32x4 r = {x0[0], x0[1], x1[0], x1[1]};
  return r;
}

// Sum / max over each 16-lane DPP row, every lane receiving its row's result. The
// steps pair lanes i^1, i^2 (quad permutations), then the two quads of each half-row
// (half-row mirror) and the two half-rows (row mirror): after the first two steps all
// lanes of a quad hold the same value, so this combines the same operands as a
// __shfl_xor tree over masks 1, 2, 4, 8, bitwise, without the trips through LDS. All
// 16 lanes of a row must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<0xB1>(x);    // quad_perm [1,0,3,2]
  x += dpp_f<0x4E>(x);    // quad_perm [2,3,0,1]
  x += dpp_f<0x141>(x);   // row_half_mirror
  x += dpp_f<0x140>(x);   // row_mirror
  return x;
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0x141>(x));
  x = fmaxf(x, dpp_f<0x140>(x));
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}

// 8 bf16 (as 4 words) -> 8 fp16 scaled by s
__device__ __forceinline__ f16x8 bf16x8_to_f16_scaled(u32x4 w, float s) {
  return cvt8h(bf16lo(w[0]) * s, bf16hi(w[0]) * s, bf16lo(w[1]) * s, bf16hi(w[1]) * s,
               bf16lo(w[2]) * s, bf16hi(w[2]) * s, bf16lo(w[3]) * s, bf16hi(w[3]) * s);
}
// 8 bf16 (as 4 words) -> 8 fp16, unscaled (exact for magnitudes in fp16's normal range)
__device__ __forceinline__ f16x8 bf16x8_to_f16(u32x4 w) {
  return cvt8h(bf16lo(w[0]), bf16hi(w[0]), bf16lo(w[1]), bf16hi(w[1]), bf16lo(w[2]), bf16hi(w[2]), bf16lo(w[3]),
               bf16hi(w[3]));
}
// 4 bf16 (as 2 words) -> 4 fp16, unscaled, as 2 words
__device__ __forceinline__ u32x2 bf16x4_to_f16(u32x2 w) {
  const u32x2 r = {cvt2h_bits(bf16lo(w[0]), bf16hi(w[0])), cvt2h_bits(bf16lo(w[1]), bf16hi(w[1]))};
  return r;
}
// 4 bf16 (as 2 words) -> 4 fp16 scaled by s, as 2 words
__device__ __forceinline__ u32x2 bf16x4_to_f16_scaled(u32x2 w, float s) {
  const u32x2 r = {cvt2h_bits(bf16lo(w[0]) * s, bf16hi(w[0]) * s), cvt2h_bits(bf16lo(w[1]) * s, bf16hi(w[1]) * s)};
  return r;
}

// Stores a wave's 32-row x (32 NDT) result (NDT 32x32 MFMA accumulators whose lane
// column l%32 is the output row and whose register rows are d) as bf16 rows scaled
// by f. The fragments go through the wave's own LDS area first, so that each store
// instruction writes whole rows (64 / (4 NDT) of them) instead of 16 bytes of 32 rows.
// Rows past the buffer's range are dropped by the hardware. AUX: the stores' cache policy
// (2 = non-temporal: the attention outputs and gradients are each read once, by a later
// kernel; measured faster for the next kernels, whose working sets they no longer evict).
constexpr int OUT_RS = 272;                 // LDS row stride of the output staging area (128 columns)
constexpr int OUT_WAVE_BYTES = 32 * OUT_RS;
// a wave's staging area for NDT 32-column tiles
template <int NDT>
constexpr int out_wave_bytes() { return 32 * (64 * NDT + 16); }
template <int NDT = 4, int AUX = 0>
__device__ __forceinline__ void store_rows_via_lds(const f32x16 (&acc)[NDT], float f, char* wave_lds,
                                                   __amdgpu_buffer_rsrc_t outr, int row0,
                                                   uint32_t row_stride_bytes, int lane) {
  constexpr int ORS = 64 * NDT + 16;        // staging row stride: the row's bytes + 16
  constexpr int CPR = 4 * NDT;              // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;             // rows per store instruction
  static_assert(32 * ORS == out_wave_bytes<NDT>(), "a wave's staging fills its area");
  const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bf16x4 o = cvt4(acc[dt][4 * m] * f, acc[dt][4 * m + 1] * f, acc[dt][4 * m + 2] * f,
                            acc[dt][4 * m + 3] * f);
      *reinterpret_cast<bf16x4*>(wave_lds + l32 * ORS + (32 * dt + 8 * m + 4 * hh) * 2) = o;
    }
#pragma unroll
  for (int k = 0; k < 32 / RPI; ++k) {
    const int row = lane / CPR + RPI * k;
    const u32x4 v = *reinterpret_cast<const u32x4*>(wave_lds + row * ORS + (lane % CPR) * 16);
    __builtin_amdgcn_raw_buffer_store_b128(v, outr, (int)((uint32_t)(row0 + row) * row_stride_bytes + (lane % CPR) * 16),
                                           0, AUX);
  }
}

// The out_lo codes of O = acc * f (lo_code against O's bf16 rounding) as int8 rows of
// 32 NDT bytes, staged like store_rows_via_lds and stored as whole 16-byte chunks
// (row_stride_bytes and the base must be multiples of 16).
template <int NDT = 4, int AUX = 0>
__device__ __forceinline__ void store_lo_rows_via_lds(const f32x16 (&acc)[NDT], float f, char* wave_lds,
                                                      __amdgpu_buffer_rsrc_t outr, int row0,
                                                      uint32_t row_stride_bytes, int lane) {
  constexpr int ORS = 32 * NDT + 16;        // staging row stride: the row's bytes + 16
  constexpr int CPR = 2 * NDT;              // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;             // rows per store instruction
  static_assert(32 * ORS <= out_wave_bytes<NDT>(), "a wave's staging fits its area");
  const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      uint32_t q[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float o = acc[dt][4 * m + i] * f;
        q[i] = (uint32_t)lo_code(o, (float)(bf16)o);
      }
      // low bytes of q0..q3 into one word (v_perm_b32 picks bytes of {src0, src1}, src1
      // the low half; selector 0x0c gives 0)
      const uint32_t lo2 = __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u);
      const uint32_t hi2 = __builtin_amdgcn_perm(q[3], q[2], 0x0c0c0400u);
      const uint32_t w = __builtin_amdgcn_perm(hi2, lo2, 0x05040100u);
      *reinterpret_cast<uint32_t*>(wave_lds + l32 * ORS + 32 * dt + 8 * m + 4 * hh) = w;
    }
#pragma unroll
  for (int k = 0; k < 32 / RPI; ++k) {
    const int row = lane / CPR + RPI * k;
    const u32x4 v = *reinterpret_cast<const u32x4*>(wave_lds + row * ORS + (lane % CPR) * 16);
    __builtin_amdgcn_raw_buffer_store_b128(v, outr, (int)((uint32_t)(row0 + row) * row_stride_bytes + (lane % CPR) * 16),
                                           0, AUX);
  }
}

// sigmoid(g) rounded to bf16, as torch.sigmoid returns it for a bf16 gate
__device__ __forceinline__ float sigmoid_bf16(float g) {
  return (float)(bf16)(1.f / (1.f + __expf(-g)));
}

// store_rows_via_lds for O, and also Y = sigmoid(gate) * O (both bf16, the product
// rounded once) for the same rows: the attention layer's output gate
// (models/layers.py:154) applied where O leaves the kernel. The gate chunks are
// loaded before O is staged so that their latency overlaps the staging.
__device__ __forceinline__ void store_rows_gated_via_lds(const f32x16 (&acc)[4], float f, char* wave_lds,
                                                         __amdgpu_buffer_rsrc_t outr, __amdgpu_buffer_rsrc_t gater,
                                                         __amdgpu_buffer_rsrc_t yr, int row0,
                                                         uint32_t o_stride_bytes, uint32_t g_stride_bytes,
                                                         uint32_t y_stride_bytes, int lane) {
  u32x4 g[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    g[k] = buf_load16(gater, (uint32_t)(row0 + (lane >> 4) + 4 * k) * g_stride_bytes + (lane & 15) * 16);
  const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bf16x4 o = cvt4(acc[dt][4 * m] * f, acc[dt][4 * m + 1] * f, acc[dt][4 * m + 2] * f,
                            acc[dt][4 * m + 3] * f);
      *reinterpret_cast<bf16x4*>(wave_lds + l32 * OUT_RS + (32 * dt + 8 * m + 4 * hh) * 2) = o;
    }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int row = (lane >> 4) + 4 * k;
    const u32x4 v = *reinterpret_cast<const u32x4*>(wave_lds + row * OUT_RS + (lane & 15) * 16);
    // O is read again only by the backward: non-temporal
    __builtin_amdgcn_raw_buffer_store_b128(v, outr, (int)((uint32_t)(row0 + row) * o_stride_bytes + (lane & 15) * 16), 0, 2);
    float y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[2 * i] = sigmoid_bf16(bf16lo(g[k][i])) * bf16lo(v[i]);
      y[2 * i + 1] = sigmoid_bf16(bf16hi(g[k][i])) * bf16hi(v[i]);
    }
    buf_store16(__builtin_bit_cast(u32x4, cvt8(y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7])), yr,
                (uint32_t)(row0 + row) * y_stride_bytes + (lane & 15) * 16);
  }
}

}  // namespace prefixlm
