// Rotary position embedding on packed [T, heads, 128] bf16 rows, the prologue the
// reference's attention layer runs before the attention op (models/layers.py:23-38,
// :138-140), and its adjoint for the backward.
//
// Forward, half-split layout (rotate_half, :23-27), per row t and dimension d < 64:
//   y[d]    = x[d]    * cos[t][d]    + (-x[d+64]) * sin[t][d]
//   y[d+64] = x[d+64] * cos[t][d+64] +   x[d]     * sin[t][d+64]
// in fp32 from the bf16 inputs and fp32 cos/sin, each product and the sum rounded
// to fp32 as two multiplies and an add (no fused multiply-add), then rounded to
// bf16: the operation order of apply_rotary_pos_emb (:36), so the result is
// bitwise that of the reference's fp32 RoPE.
// Backward (the transpose of the rotation), rounded once to bf16:
//   dx[d]    = dy[d] * cos[t][d] + dy[d+64] * sin[t][d+64]
//   dx[d+64] = dy[d+64] * cos[t][d+64] - dy[d] * sin[t][d]
// One thread handles the 8-element chunks [8c, 8c+8) and [64+8c, 64+8c+8) of one
// (row, head); y may alias x (in-place).
#pragma once
#include "common.h"

namespace prefixlm {
namespace rope {

constexpr int D = 128;

struct Params {
  const bf16* x;
  bf16* y;
  const float* cos;
  const float* sin;
  int64_t x_st, x_sh, y_st, y_sh, cs_st;   // element strides; cos/sin rows of D floats
  int T, nh, backward;
};

__device__ __forceinline__ f32x8 load8f(const float* p) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
  return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ f32x8 unpack8(u32x4 w) {
  return f32x8{bf16lo(w[0]), bf16hi(w[0]), bf16lo(w[1]), bf16hi(w[1]),
               bf16lo(w[2]), bf16hi(w[2]), bf16lo(w[3]), bf16hi(w[3])};
}

__global__ __launch_bounds__(256) void rope_kernel(Params P) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int c = (int)(gid & 7);
  const int64_t rh = gid >> 3;
  if (rh >= (int64_t)P.T * P.nh) return;
  const int t = (int)(rh / P.nh), h = (int)(rh - (int64_t)t * P.nh);
  const bf16* xp = P.x + t * P.x_st + h * P.x_sh;
  const f32x8 lo = unpack8(*reinterpret_cast<const u32x4*>(xp + 8 * c));
  const f32x8 hi = unpack8(*reinterpret_cast<const u32x4*>(xp + 64 + 8 * c));
  const float* cp = P.cos + t * P.cs_st;
  const float* sp = P.sin + t * P.cs_st;
  const f32x8 c_lo = load8f(cp + 8 * c), c_hi = load8f(cp + 64 + 8 * c);
  const f32x8 s_lo = load8f(sp + 8 * c), s_hi = load8f(sp + 64 + 8 * c);
  float r_lo[8], r_hi[8];
  if (!P.backward) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      r_lo[i] = lo[i] * c_lo[i] + (-hi[i]) * s_lo[i];
      r_hi[i] = hi[i] * c_hi[i] + lo[i] * s_hi[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      r_lo[i] = lo[i] * c_lo[i] + hi[i] * s_hi[i];
      r_hi[i] = hi[i] * c_hi[i] - lo[i] * s_lo[i];
    }
  }
  bf16* yp = P.y + t * P.y_st + h * P.y_sh;
  *reinterpret_cast<bf16x8*>(yp + 8 * c) = cvt8(r_lo[0], r_lo[1], r_lo[2], r_lo[3], r_lo[4], r_lo[5], r_lo[6], r_lo[7]);
  *reinterpret_cast<bf16x8*>(yp + 64 + 8 * c) =
      cvt8(r_hi[0], r_hi[1], r_hi[2], r_hi[3], r_hi[4], r_hi[5], r_hi[6], r_hi[7]);
}

}  // namespace rope
}  // namespace prefixlm
