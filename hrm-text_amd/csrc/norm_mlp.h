// Elementwise kernels of the HRM block around the attention layer: the SwiGLU
// activation (models/layers.py:166-168, `F.silu(gate) * up` on the two halves of the
// gate/up projection) and the weightless RMSNorm of the pre-norm block
// (models/transformer.py:87, `F.rms_norm(x, (N,), eps)`), forward and backward.
//
// All four are HBM-bound: one pass over their inputs and outputs, fp32 arithmetic,
// one bf16 rounding per output. The SwiGLU backward writes the gradient of the whole
// [T, 2F] projection output in place, so no concatenation of the two halves follows.
#pragma once
#include "common.h"

namespace prefixlm {
namespace nm {

// ---- SwiGLU -------------------------------------------------------------------------
// gu: [rows, 2F] (gate columns [0, F), up columns [F, 2F)); y, dy: [rows, F];
// dgu: [rows, 2F]. Row strides in elements; F % 8 == 0.
struct SwigluParams {
  const bf16* gu;
  const bf16* dy;
  bf16* y;
  bf16* dgu;
  int64_t gu_st, y_st, dy_st, dgu_st;
  int64_t rows, cols;
};

__device__ __forceinline__ float sigmoid_f32(float g) {
  // 1 / (1 + e^-g); e^-g overflows to inf for g < -88, giving 0 as the limit does
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e));
}

__device__ __forceinline__ void unpack8(const u32x4& w, float* f) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = bf16lo(w[e]);
    f[2 * e + 1] = bf16hi(w[e]);
  }
}

// thread = 8 consecutive columns of one row
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(SwigluParams P) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t c8 = P.cols >> 3;
  if (idx >= P.rows * c8) return;
  const int64_t r = idx / c8, c = (idx - r * c8) * 8;
  const bf16* g_row = P.gu + r * P.gu_st;
  float g[8], u[8], y[8];
  unpack8(*reinterpret_cast<const u32x4*>(g_row + c), g);
  unpack8(*reinterpret_cast<const u32x4*>(g_row + P.cols + c), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = g[e] * sigmoid_f32(g[e]) * u[e];
  *reinterpret_cast<bf16x8*>(P.y + r * P.y_st + c) = cvt8(y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]);
}

// d/dg [g s(g) u] = u s (1 + g (1 - s)), d/du = g s(g)
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(SwigluParams P) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t c8 = P.cols >> 3;
  if (idx >= P.rows * c8) return;
  const int64_t r = idx / c8, c = (idx - r * c8) * 8;
  const bf16* g_row = P.gu + r * P.gu_st;
  float g[8], u[8], dy[8], dg[8], du[8];
  unpack8(*reinterpret_cast<const u32x4*>(g_row + c), g);
  unpack8(*reinterpret_cast<const u32x4*>(g_row + P.cols + c), u);
  unpack8(*reinterpret_cast<const u32x4*>(P.dy + r * P.dy_st + c), dy);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s = sigmoid_f32(g[e]);
    dg[e] = dy[e] * u[e] * s * (1.f + g[e] * (1.f - s));
    du[e] = dy[e] * g[e] * s;
  }
  bf16* d_row = P.dgu + r * P.dgu_st;
  *reinterpret_cast<bf16x8*>(d_row + c) = cvt8(dg[0], dg[1], dg[2], dg[3], dg[4], dg[5], dg[6], dg[7]);
  *reinterpret_cast<bf16x8*>(d_row + P.cols + c) = cvt8(du[0], du[1], du[2], du[3], du[4], du[5], du[6], du[7]);
}

// ---- RMSNorm (no weight) ------------------------------------------------------------
// y = x r, r = (mean(x^2) + eps)^(-1/2) per row; r is kept (fp32 [rows]) for the backward:
// dx = r dy - x r^3 (sum(dy x) / N).
constexpr int kNormMaxChunks = 16;          // 16-byte chunks per lane: rows up to 64 * 16 * 8 = 8192
constexpr int kNormMaxCols = 64 * kNormMaxChunks * 8;

struct NormParams {
  const bf16* x;
  const bf16* dy;
  bf16* y;
  bf16* dx;
  float* rstd;
  int64_t x_st, y_st, dy_st, dx_st;
  int64_t rows;
  int cols;
  float eps;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// one wave per row, 4 rows per workgroup; the row stays in registers between the passes
// (NCH 16-byte chunks per lane, the smallest power of two covering the row)
template <int NCH>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(NormParams P) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= P.rows) return;
  const int lane = threadIdx.x & 63, nc = P.cols >> 3;
  const bf16* xr = P.x + row * P.x_st;
  u32x4 xv[NCH];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nc) {
      xv[k] = *reinterpret_cast<const u32x4*>(xr + 8 * c);
      float f[8];
      unpack8(xv[k], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
  ss = wave_sum(ss);
  const float r = __builtin_amdgcn_rsqf(ss / (float)P.cols + P.eps);
  if (lane == 0) P.rstd[row] = r;
  if (P.y == nullptr) return;   // the row scales only (the projection GEMM applies them)
  bf16* yr = P.y + row * P.y_st;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nc) {
      float f[8];
      unpack8(xv[k], f);
      *reinterpret_cast<bf16x8*>(yr + 8 * c) =
          cvt8(f[0] * r, f[1] * r, f[2] * r, f[3] * r, f[4] * r, f[5] * r, f[6] * r, f[7] * r);
    }
  }
}

template <int NCH>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(NormParams P) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= P.rows) return;
  const int lane = threadIdx.x & 63, nc = P.cols >> 3;
  const bf16* xr = P.x + row * P.x_st;
  const bf16* dyr = P.dy + row * P.dy_st;
  u32x4 xv[NCH], dv[NCH];
  float sd = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nc) {
      xv[k] = *reinterpret_cast<const u32x4*>(xr + 8 * c);
      dv[k] = *reinterpret_cast<const u32x4*>(dyr + 8 * c);
      float fx[8], fd[8];
      unpack8(xv[k], fx);
      unpack8(dv[k], fd);
#pragma unroll
      for (int e = 0; e < 8; ++e) sd += fd[e] * fx[e];
    }
  }
  sd = wave_sum(sd);
  const float r = P.rstd[row];
  const float a = r * r * r * sd / (float)P.cols;
  bf16* dxr = P.dx + row * P.dx_st;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nc) {
      float fx[8], fd[8], o[8];
      unpack8(xv[k], fx);
      unpack8(dv[k], fd);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = r * fd[e] - a * fx[e];
      *reinterpret_cast<bf16x8*>(dxr + 8 * c) = cvt8(o[0], o[1], o[2], o[3], o[4], o[5], o[6], o[7]);
    }
  }
}

}  // namespace nm
}  // namespace prefixlm
