// RMSNorm of the CA-S decoder (cuda/continuum_attention.py:817-823,
// y = weight * x * rsqrt(mean(x^2) + eps) over the last dimension), forward
// and backward as single HIP passes.  The reference runs it as a chain of
// torch elementwise and reduction kernels in fp32 (square, mean, add, rsqrt,
// two multiplies, and their gradients); here the forward is one work group
// per row and the backward one pass over the rows plus a dweight column sum.
//
// The forward writes y in the consumer's dtype: under bf16/fp16 autocast the
// next op is a linear layer whose input autocast would round to that dtype,
// so writing the rounded value (round to nearest even) is what the reference
// computes.  The backward takes dy in the same dtype, computes in fp32 and
// returns dx (fp32) and dweight; dweight = sum over rows of dy * x * rstd is
// reduced in a fixed order (per-block partials, then one column sum).
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

namespace {

__device__ __forceinline__ float load_any(const void* base, size_t i, int dtype) {
  if (dtype == kDtypeF32) return static_cast<const float*>(base)[i];
  if (dtype == kDtypeBF16)
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i]) << 16);
  return __half2float(static_cast<const __half*>(base)[i]);
}

__device__ __forceinline__ void store_any(void* base, size_t i, int dtype, float v) {
  if (dtype == kDtypeF32) {
    static_cast<float*>(base)[i] = v;
  } else if (dtype == kDtypeBF16) {
    const uint32_t u = __float_as_uint(v);
    static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  } else {
    static_cast<__half*>(base)[i] = __float2half(v);
  }
}

// sum over the 256 threads of a work group (fixed order)
__device__ __forceinline__ float block_sum(float x, float* red) {
  x = wave_sum(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

}  // namespace

// One work group per row.
__global__ __launch_bounds__(256) void ca_rmsnorm_fwd_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ w,
                                                             void* __restrict__ y, int ydtype,
                                                             float* __restrict__ rstd, int C,
                                                             float eps) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  const float* xr = x + row * C;
  float ss = 0.f;
  for (int c = threadIdx.x; c < C; c += 256) ss = fmaf(xr[c], xr[c], ss);
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)C + eps);
  for (int c = threadIdx.x; c < C; c += 256) store_any(y, row * C + c, ydtype, w[c] * xr[c] * r);
  if (threadIdx.x == 0) rstd[row] = r;
}

// Rows [rows_per_block * blockIdx.x, ...): dx = rstd * (w*dy - xh * mean(xh * w*dy)),
// xh = x * rstd; the block's partial dweight = sum over its rows of dy * xh.
__global__ __launch_bounds__(256) void ca_rmsnorm_bwd_kernel(
    const void* __restrict__ dy, int dydtype, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ rstd, float* __restrict__ dx,
    float* __restrict__ dw_part, int N, int C, int rows_per_block) {
  __shared__ float red[4];
  constexpr int kMaxCols = 16;  // C <= 256 * kMaxCols
  float dwacc[kMaxCols];
#pragma unroll
  for (int u = 0; u < kMaxCols; ++u) dwacc[u] = 0.f;
  const int r0 = blockIdx.x * rows_per_block;
  const int r1 = min(r0 + rows_per_block, N);
  for (int row = r0; row < r1; ++row) {
    const size_t base = (size_t)row * C;
    const float r = rstd[row];
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < kMaxCols; ++u) {
      const int c = threadIdx.x + 256 * u;
      if (c < C) s = fmaf(x[base + c] * r, w[c] * load_any(dy, base + c, dydtype), s);
    }
    const float mean = block_sum(s, red) / (float)C;
#pragma unroll
    for (int u = 0; u < kMaxCols; ++u) {
      const int c = threadIdx.x + 256 * u;
      if (c < C) {
        const float g = load_any(dy, base + c, dydtype);
        const float xh = x[base + c] * r;
        dx[base + c] = r * fmaf(-xh, mean, w[c] * g);
        dwacc[u] = fmaf(g, xh, dwacc[u]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kMaxCols; ++u) {
    const int c = threadIdx.x + 256 * u;
    if (c < C) dw_part[(size_t)blockIdx.x * C + c] = dwacc[u];
  }
}

// dweight[c] = sum over blocks of the partials: 64 columns per work group,
// each wave sums a contiguous quarter of the partials in block order, and the
// four quarter sums are added in wave order.
__global__ __launch_bounds__(256) void ca_rmsnorm_dw_kernel(const float* __restrict__ dw_part,
                                                            float* __restrict__ dw, int nblocks,
                                                            int C) {
  __shared__ float red[4][64];
  const int c = blockIdx.x * 64 + (threadIdx.x & 63);
  const int q = threadIdx.x >> 6;
  const int b0 = q * nblocks / 4, b1 = (q + 1) * nblocks / 4;
  float s = 0.f;
  if (c < C)
    for (int b = b0; b < b1; ++b) s += dw_part[(size_t)b * C + c];
  red[q][threadIdx.x & 63] = s;
  __syncthreads();
  if (q == 0 && c < C) dw[c] = (red[0][threadIdx.x] + red[1][threadIdx.x]) +
                               (red[2][threadIdx.x] + red[3][threadIdx.x]);
}

// Rows per backward work group: enough groups to fill the chip (up to
// kRmsMaxBlocks), at least one row each.
int rmsnorm_rows_per_block(int N) {
  const int rpb = (N + kRmsMaxBlocks - 1) / kRmsMaxBlocks;
  return rpb > 1 ? rpb : 1;
}
int rmsnorm_bwd_blocks(int N) {
  const int rpb = rmsnorm_rows_per_block(N);
  return (N + rpb - 1) / rpb;
}

hipError_t launch_rmsnorm_fwd(const float* x, const float* w, void* y, int ydtype, float* rstd,
                              int N, int C, float eps, hipStream_t s) {
  hipLaunchKernelGGL(ca_rmsnorm_fwd_kernel, dim3(N), dim3(256), 0, s, x, w, y, ydtype, rstd, C, eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_bwd(const void* dy, int dydtype, const float* x, const float* w,
                              const float* rstd, float* dx, float* dw, float* dw_part, int N,
                              int C, hipStream_t s) {
  const int nb = rmsnorm_bwd_blocks(N);
  hipLaunchKernelGGL(ca_rmsnorm_bwd_kernel, dim3(nb), dim3(256), 0, s, dy, dydtype, x, w, rstd, dx,
                     dw_part, N, C, rmsnorm_rows_per_block(N));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ca_rmsnorm_dw_kernel, dim3((C + 63) / 64), dim3(256), 0, s, dw_part, dw, nb, C);
  return hipGetLastError();
}

}  // namespace ca
