// RMSNorm of the CA-S decoder (cuda/continuum_attention.py:817-823,
// y = weight * x * rsqrt(mean(x^2) + eps) over the last dimension), forward
// and backward as single HIP passes.  The reference runs it as a chain of
// torch elementwise and reduction kernels in fp32 (square, mean, add, rsqrt,
// two multiplies, and their gradients); here the forward is one wave per row
// and the backward one pass over the rows plus a dweight column sum.
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

// VEC consecutive elements starting at i (VEC = 4: 16-byte fp32 or 8-byte
// bf16/fp16 accesses; the caller guarantees the alignment).
template <int VEC>
__device__ __forceinline__ void load_vec(const void* base, size_t i, int dtype, float* v) {
  if constexpr (VEC == 1) {
    v[0] = load_any(base, i, dtype);
  } else {
    if (dtype == kDtypeF32) {
      const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
      v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
      const uint32_t h[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = dtype == kDtypeBF16 ? __uint_as_float(h[e] << 16)
                                   : __half2float(__ushort_as_half(static_cast<unsigned short>(h[e])));
    }
  }
}

__device__ __forceinline__ uint32_t to_bits16(float v, int dtype) {
  if (dtype == kDtypeBF16) {
    const uint32_t u = __float_as_uint(v);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  }
  return __half_as_ushort(__float2half(v));
}

template <int VEC>
__device__ __forceinline__ void store_vec(void* base, size_t i, int dtype, const float* v) {
  if constexpr (VEC == 1) {
    store_any(base, i, dtype, v[0]);
  } else {
    if (dtype == kDtypeF32) {
      *reinterpret_cast<float4*>(static_cast<float*>(base) + i) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint2 u;
      u.x = to_bits16(v[0], dtype) | (to_bits16(v[1], dtype) << 16);
      u.y = to_bits16(v[2], dtype) | (to_bits16(v[3], dtype) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + i) = u;
    }
  }
}

}  // namespace

// One wave per row, four rows per work group; lane l holds columns
// VEC*(l + 64*u).  KMAX > 0: the row is read once into registers (u < KMAX,
// C <= 64*VEC*KMAX) with every load issued before the first use; KMAX = 0:
// any C, loops that read the row twice.  ADD: the normalised row is
// s = x + res (res in rdtype), and s is written to sum_out (fp32).  No
// work-group barrier: a wave past the last row exits.
template <int VEC, int KMAX, bool ADD>
__global__ __launch_bounds__(256) void ca_rmsnorm_fwd_kernel(
    const float* __restrict__ x, const void* __restrict__ res, int rdtype,
    float* __restrict__ sum_out, const float* __restrict__ w, void* __restrict__ y, int ydtype,
    float* __restrict__ rstd, int N, int C, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;
  const size_t base = (size_t)row * C;
  // the row's values (x, or x + res) at columns c .. c+VEC-1
  auto load_row = [&](int c, float* v) {
    load_vec<VEC>(x, base + c, kDtypeF32, v);
    if constexpr (ADD) {
      float rv[VEC];
      load_vec<VEC>(res, base + c, rdtype, rv);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] += rv[e];
    }
  };
  float ss = 0.f;
  if constexpr (KMAX > 0) {
    float xv[KMAX][VEC];
#pragma unroll
    for (int u = 0; u < KMAX; ++u) {
      const int c = (lane + 64 * u) * VEC;
      if (c < C) {
        load_row(c, xv[u]);
        if constexpr (ADD) store_vec<VEC>(sum_out, base + c, kDtypeF32, xv[u]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) xv[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < KMAX; ++u)
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss = fmaf(xv[u][e], xv[u][e], ss);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)C + eps);
#pragma unroll
    for (int u = 0; u < KMAX; ++u) {
      const int c = (lane + 64 * u) * VEC;
      if (c < C) {
        float wv[VEC];
        load_vec<VEC>(w, c, kDtypeF32, wv);
#pragma unroll
        for (int e = 0; e < VEC; ++e) wv[e] = wv[e] * xv[u][e] * r;
        store_vec<VEC>(y, base + c, ydtype, wv);
      }
    }
    if (lane == 0) rstd[row] = r;
  } else {
    for (int c = lane * VEC; c < C; c += 64 * VEC) {
      float xv[VEC];
      load_row(c, xv);
      if constexpr (ADD) store_vec<VEC>(sum_out, base + c, kDtypeF32, xv);
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss = fmaf(xv[e], xv[e], ss);
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)C + eps);
    for (int c = lane * VEC; c < C; c += 64 * VEC) {
      float xv[VEC], wv[VEC];
      load_row(c, xv);
      load_vec<VEC>(w, c, kDtypeF32, wv);
#pragma unroll
      for (int e = 0; e < VEC; ++e) xv[e] = wv[e] * xv[e] * r;
      store_vec<VEC>(y, base + c, ydtype, xv);
    }
    if (lane == 0) rstd[row] = r;
  }
}

// Rows [rows_per_block * blockIdx.x, ...), one wave per row in turn:
// dx = rstd * (w*dy - xh * mean(xh * w*dy)), xh = x * rstd.  Each wave
// accumulates sum(dy * xh) over its rows in its own LDS row of C floats
// (dynamic LDS, 4*C floats); the work group's dweight partial is the sum of
// the four rows in wave order.  KMAX as in the forward (x, dy and w of the
// row held in registers).  ADD (x is the sum s = x + res of the forward):
// dx += dsum (the gradient s receives from its other consumers, if any), and
// dx is also written to dres in rdtype, the gradient of res.
template <int VEC, int KMAX, bool ADD>
__global__ __launch_bounds__(256) void ca_rmsnorm_bwd_kernel(
    const void* __restrict__ dy, int dydtype, const float* __restrict__ dsum,
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ rstd,
    float* __restrict__ dx, void* __restrict__ dres, int rdtype, float* __restrict__ dw_part,
    int N, int C, int rows_per_block) {
  extern __shared__ float acc[];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* mine = acc + (size_t)wv * C;
  for (int c = lane * VEC; c < C; c += 64 * VEC)
#pragma unroll
    for (int e = 0; e < VEC; ++e) mine[c + e] = 0.f;
  const int r0 = blockIdx.x * rows_per_block;
  const int r1 = min(r0 + rows_per_block, N);
  // the gradient d of columns c .. c+VEC-1 of the row at base: stored to dx
  // (and, with ADD, plus dsum, to dx and dres)
  auto put = [&](size_t base, int c, float* d) {
    if constexpr (ADD) {
      if (dsum) {
        float e2[VEC];
        load_vec<VEC>(dsum, base + c, kDtypeF32, e2);
#pragma unroll
        for (int e = 0; e < VEC; ++e) d[e] += e2[e];
      }
      store_vec<VEC>(dres, base + c, rdtype, d);
    }
    store_vec<VEC>(dx, base + c, kDtypeF32, d);
  };
  if constexpr (KMAX > 0) {
    float wt[KMAX][VEC];
#pragma unroll
    for (int u = 0; u < KMAX; ++u) {
      const int c = (lane + 64 * u) * VEC;
      if (c < C) {
        load_vec<VEC>(w, c, kDtypeF32, wt[u]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) wt[u][e] = 0.f;
      }
    }
    for (int row = r0 + wv; row < r1; row += 4) {
      const size_t base = (size_t)row * C;
      const float r = rstd[row];
      float xv[KMAX][VEC], g[KMAX][VEC];
#pragma unroll
      for (int u = 0; u < KMAX; ++u) {
        const int c = (lane + 64 * u) * VEC;
        if (c < C) {
          load_vec<VEC>(x, base + c, kDtypeF32, xv[u]);
          load_vec<VEC>(dy, base + c, dydtype, g[u]);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) xv[u][e] = g[u][e] = 0.f;
        }
      }
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < KMAX; ++u)
#pragma unroll
        for (int e = 0; e < VEC; ++e) s = fmaf(xv[u][e] * r, wt[u][e] * g[u][e], s);
      const float mean = wave_sum(s) / (float)C;
#pragma unroll
      for (int u = 0; u < KMAX; ++u) {
        const int c = (lane + 64 * u) * VEC;
        if (c < C) {
          float d[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float xh = xv[u][e] * r;
            d[e] = r * fmaf(-xh, mean, wt[u][e] * g[u][e]);
            mine[c + e] = fmaf(g[u][e], xh, mine[c + e]);
          }
          put(base, c, d);
        }
      }
    }
  } else {
    for (int row = r0 + wv; row < r1; row += 4) {
      const size_t base = (size_t)row * C;
      const float r = rstd[row];
      float s = 0.f;
      for (int c = lane * VEC; c < C; c += 64 * VEC) {
        float xv[VEC], wt[VEC], g[VEC];
        load_vec<VEC>(x, base + c, kDtypeF32, xv);
        load_vec<VEC>(w, c, kDtypeF32, wt);
        load_vec<VEC>(dy, base + c, dydtype, g);
#pragma unroll
        for (int e = 0; e < VEC; ++e) s = fmaf(xv[e] * r, wt[e] * g[e], s);
      }
      const float mean = wave_sum(s) / (float)C;
      for (int c = lane * VEC; c < C; c += 64 * VEC) {
        float xv[VEC], wt[VEC], g[VEC], d[VEC];
        load_vec<VEC>(x, base + c, kDtypeF32, xv);
        load_vec<VEC>(w, c, kDtypeF32, wt);
        load_vec<VEC>(dy, base + c, dydtype, g);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float xh = xv[e] * r;
          d[e] = r * fmaf(-xh, mean, wt[e] * g[e]);
          mine[c + e] = fmaf(g[e], xh, mine[c + e]);
        }
        put(base, c, d);
      }
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += 256)
    dw_part[(size_t)blockIdx.x * C + c] = (acc[c] + acc[C + c]) + (acc[2 * C + c] + acc[3 * C + c]);
}

// dweight[c] = sum over blocks of the partials: 16 columns per work group,
// 16 slices of consecutive blocks each summed in block order, then the slice
// sums added in slice order.
__global__ __launch_bounds__(256) void ca_rmsnorm_dw_kernel(const float* __restrict__ dw_part,
                                                            float* __restrict__ dw, int nblocks,
                                                            int C) {
  __shared__ float red[16][17];
  const int cl = threadIdx.x & 15, q = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + cl;
  const int b0 = q * nblocks / 16, b1 = (q + 1) * nblocks / 16;
  float s = 0.f;
  if (c < C) {
#pragma unroll 4
    for (int b = b0; b < b1; ++b) s += dw_part[(size_t)b * C + c];
  }
  red[q][cl] = s;
  __syncthreads();
  if (q == 0 && c < C) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += red[i][cl];
    dw[c] = t;
  }
}

// Rows per backward work group: at least one per wave, and enough groups to
// fill the chip, up to kRmsMaxBlocks.
int rmsnorm_rows_per_block(int N) {
  const int rpb = (N + kRmsMaxBlocks - 1) / kRmsMaxBlocks;
  return rpb > 4 ? rpb : 4;
}
int rmsnorm_bwd_blocks(int N) {
  const int rpb = rmsnorm_rows_per_block(N);
  return (N + rpb - 1) / rpb;
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The 4-wide path needs C % 4 == 0 and 16-byte aligned bases (every row of
// an fp32 tensor is then 16-byte aligned, of a 16-bit tensor 8-byte aligned).
template <bool ADD>
static hipError_t rms_fwd(const float* x, const void* res, int rdtype, float* sum_out,
                          const float* w, void* y, int ydtype, float* rstd, int N, int C,
                          float eps, hipStream_t s) {
  const bool v4 = C % 4 == 0 && al16(x) && al16(w) && al16(y) && (!ADD || (al16(res) && al16(sum_out)));
  const dim3 grid((N + 3) / 4);
  if (v4 && C <= 1024)
    hipLaunchKernelGGL((ca_rmsnorm_fwd_kernel<4, 4, ADD>), grid, dim3(256), 0, s, x, res, rdtype,
                       sum_out, w, y, ydtype, rstd, N, C, eps);
  else if (v4)
    hipLaunchKernelGGL((ca_rmsnorm_fwd_kernel<4, 16, ADD>), grid, dim3(256), 0, s, x, res, rdtype,
                       sum_out, w, y, ydtype, rstd, N, C, eps);
  else
    hipLaunchKernelGGL((ca_rmsnorm_fwd_kernel<1, 0, ADD>), grid, dim3(256), 0, s, x, res, rdtype,
                       sum_out, w, y, ydtype, rstd, N, C, eps);
  return hipGetLastError();
}

template <bool ADD>
static hipError_t rms_bwd(const void* dy, int dydtype, const float* dsum, const float* x,
                          const float* w, const float* rstd, float* dx, void* dres, int rdtype,
                          float* dw, float* dw_part, int N, int C, hipStream_t s) {
  const int nb = rmsnorm_bwd_blocks(N);
  const int rpb = rmsnorm_rows_per_block(N);
  const size_t lds = 4 * (size_t)C * sizeof(float);
  const bool v4 = C % 4 == 0 && al16(dy) && al16(x) && al16(w) && al16(dx) &&
                  (!ADD || (al16(dres) && (!dsum || al16(dsum))));
  if (v4 && C <= 1024)
    hipLaunchKernelGGL((ca_rmsnorm_bwd_kernel<4, 4, ADD>), dim3(nb), dim3(256), lds, s, dy, dydtype,
                       dsum, x, w, rstd, dx, dres, rdtype, dw_part, N, C, rpb);
  else if (v4)
    hipLaunchKernelGGL((ca_rmsnorm_bwd_kernel<4, 16, ADD>), dim3(nb), dim3(256), lds, s, dy, dydtype,
                       dsum, x, w, rstd, dx, dres, rdtype, dw_part, N, C, rpb);
  else
    hipLaunchKernelGGL((ca_rmsnorm_bwd_kernel<1, 0, ADD>), dim3(nb), dim3(256), lds, s, dy, dydtype,
                       dsum, x, w, rstd, dx, dres, rdtype, dw_part, N, C, rpb);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ca_rmsnorm_dw_kernel, dim3((C + 15) / 16), dim3(256), 0, s, dw_part, dw, nb, C);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_fwd(const float* x, const void* res, int rdtype, float* sum_out,
                              const float* w, void* y, int ydtype, float* rstd, int N, int C,
                              float eps, hipStream_t s) {
  return res ? rms_fwd<true>(x, res, rdtype, sum_out, w, y, ydtype, rstd, N, C, eps, s)
             : rms_fwd<false>(x, nullptr, kDtypeF32, nullptr, w, y, ydtype, rstd, N, C, eps, s);
}

hipError_t launch_rmsnorm_bwd(const void* dy, int dydtype, const float* dsum, const float* x,
                              const float* w, const float* rstd, float* dx, void* dres, int rdtype,
                              float* dw, float* dw_part, int N, int C, hipStream_t s) {
  return dres ? rms_bwd<true>(dy, dydtype, dsum, x, w, rstd, dx, dres, rdtype, dw, dw_part, N, C, s)
              : rms_bwd<false>(dy, dydtype, nullptr, x, w, rstd, dx, nullptr, kDtypeF32, dw, dw_part,
                               N, C, s);
}

}  // namespace ca
