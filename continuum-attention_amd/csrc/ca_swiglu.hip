// SwiGLU gate of the TinyLM MLP (architecture.py:180-188):
//   u = gate_up(x) = [g | v] (two halves of H columns per row),
//   h = silu(g) * v,
// and its gradient du = [dg | dv] for dh, each as one pass over the rows
// (the reference runs silu, the product and their backward as separate torch
// kernels and concatenates the two halves of the gradient).  The arithmetic
// follows torch's kernels in order: silu(g) = g / (1 + exp(-g)); the product
// rounds silu(g) first; dv = dh * silu(g); dg = (dh * v) * s * (1 + g (1 - s))
// with s = 1 / (1 + exp(-g)).  The exponent argument is capped at 88 (exp
// stays finite: silu(g) of g < -88 is a denormal where torch gives -0).

#include <hip/hip_runtime.h>

#include "ca_kernels.h"

namespace ca {

namespace {

__device__ __forceinline__ float neg_exp(float g) { return expf(fminf(-g, 88.0f)); }

// one float4 of columns (4c4 .. 4c4+3) of one row per thread
__global__ __launch_bounds__(256) void ca_swiglu_fwd_kernel(const float* __restrict__ u,
                                                            float* __restrict__ h, int N, int H) {
  const int H4 = H / 4;
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)N * H4) return;
  const long long row = idx / H4;
  const int c4 = (int)(idx - row * H4);
  const float4 g = reinterpret_cast<const float4*>(u + row * 2 * H)[c4];
  const float4 v = reinterpret_cast<const float4*>(u + row * 2 * H + H)[c4];
  float4 o;
  o.x = (g.x / (1.0f + neg_exp(g.x))) * v.x;
  o.y = (g.y / (1.0f + neg_exp(g.y))) * v.y;
  o.z = (g.z / (1.0f + neg_exp(g.z))) * v.z;
  o.w = (g.w / (1.0f + neg_exp(g.w))) * v.w;
  reinterpret_cast<float4*>(h + row * H)[c4] = o;
}

__device__ __forceinline__ void swiglu_grad(float g, float v, float dh, float& dg, float& dv) {
  const float e = neg_exp(g);
  dv = dh * (g / (1.0f + e));
  const float s = 1.0f / (1.0f + e);
  dg = ((dh * v) * s) * (1.0f + g * (1.0f - s));
}

__global__ __launch_bounds__(256) void ca_swiglu_bwd_kernel(const float* __restrict__ u,
                                                            const float* __restrict__ dh,
                                                            float* __restrict__ du, int N, int H) {
  const int H4 = H / 4;
  const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long long)N * H4) return;
  const long long row = idx / H4;
  const int c4 = (int)(idx - row * H4);
  const float4 g = reinterpret_cast<const float4*>(u + row * 2 * H)[c4];
  const float4 v = reinterpret_cast<const float4*>(u + row * 2 * H + H)[c4];
  const float4 d = reinterpret_cast<const float4*>(dh + row * H)[c4];
  float4 dg, dv;
  swiglu_grad(g.x, v.x, d.x, dg.x, dv.x);
  swiglu_grad(g.y, v.y, d.y, dg.y, dv.y);
  swiglu_grad(g.z, v.z, d.z, dg.z, dv.z);
  swiglu_grad(g.w, v.w, d.w, dg.w, dv.w);
  reinterpret_cast<float4*>(du + row * 2 * H)[c4] = dg;
  reinterpret_cast<float4*>(du + row * 2 * H + H)[c4] = dv;
}

inline unsigned swiglu_blocks(int N, int H) {
  return (unsigned)(((long long)N * (H / 4) + 255) / 256);
}

}  // namespace

hipError_t launch_swiglu_fwd(const float* u, float* h, int N, int H, hipStream_t s) {
  hipLaunchKernelGGL(ca_swiglu_fwd_kernel, dim3(swiglu_blocks(N, H)), dim3(256), 0, s, u, h, N, H);
  return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const float* u, const float* dh, float* du, int N, int H,
                             hipStream_t s) {
  hipLaunchKernelGGL(ca_swiglu_bwd_kernel, dim3(swiglu_blocks(N, H)), dim3(256), 0, s, u, dh, du,
                     N, H);
  return hipGetLastError();
}

}  // namespace ca
