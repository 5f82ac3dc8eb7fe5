// AdamW step of the CA-S decoder's training loop (torch.optim.AdamW as the
// reference builds it, cuda/runtime.py:87-88, after
// torch.nn.utils.clip_grad_norm_, cuda/continuum_attention.py:1205-1228) over
// a list of tensors in two launches plus one reduction:
//
//   1. ca_grad_sumsq_kernel: sum of squares of every gradient, one partial per
//      chunk; ca_clip_coef_kernel sums the partials in chunk order and writes
//      clip_coef = min(1, max_norm / (sqrt(total) + 1e-6)) to device memory
//      (no host synchronisation).
//   2. ca_adamw_kernel: per element, with g = grad * clip_coef,
//        p = p * (1 - lr*wd);  m = m + (1 - b1) * (g - m);
//        v = v * b2 + (1 - b2) * g * g;
//        p = p - (lr / bc1) * m / (sqrt(v) / sqrt(bc2) + eps)
//      (torch's AdamW update, bc = bias corrections of the step), and, for
//      tensors with a bf16 shadow, shadow = bf16(p) rounded to nearest even:
//      the value bf16 autocast casts the weight to in the next forward.
//
// Gradients are fp32 or bf16 (the gradient of a bf16 shadow weight, which
// autocast would have upcast to fp32 without changing its value).  Work is
// split into chunks of kOptChunk elements; a chunk table (tensor index,
// chunk index) lives in device memory next to the tensor table.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

namespace {

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// four gradient values at element e (e % 4 == 0, e + 3 < n)
__device__ __forceinline__ f32x4 load_grad4(const void* g, int64_t e, int dtype) {
  if (dtype == kDtypeF32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(g) + e);
  const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(g) + e);
  return f32x4{bf16_bits_to_f32(u.x & 0xffffu), bf16_bits_to_f32(u.x >> 16),
               bf16_bits_to_f32(u.y & 0xffffu), bf16_bits_to_f32(u.y >> 16)};
}

__device__ __forceinline__ float load_grad1(const void* g, int64_t e, int dtype) {
  if (dtype == kDtypeF32) return static_cast<const float*>(g)[e];
  return bf16_bits_to_f32(static_cast<const uint16_t*>(g)[e]);
}

// One chunk: elements [c0, c1) of tensor t, the float4 body and a scalar tail.
// Tensor bases are 16-byte aligned and chunk starts are multiples of 4.
struct ChunkRange {
  int64_t c0, c1;
};

// empty when the chunk index is outside the tensor
__device__ __forceinline__ ChunkRange chunk_range(const CaOptTensor& t, int chunk) {
  const int64_t c0 = chunk < 0 ? t.numel : (int64_t)chunk * kOptChunk;
  const int64_t c1 = c0 + kOptChunk < t.numel ? c0 + kOptChunk : t.numel;
  return ChunkRange{c0 < c1 ? c0 : c1, c1};
}

}  // namespace

__global__ __launch_bounds__(256) void ca_grad_sumsq_kernel(const CaOptTensor* __restrict__ tensors,
                                                            int ntensors,
                                                            const int2* __restrict__ chunks,
                                                            float* __restrict__ partial) {
  __shared__ float red[4];
  const int2 ck = chunks[blockIdx.x];
  if (ck.x < 0 || ck.x >= ntensors) {  // a malformed table entry adds nothing
    if (threadIdx.x == 0) partial[blockIdx.x] = 0.f;
    return;
  }
  const CaOptTensor t = tensors[ck.x];
  const ChunkRange r = chunk_range(t, ck.y);
  const int64_t body_end = r.c0 + ((r.c1 - r.c0) & ~int64_t(3));
  float s = 0.f;
  for (int64_t e = r.c0 + 4 * (int64_t)threadIdx.x; e < body_end; e += 4 * 256) {
    const f32x4 g = load_grad4(t.grad, e, t.grad_dtype);
    s = fmaf(g[0], g[0], s);
    s = fmaf(g[1], g[1], s);
    s = fmaf(g[2], g[2], s);
    s = fmaf(g[3], g[3], s);
  }
  for (int64_t e = body_end + threadIdx.x; e < r.c1; e += 256) {
    const float g = load_grad1(t.grad, e, t.grad_dtype);
    s = fmaf(g, g, s);
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// One work group: the partials in a fixed order, then the clip coefficient.
__global__ __launch_bounds__(256) void ca_clip_coef_kernel(const float* __restrict__ partial,
                                                           int nchunks, float max_norm,
                                                           float* __restrict__ total_norm,
                                                           float* __restrict__ coef) {
  __shared__ float red[4];
  float s = 0.f;
  for (int c = threadIdx.x; c < nchunks; c += 256) s += partial[c];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float norm = sqrtf((red[0] + red[1]) + (red[2] + red[3]));
    total_norm[0] = norm;
    // clip_grad_norm_'s clamp(max_norm / (norm + 1e-6), max=1): an infinite
    // norm gives 0, a NaN norm gives NaN (the comparison is false for NaN)
    const float c = max_norm / (norm + 1e-6f);
    coef[0] = max_norm > 0.f ? (c >= 1.f ? 1.f : c) : 1.f;
  }
}

__global__ __launch_bounds__(256) void ca_adamw_kernel(const CaOptTensor* __restrict__ tensors,
                                                       int ntensors,
                                                       const int2* __restrict__ chunks,
                                                       const float* __restrict__ coef_ptr,
                                                       CaAdamwScalars k) {
  const int2 ck = chunks[blockIdx.x];
  if (ck.x < 0 || ck.x >= ntensors) return;
  const CaOptTensor t = tensors[ck.x];
  const ChunkRange r = chunk_range(t, ck.y);
  const float coef = coef_ptr ? coef_ptr[0] : 1.f;
  auto update = [&](float& p, float g, float& m, float& v) {
    g *= coef;
    p *= k.decay;
    m = m + k.one_minus_beta1 * (g - m);
    v = v * k.beta2 + k.one_minus_beta2 * g * g;
    const float denom = sqrtf(v) / k.bc2_sqrt + k.eps;
    p = p + k.neg_step_size * (m / denom);
  };
  const int64_t body_end = r.c0 + ((r.c1 - r.c0) & ~int64_t(3));
  for (int64_t e = r.c0 + 4 * (int64_t)threadIdx.x; e < body_end; e += 4 * 256) {
    f32x4 p = *reinterpret_cast<const f32x4*>(t.param + e);
    f32x4 m = *reinterpret_cast<const f32x4*>(t.exp_avg + e);
    f32x4 v = *reinterpret_cast<const f32x4*>(t.exp_avg_sq + e);
    const f32x4 g = load_grad4(t.grad, e, t.grad_dtype);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float pj = p[j], mj = m[j], vj = v[j];
      update(pj, g[j], mj, vj);
      p[j] = pj;
      m[j] = mj;
      v[j] = vj;
    }
    *reinterpret_cast<f32x4*>(t.param + e) = p;
    *reinterpret_cast<f32x4*>(t.exp_avg + e) = m;
    *reinterpret_cast<f32x4*>(t.exp_avg_sq + e) = v;
    if (t.shadow) {
      uint2 u;
      u.x = f32_to_bf16_rne(p[0]) | (f32_to_bf16_rne(p[1]) << 16);
      u.y = f32_to_bf16_rne(p[2]) | (f32_to_bf16_rne(p[3]) << 16);
      *reinterpret_cast<uint2*>(t.shadow + e) = u;
    }
  }
  for (int64_t e = body_end + threadIdx.x; e < r.c1; e += 256) {
    float p = t.param[e], m = t.exp_avg[e], v = t.exp_avg_sq[e];
    update(p, load_grad1(t.grad, e, t.grad_dtype), m, v);
    t.param[e] = p;
    t.exp_avg[e] = m;
    t.exp_avg_sq[e] = v;
    if (t.shadow) t.shadow[e] = static_cast<uint16_t>(f32_to_bf16_rne(p));
  }
}

// bf16 shadows of fp32 tensors (refresh after the weights change elsewhere)
__global__ __launch_bounds__(256) void ca_shadow_kernel(const CaOptTensor* __restrict__ tensors,
                                                        int ntensors,
                                                        const int2* __restrict__ chunks) {
  const int2 ck = chunks[blockIdx.x];
  if (ck.x < 0 || ck.x >= ntensors) return;
  const CaOptTensor t = tensors[ck.x];
  if (!t.shadow) return;
  const ChunkRange r = chunk_range(t, ck.y);
  for (int64_t e = r.c0 + threadIdx.x; e < r.c1; e += 256)
    t.shadow[e] = static_cast<uint16_t>(f32_to_bf16_rne(t.param[e]));
}

hipError_t launch_grad_sumsq(const CaOptTensor* tensors, int ntensors, const int2* chunks,
                             int nchunks, float* partial, float max_norm, float* total_norm,
                             float* coef, hipStream_t s) {
  hipLaunchKernelGGL(ca_grad_sumsq_kernel, dim3(nchunks), dim3(256), 0, s, tensors, ntensors, chunks,
                     partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ca_clip_coef_kernel, dim3(1), dim3(256), 0, s, partial, nchunks, max_norm,
                     total_norm, coef);
  return hipGetLastError();
}

hipError_t launch_adamw(const CaOptTensor* tensors, int ntensors, const int2* chunks, int nchunks,
                        const float* coef, const CaAdamwScalars& k, hipStream_t s) {
  hipLaunchKernelGGL(ca_adamw_kernel, dim3(nchunks), dim3(256), 0, s, tensors, ntensors, chunks, coef,
                     k);
  return hipGetLastError();
}

hipError_t launch_shadow(const CaOptTensor* tensors, int ntensors, const int2* chunks, int nchunks,
                         hipStream_t s) {
  hipLaunchKernelGGL(ca_shadow_kernel, dim3(nchunks), dim3(256), 0, s, tensors, ntensors, chunks);
  return hipGetLastError();
}

}  // namespace ca
