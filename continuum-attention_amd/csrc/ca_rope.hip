// Prologue / epilogue of the CA operator inside its decoder caller
// (ContinuumSelfAttention.forward, cuda/continuum_attention.py:848-854):
// qkv projection output -> RoPE -> per-head fp32 q, k, v, and back.
//
// The reference runs these steps as separate torch ops: a permute of the qkv
// projection, RoPE on q and k in the autocast dtype (six elementwise ops,
// cuda/continuum_attention.py:826-835), the operator's own float casts, and
// the inverse chain in autograd.  Here each direction is one HBM pass:
//
//   ca_qkv_in_kernel      qkv [B,T,3,H,D] (bf16/fp16/fp32) -> q, k, v fp32
//                         [B,H,T,D], RoPE applied to q and k in fp32
//   ca_relayout_kernel    <true>:  y fp32 [B,H,T,D] -> [B,T,H*D] in the
//                         model dtype; <false>: dY [B,T,H*D] (any dtype) ->
//                         fp32 [B,H,T,D]
//   ca_qkv_grad_kernel    dq, dk, dv fp32 [B,H,T,D] -> dqkv [B,T,3,H,D],
//                         the transposed rotation applied to dq and dk
//
// RoPE rotates interleaved pairs (x0, x1) of the head dimension by the angle
// t * theta^(-2i/D): x0' = x0 c - x1 s, x1' = x1 c + x0 s.  The (c, s) table
// [T][D/2][2] fp32 is supplied by the caller (the reference's own fp32
// table), so the angles are bit-identical to the reference's; the rotation
// itself is computed in fp32 (the reference rounds it to the autocast dtype).
// One thread handles four consecutive head-dim entries (two pairs).
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

namespace {

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
// round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ f32x4 load4(const void* base, size_t idx, int dtype) {
  if (dtype == kDtypeF32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + idx);
  if (dtype == kDtypeBF16) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
    return f32x4{bf16_to_f32(u.x & 0xffff), bf16_to_f32(u.x >> 16), bf16_to_f32(u.y & 0xffff),
                 bf16_to_f32(u.y >> 16)};
  }
  const __half* h = static_cast<const __half*>(base) + idx;
  return f32x4{__half2float(h[0]), __half2float(h[1]), __half2float(h[2]), __half2float(h[3])};
}

__device__ __forceinline__ void store4(void* base, size_t idx, int dtype, f32x4 v) {
  if (dtype == kDtypeF32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(base) + idx) = v;
  } else if (dtype == kDtypeBF16) {
    uint2 u;
    u.x = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
    u.y = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + idx) = u;
  } else {
    __half* h = static_cast<__half*>(base) + idx;
    h[0] = __float2half(v[0]); h[1] = __float2half(v[1]);
    h[2] = __float2half(v[2]); h[3] = __float2half(v[3]);
  }
}

// rotation of the two pairs held in x by the table entries of pairs p, p+1
__device__ __forceinline__ f32x4 rotate(f32x4 x, const float* cs, bool transpose) {
  const f32x4 t = *reinterpret_cast<const f32x4*>(cs);  // c0 s0 c1 s1
  const float s0 = transpose ? -t[1] : t[1], s1 = transpose ? -t[3] : t[3];
  return f32x4{x[0] * t[0] - x[1] * s0, x[1] * t[0] + x[0] * s0, x[2] * t[2] - x[3] * s1,
               x[3] * t[2] + x[2] * s1};
}

}  // namespace

// One thread per (b, t, part, h, 4 head-dim entries), in qkv's memory order.
__global__ __launch_bounds__(256) void ca_qkv_in_kernel(const void* __restrict__ qkv, int dtype,
                                                        const float* __restrict__ cs,
                                                        float* __restrict__ q, float* __restrict__ k,
                                                        float* __restrict__ v, int B, int T, int H,
                                                        int D) {
  const int C4 = D / 4;
  const size_t total = (size_t)B * T * 3 * H * C4;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const int c4 = static_cast<int>(e % C4);
  size_t r = e / C4;
  const int h = static_cast<int>(r % H); r /= H;
  const int part = static_cast<int>(r % 3); r /= 3;
  const int t = static_cast<int>(r % T);
  const int b = static_cast<int>(r / T);
  f32x4 x = load4(qkv, e * 4, dtype);
  if (part < 2 && cs) x = rotate(x, cs + ((size_t)t * (D / 2) + 2 * c4) * 2, false);
  float* dst = part == 0 ? q : (part == 1 ? k : v);
  *reinterpret_cast<f32x4*>(dst + (((size_t)b * H + h) * T + t) * D + 4 * c4) = x;
}

// dqkv = [R^T dq, R^T dk, dv] in qkv's layout; one thread per output float4.
__global__ __launch_bounds__(256) void ca_qkv_grad_kernel(const float* __restrict__ dq,
                                                          const float* __restrict__ dk,
                                                          const float* __restrict__ dv,
                                                          const float* __restrict__ cs,
                                                          void* __restrict__ dqkv, int dtype, int B,
                                                          int T, int H, int D) {
  const int C4 = D / 4;
  const size_t total = (size_t)B * T * 3 * H * C4;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const int c4 = static_cast<int>(e % C4);
  size_t r = e / C4;
  const int h = static_cast<int>(r % H); r /= H;
  const int part = static_cast<int>(r % 3); r /= 3;
  const int t = static_cast<int>(r % T);
  const int b = static_cast<int>(r / T);
  const float* src = part == 0 ? dq : (part == 1 ? dk : dv);
  f32x4 g = *reinterpret_cast<const f32x4*>(src + (((size_t)b * H + h) * T + t) * D + 4 * c4);
  if (part < 2 && cs) g = rotate(g, cs + ((size_t)t * (D / 2) + 2 * c4) * 2, true);
  store4(dqkv, e * 4, dtype, g);
}

// [B,H,T,D] fp32 <-> [B,T,H*D] (any dtype); one thread per float4 of the
// token-major side.
template <bool kToTokens>
__global__ __launch_bounds__(256) void ca_relayout_kernel(const void* __restrict__ src,
                                                          void* __restrict__ dst, int dtype, int B,
                                                          int H, int T, int D) {
  const int C4 = D / 4;
  const size_t total = (size_t)B * T * H * C4;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= total) return;
  const int c4 = static_cast<int>(e % C4);
  size_t r = e / C4;
  const int h = static_cast<int>(r % H); r /= H;
  const int t = static_cast<int>(r % T);
  const int b = static_cast<int>(r / T);
  const size_t hidx = (((size_t)b * H + h) * T + t) * D + 4 * c4;
  if (kToTokens) {
    store4(dst, e * 4, dtype, *reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + hidx));
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(dst) + hidx) = load4(src, e * 4, dtype);
  }
}

static dim3 grid_for(size_t n) { return dim3(static_cast<unsigned>((n + 255) / 256)); }

hipError_t launch_qkv_in(const void* qkv, int dtype, const float* cs, float* q, float* k, float* v,
                         int B, int T, int H, int D, hipStream_t s) {
  hipLaunchKernelGGL(ca_qkv_in_kernel, grid_for((size_t)B * T * 3 * H * (D / 4)), dim3(256), 0, s,
                     qkv, dtype, cs, q, k, v, B, T, H, D);
  return hipGetLastError();
}

hipError_t launch_qkv_grad(const float* dq, const float* dk, const float* dv, const float* cs,
                           void* dqkv, int dtype, int B, int T, int H, int D, hipStream_t s) {
  hipLaunchKernelGGL(ca_qkv_grad_kernel, grid_for((size_t)B * T * 3 * H * (D / 4)), dim3(256), 0, s,
                     dq, dk, dv, cs, dqkv, dtype, B, T, H, D);
  return hipGetLastError();
}

hipError_t launch_relayout(const void* src, void* dst, int dtype, bool to_tokens, int B, int H,
                           int T, int D, hipStream_t s) {
  const dim3 g = grid_for((size_t)B * T * H * (D / 4));
  if (to_tokens)
    hipLaunchKernelGGL(ca_relayout_kernel<true>, g, dim3(256), 0, s, src, dst, dtype, B, H, T, D);
  else
    hipLaunchKernelGGL(ca_relayout_kernel<false>, g, dim3(256), 0, s, src, dst, dtype, B, H, T, D);
  return hipGetLastError();
}

}  // namespace ca
