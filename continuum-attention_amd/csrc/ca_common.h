// Shared device code for the Continuum Attention (CA) HIP kernels (gfx950).
//
// Segment math
// ------------
// A segment joins two adjacent keys (left l, right r) of one query row.  With
// scores in log2 units (the kernels pre-scale q by c_h*log2(e)) the natural
// score difference is t = |s_r - s_l| * ln2, and with the row shift m the
// endpoint weights are p = 2^(s - m).  Writing hi/lo for the endpoint with the
// larger/smaller score, Pmax = p_hi, Pmin = p_lo = Pmax e^-t, and the decaying
// integrals K_n(t) = int_0^1 u^n e^{-t u} du, the reference's segment terms
// (architecture.py:32-62,91-96; analytic_reference.py:12-75) become
//
//   share to hi endpoint   E*B  = Pmax (K0 - K1) = (t Pmax - (Pmax - Pmin)) / t^2
//   share to lo endpoint   E*A  = Pmax  K1       = ((Pmax - Pmin) - t Pmin) / t^2
//   second moment          E*K2 = Pmax  K2       = (2 E*A - Pmin) / t
//
// and the score-gradient contributions of the segment are
//   dS_hi += g_hi (EB - EA + EK2) + g_lo (EA - EK2)
//   dS_lo += g_hi (EA - EK2)      + g_lo EK2.
// This is the reference's J0/J1/J2 form rewritten with the mirror identity
// e^{-max(d,0)}(J0-J1)(d) = m1(-d) (pinned in tests/test_oracle.py), so one
// set of decaying integrals serves both signs of the difference and nothing
// subtracts nearly equal closed-form terms below the series threshold.
// For t < 0.75 the integrals use fitted degree-5 polynomials; the closed
// forms are used above, where their cancellation costs < 4 bits.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ca {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kSeriesT = 0.75f;    // fitted polynomials below, closed form at/above
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" sentinel
constexpr float kLazyRescale = 8.0f;  // forward keeps p <= 2^8 between rescales

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Per-head score scale in log2 units: exp(log_gain[h]) / sqrt(D) * log2(e)
// (the reference's scale, cuda/continuum_attention.py:656-657, times log2 e).
__device__ __forceinline__ float head_scale_log2(const float* log_gain, int head, int D) {
  return expf(log_gain[head]) / sqrtf((float)D) * kLog2e;
}

// Value held by lane (l ^ 32): exchanges the two 32-lane halves of a wave.
__device__ __forceinline__ float xhalf(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return (threadIdx.x & 32) ? __uint_as_float(r[0]) : __uint_as_float(r[1]);
}

// Wave-uniform "any lane" test.
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// Orders LDS traffic of one wave that exchanges data through LDS between its
// own lanes (no other wave touches the region).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_sum(float x) {
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// --- decaying integrals below the switch point (t < 0.75) -----------------
// Degree-5 polynomials fitted (weighted least squares with Lawson
// reweighting toward minimax relative error) to K1 = int u e^{-tu},
// K0-K1 = int (1-u) e^{-tu} and K2 = int u^2 e^{-tu} on [0, 0.75]: max
// relative error 2.8e-8 / 3.6e-9 / 3.8e-8 in exact arithmetic, ~1.6e-7 with
// float32 Horner evaluation.  tests/test_device_math.py re-checks these
// constants (parsed from this file) against the float64 oracle.
__device__ __forceinline__ float poly5(float t, float c0, float c1, float c2, float c3, float c4,
                                       float c5) {
  float r = fmaf(c5, t, c4);
  r = fmaf(r, t, c3);
  r = fmaf(r, t, c2);
  r = fmaf(r, t, c1);
  return fmaf(r, t, c0);
}
// CA_SERIES_K1
__device__ __forceinline__ float series_K1(float t) {
  return poly5(t, 4.999999862e-01f, -3.333320860e-01f, 1.249812735e-01f, -3.322858567e-02f,
               6.674105707e-03f, -8.569940316e-04f);
}
// CA_SERIES_K0MK1
__device__ __forceinline__ float series_K0mK1(float t) {
  return poly5(t, 4.999999982e-01f, -1.666664961e-01f, 4.166404157e-02f, -8.318396947e-03f,
               1.349916558e-03f, -1.501583445e-04f);
}
// CA_SERIES_K2
__device__ __forceinline__ float series_K2(float t) {
  return poly5(t, 3.333333207e-01f, -2.499988710e-01f, 9.998316696e-02f, -2.768409257e-02f,
               5.711472720e-03f, -7.451890149e-04f);
}

// Forward shares of one segment: L -> left key, R -> right key.
// sl/sr are log2-unit scores, pl/pr their weights 2^(s-m).
__device__ __forceinline__ void seg_shares(float sl, float sr, float pl, float pr, float& L,
                                           float& R) {
  const float d2 = sr - sl;
  const float t = fabsf(d2) * kLn2;
  const float pmax = fmaxf(pl, pr), pmin = fminf(pl, pr);
  const float inv_t2 = fast_rcp(t * t);
  const float dl = pmax - pmin;
  const float ea_c = fmaf(-t, pmin, dl) * inv_t2;
  const float eb_c = fmaf(t, pmax, -dl) * inv_t2;
  // both branches are evaluated and selected (no divergent control flow)
  const float ea_s = pmax * series_K1(t);
  const float eb_s = pmax * series_K0mK1(t);
  const bool small = t < kSeriesT;
  const float ea = small ? ea_s : ea_c;
  const float eb = small ? eb_s : eb_c;
  const bool up = d2 >= 0.0f;
  R = up ? eb : ea;
  L = up ? ea : eb;
}

// Forward shares and score-gradient contributions of one segment.
// gl/gr are the centred, 1/Z-scaled weight gradients g = (dY.v - Dl) / Z.
__device__ __forceinline__ void seg_shares_grad(float sl, float sr, float pl, float pr, float gl,
                                                float gr, float& L, float& R, float& dL,
                                                float& dR) {
  const float d2 = sr - sl;
  const float t = fabsf(d2) * kLn2;
  const float pmax = fmaxf(pl, pr), pmin = fminf(pl, pr);
  const float inv_t2 = fast_rcp(t * t);
  const float dl = pmax - pmin;
  const float ea_c = fmaf(-t, pmin, dl) * inv_t2;
  const float eb_c = fmaf(t, pmax, -dl) * inv_t2;
  const float ek_c = fmaf(2.0f, ea_c, -pmin) * (t * inv_t2);
  const float ea_s = pmax * series_K1(t);
  const float eb_s = pmax * series_K0mK1(t);
  const float ek_s = pmax * series_K2(t);
  const bool small = t < kSeriesT;
  const float ea = small ? ea_s : ea_c;
  const float eb = small ? eb_s : eb_c;
  const float ek = small ? ek_s : ek_c;
  const bool up = d2 >= 0.0f;
  const float ghi = up ? gr : gl;
  const float glo = up ? gl : gr;
  const float ex = ea - ek;
  const float dhi = fmaf(ghi, eb - ea + ek, glo * ex);
  const float dlo = fmaf(ghi, ex, glo * ek);
  R = up ? eb : ea;
  L = up ? ea : eb;
  dR = up ? dhi : dlo;
  dL = up ? dlo : dhi;
}

// 32x32x2 MFMA output layout: register r of lane l holds row
// 8*(r/4) + 4*(l/32) + r%4 and column l%32.  For an S^T tile (rows = keys) the
// kernels permute keys so that register r of lane half h is key 16*h + r.
// This returns the key (0..31) an A-operand lane must supply for that order.
__device__ __forceinline__ int key_of_arow(int lane) {
  const int i = lane & 31;
  return (((i >> 2) & 1) << 4) | ((i >> 3) << 2) | (i & 3);
}

}  // namespace ca
