// Shared device code for the Continuum Attention (CA) HIP kernels (gfx950).
//
// Segment math
// ------------
// A segment joins two adjacent keys (left l, right r) of one query row.  The
// kernels keep scores in log2 units relative to the row shift m (q is
// pre-scaled by c_h*log2(e) and -m rides in the MFMA accumulator), so the
// endpoint weights are p = 2^s and the signed natural difference is
// x = (s_r - s_l) * ln2.  With J_n(x) = int_0^1 u^n e^{x u} du the
// reference's segment terms (architecture.py:32-62,91-96;
// analytic_reference.py:12-75, there written with shifted moments of |x|) are
//
//   right share   R = p_l J1(x)          left share  L = p_l (J0 - J1)(x)
//   p_l J2(x)     (second moment, backward only)
//
// and the score-gradient contributions, with centred, 1/Z-scaled weight
// gradients g_l, g_r, are
//
//   dS_r += g_l (R - p_l J2) + g_r p_l J2
//   dS_l += g_l (L - R + p_l J2) + g_r (R - p_l J2).
//
// For |x| >= 0.5 the closed forms, using p_l e^x = p_r and dp = p_r - p_l,
//   p_l J0 = dp / x,   R = (p_r - dp/x) / x,   L = dp/x - R,
//   p_l J2 = (p_r - 2R) / x
// need a single reciprocal and no ordering of the endpoints.  For |x| < 0.5
// they cancel, and R = p_l J1(x), L = p_r J1(-x) (mirror identity
// e^{x}J1(-x) = (J0-J1)(x), pinned in tests/test_oracle.py), with J1 and J2
// split into even and odd parts J(x) = E(x^2) + x O(x^2) so one evaluation
// serves both shares.  The polynomial coefficients are fitted (weighted least
// squares with Lawson reweighting toward minimax relative error) on
// [-0.5, 0.5] with quadratic E and O: max relative error 1.7e-7 (J1) and
// 2.2e-7 (J2) in exact arithmetic, about float32 resolution.  tests/test_device_math.py re-checks these
// constants and formulas in float32 against the float64 oracle.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ca {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kSeriesT = 0.5f;     // |x| below: fitted polynomials; at/above: closed form
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" sentinel
constexpr float kLazyRescale = 8.0f;  // forward keeps p <= 2^8 between rescales

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// fp32 products on the bf16 matrix cores ("bf16x6").  An fp32 value is split
// into three round-to-nearest bf16 limbs, x = h + m + l exactly (the 24-bit
// significand in three 8-bit limbs, while the limbs stay in bf16's normal
// range, |x| >= 2^-110), and a product a*b is the sum of the six limb
// products whose orders add to <= 2: h*h, h*m, m*h, h*l, m*m, l*h.
// The dropped terms are <= 2^-26 |a b|, each limb product is exact and the
// MFMA accumulates in fp32, so a dot product carries fp32-level error (below
// that of a sequential fp32 FMA chain for D = 64) while
// v_mfma_f32_32x32x16_bf16 does 8x the multiply-adds of the fp32
// v_mfma_f32_32x32x2_f32 per instruction.  The six products are issued small
// terms first.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct Limbs {  // one 8-element MFMA operand in three limbs (4 VGPRs each)
  bf16x8 h, m, l;
};

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// c += a * b over 16 k values, to fp32 accuracy
__device__ __forceinline__ f32x16 mfma_x6(const Limbs& a, const Limbs& b, f32x16 c) {
  c = mfma_bf16(a.l, b.h, c);
  c = mfma_bf16(a.m, b.m, c);
  c = mfma_bf16(a.h, b.l, c);
  c = mfma_bf16(a.m, b.h, c);
  c = mfma_bf16(a.h, b.m, c);
  return mfma_bf16(a.h, b.h, c);
}

// 16x16x32 tile (v_mfma_f32_16x16x32_bf16): A lane l supplies row l%16,
// k = 8*(l/16) + e; B lane l supplies column l%16, same k; the result lane l
// holds column l%16, rows 4*(l/16) + r.
__device__ __forceinline__ f32x4 mfma16_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16_x6(const Limbs& a, const Limbs& b, f32x4 c) {
  c = mfma16_bf16(a.l, b.h, c);
  c = mfma16_bf16(a.m, b.m, c);
  c = mfma16_bf16(a.h, b.l, c);
  c = mfma16_bf16(a.m, b.h, c);
  c = mfma16_bf16(a.h, b.m, c);
  return mfma16_bf16(a.h, b.h, c);
}

// One of the six limb products of mfma16_x6 (step 0..5, small terms first);
// issuing step k on several independent accumulators before step k+1 keeps
// dependent MFMAs apart.
__device__ __forceinline__ f32x4 mfma16_step(int step, const Limbs& a, const Limbs& b, f32x4 c) {
  switch (step) {
    case 0: return mfma16_bf16(a.l, b.h, c);
    case 1: return mfma16_bf16(a.m, b.m, c);
    case 2: return mfma16_bf16(a.h, b.l, c);
    case 3: return mfma16_bf16(a.m, b.h, c);
    case 4: return mfma16_bf16(a.h, b.m, c);
    default: return mfma16_bf16(a.h, b.h, c);
  }
}

// bf16-valued operands: an fp32 value that is exactly a bf16 number splits
// into h = the value and m = l = 0, so the limb products that use its m or l
// limb are exactly zero and are skipped (an MFMA adding zero products leaves
// the accumulator unchanged, so the result is the same bit for bit).
// limb_step_used<ABF, BBF>(st): step st of mfma16_step (a.l b.h, a.m b.m,
// a.h b.l, a.m b.h, a.h b.m, a.h b.h) is nonzero when operand a (ABF) / b
// (BBF) is bf16-valued.
template <bool ABF, bool BBF>
__host__ __device__ constexpr bool limb_step_used(int st) {
  const bool a_low = st == 0 || st == 1 || st == 3;  // uses a.m or a.l
  const bool b_low = st == 1 || st == 2 || st == 4;  // uses b.m or b.l
  return !(ABF && a_low) && !(BBF && b_low);
}
// c += a * b over 16 k values (32x32x16 tiles) with bf16-valued a: the three
// products of a.h, small terms first (the nonzero steps of mfma_x6)
__device__ __forceinline__ f32x16 mfma_x3_abf(bf16x8 ah, const Limbs& b, f32x16 c) {
  c = mfma_bf16(ah, b.l, c);
  c = mfma_bf16(ah, b.m, c);
  return mfma_bf16(ah, b.h, c);
}

// Transposed LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane
// i receives element (i & 3) of the 4 bf16 that lanes 4j + (i >> 2) address,
// for j = 0..3.  With lane i' = 4j + m pointing at row r0 + j, column c0 + 4m
// of a row-major bf16 tile, lane i gets column c0 + i of rows r0..r0+3.  Two
// such reads give one 8-element MFMA operand.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ bf16x8 lds_read_tr8(const __bf16* p0, const __bf16* p1) {
  typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
  const s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(p0));
  const s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(p1));
  const s16x8 v = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);  // whole-vector casts only
}

// Lane j of each 16-lane row receives x of lane j-1 (lane 0: 0) / of lane j+1
// (lane 15: 0).
__device__ __forceinline__ float row_shr1(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_shl1(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x101, 0xf, 0xf, true));
}

// two floats -> packed bf16 pair, round to nearest even; a in the low half
__device__ __forceinline__ unsigned cvt_pk_bf16(float a, float b) {
  unsigned r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// limbs of the pair (a, b): h, m, l packed pairs
__device__ __forceinline__ void split_pair(float a, float b, unsigned& h, unsigned& m,
                                           unsigned& l) {
  h = cvt_pk_bf16(a, b);
  const float ra = a - __uint_as_float(h << 16), rb = b - __uint_as_float(h & 0xffff0000u);
  m = cvt_pk_bf16(ra, rb);
  const float sa = ra - __uint_as_float(m << 16), sb = rb - __uint_as_float(m & 0xffff0000u);
  l = cvt_pk_bf16(sa, sb);
}
// limbs of 8 floats (one MFMA operand)
__device__ __forceinline__ Limbs split8(const float* x) {
  u32x4 H, M, L;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    unsigned h, m, l;
    split_pair(x[2 * p], x[2 * p + 1], h, m, l);
    H[p] = h;
    M[p] = m;
    L[p] = l;
  }
  return Limbs{__builtin_bit_cast(bf16x8, H), __builtin_bit_cast(bf16x8, M),
               __builtin_bit_cast(bf16x8, L)};
}

// Wave priority raised over a wave's matrix-product blocks (s_setprio), so
// the SIMD's other waves fill the VALU while those MFMAs are issued.  ON for
// operands that take all six limb products: fp32 config 2 dK/dV 0.2698 ->
// 0.2677 ms, op 0.5418 -> 0.5389 ms (mean of four runs each), dQ 0.0736 ->
// 0.0731 ms (two runs each); bf16 operands (fewer products) measured 1.5%
// slower with it.
template <bool ON>
__device__ __forceinline__ void prio_mfma_begin() { if (ON) __builtin_amdgcn_s_setprio(1); }
template <bool ON>
__device__ __forceinline__ void prio_mfma_end() { if (ON) __builtin_amdgcn_s_setprio(0); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---- buffer loads -----------------------------------------------------------
// A raw buffer resource over `bytes` bytes at `base`: a load's address is
// base + voffset + soffset, with a per-lane 32-bit voffset and a uniform
// soffset (an SGPR), so loop-invariant per-lane offsets cost no address
// arithmetic; loads whose voffset lies at or past `bytes` return zeros.  The
// range must stay below 4 GiB.  0x00020000 is the gfx9 descriptor word 3 for
// untyped 32-bit data.
// `base` and `bytes` must be the same in every lane (a slice's or a whole
// tensor's); they are taken from the first active lane, so the descriptor
// sits in scalar registers even where the compiler formed them in vector
// registers (the slice index's division by H runs on the VALU) -- otherwise
// every load through it is wrapped in a loop over the lanes' descriptors.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)a);
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(a >> 32));
  void* p = reinterpret_cast<void*>(((unsigned long long)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, __builtin_amdgcn_readfirstlane((int)bytes),
                                           0x00020000);
}
__device__ __forceinline__ u32x4 buffer_ld16(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                             unsigned soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ u32x2 buffer_ld8(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// ---- operand views --------------------------------------------------------
// Element (slice bh = b*H + h, row t, column d) of an operand of element type
// E sits at  base + b*bstride + h*hstride + t*rstride + d.  The operator's own
// tensors [B,H,T,D] (fp32) use (H*T*D, T*D, D); inside the decoder the
// qkv projection output [B,T,3,H,D] serves q, k and v directly (bases H*D
// apart, strides (3*T*H*D, D, 3*H*D)), and the attention output / its
// gradient [B,T,H,D] uses (T*H*D, D, H*D).  Rows of D elements are
// contiguous and start 16-byte (fp32) or 8-byte (16-bit types) aligned.
struct View {
  void* base;
  long long bstride, hstride, rstride;
};
template <class E>
__device__ __forceinline__ E* view_slice(const View& v, int bh, int H) {
  return static_cast<E*>(v.base) + (long long)(bh / H) * v.bstride + (long long)(bh % H) * v.hstride;
}

// Four consecutive elements as loaded (raw) and converted to fp32.  16-bit
// types are stored as bf16 or IEEE half; conversions round to nearest even.
template <class E> struct Raw4;
template <> struct Raw4<float> { typedef f32x4 type; };
template <> struct Raw4<__bf16> { typedef u32x2 type; };
template <> struct Raw4<_Float16> { typedef u32x2 type; };

template <class E>
__device__ __forceinline__ typename Raw4<E>::type ld_raw4(const E* p) {
  return *reinterpret_cast<const typename Raw4<E>::type*>(p);
}
__device__ __forceinline__ f32x4 raw_to_f32(f32x4 r, const float*) { return r; }
__device__ __forceinline__ f32x4 raw_to_f32(u32x2 r, const __bf16*) {
  return f32x4{__uint_as_float(r[0] << 16), __uint_as_float(r[0] & 0xffff0000u),
               __uint_as_float(r[1] << 16), __uint_as_float(r[1] & 0xffff0000u)};
}
__device__ __forceinline__ f32x4 raw_to_f32(u32x2 r, const _Float16*) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 a = __builtin_bit_cast(h4, r);  // whole-vector cast (see bf16x8 below)
  return f32x4{(float)a[0], (float)a[1], (float)a[2], (float)a[3]};
}
// Four consecutive elements through a buffer resource (zeros past its range).
__device__ __forceinline__ f32x4 buffer_ld_raw4(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                const float*) {
  return __builtin_bit_cast(f32x4, buffer_ld16(r, voff, 0));
}
template <class E>
__device__ __forceinline__ u32x2 buffer_ld_raw4(__amdgpu_buffer_rsrc_t r, unsigned voff, const E*) {
  return buffer_ld8(r, voff, 0);
}
// Bytes a buffer resource over rows 0 .. T-1 (row stride rstride, D elements
// of `esize` bytes each) must cover; loads of rows T .. T+31 read zeros.  The
// host refuses views for which this (with 32 rows of slack) reaches 4 GiB.
__host__ __device__ inline unsigned long long view_rows_bytes(int T, long long rstride, int D,
                                                              int esize) {
  return ((unsigned long long)(T - 1) * rstride + D) * esize;
}

template <class E>
__device__ __forceinline__ f32x4 ld4(const E* p) {
  return raw_to_f32(ld_raw4(p), p);
}
template <class E>
__device__ __forceinline__ float ld1(const E* p) {
  return (float)*p;
}
__device__ __forceinline__ float ld1(const __bf16* p) {
  return __uint_as_float((unsigned)*reinterpret_cast<const unsigned short*>(p) << 16);
}

__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void st4(__bf16* p, f32x4 v) {
  *reinterpret_cast<u32x2*>(p) = u32x2{cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3])};
}
__device__ __forceinline__ void st4(_Float16* p, f32x4 v) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  *reinterpret_cast<h4*>(p) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}
__device__ __forceinline__ void st1(float* p, float v) { *p = v; }
__device__ __forceinline__ void st1(__bf16* p, float v) {
  *reinterpret_cast<unsigned short*>(p) = (unsigned short)(cvt_pk_bf16(v, 0.f) & 0xffffu);
}
__device__ __forceinline__ void st1(_Float16* p, float v) { *p = (_Float16)v; }

// RoPE of four consecutive head-dim entries d0..d0+3 (two interleaved pairs)
// of row t: cs is the fp32 table [T][D/2][2] = (cos, sin), whose row t holds D
// floats, so the two pairs' entries are cs[t*D + d0 .. d0+3].  Forward
// rotation x0' = x0 c - x1 s, x1' = x1 c + x0 s; `inverse` applies the
// transpose (the gradient's rotation back).
__device__ __forceinline__ f32x4 rope4(f32x4 x, f32x4 t, bool inverse) {
  const float s0 = inverse ? -t[1] : t[1], s1 = inverse ? -t[3] : t[3];
  return f32x4{x[0] * t[0] - x[1] * s0, x[1] * t[0] + x[0] * s0, x[2] * t[2] - x[3] * s1,
               x[3] * t[2] + x[2] * s1};
}
__device__ __forceinline__ f32x4 rope_entry(const float* cs, long long t, int D, int d0) {
  return *reinterpret_cast<const f32x4*>(cs + t * D + d0);
}

// fp32 value rounded to the element type E (round to nearest even) and back;
// the identity for fp32.
template <class E> __device__ __forceinline__ float round_to(float x) { return x; }
template <> __device__ __forceinline__ float round_to<__bf16>(float x) {
  return __uint_as_float(cvt_pk_bf16(x, 0.f) << 16);
}
template <> __device__ __forceinline__ float round_to<_Float16>(float x) {
  return (float)(_Float16)x;
}
// RoPE of an operand of element type E the way the reference computes it in
// that type (cuda/continuum_attention.py:826-835, q * cos + rotate(q) * sin
// with cos and sin cast to q's dtype): for 16-bit E each product and the sum
// are rounded to E, so the rotated values are E-valued (with t, the (cos,
// sin) pairs, given already rounded to E, every step is the reference's own
// rounding: products of two E values and their sums are formed in fp32 as
// torch's 16-bit arithmetic forms them).  fp32 operands rotate in fp32.
template <class E> __device__ __forceinline__ f32x4 rope4_in(f32x4 x, f32x4 t) {
  if constexpr (sizeof(E) == sizeof(float)) {
    return rope4(x, t, false);
  } else {
    const float c0 = t[0], s0 = t[1], c1 = t[2], s1 = t[3];
    return f32x4{round_to<E>(round_to<E>(x[0] * c0) - round_to<E>(x[1] * s0)),
                 round_to<E>(round_to<E>(x[1] * c0) + round_to<E>(x[0] * s0)),
                 round_to<E>(round_to<E>(x[2] * c1) - round_to<E>(x[3] * s1)),
                 round_to<E>(round_to<E>(x[3] * c1) + round_to<E>(x[2] * s1))};
  }
}

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

__device__ __forceinline__ float poly2(float y, float c0, float c1, float c2) {
  return fmaf(fmaf(c2, y, c1), y, c0);
}
// CA_J1_EVEN
__device__ __forceinline__ float j1_even(float y) {
  return poly2(y, 5.000000812e-01f, 1.249939939e-01f, 7.009293473e-03f);
}
// CA_J1_ODD
__device__ __forceinline__ float j1_odd(float y) {
  return poly2(y, 3.333331177e-01f, 3.333620685e-02f, 1.187037119e-03f);
}
// CA_J2_EVEN
__device__ __forceinline__ float j2_even(float y) {
  return poly2(y, 3.333334046e-01f, 9.999468968e-02f, 6.009913146e-03f);
}
// CA_J2_ODD
__device__ __forceinline__ float j2_odd(float y) {
  return poly2(y, 2.499997786e-01f, 2.778081007e-02f, 1.037130167e-03f);
}

// Forward shares of one segment: L -> left key, R -> right key.
// x is the signed natural score difference s_r - s_l; pl/pr are the endpoint
// weights relative to the row shift.  seg_shares takes log2-unit scores sl/sr
// (pl/pr = 2^sl, 2^sr) instead of x.
// Both branches are evaluated and selected (no divergent control flow).
__device__ __forceinline__ void seg_shares_x(float x, float pl, float pr, float& L, float& R) {
  const float dp = pr - pl;
  const float inv_x = fast_rcp(x);
  // a = dp/x = p_l J0 enters both shares through fused multiply-adds
  const float rc = fmaf(-dp, inv_x, pr) * inv_x;  // (p_r - a) / x = p_l J1
  const float lc = fmaf(dp, inv_x, -rc);          // a - R = p_l (J0 - J1)
  const float y = x * x;
  const float e1 = j1_even(y), o1 = j1_odd(y);
  const float rs = pl * fmaf(x, o1, e1);   // p_l J1(x)
  const float ls = pr * fmaf(-x, o1, e1);  // p_r J1(-x)
  const bool small = fabsf(x) < kSeriesT;
  R = small ? rs : rc;
  L = small ? ls : lc;
}
__device__ __forceinline__ void seg_shares(float sl, float sr, float pl, float pr, float& L,
                                           float& R) {
  seg_shares_x((sr - sl) * kLn2, pl, pr, L, R);
}

// Forward shares and score-gradient contributions of one segment.
// gl/gr are the centred, 1/Z-scaled weight gradients g = (dY.v - Dl) / Z.
__device__ __forceinline__ void seg_shares_grad_x(float x, float pl, float pr, float gl, float gr,
                                                  float& L, float& R, float& dL, float& dR) {
  const float dp = pr - pl;
  const float inv_x = fast_rcp(x);
  const float rc = fmaf(-dp, inv_x, pr) * inv_x;
  const float lc = fmaf(dp, inv_x, -rc);
  const float j2c = fmaf(-2.0f, rc, pr) * inv_x;  // p_l J2
  const float y = x * x;
  const float e1 = j1_even(y), o1 = j1_odd(y);
  const float rs = pl * fmaf(x, o1, e1);
  const float ls = pr * fmaf(-x, o1, e1);
  const float j2s = pl * fmaf(x, j2_odd(y), j2_even(y));
  const bool small = fabsf(x) < kSeriesT;
  R = small ? rs : rc;
  L = small ? ls : lc;
  const float j2 = small ? j2s : j2c;
  const float xm = R - j2;  // p_l (J1 - J2)
  dR = fmaf(gl, xm, gr * j2);
  dL = fmaf(gl, L - xm, gr * xm);
}
__device__ __forceinline__ void seg_shares_grad(float sl, float sr, float pl, float pr, float gl,
                                                float gr, float& L, float& R, float& dL,
                                                float& dR) {
  seg_shares_grad_x((sr - sl) * kLn2, pl, pr, gl, gr, L, R, dL, dR);
}

__device__ __forceinline__ float wave_max(float x) {
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
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
