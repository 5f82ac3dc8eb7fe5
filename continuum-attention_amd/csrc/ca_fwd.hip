// Continuum Attention forward (gfx950, fp32 products on the bf16 matrix cores).
//
// Replaces, for the forward pass, the per-query-tile loop of
// _CAExactTiled.forward (cuda/continuum_attention.py:650-694): the QK^T bmm,
// the weight kernel (ca_weights_kernel / ca_forward_half_kernel,
// cuda/continuum_attention.py:136-163,300-328) and the W.V bmm, fused so that
// neither scores nor weights leave registers.
//
// Work item: one 128-query group (4 waves x 32 queries) of one (b,h) slice and
// one contiguous range ("split") of 32-key weight tiles.  The 4 waves share
// double-buffered K/V tiles in LDS, stored as bf16 limb planes (the split of
// each fp32 value into three bf16 limbs happens once, when the tile is
// staged).  Items are launched heaviest-first; groups whose key range spans
// several splits write un-normalised partials that ca_fwd_combine merges
// (log-sum-exp style; deterministic order).
//
// Both products run as bf16x6 (six limb products per fp32 product, fp32
// accumulation; mfma_x6) on v_mfma_f32_32x32x16_bf16.  Per wave, the S^T =
// K Q^T tile (32 keys x 32 queries) has keys permuted so that lane (q, h)
// holds 16 consecutive keys of query q; the K tile is stored in that row
// order.  Segment neighbours are then in the same lane; only the segment
// crossing the two lane halves needs permlane32_swap.  In O^T += V^T W^T the
// MFMA's k index 8h + e of k-block kb stands for weight key 16h + 8kb + e, so
// each lane feeds its own weights as the B operand and reads V^T (stored
// transposed) with one 16-byte LDS read per limb.
//
// Weight tile t covers weight keys [32t, 32t+32); its score tile covers keys
// [32t+1, 32t+33).  Lane half h, register n: score key 32t+1+16h+n, weight
// key 32t+16h+n.  The segment ending at score key k gives its left share to
// weight key k-1 (same register) and its right share to weight key k (next
// register; carried across halves / tiles).
#include <type_traits>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

template <int D>
struct Fwd {
  static constexpr int DH = D / 2;            // d values per lane half in the S^T operand
  static constexpr int KB = (DH + 7) / 8;     // 16-wide k blocks of S^T (8 d per lane half each)
  static constexpr int NMB = (D + 31) / 32;   // 32-row d blocks of O^T
  static constexpr int C4 = D / 4;            // float4 chunks per row
  static constexpr int CH = DH / 4;           // float4 chunks per lane half
  static constexpr int TILE_F4 = 32 * C4;     // float4 per 32-row tile
  static constexpr int LD_PER_THREAD = (TILE_F4 + 255) / 256;
  static constexpr int VUNITS = 16 * C4;      // (key pair, float4 chunk) units of a V tile
  static constexpr int VLD = (VUNITS + 255) / 256;
  // K limb plane: row p = key key_of_arow(p); two halves of 8*KB bf16 (d values
  // h*DH + ..., zero-padded when DH < 8) and 16 bf16 of padding (160-byte rows
  // for D = 64: the 16-byte A-operand reads hit distinct banks).
  static constexpr int KROW = 16 * KB + 16;
  static constexpr int KPLANE = 32 * KROW;
  // V^T limb plane: row d holds the 32 weight keys of the tile (+8 padding).
  static constexpr int VROW = 40;
  static constexpr int VPLANE = D * VROW;
};

// LDS row of the permuted K tile that holds tile key k (inverse of key_of_arow).
__device__ __forceinline__ int arow_of_key(int k) {
  return (((k >> 2) & 3) << 3) | (((k >> 4) & 1) << 2) | (k & 3);
}

// Item decoding: items are (group g, split s) in descending g, then s.
__device__ __forceinline__ void fwd_decode_item(int item, int G, int T, int C, int& g, int& s,
                                                int& nsplit) {
  const int ntiles_all = (T + 31) / 32;
  for (int gg = G - 1; gg >= 0; --gg) {
    int nt = min(4 * gg + 4, ntiles_all);
    int ns = (nt + C - 1) / C;
    if (item < ns) {
      g = gg;
      s = item;
      nsplit = ns;
      return;
    }
    item -= ns;
  }
  g = -1; s = 0; nsplit = 0;
}

// q . k of key `key` (RoPE applied to the key when `rope`), reduced over the
// two lane halves that hold the query's halves.
template <int D, class E>
__device__ __forceinline__ float halo_dot(const float* qreg, const E* __restrict__ Ks,
                                          long long rstride, const float* __restrict__ rope,
                                          int key) {
  constexpr int DH = D / 2;
  const int h = (threadIdx.x >> 5) & 1;
  const E* kp = Ks + (long long)key * rstride + h * DH;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < DH / 4; ++c) {
    f32x4 kv = ld4(kp + 4 * c);
    if (rope) kv = rope4_in<E>(kv, rope_entry(rope, key, D, h * DH + 4 * c));
    acc = fmaf(qreg[4 * c + 0], kv[0], acc);
    acc = fmaf(qreg[4 * c + 1], kv[1], acc);
    acc = fmaf(qreg[4 * c + 2], kv[2], acc);
    acc = fmaf(qreg[4 * c + 3], kv[3], acc);
  }
  return acc + xhalf(acc);
}

// Waves per SIMD the register budget is set for: bf16 operands stage one
// limb plane and take one product per k block of S, so with keys rotated
// beforehand (no table reads) they fit four (128 VGPRs, 20 KB of LDS per
// work group; one CA-S layer's forward 0.0708 -> 0.0689 ms), with in-kernel
// key rotation three; other operand types two.
template <int D, class E, bool ROPE>
constexpr int fwd_waves_per_simd() {
  return D > 64 ? 1 : std::is_same<E, __bf16>::value ? (ROPE ? 3 : 4) : 2;
}

template <int D, class E, bool ROPE>
__global__ __launch_bounds__(256, (fwd_waves_per_simd<D, E, ROPE>())) void ca_fwd_kernel(
    View Qv, View Kv, View Vv, const float* __restrict__ rope, const float* __restrict__ log_gain,
    float* __restrict__ O, View Ov, float* __restrict__ stats, float* __restrict__ part, int BH,
    int H, int T, int C, int G, int smax) {
  using P = Fwd<D>;
  // bf16 operands (with RoPE rounded to bf16 as the reference does) are
  // bf16-valued: their limb split is h = the value, m = l = 0, so a K or V
  // tile is staged as its h plane alone and every product with it takes the
  // three nonzero limb products (mfma_x3_abf), bit for bit the same sums.
  constexpr bool BF = std::is_same<E, __bf16>::value;
  constexpr int NL = BF ? 1 : 3;  // limb planes staged per K and V tile
  // [buffer][limb][plane]
  __shared__ __attribute__((aligned(16))) __bf16 lds_k[2][NL][P::KPLANE];
  __shared__ __attribute__((aligned(16))) __bf16 lds_vt[2][NL][P::VPLANE];

  const int bh = blockIdx.x % BH;
  const int item = blockIdx.x / BH;
  int g, split, nsplit;
  fwd_decode_item(item, G, T, C, g, split, nsplit);
  if (g < 0) return;

  const int ntiles_all = (T + 31) / 32;
  const int nt = min(4 * g + 4, ntiles_all);
  const int t_b = split * C;
  const int t_e = min(nt, t_b + C);

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int q = lane & 31;
  const int h = lane >> 5;
  const int i = 128 * g + 32 * w + q;  // this lane's query
  const bool qvalid = i < T;
  const int wave_tmax = 4 * g + w;      // diagonal tile of this wave
  const bool wave_active = (128 * g + 32 * w < T) && (t_b <= wave_tmax);

  const size_t slice = (size_t)bh * T * D;
  const E* __restrict__ Qs = view_slice<const E>(Qv, bh, H);
  const E* __restrict__ Ks = view_slice<const E>(Kv, bh, H);
  const E* __restrict__ Vs = view_slice<const E>(Vv, bh, H);
  const long long krs = Kv.rstride, vrs = Vv.rstride;
  // RoPE: q is rotated (once per lane) whenever `rope` is given; the keys are
  // rotated as they are read only when ROPE (otherwise they arrive rotated,
  // or unrotated without RoPE), so the compiler drops every key rotation
  const float* __restrict__ rope_k = ROPE ? rope : nullptr;
  const int head = bh % H;
  const float cl2 = head_scale_log2(log_gain, head, D);

  // lane (q,h) holds Q[i][h*DH + k].  The scores are scaled after the
  // product, as the reference scales q.k (s = c log2e (q.k) - m_ref, one
  // fused multiply-add per score): bf16 operands then stay bf16-valued, and
  // their S^T takes one limb product per k block.
  float qreg[P::DH];
  {
    const E* qp = Qs + (long long)(qvalid ? i : 0) * Qv.rstride + h * P::DH;
#pragma unroll
    for (int c = 0; c < P::CH; ++c) {
      f32x4 v4 = qvalid ? ld4(qp + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
      if (rope && qvalid) v4 = rope4_in<E>(v4, rope_entry(rope, i, D, h * P::DH + 4 * c));
      qreg[4 * c + 0] = v4[0];
      qreg[4 * c + 1] = v4[1];
      qreg[4 * c + 2] = v4[2];
      qreg[4 * c + 3] = v4[3];
    }
  }

  // ---- split-start state -------------------------------------------------
  float m_ref = 0.f, s_carry = 0.f, r_carry = 0.f, zsum = 0.f;
  if (wave_active) {
    if (t_b == 0) {
      m_ref = halo_dot<D>(qreg, Ks, krs, rope_k, 0) * cl2;
      s_carry = 0.0f;  // score of key 0 relative to m_ref
    } else {
      const int k0 = 32 * t_b;  // <= first query of this wave, so both halo keys are visible
      s_carry = halo_dot<D>(qreg, Ks, krs, rope_k, k0) * cl2;
      const float s_prev = halo_dot<D>(qreg, Ks, krs, rope_k, k0 - 1) * cl2;
      m_ref = fmaxf(s_carry, s_prev);
      float l_unused;
      seg_shares(s_prev, s_carry, fast_exp2(s_prev - m_ref), fast_exp2(s_carry - m_ref), l_unused,
                 r_carry);
      s_carry -= m_ref;  // carried scores are kept relative to m_ref
    }
  }

  // B operand of S^T in limbs: k block kb, element e = Q[i][h*DH + 8kb + e]
  Limbs qb[P::KB];
#pragma unroll
  for (int kb = 0; kb < P::KB; ++kb) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (8 * kb + e < P::DH) ? qreg[8 * kb + e] : 0.f;
    qb[kb] = split8(x);
  }

  f32x16 acc_o[P::NMB];
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[mb][r] = 0.f;

  // Half-padded K rows (DH < 8) keep zeros in their pad slots: clear both
  // buffers once; the tile stores never write the pads.
  if (P::DH < 8) {
    unsigned* z = reinterpret_cast<unsigned*>(&lds_k[0][0][0]);
    for (int e = tid; e < 2 * NL * P::KPLANE / 2; e += 256) z[e] = 0u;
    __syncthreads();
  }

  // ---- cooperative tile loads ------------------------------------------
  // K: float4 chunk e -> score key 32t+1+row, d = 4c..4c+3.  V: unit u ->
  // weight keys 32t+2pp, +1 (a key pair, so the transposed store writes
  // packed bf16 pairs), d = 4c..4c+3, with pp = u % 16 the fast index: the 16
  // lanes of one c write 16 consecutive words of each V^T row, and the four c
  // of a wave rows 80 words apart, so the stores of a wave hit 64 distinct
  // banks (the loads still read whole 64-byte row segments).
  // The loads of the next tile stay raw (input element type, RoPE entries
  // beside them) until store_tile, so the tile in flight is not waited for.
  typedef typename Raw4<E>::type R4;
  R4 pre_k[P::LD_PER_THREAD], pre_v[P::VLD][2];
  f32x4 pre_cs[ROPE ? P::LD_PER_THREAD : 1];
  // K, V (and RoPE table) rows through buffer resources: rows at or past T
  // read as zeros (the hardware range check), and a tile's offsets are the
  // thread's fixed offsets plus one uniform step per tile.
  constexpr unsigned kEsz = sizeof(E);
  const __amdgpu_buffer_rsrc_t kres = buffer_rsrc(Ks, (unsigned)view_rows_bytes(T, krs, D, kEsz));
  const __amdgpu_buffer_rsrc_t vres = buffer_rsrc(Vs, (unsigned)view_rows_bytes(T, vrs, D, kEsz));
  const __amdgpu_buffer_rsrc_t cres =
      buffer_rsrc(ROPE ? rope_k : log_gain, ROPE ? (unsigned)(T * D * sizeof(float)) : 0u);
  const unsigned kstep = 32u * (unsigned)krs * kEsz, vstep = 32u * (unsigned)vrs * kEsz;
  const unsigned vrow = (unsigned)vrs * kEsz;
  unsigned koff[P::LD_PER_THREAD], csoff[P::LD_PER_THREAD], voff[P::VLD];
#pragma unroll
  for (int j = 0; j < P::LD_PER_THREAD; ++j) {
    const int e = tid + 256 * j;
    const int row = e / P::C4, c = e % P::C4;  // score key 32t + 1 + row
    koff[j] = ((unsigned)(1 + row) * (unsigned)krs + 4 * c) * kEsz;
    csoff[j] = ((unsigned)(1 + row) * D + 4 * c) * (unsigned)sizeof(float);
  }
#pragma unroll
  for (int j = 0; j < P::VLD; ++j) {
    const int u = tid + 256 * j;
    const int pp = u % 16, c = u / 16;  // weight keys 32t + 2pp, +1
    voff[j] = ((unsigned)(2 * pp) * (unsigned)vrs + 4 * c) * kEsz;
  }
  auto load_tile = [&](int t) {
#pragma unroll
    for (int j = 0; j < P::LD_PER_THREAD; ++j) {
      const int e = tid + 256 * j;
      if (P::TILE_F4 % 256 == 0 || e < P::TILE_F4) {
        pre_k[j] = buffer_ld_raw4(kres, koff[j] + t * kstep, Ks);
        if constexpr (ROPE)
          pre_cs[j] = __builtin_bit_cast(f32x4, buffer_ld16(cres, csoff[j] + t * (32u * D * 4u), 0));
      }
    }
#pragma unroll
    for (int j = 0; j < P::VLD; ++j) {
      const int u = tid + 256 * j;
      if (P::VUNITS % 256 == 0 || u < P::VUNITS) {
        pre_v[j][0] = buffer_ld_raw4(vres, voff[j] + t * vstep, Vs);
        pre_v[j][1] = buffer_ld_raw4(vres, voff[j] + t * vstep + vrow, Vs);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < P::LD_PER_THREAD; ++j) {
      const int e = tid + 256 * j;
      if (e < P::TILE_F4) {
        const int row = e / P::C4, c = e % P::C4;
        const int d = 4 * c, half = d / P::DH;
        const int off = arow_of_key(row) * P::KROW + half * 8 * P::KB + (d - half * P::DH);
        if constexpr (BF && !ROPE) {
          // the raw bf16 row chunk is its own h limb
          *reinterpret_cast<u32x2*>(&lds_k[buf][0][off]) = pre_k[j];
        } else {
          f32x4 kv = raw_to_f32(pre_k[j], Ks);
          if constexpr (ROPE) kv = rope4_in<E>(kv, pre_cs[j]);
          if constexpr (BF) {
            // rotated and rounded to bf16: exact in one limb
            *reinterpret_cast<u32x2*>(&lds_k[buf][0][off]) =
                u32x2{cvt_pk_bf16(kv[0], kv[1]), cvt_pk_bf16(kv[2], kv[3])};
          } else {
            unsigned h0, m0, l0, h1, m1, l1;
            split_pair(kv[0], kv[1], h0, m0, l0);
            split_pair(kv[2], kv[3], h1, m1, l1);
            *reinterpret_cast<u32x2*>(&lds_k[buf][0][off]) = u32x2{h0, h1};
            *reinterpret_cast<u32x2*>(&lds_k[buf][1][off]) = u32x2{m0, m1};
            *reinterpret_cast<u32x2*>(&lds_k[buf][2][off]) = u32x2{l0, l1};
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < P::VLD; ++j) {
      const int u = tid + 256 * j;
      if (u < P::VUNITS) {
        const int pp = u % 16, c = u / 16;
        if constexpr (BF) {
          // V^T row 4c + x, keys 2pp, 2pp + 1: the bf16 halves of the two rows
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            const unsigned wa = pre_v[j][0][x >> 1], wb = pre_v[j][1][x >> 1];
            const unsigned pair = (x & 1) ? ((wa >> 16) | (wb & 0xffff0000u))
                                          : ((wa & 0xffffu) | (wb << 16));
            *reinterpret_cast<unsigned*>(&lds_vt[buf][0][(4 * c + x) * P::VROW + 2 * pp]) = pair;
          }
        } else {
          const f32x4 va = raw_to_f32(pre_v[j][0], Vs), vb = raw_to_f32(pre_v[j][1], Vs);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            unsigned hv, mv, lv;
            split_pair(va[x], vb[x], hv, mv, lv);
            const int off = (4 * c + x) * P::VROW + 2 * pp;
            *reinterpret_cast<unsigned*>(&lds_vt[buf][0][off]) = hv;
            *reinterpret_cast<unsigned*>(&lds_vt[buf][1][off]) = mv;
            *reinterpret_cast<unsigned*>(&lds_vt[buf][2][off]) = lv;
          }
        }
      }
    }
  };

  load_tile(t_b);
  store_tile(0);
  __syncthreads();

  const bool dok = q < D;  // only D < 32 pads the d block of O^T

  for (int t = t_b; t < t_e; ++t) {
    const int buf = (t - t_b) & 1;
    if (t + 1 < t_e) load_tile(t + 1);

    // The first tile (first half-token cap) and the diagonal tile (causal mask,
    // last cap) take the general path; every other tile needs neither.
    auto tile = [&](auto general_tag) {
      constexpr bool kGeneral = decltype(general_tag)::value;
      const bool diag = kGeneral && (t == wave_tmax);
      // ---- S^T = c log2e (K Q^T) - m_ref (log2 units; the scale and the
      //      row shift are one fused multiply-add per score) ----
      f32x16 sacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
      prio_mfma_begin<!BF>();
      {
        const __bf16* krow = &lds_k[buf][0][q * P::KROW + h * 8 * P::KB];
#pragma unroll
        for (int kb = 0; kb < P::KB; ++kb) {
          if constexpr (BF) {
            // both operands bf16-valued: the h limbs carry the whole product
            sacc = mfma_bf16(*reinterpret_cast<const bf16x8*>(krow + 8 * kb), qb[kb].h, sacc);
          } else {
            Limbs ka;
            ka.h = *reinterpret_cast<const bf16x8*>(krow + 8 * kb);
            ka.m = *reinterpret_cast<const bf16x8*>(krow + P::KPLANE + 8 * kb);
            ka.l = *reinterpret_cast<const bf16x8*>(krow + 2 * P::KPLANE + 8 * kb);
            sacc = mfma_x6(ka, qb[kb], sacc);
          }
        }
      }
      prio_mfma_end<!BF>();
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = fmaf(sacc[r], cl2, -m_ref);
      const int kbase = 32 * t + 1 + 16 * h;  // score key of register 0
      // ---- row max of the tile (visible keys only), relative to m_ref ----
      float mt = kNegBig;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool vis = !diag || (kbase + r <= i);
        mt = fmaxf(mt, vis ? sacc[r] : kNegBig);
      }
      mt = fmaxf(mt, xhalf(mt));
      // Lazy rescale, decided per query: a lane whose own max did not grow
      // shifts by exactly 0 and scales by exactly 1, so no query's rounding
      // depends on other (possibly later) queries of the wave.
      const bool grow = mt > kLazyRescale;
      if (wave_any(grow)) {
        const float shift = grow ? mt : 0.0f;
        const float alpha = grow ? fast_exp2(-shift) : 1.0f;
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc_o[mb][r] *= alpha;
        zsum *= alpha;
        r_carry *= alpha;
        m_ref += shift;
        s_carry -= shift;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] -= shift;
      }
      if (diag) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = (kbase + r <= i) ? sacc[r] : 0.0f;
      }
      // ---- left neighbour of register 0, and carries (all relative to m_ref) ----
      const float xs15 = xhalf(sacc[15]);
      float sl = h ? xs15 : s_carry;
      s_carry = xs15;  // next tile, half 0: score key 32t+32
      float pl = fast_exp2(sl);

      // ---- stream over segments; weights overwrite sacc in place ----
      // weight register r (weight key kbase-1+r) = left share of segment r
      // + right share of segment r-1 (+ caps); register 0's incoming right
      // share is added after the loop.
      float r_prev = 0.f, zt = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float sr = sacc[r];
        const float pr = fast_exp2(sr);
        float Lv, Rv;
        seg_shares(sl, sr, pl, pr, Lv, Rv);
        const bool seg_ok = !diag || (kbase + r <= i);
        Lv = seg_ok ? Lv : 0.0f;
        Rv = seg_ok ? Rv : 0.0f;
        float x = Lv + r_prev;
        const int wk = kbase - 1 + r;  // weight key, its score is sl
        if constexpr (kGeneral) {
          const float cap_last = (diag && wk == i) ? 0.5f * pl : 0.0f;  // last half-token cap
          const float cap_first = wk == 0 ? 0.5f * pl : 0.0f;           // first half-token cap
          x += cap_last + cap_first;
        }
        sacc[r] = x;
        zt += x;
        r_prev = Rv;
        sl = sr;
        pl = pr;
      }
      const float xr15 = xhalf(r_prev);
      const float r_in = h ? xr15 : r_carry;
      r_carry = xr15;
      sacc[0] += r_in;
      zsum += zt + r_in;
      prio_mfma_begin<!BF>();

      // ---- O^T += V^T W^T: k block kb, element e = weight key 16h + 8kb + e ----
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = sacc[8 * kb + e];
        const Limbs wb = split8(x);
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb) {
          const __bf16* vrow = &lds_vt[buf][0][(dok ? 32 * mb + q : 0) * P::VROW + 16 * h + 8 * kb];
          if constexpr (BF) {
            const bf16x8 vh = dok ? *reinterpret_cast<const bf16x8*>(vrow) : bf16x8{};
            acc_o[mb] = mfma_x3_abf(vh, wb, acc_o[mb]);
          } else {
            Limbs va;
            va.h = *reinterpret_cast<const bf16x8*>(vrow);
            va.m = *reinterpret_cast<const bf16x8*>(vrow + P::VPLANE);
            va.l = *reinterpret_cast<const bf16x8*>(vrow + 2 * P::VPLANE);
            if (!dok) va = Limbs{bf16x8{}, bf16x8{}, bf16x8{}};
            acc_o[mb] = mfma_x6(va, wb, acc_o[mb]);
          }
        }
      }
      prio_mfma_end<!BF>();
    };
    if (wave_active && t <= wave_tmax) {
      if (t == 0 || t == wave_tmax)
        tile(std::true_type{});
      else
        tile(std::false_type{});
    }

    if (t + 1 < t_e) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  if (128 * g + 32 * w >= T) return;
  const float ztot = zsum + xhalf(zsum);
  const bool single = (nsplit == 1);
  float* dst;
  float scl;
  if (single) {
    dst = O + slice + (size_t)i * D;
    scl = 1.0f / ztot;
  } else {
    // part layout: [BH][smax][T][D] outputs then [BH][smax][T][2] (m, Z)
    dst = part + (((size_t)bh * smax + split) * T + i) * D;
    scl = 1.0f;
  }
  if (!wave_active) {
    // this wave's queries see none of this split's keys: empty partial
    if (qvalid) {
      for (int d = h; d < D; d += 2) dst[d] = 0.f;
      if (h == 0) {
        float* mz = part + (size_t)BH * smax * T * D + (((size_t)bh * smax + split) * T + i) * 2;
        mz[0] = -1e30f;
        mz[1] = 0.f;
      }
    }
    return;
  }
  if (!qvalid) return;
  // a single-split row is final: also written token-major in the input type
  E* otok = (single && Ov.base) ? view_slice<E>(Ov, bh, H) + (long long)i * Ov.rstride : nullptr;
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = 32 * mb + 8 * r4 + 4 * h;
      if (d0 < D) {
        f32x4 v4 = {acc_o[mb][4 * r4 + 0] * scl, acc_o[mb][4 * r4 + 1] * scl,
                    acc_o[mb][4 * r4 + 2] * scl, acc_o[mb][4 * r4 + 3] * scl};
        *reinterpret_cast<f32x4*>(dst + d0) = v4;
        if (otok) st4(otok + d0, v4);
      }
    }
  }
  if (h == 0) {
    if (single) {
      stats[((size_t)bh * T + i) * 2 + 0] = m_ref;
      stats[((size_t)bh * T + i) * 2 + 1] = scl;
    } else {
      float* mz = part + (size_t)BH * smax * T * D + (((size_t)bh * smax + split) * T + i) * 2;
      mz[0] = m_ref;
      mz[1] = ztot;
    }
  }
}

// ---- the 16x16x32 forward ---------------------------------------------------
// The same work item (a 128-query group of one slice and a split of its
// 32-key weight tiles) on eight waves of 16 queries each, with both products
// on v_mfma_f32_16x16x32_bf16 (16.8 cycles per instruction against 40 for
// 32x32x16, measured: 16% less matrix time for the same flops) and about 120
// VGPRs, so that a CU holds two work groups of eight waves: four waves per
// SIMD instead of two, which hides more of the segment math's latency.
//
// Lane layout.  A wave computes S^T = K Q^T for its 16 queries and a 32-key
// score tile as two 16x16 blocks.  Lane l holds query l%16; its lane row
// G = l/16 holds score keys kbase .. kbase+7 (kbase = 32t+1+8G) in registers
// sc[0..7]: the K tile is staged with key 8G + 4b + r in LDS row
// 16b + 4G + r (k16_row), so the rows 4G..4G+3 that the MFMA returns in lane
// row G of block b are those keys.  Segment neighbours are then in the same
// lane, except the left neighbour of register 0 (register 7 of lane row
// G-1, or the previous tile's for G = 0), reached by a rotation of the lane
// rows.  In O^T += V^T W^T the k index of lane row G is 8G + e, the weight
// keys 32t + 8G + e that the lane itself holds, so each lane feeds its own
// weights as the B operand.
template <int D>
struct Fwd16 {
  static constexpr int KS = D / 32;         // 32-wide k steps of S^T (d)
  static constexpr int NMB = D / 16;        // 16-row d blocks of O^T
  static constexpr int C4 = D / 4;          // float4 chunks per row
  static constexpr int KROW = D + 16;       // bf16 row stride of a K plane (160 bytes at D = 64)
  static constexpr int KPLANE = 32 * KROW;
  static constexpr int VROW = 40;           // V^T row: 32 keys + 8 padding
  static constexpr int VPLANE = D * VROW;
  static constexpr int KCH = 32 * C4;       // K float4 chunks per tile
  static constexpr int KLD = (KCH + 511) / 512;
  static constexpr int VUNITS = 16 * C4;    // (key pair, float4 chunk) units of a V tile
  static constexpr int VLD = (VUNITS + 511) / 512;
};

// LDS row of the staged K tile that holds score key k (0..31) of the tile.
__device__ __forceinline__ int k16_row(int k) { return 16 * ((k >> 2) & 1) + 4 * (k >> 3) + (k & 3); }

// Value held by lane l ^ 16 (swaps lane rows 0 <-> 1 and 2 <-> 3).
__device__ __forceinline__ float xrow16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return (threadIdx.x & 16) ? __uint_as_float(r[0]) : __uint_as_float(r[1]);
}
// Value held by the same lane of the previous lane row (row G-1; row 0
// receives row 3's): G odd is lane l ^ 16, G even lane l ^ 48.
__device__ __forceinline__ float rot_row(float x) {
  const float a = xrow16(x), b = xrow16(xhalf(x));
  return (threadIdx.x & 16) ? a : b;
}

// q . k of key `key` (RoPE applied to the key when `rope`): each lane row
// holds 16 of the query's d values (d = 32ks + 8G + e), reduced over the rows.
template <int D, class E>
__device__ __forceinline__ float halo_dot16(const float (&qv)[Fwd16<D>::KS][8],
                                            const E* __restrict__ Ks, long long rstride,
                                            const float* __restrict__ rope, int key) {
  const int G = (threadIdx.x >> 4) & 3;
  const E* kp = Ks + (long long)key * rstride;
  float acc = 0.0f;
#pragma unroll
  for (int ks = 0; ks < Fwd16<D>::KS; ++ks)
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int d0 = 32 * ks + 8 * G + 4 * h2;
      f32x4 kv = ld4(kp + d0);
      if (rope) kv = rope4_in<E>(kv, rope_entry(rope, key, D, d0));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(qv[ks][4 * h2 + e], kv[e], acc);
    }
  acc += xrow16(acc);
  return acc + xhalf(acc);
}

// Waves per SIMD: two work groups of eight waves per CU at D <= 64; one at
// D = 128 (its double-buffered tiles take 116 KB of LDS).
template <int D, class E, bool ROPE>
constexpr int fwd16_waves_per_simd() {
  return D > 64 ? 2 : 4;
}

template <int D, class E, bool ROPE>
__global__ __launch_bounds__(512, (fwd16_waves_per_simd<D, E, ROPE>())) void ca_fwd16_kernel(
    View Qv, View Kv, View Vv, const float* __restrict__ rope, const float* __restrict__ log_gain,
    float* __restrict__ O, View Ov, float* __restrict__ stats, float* __restrict__ part, int BH,
    int H, int T, int C, int G, int smax) {
  using P = Fwd16<D>;
  constexpr bool BF = std::is_same<E, __bf16>::value;
  constexpr int NL = BF ? 1 : 3;  // limb planes staged per K and V tile
  __shared__ __attribute__((aligned(16))) __bf16 lds_k[2][NL][P::KPLANE];
  __shared__ __attribute__((aligned(16))) __bf16 lds_vt[2][NL][P::VPLANE];

  const int bh = blockIdx.x % BH;
  const int item = blockIdx.x / BH;
  int g, split, nsplit;
  fwd_decode_item(item, G, T, C, g, split, nsplit);
  if (g < 0) return;

  const int ntiles_all = (T + 31) / 32;
  const int nt = min(4 * g + 4, ntiles_all);
  const int t_b = split * C;
  const int t_e = min(nt, t_b + C);

  const int tid = threadIdx.x;
  const int w = tid >> 6;          // 0..7
  const int lane = tid & 63;
  const int q16 = lane & 15;
  const int G4 = lane >> 4;        // lane row
  const int i = 128 * g + 16 * w + q16;  // this lane's query
  const bool qvalid = i < T;
  const int wave_tmax = 4 * g + (w >> 1);  // diagonal weight tile of this wave
  const bool wave_active = (128 * g + 16 * w < T) && (t_b <= wave_tmax);

  const size_t slice = (size_t)bh * T * D;
  const E* __restrict__ Qs = view_slice<const E>(Qv, bh, H);
  const E* __restrict__ Ks = view_slice<const E>(Kv, bh, H);
  const E* __restrict__ Vs = view_slice<const E>(Vv, bh, H);
  const long long krs = Kv.rstride, vrs = Vv.rstride;
  const float* __restrict__ rope_k = ROPE ? rope : nullptr;
  const int head = bh % H;
  const float cl2 = head_scale_log2(log_gain, head, D);

  // lane (q16, G) holds Q[i][32ks + 8G + e] (rotated when `rope`)
  float qv[P::KS][8];
  {
    const E* qp = Qs + (long long)(qvalid ? i : 0) * Qv.rstride;
#pragma unroll
    for (int ks = 0; ks < P::KS; ++ks)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int d0 = 32 * ks + 8 * G4 + 4 * h2;
        f32x4 v4 = qvalid ? ld4(qp + d0) : f32x4{0.f, 0.f, 0.f, 0.f};
        if (rope && qvalid) v4 = rope4_in<E>(v4, rope_entry(rope, i, D, d0));
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[ks][4 * h2 + e] = v4[e];
      }
  }

  // ---- split-start state (as in ca_fwd_kernel) ----
  float m_ref = 0.f, s_carry = 0.f, r_carry = 0.f, zsum = 0.f;
  if (wave_active) {
    if (t_b == 0) {
      m_ref = halo_dot16<D>(qv, Ks, krs, rope_k, 0) * cl2;
    } else {
      const int k0 = 32 * t_b;
      s_carry = halo_dot16<D>(qv, Ks, krs, rope_k, k0) * cl2;
      const float s_prev = halo_dot16<D>(qv, Ks, krs, rope_k, k0 - 1) * cl2;
      m_ref = fmaxf(s_carry, s_prev);
      float l_unused;
      seg_shares(s_prev, s_carry, fast_exp2(s_prev - m_ref), fast_exp2(s_carry - m_ref), l_unused,
                 r_carry);
      s_carry -= m_ref;
    }
  }

  // B operand of S^T: k step ks, element e = Q[i][32ks + 8G + e]
  Limbs qb[P::KS];
#pragma unroll
  for (int ks = 0; ks < P::KS; ++ks) qb[ks] = split8(qv[ks]);

  f32x4 acc_o[P::NMB];
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb) acc_o[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- cooperative tile loads (512 threads) ----
  // K: float4 chunk e -> score key 32t+1+row, d = 4c..4c+3, stored in LDS row
  // k16_row(row).  V: unit u -> weight keys 32t+2pp, +1, d = 4c..4c+3,
  // stored transposed as packed pairs (pp = u % 16 the fast index).
  typedef typename Raw4<E>::type R4;
  R4 pre_k[P::KLD], pre_v[P::VLD][2];
  f32x4 pre_cs[ROPE ? P::KLD : 1];
  constexpr unsigned kEsz = sizeof(E);
  const __amdgpu_buffer_rsrc_t kres = buffer_rsrc(Ks, (unsigned)view_rows_bytes(T, krs, D, kEsz));
  const __amdgpu_buffer_rsrc_t vres = buffer_rsrc(Vs, (unsigned)view_rows_bytes(T, vrs, D, kEsz));
  const __amdgpu_buffer_rsrc_t cres =
      buffer_rsrc(ROPE ? rope_k : log_gain, ROPE ? (unsigned)(T * D * sizeof(float)) : 0u);
  const unsigned kstep = 32u * (unsigned)krs * kEsz, vstep = 32u * (unsigned)vrs * kEsz;
  const unsigned vrow = (unsigned)vrs * kEsz;
  unsigned koff[P::KLD], csoff[P::KLD], voff[P::VLD];
#pragma unroll
  for (int j = 0; j < P::KLD; ++j) {
    const int e = tid + 512 * j;
    const int row = e / P::C4, c = e % P::C4;
    koff[j] = ((unsigned)(1 + row) * (unsigned)krs + 4 * c) * kEsz;
    csoff[j] = ((unsigned)(1 + row) * D + 4 * c) * (unsigned)sizeof(float);
  }
#pragma unroll
  for (int j = 0; j < P::VLD; ++j) {
    const int u = tid + 512 * j;
    const int pp = u % 16, c = u / 16;
    voff[j] = ((unsigned)(2 * pp) * (unsigned)vrs + 4 * c) * kEsz;
  }
  auto load_tile = [&](int t) {
#pragma unroll
    for (int j = 0; j < P::KLD; ++j) {
      const int e = tid + 512 * j;
      if (P::KCH % 512 == 0 || e < P::KCH) {
        pre_k[j] = buffer_ld_raw4(kres, koff[j] + t * kstep, Ks);
        if constexpr (ROPE)
          pre_cs[j] = __builtin_bit_cast(f32x4, buffer_ld16(cres, csoff[j] + t * (32u * D * 4u), 0));
      }
    }
#pragma unroll
    for (int j = 0; j < P::VLD; ++j) {
      const int u = tid + 512 * j;
      if (P::VUNITS % 512 == 0 || u < P::VUNITS) {
        pre_v[j][0] = buffer_ld_raw4(vres, voff[j] + t * vstep, Vs);
        pre_v[j][1] = buffer_ld_raw4(vres, voff[j] + t * vstep + vrow, Vs);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < P::KLD; ++j) {
      const int e = tid + 512 * j;
      if (P::KCH % 512 == 0 || e < P::KCH) {
        const int row = e / P::C4, c = e % P::C4;
        const int off = k16_row(row) * P::KROW + 4 * c;
        if constexpr (BF && !ROPE) {
          *reinterpret_cast<u32x2*>(&lds_k[buf][0][off]) = pre_k[j];
        } else {
          f32x4 kv = raw_to_f32(pre_k[j], Ks);
          if constexpr (ROPE) kv = rope4_in<E>(kv, pre_cs[j]);
          if constexpr (BF) {
            *reinterpret_cast<u32x2*>(&lds_k[buf][0][off]) =
                u32x2{cvt_pk_bf16(kv[0], kv[1]), cvt_pk_bf16(kv[2], kv[3])};
          } else {
            unsigned h0, m0, l0, h1, m1, l1;
            split_pair(kv[0], kv[1], h0, m0, l0);
            split_pair(kv[2], kv[3], h1, m1, l1);
            *reinterpret_cast<u32x2*>(&lds_k[buf][0][off]) = u32x2{h0, h1};
            *reinterpret_cast<u32x2*>(&lds_k[buf][1][off]) = u32x2{m0, m1};
            *reinterpret_cast<u32x2*>(&lds_k[buf][2][off]) = u32x2{l0, l1};
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < P::VLD; ++j) {
      const int u = tid + 512 * j;
      if (P::VUNITS % 512 == 0 || u < P::VUNITS) {
        const int pp = u % 16, c = u / 16;
        if constexpr (BF) {
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            const unsigned wa = pre_v[j][0][x >> 1], wb = pre_v[j][1][x >> 1];
            const unsigned pair = (x & 1) ? ((wa >> 16) | (wb & 0xffff0000u))
                                          : ((wa & 0xffffu) | (wb << 16));
            *reinterpret_cast<unsigned*>(&lds_vt[buf][0][(4 * c + x) * P::VROW + 2 * pp]) = pair;
          }
        } else {
          const f32x4 va = raw_to_f32(pre_v[j][0], Vs), vb = raw_to_f32(pre_v[j][1], Vs);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            unsigned hv, mv, lv;
            split_pair(va[x], vb[x], hv, mv, lv);
            const int off = (4 * c + x) * P::VROW + 2 * pp;
            *reinterpret_cast<unsigned*>(&lds_vt[buf][0][off]) = hv;
            *reinterpret_cast<unsigned*>(&lds_vt[buf][1][off]) = mv;
            *reinterpret_cast<unsigned*>(&lds_vt[buf][2][off]) = lv;
          }
        }
      }
    }
  };

  load_tile(t_b);
  store_tile(0);
  __syncthreads();

  for (int t = t_b; t < t_e; ++t) {
    const int buf = (t - t_b) & 1;
    if (t + 1 < t_e) load_tile(t + 1);

    auto tile = [&](auto general_tag) {
      constexpr bool kGeneral = decltype(general_tag)::value;
      const bool diag = kGeneral && (t == wave_tmax);
      // ---- S^T = c log2e (K Q^T) - m_ref, two 16-key blocks ----
      f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      prio_mfma_begin<!BF>();
#pragma unroll
      for (int ks = 0; ks < P::KS; ++ks) {
        const __bf16* kr0 = &lds_k[buf][0][q16 * P::KROW + 32 * ks + 8 * G4];
        const __bf16* kr1 = kr0 + 16 * P::KROW;
        if constexpr (BF) {
          sacc[0] = mfma16_bf16(*reinterpret_cast<const bf16x8*>(kr0), qb[ks].h, sacc[0]);
          sacc[1] = mfma16_bf16(*reinterpret_cast<const bf16x8*>(kr1), qb[ks].h, sacc[1]);
        } else {
          Limbs ka0, ka1;
          ka0.h = *reinterpret_cast<const bf16x8*>(kr0);
          ka0.m = *reinterpret_cast<const bf16x8*>(kr0 + P::KPLANE);
          ka0.l = *reinterpret_cast<const bf16x8*>(kr0 + 2 * P::KPLANE);
          ka1.h = *reinterpret_cast<const bf16x8*>(kr1);
          ka1.m = *reinterpret_cast<const bf16x8*>(kr1 + P::KPLANE);
          ka1.l = *reinterpret_cast<const bf16x8*>(kr1 + 2 * P::KPLANE);
#pragma unroll
          for (int st = 0; st < 6; ++st) {
            sacc[0] = mfma16_step(st, ka0, qb[ks], sacc[0]);
            sacc[1] = mfma16_step(st, ka1, qb[ks], sacc[1]);
          }
        }
      }
      prio_mfma_end<!BF>();
      float sc[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) sc[r] = fmaf(sacc[r >> 2][r & 3], cl2, -m_ref);
      const int kbase = 32 * t + 1 + 8 * G4;  // score key of sc[0]
      // ---- row max of the tile (visible keys only), relative to m_ref ----
      float mt = kNegBig;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const bool vis = !diag || (kbase + r <= i);
        mt = fmaxf(mt, vis ? sc[r] : kNegBig);
      }
      mt = fmaxf(mt, xrow16(mt));
      mt = fmaxf(mt, xhalf(mt));
      const bool grow = mt > kLazyRescale;
      if (wave_any(grow)) {
        const float shift = grow ? mt : 0.0f;
        const float alpha = grow ? fast_exp2(-shift) : 1.0f;
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb) acc_o[mb] *= alpha;
        zsum *= alpha;
        r_carry *= alpha;
        m_ref += shift;
        s_carry -= shift;
#pragma unroll
        for (int r = 0; r < 8; ++r) sc[r] -= shift;
      }
      if (diag) {
#pragma unroll
        for (int r = 0; r < 8; ++r) sc[r] = (kbase + r <= i) ? sc[r] : 0.0f;
      }
      // ---- left neighbour of sc[0] and carries (relative to m_ref) ----
      const float s_rot = rot_row(sc[7]);
      float sl = G4 == 0 ? s_carry : s_rot;
      s_carry = s_rot;  // row 0 of the next tile: score key 32t+32
      float pl = fast_exp2(sl);

      // ---- segments: weight register r (weight key kbase-1+r) = left share
      // of segment r + right share of segment r-1 (+ caps) ----
      float wt[8];
      float r_prev = 0.f, zt = 0.f;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float sr = sc[r];
        const float pr = fast_exp2(sr);
        float Lv, Rv;
        seg_shares(sl, sr, pl, pr, Lv, Rv);
        const bool seg_ok = !diag || (kbase + r <= i);
        Lv = seg_ok ? Lv : 0.0f;
        Rv = seg_ok ? Rv : 0.0f;
        float x = Lv + r_prev;
        const int wk = kbase - 1 + r;
        if constexpr (kGeneral) {
          const float cap_last = (diag && wk == i) ? 0.5f * pl : 0.0f;
          const float cap_first = wk == 0 ? 0.5f * pl : 0.0f;
          x += cap_last + cap_first;
        }
        wt[r] = x;
        zt += x;
        r_prev = Rv;
        sl = sr;
        pl = pr;
      }
      const float r_rot = rot_row(r_prev);
      const float r_in = G4 == 0 ? r_carry : r_rot;
      r_carry = r_rot;
      wt[0] += r_in;
      zsum += zt + r_in;

      // ---- O^T += V^T W^T: k = weight key 8G + e, d blocks in pairs ----
      const Limbs wb = split8(wt);
      prio_mfma_begin<!BF>();
#pragma unroll
      for (int m2 = 0; m2 < P::NMB; m2 += 2) {
        Limbs va[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const __bf16* vr = &lds_vt[buf][0][(16 * (m2 + u) + q16) * P::VROW + 8 * G4];
          va[u].h = *reinterpret_cast<const bf16x8*>(vr);
          if (BF) {
            va[u].m = va[u].l = bf16x8{};
          } else {
            va[u].m = *reinterpret_cast<const bf16x8*>(vr + P::VPLANE);
            va[u].l = *reinterpret_cast<const bf16x8*>(vr + 2 * P::VPLANE);
          }
        }
#pragma unroll
        for (int st = 0; st < 6; ++st) {
          if (limb_step_used<BF, false>(st)) {
            acc_o[m2] = mfma16_step(st, va[0], wb, acc_o[m2]);
            acc_o[m2 + 1] = mfma16_step(st, va[1], wb, acc_o[m2 + 1]);
          }
        }
      }
      prio_mfma_end<!BF>();
    };
    if (wave_active && t <= wave_tmax) {
      if (t == 0 || t == wave_tmax)
        tile(std::true_type{});
      else
        tile(std::false_type{});
    }

    if (t + 1 < t_e) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane (q16, G) holds d = 16mb + 4G + r of its query ----
  if (128 * g + 16 * w >= T) return;
  float ztot = zsum + xrow16(zsum);
  ztot += xhalf(ztot);
  const bool single = (nsplit == 1);
  float* dst;
  float scl;
  if (single) {
    dst = O + slice + (size_t)i * D;
    scl = 1.0f / ztot;
  } else {
    dst = part + (((size_t)bh * smax + split) * T + i) * D;
    scl = 1.0f;
  }
  if (!wave_active) {
    if (qvalid) {
      for (int d = G4; d < D; d += 4) dst[d] = 0.f;
      if (G4 == 0) {
        float* mz = part + (size_t)BH * smax * T * D + (((size_t)bh * smax + split) * T + i) * 2;
        mz[0] = -1e30f;
        mz[1] = 0.f;
      }
    }
    return;
  }
  if (!qvalid) return;
  E* otok = (single && Ov.base) ? view_slice<E>(Ov, bh, H) + (long long)i * Ov.rstride : nullptr;
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb) {
    const int d0 = 16 * mb + 4 * G4;
    const f32x4 v4 = acc_o[mb] * scl;
    *reinterpret_cast<f32x4*>(dst + d0) = v4;
    if (otok) st4(otok + d0, v4);
  }
  if (G4 == 0) {
    if (single) {
      stats[((size_t)bh * T + i) * 2 + 0] = m_ref;
      stats[((size_t)bh * T + i) * 2 + 1] = scl;
    } else {
      float* mz = part + (size_t)BH * smax * T * D + (((size_t)bh * smax + split) * T + i) * 2;
      mz[0] = m_ref;
      mz[1] = ztot;
    }
  }
}

// Merges split partials of rows whose group spans more than one split: one
// float4 chunk of one row per thread, splits summed in index order.
template <int D, class E>
__global__ __launch_bounds__(256) void ca_fwd_combine_kernel(const float* __restrict__ part,
                                                             float* __restrict__ O, View Ov,
                                                             float* __restrict__ stats, int BH,
                                                             int H, int T, int C, int smax) {
  constexpr int C4 = D / 4;
  const int tix = blockIdx.x * 256 + threadIdx.x;
  const int row = tix / C4, c = tix % C4;
  if (row >= BH * T) return;
  const int bh = row / T, i = row % T;
  const int g = i / 128;
  const int ntiles_all = (T + 31) / 32;
  const int nt = min(4 * g + 4, ntiles_all);
  const int ns = (nt + C - 1) / C;
  if (ns <= 1) return;
  const float* mz = part + (size_t)BH * smax * T * D;
  float M = kNegBig;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, mz[(((size_t)bh * smax + s) * T + i) * 2]);
  float Z = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < ns; ++s) {
    const size_t base = ((size_t)bh * smax + s) * T + i;
    const float f = fast_exp2(mz[base * 2] - M);
    Z = fmaf(mz[base * 2 + 1], f, Z);
    acc += reinterpret_cast<const f32x4*>(part + base * D)[c] * f;
  }
  const float invz = 1.0f / Z;
  reinterpret_cast<f32x4*>(O + (size_t)row * D)[c] = acc * invz;
  if (Ov.base) st4(view_slice<E>(Ov, bh, H) + (long long)i * Ov.rstride + 4 * c, acc * invz);
  if (c == 0) {
    stats[(size_t)row * 2 + 0] = M;
    stats[(size_t)row * 2 + 1] = invz;
  }
}

// Head dims that run the 16x16x32 forward (the 32x32x16 kernel serves the
// others).
template <int D>
constexpr bool fwd_uses_16x16() {
  return D == 64 || D == 128;
}

template <int D, class E>
hipError_t launch_fwd(const FwdIO& io, float* part, int B, int H, int T, int C,
                      hipStream_t stream) {
  const int BH = B * H;
  const int G = (T + 127) / 128;
  const int smax = fwd_max_splits(T, C);
  const int items = fwd_num_items(T, C);
  timer_begin(kFwd, stream);
  if constexpr (fwd_uses_16x16<D>()) {
    if (io.rope && !io.k_rotated)
      hipLaunchKernelGGL((ca_fwd16_kernel<D, E, true>), dim3(items * BH), dim3(512), 0, stream,
                         io.q, io.k, io.v, io.rope, io.log_gain, io.y, io.out, io.stats, part, BH, H,
                         T, C, G, smax);
    else
      hipLaunchKernelGGL((ca_fwd16_kernel<D, E, false>), dim3(items * BH), dim3(512), 0, stream,
                         io.q, io.k, io.v, io.rope, io.log_gain, io.y, io.out, io.stats, part, BH, H,
                         T, C, G, smax);
  } else {
    if (io.rope && !io.k_rotated)
      hipLaunchKernelGGL((ca_fwd_kernel<D, E, true>), dim3(items * BH), dim3(256), 0, stream, io.q,
                         io.k, io.v, io.rope, io.log_gain, io.y, io.out, io.stats, part, BH, H, T,
                         C, G, smax);
    else
      hipLaunchKernelGGL((ca_fwd_kernel<D, E, false>), dim3(items * BH), dim3(256), 0, stream, io.q,
                         io.k, io.v, io.rope, io.log_gain, io.y, io.out, io.stats, part, BH, H, T,
                         C, G, smax);
  }
  timer_end(kFwd, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (smax > 1) {
    const int rows = BH * T;
    timer_begin(kFwdCombine, stream);
    hipLaunchKernelGGL((ca_fwd_combine_kernel<D, E>), dim3((rows * (D / 4) + 255) / 256), dim3(256),
                       0, stream, part, io.y, io.out, io.stats, BH, H, T, C, smax);
    timer_end(kFwdCombine, stream);
    e = hipGetLastError();
  }
  return e;
}

// Keys rotated once for the kernels that read them many times: row t of
// slice bh of the key view, RoPE applied as the reference computes it in E
// (rope4_in), written to out[bh][t][D] in E.  One thread per 4 elements.
template <int D, class E>
__global__ __launch_bounds__(256) void ca_rope_keys_kernel(View Kv, const float* __restrict__ rope,
                                                           E* __restrict__ out, int BH, int H,
                                                           int T) {
  constexpr int C4 = D / 4;
  const long long tix = (long long)blockIdx.x * 256 + threadIdx.x;
  if (tix >= (long long)BH * T * C4) return;
  const int c = (int)(tix % C4);
  const long long row = tix / C4;
  const int bh = (int)(row / T), t = (int)(row % T);
  const E* src = view_slice<const E>(Kv, bh, H) + (long long)t * Kv.rstride + 4 * c;
  st4(out + row * D + 4 * c, rope4_in<E>(ld4(src), rope_entry(rope, t, D, 4 * c)));
}

template <int D, class E>
hipError_t launch_rope_keys(View k, const float* rope, void* out, int BH, int H, int T,
                            hipStream_t stream) {
  const long long n = (long long)BH * T * (D / 4);
  hipLaunchKernelGGL((ca_rope_keys_kernel<D, E>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     stream, k, rope, static_cast<E*>(out), BH, H, T);
  return hipGetLastError();
}

#define CA_INST_FWD(DD, EE)                                                                       \
  template hipError_t launch_fwd<DD, EE>(const FwdIO&, float*, int, int, int, int, hipStream_t);   \
  template hipError_t launch_rope_keys<DD, EE>(View, const float*, void*, int, int, int, hipStream_t);
#define CA_INST_FWD_ALL(EE) \
  CA_INST_FWD(8, EE) CA_INST_FWD(16, EE) CA_INST_FWD(32, EE) CA_INST_FWD(64, EE) CA_INST_FWD(128, EE)
CA_INST_FWD_ALL(float)
CA_INST_FWD_ALL(__bf16)
CA_INST_FWD_ALL(_Float16)

}  // namespace ca
