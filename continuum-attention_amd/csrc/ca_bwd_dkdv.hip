// dK and dV of the Continuum Attention backward (gfx950): the ca_bwd_dkdv
// kernel of the backward described in ca_bwd.hip, in a translation unit of
// its own so that it can be compiled with its own instruction-scheduling
// strategy (build.py: max-ilp here, measured 2% faster for this kernel and
// slower for the others).
//
// Score-tile layout: the 16x16 result of S / dP' puts slot j
// (key 14*kb - 1 + j) in lane j of each 16-lane row and queries 4*(l/16) + r
// in its registers, so the two neighbours of a segment sit in adjacent lanes
// of one DPP row (row_shr / row_shl).  p = 2^(s - m) stays unnormalised and
// dY arrives pre-scaled by 1/Z, so the weight gradient g = dY.v/Z - Dl/Z comes
// straight out of the MFMA (its accumulator starts at -Dl/Z) and dV = W^T dY
// is formed as w^T (dY/Z) with no per-row scaling in the kernel.
#include <type_traits>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

template <int D, int QL>
struct Bwd {
  static constexpr int C4 = D / 4;             // float4 chunks per row
  static constexpr int KB = (D + 31) / 32;     // 32-wide k blocks of S / dP'
  static constexpr int NMB = (D + 15) / 16;    // 16-row d blocks of dV^T / dK^T
  // bf16 row stride of a staged tile: 160-byte rows for D = 64 keep both the
  // 16-row row-wise reads and the transposed reads free of bank conflicts
  static constexpr int LDR = D + 16;
  static constexpr int LIMB = 32 * LDR;        // bf16 per limb plane of a tile
  static constexpr int PLANES = QL + 3;        // QL Q limbs (h[, m, l]), then dY/Z limbs h, m, l
  static constexpr int TILE = PLANES * LIMB;
  static constexpr int RCH = D / 8;            // 16-byte chunks per row and plane
  static constexpr int CHUNKS = PLANES * 32 * RCH;  // chunks staged per tile
  static constexpr int CPT = (CHUNKS + 255) / 256;
};

// Waves per SIMD the register budget is set for: bf16 operands need fewer
// limb registers and fit three (156 VGPRs at D = 64, 41 KB of LDS per work
// group), which hides more of the segment math's latency (one CA-S layer:
// 0.137 -> 0.132 ms); fp32 and fp16 operands keep two, except the
// single-buffered variant (SB): one staged tile (31 KB) and no register
// prefetch across the tile's work, three waves (168 VGPRs).  SB issues the
// next tile's loads when its own products are issued, waits at the barrier
// for the other waves, then stores: the load latency overlaps the barrier
// wait and the other resident work groups' work.  fp32 at D = 64 runs it on
// every grid (config 2 dK/dV 0.309 -> 0.291 ms, [1,16,2048,64] 0.162 ->
// 0.161 ms against the double-buffered two-wave kernel on one box).
// Direction of each item's walk over its query tiles (see the tile loop).
constexpr bool kDkdvDescending = true;

template <int D, class E, bool SB>
constexpr int dkdv_waves_per_simd() {
  return D > 64 ? 1 : (q_limb_planes<E>() == 1 || SB) ? 3 : 2;
}
// the single-buffered variant is built for fp32 operands at D = 64
template <int D, class E>
constexpr bool dkdv_has_single_buffer() {
  return D == 64 && std::is_same<E, float>::value;
}

template <int D, class E, bool SB>
__global__ __launch_bounds__(256, (dkdv_waves_per_simd<D, E, SB>())) void ca_bwd_dkdv_kernel(
    View Kv, View Vv, const float* __restrict__ rope, const float* __restrict__ rope_k,
    const __bf16* __restrict__ limbs,
    const float* __restrict__ qstat, const float* __restrict__ log_gain, View dKv, View dVv,
    float* __restrict__ dsbuf, float* __restrict__ kv_part, float* __restrict__ gain_part,
    BwdPass pass, int BH, int H, int T, int chunk, int n_items, int n_part, bool kv_f32) {
  // bf16 operands: Q, K (rotated and rounded as the reference rounds them)
  // and V are bf16-valued, so the tile carries Q's h limb alone and the
  // products with Q or V skip their zero limb products (limb_step_used), with
  // the same sums bit for bit; S is q.k of the h limbs, scaled after the
  // product.  Other operand types: K enters S scaled by the head's gain, in
  // three limbs.
  constexpr bool BF = q_limb_planes<E>() == 1;
  using P = Bwd<D, q_limb_planes<E>()>;
  constexpr int NBUF = SB ? 1 : 2;
  __shared__ __attribute__((aligned(16))) __bf16 tiles[NBUF][P::TILE];
  // per staged row: -m (tstat[b][0][row]) and -Dl/Z (tstat[b][1][row]), in
  // the order of the S / dP' accumulator registers
  __shared__ __attribute__((aligned(16))) float tstat[NBUF][2][32];

  const int nkb = bwd_num_key_blocks(T);
  const int bh = blockIdx.x % BH;
  const int item = blockIdx.x / BH;  // ascending: heaviest first
  // item -> (key-block group, chunk of its query tiles in this pass)
  int wg = item, ch = 0, nch = 1;
  if (chunk < pass.qb - pass.qa) {
    const int G = pass.kv_groups;
    wg = 0;
    ch = item;
    nch = dkdv_group_chunks(0, pass, chunk);
    while (ch >= nch && wg < G - 1) {
      ch -= nch;
      ++wg;
      nch = dkdv_group_chunks(wg, pass, chunk);
    }
  }
  const int w0 = kDkdvKeys * wg;

  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int lane = tid & 63;
  const int j = lane & 15;  // slot
  const int g = lane >> 4;  // k group / row group
  const int kb16 = kDkdvWaves * wg + wv;
  const int key_j = kBwdKeys * kb16 - 1 + j;  // key of this lane's slot
  const int kmin = kBwdKeys * kb16 - 1;        // key of slot 0

  const float cl2 = head_scale_log2(log_gain, bh % H, D);

  // Stale LDS bits must not reach an MFMA as NaN through padding columns.
  {
    unsigned* z = reinterpret_cast<unsigned*>(&tiles[0][0]);
    for (int e = tid; e < NBUF * P::TILE / 2; e += 256) z[e] = 0u;
  }

  // K (rotated here when `rope_k`; otherwise it arrives rotated, or without
  // RoPE; then scaled by c log2e, except bf16 operands, whose scores are
  // scaled after the product) and V of this lane's slot: B operands of S /
  // dP', k block kb, element e = d 32kb + 8g + e.
  Limbs kl[P::KB], vl[P::KB];
#pragma unroll
  for (int kb = 0; kb < P::KB; ++kb) {
    float xk[8], xv[8];
    const int d0 = 32 * kb + 8 * g;
    const bool ok = key_j >= 0 && key_j < T && d0 < D;
    const int krow = ok ? key_j : 0;
    const E* kp = view_slice<const E>(Kv, bh, H) + (long long)krow * Kv.rstride + (ok ? d0 : 0);
    const E* vp = view_slice<const E>(Vv, bh, H) + (long long)krow * Vv.rstride + (ok ? d0 : 0);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const bool ok2 = ok && d0 + 4 * h2 < D;
      f32x4 a = ok2 ? ld4(kp + 4 * h2) : f32x4{0.f, 0.f, 0.f, 0.f};
      if (rope_k && ok2) a = rope4_in<E>(a, rope_entry(rope_k, krow, D, d0 + 4 * h2));
      if (!BF) a *= cl2;
      const f32x4 b = ok2 ? ld4(vp + 4 * h2) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xk[4 * h2 + e] = a[e];
        xv[4 * h2 + e] = b[e];
      }
    }
    kl[kb] = split8(xk);
    vl[kb] = split8(xv);
  }

  f32x4 accv[P::NMB], acck[P::NMB];
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb) {
    accv[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    acck[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- query-tile staging (all waves), one tile ahead ----
  // Tile qt of the pass is one contiguous block of six limb planes [32][D]
  // (rows past T are zero) and 32 row statistics: thread tid copies 16-byte
  // chunks tid + 256u of the block, so the only per-tile address work is the
  // uniform block base.
  const int ntiles = bwd_pass_tiles(pass);
  constexpr unsigned kTileBytes = limb_tile_elems(D, P::PLANES) * sizeof(__bf16);
  const __amdgpu_buffer_rsrc_t lrs =
      buffer_rsrc(limbs + (size_t)bh * ntiles * limb_tile_elems(D, P::PLANES), ntiles * kTileBytes);
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(qstat + (size_t)bh * ntiles * 64, ntiles * 256u);
  u32x4 pre[P::CPT];
  u32x4 pre_st = {0u, 0u, 0u, 0u};
  auto load_tile = [&](int qt) {
    const unsigned t = qt - pass.qa;
#pragma unroll
    for (int u = 0; u < P::CPT; ++u) {
      const int e = tid + 256 * u;
      if (P::CHUNKS % 256 == 0 || e < P::CHUNKS)
        pre[u] = buffer_ld16(lrs, 16u * tid, t * kTileBytes + 4096u * u);
    }
    if (tid < 16) pre_st = buffer_ld16(srs, 16u * tid, t * 256u);
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < P::CPT; ++u) {
      const int e = tid + 256 * u;
      if (P::CHUNKS % 256 == 0 || e < P::CHUNKS) {
        const int pl = e / (32 * P::RCH), rem = e % (32 * P::RCH);
        const int row = rem / P::RCH, ch = rem % P::RCH;
        *reinterpret_cast<u32x4*>(&tiles[buf][pl * P::LIMB + row * P::LDR + 8 * ch]) = pre[u];
      }
    }
    if (tid < 16) {
      *reinterpret_cast<u32x2*>(&tstat[buf][0][2 * tid]) = u32x2{pre_st[0], pre_st[2]};
      *reinterpret_cast<u32x2*>(&tstat[buf][1][2 * tid]) = u32x2{pre_st[1], pre_st[3]};
    }
  };

  // query tiles of this item: a chunk of the pass's tiles that see an owned
  // key of the work group, walked from the last down (kDkdvDescending): the
  // work groups of a slice that are resident together then all start at the
  // pass's last tile and read each query tile at about the same time, so it
  // is fetched once into the XCD's L2 and re-read from there (walked upwards,
  // key group wg starts at tile 1.75 wg and the resident groups read tiles
  // up to ~40 apart)
  const int ntl = dkdv_group_tiles(wg, pass);
  const int clen = (ntl + nch - 1) / nch;
  const int qt0 = dkdv_group_first_tile(wg, pass) + ch * clen;
  const int qt_end = min(qt0 + clen, pass.qb);
  const int ntile = qt_end > qt0 ? qt_end - qt0 : 0;
  constexpr int kStep = kDkdvDescending ? -1 : 1;
  const int qt_first = kDkdvDescending ? qt_end - 1 : qt0;
  // this lane's spilled dS column in tile qt: owned slots 1 .. 14 hold keys
  // 14 kb16 .. +13; tile qt's columns start at ds_tile, moved per tile
  size_t ds_tile = (size_t)bh * pass.ds_slice + (ds_floats_before(qt_first) - pass.ds0);
  const int ds_key = kBwdKeys * kb16 + j - 1;
  const bool ds_lane = j >= 1 && j <= kBwdKeys;
  __syncthreads();          // LDS clear before the first store
  if (ntile > 0) {
    load_tile(qt_first);
    store_tile(0);
  }
  __syncthreads();

  for (int n = 0; n < ntile; ++n) {
    const int qt = qt_first + kStep * n;
    const bool more = n + 1 < ntile;
    const int buf = SB ? 0 : n & 1;
    if (!SB && more) load_tile(qt + kStep);
    const int i0 = 32 * qt;
    // the wave's block meets this tile (and exists)
    const bool work = kb16 < nkb && kBwdKeys * kb16 <= i0 + 31;
    if (work) {
      const __bf16* Tq = &tiles[buf][0];
      const __bf16* Ty = &tiles[buf][(P::PLANES - 3) * P::LIMB];

      // ---- S - m and dP' - Dl/Z (row blocks rb: queries i0 + 16rb + 4g + r) ----
      // bf16 operands: S accumulates q.k from zero (Q and K bf16-valued: the
      // h limb product alone) and takes c log2e and -m in one fused
      // multiply-add; otherwise K carries c log2e and the accumulator starts
      // from -m.
      f32x4 sacc[2], pacc[2], negm[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        negm[rb] = *reinterpret_cast<const f32x4*>(&tstat[buf][0][16 * rb + 4 * g]);
        sacc[rb] = BF ? f32x4{0.f, 0.f, 0.f, 0.f} : negm[rb];
        pacc[rb] = *reinterpret_cast<const f32x4*>(&tstat[buf][1][16 * rb + 4 * g]);
      }
      prio_mfma_begin<!BF>();
#pragma unroll
      for (int kb = 0; kb < P::KB; ++kb) {
        const int col = 32 * kb + 8 * g;
        Limbs qa[2], ya[2];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          qa[rb] = ya[rb] = Limbs{bf16x8{}, bf16x8{}, bf16x8{}};
          if (col < D) {
            const int o = (16 * rb + j) * P::LDR + col;
            qa[rb].h = *reinterpret_cast<const bf16x8*>(Tq + o);
            if (!BF) {
              qa[rb].m = *reinterpret_cast<const bf16x8*>(Tq + P::LIMB + o);
              qa[rb].l = *reinterpret_cast<const bf16x8*>(Tq + 2 * P::LIMB + o);
            }
            ya[rb].h = *reinterpret_cast<const bf16x8*>(Ty + o);
            ya[rb].m = *reinterpret_cast<const bf16x8*>(Ty + P::LIMB + o);
            ya[rb].l = *reinterpret_cast<const bf16x8*>(Ty + 2 * P::LIMB + o);
          }
        }
        // four independent accumulators per limb product
#pragma unroll
        for (int st = 0; st < 6; ++st) {
          if (limb_step_used<BF, BF>(st)) sacc[0] = mfma16_step(st, qa[0], kl[kb], sacc[0]);
          if (limb_step_used<false, BF>(st)) pacc[0] = mfma16_step(st, ya[0], vl[kb], pacc[0]);
          if (limb_step_used<BF, BF>(st)) sacc[1] = mfma16_step(st, qa[1], kl[kb], sacc[1]);
          if (limb_step_used<false, BF>(st)) pacc[1] = mfma16_step(st, ya[1], vl[kb], pacc[1]);
        }
      }
      prio_mfma_end<!BF>();
      if (BF) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int r = 0; r < 4; ++r) sacc[rb][r] = fmaf(sacc[rb][r], cl2, negm[rb][r]);
      }

      // ---- segments along the slots (adjacent lanes of each DPP row) ----
      // Tiles where every slot key is visible to every query, with no key 0
      // and no row past T, take the fast path; the cap of key i can then only
      // fall on slot 15, which is not owned.
      const bool need_mask = (kmin < 1) || (kmin + 15 > i0) || (i0 + 31 >= T);
      float wout[2][4], dout_s[2][4];
      auto segments = [&](auto general_tag) {
        constexpr bool kGeneral = decltype(general_tag)::value;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = i0 + 16 * rb + 4 * g + r;
            const bool vis = !kGeneral || (key_j >= 0 && key_j <= i && i < T);
            const float s = vis ? sacc[rb][r] : 0.f;   // s - m
            const float gg = vis ? pacc[rb][r] : 0.f;  // g = dY.v/Z - Dl/Z
            const float p = fast_exp2(s);
            const float sl = row_shr1(s), pl = row_shr1(p), gl = row_shr1(gg);
            float Lv, Rv, dLv, dRv;
            seg_shares_grad(sl, s, pl, p, gl, gg, Lv, Rv, dLv, dRv);
            // Segment (slot j-1, slot j), both keys visible.  Lane 0 has no
            // left neighbour: its right shares land on slot 0, which is not
            // owned, and its left shares are read by no lane (row_shl reads
            // lane j+1), so only the general path needs the mask.
            if (kGeneral) {
              const bool ok = j >= 1 && key_j >= 1 && key_j <= i && i < T;
              Lv = ok ? Lv : 0.f;
              Rv = ok ? Rv : 0.f;
              dLv = ok ? dLv : 0.f;
              dRv = ok ? dRv : 0.f;
            }
            // left shares of segment (j, j+1) arrive from lane j+1
            float w = Rv + row_shl1(Lv);
            float ds = dRv + row_shl1(dLv);
            if (kGeneral) {
              // half-token caps on the first key and the last visible key
              const float cap = (vis && key_j == 0 ? 0.5f * p : 0.f) + (vis && key_j == i ? 0.5f * p : 0.f);
              w += cap;
              ds = fmaf(cap, gg, ds);
            }
            // Slots 0 and 15 are not owned: their w and dS only reach dV / dK
            // columns that are never stored, and they are not spilled.
            wout[rb][r] = w;
            dout_s[rb][r] = ds;
          }
        }
      };
      if (need_mask)
        segments(std::true_type{});
      else
        segments(std::false_type{});

      // ---- dS of (query tile qt, the block's keys) for the dQ pass ----
      if (ds_lane) {
        float* col = dsbuf + ds_tile + (size_t)ds_key * kDsColFloats + 4 * g;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          *reinterpret_cast<f32x4*>(col + 16 * rb) =
              f32x4{dout_s[rb][0], dout_s[rb][1], dout_s[rb][2], dout_s[rb][3]};
      }

      // ---- dV^T += (dY/Z)^T w and dK^T += Q^T dS ----
      // k element e of group g <-> query (e < 4 ? 4g + e : 16 + 4g + e - 4),
      // i.e. register (rb = e / 4, r = e % 4) of this lane.
      float xw[8], xd[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xw[e] = wout[e >> 2][e & 3];
        xd[e] = dout_s[e >> 2][e & 3];
      }
      const Limbs wb = split8(xw), db = split8(xd);
      prio_mfma_begin<!BF>();
      const int src_row = 4 * g + (j >> 2), src_col = 4 * (j & 3);
#pragma unroll
      for (int mb = 0; mb < P::NMB; ++mb) {
        const int o0 = src_row * P::LDR + 16 * mb + src_col;
        const int o1 = o0 + 16 * P::LDR;
        Limbs ya, qa;
        ya.h = lds_read_tr8(Ty + o0, Ty + o1);
        ya.m = lds_read_tr8(Ty + P::LIMB + o0, Ty + P::LIMB + o1);
        ya.l = lds_read_tr8(Ty + 2 * P::LIMB + o0, Ty + 2 * P::LIMB + o1);
        qa.h = lds_read_tr8(Tq + o0, Tq + o1);
        if (BF) {
          qa.m = qa.l = bf16x8{};
        } else {
          qa.m = lds_read_tr8(Tq + P::LIMB + o0, Tq + P::LIMB + o1);
          qa.l = lds_read_tr8(Tq + 2 * P::LIMB + o0, Tq + 2 * P::LIMB + o1);
        }
#pragma unroll
        for (int st = 0; st < 6; ++st) {
          accv[mb] = mfma16_step(st, ya, wb, accv[mb]);
          if (limb_step_used<BF, false>(st)) acck[mb] = mfma16_step(st, qa, db, acck[mb]);
        }
      }
      prio_mfma_end<!BF>();
    }
    if (more) {
      if (kDkdvDescending)
        ds_tile -= (size_t)kDsColFloats * kBwdKeys * ds_kb_count(qt - 1);
      else
        ds_tile += (size_t)kDsColFloats * kBwdKeys * ds_kb_count(qt);
    }
    if (SB) {
      if (more) {
        load_tile(qt + kStep);  // issued before the barrier: its latency overlaps the wait
        __syncthreads();  // every wave is done with the tile
        store_tile(0);
      }
    } else if (more) {
      store_tile(buf ^ 1);
    }
    __syncthreads();
  }

  // ---- epilogue: lane (slot j, group g) holds d = 16mb + 4g + r of its key ----
  // A single-chunk group writes dK/dV; the chunks of a longer group write
  // partials [key of the group][dV, dK][D] that ca_bwd_merge sums.
  // Each item also writes its part of the gain gradient
  //   dlog_gain = sum_ij dS_ij s_ij = sum_j k_j . dK_j = sum_j (k_j - k_0) . dK_j
  // (the last because sum_j dK_j = c sum_i q_i sum_j dS_ij = 0: every row of
  // dS sums to zero), with k_0 the slice's first key: near-duplicate keys
  // then contribute small differences instead of cancelling terms.
  float gsum = 0.f;
  const bool owned_key = j >= 1 && j <= kBwdKeys && key_j < T && kb16 < nkb;
  if (owned_key) {
    const float ck = cl2 * kLn2;
    const E* k0 = view_slice<const E>(Kv, bh, H);
    const E* kj = k0 + (long long)key_j * Kv.rstride;
#pragma unroll
    for (int mb = 0; mb < P::NMB; ++mb) {
      const int d0 = 16 * mb + 4 * g;
      if (d0 < D) {
        f32x4 a = ld4(kj + d0), b = ld4(k0 + d0);
        if (rope_k) {
          a = rope4_in<E>(a, rope_entry(rope_k, key_j, D, d0));
          b = rope4_in<E>(b, rope_entry(rope_k, 0, D, d0));
        }
        const f32x4 dk = acck[mb] * ck;
#pragma unroll
        for (int r = 0; r < 4; ++r) gsum = fmaf(a[r] - b[r], dk[r], gsum);
      }
    }
  }
  {
    __shared__ float gred[kDkdvWaves];
    gsum = wave_sum(gsum);
    if (lane == 0) gred[wv] = gsum;
    __syncthreads();
    if (tid == 0) gain_part[(size_t)bh * n_items + item] = (gred[0] + gred[1]) + (gred[2] + gred[3]);
  }
  if (owned_key) {
    const float ck = cl2 * kLn2;
    if (nch == 1) {
      // dK rotated back by the transposed RoPE (the gradient of the un-rotated
      // k); added to what earlier passes wrote for this key group (in E, or
      // in fp32 sums when kv_f32)
      const bool accumulate = dkdv_qt0(wg) < pass.qa;
      auto write = [&](auto* pv, auto* pk) {
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb) {
          const int d0 = 16 * mb + 4 * g;
          if (d0 < D) {
            f32x4 gv = accv[mb];
            f32x4 gk = acck[mb] * ck;
            if (rope) gk = rope4(gk, rope_entry(rope, key_j, D, d0), true);
            if (accumulate) {
              gv += ld4(pv + d0);
              gk += ld4(pk + d0);
            }
            st4(pv + d0, gv);
            st4(pk + d0, gk);
          }
        }
      };
      if (std::is_same<E, float>::value || kv_f32)
        write(view_slice<float>(dVv, bh, H) + (long long)key_j * dVv.rstride,
              view_slice<float>(dKv, bh, H) + (long long)key_j * dKv.rstride);
      else
        write(view_slice<E>(dVv, bh, H) + (long long)key_j * dVv.rstride,
              view_slice<E>(dKv, bh, H) + (long long)key_j * dKv.rstride);
    } else {
      float* pv = kv_part + (((size_t)bh * n_part + item) * kDkdvKeys + (key_j - w0)) * 2 * D;
      float* pk = pv + D;
#pragma unroll
      for (int mb = 0; mb < P::NMB; ++mb) {
        const int d0 = 16 * mb + 4 * g;
        if (d0 < D) {
          *reinterpret_cast<f32x4*>(pv + d0) = accv[mb];
          *reinterpret_cast<f32x4*>(pk + d0) = acck[mb] * ck;
        }
      }
    }
  }
}

template <int D, class E>
hipError_t launch_bwd_dkdv(const BwdIO& io, const BwdWork& ws, const BwdPass& pass,
                           const DkdvSplit& kvs, int BH, int H, int T, hipStream_t stream) {
  // the single-buffered variant wherever it is built
  auto kernel = ca_bwd_dkdv_kernel<D, E, dkdv_has_single_buffer<D, E>()>;
  hipLaunchKernelGGL(kernel, dim3(kvs.items * BH), dim3(256), 0, stream, io.k,
                     io.v, io.rope, io.k_rotated ? nullptr : io.rope, ws.limbs, ws.qstat,
                     io.log_gain, io.dk, io.dv, ws.dsbuf,
                     ws.kv_part, ws.gain_part, pass, BH, H, T, kvs.chunk, kvs.items,
                     kvs.part_items, io.kv_f32);
  return hipGetLastError();
}

#define CA_INSTANTIATE_DKDV(DD, EE)                                                          \
  template hipError_t launch_bwd_dkdv<DD, EE>(const BwdIO&, const BwdWork&, const BwdPass&,   \
                                              const DkdvSplit&, int, int, int, hipStream_t);
#define CA_INSTANTIATE_DKDV_ALL(EE)                                                          \
  CA_INSTANTIATE_DKDV(8, EE) CA_INSTANTIATE_DKDV(16, EE) CA_INSTANTIATE_DKDV(32, EE)         \
  CA_INSTANTIATE_DKDV(64, EE) CA_INSTANTIATE_DKDV(128, EE)
CA_INSTANTIATE_DKDV_ALL(float)
CA_INSTANTIATE_DKDV_ALL(__bf16)
CA_INSTANTIATE_DKDV_ALL(_Float16)
#undef CA_INSTANTIATE_DKDV
#undef CA_INSTANTIATE_DKDV_ALL

}  // namespace ca
