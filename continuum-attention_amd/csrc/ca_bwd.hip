// Continuum Attention backward (gfx950), analytic first-order VJP.
//
// Replaces the per-query-tile loop of _CAExactTiled.backward
// (cuda/continuum_attention.py:697-766): the QK^T and dY.V^T recomputation,
// the fused score-VJP kernels (ca_backward_fused_kernel /
// ca_backward_half_kernel, cuda/continuum_attention.py:230-293,337-405) and
// the dV/dQ/dK/dRho contractions.
//
// Kernels (all deterministic, no atomics):
//   ca_bwd_prep     per query row: Dl_i = dY_i . y_i (the reference forms the
//                   same row mean at cuda/continuum_attention.py:268-269),
//                   Q_i and dY_i / Z_i split into bf16 limb planes, and
//                   (-m_i, -Dl_i / Z_i).
//   ca_bwd_dkdv     (ca_bwd_dkdv.hip) one work group per (slice, 56 keys); wave w owns 14 keys
//                   (16 MFMA slots).  The 4 waves walk the query tiles
//                   together: each 32-query tile of Q and dY/Z limbs is staged
//                   once in LDS (double-buffered) and read by every wave both
//                   row-wise (S = Q K^T, dP' = (dY/Z) V^T) and transposed
//                   (dV^T += (dY/Z)^T W, dK^T += Q^T dS) with
//                   ds_read_b64_tr_b16.  K and V of the wave's slots stay in
//                   registers as bf16 limbs for the whole launch.  All four
//                   products are bf16x6 on v_mfma_f32_16x16x32_bf16.  dS of
//                   the owned keys is also spilled, one 32-query column per
//                   (query tile, key), for the dQ pass.
//                   Each item also forms its gain partial
//                   sum_j (k_j - k_0) . dK_j (= sum_ij dS_ij s_ij, since
//                   s_ij = c q_i . k_j and every row of dS sums to zero).
//   ca_bwd_dq       dQ = c dS (K - k_ref) over the spilled rows, one work
//                   item per (slice, 128 queries, chunk of 32-key stages); H
//                   extra work groups sum the gain partials into dRho_h, and
//                   one more per split dK/dV key group sums its chunk partials.
//   ca_bwd_merge    sums the dQ chunk partials of split groups (launched only
//                   when a split leaves some).
//
// Score-tile layout in ca_bwd_dkdv: the 16x16 result of S / dP' puts slot j
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


// One thread per (row of the pass's query tiles, 8 elements): Dl = dY . y,
// then the Q and dY/Z limbs of the 8 elements (one 16-byte store per plane)
// and, per row, (-m, -Dl/Z).  The limb planes are tile-major: tile j of the
// pass in slice bh is the block limbs[(bh * ntiles + j) * P * 32 * D ..] of
// P planes [32 rows][D] (P = q_limb_planes<E>() + 3).  Rows past T (in the
// last tile) are written as zeros, so the dK/dV kernel stages whole tiles
// without bounds tests.
template <int D, class E>
__global__ __launch_bounds__(256) void ca_bwd_prep_kernel(View Qv, const float* __restrict__ rope,
                                                          View dYv,
                                                          const float* __restrict__ out,
                                                          const float* __restrict__ stats,
                                                          __bf16* __restrict__ limbs,
                                                          float* __restrict__ qstat, int H, int T,
                                                          int row0, int ntiles, int rows) {
  constexpr int C8 = D / 8;
  const int tix = blockIdx.x * 256 + threadIdx.x;
  const int row = tix / C8, c = tix % C8;  // row = bh * 32 ntiles + (t - row0)
  if (row >= rows) return;
  const int prows = 32 * ntiles;
  const int bh = row / prows, r = row % prows, t = row0 + r;
  const bool ok = t < T;
  const size_t grow = (size_t)bh * T + (ok ? t : 0);  // row of y and stats
  const E* qp = view_slice<const E>(Qv, bh, H) + (long long)(ok ? t : 0) * Qv.rstride + 8 * c;
  const E* dp = view_slice<const E>(dYv, bh, H) + (long long)(ok ? t : 0) * dYv.rstride + 8 * c;
  f32x4 dy[2], y[2], qq[2];
  float m = 0.f, invz = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    dy[u] = y[u] = qq[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (ok) {
      dy[u] = ld4(dp + 4 * u);
      y[u] = reinterpret_cast<const f32x4*>(out + grow * D + 8 * c)[u];
      qq[u] = ld4(qp + 4 * u);
      if (rope) qq[u] = rope4_in<E>(qq[u], rope_entry(rope, t, D, 8 * c + 4 * u));
    }
  }
  if (ok) {
    m = stats[grow * 2 + 0];
    invz = stats[grow * 2 + 1];
  }
  float x = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u)
    x += dy[u][0] * y[u][0] + dy[u][1] * y[u][1] + dy[u][2] * y[u][2] + dy[u][3] * y[u][3];
#pragma unroll
  for (int o = C8 / 2; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  constexpr int QL = q_limb_planes<E>();
  __bf16* tile = limbs + ((size_t)bh * ntiles + r / 32) * limb_tile_elems(D, QL + 3) +
                 (r % 32) * D + 8 * c;
  auto put = [&](int p0, int nl, const f32x4* v, float scale) {
    float e[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) e[u] = v[u >> 2][u & 3] * scale;
    const Limbs lb = split8(e);
    *reinterpret_cast<bf16x8*>(tile + (p0 + 0) * 32 * D) = lb.h;
    if (nl > 1) {
      *reinterpret_cast<bf16x8*>(tile + (p0 + 1) * 32 * D) = lb.m;
      *reinterpret_cast<bf16x8*>(tile + (p0 + 2) * 32 * D) = lb.l;
    }
  };
  put(0, QL, qq, 1.0f);  // bf16 operands: Q is bf16-valued, its h limb is exact
  put(QL, 3, dy, invz);
  if (c == 0) {
    // negated: the dK/dV kernel starts its S and dP' accumulators from them
    qstat[(size_t)row * 2 + 0] = -m;
    qstat[(size_t)row * 2 + 1] = -(x * invz);
  }
}

// dQ = c dS (K - k_ref) over the dS columns spilled by ca_bwd_dkdv, as bf16x6
// products on v_mfma_f32_16x16x32_bf16 (k = one stage of 32 consecutive
// keys).  Work item: one chunk of the key stages of a 128-query group (four
// 32-query tiles, one per wave) of one slice; the wave of tile qt takes the
// chunk's stages up to qt.  Per stage the 32 K rows are staged in LDS
// (double-buffered) as row-major bf16 limb planes [key][d], relative to
// k_ref, and shared by the four waves.  A operand: lane (query 16rb + l%16,
// group g) holds dS of keys 8g .. 8g+7 of the stage (gathered from their
// spilled key columns), split into limbs in registers;
// B operand: lane (d = 16nb + l%16, g) gets the same 8 keys of column d
// through two transposed reads.  Invisible keys carry dS = 0 in the spill and keys past T
// are zeroed at load, so no other masks are needed.  A single-chunk group
// writes dQ; the chunks of a longer group write partial tiles that
// ca_bwd_merge sums.
// Gain gradient: dlog_gain[h] = the fixed-order sum over batch and dK/dV
// items of the partials the dK/dV kernel wrote (added to the earlier passes'
// sum after the first pass).  Launched as H extra work groups of the dQ grid
// (after the dQ items, followed by the dK/dV partial merges).
__device__ __forceinline__ void gain_sum(const float* __restrict__ gain_part,
                                         float* __restrict__ dlog_gain, int h, int B, int H,
                                         int n_kv_items, bool first) {
  __shared__ float wsum[4];
  const int tid = threadIdx.x;
  float acc = 0.f;
  for (int b = 0; b < B; ++b)
    for (int k = tid; k < n_kv_items; k += 256) acc += gain_part[((size_t)b * H + h) * n_kv_items + k];
  acc = wave_sum(acc);
  if ((tid & 63) == 0) wsum[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    const float part_sum = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    dlog_gain[h] = first ? part_sum : dlog_gain[h] + part_sum;
  }
}

// Sum of the dK/dV chunk partials of multi-chunk key group wg of slice bh,
// in chunk order (dK rotated back when RoPE is on), written to dK and dV or,
// when an earlier pass already wrote this key group, added to them.  Run by
// extra work groups of the dQ launch, which follows the dK/dV launch that
// wrote the partials.
// Work groups per merged group in the two merges below: one float4 of the
// group's partial tiles per thread (the groups are few, so a work group per
// group left most of the GPU idle: one CA-S layer's dQ merge 14 -> 8 us).
template <int D>
constexpr int kv_merge_slices() { return (kDkdvKeys * 2 * (D / 4) + 255) / 256; }
template <int D>
constexpr int dq_merge_slices() { return (kDqRows * (D / 4) + 255) / 256; }

template <int D, class E>
__device__ __forceinline__ void merge_kv_group(const float* __restrict__ kv_part,
                                               const float* __restrict__ rope, const View& dKv,
                                               const View& dVv, const BwdPass& pass, int bh,
                                               int wg, int slice, int H, int T, int kv_chunk,
                                               int kv_part_items, bool kv_f32) {
  constexpr int C4 = D / 4;
  const int tid = threadIdx.x + 256 * slice;
  int first = 0;  // item index of the group's chunk 0 (multi-chunk groups come first)
  for (int gg = 0; gg < wg; ++gg) first += dkdv_group_chunks(gg, pass, kv_chunk);
  const int nch = dkdv_group_chunks(wg, pass, kv_chunk);
  const bool accumulate = dkdv_qt0(wg) < pass.qa;
  const f32x4* part = reinterpret_cast<const f32x4*>(
      kv_part + ((size_t)bh * kv_part_items + first) * kDkdvKeys * 2 * D);
  const int w0 = kDkdvKeys * wg;
  for (int e = tid; e < kDkdvKeys * 2 * C4; e += 256 * kv_merge_slices<D>()) {
    const int kl = e / (2 * C4), which = (e / C4) % 2, c4 = e % C4;
    const int key = w0 + kl;
    if (key >= T) break;
    f32x4 s = part[e];
    for (int cc = 1; cc < nch; ++cc) s += part[(size_t)cc * kDkdvKeys * 2 * C4 + e];
    const View& ov = which ? dKv : dVv;
    if (which && rope) s = rope4(s, rope_entry(rope, key, D, 4 * c4), true);
    auto write = [&](auto* dst) {
      if (accumulate) s += ld4(dst);
      st4(dst, s);
    };
    if (std::is_same<E, float>::value || kv_f32)
      write(view_slice<float>(ov, bh, H) + (long long)key * ov.rstride + 4 * c4);
    else
      write(view_slice<E>(ov, bh, H) + (long long)key * ov.rstride + 4 * c4);
  }
}

template <int D>
struct DqP {
  static constexpr int NB = (D + 15) / 16;            // 16-column d blocks of dQ
  static constexpr int C4 = D / 4;
  static constexpr int UNITS = 32 * C4;               // (key of the stage, float4) per stage
  static constexpr int UPT = (UNITS + 255) / 256;
  static constexpr int LDK = NB * 16 + 16;            // bf16 row stride (160 bytes for D = 64)
  static constexpr int PLANE = 32 * LDK;              // bf16 per limb plane of a stage
  static constexpr int STAGE = 3 * PLANE;
};

// bf16 operands (the h plane of K alone) are held to four waves per SIMD
template <int D, class E, bool ROPE>
__global__ __launch_bounds__(256, (std::is_same<E, __bf16>::value && D <= 64 ? 4 : 1)) void ca_bwd_dq_kernel(const float* __restrict__ dsbuf,
                                                        View Kv, const float* __restrict__ rope,
                                                        const float* __restrict__ log_gain,
                                                        View dQv, float* __restrict__ dq_part,
                                                        const float* __restrict__ gain_part,
                                                        float* __restrict__ dlog_gain, BwdPass pass,
                                                        int B, int H, int T, int chunk,
                                                        int n_items, int n_part, int n_kv_items,
                                                        const float* __restrict__ kv_part,
                                                        View dKv, View dVv, int kv_chunk,
                                                        int kv_part_items, bool kv_f32) {
  using P = DqP<D>;
  const int BH = B * H;
  if ((int)blockIdx.x >= n_items * BH) {
    const int x = blockIdx.x - n_items * BH;
    if (x < H)  // the H gain work groups
      gain_sum(gain_part, dlog_gain, x, B, H, n_kv_items, pass.first);
    else {      // then kv_merge_slices per (multi-chunk dK/dV key group, slice)
      const int y = (x - H) / kv_merge_slices<D>(), sl = (x - H) % kv_merge_slices<D>();
      merge_kv_group<D, E>(kv_part, rope, dKv, dVv, pass, y % BH, y / BH, sl, H, T, kv_chunk,
                           kv_part_items, kv_f32);
    }
    return;
  }
  __shared__ __attribute__((aligned(16))) __bf16 kst[2 * P::STAGE];
  const int nqt = num_q_tiles(T);
  const int bh = blockIdx.x % BH;
  // Items are dispatched lightest first (the reverse of their numbering):
  // the dK/dV kernel walks its query tiles downwards, so the dS columns of
  // the low query tiles are the ones it wrote last and most likely still
  // in cache (config 2 dQ 0.082 -> 0.076 ms against heaviest first; the
  // split chunks keep the grid balanced either way).
  const int item = n_items - 1 - (int)blockIdx.x / BH;
  // item -> (group, chunk), heaviest groups of the pass first
  int qg = pass.g1 - 1, ch = item, nch = dq_group_chunks(qg, T, chunk);
  while (ch >= nch && qg > pass.g0) {
    ch -= nch;
    --qg;
    nch = dq_group_chunks(qg, T, chunk);
  }
  const int gstages = dq_group_stages(qg, T);
  const int clen = (gstages + nch - 1) / nch;
  const int st_lo = ch * clen;
  const int st_hi = min(st_lo + clen, gstages);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int qt = kDqTiles * qg + w;
  const bool wave_on = qt < nqt;
  const float c = head_scale_log2(log_gain, bh % H, D) * kLn2;
  // stages of this chunk met by the wave's tile (stage s holds keys 32s .. 32s+31)
  const int my_end = wave_on ? min(qt + 1, st_hi) : 0;
  const int iters = st_hi > st_lo ? st_hi - st_lo : 0;
  // dS of this lane: rows 16rb + l16 of the wave's tile, keys 32s + 8g .. +7
  // (one dword of each key's column)
  const float* arow = dsbuf + (size_t)bh * pass.ds_slice +
                      (ds_floats_before(wave_on ? qt : pass.qa) - pass.ds0) + l16;

  f32x4 acc[2][P::NB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int nb = 0; nb < P::NB; ++nb) acc[rb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Every row of dS sums to zero (the weights are invariant to a common score
  // shift), so dQ_i = c sum_j dS_ij (k_j - k_ref) for any k_ref.  The staged
  // keys are taken relative to the key at the group's first query: when
  // neighbouring keys nearly coincide the products stay small instead of
  // cancelling (|k| ~ 1 against |k_j - k_ref| ~ 1e-2 in the near-duplicate-key
  // case).  All chunks of a group use the same k_ref, so the k_ref terms
  // cancel in the sum of the chunk partials.
  // Staging unit u: slot (key of the stage) u / C4, d = 4(u % C4)..+3; a
  // thread's units all have d chunk tid % C4, since 256 % C4 == 0.
  // rows of K (rotated here when ROPE; otherwise they arrive rotated, or
  // without RoPE): loaded raw a stage ahead and converted, rotated and
  // shifted when stored.  dQ is rotated back whenever `rope` is given.
  const float* __restrict__ rope_k = ROPE ? rope : nullptr;  // drops every key rotation
  const E* __restrict__ Ks = view_slice<const E>(Kv, bh, H);
  const long long krs = Kv.rstride;
  auto k_row4 = [&](int key, int d0) {
    f32x4 x = ld4(Ks + (long long)key * krs + d0);
    return rope_k ? rope4_in<E>(x, rope_entry(rope_k, key, D, d0)) : x;
  };
  typedef typename Raw4<E>::type R4;
  R4 pre[P::UPT];
  f32x4 pre_cs[ROPE ? P::UPT : 1];
  // bf16 operands: the keys are bf16-valued, and so are the stage's rows
  // without the k_ref shift: they are staged as their h plane alone, each
  // dS limb times k is exact in fp32, and the products with the zero m and l
  // limbs are skipped (the shift, which keeps near-coinciding keys' products
  // small, matters at fp32 key spacings; bf16 keys differ by at least 2^-8
  // of their size, so the unshifted sum loses at most 2^-16 of it)
  constexpr bool BF = std::is_same<E, __bf16>::value;
  const f32x4 kref = BF ? f32x4{0.f, 0.f, 0.f, 0.f} : k_row4(kDqRows * qg, 4 * (tid % P::C4));
  // K rows (and RoPE table rows) through buffer resources: a stage's offsets
  // are the thread's fixed offsets plus one uniform step per stage, and rows
  // at or past T read as zeros.  Those rows become -k_ref after the shift and
  // meet dS = 0 (keys past T carry no dS), so they add exactly nothing.
  constexpr unsigned kEsz = sizeof(E);
  const __amdgpu_buffer_rsrc_t kres = buffer_rsrc(Ks, (unsigned)view_rows_bytes(T, krs, D, kEsz));
  const __amdgpu_buffer_rsrc_t cres =
      buffer_rsrc(ROPE ? rope_k : log_gain, ROPE ? (unsigned)(T * D * sizeof(float)) : 0u);
  const unsigned kstep = 32u * (unsigned)krs * kEsz;
  unsigned koff[P::UPT], csoff[P::UPT];
#pragma unroll
  for (int uu = 0; uu < P::UPT; ++uu) {
    const int u = tid + 256 * uu;
    const unsigned row = 32u * st_lo + u / P::C4, c = u % P::C4;  // key of stage 0
    koff[uu] = (row * (unsigned)krs + 4 * c) * kEsz;
    csoff[uu] = (row * D + 4 * c) * (unsigned)sizeof(float);
  }
  auto load_k = [&](int it) {
#pragma unroll
    for (int uu = 0; uu < P::UPT; ++uu) {
      const int u = tid + 256 * uu;
      if (P::UNITS % 256 == 0 || u < P::UNITS) {
        pre[uu] = buffer_ld_raw4(kres, koff[uu] + it * kstep, Ks);
        if constexpr (ROPE)
          pre_cs[uu] = __builtin_bit_cast(f32x4, buffer_ld16(cres, csoff[uu] + it * (32u * D * 4u), 0));
      }
    }
  };
  // The shift is applied when the prefetched rows are stored, so the loads
  // issued a stage ahead are not waited for inside the MFMA loop.
  auto store_k = [&](int buf) {
#pragma unroll
    for (int uu = 0; uu < P::UPT; ++uu) {
      const int u = tid + 256 * uu;
      if (P::UNITS % 256 == 0 || u < P::UNITS) {
        f32x4 kx = raw_to_f32(pre[uu], Ks);
        if constexpr (ROPE) kx = rope4_in<E>(kx, pre_cs[uu]);
        const int off = buf * P::STAGE + (u / P::C4) * P::LDK + 4 * (u % P::C4);
        if constexpr (BF) {
          *reinterpret_cast<u32x2*>(&kst[off]) =
              u32x2{cvt_pk_bf16(kx[0], kx[1]), cvt_pk_bf16(kx[2], kx[3])};
        } else {
          const f32x4 kv = kx - kref;
          unsigned h0, m0, l0, h1, m1, l1;
          split_pair(kv[0], kv[1], h0, m0, l0);
          split_pair(kv[2], kv[3], h1, m1, l1);
          *reinterpret_cast<u32x2*>(&kst[off]) = u32x2{h0, h1};
          *reinterpret_cast<u32x2*>(&kst[off + P::PLANE]) = u32x2{m0, m1};
          *reinterpret_cast<u32x2*>(&kst[off + 2 * P::PLANE]) = u32x2{l0, l1};
        }
      }
    }
  };
  // dS of the lane for stage st_lo + it (called only for stages below
  // my_end), both row blocks: for each of its 8 keys one dword per row block,
  // where the 16 lanes of a group read 64 contiguous bytes of the key's
  // column.  Keys at or past T (in the stage that holds T) have no spill
  // entry: they read as 0.
  auto load_a = [&](int it, float (&a)[2][8]) {
    const int k0 = 32 * (st_lo + it) + 8 * g;
    const float* src = arow + (size_t)k0 * kDsColFloats;
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) a[rb][e] = src[e * kDsColFloats + 16 * rb];
    if (k0 + 8 > T) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int e = 0; e < 8; ++e) a[rb][e] = k0 + e < T ? a[rb][e] : 0.f;
    }
  };

  // Zero the d columns past D (D < 16 pads the staged rows to 16 columns).
  if (D < 16) {
    for (int e = tid; e < P::STAGE; e += 256) reinterpret_cast<unsigned*>(kst)[e] = 0u;
    __syncthreads();
  }
  float a_next[2][8];
  if (st_lo < my_end) load_a(0, a_next);
  load_k(0);
  store_k(0);
  __syncthreads();
  // transposed reads: source lane 4j + m of group g points at key 8g + j
  // (+4 for the second read) of the stage, column 16nb + 4m
  const int srow = 8 * g + (l16 >> 2);
  for (int it = 0; it < iters; ++it) {
    const int buf = it & 1;
    if (it + 1 < iters) load_k(it + 1);
    if (st_lo + it < my_end) {
      float a[2][8];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int e = 0; e < 8; ++e) a[rb][e] = a_next[rb][e];
      if (st_lo + it + 1 < my_end) load_a(it + 1, a_next);
      const Limbs al0 = split8(a[0]), al1 = split8(a[1]);
      prio_mfma_begin<!BF>();
      const __bf16* kb_base = kst + buf * P::STAGE;
#pragma unroll
      for (int nb = 0; nb < P::NB; ++nb) {
        const int o0 = srow * P::LDK + 16 * nb + 4 * (l16 & 3);
        const int o1 = o0 + 4 * P::LDK;
        Limbs bl;
        bl.h = lds_read_tr8(kb_base + o0, kb_base + o1);
        if (BF) {
          bl.m = bl.l = bf16x8{};
        } else {
          bl.m = lds_read_tr8(kb_base + P::PLANE + o0, kb_base + P::PLANE + o1);
          bl.l = lds_read_tr8(kb_base + 2 * P::PLANE + o0, kb_base + 2 * P::PLANE + o1);
        }
#pragma unroll
        for (int st = 0; st < 6; ++st) {
          if (limb_step_used<false, BF>(st)) {
            acc[0][nb] = mfma16_step(st, al0, bl, acc[0][nb]);
            acc[1][nb] = mfma16_step(st, al1, bl, acc[1][nb]);
          }
        }
      }
      prio_mfma_end<!BF>();
    }
    if (it + 1 < iters) store_k(buf ^ 1);
    __syncthreads();
  }
  // lane (d = 16nb + l16, group g) holds rows 16rb + 4g + r of the wave's
  // tile; the other column of d's RoPE pair (d ^ 1) is in lane l16 ^ 1
  if (wave_on) {
    // single-chunk groups write dQ; chunk partials are item-indexed tiles
    // [kDqRows queries][D] (items of multi-chunk groups are numbered first),
    // summed and rotated back by the merge.  The rotation test is taken once,
    // outside the unrolled stores, so each version issues its loads together.
    const bool single = nch == 1;
    float* part = dq_part + ((size_t)bh * n_part + item) * kDqRows * D;
    E* dQs = view_slice<E>(dQv, bh, H);
    const bool odd = l16 & 1;
    auto store = [&](auto rotate_tag) {
      constexpr bool kRot = decltype(rotate_tag)::value;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int nb = 0; nb < P::NB; ++nb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int rloc = 32 * w + 16 * rb + 4 * g + r;
            const int row = kDqRows * qg + rloc;
            const int d = 16 * nb + l16;
            const float val = acc[rb][nb][r] * c;
            const float val_pair = kRot ? __shfl_xor(val, 1) : 0.f;
            if (row < T && d < D) {
              if (single) {
                float o = val;
                if (kRot) {
                  // transposed rotation back to the un-rotated q
                  const float* e = rope + (long long)row * D + (d & ~1);
                  o = odd ? fmaf(val, e[0], -val_pair * e[1]) : fmaf(val, e[0], val_pair * e[1]);
                }
                st1(dQs + (long long)row * dQv.rstride + d, o);
              } else {
                part[(size_t)rloc * D + d] = val;
              }
            }
          }
    };
    if (rope)
      store(std::true_type{});
    else
      store(std::false_type{});
  }
}

// Merge of dQ chunk partials, in chunk order: the dq_merge_slices work
// groups (BH*gi + bh)*NS + slice sum the chunks of multi-chunk dQ group
// g1-1-gi of slice bh, one float4 of its rows per thread (rotated back when
// RoPE is on).  (The dK/dV chunk partials are summed by extra work groups of
// the dQ launch.)
template <int D, class E>
__global__ __launch_bounds__(256) void ca_bwd_merge_kernel(const float* __restrict__ dq_part,
                                                           const float* __restrict__ rope,
                                                           View dQv, BwdPass pass, int B, int H,
                                                           int T, int chunk, int n_part) {
  constexpr int C4 = D / 4;
  constexpr int NS = dq_merge_slices<D>();
  const int tid = threadIdx.x + 256 * (blockIdx.x % NS);
  const int BH = B * H;
  const int m = blockIdx.x / NS;
  const int bh = m % BH, gi = m / BH;
  const int qg = pass.g1 - 1 - gi;
  int first = 0;  // item index of the group's chunk 0
  for (int gg = pass.g1 - 1; gg > qg; --gg) first += dq_group_chunks(gg, T, chunk);
  const int nch = dq_group_chunks(qg, T, chunk);
  const f32x4* part = reinterpret_cast<const f32x4*>(dq_part + ((size_t)bh * n_part + first) * kDqRows * D);
  E* dQs = view_slice<E>(dQv, bh, H);
  for (int e = tid; e < kDqRows * C4; e += 256 * NS) {
    const int row = kDqRows * qg + e / C4, c4 = e % C4;
    if (row >= T) break;
    f32x4 s = part[e];
    for (int cc = 1; cc < nch; ++cc) s += part[(size_t)cc * kDqRows * C4 + e];
    if (rope) s = rope4(s, rope_entry(rope, row, D, 4 * c4), true);
    st4(dQs + (long long)row * dQv.rstride + 4 * c4, s);
  }
}

// dK and dV summed over the passes in fp32 ([BH][T][D] each) rounded to the
// element type into their views: one thread per (slice row, 4 values).
template <int D, class E>
__global__ __launch_bounds__(256) void ca_kv_cast_kernel(const float* __restrict__ dk_sum,
                                                         const float* __restrict__ dv_sum,
                                                         View dKv, View dVv, int BH, int H,
                                                         int T) {
  constexpr int C4 = D / 4;
  const long long tix = (long long)blockIdx.x * 256 + threadIdx.x;
  if (tix >= (long long)BH * T * C4) return;
  const int c = (int)(tix % C4);
  const long long row = tix / C4;
  const int bh = (int)(row / T), t = (int)(row % T);
  const long long src = row * D + 4 * c;
  st4(view_slice<E>(dKv, bh, H) + (long long)t * dKv.rstride + 4 * c,
      *reinterpret_cast<const f32x4*>(dk_sum + src));
  st4(view_slice<E>(dVv, bh, H) + (long long)t * dVv.rstride + 4 * c,
      *reinterpret_cast<const f32x4*>(dv_sum + src));
}

template <int D, class E>
hipError_t launch_kv_cast(const float* dk_sum, const float* dv_sum, View dk, View dv, int BH,
                          int H, int T, hipStream_t stream) {
  const long long n = (long long)BH * T * (D / 4);
  hipLaunchKernelGGL((ca_kv_cast_kernel<D, E>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     stream, dk_sum, dv_sum, dk, dv, BH, H, T);
  return hipGetLastError();
}

template <int D, class E>
hipError_t launch_bwd(const BwdIO& io, const BwdWork& ws, const BwdPass& pass, const DqSplit& sp,
                      const DkdvSplit& kvs, int B, int H, int T, hipStream_t stream) {
  const int BH = B * H;
  const int ntiles = bwd_pass_tiles(pass);
  const int rows = BH * 32 * ntiles;
  timer_begin(kBwdPrep, stream);
  hipLaunchKernelGGL((ca_bwd_prep_kernel<D, E>), dim3((rows * (D / 8) + 255) / 256), dim3(256), 0,
                     stream, io.q, io.rope, io.dout, io.y, io.stats, ws.limbs, ws.qstat, H, T,
                     pass.row0, ntiles, rows);
  timer_end(kBwdPrep, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(kBwdDkdv, stream);
  e = launch_bwd_dkdv<D, E>(io, ws, pass, kvs, BH, H, T, stream);
  timer_end(kBwdDkdv, stream);
  if (e != hipSuccess) return e;
  timer_begin(kBwdDq, stream);
  // the dQ grid's extra work groups: H that sum the gain partials of the dK/dV
  // items, then kv_merge_slices per (multi-chunk dK/dV key group, slice) that
  // sum its chunk partials
  const dim3 dq_grid(sp.items * BH + H + kvs.multi_groups * BH * kv_merge_slices<D>());
  if (io.rope && !io.k_rotated)
    hipLaunchKernelGGL((ca_bwd_dq_kernel<D, E, true>), dq_grid, dim3(256), 0, stream, ws.dsbuf,
                       io.k, io.rope, io.log_gain, io.dq, ws.dq_part, ws.gain_part, io.dlog_gain,
                       pass, B, H, T, sp.chunk, sp.items, sp.part_items, kvs.items, ws.kv_part,
                       io.dk, io.dv, kvs.chunk, kvs.part_items, io.kv_f32);
  else
    hipLaunchKernelGGL((ca_bwd_dq_kernel<D, E, false>), dq_grid, dim3(256), 0, stream, ws.dsbuf,
                       io.k, io.rope, io.log_gain, io.dq, ws.dq_part, ws.gain_part, io.dlog_gain,
                       pass, B, H, T, sp.chunk, sp.items, sp.part_items, kvs.items, ws.kv_part,
                       io.dk, io.dv, kvs.chunk, kvs.part_items, io.kv_f32);
  timer_end(kBwdDq, stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // dQ chunk partials (small grids only) are merged by a launch of their own
  if (sp.multi_groups == 0) return hipSuccess;
  timer_begin(kBwdGain, stream);
  hipLaunchKernelGGL((ca_bwd_merge_kernel<D, E>), dim3(BH * sp.multi_groups * dq_merge_slices<D>()),
                     dim3(256), 0, stream,
                     ws.dq_part, io.rope, io.dq, pass, B, H, T, sp.chunk, sp.part_items);
  timer_end(kBwdGain, stream);
  return hipGetLastError();
}

#define CA_INST_BWD(DD, EE)                                                                     \
  template hipError_t launch_bwd<DD, EE>(const BwdIO&, const BwdWork&, const BwdPass&,          \
                                         const DqSplit&, const DkdvSplit&, int, int, int,       \
                                         hipStream_t);                                          \
  template hipError_t launch_kv_cast<DD, EE>(const float*, const float*, View, View, int, int,  \
                                             int, hipStream_t);
#define CA_INST_BWD_ALL(EE) \
  CA_INST_BWD(8, EE) CA_INST_BWD(16, EE) CA_INST_BWD(32, EE) CA_INST_BWD(64, EE) CA_INST_BWD(128, EE)
CA_INST_BWD_ALL(float)
CA_INST_BWD_ALL(__bf16)
CA_INST_BWD_ALL(_Float16)

}  // namespace ca
