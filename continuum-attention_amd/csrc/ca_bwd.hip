// Continuum Attention backward (gfx950, fp32 MFMA), analytic first-order VJP.
//
// Replaces the per-query-tile loop of _CAExactTiled.backward
// (cuda/continuum_attention.py:697-766): the QK^T and dY.V^T recomputation,
// the fused score-VJP kernels (ca_backward_fused_kernel /
// ca_backward_half_kernel, cuda/continuum_attention.py:230-293,337-405) and
// the dV/dQ/dK/dRho contractions.
//
// Kernels (all deterministic, no atomics):
//   ca_bwd_rowdot   Dl_i = dY_i . y_i   (equals sum_j W_ij dW_ij; the reference
//                   forms the same row mean at cuda/continuum_attention.py:268-269)
//   ca_bwd_dkdv     one work group per (slice, 30-key block); 4 waves take
//                   interleaved 32-query tiles.  Per tile: S^T = K Q^T and
//                   dP^T = V dY^T by MFMA (K, V slot rows from LDS shared by
//                   the work group; Q, dY rows straight from the lane's own
//                   prefetched registers), W and dS in registers, then
//                   dV^T += dY^T W and dK^T += Q^T dS by MFMA (W, dS through a
//                   transposed LDS tile; dY^T, then Q^T, read column-wise
//                   from the wave's row tile).  dS is also written,
//                   straight from registers, as 32x32 row blocks for the dQ
//                   pass.  ~68 KB of LDS and <= 256 VGPRs: two work groups
//                   share a CU and hide each other's staging, waits and
//                   epilogue behind their MFMA phases.
//   ca_bwd_dq       dQ = c dS (K - k_ref), one work group per (slice, 64
//                   queries); its epilogue also forms the gain partial
//                   sum_i q_i . dQ_i (= sum_ij dS_ij s_ij, since s_ij = c q_i . k_j).
//   ca_bwd_gain     dRho_h = sum over batch and query groups of the partials.
//
// Key-block layout: the work group owns weight keys [w0, w0+30); its 32 MFMA
// key slots are keys w0-1 .. w0+30 (slot s = key w0-1+s), so both neighbours
// of every owned key are inside the tile.  Lane half h, register n holds slot
// 16h+n of query q.
#include <type_traits>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

template <int D>
struct Bwd {
  static constexpr int DH = D / 2;            // d values per lane half (k-range split)
  static constexpr int NMB = (D + 31) / 32;   // 32-row d blocks of dV^T / dK^T
  static constexpr int C4 = D / 4;            // float4 chunks per row
  static constexpr int CH = DH / 4;           // chunks per lane half
  static constexpr int LDQ = D + 4;           // padded row stride: K/V slot tiles and Q tile
  static constexpr int LDX = kBwdSlots + 1;   // row stride of the [slot][query] transpose tile
  static constexpr int SLOT_FLOATS = 32 * LDQ;
  static constexpr int QT_FLOATS = 32 * LDQ;
  static constexpr int XT_FLOATS = ((kBwdSlots * LDX + 3) / 4) * 4;
  static constexpr int WAVE_FLOATS = QT_FLOATS + XT_FLOATS;
  static constexpr int MAIN_FLOATS = 2 * SLOT_FLOATS + 4 * WAVE_FLOATS;
  static constexpr int RED_FLOATS = 4 * NMB * 16 * 64;  // epilogue: one matrix, all waves
  static constexpr int LDS_FLOATS = MAIN_FLOATS > RED_FLOATS ? MAIN_FLOATS : RED_FLOATS;
};

// Dl_i = dY_i . y_i: one float4 chunk per thread, D/4 lanes per row.
template <int D>
__global__ __launch_bounds__(256) void ca_bwd_rowdot_kernel(const float* __restrict__ dout,
                                                            const float* __restrict__ out,
                                                            float* __restrict__ dvec, int rows) {
  constexpr int C4 = D / 4;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int row = t / C4, c = t % C4;
  float x = 0.f;
  if (row < rows) {
    const f32x4 a = reinterpret_cast<const f32x4*>(dout + (size_t)row * D)[c];
    const f32x4 b = reinterpret_cast<const f32x4*>(out + (size_t)row * D)[c];
    x = a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
  }
#pragma unroll
  for (int o = C4 / 2; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  if (row < rows && c == 0) dvec[row] = x;
}

template <int D>
__global__ __launch_bounds__(256, 2) void ca_bwd_dkdv_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ stats, const float* __restrict__ dvec,
    const float* __restrict__ log_gain, float* __restrict__ dK, float* __restrict__ dV,
    float* __restrict__ dsbuf, int BH, int H, int T) {
  using P = Bwd<D>;
  extern __shared__ float lds[];

  const int nqt = num_q_tiles(T);
  const int bh = blockIdx.x % BH;
  const int kb = blockIdx.x / BH;  // ascending: heaviest key blocks first
  const int w0 = kBwdKeys * kb;

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int q = lane & 31;
  const int h = lane >> 5;

  float* Ks = lds;                     // K slot rows, scaled by c log2e
  float* Vs = lds + P::SLOT_FLOATS;    // V slot rows
  float* At = lds + 2 * P::SLOT_FLOATS + w * P::WAVE_FLOATS;  // this wave's dY, then Q, tile
  float* Xt = At + P::QT_FLOATS;       // this wave's W / dS tile, [slot][query]

  const size_t slice = (size_t)bh * T * D;
  const float cl2 = head_scale_log2(log_gain, bh % H, D);

  // ---- the block's 32 K and V slot rows (slot s = key w0-1+s), shared by the waves ----
  for (int e = tid; e < 32 * P::C4; e += 256) {
    const int s = e / P::C4, c = e % P::C4;
    const int key = w0 - 1 + s;
    f32x4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
    if (key >= 0 && key < T) {
      kv = reinterpret_cast<const f32x4*>(K + slice + (size_t)key * D)[c] * cl2;
      vv = reinterpret_cast<const f32x4*>(V + slice + (size_t)key * D)[c];
    }
    *reinterpret_cast<f32x4*>(Ks + s * P::LDQ + 4 * c) = kv;
    *reinterpret_cast<f32x4*>(Vs + s * P::LDQ + 4 * c) = vv;
  }

  f32x16 accv[P::NMB], acck[P::NMB];
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      accv[mb][r] = 0.f;
      acck[mb][r] = 0.f;
    }
  const int qt0 = w0 / 32;  // first query tile that sees an owned key
  // dS block index of (this wave's current query tile, kb)
  long long ds_blk = (long long)bh * ds_blocks_before(nqt) + ds_blocks_before(qt0 + w) + kb;
  // This lane's own query row half of Q and dY for the next tile (the B
  // operands of S^T / dP^T), plus its row stats; loaded a tile ahead, dY and
  // stats as soon as the current ones are consumed, Q after its tile is staged.
  f32x4 pf_q[P::CH], pf_o[P::CH];
  float pf_m2 = 0.f, pf_invz = 0.f, pf_d = 0.f;
  auto prefetch_rows = [&](int qt, const float* __restrict__ src, f32x4* dst) {
    const int i = 32 * qt + q;
    const bool ok = i < T;
    const f32x4* rp = reinterpret_cast<const f32x4*>(src + slice + (size_t)(ok ? i : 0) * D + h * P::DH);
#pragma unroll
    for (int c = 0; c < P::CH; ++c) dst[c] = ok ? rp[c] : f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto prefetch_stats = [&](int qt) {
    const int i = 32 * qt + q;
    const bool ok = i < T;
    pf_m2 = ok ? stats[((size_t)bh * T + i) * 2 + 0] : 0.f;
    pf_invz = ok ? stats[((size_t)bh * T + i) * 2 + 1] : 0.f;
    pf_d = ok ? dvec[(size_t)bh * T + i] : 0.f;
  };
  if (qt0 + w < nqt) {
    prefetch_rows(qt0 + w, Q, pf_q);
    prefetch_rows(qt0 + w, dO, pf_o);
    prefetch_stats(qt0 + w);
  }

  const int arow = key_of_arow(lane);  // slot row this lane feeds to the S^T / dP^T A operand
  const bool dok = q < D;              // D < 32 pads the d rows of dV^T / dK^T
  const int dcol = dok ? q : 0;
  __syncthreads();

  for (int qt = qt0 + w; qt < nqt; qt += 4) {
    const int i0 = 32 * qt;
    const int i = i0 + q;
    const float m2 = pf_m2, invz = pf_invz, dz = pf_d * pf_invz;

    // ---- dY row (this lane's half) into the wave's tile for the dV pass ----
#pragma unroll
    for (int c = 0; c < P::CH; ++c)
      *reinterpret_cast<f32x4*>(At + q * P::LDQ + h * P::DH + 4 * c) = pf_o[c];

    // ---- S^T (minus the row shift, folded into the accumulator) and dP^T ----
    // A operands from the shared slot tiles (chunk c+1 read before the MFMAs
    // of chunk c issue), B operands from this lane's own prefetched rows.
    f32x16 sacc, pacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = -m2;
      pacc[r] = 0.f;
    }
    {
      const float* krow = Ks + arow * P::LDQ + h * P::DH;
      const float* vrow = Vs + arow * P::LDQ + h * P::DH;
      f32x4 kv_n = *reinterpret_cast<const f32x4*>(krow);
      f32x4 vv_n = *reinterpret_cast<const f32x4*>(vrow);
#pragma unroll
      for (int c = 0; c < P::CH; ++c) {
        const f32x4 kv = kv_n, vv = vv_n;
        if (c + 1 < P::CH) {
          kv_n = *reinterpret_cast<const f32x4*>(krow + 4 * (c + 1));
          vv_n = *reinterpret_cast<const f32x4*>(vrow + 4 * (c + 1));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sacc = mfma32(kv[e], pf_q[c][e], sacc);
          pacc = mfma32(vv[e], pf_o[c][e], pacc);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // ---- weights and score gradients of this lane's 16 slots ----
    // Streams over the slots; W overwrites sacc and dS overwrites pacc in place.
    // Tiles that may hold invisible keys (or key 0 / the caps) take the general
    // path; all others need no masks.
    const int kbase = w0 - 1 + 16 * h;  // key of register 0
    const bool need_mask = (w0 == 0) || (w0 + kBwdKeys > i0) || (i0 + 32 > T);
    auto segments = [&](auto general_tag) {
      constexpr bool kGeneral = decltype(general_tag)::value;
      auto slot_vis = [&](int n) {
        const int key = kbase + n;
        return !kGeneral || (key >= 0 && key <= i);
      };
      // half 1's first segment starts at half 0's last slot
      float sl, pl, gl;
      {
        const bool v15 = slot_vis(15);
        const float s15 = v15 ? sacc[15] : 0.f;
        const float g15 = v15 ? fmaf(pacc[15], invz, -dz) : 0.f;
        sl = xhalf(s15);
        pl = fast_exp2(sl);
        gl = xhalf(g15);
      }
      float r_prev = 0.f, dr_prev = 0.f, xl0 = 0.f, xdl0 = 0.f;
      // finalises slot n from its own (p, g), incoming right and outgoing left shares
      auto finish = [&](int n, float pv, float gv, float wv, float dv) {
        if (kGeneral) {
          // half-token caps on the first key and the last visible key (both when i == 0)
          const int key = kbase + n;
          const bool vis = slot_vis(n);
          const float cap = (vis && key == 0 ? 0.5f * pv : 0.f) + (vis && key == i ? 0.5f * pv : 0.f);
          wv += cap;
          dv = fmaf(cap, gv, dv);
        }
        const int slot = 16 * h + n;
        const bool owned = slot >= 1 && slot <= kBwdKeys;
        sacc[n] = owned ? wv * invz : 0.f;
        pacc[n] = owned ? dv : 0.f;
      };
#pragma unroll
      for (int n = 0; n < 16; ++n) {
        const bool vis = slot_vis(n);
        const float sr = vis ? sacc[n] : 0.f;  // s - m2
        const float gr = vis ? fmaf(pacc[n], invz, -dz) : 0.f;
        const float pr = fast_exp2(sr);
        float Lv, Rv, dLv, dRv;
        seg_shares_grad(sl, sr, pl, pr, gl, gr, Lv, Rv, dLv, dRv);
        const int key = kbase + n;  // right key of this segment
        bool ok = (n > 0) || (h == 1);
        if (kGeneral) ok = ok && key >= 1 && key <= i;
        Lv = ok ? Lv : 0.f;
        Rv = ok ? Rv : 0.f;
        dLv = ok ? dLv : 0.f;
        dRv = ok ? dRv : 0.f;
        if (n == 0) {
          xl0 = xhalf(Lv);  // half 1's first left share belongs to half 0's last slot
          xdl0 = xhalf(dLv);
        } else {
          finish(n - 1, pl, gl, r_prev + Lv, dr_prev + dLv);
        }
        r_prev = Rv;
        dr_prev = dRv;
        sl = sr;
        pl = pr;
        gl = gr;
      }
      finish(15, pl, gl, r_prev + (h ? 0.f : xl0), dr_prev + (h ? 0.f : xdl0));
    };
    if (need_mask)
      segments(std::true_type{});
    else
      segments(std::false_type{});

    // ---- dS row block for the dQ pass: row q, slots 16h..16h+15 ----
    {
      float* dst = dsbuf + ((size_t)ds_blk * kDsBlockFloats) + q * kBwdSlots + 16 * h;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<f32x4*>(dst + 4 * c) =
            f32x4{pacc[4 * c], pacc[4 * c + 1], pacc[4 * c + 2], pacc[4 * c + 3]};
      ds_blk += ds_kb_count(qt) + ds_kb_count(qt + 1) + ds_kb_count(qt + 2) + ds_kb_count(qt + 3);
    }

    // ---- acc^T[d][slot] += sum_query A[query][d] X[query][slot] ----
    // X (W or dS, held per query lane) goes through the [slot][query] tile, A
    // (dY, then Q) is read column-wise from the wave's row tile; at step r
    // lane half h contributes query 16h + r.
    auto put_x = [&](const f32x16& x) {
#pragma unroll
      for (int n = 0; n < 16; ++n) Xt[(16 * h + n) * P::LDX + q] = x[n];
    };
    const float* xcol = Xt + q * P::LDX + 16 * h;    // B operand: slot q, query 16h + r
    const float* acol = At + 16 * h * P::LDQ + dcol;  // A operand: row 16h + r, column d
    auto mma_x = [&](f32x16 (&acc)[P::NMB]) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float b = xcol[r];
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb) {
          const float a = dok ? acol[r * P::LDQ + 32 * mb] : 0.f;
          acc[mb] = mfma32(a, b, acc[mb]);
        }
      }
    };
    put_x(sacc);
    wave_lds_sync();
    // the next tile's dY row and stats fly during the dV and dK MFMAs
    if (qt + 4 < nqt) {
      prefetch_rows(qt + 4, dO, pf_o);
      prefetch_stats(qt + 4);
    }
    mma_x(accv);  // dV^T += dY^T W
    wave_lds_sync();
    put_x(pacc);
#pragma unroll
    for (int c = 0; c < P::CH; ++c)
      *reinterpret_cast<f32x4*>(At + q * P::LDQ + h * P::DH + 4 * c) = pf_q[c];
    wave_lds_sync();
    if (qt + 4 < nqt) prefetch_rows(qt + 4, Q, pf_q);
    mma_x(acck);  // dK^T += Q^T dS
    wave_lds_sync();
  }

  // ---- reduce the 4 waves' partial dV^T / dK^T through LDS, one matrix at a time ----
  constexpr int NE = P::NMB * 16;  // accumulator elements per lane per matrix
  constexpr int NG = P::NMB * 4;   // float4 groups per lane per matrix
  auto reduce_store = [&](const f32x16 (&acc)[P::NMB], float* __restrict__ out, float scale) {
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) lds[(w * NE + mb * 16 + r) * 64 + lane] = acc[mb][r];
    __syncthreads();
    // column q of the accumulator is slot q; register group r4 holds d = 32mb + 8r4 + 4h + 0..3
    for (int gi = w; gi < NG; gi += 4) {
      const int mb = gi / 4, r4 = gi % 4;
      const int key = w0 - 1 + q;
      const int d0 = 32 * mb + 8 * r4 + 4 * h;
      f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < 4; ++ww)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) sum[e4] += lds[(ww * NE + mb * 16 + 4 * r4 + e4) * 64 + lane];
      if (q >= 1 && q <= kBwdKeys && key < T && d0 < D)
        *reinterpret_cast<f32x4*>(out + slice + (size_t)key * D + d0) = sum * scale;
    }
  };
  reduce_store(accv, dV, 1.0f);
  reduce_store(acck, dK, cl2 * kLn2);
}

// dQ = c dS (K - k_ref) as a tiled GEMM over the 32x32 dS blocks written by
// ca_bwd_dkdv.  Work item: one chunk of the key blocks of a 64-query group
// (two 32-query tiles) of one slice; wave w takes query tile w&1 and the
// chunk's key blocks of parity w>>1.  Per stage the 32 K rows of two
// consecutive key blocks (slots 30kb-1 .. 30kb+30 each) are staged in LDS
// (double-buffered) and shared by all four waves; lane half h supplies slots
// 16h + s at k-step s.  Halo slots and invisible keys carry dS = 0, so no
// masks are needed.  The dS operand of the wave's next block is prefetched
// into registers.  The two parities are summed through LDS at the end (fixed
// order).  A single-chunk group writes dQ; the chunks of a longer group write
// partial tiles that ca_bwd_gain_merge sums.  Every item writes its gain
// partial sum_i q_i . dQ_i(chunk) (linear in dQ, so the partials add up).
template <int D>
__global__ __launch_bounds__(256) void ca_bwd_dq_kernel(const float* __restrict__ dsbuf,
                                                        const float* __restrict__ Q,
                                                        const float* __restrict__ K,
                                                        const float* __restrict__ log_gain,
                                                        float* __restrict__ dQ,
                                                        float* __restrict__ dq_part,
                                                        float* __restrict__ gain_part, int BH,
                                                        int H, int T, int chunk, int n_items,
                                                        int n_part) {
  using P = Bwd<D>;
  constexpr int KF4 = 2 * kBwdSlots * P::C4;  // float4 per stage (two key blocks)
  constexpr int KLD = (KF4 + 255) / 256;      // float4 loads per thread
  constexpr int RED4 = 2 * P::NMB * 16 * 64 / 4;      // float4 of the final parity reduction
  // The K stages and the final reduction buffer are live at disjoint times and
  // share one allocation (fewer LDS bytes per work group, more resident groups).
  __shared__ f32x4 smem[2 * KF4 > RED4 ? 2 * KF4 : RED4];
  f32x4 (*kst)[KF4] = reinterpret_cast<f32x4 (*)[KF4]>(smem);
  float* red = reinterpret_cast<float*>(smem);
  __shared__ float gred[2];
  const int nqt = num_q_tiles(T);
  const int nkb = bwd_num_key_blocks(T);
  const int bh = blockIdx.x % BH;
  const int item = blockIdx.x / BH;
  // item -> (group, chunk), heaviest groups first
  int qg = dq_num_groups(T) - 1, ch = item, nch = dq_group_chunks(qg, T, chunk);
  while (ch >= nch && qg > 0) {
    ch -= nch;
    --qg;
    nch = dq_group_chunks(qg, T, chunk);
  }
  const int gblocks = dq_group_blocks(qg, T);
  const int clen = (gblocks + nch - 1) / nch;
  const int kb_lo = ch * clen;
  const int kb_hi = min(kb_lo + clen, gblocks);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, q = lane & 31, h = lane >> 5;
  const int qsub = w & 1, par = w >> 1;
  const int qt = 2 * qg + qsub;
  const bool wave_on = qt < nqt;
  const size_t slice = (size_t)bh * T * D;
  const float c = head_scale_log2(log_gain, bh % H, D) * kLn2;
  // key blocks of this chunk met by the wave's tile
  const int my_end = wave_on ? min(min(ds_kb_count(qt), nkb), kb_hi) : 0;
  const int iters = kb_hi > kb_lo ? (kb_hi - kb_lo + 1) / 2 : 0;
  const float* arow =
      dsbuf + ((size_t)bh * ds_blocks_before(nqt) + ds_blocks_before(wave_on ? qt : 0)) * kDsBlockFloats +
      q * kBwdSlots + 16 * h;

  f32x16 acc[P::NMB];
#pragma unroll
  for (int nb = 0; nb < P::NMB; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0.f;

  // Every row of dS sums to zero (the weights are invariant to a common score
  // shift), so dQ_i = c sum_j dS_ij (k_j - k_ref) for any k_ref.  The staged
  // keys are taken relative to the key at the group's first query: when
  // neighbouring keys nearly coincide the products stay small instead of
  // cancelling in fp32 (|k| ~ 1 against |k_j - k_ref| ~ 1e-2 in the
  // near-duplicate-key case), and the gain partial sum_i q_i . dQ_i inherits
  // the same accuracy.  All chunks of a group use the same k_ref, so the
  // k_ref terms cancel in the sum of the chunk partials.
  f32x4 kref[KLD];
  {
    const f32x4* kr = reinterpret_cast<const f32x4*>(K + slice + (size_t)(64 * qg) * D);
#pragma unroll
    for (int j = 0; j < KLD; ++j) kref[j] = kr[(tid + 256 * j) % P::C4];
  }
  f32x4 pre[KLD];
  auto load_k = [&](int it) {
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      const int e = tid + 256 * j;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (e < KF4) {
        const int row = e / P::C4;  // 32 * (block in stage) + slot
        const int key = kBwdKeys * (kb_lo + 2 * it + (row >> 5)) - 1 + (row & 31);
        if (key >= 0 && key < T)
          v = reinterpret_cast<const f32x4*>(K + slice + (size_t)key * D)[e % P::C4];
      }
      pre[j] = v;
    }
  };
  // the shift is applied when the prefetched rows are stored, so the loads
  // issued a stage ahead are not waited for inside the MFMA loop
  auto store_k = [&](int buf) {
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      const int e = tid + 256 * j;
      if (e < KF4) kst[buf][e] = pre[j] - kref[j];
    }
  };
  auto load_a = [&](int kbm, float* a) {
    const f32x4* src = reinterpret_cast<const f32x4*>(arow + (size_t)kbm * kDsBlockFloats);
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const f32x4 v4 = src[c4];
      a[4 * c4 + 0] = v4[0]; a[4 * c4 + 1] = v4[1]; a[4 * c4 + 2] = v4[2]; a[4 * c4 + 3] = v4[3];
    }
  };

  float a_next[16];
  if (kb_lo + par < my_end) load_a(kb_lo + par, a_next);
  load_k(0);
  store_k(0);
  __syncthreads();
  const int dcol = (q < D) ? q : 0;
  for (int it = 0; it < iters; ++it) {
    const int buf = it & 1;
    if (it + 1 < iters) load_k(it + 1);
    const int kbm = kb_lo + 2 * it + par;
    if (kbm < my_end) {
      float a[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) a[r] = a_next[r];
      if (kbm + 2 < my_end) load_a(kbm + 2, a_next);
      const float* kbp = reinterpret_cast<const float*>(&kst[buf][0]) + (32 * par + 16 * h) * D + dcol;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int nb = 0; nb < P::NMB; ++nb) {
          const float b = (32 * nb + q < D) ? kbp[r * D + 32 * nb] : 0.f;
          acc[nb] = mfma32(a[r], b, acc[nb]);
        }
      }
    }
    if (it + 1 < iters) store_k(buf ^ 1);
    __syncthreads();
  }
  // Q rows for the gain partial, loaded as one batch before the reduction
  float qv[P::NMB][16];
  if (par == 0 && wave_on) {
#pragma unroll
    for (int nb = 0; nb < P::NMB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * qt + 8 * (r >> 2) + 4 * h + (r & 3);
        const int d = 32 * nb + q;
        qv[nb][r] = (row < T && d < D) ? Q[slice + (size_t)row * D + d] : 0.f;
      }
  }
  if (par == 1) {
#pragma unroll
    for (int nb = 0; nb < P::NMB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((qsub * P::NMB + nb) * 16 + r) * 64 + lane] = acc[nb][r];
  }
  __syncthreads();
  if (par == 0) {
    float g = 0.f;
    if (wave_on) {
      // single-chunk groups write dQ; chunk partials are item-indexed tiles
      // [64 queries][D] (items of multi-chunk groups are numbered first)
      float* dst = nch == 1 ? dQ + slice + (size_t)(64 * qg) * D
                            : dq_part + ((size_t)bh * n_part + item) * 64 * D;
#pragma unroll
      for (int nb = 0; nb < P::NMB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float sum = acc[nb][r] + red[((qsub * P::NMB + nb) * 16 + r) * 64 + lane];
          const int rloc = 32 * qsub + 8 * (r >> 2) + 4 * h + (r & 3);
          const int d = 32 * nb + q;
          const float val = sum * c;
          g = fmaf(qv[nb][r], val, g);
          if (64 * qg + rloc < T && d < D) dst[(size_t)rloc * D + d] = val;
        }
    }
    g = wave_sum(g);
    if (lane == 0) gred[qsub] = g;
  }
  __syncthreads();
  if (tid == 0) gain_part[(size_t)bh * n_items + item] = gred[0] + gred[1];
}

// Work groups [0, H): dRho_h = sum over batch and dQ items of the gain
// partials (fixed order).  Work groups H + BH*gi + bh: dQ of multi-chunk
// group nqg-1-gi of slice bh, the sum of its chunk partials in chunk order.
template <int D>
__global__ __launch_bounds__(256) void ca_bwd_gain_merge_kernel(
    const float* __restrict__ gain_part, const float* __restrict__ dq_part,
    float* __restrict__ dlog_gain, float* __restrict__ dQ, int B, int H, int T, int chunk,
    int n_items, int n_part) {
  const int tid = threadIdx.x;
  if (blockIdx.x < H) {
    __shared__ float wsum[4];
    const int h = blockIdx.x;
    float acc = 0.f;
    for (int b = 0; b < B; ++b)
      for (int k = tid; k < n_items; k += 256) acc += gain_part[((size_t)b * H + h) * n_items + k];
    acc = wave_sum(acc);
    if ((tid & 63) == 0) wsum[tid >> 6] = acc;
    __syncthreads();
    if (tid == 0) dlog_gain[h] = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    return;
  }
  constexpr int C4 = D / 4;
  const int BH = B * H;
  const int m = blockIdx.x - H;
  const int bh = m % BH, gi = m / BH;
  const int qg = dq_num_groups(T) - 1 - gi;
  int first = 0;  // item index of the group's chunk 0
  for (int g = dq_num_groups(T) - 1; g > qg; --g) first += dq_group_chunks(g, T, chunk);
  const int nch = dq_group_chunks(qg, T, chunk);
  const f32x4* part = reinterpret_cast<const f32x4*>(dq_part + ((size_t)bh * n_part + first) * 64 * D);
  f32x4* out = reinterpret_cast<f32x4*>(dQ + ((size_t)bh * T + 64 * qg) * D);
  for (int e = tid; e < 64 * C4; e += 256) {
    if (64 * qg + e / C4 >= T) break;
    f32x4 s = part[e];
    for (int ch = 1; ch < nch; ++ch) s += part[(size_t)ch * 16 * D + e];
    out[e] = s;
  }
}

template <int D>
hipError_t launch_bwd(const float* q, const float* k, const float* v, const float* log_gain,
                      const float* o, const float* stats, const float* dout, float* dq, float* dk,
                      float* dv, float* dlog_gain, float* dsbuf, float* dvec, float* gain_part,
                      float* dq_part, const DqSplit& sp, int B, int H, int T,
                      hipStream_t stream) {
  using P = Bwd<D>;
  const int BH = B * H;
  const int rows = BH * T;
  timer_begin(kBwdRowdot, stream);
  hipLaunchKernelGGL(ca_bwd_rowdot_kernel<D>, dim3((rows * (D / 4) + 255) / 256), dim3(256), 0,
                     stream, dout, o, dvec, rows);
  timer_end(kBwdRowdot, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds_bytes = sizeof(float) * P::LDS_FLOATS;
  const int nkb = bwd_num_key_blocks(T);
  timer_begin(kBwdDkdv, stream);
  hipLaunchKernelGGL(ca_bwd_dkdv_kernel<D>, dim3(nkb * BH), dim3(256), lds_bytes, stream, q, k,
                     v, dout, stats, dvec, log_gain, dk, dv, dsbuf, BH, H, T);
  timer_end(kBwdDkdv, stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(kBwdDq, stream);
  hipLaunchKernelGGL(ca_bwd_dq_kernel<D>, dim3(sp.items * BH), dim3(256), 0, stream, dsbuf, q, k,
                     log_gain, dq, dq_part, gain_part, BH, H, T, sp.chunk, sp.items,
                     sp.part_items);
  timer_end(kBwdDq, stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(kBwdGain, stream);
  hipLaunchKernelGGL(ca_bwd_gain_merge_kernel<D>, dim3(H + BH * sp.multi_groups), dim3(256), 0,
                     stream, gain_part, dq_part, dlog_gain, dq, B, H, T, sp.chunk, sp.items,
                     sp.part_items);
  timer_end(kBwdGain, stream);
  return hipGetLastError();
}

template <int D>
hipError_t set_bwd_attrs() {
  using P = Bwd<D>;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&ca_bwd_dkdv_kernel<D>),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)(sizeof(float) * P::LDS_FLOATS));
}

template hipError_t set_bwd_attrs<8>();
template hipError_t set_bwd_attrs<16>();
template hipError_t set_bwd_attrs<32>();
template hipError_t set_bwd_attrs<64>();

#define CA_INST_BWD(DD)                                                                        \
  template hipError_t launch_bwd<DD>(const float*, const float*, const float*, const float*,   \
                                     const float*, const float*, const float*, float*, float*, \
                                     float*, float*, float*, float*, float*, float*,           \
                                     const DqSplit&, int, int, int, hipStream_t);
CA_INST_BWD(8)
CA_INST_BWD(16)
CA_INST_BWD(32)
CA_INST_BWD(64)

}  // namespace ca
