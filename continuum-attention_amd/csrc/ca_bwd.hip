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
//   ca_bwd_dkdv     one work group per (slice, 62-key block); 4 waves take
//                   interleaved 32-query tiles.  Per tile: S^T = K Q^T and
//                   dP^T = V dY^T by MFMA, W and dS in registers, then
//                   dV^T += dY^T W and dK^T += Q^T dS by MFMA after an LDS
//                   transpose.  dS is also written, straight from registers,
//                   as 32x64 row blocks for the dQ pass.
//   ca_bwd_dq       dQ = c dS K, one work group per (slice, 64 queries); its
//                   epilogue also forms the gain partial sum_i q_i . dQ_i
//                   (= sum_ij dS_ij s_ij, since s_ij = c q_i . k_j).
//   ca_bwd_gain     dRho_h = sum over batch and query groups of the partials.
//
// Key-block layout: the work group owns weight keys [w0, w0+62); its 64 MFMA
// key slots are keys w0-1 .. w0+62 (slot s = key w0-1+s), so both neighbours
// of every owned key are inside the tile.  Lane half h, register n holds slot
// 32h+n of query q.
#include <type_traits>

#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

template <int D>
struct Bwd {
  static constexpr int DH = D / 2;
  static constexpr int NMB = (D + 31) / 32;
  static constexpr int C4 = D / 4;
  static constexpr int CH = DH / 4;
  static constexpr int LDQ = D + 4;   // padded row stride (floats) of the Q / dY tiles
  static constexpr int LDW = 64 + 4;  // padded row stride of the W / dS tiles
  static constexpr int WAVE_FLOATS = 2 * 32 * LDQ + 2 * 32 * LDW;
  static constexpr int LDS_FLOATS = 4 * WAVE_FLOATS + 64 * D;  // + shared V slots
};

// XOR swizzle of the V-slot float4 chunks: the A-operand rows read together
// (slots 16b+{0..3} and 32+16b+{0..3}, ...) land in distinct bank groups.
__device__ __forceinline__ int vswz(int row, int chunks_per_half) {
  return ((row & 3) | ((row >> 3) & 4)) & (chunks_per_half - 1);
}

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
__global__ __launch_bounds__(256) void ca_bwd_dkdv_kernel(
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

  float* Qt = lds + w * P::WAVE_FLOATS;
  float* dOt = Qt + 32 * P::LDQ;
  float* Wt = dOt + 32 * P::LDQ;
  float* dSt = Wt + 32 * P::LDW;

  const size_t slice = (size_t)bh * T * D;
  const int head = bh % H;
  const float cl2 = head_scale_log2(log_gain, head, D);

  // A operands of S^T = K Q^T (registers) and dP^T = V dY^T (work-group
  // shared LDS, XOR-swizzled float4 chunks): rows of this block's 64 slots.
  f32x4* vsl = reinterpret_cast<f32x4*>(lds + 4 * P::WAVE_FLOATS);
  for (int e = tid; e < 64 * P::C4; e += 256) {
    const int row = e / P::C4, c = e % P::C4;
    const int key = w0 - 1 + row;
    f32x4 vv = {0.f, 0.f, 0.f, 0.f};
    if (key >= 0 && key < T) vv = reinterpret_cast<const f32x4*>(V + slice + (size_t)key * D)[c];
    const int half = c / P::CH, cc = c % P::CH;
    vsl[row * P::C4 + half * P::CH + (cc ^ vswz(row, P::CH))] = vv;
  }
  float ka[2][P::DH];
  int vrow[2];
  {
    const int i = lane & 31;
    const int rsub = ((i >> 3) << 2) | (i & 3);
    const int hh = (i >> 2) & 1;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      vrow[b] = 32 * hh + 16 * b + rsub;
      const int key = w0 - 1 + vrow[b];
      const bool ok = key >= 0 && key < T;
      const f32x4* kp = reinterpret_cast<const f32x4*>(K + slice + (size_t)(ok ? key : 0) * D + h * P::DH);
#pragma unroll
      for (int c = 0; c < P::CH; ++c) {
        f32x4 kv = ok ? kp[c] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) ka[b][4 * c + e] = kv[e];
      }
    }
  }
  __syncthreads();

  f32x16 accv[P::NMB][2], acck[P::NMB][2];
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        accv[mb][nb][r] = 0.f;
        acck[mb][nb][r] = 0.f;
      }
  const int qt0 = w0 / 32;
  // dS block index of (this wave's current query tile, kb)
  long long ds_blk = (long long)bh * ds_blocks_before(nqt) + ds_blocks_before(qt0 + w) + kb;
  // Next query tile of this wave, prefetched into registers while the current
  // tile's dV/dK MFMAs run (32 rows x D floats of Q and of dY, plus row stats).
  constexpr int PF = (32 * P::C4 + 63) / 64;  // float4 per lane per matrix
  f32x4 pf_q[PF], pf_o[PF];
  float pf_m2 = 0.f, pf_invz = 0.f, pf_d = 0.f;
  auto prefetch = [&](int qt) {
    const int i0 = 32 * qt;
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int e = lane + 64 * j;
      const int row = e / P::C4, c = e % P::C4;
      const int qi = i0 + row;
      f32x4 qv = {0.f, 0.f, 0.f, 0.f}, ov = {0.f, 0.f, 0.f, 0.f};
      if (e < 32 * P::C4 && qi < T) {
        qv = reinterpret_cast<const f32x4*>(Q + slice + (size_t)qi * D)[c];
        ov = reinterpret_cast<const f32x4*>(dO + slice + (size_t)qi * D)[c];
      }
      pf_q[j] = qv;
      pf_o[j] = ov;
    }
    const int i = i0 + q;
    pf_m2 = 0.f; pf_invz = 0.f; pf_d = 0.f;
    if (i < T) {
      pf_m2 = stats[((size_t)bh * T + i) * 2 + 0];
      pf_invz = stats[((size_t)bh * T + i) * 2 + 1];
      pf_d = dvec[(size_t)bh * T + i];
    }
  };
  if (qt0 + w < nqt) prefetch(qt0 + w);

  for (int qt = qt0 + w; qt < nqt; qt += 4) {
    const int i0 = 32 * qt;
    // ---- stage this wave's Q (pre-scaled) and dY tiles from the prefetch ----
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int e = lane + 64 * j;
      if (e < 32 * P::C4) {
        const int row = e / P::C4, c = e % P::C4;
        *reinterpret_cast<f32x4*>(Qt + row * P::LDQ + 4 * c) = pf_q[j] * cl2;
        *reinterpret_cast<f32x4*>(dOt + row * P::LDQ + 4 * c) = pf_o[j];
      }
    }
    const int i = i0 + q;
    const float m2 = pf_m2, invz = pf_invz, dz = pf_d * pf_invz;
    wave_lds_sync();

    // ---- S^T (minus the row shift, folded into the accumulator) and dP^T ----
    // Operands of chunk c+1 are read from LDS before the MFMAs of chunk c issue.
    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[b][r] = -m2;
        pacc[b][r] = 0.f;
      }
    {
      const f32x4* qrow = reinterpret_cast<const f32x4*>(Qt + q * P::LDQ + h * P::DH);
      const f32x4* orow = reinterpret_cast<const f32x4*>(dOt + q * P::LDQ + h * P::DH);
      f32x4 qv_n, ov_n, vv_n[2];
      auto fetch = [&](int c) {
        qv_n = qrow[c];
        ov_n = orow[c];
#pragma unroll
        for (int b = 0; b < 2; ++b)
          vv_n[b] = vsl[vrow[b] * P::C4 + h * P::CH + (c ^ vswz(vrow[b], P::CH))];
      };
      fetch(0);
#pragma unroll
      for (int c = 0; c < P::CH; ++c) {
        const f32x4 qv = qv_n, ov = ov_n, vv0 = vv_n[0], vv1 = vv_n[1];
        if (c + 1 < P::CH) fetch(c + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sacc[0] = mfma32(ka[0][4 * c + e], qv[e], sacc[0]);
          pacc[0] = mfma32(vv0[e], ov[e], pacc[0]);
          sacc[1] = mfma32(ka[1][4 * c + e], qv[e], sacc[1]);
          pacc[1] = mfma32(vv1[e], ov[e], pacc[1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // ---- weights and score gradients of this lane's 32 slots ----
    // Streams over the slots; W overwrites sacc and dS overwrites pacc in place.
    // Tiles that may hold invisible keys (or key 0 / the caps) take the general
    // path; all others need no masks.
    const int kbase = w0 - 1 + 32 * h;  // key of register 0
    const bool need_mask = (w0 == 0) || (w0 + 62 > i0) || (i0 + 32 > T);
    auto segments = [&](auto general_tag) {
      constexpr bool kGeneral = decltype(general_tag)::value;
      auto slot_vis = [&](int n) {
        const int key = kbase + n;
        return !kGeneral || (key >= 0 && key <= i);
      };
      // half 1's first segment starts at half 0's last slot
      float sl, pl, gl;
      {
        const bool v31 = slot_vis(31);
        const float s31 = v31 ? sacc[1][15] : 0.f;
        const float g31 = v31 ? fmaf(pacc[1][15], invz, -dz) : 0.f;
        sl = xhalf(s31);
        pl = fast_exp2(sl);
        gl = xhalf(g31);
      }
      float r_prev = 0.f, dr_prev = 0.f, xl0 = 0.f, xdl0 = 0.f;
      // finalises slot n from its own (s,p,g), incoming right and outgoing left shares
      auto finish = [&](int n, float sv, float pv, float gv, float wv, float dv) {
        if (kGeneral) {
          // half-token caps on the first key and the last visible key (both when i == 0)
          const int key = kbase + n;
          const bool vis = slot_vis(n);
          const float cap = (vis && key == 0 ? 0.5f * pv : 0.f) + (vis && key == i ? 0.5f * pv : 0.f);
          wv += cap;
          dv = fmaf(cap, gv, dv);
        }
        const int slot = 32 * h + n;
        const bool owned = slot >= 1 && slot <= 62;
        dv = owned ? dv : 0.f;
        sacc[n >> 4][n & 15] = owned ? wv * invz : 0.f;
        pacc[n >> 4][n & 15] = dv;
      };
#pragma unroll
      for (int n = 0; n < 32; ++n) {
        const bool vis = slot_vis(n);
        const float sr = vis ? sacc[n >> 4][n & 15] : 0.f;  // s - m2
        const float gr = vis ? fmaf(pacc[n >> 4][n & 15], invz, -dz) : 0.f;
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
          finish(n - 1, sl, pl, gl, r_prev + Lv, dr_prev + dLv);
        }
        r_prev = Rv;
        dr_prev = dRv;
        sl = sr;
        pl = pr;
        gl = gr;
      }
      finish(31, sl, pl, gl, r_prev + (h ? 0.f : xl0), dr_prev + (h ? 0.f : xdl0));
    };
    if (need_mask)
      segments(std::true_type{});
    else
      segments(std::false_type{});

    // ---- dS row block for the dQ pass: row q, slots 32h..32h+31 ----
    {
      float* dst = dsbuf + ((size_t)ds_blk << 11) + q * 64 + 32 * h;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<f32x4*>(dst + 16 * b + 4 * c) =
              f32x4{pacc[b][4 * c], pacc[b][4 * c + 1], pacc[b][4 * c + 2], pacc[b][4 * c + 3]};
      ds_blk += ds_kb_count(qt) + ds_kb_count(qt + 1) + ds_kb_count(qt + 2) + ds_kb_count(qt + 3);
    }

    // ---- transpose through LDS ----
    {
      float* wrow = Wt + q * P::LDW + 32 * h;
      float* drow = dSt + q * P::LDW + 32 * h;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          *reinterpret_cast<f32x4*>(wrow + 16 * b + 4 * c) =
              f32x4{sacc[b][4 * c], sacc[b][4 * c + 1], sacc[b][4 * c + 2], sacc[b][4 * c + 3]};
          *reinterpret_cast<f32x4*>(drow + 16 * b + 4 * c) =
              f32x4{pacc[b][4 * c], pacc[b][4 * c + 1], pacc[b][4 * c + 2], pacc[b][4 * c + 3]};
        }
    }
    wave_lds_sync();
    if (qt + 4 < nqt) prefetch(qt + 4);

    // ---- dV^T += dY^T W,  dK^T += Q^T dS ----
    // Operands of query row r+1 are read from LDS before the MFMAs of row r.
    {
      const int col0 = q < D ? q : 0;
      float ado_n[P::NMB], aq_n[P::NMB], bw_n[2], bd_n[2];
      auto fetch = [&](int r) {
        const int qr = 16 * h + r;
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb) {
          const bool dok = 32 * mb + q < D;
          ado_n[mb] = dok ? dOt[qr * P::LDQ + 32 * mb + col0] : 0.f;
          aq_n[mb] = dok ? Qt[qr * P::LDQ + 32 * mb + col0] : 0.f;
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          bw_n[nb] = Wt[qr * P::LDW + 32 * nb + q];
          bd_n[nb] = dSt[qr * P::LDW + 32 * nb + q];
        }
      };
      fetch(0);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float ado[P::NMB], aq[P::NMB], bw[2], bd[2];
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb) {
          ado[mb] = ado_n[mb];
          aq[mb] = aq_n[mb];
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          bw[nb] = bw_n[nb];
          bd[nb] = bd_n[nb];
        }
        if (r + 1 < 16) fetch(r + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            accv[mb][nb] = mfma32(ado[mb], bw[nb], accv[mb][nb]);
            acck[mb][nb] = mfma32(aq[mb], bd[nb], acck[mb][nb]);
          }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // ---- reduce the 4 waves' partial dV^T / dK^T through LDS ----
  __syncthreads();
  constexpr int NE = P::NMB * 2 * 16;  // accumulator elements per lane per matrix
  float* redv = lds;
  float* redk = lds + 4 * NE * 64;
#pragma unroll
  for (int mb = 0; mb < P::NMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int e = (mb * 2 + nb) * 16 + r;
        redv[(w * NE + e) * 64 + lane] = accv[mb][nb][r];
        redk[(w * NE + e) * 64 + lane] = acck[mb][nb][r];
      }
  __syncthreads();
  // groups of 4 consecutive d (one float4 store) are split across the waves
  constexpr int NG = P::NMB * 2 * 4;
  for (int gi = w; gi < NG; gi += 4) {
    const int mb = gi / 8, nb = (gi / 4) % 2, r4 = gi % 4;
    const int slot = 32 * nb + q;
    const int key = w0 - 1 + slot;
    const int d0 = 32 * mb + 8 * r4 + 4 * h;
    f32x4 sv = {0.f, 0.f, 0.f, 0.f}, sk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < 4; ++ww)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int e = (mb * 2 + nb) * 16 + 4 * r4 + e4;
        sv[e4] += redv[(ww * NE + e) * 64 + lane];
        sk[e4] += redk[(ww * NE + e) * 64 + lane];
      }
    if (slot >= 1 && slot <= 62 && key < T && d0 < D) {
      *reinterpret_cast<f32x4*>(dV + slice + (size_t)key * D + d0) = sv;
      *reinterpret_cast<f32x4*>(dK + slice + (size_t)key * D + d0) = sk * kLn2;
    }
  }
}

// dQ = c dS K as a tiled GEMM over the dS row blocks written by ca_bwd_dkdv.
// Work group: 64 queries (two 32-query tiles) of one slice.  Per key block kb
// the 64 K rows of its slots (keys 62kb-1 .. 62kb+62) are staged in LDS
// (double-buffered) and shared by all four waves: wave w takes query tile
// w&1 and the slot half w>>1 of the MFMA k-range (lane half h supplies slots
// 32h + s at k-step s).  Halo slots and invisible keys carry dS = 0, so no
// masks are needed.  The dS operand of the next block is prefetched into
// registers.  The two halves are summed through LDS at the end (fixed
// order), and the epilogue writes the work group's gain partial
// sum_i q_i . dQ_i (fixed order).
template <int D>
__global__ __launch_bounds__(256) void ca_bwd_dq_kernel(const float* __restrict__ dsbuf,
                                                        const float* __restrict__ Q,
                                                        const float* __restrict__ K,
                                                        const float* __restrict__ log_gain,
                                                        float* __restrict__ dQ,
                                                        float* __restrict__ gain_part, int BH,
                                                        int H, int T) {
  using P = Bwd<D>;
  constexpr int KF4 = 64 * P::C4;                     // float4 per 64-row K stage
  constexpr int KLD = (KF4 + 255) / 256;              // float4 loads per thread
  constexpr int RED4 = 2 * P::NMB * 16 * 64 / 4;      // float4 of the final parity reduction
  // The K stages and the final reduction buffer are live at disjoint times and
  // share one allocation (fewer LDS bytes per work group, more resident groups).
  __shared__ f32x4 smem[2 * KF4 > RED4 ? 2 * KF4 : RED4];
  f32x4 (*kst)[KF4] = reinterpret_cast<f32x4 (*)[KF4]>(smem);
  float* red = reinterpret_cast<float*>(smem);
  __shared__ float gred[2];
  const int nqt = num_q_tiles(T);
  const int nqg = dq_num_groups(T);
  const int nkb = bwd_num_key_blocks(T);
  const int bh = blockIdx.x % BH;
  const int qg = nqg - 1 - blockIdx.x / BH;  // heaviest (longest rows) first
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, q = lane & 31, h = lane >> 5;
  const int qsub = w & 1, par = w >> 1;
  const int qt = 2 * qg + qsub;
  const bool wave_on = qt < nqt;
  const size_t slice = (size_t)bh * T * D;
  const float c = head_scale_log2(log_gain, bh % H, D) * kLn2;
  // key blocks met by this wave's tile and by the work group's last tile
  const int my_kb = wave_on ? min(ds_kb_count(qt), nkb) : 0;
  const int iters = min(ds_kb_count(min(2 * qg + 1, nqt - 1)), nkb);
  const float* arow = dsbuf +
                      (((size_t)bh * ds_blocks_before(nqt) + ds_blocks_before(wave_on ? qt : 0)) << 11) +
                      q * 64 + 32 * h + 16 * par;

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
  // the same accuracy.
  f32x4 kref[KLD];
  {
    const f32x4* kr = reinterpret_cast<const f32x4*>(K + slice + (size_t)(64 * qg) * D);
#pragma unroll
    for (int j = 0; j < KLD; ++j) kref[j] = kr[(tid + 256 * j) % P::C4];
  }
  f32x4 pre[KLD];
  auto load_k = [&](int kb) {
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      const int e = tid + 256 * j;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (e < KF4) {
        const int key = kBwdKeys * kb - 1 + e / P::C4;
        if (key >= 0 && key < T)
          v = reinterpret_cast<const f32x4*>(K + slice + (size_t)key * D)[e % P::C4];
      }
      pre[j] = v;
    }
  };
  // the shift is applied when the prefetched rows are stored, so the loads
  // issued a block ahead are not waited for inside the MFMA loop
  auto store_k = [&](int buf) {
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      const int e = tid + 256 * j;
      if (e < KF4) kst[buf][e] = pre[j] - kref[j];
    }
  };
  auto load_a = [&](int kb, float* a) {
    const f32x4* src = reinterpret_cast<const f32x4*>(arow + ((size_t)kb << 11));
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const f32x4 v4 = src[c4];
      a[4 * c4 + 0] = v4[0]; a[4 * c4 + 1] = v4[1]; a[4 * c4 + 2] = v4[2]; a[4 * c4 + 3] = v4[3];
    }
  };

  float a_next[16];
  if (my_kb > 0) load_a(0, a_next);
  load_k(0);
  store_k(0);
  __syncthreads();
  const int dcol = (q < D) ? q : 0;
  for (int it = 0; it < iters; ++it) {
    const int buf = it & 1;
    if (it + 1 < iters) load_k(it + 1);
    if (it < my_kb) {
      float a[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) a[r] = a_next[r];
      if (it + 1 < my_kb) load_a(it + 1, a_next);
      const float* kb = reinterpret_cast<const float*>(&kst[buf][0]) + (32 * h + 16 * par) * D + dcol;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int nb = 0; nb < P::NMB; ++nb) {
          const float b = (32 * nb + q < D) ? kb[r * D + 32 * nb] : 0.f;
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
#pragma unroll
      for (int nb = 0; nb < P::NMB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float sum = acc[nb][r] + red[((qsub * P::NMB + nb) * 16 + r) * 64 + lane];
          const int row = 32 * qt + 8 * (r >> 2) + 4 * h + (r & 3);
          const int d = 32 * nb + q;
          const float val = sum * c;
          g = fmaf(qv[nb][r], val, g);
          if (row < T && d < D) dQ[slice + (size_t)row * D + d] = val;
        }
    }
    g = wave_sum(g);
    if (lane == 0) gred[qsub] = g;
  }
  __syncthreads();
  if (tid == 0) gain_part[(size_t)bh * nqg + qg] = gred[0] + gred[1];
}

// dRho_h = sum over batch and query groups of the per-group partials; one
// wave per head, fixed summation order.
__global__ __launch_bounds__(64) void ca_bwd_gain_kernel(const float* __restrict__ gain_part,
                                                         float* __restrict__ dlog_gain, int B,
                                                         int H, int ngroups) {
  const int h = blockIdx.x;
  const int lane = threadIdx.x;
  float acc = 0.f;
  for (int b = 0; b < B; ++b)
    for (int k = lane; k < ngroups; k += 64) acc += gain_part[((size_t)b * H + h) * ngroups + k];
  acc = wave_sum(acc);
  if (lane == 0) dlog_gain[h] = acc;
}

template <int D>
hipError_t launch_bwd(const float* q, const float* k, const float* v, const float* log_gain,
                      const float* o, const float* stats, const float* dout, float* dq, float* dk,
                      float* dv, float* dlog_gain, float* dsbuf, float* dvec, float* gain_part,
                      int B, int H, int T, hipStream_t stream) {
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
  const int nqg = dq_num_groups(T);
  hipLaunchKernelGGL(ca_bwd_dq_kernel<D>, dim3(nqg * BH), dim3(256), 0, stream, dsbuf, q, k,
                     log_gain, dq, gain_part, BH, H, T);
  timer_end(kBwdDq, stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(kBwdGain, stream);
  hipLaunchKernelGGL(ca_bwd_gain_kernel, dim3(H), dim3(64), 0, stream, gain_part, dlog_gain, B,
                     H, nqg);
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
                                     float*, float*, float*, float*, float*, int, int, int,    \
                                     hipStream_t);
CA_INST_BWD(8)
CA_INST_BWD(16)
CA_INST_BWD(32)
CA_INST_BWD(64)

}  // namespace ca
