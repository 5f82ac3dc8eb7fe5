// Weight-materialising CA kernels: exact weights W (and their score VJP) from
// a materialised block of scores.  These are the row kernels behind the
// reference's ext.forward(scores, start) -> [W, stats] and
// ext.backward_fused(scores, gw, start) -> [W, dS]
// (cuda/continuum_attention.py:136-163, 230-293, 538-554, 578-590), used for
// weight-level diagnostics and for continuous_attention_weights(logits)
// (architecture.py:65-105) on the GPU.  The fused operator kernels never
// materialise W; these do, so they are HBM-bound row passes.
//
// Layout: scores, grad_weights, weights and grad_scores are [rows][K] fp32,
// rows = BH * Q, row r is query start + (r % Q) of slice r / Q and sees keys
// 0 .. start + r % Q (the host checks start + Q <= K).  stats is
// [rows][2] = (row max m, 1/Z) in natural units, as the reference's.
//
// One wave per row, four rows per 256-thread work group.  Lane l of step t
// owns key j = 64 t + l and evaluates the segment (j, j+1) once: its left
// share stays with key j and its right share moves to key j+1 with one lane
// shift.  Scores are read coalesced; neighbours come from lane shuffles (the
// next step's first score is prefetched for lane 63).  Three passes over the
// row (max; Z and, for the VJP, sum_j w_j gw_j; weights / gradients), so the
// row is read from HBM once and re-read from cache.
#include "ca_common.h"
#include "ca_kernels.h"

namespace ca {

namespace {

// Score (or weight gradient) of key j, or `fill` past the visible prefix.
// Invisible scores read as the row max, so every exponent stays finite; their
// terms are masked.
__device__ __forceinline__ float load_or(const float* p, int j, int n, float fill) {
  return j < n ? p[j] : fill;
}

}  // namespace

template <bool kBwd>
__global__ __launch_bounds__(256) void ca_weights_rows_kernel(
    const float* __restrict__ scores, const float* __restrict__ gw, float* __restrict__ W,
    float* __restrict__ dS, float* __restrict__ stats, int rows, int Q, int K, int start) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave; no work-group barrier below
  const int query = start + row % Q;
  const int nvis = query + 1;  // keys 0 .. query
  const size_t off = (size_t)row * K;
  const float* s = scores + off;
  const float* g = kBwd ? gw + off : nullptr;

  // pass 1: row max over the visible keys
  float m = kNegBig;
  for (int j = lane; j < nvis; j += 64) m = fmaxf(m, s[j]);
  m = wave_max(m);

  // Segment (j, j+1) of one step: shares L (to j) and R (to j+1), and the
  // endpoint weights p_j, p_{j+1}.
  auto step_shares = [&](int j0, float cur, float nxt, float& pl, float& L, float& R) {
    const int j = j0 + lane;
    float sr = __shfl_down(cur, 1);
    const float first_next = __shfl(nxt, 0);
    if (lane == 63) sr = first_next;
    pl = fast_exp2((cur - m) * kLog2e);
    const float pr = fast_exp2((sr - m) * kLog2e);
    seg_shares_x(sr - cur, pl, pr, L, R);
    const bool seg_vis = j + 1 < nvis;
    L = seg_vis ? L : 0.f;
    R = seg_vis ? R : 0.f;
  };

  // pass 2: Z = sum_j w_j and (VJP) P = sum_j w_j gw_j
  float z = 0.f, pg = 0.f;
  {
    float cur = load_or(s, lane, nvis, m);
    float carry = 0.f;  // right share arriving at key j0 from segment (j0-1, j0)
    for (int j0 = 0; j0 < nvis; j0 += 64) {
      const int j = j0 + lane;
      const float nxt = load_or(s, j + 64, nvis, m);
      float pl, L, R;
      step_shares(j0, cur, nxt, pl, L, R);
      float rin = __shfl_up(R, 1);
      const float last_r = __shfl(R, 63);
      if (lane == 0) rin = carry;
      carry = last_r;
      float w = L + rin + ((j == 0) ? 0.5f * pl : 0.f) + ((j == query) ? 0.5f * pl : 0.f);
      w = (j < nvis) ? w : 0.f;
      z += w;
      if (kBwd) pg = fmaf(w, load_or(g, j, nvis, 0.f), pg);
      cur = nxt;
    }
  }
  z = wave_sum(z);
  const float inv_z = 1.0f / z;
  const float dmean = kBwd ? wave_sum(pg) * inv_z : 0.f;  // D = sum_j W_j gw_j

  // pass 3: normalised weights and (VJP) dS
  {
    float cur = load_or(s, lane, nvis, m);
    float gcur = kBwd ? (load_or(g, lane, nvis, 0.f) - dmean) * inv_z : 0.f;
    float carry = 0.f, dcarry = 0.f;
    for (int j0 = 0; j0 < nvis; j0 += 64) {
      const int j = j0 + lane;
      const float nxt = load_or(s, j + 64, nvis, m);
      float pl, L, R;
      if (!kBwd) {
        step_shares(j0, cur, nxt, pl, L, R);
      } else {
        // centred, 1/Z-scaled weight gradient of the right key
        const float gnxt = (load_or(g, j + 64, nvis, 0.f) - dmean) * inv_z;
        float gr = __shfl_down(gcur, 1);
        const float gfirst = __shfl(gnxt, 0);
        if (lane == 63) gr = gfirst;
        float sr = __shfl_down(cur, 1);
        const float first_next = __shfl(nxt, 0);
        if (lane == 63) sr = first_next;
        pl = fast_exp2((cur - m) * kLog2e);
        const float pr = fast_exp2((sr - m) * kLog2e);
        float dL, dR;
        seg_shares_grad_x(sr - cur, pl, pr, gcur, gr, L, R, dL, dR);
        const bool seg_vis = j + 1 < nvis;
        L = seg_vis ? L : 0.f;
        R = seg_vis ? R : 0.f;
        dL = seg_vis ? dL : 0.f;
        dR = seg_vis ? dR : 0.f;
        float din = __shfl_up(dR, 1);
        const float last_d = __shfl(dR, 63);
        if (lane == 0) din = dcarry;
        dcarry = last_d;
        const float caps = ((j == 0) ? 0.5f : 0.f) + ((j == query) ? 0.5f : 0.f);
        const float ds = fmaf(caps * pl, gcur, dL + din);
        if (j < nvis) dS[off + j] = ds;
        gcur = gnxt;
      }
      float rin = __shfl_up(R, 1);
      const float last_r = __shfl(R, 63);
      if (lane == 0) rin = carry;
      carry = last_r;
      const float w = L + rin + ((j == 0) ? 0.5f * pl : 0.f) + ((j == query) ? 0.5f * pl : 0.f);
      if (j < nvis && W) W[off + j] = w * inv_z;
      cur = nxt;
    }
  }
  // future keys: exact zeros
  for (int j = nvis + lane; j < K; j += 64) {
    if (W) W[off + j] = 0.f;
    if (kBwd) dS[off + j] = 0.f;
  }
  if (!kBwd && lane == 0) {
    stats[2 * (size_t)row + 0] = m;
    stats[2 * (size_t)row + 1] = inv_z;
  }
}

hipError_t launch_weights(const float* scores, float* weights, float* stats, int BH, int Q, int K,
                          int start, hipStream_t stream) {
  const int rows = BH * Q;
  hipLaunchKernelGGL(ca_weights_rows_kernel<false>, dim3((rows + 3) / 4), dim3(256), 0, stream,
                     scores, nullptr, weights, nullptr, stats, rows, Q, K, start);
  return hipGetLastError();
}

hipError_t launch_weights_bwd(const float* scores, const float* grad_weights, float* weights,
                              float* grad_scores, int BH, int Q, int K, int start,
                              hipStream_t stream) {
  const int rows = BH * Q;
  hipLaunchKernelGGL(ca_weights_rows_kernel<true>, dim3((rows + 3) / 4), dim3(256), 0, stream,
                     scores, grad_weights, weights, grad_scores, nullptr, rows, Q, K, start);
  return hipGetLastError();
}

}  // namespace ca
