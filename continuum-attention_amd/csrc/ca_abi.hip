// C ABI of libca_hip.so: plain pointers, sizes and a HIP stream handle.
// Declarations and the reference interfaces they replace: include/continuum_attention_amd.h.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <vector>

#include "../../include/continuum_attention_amd.h"
#include "ca_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// The forward workspace is sized for the split ca::fwd_split_tiles picks when
// this many work groups are resident (the shortest the device can pick), so
// its size is a function of the shape alone.
constexpr int kFwdSplitBound = 1024;

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

int ca::check_shape(int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0 || D <= 0)
    return fail(CA_ERR_INVALID, "invalid shape B=%d H=%d T=%d D=%d (all must be positive)", B, H,
                T, D);
  if (D != 8 && D != 16 && D != 32 && D != 64 && D != 128)
    return fail(CA_ERR_UNSUPPORTED, "head dim D=%d not supported (HIP kernels cover D in {8,16,32,64,128})", D);
  if ((long long)B * H * T * D > (1ll << 31) - 1)
    return fail(CA_ERR_UNSUPPORTED, "tensor of %lld elements exceeds the 2^31 element limit",
                (long long)B * H * T * D);
  if (T > 65536) return fail(CA_ERR_UNSUPPORTED, "T=%d exceeds the supported 65536", T);
  return CA_OK;
}

namespace {
using ca::check_shape;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The dQ and dK/dV passes split their work items when their grids would not
// fill the device (ca::dq_split, ca::dkdv_split).  The workspace is sized as
// if kDqSplitBound work groups were resident, so its size does not depend on
// the device; the device's own resident counts (at most this bound) pick the
// splits.
constexpr int kDqSplitBound = 2048;

int dkdv_resident_groups() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  const int r = std::min(cus * ca::kDkdvGroupsPerCu, kDqSplitBound);
  if (dev >= 0 && dev < 64) cache[dev].store(r, std::memory_order_relaxed);
  return r;
}

// forward work groups resident on the current device (2 per CU, 1 for D > 64)
int fwd_resident_groups(int D) {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  int cus = 0;
  if (dev >= 0 && dev < 64) cus = cache[dev].load(std::memory_order_relaxed);
  if (!cus) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev >= 0 && dev < 64) cache[dev].store(cus, std::memory_order_relaxed);
  }
  return std::min(cus * (D > 64 ? 1 : 2), kFwdSplitBound);
}

int dq_resident_groups() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  const int r = std::min(cus * ca::kDqGroupsPerCu, kDqSplitBound);
  if (dev >= 0 && dev < 64) cache[dev].store(r, std::memory_order_relaxed);
  return r;
}

// Forced split lengths (ca_debug_set_splits; 0 = automatic).  When one is
// set, the workspace sizes and the launches both use it, so the two agree.
struct SplitOverride {
  int fwd_tiles = 0, dq_stages = 0, dkdv_tiles = 0;
};
SplitOverride g_split;

// Workspace cap (ca_set_workspace_cap): the size the workspace-size functions
// report when the full (single-pass, shortest-split) workspace is larger;
// 0 means no cap.
size_t g_workspace_cap = size_t(1) << 30;

// Forward split length for a workspace of `bytes`: the device's own choice
// (for_sizing: the shortest any device can pick), lengthened until the split
// partials fit; a split as long as the longest row needs no partials.
int fwd_split(int BH, int T, int D, bool for_sizing, size_t bytes = SIZE_MAX) {
  if (g_split.fwd_tiles > 0) return g_split.fwd_tiles;
  const int C = ca::fwd_split_tiles(BH, T, for_sizing ? kFwdSplitBound : fwd_resident_groups(D));
  if (ca::fwd_part_floats(BH, T, C, D) * sizeof(float) <= bytes) return C;
  const int G = (T + 127) / 128;
  const int max_tiles = ca::fwd_group_tiles(G - 1, T);
  const size_t per_split = (size_t)BH * T * (D + 2) * sizeof(float);
  const size_t fit = bytes / per_split;  // splits the partials can hold
  if (fit < 2) return max_tiles;
  const int cf = (int)((max_tiles + fit - 1) / fit);
  return cf > C ? cf : C;
}
ca::DqSplit dq_split_for(int BH, int T, int D, const ca::BwdPass& p, bool for_sizing) {
  if (g_split.dq_stages > 0) return ca::dq_split_chunk(T, p, g_split.dq_stages);
  // D = 128 kernels hold fewer dQ work groups per CU (two instead of three)
  const int res = for_sizing ? kDqSplitBound : (D > 64 ? dq_resident_groups() * 2 / 3 : dq_resident_groups());
  return ca::dq_split(BH, T, p, res);
}
ca::DkdvSplit dkdv_split_for(int BH, int D, int dtype, const ca::BwdPass& p, bool for_sizing) {
  if (g_split.dkdv_tiles > 0) return ca::dkdv_split_chunk(p, g_split.dkdv_tiles);
  // D = 128: one dK/dV work group per CU instead of two (registers and LDS).
  // bf16 operands at D <= 64: three per CU, and the split test asks for 1.5
  // rounds of them (9/4 of the two-per-CU count; at [1,16,2048,64] chunks of
  // 16 tiles took 0.277 ms per fwd+bwd against 0.283 ms for 24 and 0.281 ms
  // for 12).
  // fp32 operands at D = 64 (the single-buffered kernel, three per CU): split
  // only below 1.5 rounds of three per CU (config 2, 37 key groups x 32
  // slices, stays unsplit: 24-tile chunks made dK/dV 8 us faster and the
  // dQ launch, which merges their partials, 13 us slower), then from 16-tile
  // chunks down until one round is filled.  Kernel time per fwd+bwd
  // (rocprof, sum of the operator's kernels) against the earlier rule (1.5
  // rounds, from 24 tiles): [16,4,512,64] (one CA-P layer) 125.1 -> 117.4 us
  // (12-tile chunks instead of 6), [2,8,1024,64] 118.5 -> 111.8 us,
  // [1,16,1024,64] 118.3 -> 112.2 us, [4,8,700,64] 119.1 -> 114.4 us,
  // [1,32,1500,64] 368.4 -> 354.2 us (16 instead of 24), but [2,4,2048,64]
  // 176.8 -> 183.3 us (12 instead of 8); config 2, config 5 and
  // [1,16,2048,64] keep their lengths.  The workspace is
  // sized for chunks from kDkdvChunkTiles down (for_sizing), so a shorter
  // first chunk is taken only where its items and partials fit that size;
  // elsewhere the earlier rule applies.
  int res = kDqSplitBound;
  long long want = -1;
  if (!for_sizing) {
    const int two_per_cu = dkdv_resident_groups();
    if (D > 64) {
      res = two_per_cu / 2;
    } else if (dtype == CA_DTYPE_BF16) {
      res = std::min(two_per_cu * 9 / 4, kDqSplitBound);
    } else if (dtype == CA_DTYPE_F32 && D == 64) {
      res = std::min(two_per_cu * 9 / 4, kDqSplitBound);
      want = res;
      const ca::DkdvSplit s =
          ca::dkdv_split(BH, p, std::min(two_per_cu * 3 / 2, kDqSplitBound), want, 16);
      const ca::DkdvSplit sized = dkdv_split_for(BH, D, dtype, p, true);
      if (s.items <= sized.items && s.part_items <= sized.part_items) return s;
    } else {
      res = two_per_cu;
    }
  }
  return ca::dkdv_split(BH, p, res, want);
}

// Workspace layout of one backward pass (every pass lays its buffers out from
// the start of the workspace; nothing in it outlives the pass).
struct BwdLayout {
  size_t ds, limbs, qstat, gain, dqpart, kvpart, total;
};
BwdLayout bwd_layout(int B, int H, int T, int D, const ca::BwdPass& p) {
  const int BH = B * H;
  const ca::DqSplit sp = dq_split_for(BH, T, D, p, true);  // the largest split
  const ca::DkdvSplit kvs = dkdv_split_for(BH, D, CA_DTYPE_F32, p, true);
  BwdLayout L;
  L.ds = 0;
  L.limbs = align256((size_t)BH * p.ds_slice * sizeof(float));
  L.qstat = L.limbs + align256(ca::bwd_limb_elems(BH, p, D) * sizeof(uint16_t));
  L.gain = L.qstat + align256(ca::bwd_qstat_floats(BH, p) * sizeof(float));
  L.dqpart = L.gain + align256((size_t)BH * kvs.items * sizeof(float));
  L.kvpart = L.dqpart + align256((size_t)BH * sp.part_items * ca::kDqRows * D * sizeof(float));
  L.total = L.kvpart + align256((size_t)BH * kvs.part_items * ca::kDkdvKeys * 2 * D * sizeof(float));
  return L;
}
size_t bwd_full_bytes(int B, int H, int T, int D) {
  return bwd_layout(B, H, T, D, ca::bwd_pass(T, 0, ca::dq_num_groups(T))).total;
}
// Room for the rotated keys of the token-major entry points ([B*H][T][D],
// 4-byte elements: enough for every operand type).
size_t rotated_keys_bytes(int B, int H, int T, int D) {
  return align256((size_t)B * H * T * D * sizeof(float));
}

// Backward passes for a workspace of `bytes`: ranges of dQ groups from the
// first on, each as long as its layout fits (a layout only grows when its
// range does).  False when a single group does not fit.
bool plan_passes(int B, int H, int T, int D, size_t bytes, std::vector<ca::BwdPass>* passes) {
  const int G = ca::dq_num_groups(T);
  passes->clear();
  int g0 = 0;
  while (g0 < G) {
    if (bwd_layout(B, H, T, D, ca::bwd_pass(T, g0, g0 + 1)).total > bytes) return false;
    int lo = g0 + 1, hi = G;  // largest g1 in [lo, hi] that fits
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (bwd_layout(B, H, T, D, ca::bwd_pass(T, g0, mid)).total <= bytes) lo = mid;
      else hi = mid - 1;
    }
    passes->push_back(ca::bwd_pass(T, g0, lo));
    g0 = lo;
  }
  return true;
}

// Bytes of the fp32 dK and dV sums of `slices` slices, which the token-major
// backward keeps at the start of its workspace when it runs in passes.
size_t kv_sum_bytes(int slices, int T, int D) {
  return 2 * align256((size_t)slices * T * D * sizeof(float));
}

// A backward plan.  The slices run as one set (every slice) or, when not even
// one 128-query group of every slice fits, as sets of consecutive heads of
// one batch: slices are independent, so a set is the backward of a
// [1, nh, T, D] sub-problem, and its workspace grows with nh instead of B*H.
// Each set runs in passes over ranges of 128-query groups.  With kv_sums,
// the set's dK and dV are summed over its passes in fp32 (kv_sum_bytes at
// the start of the workspace, the passes' buffers after them).
struct BwdPlan {
  int hc = 0;                            // heads per set; 0: one set of every slice
  std::vector<ca::BwdPass> passes;       // passes of a set of hc heads (or of the one set)
  int tail = 0;                          // heads of each batch's last set when fewer than hc
  std::vector<ca::BwdPass> tail_passes;  // and its passes
  size_t need = 0;                       // the most workspace any pass of the plan uses
};
size_t passes_need(int B, int H, int T, int D, const std::vector<ca::BwdPass>& passes) {
  size_t need = 0;
  for (const auto& p : passes) need = std::max(need, bwd_layout(B, H, T, D, p).total);
  return need;
}
// The plan for a workspace of `bytes`: every slice in one set if one group of
// each fits, else the fewest head sets (of near-equal sizes) that fit.  False
// when not even one group of one slice fits.
bool plan_bwd(int B, int H, int T, int D, size_t bytes, bool kv_sums, BwdPlan* plan) {
  auto extra = [&](int slices) { return kv_sums ? kv_sum_bytes(slices, T, D) : size_t(0); };
  *plan = BwdPlan();
  if (bytes > extra(B * H) && plan_passes(B, H, T, D, bytes - extra(B * H), &plan->passes)) {
    plan->need = extra(B * H) + passes_need(B, H, T, D, plan->passes);
    return true;
  }
  for (int hc = H; hc >= 1; --hc) {
    if (bytes <= extra(hc)) continue;
    const int nsets = (H + hc - 1) / hc;
    const int hb = (H + nsets - 1) / nsets;  // <= hc
    const int tail = H - (nsets - 1) * hb;   // <= hb
    *plan = BwdPlan();
    if (!plan_passes(1, hb, T, D, bytes - extra(hb), &plan->passes)) continue;
    plan->hc = hb;
    plan->need = extra(hb) + passes_need(1, hb, T, D, plan->passes);
    if (tail != hb) {
      if (!plan_passes(1, tail, T, D, bytes - extra(tail), &plan->tail_passes)) continue;
      plan->tail = tail;
      plan->need = std::max(plan->need, extra(tail) + passes_need(1, tail, T, D, plan->tail_passes));
    }
    return true;
  }
  *plan = BwdPlan();
  return false;
}

// Workspace the backward asks for under the cap: the full one when it fits
// (without kv_sums), else the need of the plan for the cap, or, when no plan
// fits under the cap, the least any plan needs (sets of one head, one
// 128-query group per pass).
size_t bwd_capped_bytes(int B, int H, int T, int D, bool kv_sums) {
  if (!kv_sums) {
    const size_t full = bwd_full_bytes(B, H, T, D);
    if (g_workspace_cap == 0 || full <= g_workspace_cap) return full;
  }
  BwdPlan plan;
  if (plan_bwd(B, H, T, D, g_workspace_cap ? g_workspace_cap : SIZE_MAX, kv_sums, &plan))
    return plan.need;
  size_t need = 0;
  for (int g = 0; g < ca::dq_num_groups(T); ++g)
    need = std::max(need, bwd_layout(1, 1, T, D, ca::bwd_pass(T, g, g + 1)).total);
  return need + (kv_sums ? kv_sum_bytes(1, T, D) : 0);
}

// ---- per-kernel event timing ------------------------------------------------
struct TimedLaunch {
  int id;
  hipEvent_t start, stop;
};
bool g_timing = false;
std::vector<TimedLaunch> g_launches;  // recorded, not yet read
std::vector<hipEvent_t> g_event_pool;
int g_open_id = -1;
hipEvent_t g_open_start = nullptr;

hipEvent_t pool_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

namespace ca {
bool bwd_fits(int B, int H, int T, int D, size_t bytes) {
  BwdPlan plan;
  return plan_bwd(B, H, T, D, bytes, false, &plan);
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void timer_begin(int id, hipStream_t s) {
  if (!g_timing) return;
  g_open_start = pool_event();
  g_open_id = id;
  if (g_open_start) (void)hipEventRecord(g_open_start, s);
}
void timer_end(int id, hipStream_t s) {
  if (!g_timing || g_open_id != id || !g_open_start) return;
  hipEvent_t stop = pool_event();
  if (!stop) return;
  (void)hipEventRecord(stop, s);
  g_launches.push_back({id, g_open_start, stop});
  g_open_start = nullptr;
  g_open_id = -1;
}
}  // namespace ca

extern "C" {

int ca_timing_enable(int on) {
  g_timing = on != 0;
  for (auto& l : g_launches) {
    g_event_pool.push_back(l.start);
    g_event_pool.push_back(l.stop);
  }
  g_launches.clear();
  return CA_OK;
}

int ca_timing_read(double* total_ms, int* launches, int n) {
  if (!total_ms || !launches || n <= 0) return fail(CA_ERR_INVALID, "ca_timing_read: bad buffers");
  for (int i = 0; i < n; ++i) {
    total_ms[i] = 0.0;
    launches[i] = 0;
  }
  for (auto& l : g_launches) {
    hipError_t e = hipEventSynchronize(l.stop);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, l.start, l.stop);
    if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_timing_read: %s", hipGetErrorString(e));
    if (l.id < n) {
      total_ms[l.id] += ms;
      launches[l.id] += 1;
    }
    g_event_pool.push_back(l.start);
    g_event_pool.push_back(l.stop);
  }
  g_launches.clear();
  return CA_OK;
}


int ca_debug_set_splits(int fwd_split_tiles, int dq_chunk_stages, int dkdv_chunk_tiles) {
  if (fwd_split_tiles < 0 || dq_chunk_stages < 0 || dkdv_chunk_tiles < 0)
    return fail(CA_ERR_INVALID, "ca_debug_set_splits: lengths must be >= 0 (0 = automatic)");
  g_split.fwd_tiles = fwd_split_tiles;
  g_split.dq_stages = dq_chunk_stages;
  g_split.dkdv_tiles = dkdv_chunk_tiles;
  return CA_OK;
}

int ca_abi_version(void) { return CA_ABI_VERSION; }

const char* ca_last_error(void) { return g_err; }

int ca_set_workspace_cap(size_t bytes) {
  g_workspace_cap = bytes;
  return CA_OK;
}

size_t ca_workspace_cap(void) { return g_workspace_cap; }

size_t ca_fwd_workspace_bytes(int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0) return 0;
  const size_t cap = g_workspace_cap ? g_workspace_cap : SIZE_MAX;
  return ca::fwd_part_floats(B * H, T, fwd_split(B * H, T, D, true, cap), D) * sizeof(float);
}

size_t ca_bwd_workspace_bytes(int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0 || D <= 0) return 0;
  return bwd_capped_bytes(B, H, T, D, false);
}

// The token-major entry points add room for the keys rotated once when that
// fits under the cap (their kernels otherwise rotate each staged key tile).
size_t ca_fwd_qkv_workspace_bytes(int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0 || D <= 0) return 0;
  const size_t fwd = ca_fwd_workspace_bytes(B, H, T, D);
  const size_t with_keys = rotated_keys_bytes(B, H, T, D) + fwd;
  return g_workspace_cap == 0 || with_keys <= g_workspace_cap ? with_keys : fwd;
}

// One pass (gradients written in the element type) when it fits under the
// cap, with the rotated keys when they fit too; else passes, with dK and dV
// summed over them in fp32 in the workspace.
size_t ca_bwd_qkv_workspace_bytes(int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0 || D <= 0) return 0;
  const size_t full = bwd_full_bytes(B, H, T, D);
  const size_t with_keys = rotated_keys_bytes(B, H, T, D) + full;
  if (g_workspace_cap == 0 || with_keys <= g_workspace_cap) return with_keys;
  if (full <= g_workspace_cap) return full;
  return std::min(full, bwd_capped_bytes(B, H, T, D, true));
}

}  // extern "C"

namespace {

template <class E>
hipError_t fwd_launch(int D, const ca::FwdIO& io, float* part, int B, int H, int T, int C,
                      hipStream_t s) {
  switch (D) {
    case 8: return ca::launch_fwd<8, E>(io, part, B, H, T, C, s);
    case 16: return ca::launch_fwd<16, E>(io, part, B, H, T, C, s);
    case 32: return ca::launch_fwd<32, E>(io, part, B, H, T, C, s);
    case 64: return ca::launch_fwd<64, E>(io, part, B, H, T, C, s);
    default: return ca::launch_fwd<128, E>(io, part, B, H, T, C, s);
  }
}

template <class E>
hipError_t bwd_launch(int D, const ca::BwdIO& io, const ca::BwdWork& w, const ca::BwdPass& p,
                      const ca::DqSplit& sp, const ca::DkdvSplit& kvs, int B, int H, int T,
                      hipStream_t s) {
  switch (D) {
    case 8: return ca::launch_bwd<8, E>(io, w, p, sp, kvs, B, H, T, s);
    case 16: return ca::launch_bwd<16, E>(io, w, p, sp, kvs, B, H, T, s);
    case 32: return ca::launch_bwd<32, E>(io, w, p, sp, kvs, B, H, T, s);
    case 64: return ca::launch_bwd<64, E>(io, w, p, sp, kvs, B, H, T, s);
    default: return ca::launch_bwd<128, E>(io, w, p, sp, kvs, B, H, T, s);
  }
}

// [B,H,T,D] tensor (element units, any element type) as a view
ca::View heads_view(const void* p, int H, int T, int D) {
  return ca::View{const_cast<void*>(p), (long long)H * T * D, (long long)T * D, (long long)D};
}
size_t dtype_size(int dtype) { return dtype == CA_DTYPE_F32 ? 4 : 2; }

template <class E>
hipError_t rope_keys_launch(int D, const ca::View& k, const float* rope, void* out, int BH, int H,
                            int T, hipStream_t s) {
  switch (D) {
    case 8: return ca::launch_rope_keys<8, E>(k, rope, out, BH, H, T, s);
    case 16: return ca::launch_rope_keys<16, E>(k, rope, out, BH, H, T, s);
    case 32: return ca::launch_rope_keys<32, E>(k, rope, out, BH, H, T, s);
    case 64: return ca::launch_rope_keys<64, E>(k, rope, out, BH, H, T, s);
    default: return ca::launch_rope_keys<128, E>(k, rope, out, BH, H, T, s);
  }
}

// The token-major entry points with RoPE rotate the keys once, into the
// start of their workspace ([B*H][T][D] in the operand type, room for 4-byte
// elements), when it has that room besides what the operator needs (the
// callers check): their kernels then read the keys unrotated instead of
// rotating every staged key tile (the forward and the dQ pass stage each
// tile for many query groups).  Advances *ws / *bytes past the rotated keys.
// Without RoPE: nothing.
int rotate_keys_first(ca::View* k, bool* k_rotated, const float* rope, int dtype, char** ws,
                      size_t* bytes, int B, int H, int T, int D, void* stream) {
  const size_t need = rotated_keys_bytes(B, H, T, D);
  if (!rope || !*ws || *bytes < need) return CA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == CA_DTYPE_BF16) e = rope_keys_launch<__bf16>(D, *k, rope, *ws, B * H, H, T, s);
  else if (dtype == CA_DTYPE_F16) e = rope_keys_launch<_Float16>(D, *k, rope, *ws, B * H, H, T, s);
  else e = rope_keys_launch<float>(D, *k, rope, *ws, B * H, H, T, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "key rotation launch: %s", hipGetErrorString(e));
  *k = heads_view(*ws, H, T, D);
  *k_rotated = true;
  *ws += need;
  *bytes -= need;
  return CA_OK;
}

// Shape, workspace and launch of the forward, once the operands are views.
int fwd_common(const ca::FwdIO& io, int dtype, void* workspace, size_t workspace_bytes, int B,
               int H, int T, int D, void* stream) {
  // the device's own split, lengthened until its partials fit the workspace
  const size_t bytes = workspace ? workspace_bytes : 0;
  const int C = fwd_split(B * H, T, D, false, bytes);
  const size_t need = ca::fwd_part_floats(B * H, T, C, D) * sizeof(float);
  if (bytes < need)
    return fail(CA_ERR_WORKSPACE, "forward workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  hipError_t e;
  if (dtype == CA_DTYPE_BF16) e = fwd_launch<__bf16>(D, io, part, B, H, T, C, s);
  else if (dtype == CA_DTYPE_F16) e = fwd_launch<_Float16>(D, io, part, B, H, T, C, s);
  else e = fwd_launch<float>(D, io, part, B, H, T, C, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "forward launch: %s", hipGetErrorString(e));
  return CA_OK;
}

template <class E>
hipError_t kv_cast_launch(int D, const float* dk_sum, const float* dv_sum, const ca::View& dk,
                          const ca::View& dv, int BH, int H, int T, hipStream_t s) {
  switch (D) {
    case 8: return ca::launch_kv_cast<8, E>(dk_sum, dv_sum, dk, dv, BH, H, T, s);
    case 16: return ca::launch_kv_cast<16, E>(dk_sum, dv_sum, dk, dv, BH, H, T, s);
    case 32: return ca::launch_kv_cast<32, E>(dk_sum, dv_sum, dk, dv, BH, H, T, s);
    case 64: return ca::launch_kv_cast<64, E>(dk_sum, dv_sum, dk, dv, BH, H, T, s);
    default: return ca::launch_kv_cast<128, E>(dk_sum, dv_sum, dk, dv, BH, H, T, s);
  }
}

// view of the slices of batch b from head h0 on (elements of esz bytes)
ca::View sub_view(const ca::View& v, int b, int h0, size_t esz) {
  ca::View r = v;
  r.base = static_cast<char*>(v.base) + ((long long)b * v.bstride + (long long)h0 * v.hstride) * (long long)esz;
  return r;
}

// One set of slices (the whole problem, or heads h0 .. h0 + H - 1 of one
// batch as a [1, H, T, D] problem) in its passes.  With kv_sums, dK and dV
// are summed in fp32 at the start of the workspace and rounded into io.dk /
// io.dv at the end.
int run_set(const ca::BwdIO& io, int dtype, char* ws, const std::vector<ca::BwdPass>& passes,
            bool first_set, bool kv_sums, int B, int H, int T, int D, hipStream_t s) {
  ca::BwdIO pio = io;
  if (kv_sums) {
    const size_t half = kv_sum_bytes(B * H, T, D) / 2;
    pio.dk = heads_view(ws, H, T, D);
    pio.dv = heads_view(ws + half, H, T, D);
    pio.kv_f32 = true;
    ws += 2 * half;
  }
  for (ca::BwdPass pass : passes) {
    // dlog_gain is written by the first pass of the first set, added to after
    pass.first = first_set && pass.g0 == 0;
    const BwdLayout L = bwd_layout(B, H, T, D, pass);
    ca::BwdWork work;
    work.dsbuf = reinterpret_cast<float*>(ws + L.ds);
    work.limbs = reinterpret_cast<__bf16*>(ws + L.limbs);
    work.qstat = reinterpret_cast<float*>(ws + L.qstat);
    work.gain_part = reinterpret_cast<float*>(ws + L.gain);
    work.dq_part = reinterpret_cast<float*>(ws + L.dqpart);
    work.kv_part = reinterpret_cast<float*>(ws + L.kvpart);
    const ca::DqSplit sp = dq_split_for(B * H, T, D, pass, false);
    const ca::DkdvSplit kvs = dkdv_split_for(B * H, D, dtype, pass, false);
    hipError_t e;
    if (dtype == CA_DTYPE_BF16) e = bwd_launch<__bf16>(D, pio, work, pass, sp, kvs, B, H, T, s);
    else if (dtype == CA_DTYPE_F16) e = bwd_launch<_Float16>(D, pio, work, pass, sp, kvs, B, H, T, s);
    else e = bwd_launch<float>(D, pio, work, pass, sp, kvs, B, H, T, s);
    if (e != hipSuccess) return fail(CA_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
  }
  if (kv_sums) {
    const float* dk_sum = static_cast<const float*>(pio.dk.base);
    const float* dv_sum = static_cast<const float*>(pio.dv.base);
    hipError_t e;
    if (dtype == CA_DTYPE_BF16) e = kv_cast_launch<__bf16>(D, dk_sum, dv_sum, io.dk, io.dv, B * H, H, T, s);
    else if (dtype == CA_DTYPE_F16) e = kv_cast_launch<_Float16>(D, dk_sum, dv_sum, io.dk, io.dv, B * H, H, T, s);
    else e = kv_cast_launch<float>(D, dk_sum, dv_sum, io.dk, io.dv, B * H, H, T, s);
    if (e != hipSuccess) return fail(CA_ERR_HIP, "dK/dV rounding launch: %s", hipGetErrorString(e));
  }
  return CA_OK;
}

// The backward in the plan for the workspace it is given: one pass when the
// whole backward fits, else passes over ranges of dQ groups, of every slice or
// of sets of heads (dK, dV and dlog_gain accumulate in a fixed order).
// kv_sums: io.dk and io.dv are the element type's gradients and the passes sum
// dK and dV in fp32 first (the token-major backward in passes).
int bwd_common(const ca::BwdIO& io, int dtype, void* workspace, size_t workspace_bytes, int B,
               int H, int T, int D, void* stream, bool kv_sums) {
  BwdPlan plan;
  if (!workspace || !plan_bwd(B, H, T, D, workspace_bytes, kv_sums, &plan))
    return fail(CA_ERR_WORKSPACE, "backward workspace of %zu bytes required, %zu given",
                bwd_capped_bytes(B, H, T, D, kv_sums), workspace ? workspace_bytes : 0);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (plan.hc == 0) return run_set(io, dtype, ws, plan.passes, true, kv_sums, B, H, T, D, s);
  const size_t esz = dtype_size(dtype);
  for (int b = 0; b < B; ++b) {
    for (int h0 = 0; h0 < H; h0 += plan.hc) {
      const int nh = std::min(plan.hc, H - h0);
      ca::BwdIO sio = io;
      sio.q = sub_view(io.q, b, h0, esz);
      sio.k = sub_view(io.k, b, h0, esz);
      sio.v = sub_view(io.v, b, h0, esz);
      sio.dout = sub_view(io.dout, b, h0, esz);
      sio.dq = sub_view(io.dq, b, h0, esz);
      sio.dk = sub_view(io.dk, b, h0, io.kv_f32 ? sizeof(float) : esz);
      sio.dv = sub_view(io.dv, b, h0, io.kv_f32 ? sizeof(float) : esz);
      const size_t row0 = ((size_t)b * H + h0) * T;
      sio.y = io.y + row0 * D;
      sio.stats = io.stats + row0 * 2;
      sio.log_gain = io.log_gain + h0;
      sio.dlog_gain = io.dlog_gain + h0;
      const int rc = run_set(sio, dtype, ws, nh == plan.hc ? plan.passes : plan.tail_passes,
                             b == 0, kv_sums, 1, nh, T, D, s);
      if (rc) return rc;
    }
  }
  return CA_OK;
}

// part `part` (of `parts`) of a token-major [B,T,parts,H,D] tensor as a view
ca::View tokens_view(const void* p, int dtype, int part, int parts, int T, int H, int D) {
  char* base = static_cast<char*>(const_cast<void*>(p)) + (size_t)part * H * D * dtype_size(dtype);
  return ca::View{base, (long long)T * parts * H * D, (long long)D, (long long)parts * H * D};
}
bool aligned_to(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

extern "C" {

int ca_fwd_f32(const float* q, const float* k, const float* v, const float* log_gain, float* out,
               float* stats, void* workspace, size_t workspace_bytes, int B, int H, int T, int D,
               void* stream) {
  int rc = check_shape(B, H, T, D);
  if (rc) return rc;
  if (!q || !k || !v || !log_gain || !out || !stats)
    return fail(CA_ERR_INVALID, "null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(CA_ERR_INVALID, "q, k, v and out must be 16-byte aligned");
  ca::FwdIO io{heads_view(q, H, T, D), heads_view(k, H, T, D), heads_view(v, H, T, D), nullptr,
               false, log_gain, out, ca::View{nullptr, 0, 0, 0}, stats};
  return fwd_common(io, CA_DTYPE_F32, workspace, workspace_bytes, B, H, T, D, stream);
}

int ca_bwd_f32(const float* q, const float* k, const float* v, const float* log_gain,
               const float* out, const float* stats, const float* dout, float* dq, float* dk,
               float* dv, float* dlog_gain, void* workspace, size_t workspace_bytes, int B, int H,
               int T, int D, void* stream) {
  int rc = check_shape(B, H, T, D);
  if (rc) return rc;
  if (!q || !k || !v || !log_gain || !out || !stats || !dout || !dq || !dk || !dv || !dlog_gain)
    return fail(CA_ERR_INVALID, "null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !aligned16(dout) ||
      !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return fail(CA_ERR_INVALID, "q, k, v, out, dout, dq, dk and dv must be 16-byte aligned");
  ca::BwdIO io{heads_view(q, H, T, D), heads_view(k, H, T, D), heads_view(v, H, T, D), nullptr,
               false, log_gain, out, stats, heads_view(dout, H, T, D), heads_view(dq, H, T, D),
               heads_view(dk, H, T, D), heads_view(dv, H, T, D), dlog_gain};
  return bwd_common(io, CA_DTYPE_F32, workspace, workspace_bytes, B, H, T, D, stream, false);
}

static int check_qkv(const char* fn, int dtype, const void* qkv, const float* rope_cs,
                     const float* y, const void* tok, int T, int H, int D) {
  if (dtype != CA_DTYPE_F32 && dtype != CA_DTYPE_BF16 && dtype != CA_DTYPE_F16)
    return fail(CA_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  // the forward reads one head's key and value rows of qkv (and 32 rows past
  // T) through 32-bit byte offsets
  if (ca::view_rows_bytes(T + 32, 3LL * H * D, D, (int)dtype_size(dtype)) >= (1ULL << 32))
    return fail(CA_ERR_UNSUPPORTED,
                "%s: one head's rows of qkv span 4 GiB or more (T=%d, H*D=%d); the kernels "
                "address them with 32-bit offsets", fn, T, H * D);
  const size_t a = dtype == CA_DTYPE_F32 ? 16 : 8;
  if (!aligned_to(qkv, a) || !aligned_to(tok, a) || !aligned16(y) ||
      (rope_cs && !aligned16(rope_cs)))
    return fail(CA_ERR_INVALID, "%s: misaligned buffer (qkv and the token-major output %zu-byte, "
                "y and rope_cs 16-byte)", fn, a);
  return CA_OK;
}

int ca_fwd_qkv(const void* qkv, int dtype, const float* rope_cs, const float* log_gain, float* y,
               void* out, float* stats, void* workspace, size_t workspace_bytes, int B, int T,
               int H, int D, void* stream) {
  int rc = check_shape(B, H, T, D);
  if (rc) return rc;
  if (!qkv || !log_gain || !y || !out || !stats)
    return fail(CA_ERR_INVALID, "ca_fwd_qkv: null pointer");
  rc = check_qkv("ca_fwd_qkv", dtype, qkv, rope_cs, y, out, T, H, D);
  if (rc) return rc;
  ca::FwdIO io{tokens_view(qkv, dtype, 0, 3, T, H, D), tokens_view(qkv, dtype, 1, 3, T, H, D),
               tokens_view(qkv, dtype, 2, 3, T, H, D), rope_cs, false, log_gain, y,
               tokens_view(out, dtype, 0, 1, T, H, D), stats};
  char* ws = static_cast<char*>(workspace);
  size_t bytes = workspace_bytes;
  if (workspace &&
      workspace_bytes >= rotated_keys_bytes(B, H, T, D) + ca_fwd_workspace_bytes(B, H, T, D)) {
    rc = rotate_keys_first(&io.k, &io.k_rotated, rope_cs, dtype, &ws, &bytes, B, H, T, D, stream);
    if (rc) return rc;
  }
  return fwd_common(io, dtype, ws, bytes, B, H, T, D, stream);
}

int ca_bwd_qkv(const void* qkv, int dtype, const float* rope_cs, const float* log_gain,
               const float* y, const float* stats, const void* dout, void* dqkv,
               float* dlog_gain, void* workspace, size_t workspace_bytes, int B, int T, int H,
               int D, void* stream) {
  int rc = check_shape(B, H, T, D);
  if (rc) return rc;
  if (!qkv || !log_gain || !y || !stats || !dout || !dqkv || !dlog_gain)
    return fail(CA_ERR_INVALID, "ca_bwd_qkv: null pointer");
  rc = check_qkv("ca_bwd_qkv", dtype, qkv, rope_cs, y, dout, T, H, D);
  if (rc) return rc;
  if (!aligned_to(dqkv, dtype == CA_DTYPE_F32 ? 16 : 8))
    return fail(CA_ERR_INVALID, "ca_bwd_qkv: misaligned dqkv");
  ca::BwdIO io{tokens_view(qkv, dtype, 0, 3, T, H, D), tokens_view(qkv, dtype, 1, 3, T, H, D),
               tokens_view(qkv, dtype, 2, 3, T, H, D), rope_cs, false, log_gain, y, stats,
               tokens_view(dout, dtype, 0, 1, T, H, D), tokens_view(dqkv, dtype, 0, 3, T, H, D),
               tokens_view(dqkv, dtype, 1, 3, T, H, D), tokens_view(dqkv, dtype, 2, 3, T, H, D),
               dlog_gain};
  char* ws = static_cast<char*>(workspace);
  size_t bytes = workspace_bytes;
  const size_t full = bwd_full_bytes(B, H, T, D);
  if (workspace && workspace_bytes >= full) {
    // one pass, gradients written in the element type (keys rotated once
    // when the workspace also has room for them)
    if (workspace_bytes >= rotated_keys_bytes(B, H, T, D) + full) {
      rc = rotate_keys_first(&io.k, &io.k_rotated, rope_cs, dtype, &ws, &bytes, B, H, T, D, stream);
      if (rc) return rc;
    }
    return bwd_common(io, dtype, ws, bytes, B, H, T, D, stream, false);
  }
  // passes: the element type cannot carry dK and dV across them without
  // rounding each pass's sum, so they are summed in fp32 and rounded once
  return bwd_common(io, dtype, ws, bytes, B, H, T, D, stream, true);
}

static int check_rows(const char* fn, int BH, int Q, int K, int start) {
  if (BH <= 0 || Q <= 0 || K <= 0 || start < 0)
    return fail(CA_ERR_INVALID, "%s: invalid shape BH=%d Q=%d K=%d start=%d", fn, BH, Q, K, start);
  if ((long long)start + Q > K)
    return fail(CA_ERR_INVALID,
                "%s: queries start..start+Q-1 = %d..%lld need their keys, but K=%d < start+Q", fn,
                start, (long long)start + Q - 1, K);
  if ((long long)BH * Q > (1ll << 31) - 1)
    return fail(CA_ERR_UNSUPPORTED, "%s: BH*Q=%lld rows exceed 2^31-1", fn, (long long)BH * Q);
  return CA_OK;
}

int ca_weights_f32(const float* scores, float* weights, float* stats, int BH, int Q, int K,
                   int start, void* stream) {
  int rc = check_rows("ca_weights_f32", BH, Q, K, start);
  if (rc) return rc;
  if (!scores || !weights || !stats) return fail(CA_ERR_INVALID, "ca_weights_f32: null pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kWeights, s);
  hipError_t e = ca::launch_weights(scores, weights, stats, BH, Q, K, start, s);
  ca::timer_end(ca::kWeights, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_weights_f32 launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_weights_bwd_f32(const float* scores, const float* grad_weights, float* weights,
                       float* grad_scores, int BH, int Q, int K, int start, void* stream) {
  int rc = check_rows("ca_weights_bwd_f32", BH, Q, K, start);
  if (rc) return rc;
  if (!scores || !grad_weights || !grad_scores)
    return fail(CA_ERR_INVALID, "ca_weights_bwd_f32: null pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kWeightsBwd, s);
  hipError_t e = ca::launch_weights_bwd(scores, grad_weights, weights, grad_scores, BH, Q, K,
                                        start, s);
  ca::timer_end(ca::kWeightsBwd, s);
  if (e != hipSuccess)
    return fail(CA_ERR_HIP, "ca_weights_bwd_f32 launch: %s", hipGetErrorString(e));
  return CA_OK;
}

static int check_swiglu(const char* fn, const void* a, const void* b, const void* c, int N,
                        int H) {
  if (N <= 0 || H <= 0 || H % 4) return fail(CA_ERR_INVALID, "%s: invalid shape N=%d H=%d (H %% 4 == 0)", fn, N, H);
  if ((long long)N * 2 * H > (1ll << 40)) return fail(CA_ERR_UNSUPPORTED, "%s: tensor too large", fn);
  if (!a || !b || !c) return fail(CA_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return fail(CA_ERR_INVALID, "%s: pointers must be 16-byte aligned", fn);
  return CA_OK;
}

int ca_swiglu_fwd_f32(const float* u, float* h, int N, int H, void* stream) {
  int rc = check_swiglu("ca_swiglu_fwd_f32", u, h, h, N, H);
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kSwigluFwd, s);
  hipError_t e = ca::launch_swiglu_fwd(u, h, N, H, s);
  ca::timer_end(ca::kSwigluFwd, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_swiglu_fwd_f32 launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_swiglu_bwd_f32(const float* u, const float* dh, float* du, int N, int H, void* stream) {
  int rc = check_swiglu("ca_swiglu_bwd_f32", u, dh, du, N, H);
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kSwigluBwd, s);
  hipError_t e = ca::launch_swiglu_bwd(u, dh, du, N, H, s);
  ca::timer_end(ca::kSwigluBwd, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_swiglu_bwd_f32 launch: %s", hipGetErrorString(e));
  return CA_OK;
}

static int check_norm(const char* fn, int N, int C, int dtype) {
  if (N <= 0 || C <= 0) return fail(CA_ERR_INVALID, "%s: invalid shape N=%d C=%d", fn, N, C);
  if (C > ca::kRmsMaxCols) return fail(CA_ERR_UNSUPPORTED, "%s: C=%d exceeds %d", fn, C, ca::kRmsMaxCols);
  if (dtype != CA_DTYPE_F32 && dtype != CA_DTYPE_BF16 && dtype != CA_DTYPE_F16)
    return fail(CA_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if ((long long)N * C > (1ll << 31) - 1) return fail(CA_ERR_UNSUPPORTED, "%s: tensor too large", fn);
  return CA_OK;
}

int ca_rmsnorm_fwd(const float* x, const float* weight, void* y, int ydtype, float* rstd, int N,
                   int C, float eps, void* stream) {
  int rc = check_norm("ca_rmsnorm_fwd", N, C, ydtype);
  if (rc) return rc;
  if (!x || !weight || !y || !rstd) return fail(CA_ERR_INVALID, "ca_rmsnorm_fwd: null pointer");
  if (!(eps >= 0.f)) return fail(CA_ERR_INVALID, "ca_rmsnorm_fwd: eps must be >= 0");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kRmsFwd, s);
  hipError_t e = ca::launch_rmsnorm_fwd(x, nullptr, CA_DTYPE_F32, nullptr, weight, y, ydtype, rstd,
                                        N, C, eps, s);
  ca::timer_end(ca::kRmsFwd, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_rmsnorm_fwd launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_add_rmsnorm_fwd(const float* x, const void* res, int rdtype, float* sum_out,
                       const float* weight, void* y, int ydtype, float* rstd, int N, int C,
                       float eps, void* stream) {
  int rc = check_norm("ca_add_rmsnorm_fwd", N, C, ydtype);
  if (rc) return rc;
  if (rdtype != CA_DTYPE_F32 && rdtype != CA_DTYPE_BF16 && rdtype != CA_DTYPE_F16)
    return fail(CA_ERR_INVALID, "ca_add_rmsnorm_fwd: unknown dtype %d", rdtype);
  if (!x || !res || !sum_out || !weight || !y || !rstd)
    return fail(CA_ERR_INVALID, "ca_add_rmsnorm_fwd: null pointer");
  if (!(eps >= 0.f)) return fail(CA_ERR_INVALID, "ca_add_rmsnorm_fwd: eps must be >= 0");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kRmsFwd, s);
  hipError_t e = ca::launch_rmsnorm_fwd(x, res, rdtype, sum_out, weight, y, ydtype, rstd, N, C, eps, s);
  ca::timer_end(ca::kRmsFwd, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_add_rmsnorm_fwd launch: %s", hipGetErrorString(e));
  return CA_OK;
}

size_t ca_rmsnorm_bwd_workspace_bytes(int N, int C) {
  if (N <= 0 || C <= 0) return 0;
  return (size_t)ca::rmsnorm_bwd_blocks(N) * C * sizeof(float);
}

int ca_rmsnorm_bwd(const void* dy, int dydtype, const float* x, const float* weight,
                   const float* rstd, float* dx, float* dweight, void* workspace,
                   size_t workspace_bytes, int N, int C, void* stream) {
  int rc = check_norm("ca_rmsnorm_bwd", N, C, dydtype);
  if (rc) return rc;
  if (!dy || !x || !weight || !rstd || !dx || !dweight)
    return fail(CA_ERR_INVALID, "ca_rmsnorm_bwd: null pointer");
  const size_t need = ca_rmsnorm_bwd_workspace_bytes(N, C);
  if (!workspace || workspace_bytes < need)
    return fail(CA_ERR_WORKSPACE, "ca_rmsnorm_bwd: workspace of %zu bytes required, %zu given", need,
                workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kRmsBwd, s);
  hipError_t e = ca::launch_rmsnorm_bwd(dy, dydtype, nullptr, x, weight, rstd, dx, nullptr,
                                        CA_DTYPE_F32, dweight, static_cast<float*>(workspace), N, C, s);
  ca::timer_end(ca::kRmsBwd, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_rmsnorm_bwd launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_add_rmsnorm_bwd(const void* dy, int dydtype, const float* dsum, const float* sum,
                       const float* weight, const float* rstd, float* dx, void* dres, int rdtype,
                       float* dweight, void* workspace, size_t workspace_bytes, int N, int C,
                       void* stream) {
  int rc = check_norm("ca_add_rmsnorm_bwd", N, C, dydtype);
  if (rc) return rc;
  if (rdtype != CA_DTYPE_F32 && rdtype != CA_DTYPE_BF16 && rdtype != CA_DTYPE_F16)
    return fail(CA_ERR_INVALID, "ca_add_rmsnorm_bwd: unknown dtype %d", rdtype);
  if (!dy || !sum || !weight || !rstd || !dx || !dres || !dweight)
    return fail(CA_ERR_INVALID, "ca_add_rmsnorm_bwd: null pointer");
  const size_t need = ca_rmsnorm_bwd_workspace_bytes(N, C);
  if (!workspace || workspace_bytes < need)
    return fail(CA_ERR_WORKSPACE, "ca_add_rmsnorm_bwd: workspace of %zu bytes required, %zu given",
                need, workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  ca::timer_begin(ca::kRmsBwd, s);
  hipError_t e = ca::launch_rmsnorm_bwd(dy, dydtype, dsum, sum, weight, rstd, dx, dres, rdtype,
                                        dweight, static_cast<float*>(workspace), N, C, s);
  ca::timer_end(ca::kRmsBwd, s);
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_add_rmsnorm_bwd launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_opt_chunk_elems(void) { return ca::kOptChunk; }

static int check_opt(const char* fn, const ca_opt_tensor* tensors, int ntensors, const int* chunks,
                     int nchunks) {
  if (!tensors || !chunks) return fail(CA_ERR_INVALID, "%s: null tensor or chunk table", fn);
  if (ntensors <= 0 || nchunks <= 0) return fail(CA_ERR_INVALID, "%s: empty tensor or chunk table", fn);
  if ((reinterpret_cast<uintptr_t>(tensors) & 7) || (reinterpret_cast<uintptr_t>(chunks) & 7))
    return fail(CA_ERR_INVALID, "%s: tables must be 8-byte aligned", fn);
  return CA_OK;
}

int ca_grad_clip_coef(const ca_opt_tensor* tensors, int ntensors, const int* chunks, int nchunks,
                      float* partial, float max_norm, float* total_norm, float* coef,
                      void* stream) {
  int rc = check_opt("ca_grad_clip_coef", tensors, ntensors, chunks, nchunks);
  if (rc) return rc;
  if (!partial || !total_norm || !coef) return fail(CA_ERR_INVALID, "ca_grad_clip_coef: null pointer");
  hipError_t e = ca::launch_grad_sumsq(tensors, ntensors, reinterpret_cast<const int2*>(chunks), nchunks,
                                       partial, max_norm, total_norm, coef,
                                       reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_grad_clip_coef launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_adamw_step(const ca_opt_tensor* tensors, int ntensors, const int* chunks, int nchunks,
                  const float* coef, float lr, float beta1, float beta2, float eps,
                  float weight_decay, int step, void* stream) {
  int rc = check_opt("ca_adamw_step", tensors, ntensors, chunks, nchunks);
  if (rc) return rc;
  if (step < 1) return fail(CA_ERR_INVALID, "ca_adamw_step: step must be >= 1, got %d", step);
  if (!(beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f))
    return fail(CA_ERR_INVALID, "ca_adamw_step: betas must be in [0, 1)");
  // bias corrections in double, as torch's AdamW computes them on the host
  const double bc1 = 1.0 - std::pow((double)beta1, (double)step);
  const double bc2 = 1.0 - std::pow((double)beta2, (double)step);
  ca::CaAdamwScalars k;
  k.decay = (float)(1.0 - (double)lr * (double)weight_decay);
  k.one_minus_beta1 = (float)(1.0 - (double)beta1);
  k.beta2 = beta2;
  k.one_minus_beta2 = (float)(1.0 - (double)beta2);
  k.bc2_sqrt = (float)std::sqrt(bc2);
  k.eps = eps;
  k.neg_step_size = (float)(-(double)lr / bc1);
  hipError_t e = ca::launch_adamw(tensors, ntensors, reinterpret_cast<const int2*>(chunks), nchunks,
                                  coef, k, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_adamw_step launch: %s", hipGetErrorString(e));
  return CA_OK;
}

int ca_bf16_shadow(const ca_opt_tensor* tensors, int ntensors, const int* chunks, int nchunks,
                   void* stream) {
  int rc = check_opt("ca_bf16_shadow", tensors, ntensors, chunks, nchunks);
  if (rc) return rc;
  hipError_t e = ca::launch_shadow(tensors, ntensors, reinterpret_cast<const int2*>(chunks), nchunks,
                                   reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(CA_ERR_HIP, "ca_bf16_shadow launch: %s", hipGetErrorString(e));
  return CA_OK;
}

}  // extern "C"
