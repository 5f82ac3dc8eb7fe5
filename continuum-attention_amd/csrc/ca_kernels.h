// Internal launch interface between the C ABI (ca_abi.hip) and the kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include <cmath>
#include <type_traits>

#include "../../include/continuum_attention_amd.h"
#include "ca_common.h"

namespace ca {

// Forward work decomposition: 128-query groups, 32-key weight tiles, splits of
// at most C tiles per work item.
inline int fwd_group_tiles(int g, int T) {
  const int all = (T + 31) / 32;
  return (4 * g + 4 < all) ? 4 * g + 4 : all;
}
inline int fwd_max_splits(int T, int C) {
  const int G = (T + 127) / 128;
  return (fwd_group_tiles(G - 1, T) + C - 1) / C;
}
inline int fwd_num_items(int T, int C) {
  const int G = (T + 127) / 128;
  int n = 0;
  for (int g = 0; g < G; ++g) n += (fwd_group_tiles(g, T) + C - 1) / C;
  return n;
}
// Split length: 12 tiles up to T = 2048; for short rows (at most four
// 128-query groups) 8, 6 or 4 while the grid of BH * items would not fill
// `resident` work groups; past T = 2048, 12 sqrt(T / 2048) tiles rounded to a
// multiple of 4 (16, 24, 32, 48 at T = 4096 .. 32768), as the grid then
// fills the device either way and each split adds combine traffic (same-box
// fwd+bwd at [1,16,T,64] with 12 tiles against the longer split: T = 4096
// 1.026 -> 1.017 ms, 8192 4.04 -> 4.00 ms, 16384 16.27 -> 15.81 ms; at T =
// 2048 longer splits were no faster).
constexpr int kFwdSplitTiles = 12;
constexpr int kFwdSplitSmall[] = {8, 6, 4};
constexpr int kFwdSplitShortT = 512;
constexpr int kFwdSplitLongT = 2048;
inline int fwd_split_tiles(int BH, int T, int resident) {
  int C = kFwdSplitTiles;
  if (T > kFwdSplitLongT) {
    const double c = kFwdSplitTiles * std::sqrt((double)T / kFwdSplitLongT);
    return 4 * (int)std::lround(c / 4.0);
  }
  if (T > kFwdSplitShortT) return C;
  for (int c : kFwdSplitSmall) {
    if ((long long)fwd_num_items(T, C) * BH >= resident) break;
    C = c;
  }
  return C;
}
inline size_t fwd_part_floats(int BH, int T, int C, int D) {
  const int smax = fwd_max_splits(T, C);
  if (smax <= 1) return 0;
  return (size_t)BH * smax * T * (D + 2);  // D outputs + (m, Z) per row and split
}

// Backward key blocks.  One dK/dV wave owns 14 keys and feeds 16 MFMA slots
// (slot s = key 14*kb - 1 + s), so both neighbours of every owned key are
// inside its block; a dK/dV work group takes kDkdvWaves consecutive blocks.
// The dS spill for the dQ pass is stored per (32-query tile, block).
constexpr int kBwdKeys = 14;
constexpr int kBwdSlots = 16;
constexpr int kDkdvWaves = 4;
__host__ __device__ inline int bwd_num_key_blocks(int T) { return (T + kBwdKeys - 1) / kBwdKeys; }
__host__ __device__ inline int num_q_tiles(int T) { return (T + 31) / 32; }
// dQ work groups take kDqTiles consecutive 32-query tiles (kDqRows queries).
constexpr int kDqTiles = 4;
constexpr int kDqRows = 32 * kDqTiles;
__host__ __device__ inline int dq_num_groups(int T) { return (num_q_tiles(T) + kDqTiles - 1) / kDqTiles; }

// sum_{i=0}^{n-1} floor((a*i + b) / m) for n, m >= 1 and a, b >= 0 (Euclid-like
// reduction, O(log m) steps).
__host__ __device__ inline long long floor_sum(long long n, long long m, long long a, long long b) {
  long long ans = 0;
  while (true) {
    if (a >= m) {
      ans += (n - 1) * n / 2 * (a / m);
      a %= m;
    }
    if (b >= m) {
      ans += n * (b / m);
      b %= m;
    }
    const long long y_max = a * n + b;
    if (y_max < m) break;
    n = y_max / m;
    b = y_max % m;
    const long long t = m;
    m = a;
    a = t;
  }
  return ans;
}

// dS spill for the dQ pass, key-major: for every query tile qt the keys of
// the dK/dV key blocks that meet it (keys 0 .. 14 ds_kb_count(qt) - 1), each
// as one column of 32 floats (dS of the tile's 32 queries, 128 bytes), tiles
// in order.  Invisible keys hold 0; keys past T are never written.  Each key
// column is written by the four lanes of one dK/dV wave that own the key, as
// two 16-byte stores each, so every 128-byte line is written whole by one
// wave; no key is stored twice (the halo slots are not spilled).  The dQ pass
// gathers 8-key runs of one query from 8 columns (one dword per key).
constexpr int kDsColFloats = 32;
__host__ __device__ inline int ds_kb_count(int qt) { return (32 * qt + 31) / kBwdKeys + 1; }
// floats of the columns of tiles 0 .. qt-1: 32 * 14 * sum of ds_kb_count(t)
__host__ __device__ inline long long ds_floats_before(int qt) {
  return qt <= 0 ? 0 : (long long)kDsColFloats * kBwdKeys * (qt + floor_sum(qt, kBwdKeys, 32, 31));
}

// Backward passes.  The backward's workspace (dS spill, limb planes, row
// statistics, partials) grows with the query rows it holds, the dS spill as
// O(T^2); so that a bounded workspace serves any T, the backward can run in
// passes over ranges of 128-query (dQ) groups.  A pass handles dQ groups
// [g0, g1) = query tiles [qa, qb) = rows [row0, row0 + rows): its prep,
// dK/dV, dQ and merge launches see only those queries.  dQ rows and their dS
// are complete within a pass; dK and dV receive every pass's contribution in
// pass order (the first pass that reaches a key group writes, later ones
// add), and dlog_gain likewise.  One pass covering everything is the
// ordinary backward.
struct BwdPass {
  int g0, g1;         // dQ groups of the pass
  int qa, qb;         // query tiles
  int row0, rows;     // first query row, and rows per slice held in the limb planes
  long long ds0;      // dS floats per slice before tile qa
  long long ds_slice; // dS floats per slice in this pass
  int kv_groups;      // dK/dV key groups that meet the pass's tiles (wg < kv_groups)
  int first;          // 1 for the first pass (dlog_gain written, not added)
};
__host__ __device__ inline BwdPass bwd_pass(int T, int g0, int g1) {
  const int nqt = num_q_tiles(T);
  BwdPass p;
  p.g0 = g0;
  p.g1 = g1;
  p.qa = kDqTiles * g0;
  p.qb = kDqTiles * g1 < nqt ? kDqTiles * g1 : nqt;
  p.row0 = 32 * p.qa;
  const int row1 = 32 * p.qb < T ? 32 * p.qb : T;
  p.rows = row1 - p.row0;
  p.ds0 = ds_floats_before(p.qa);
  p.ds_slice = ds_floats_before(p.qb) - p.ds0;
  const int nkb = bwd_num_key_blocks(T);
  const int ngroups = (nkb + 3) / 4;
  // key group wg (keys 56 wg ..) first meets tile 56 wg / 32; it meets this
  // pass's tiles when that is below qb
  const int need = (32 * p.qb + 55) / 56;
  p.kv_groups = need < ngroups ? need : ngroups;
  p.first = g0 == 0;
  return p;
}

// dQ work items: a 128-query group of one slice and one chunk of its key
// stages (32 keys each; the group's last tile qt needs stages 0 .. qt).  A
// group of n stages is cut into ceil(n / chunk) near-equal chunks (split-K)
// when the unsplit grid would not fill the GPU for one round, so that the
// longest rows do not leave it waiting on a few work groups; with a full grid
// every group is one item (chunk >= num_q_tiles).  Items are numbered per
// slice from the last (heaviest) group of the pass down, so the chunks of
// multi-chunk groups come first; those items write partial dQ tiles that a
// second kernel sums in chunk order.
constexpr int kDqChunkStages = 28;       // split chunk length in 32-key stages (896 keys)
constexpr int kDqChunkStagesShort = 21;  // when 28-stage chunks still leave the GPU short of a round
// key stages of group qg (those met by its last query tile)
__host__ __device__ inline int dq_group_stages(int qg, int T) {
  const int nqt = num_q_tiles(T);
  const int last = kDqTiles * qg + kDqTiles - 1 < nqt ? kDqTiles * qg + kDqTiles - 1 : nqt - 1;
  return last + 1;
}
__host__ __device__ inline int dq_group_chunks(int qg, int T, int chunk) {
  return (dq_group_stages(qg, T) + chunk - 1) / chunk;
}
struct DqSplit {
  int chunk;         // key stages per chunk (upper bound)
  int items;         // work items per slice
  int part_items;    // of which write partial tiles (chunks of multi-chunk groups)
  int multi_groups;  // groups with more than one chunk (the last ones)
};
inline DqSplit dq_split_chunk(int T, const BwdPass& p, int chunk) {
  DqSplit s{chunk, 0, 0, 0};
  for (int g = p.g0; g < p.g1; ++g) {
    const int n = dq_group_chunks(g, T, s.chunk);
    s.items += n;
    if (n > 1) {
      s.part_items += n;
      ++s.multi_groups;
    }
  }
  return s;
}
// resident_groups: dQ work groups the GPU holds at once (0: never split).
// Splitting more finely only adds work groups (and partial tiles), so the
// workspace sized for the largest resident_groups covers every smaller one.
// Shorter chunks while the grid would fill less than half a round (few
// slices, short rows): more dQ work groups, at the price of more partials to
// merge, which outweighs the gain once half a round is filled.
constexpr int kDqChunkSmall[] = {14, 10, 7};
inline DqSplit dq_split(int BH, int T, const BwdPass& p, int resident_groups) {
  if ((long long)(p.g1 - p.g0) * BH >= resident_groups)
    return dq_split_chunk(T, p, num_q_tiles(T));
  DqSplit s = dq_split_chunk(T, p, kDqChunkStages);
  if ((long long)s.items * BH >= resident_groups) return s;
  s = dq_split_chunk(T, p, kDqChunkStagesShort);
  for (int c : kDqChunkSmall) {
    if (2LL * s.items * BH >= resident_groups) break;
    s = dq_split_chunk(T, p, c);
  }
  return s;
}
// dQ work groups per CU the split heuristic counts as resident: 3, although
// the D = 64 kernel's 124 VGPRs allow 4 (counting 4 picks shorter chunks at
// [2,16,2048,64], measured 4% slower)
constexpr int kDqGroupsPerCu = 3;

// dK/dV work items: key-block group wg (kDkdvWaves blocks, kDkdvKeys keys) of
// one slice and a chunk of the pass's query tiles that see its keys.  When
// the grid of whole groups would not fill the GPU for two rounds (small B*H),
// a group's query range is cut into chunks of at most kDkdvChunkTiles tiles,
// so the groups with the longest ranges do not set the launch time alone; the
// chunks write partial dK/dV that a merge sums in chunk order.  Items are
// numbered per slice from group 0 (the longest range) up, chunks of a group
// together.
constexpr int kDkdvKeys = kDkdvWaves * kBwdKeys;
constexpr int kDkdvChunkTiles = 24;
constexpr int kDkdvGroupsPerCu = 2;
__host__ __device__ inline int dkdv_num_groups(int T) {
  return (bwd_num_key_blocks(T) + kDkdvWaves - 1) / kDkdvWaves;
}
// first query tile that sees key group wg
__host__ __device__ inline int dkdv_qt0(int wg) { return kDkdvKeys * wg / 32; }
// the pass's tiles of group wg (wg < p.kv_groups): max(qt0, qa) .. qb-1
__host__ __device__ inline int dkdv_group_first_tile(int wg, const BwdPass& p) {
  const int a = dkdv_qt0(wg);
  return a > p.qa ? a : p.qa;
}
__host__ __device__ inline int dkdv_group_tiles(int wg, const BwdPass& p) {
  return p.qb - dkdv_group_first_tile(wg, p);
}
__host__ __device__ inline int dkdv_group_chunks(int wg, const BwdPass& p, int chunk) {
  return (dkdv_group_tiles(wg, p) + chunk - 1) / chunk;
}
struct DkdvSplit {
  int chunk;         // query tiles per chunk (upper bound)
  int items;         // work items per slice
  int part_items;    // of which write partial dK/dV (chunks of multi-chunk groups)
  int multi_groups;  // groups with more than one chunk (the first ones)
};
inline DkdvSplit dkdv_split_chunk(const BwdPass& p, int chunk) {
  DkdvSplit s{chunk, 0, 0, 0};
  for (int g = 0; g < p.kv_groups; ++g) {
    const int n = dkdv_group_chunks(g, p, chunk);
    s.items += n;
    if (n > 1) {
      s.part_items += n;
      ++s.multi_groups;
    }
  }
  return s;
}
// Shorter chunks while the first length (kDkdvChunkTiles unless given)
// leaves less than one round (fewer would only add partials and merge
// work): the first length whose items fill a round is taken, else the last.
// resident_groups: dK/dV work groups the GPU holds at once (0: never split).
constexpr int kDkdvChunkSmall[] = {16, 12, 8, 6};
// want_groups: split only when the whole groups number fewer (default: two
// rounds of resident_groups).
inline DkdvSplit dkdv_split(int BH, const BwdPass& p, int resident_groups, long long want_groups = -1,
                            int first_chunk = kDkdvChunkTiles) {
  const long long want = want_groups >= 0 ? want_groups : 2LL * resident_groups;
  if ((long long)p.kv_groups * BH >= want) return dkdv_split_chunk(p, p.qb - p.qa);
  DkdvSplit s = dkdv_split_chunk(p, first_chunk);
  for (int c : kDkdvChunkSmall) {
    if (c >= first_chunk) continue;
    if ((long long)s.items * BH >= resident_groups) break;
    s = dkdv_split_chunk(p, c);
  }
  return s;
}

// Per-kernel HIP-event timing (diagnostics; off unless ca_timing_enable(1)).
enum KernelId {
  kFwd = 0, kFwdCombine, kBwdPrep, kBwdDkdv, kBwdDq, kBwdGain, kWeights, kWeightsBwd, kRmsFwd,
  kRmsBwd, kSwigluFwd, kSwigluBwd, kNumKernels
};

// Element types of the prologue / epilogue buffers (CA_DTYPE_* in the ABI).
constexpr int kDtypeF32 = 0, kDtypeBF16 = 1, kDtypeF16 = 2;
void timer_begin(int id, hipStream_t s);
void timer_end(int id, hipStream_t s);
// Whether the backward of this shape can run in a workspace of `bytes`
// (in one pass, or in passes over query-group ranges of all slices or of
// sets of heads).
bool bwd_fits(int B, int H, int T, int D, size_t bytes);
// Shape check of the operator's entry points: CA_OK, or an error code
// (CA_ERR_INVALID for non-positive sizes, CA_ERR_UNSUPPORTED for head dims
// and sizes outside the kernels' range) with ca_last_error() set.
int check_shape(int B, int H, int T, int D);
// Sets the calling thread's ca_last_error() text; returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// RMSNorm of the decoder caller (ca_norm.hip).  The backward splits the rows
// over at most kRmsMaxBlocks work groups and keeps one dweight partial per group.
constexpr int kRmsMaxBlocks = 512;
constexpr int kRmsMaxCols = 4096;  // dynamic LDS of the backward: 16*C bytes <= 64 KB
int rmsnorm_rows_per_block(int N);
int rmsnorm_bwd_blocks(int N);
// res != nullptr: normalise s = x + res and write s to sum_out.
hipError_t launch_rmsnorm_fwd(const float* x, const void* res, int rdtype, float* sum_out,
                              const float* w, void* y, int ydtype, float* rstd, int N, int C,
                              float eps, hipStream_t s);
// dres != nullptr: x is the forward's s; dx = (norm gradient) + dsum (if
// dsum != nullptr), also written to dres in rdtype.
hipError_t launch_rmsnorm_bwd(const void* dy, int dydtype, const float* dsum, const float* x,
                              const float* w, const float* rstd, float* dx, void* dres, int rdtype,
                              float* dw, float* dw_part, int N, int C, hipStream_t s);

// SwiGLU gate of the TinyLM MLP (ca_swiglu.hip): u [N][2H] = [g | v],
// h [N][H] = silu(g) * v, du [N][2H]; H % 4 == 0, 16-byte aligned rows.
hipError_t launch_swiglu_fwd(const float* u, float* h, int N, int H, hipStream_t s);
hipError_t launch_swiglu_bwd(const float* u, const float* dh, float* du, int N, int H,
                             hipStream_t s);

// AdamW step (ca_optim.hip): chunks of kOptChunk elements.
constexpr int kOptChunk = 16384;
using CaOptTensor = ca_opt_tensor;
struct CaAdamwScalars {
  float decay;            // 1 - lr * weight_decay
  float one_minus_beta1;
  float beta2;
  float one_minus_beta2;
  float bc2_sqrt;         // sqrt(1 - beta2^step)
  float eps;
  float neg_step_size;    // -lr / (1 - beta1^step)
};
hipError_t launch_grad_sumsq(const CaOptTensor* tensors, int ntensors, const int2* chunks,
                             int nchunks, float* partial, float max_norm, float* total_norm,
                             float* coef, hipStream_t s);
hipError_t launch_adamw(const CaOptTensor* tensors, int ntensors, const int2* chunks, int nchunks,
                        const float* coef, const CaAdamwScalars& k, hipStream_t s);
hipError_t launch_shadow(const CaOptTensor* tensors, int ntensors, const int2* chunks, int nchunks,
                         hipStream_t s);

// Weight-materialising row kernels (ca_weights.hip).
hipError_t launch_weights(const float* scores, float* weights, float* stats, int BH, int Q, int K,
                          int start, hipStream_t stream);
hipError_t launch_weights_bwd(const float* scores, const float* grad_weights, float* weights,
                              float* grad_scores, int BH, int Q, int K, int start,
                              hipStream_t stream);

// Operands of the forward and backward as strided views (View, ca_common.h)
// of element type E (float, __bf16 or _Float16, a launch template
// parameter): the operator's own fp32 [B,H,T,D] tensors, or inside the
// decoder the token-major qkv projection output [B,T,3,H,D] with RoPE applied
// to q and k as they are read.
struct FwdIO {
  View q, k, v;            // inputs
  const float* rope;       // [T][D/2][2] (cos, sin) for q and k, or nullptr
  bool k_rotated;          // k is already rotated (launch_rope_keys): rope applies to q only
  const float* log_gain;   // [H]
  float* y;                // fp32 [B,H,T,D] output (read by the backward)
  View out;                // optional copy of the output in E (base nullptr: none)
  float* stats;            // [B*H*T][2]
};
struct BwdIO {
  View q, k, v;            // the forward's inputs
  const float* rope;       // as in FwdIO; the gradients of q and k are rotated back
  bool k_rotated;          // k is already rotated: rope applies to q and the gradients only
  const float* log_gain;
  const float* y;          // fp32 [B,H,T,D] forward output
  const float* stats;
  View dout;               // dL/d(output), element type E
  View dq, dk, dv;         // gradients, element type E (dk, dv: fp32 when kv_f32)
  float* dlog_gain;        // [H]
  // dk and dv are fp32 views whatever E is: the token-major backward in
  // passes sums dK and dV over the passes in fp32 and rounds them to E once
  // (launch_kv_cast) instead of after every pass
  bool kv_f32 = false;
};

template <int D, class E>
hipError_t launch_fwd(const FwdIO& io, float* part, int B, int H, int T, int C,
                      hipStream_t stream);
// Rotated keys [B*H][T][D] in E (out) from the key view k, for a forward or
// backward that then reads them with k_rotated set.
template <int D, class E>
hipError_t launch_rope_keys(View k, const float* rope, void* out, int BH, int H, int T,
                            hipStream_t stream);

// Backward workspace buffers of one pass (sizes: the pass's dS blocks, limb
// planes and qstat rows, gain partials per dQ item, dQ and dK/dV chunk
// partials).
struct BwdWork {
  float* dsbuf;       // dS spill, 32x16 blocks
  __bf16* limbs;      // per slice and query tile of the pass, six bf16 planes [32 rows][D]:
                      // Q limbs h, m, l; dY/Z limbs h, m, l ([BH][tile][plane][32][D])
  float* qstat;       // per slice and padded row of the pass's tiles: (-m, -D/Z)
  float* gain_part;   // per dQ item
  float* dq_part;     // dQ chunk partials
  float* kv_part;     // dK/dV chunk partials: [BH][part item][kDkdvKeys][2][D]
};

// dK/dV kernel of the backward (ca_bwd_dkdv.hip, its own translation unit).
template <int D, class E>
hipError_t launch_bwd_dkdv(const BwdIO& io, const BwdWork& ws, const BwdPass& pass,
                           const DkdvSplit& kvs, int BH, int H, int T, hipStream_t stream);
// The limb planes and row statistics are kept per whole 32-query tile (tile-
// major, rows past T zero) so that the dK/dV kernel stages a tile as one
// contiguous block with no bounds tests.
__host__ __device__ inline int bwd_pass_tiles(const BwdPass& p) { return p.qb - p.qa; }
// Limb planes per staged query tile: the Q limbs, then the three dY/Z limbs.
// bf16 operands have a bf16-valued Q (RoPE included, rounded as the
// reference rounds it), whose m and l limbs are zero: its tiles carry the h
// plane alone.  Workspaces are sized for six planes.
template <class E> __host__ __device__ constexpr int q_limb_planes() {
  return std::is_same<E, __bf16>::value ? 1 : 3;
}
__host__ __device__ constexpr int limb_tile_elems(int D, int planes = 6) { return planes * 32 * D; }
inline size_t bwd_limb_elems(int BH, const BwdPass& p, int D) {
  return (size_t)BH * bwd_pass_tiles(p) * limb_tile_elems(D);
}
inline size_t bwd_qstat_floats(int BH, const BwdPass& p) { return (size_t)BH * bwd_pass_tiles(p) * 32 * 2; }

template <int D, class E>
hipError_t launch_bwd(const BwdIO& io, const BwdWork& ws, const BwdPass& pass, const DqSplit& sp,
                      const DkdvSplit& kvs, int B, int H, int T, hipStream_t stream);
// dK and dV summed in fp32 ([BH][T][D] each, dk_sum and dv_sum) rounded to
// E into the views dk and dv (slices bh = 0 .. BH-1 of H heads per batch).
template <int D, class E>
hipError_t launch_kv_cast(const float* dk_sum, const float* dv_sum, View dk, View dv, int BH,
                          int H, int T, hipStream_t stream);

}  // namespace ca
