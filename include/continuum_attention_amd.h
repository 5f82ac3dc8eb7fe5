/* C ABI of the MI355X-native Continuum Attention operator (libca_hip.so).
 *
 * Plain pointers, sizes and an opaque HIP stream handle; no torch or HIP types
 * in the signatures.  All tensors are float32, contiguous, device-resident,
 * laid out [B, H, T, D] (row-major, D fastest).  The caller allocates every
 * output and workspace; the library allocates nothing.  Every call is
 * asynchronous on `stream` (NULL = the default stream) and returns CA_OK or an
 * error code whose text ca_last_error() returns (thread-local).
 *
 * Every tensor pointer of ca_fwd_f32 and ca_bwd_f32 (q, k, v, out, dout, dq,
 * dk, dv) must be 16-byte aligned: the kernels move rows as 16-byte vectors.
 *
 * This library replaces the native half of the reference operator
 * (akhadangi/continuum-attention):
 *   - the pybind extension built by _ca_cuda_extension
 *     (cuda/continuum_attention.py:35-63, 608-620), and
 *   - the per-query-tile bmm + kernel loops of _CAExactTiled.forward/backward
 *     (cuda/continuum_attention.py:650-766),
 * behind the same Python entry point continuum_attention(q,k,v,log_gain,
 * query_tile) (cuda/continuum_attention.py:768-783).
 */
#ifndef CONTINUUM_ATTENTION_AMD_H
#define CONTINUUM_ATTENTION_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CA_ABI_VERSION 1

enum {
  CA_OK = 0,
  CA_ERR_INVALID = 1,     /* bad pointer, alignment or shape */
  CA_ERR_UNSUPPORTED = 2, /* head dim or size outside the kernels' range */
  CA_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  CA_ERR_HIP = 4          /* a HIP launch or runtime call failed */
};

/* Version of this ABI (CA_ABI_VERSION). */
int ca_abi_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char* ca_last_error(void);

/* Workspace bound.  The reference's query_tile bounds the memory of its
 * materialised [B*H, query_tile, T] weights (cuda/continuum_attention.py:957);
 * here the workspaces are bounded instead: ca_fwd_f32 lengthens its work
 * splits until their partials fit the workspace it is given (none at all
 * needs no workspace), and ca_bwd_f32 runs in passes over ranges of
 * 128-query groups sized to the workspace it is given, of every slice or,
 * when not even one group of every slice fits, of sets of consecutive heads
 * of one batch (dK, dV and dlog_gain are summed over the passes in a fixed
 * order).  The size functions below report the full-speed size, or, when
 * that exceeds the cap, the size of the plan that fits under it (or, below
 * the least any plan needs, one 128-query group of one slice, that least
 * size).  The cap is process-wide; default 1 GiB, 0 = no cap.  Results are
 * deterministic for a given workspace size; different sizes sum in
 * different orders and may differ by rounding. */
int ca_set_workspace_cap(size_t bytes);
size_t ca_workspace_cap(void);

/* Bytes of device workspace ca_fwd_f32 asks for (may be 0; see above). */
size_t ca_fwd_workspace_bytes(int B, int H, int T, int D);

/* Forward: out = W(S) v with S = exp(log_gain[h]) / sqrt(D) * q k^T, exact CA
 * weights W (segment moments, half-token caps, causal).  Also writes per-row
 * statistics stats[B*H*T][2] = (row shift in log2 units, 1/Z) that
 * ca_bwd_f32 consumes.  log_gain has H entries.  D in {8, 16, 32, 64, 128}.
 * Replaces: _CAExactTiled.forward (cuda/continuum_attention.py:651-694) with
 * ext.forward / ext.forward_half / ext.direct_output
 * (cuda/continuum_attention.py:460-471, 556-590). */
int ca_fwd_f32(const float* q, const float* k, const float* v, const float* log_gain, float* out,
               float* stats, void* workspace, size_t workspace_bytes, int B, int H, int T, int D,
               void* stream);

/* Bytes of device workspace ca_bwd_f32 asks for (see above); the minimum is
 * what one 128-query group of every slice needs. */
size_t ca_bwd_workspace_bytes(int B, int H, int T, int D);

/* Backward (first order): given dout = dL/dout, writes dq, dk, dv ([B,H,T,D])
 * and dlog_gain[H] = sum dS * S.  out and stats must come from ca_fwd_f32 on
 * the same inputs.
 * Replaces: _CAExactTiled.backward (cuda/continuum_attention.py:697-766) with
 * ext.backward_fused / ext.backward_half(_gw16) / ext.backward
 * (cuda/continuum_attention.py:487-554, 592-605). */
int ca_bwd_f32(const float* q, const float* k, const float* v, const float* log_gain,
               const float* out, const float* stats, const float* dout, float* dq, float* dk,
               float* dv, float* dlog_gain, void* workspace, size_t workspace_bytes, int B, int H,
               int T, int D, void* stream);

/* Size of the static scratch array of ca_bwd_f32_noalloc, in MiB. */
#define CA_NOALLOC_SCRATCH_MB 512

/* ca_bwd_f32 without a workspace argument: the workspace is a static device
 * array of CA_NOALLOC_SCRATCH_MB MiB that the library holds on each device it
 * runs on until the process ends.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  It allocates
 * nothing.  The shape is checked first, as ca_bwd_f32 checks it; a shape
 * whose full backward workspace exceeds the array runs in passes sized to
 * it (over query ranges of every slice or of sets of heads), and a shape
 * whose least plan needs more would fail with CA_ERR_WORKSPACE before any
 * launch (none of the shapes the kernels accept does: one 128-query group of
 * one slice needs at most 32 MiB).  All calls on one device share its
 * array, so calls that overlap in time on one device (other streams, other
 * threads) race and must be serialised by the caller. */
int ca_bwd_f32_noalloc(const float* q, const float* k, const float* v, const float* log_gain,
                       const float* out, const float* stats, const float* dout, float* dq,
                       float* dk, float* dv, float* dlog_gain, int B, int H, int T, int D,
                       void* stream);

/* ---- Weight-materialising row kernels -------------------------------------
 * scores, grad_weights, weights and grad_scores are [BH][Q][K] fp32 (K
 * fastest); row (b, r) is query start + r and sees keys 0 .. start + r, so
 * start + Q <= K is required.  Entries of keys beyond a row's visible prefix
 * are written as exact zeros.  Scores are the scaled logits (natural units). */

/* Exact CA weights W and row statistics stats[BH*Q][2] = (row max m, 1/Z).
 * Replaces: ext.forward(scores, start) -> [W, stats]
 * (cuda/continuum_attention.py:578-590, kernel ca_weights_kernel :136-163). */
int ca_weights_f32(const float* scores, float* weights, float* stats, int BH, int Q, int K,
                   int start, void* stream);

/* Score VJP: grad_scores = dL/dscores given grad_weights = dL/dW, with the
 * weighted row mean computed in the kernel; also writes W when weights is not
 * NULL.  Replaces: ext.backward_fused(scores, gw, start) -> [W, dS]
 * (cuda/continuum_attention.py:538-554, kernel ca_backward_fused_kernel
 * :230-293); ext.backward(scores, W, stats, gw, means, start) -> dS
 * (:592-605) computes the same dS. */
int ca_weights_bwd_f32(const float* scores, const float* grad_weights, float* weights,
                       float* grad_scores, int BH, int Q, int K, int start, void* stream);

/* ---- The operator inside the decoder ---------------------------------------
 * The same forward and backward reading the decoder's qkv projection output
 * directly: qkv is [B, T, 3, H, D] (the projection's [B, T, 3*H*D] output,
 * token-major) of element type `dtype` (CA_DTYPE_*), q and k are rotated by
 * RoPE as the kernels read them, and the attention output is written
 * token-major [B, T, H*D] in the same type, ready for the output projection.
 * rope_cs is the fp32 table [T][D/2][2] = (cos, sin) of t * theta^(-2i/D)
 * for interleaved pairs (cuda/continuum_attention.py:826-835); NULL means no
 * rotation.  The rotation is computed as the reference computes it in the
 * operand type: for bf16 and fp16, q * cos and rotate(q) * sin each rounded
 * to that type and then their sum (pass the table's values rounded to the
 * type, as the reference casts cos and sin, to reproduce its rotation bit for
 * bit); for fp32 in fp32.  The gradients' rotation back is computed in fp32
 * and rounded once.  y is the fp32 [B, H, T, D] output the backward needs
 * (as ca_fwd_f32's `out`); stats as in ca_fwd_f32.  The forward's workspace
 * is ca_fwd_qkv_workspace_bytes (with RoPE it starts with the keys rotated
 * once for the kernels; a workspace of ca_fwd_workspace_bytes also works,
 * the kernels then rotate every staged key tile).  D in {8, 16, 32, 64,
 * 128}; qkv, out, dout and dqkv 8-byte (16-bit types) or 16-byte (fp32)
 * aligned, y 16-byte aligned.  One head's key and value rows of qkv must
 * span less than 4 GiB (CA_ERR_UNSUPPORTED otherwise).
 * Replaces: the reshape/permute/unbind of the projection, apply_rope, the
 * operator, and the transpose/reshape of its output in
 * ContinuumSelfAttention.forward (cuda/continuum_attention.py:848-854), and
 * their autograd. */
enum { CA_DTYPE_F32 = 0, CA_DTYPE_BF16 = 1, CA_DTYPE_F16 = 2 };

size_t ca_fwd_qkv_workspace_bytes(int B, int H, int T, int D);
int ca_fwd_qkv(const void* qkv, int dtype, const float* rope_cs, const float* log_gain, float* y,
               void* out, float* stats, void* workspace, size_t workspace_bytes, int B, int T,
               int H, int D, void* stream);

/* Backward of ca_fwd_qkv: dout [B, T, H*D] (dtype) -> dqkv [B, T, 3, H, D]
 * (dtype; the gradients of q and k rotated back by the transposed RoPE) and
 * dlog_gain[H].  With a workspace that holds the whole backward it runs in
 * one pass and writes the gradients in the element type (with RoPE and room
 * for B*H*T*D*4 more bytes, rounded up to 256, the keys are also rotated
 * once into it).  Under the cap, with less, it runs in passes over query
 * ranges of all slices or of sets of heads, summing dK and dV over the
 * passes in fp32 buffers at the start of the workspace and rounding them
 * into dqkv once (dq is complete within a pass).  ca_bwd_qkv_workspace_bytes
 * reports the one-pass size (with the rotated keys when they fit) while it
 * fits under the cap, else the size of the plan for the cap. */
size_t ca_bwd_qkv_workspace_bytes(int B, int H, int T, int D);
int ca_bwd_qkv(const void* qkv, int dtype, const float* rope_cs, const float* log_gain,
               const float* y, const float* stats, const void* dout, void* dqkv,
               float* dlog_gain, void* workspace, size_t workspace_bytes, int B, int T, int H,
               int D, void* stream);

/* ---- SwiGLU gate of the TinyLM MLP ----------------------------------------
 * No reference counterpart: F.silu(gate) * value of SwiGLU.forward
 * (architecture.py:186-188), run there as torch's silu and multiply kernels,
 * and their autograd with the chunk's gradient concatenation.  u [N][2H] fp32
 * = [gate | value] (the gate_up projection's output), h [N][H] fp32, dh
 * [N][H], du [N][2H] = [d gate | d value]; H % 4 == 0, pointers 16-byte
 * aligned. */
int ca_swiglu_fwd_f32(const float* u, float* h, int N, int H, void* stream);
int ca_swiglu_bwd_f32(const float* u, const float* dh, float* du, int N, int H, void* stream);

/* ---- RMSNorm of the decoder caller ----------------------------------------
 * y = weight * x * rsqrt(mean(x^2) + eps) over rows of C values
 * (RMSNorm.forward, cuda/continuum_attention.py:817-823, run there as a chain
 * of torch fp32 elementwise/reduction ops and their autograd).  x [N][C] fp32,
 * weight [C] fp32, y [N][C] of type ydtype (CA_DTYPE_*; bf16/fp16 round to
 * nearest even, the value autocast feeds the next linear layer), rstd [N]
 * fp32 = 1 / sqrt(mean(x^2) + eps).  C <= 4096. */
int ca_rmsnorm_fwd(const float* x, const float* weight, void* y, int ydtype, float* rstd, int N,
                   int C, float eps, void* stream);
/* Bytes of device workspace ca_rmsnorm_bwd needs (per-block dweight partials). */
size_t ca_rmsnorm_bwd_workspace_bytes(int N, int C);
/* dx [N][C] fp32 and dweight [C] fp32 from dy [N][C] (dydtype), x, weight and
 * the forward's rstd; dweight is summed in a fixed order. */
int ca_rmsnorm_bwd(const void* dy, int dydtype, const float* x, const float* weight,
                   const float* rstd, float* dx, float* dweight, void* workspace,
                   size_t workspace_bytes, int N, int C, void* stream);
/* Residual add feeding the norm, as the decoder block chains them
 * (x = x + branch, then RMSNorm of x; CADecoderBlock.forward and
 * ContinuumDecoderLM.forward, cuda/continuum_attention.py:878-880, 906-911):
 * sum_out = x + res (fp32, res of type rdtype) and y = RMSNorm(sum_out) in
 * one pass. */
int ca_add_rmsnorm_fwd(const float* x, const void* res, int rdtype, float* sum_out,
                       const float* weight, void* y, int ydtype, float* rstd, int N, int C,
                       float eps, void* stream);
/* Its gradient: dx = RMSNorm gradient at sum (the forward's sum_out) + dsum
 * (the gradient sum receives from its other consumers; NULL for none), fp32;
 * dres = dx in rdtype (the residual branch's gradient); dweight as in
 * ca_rmsnorm_bwd, same workspace size. */
int ca_add_rmsnorm_bwd(const void* dy, int dydtype, const float* dsum, const float* sum,
                       const float* weight, const float* rstd, float* dx, void* dres, int rdtype,
                       float* dweight, void* workspace, size_t workspace_bytes, int N, int C,
                       void* stream);

/* ---- AdamW step of the decoder's training loop ------------------------------
 * torch.optim.AdamW as the reference builds it (cuda/runtime.py:87-88) after
 * torch.nn.utils.clip_grad_norm_ (cuda/continuum_attention.py:1205-1228),
 * over a list of tensors described in device memory.  A tensor's gradient is
 * fp32 or bf16 (CA_DTYPE_*); `shadow`, when not NULL, is a bf16 copy of the
 * parameter that the step refreshes (round to nearest even: the value bf16
 * autocast would cast the weight to).  Every pointer is 16-byte aligned.
 * Work is split into chunks of ca_opt_chunk_elems() elements; `chunks` holds
 * nchunks pairs (tensor index, chunk index within the tensor), covering every
 * tensor exactly once.  No counterpart in the reference's native code (it
 * runs torch's optimizer kernels). */
typedef struct {
  float* param;
  const void* grad;
  float* exp_avg;
  float* exp_avg_sq;
  unsigned short* shadow;
  long long numel;
  int grad_dtype;
  int reserved;
} ca_opt_tensor;
int ca_opt_chunk_elems(void);
/* Sum of squares of every gradient (partial: nchunks floats of workspace),
 * then, on the device, total_norm = sqrt(sum) and
 * coef = min(1, max_norm / (total_norm + 1e-6)) (1 when max_norm <= 0). */
int ca_grad_clip_coef(const ca_opt_tensor* tensors, int ntensors, const int* chunks, int nchunks,
                      float* partial, float max_norm, float* total_norm, float* coef,
                      void* stream);
/* One AdamW step (step >= 1: the bias corrections' exponent) with every
 * gradient multiplied by *coef (coef NULL: 1). */
int ca_adamw_step(const ca_opt_tensor* tensors, int ntensors, const int* chunks, int nchunks,
                  const float* coef, float lr, float beta1, float beta2, float eps,
                  float weight_decay, int step, void* stream);
/* shadow = bf16(param) for every tensor that has a shadow. */
int ca_bf16_shadow(const ca_opt_tensor* tensors, int ntensors, const int* chunks, int nchunks,
                   void* stream);

/* ---- Diagnostics (no counterpart in the reference; used by bench.py) -------
 * Per-kernel timing with HIP events recorded on the launch stream around each
 * kernel launch of the calls above.  Kernel ids: 0 forward, 1 forward split
 * combine, 2 backward prep, 3 backward dK/dV, 4 backward dQ (with the gain
 * sum), 5 backward chunk-partial merge, 6 weights, 7 weights backward, 8 RMSNorm forward,
 * 9 RMSNorm backward, 10 SwiGLU forward, 11 SwiGLU backward.
 * ca_timing_enable(on) turns recording on/off and discards
 * unread records; ca_timing_read waits for the recorded events and returns the
 * summed milliseconds and launch counts per id (n entries), then clears them.
 * Not thread-safe; meant for single-threaded benchmarking. */
int ca_timing_enable(int on);
int ca_timing_read(double* total_ms, int* launches, int n);

/* Forces the work-split lengths of ca_fwd_f32 / ca_bwd_f32 (0 = automatic,
 * the default): forward split length in 32-key tiles, dQ chunk length in
 * 32-key stages, dK/dV chunk length in 32-query tiles.  While set, the
 * workspace-size functions return the sizes for the forced lengths, so size
 * queries and calls must see the same setting.  Process-wide, not
 * thread-safe; no counterpart in the reference: it lets tests run every
 * split length the automatic choice can pick (which depends on the device's
 * CU count) at small shapes. */
int ca_debug_set_splits(int fwd_split_tiles, int dq_chunk_stages, int dkdv_chunk_tiles);

#ifdef __cplusplus
}
#endif

#endif /* CONTINUUM_ATTENTION_AMD_H */
