/*
 * scree_hip.h -- C ABI of the MI355X (gfx950) varlen kernel library
 * (libscree_hip.so).
 *
 * Conventions
 *   - Plain pointers and sizes only.  Every tensor is caller-owned device
 *     memory; the library never allocates.  Scratch memory is passed in as a
 *     `workspace` whose size the matching *_workspace_bytes() call reports.
 *   - `stream` is a hipStream_t passed as void* (NULL = legacy default
 *     stream).  All work is enqueued on it; no call synchronises the host.
 *   - Return value: SCREE_OK (0) or a negative SCREE_ERR_* code.  Arguments
 *     are validated on the host before anything is launched;
 *     scree_last_error() returns a message for the calling thread's last
 *     failure.
 *   - dtype codes: SCREE_DTYPE_F32 / F16 / BF16.  Attention takes F16 or
 *     BF16 on the matrix-instruction kernels (the types the reference's GPU
 *     launcher asserts, src/scree/kernels/triton/varlen_attention.py:213-215)
 *     and F32 on FP32-FMA kernels (what the reference's Array-level torch
 *     branch computes fp32 arrays with, reference/varlen_attention.py:90-113:
 *     every operand stays fp32; no grouped-query dK/dV split); the norms take
 *     all three.
 *   - `cu_seqlens` is the int32 offsets vector of length batch+1 (the
 *     scree.Array `offsets`, src/scree/_core.py:22-62), resident on the
 *     device.  It is read only by device code: no call copies it to the host.
 *
 * Layouts
 *   - Attention tensors are (total_tokens, heads, head_dim) with the
 *     head_dim axis contiguous; row and head strides are given in elements
 *     and must keep every row 16-byte aligned.  head_dim is 16, 32, 64, 128
 *     or 256 (SCREE_ERR_UNSUPPORTED otherwise); the reference's launcher
 *     takes any power of two (src/scree/kernels/triton/varlen_attention.py:217).  lse and delta are contiguous
 *     (total_tokens, heads) fp32.  With total_tokens == 0 (every sequence
 *     empty) the tensor pointers may be NULL, as empty tensors may have no
 *     storage: the call validates the rest and launches nothing.
 *   - Norm tensors are contiguous (rows, dim); rstd / mean are (rows) fp32.
 */
#ifndef SCREE_HIP_H
#define SCREE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SCREE_ABI_VERSION 1

enum {
  SCREE_DTYPE_F32 = 0,
  SCREE_DTYPE_F16 = 1,
  SCREE_DTYPE_BF16 = 2
};

enum {
  SCREE_OK = 0,
  SCREE_ERR_INVALID = -1,     /* bad pointer, size, stride or alignment   */
  SCREE_ERR_UNSUPPORTED = -2, /* dtype / head_dim this build does not do  */
  SCREE_ERR_WORKSPACE = -3,   /* workspace missing or too small           */
  SCREE_ERR_HIP = -4          /* the HIP runtime reported a launch error  */
};

/* Library ABI version (SCREE_ABI_VERSION of the build). */
int scree_abi_version(void);

/* Message describing the calling thread's most recent failure ("" if none). */
const char* scree_last_error(void);

/* ---------------------------------------------------------------- attention
 * Replaces the Triton launchers
 *   varlen_attention_triton           src/scree/kernels/triton/varlen_attention.py:165-268
 *   varlen_attention_triton_backward  src/scree/kernels/triton/_backward.py:288-396
 * and the padded (batch, cdiv(max_seq, 64), heads) grid plus the host
 * `.item()` sync on max_seq they use (varlen_attention.py:220-236,
 * _backward.py:320-321).
 */

/* Bytes of workspace scree_attn_schedule needs for `batch` sequences holding
 * `total_tokens` tokens in all (independent of heads and causality): a
 * 16-byte header and two lists of ceil(total_tokens / 128) + batch 16-byte
 * items, plus, past 2048 sequences (where the lists keep natural order),
 * batch + 1 prefix sums rounded up to 16 bytes. */
size_t scree_attn_workspace_bytes(int batch, int64_t total_tokens, int head_dim);

/* 1 when scree_attn_fwd / scree_attn_fwd_gqa read a work list that
 * scree_attn_schedule must write first; 0 when the forward derives every
 * workgroup's item from cu_seqlens itself and writes the header and the
 * work-order list into its workspace as scree_attn_schedule writes them, so
 * the backward calls of the same problem (same cu_seqlens, total_tokens,
 * heads, head_dim, causal) on that workspace need no schedule call.  The
 * sequence-major list, which launches of many workgroups per XCD read, is
 * left as it was: any other call on the workspace -- a forward or backward
 * of another problem, e.g. with more heads -- needs scree_attn_schedule.
 * The forward derives for at most 64 sequences in a launch of at most 2048
 * workgroups at head_dim <= 64, 1024 at head_dim 128, 512 at 256, i.e.
 * (ceil(total_tokens / 128) + batch) * heads within that bound; past it the
 * derivation (~150 instructions per workgroup) costs more than the scheduler
 * launch.  Backward calls that no forward on their workspace precedes always
 * need scree_attn_schedule.  No counterpart in the reference. */
int scree_attn_needs_schedule(int batch, int64_t total_tokens, int heads, int head_dim);

/* Workspace bytes that let the grouped-query backward split each K/V head's
 * group of query heads over several workgroups (>= scree_attn_workspace_bytes;
 * equal to it when heads == kv_heads or the grid already fills the GPU).
 * The schedule occupies the front as before; the rest holds the parts' fp32
 * dK / dV sums, which a reduce kernel adds up after the dK/dV pass.  scree_attn_bwd_gqa / _bwd_dkv_gqa split
 * only when given at least this many bytes, else they run one workgroup per
 * (item, K/V head).  A split backward writes its partial sums into the
 * workspace, so backward calls that may run at the same time (different
 * streams) need workspaces of their own; the schedule part is only read.
 * No counterpart in the reference (it has no grouped-query attention,
 * docs/kernels.md:177). */
size_t scree_attn_bwd_workspace_bytes_gqa(int batch, int64_t total_tokens, int heads,
                                          int kv_heads, int head_dim);

/* Build the longest-work-first tile list for `cu_seqlens` into `workspace`.
 * Must precede scree_attn_fwd with the same cu_seqlens, head_dim and causal
 * flag when scree_attn_needs_schedule returns 1, and the backward calls
 * unless a forward on the same workspace came first (calling it anyway is
 * harmless); the workspace may then be reused by any number of forward and
 * backward calls.  A call that reads a workspace neither wrote gives wrong
 * results but never reads or writes outside its tensors: the kernels skip
 * items that no schedule can hold.  No counterpart in the reference (its
 * grid is padded, src/scree/kernels/triton/varlen_attention.py:236). */
int scree_attn_schedule(const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                        int head_dim, int causal, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Forward: o = softmax(scale * q k^T [causal-masked]) v per sequence and
 * lse = natural-log logsumexp of the scaled scores per (token, head).
 * strides[8] = {q_row, q_head, k_row, k_head, v_row, v_head, o_row, o_head}.
 * When scree_attn_needs_schedule returns 0 it derives its work items from
 * cu_seqlens and writes the header and work-order list into `workspace`;
 * otherwise it reads the lists scree_attn_schedule wrote there.
 * Replaces _varlen_attn_fwd_kernel + launcher
 * (src/scree/kernels/triton/varlen_attention.py:35-268). */
int scree_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                   const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                   int head_dim, const int64_t* strides, float softmax_scale, int causal,
                   int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Backward: dq, dk, dv from dout, the forward's inputs, its output o and lse.
 * delta (total_tokens, heads) fp32 receives rowsum(o * dout).
 * strides[16] = {dout, q, k, v, o, dq, dk, dv} x {row, head}.
 * Replaces _varlen_attn_bwd_{preprocess,dkv,dq}_kernel + launcher
 * (src/scree/kernels/triton/_backward.py:36-396). */
int scree_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                   const void* o, const float* lse, void* dq, void* dk, void* dv, float* delta,
                   const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                   int head_dim, const int64_t* strides, float softmax_scale, int causal,
                   int dtype, const void* workspace, size_t workspace_bytes, void* stream);

/* The two stages of scree_attn_bwd, for callers that schedule or time them
 * separately; dq must run first because it writes delta.
 * scree_attn_bwd_dq: dq and delta.  strides[12] = {dout, q, k, v, o, dq} x {row, head}.
 * scree_attn_bwd_dkv: dk and dv from delta.  strides[12] = {dout, q, k, v, dk, dv} x {row, head}.
 * Together they replace the reference's three backward kernels
 * (src/scree/kernels/triton/_backward.py:36-285): Delta is folded into the
 * dQ pass. */
int scree_attn_bwd_dq(const void* dout, const void* q, const void* k, const void* v,
                      const void* o, const float* lse, void* dq, float* delta,
                      const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                      int head_dim, const int64_t* strides, float softmax_scale, int causal,
                      int dtype, const void* workspace, size_t workspace_bytes, void* stream);

int scree_attn_bwd_dkv(const void* dout, const void* q, const void* k, const void* v,
                       const float* lse, const float* delta, void* dk, void* dv,
                       const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                       int head_dim, const int64_t* strides, float softmax_scale, int causal,
                       int dtype, const void* workspace, size_t workspace_bytes, void* stream);

/* Grouped-query forms of the four calls above: q, o, dout, dq, lse and delta
 * have `heads` heads, k, v, dk and dv have `kv_heads` (a divisor of heads);
 * query head h attends with K/V head h / (heads / kv_heads), and dk / dv sum
 * the contributions of each group's query heads (no atomics: one workgroup
 * owns each K/V block and sweeps its group).  With kv_heads == heads they are
 * the calls above.  No counterpart in the reference, whose Q, K and V must
 * share a head count (docs/kernels.md:177 lists GQA as missing); its head
 * indexing is src/scree/kernels/triton/varlen_attention.py:64-66,84-90. */
int scree_attn_fwd_gqa(const void* q, const void* k, const void* v, void* o, float* lse,
                       const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                       int kv_heads, int head_dim, const int64_t* strides, float softmax_scale,
                       int causal, int dtype, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Allocation-free forward.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as scree_attn_fwd_gqa minus the workspace: the work lists are
 * built on `stream` (by scree_attn_schedule, or by the forward itself when
 * scree_attn_needs_schedule returns 0) into a static device array of
 * SCREE_ATTN_NOALLOC_SCHEDULE_BYTES per GPU, which holds
 * scree_attn_workspace_bytes() up to that size: 2 * (ceil(total_tokens / 128)
 * + batch) * 16 + 16 bytes (plus the prefix sums past 2048 sequences), i.e.
 * about 8 million tokens.  Larger problems get
 * SCREE_ERR_UNSUPPORTED before anything is launched.  Calls no allocating
 * routine.  Calls that overlap on one GPU (several streams or host threads)
 * race on the array; serialise them. */
#define SCREE_ATTN_NOALLOC_SCHEDULE_BYTES (1 << 21)
int scree_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* o, float* lse,
                           const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                           int kv_heads, int head_dim, const int64_t* strides,
                           float softmax_scale, int causal, int dtype, void* stream);
int scree_attn_bwd_gqa(const void* dout, const void* q, const void* k, const void* v,
                       const void* o, const float* lse, void* dq, void* dk, void* dv, float* delta,
                       const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                       int kv_heads, int head_dim, const int64_t* strides, float softmax_scale,
                       int causal, int dtype, const void* workspace, size_t workspace_bytes,
                       void* stream);
int scree_attn_bwd_dq_gqa(const void* dout, const void* q, const void* k, const void* v,
                          const void* o, const float* lse, void* dq, float* delta,
                          const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                          int kv_heads, int head_dim, const int64_t* strides, float softmax_scale,
                          int causal, int dtype, const void* workspace, size_t workspace_bytes,
                          void* stream);
int scree_attn_bwd_dkv_gqa(const void* dout, const void* q, const void* k, const void* v,
                           const float* lse, const float* delta, void* dk, void* dv,
                           const int32_t* cu_seqlens, int batch, int64_t total_tokens, int heads,
                           int kv_heads, int head_dim, const int64_t* strides,
                           float softmax_scale, int causal, int dtype, const void* workspace,
                           size_t workspace_bytes, void* stream);

/* -------------------------------------------------------------------- norms
 * Replace varlen_rmsnorm_triton (src/scree/kernels/triton/varlen_rmsnorm.py:17-99)
 * and varlen_layernorm_triton (src/scree/kernels/triton/varlen_layernorm.py:14-109).
 * `weight` / `bias` may be NULL; when given they have the activation dtype
 * (the reference rounds them to it, varlen_rmsnorm.py:79,
 * varlen_layernorm.py:84,89).  The backward passes have no counterpart in the
 * reference, which is forward-only.
 */

/* Bytes of workspace a norm backward needs for a (rows, dim) input. */
size_t scree_norm_bwd_workspace_bytes(int64_t rows, int64_t dim);

/* y = x / sqrt(mean(x^2) + eps) [* weight]; rstd (may be NULL) = 1/sqrt(mean(x^2)+eps). */
int scree_rmsnorm_fwd(const void* x, const void* weight, void* y, float* rstd, int64_t rows,
                      int64_t dim, float eps, int dtype, void* stream);

/* dx and (if weight != NULL) dweight, stored in `dparam_dtype`, from dy, x,
 * weight and the forward's rstd. */
int scree_rmsnorm_bwd(const void* dy, const void* x, const void* weight, const float* rstd,
                      void* dx, void* dweight, int dparam_dtype, int64_t rows, int64_t dim,
                      int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* y = (x - mean) / sqrt(var + eps) [* weight] [+ bias] with the population
 * variance; mean / rstd (may be NULL) receive the row statistics. */
int scree_layernorm_fwd(const void* x, const void* weight, const void* bias, void* y,
                        float* mean, float* rstd, int64_t rows, int64_t dim, float eps,
                        int dtype, void* stream);

/* dx, dweight (if weight != NULL) and dbias (if dbias != NULL), the
 * parameter gradients stored in `dparam_dtype`. */
int scree_layernorm_bwd(const void* dy, const void* x, const void* weight, const float* mean,
                        const float* rstd, void* dx, void* dweight, void* dbias,
                        int dparam_dtype, int64_t rows, int64_t dim, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Fused residual add + RMSNorm, the pre-norm transformer step
 *   h = x + residual;  y = rmsnorm(h) [* weight]
 * of the reference's block (examples/03_train_step.py:46-48: h1 = x +
 * attn_proj, then varlen_rmsnorm(h1)) in one pass: h is x + residual rounded
 * to `dtype` exactly as the separate addition rounds it, and y is
 * scree_rmsnorm_fwd of that h, bit for bit.  h and y must not alias x or
 * residual.  No fused counterpart in the reference. */
int scree_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight, void* h,
                          void* y, float* rstd, int64_t rows, int64_t dim, float eps, int dtype,
                          void* stream);

/* Backward of scree_add_rmsnorm_fwd: dx (the gradient of both x and residual)
 * = dh + the RMSNorm input gradient of dy at h, and dweight as in
 * scree_rmsnorm_bwd.  dh, the gradient reaching h by the residual stream, may
 * be NULL (then dx is scree_rmsnorm_bwd's dx).  `workspace` as for
 * scree_rmsnorm_bwd (scree_norm_bwd_workspace_bytes). */
int scree_add_rmsnorm_bwd(const void* dy, const void* dh, const void* h, const void* weight,
                          const float* rstd, void* dx, void* dweight, int dparam_dtype,
                          int64_t rows, int64_t dim, int dtype, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ softmax
 * Replaces scree.kernels.reference.varlen_softmax
 * (src/scree/kernels/reference/varlen_softmax.py:13-63), whose torch branch
 * loops over sequences on the host (:44-51); the reference has no GPU kernel.
 * x and y are contiguous (total_tokens, features) in `dtype`: for every
 * sequence s (rows cu_seqlens[s] .. cu_seqlens[s+1]) and feature column c,
 * y = softmax over the sequence's rows of x[., c].  Statistics in fp32.
 */
int scree_varlen_softmax(const void* x, void* y, const int32_t* cu_seqlens, int batch,
                         int64_t total_tokens, int64_t features, int dtype, void* stream);

/* Gradient of scree_varlen_softmax: dx = y * (dy - sum over the sequence's
 * rows of y * dy), per column.  No kernel in the reference: its torch branch
 * is differentiated by autograd through torch.softmax per sequence
 * (varlen_softmax.py:44-51). */
int scree_varlen_softmax_bwd(const void* y, const void* dy, void* dx, const int32_t* cu_seqlens,
                             int batch, int64_t total_tokens, int64_t features, int dtype,
                             void* stream);

/* ------------------------------------------------------------ padded <-> packed
 * Replace the host loops of scree.to_padded / scree.from_padded
 * (src/scree/_core.py:161-266 and :269-301; torch branch :240-266 and
 * :278-285) and so the HF bridge built on them (src/scree/bridges/_hf_padded.py:15-46).
 * A row is `row_bytes` bytes (one token's features, any dtype).
 */

/* padded (batch, max_len, row) and mask (batch, max_len) bytes 0/1 (may be
 * NULL) from packed values (total_tokens, row) and int32 offsets (batch+1):
 * row t of batch row b is value row offsets[b] + t - lo_b when lo_b <= t <
 * lo_b + len_b (lo_b = 0, or max_len - len_b when `left`), else the fill
 * element (`elem_bytes` bytes at host pointer `fill_elem`, repeated).
 * Sequences longer than max_len keep their first max_len rows. */
int scree_to_padded(const void* values, const int32_t* offsets, int batch, int64_t total_tokens,
                    int64_t max_len, int64_t row_bytes, int left, const void* fill_elem,
                    int elem_bytes, void* padded, void* mask, void* stream);

/* offsets (batch+1, int32, device) from a (batch, max_len) byte mask: the
 * per-row count of nonzero bytes, exclusive-scanned (the reference's
 * lengths = mask[i].sum(), _core.py:282).  batch * max_len must fit int32. */
int scree_padded_offsets(const void* mask, int batch, int64_t max_len, int32_t* offsets,
                         void* stream);

/* values (total_tokens, row) from padded (batch, max_len, row): value row
 * offsets[b] + t = padded[b, t] for t < len_b (the first len_b rows of each
 * batch row, _core.py:283-284).  total_tokens = offsets[batch]. */
int scree_from_padded(const void* padded, const int32_t* offsets, int batch, int64_t max_len,
                      int64_t row_bytes, int64_t total_tokens, void* values, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SCREE_HIP_H */
