// Device-side conversions between packed varlen rows and padded batches (gfx950).
//
// Reference: src/scree/_core.py:161-301 (to_padded / from_padded) and the HF
// bridge built on them (src/scree/bridges/_hf_padded.py:15-46).  The
// reference's torch branch loops over sequences on the host with one slice
// copy each (to_padded, :257-266) and one mask-row .item() each
// (from_padded, :263); here each direction is one gather/scatter launch over
// rows, plus a small counting/scan launch that turns a mask into int32
// offsets on the device.
//
// Everything is byte-generic: a "row" is `row_bytes` bytes (one token's
// features in any dtype).  Rows move in 16-byte units when every row and both
// base pointers are 16-byte aligned, else in 4-byte or 1-byte units.  Each
// padded row is handled by a group of `tpr` threads (a power of two); a
// workgroup covers 256 / tpr padded rows per trip and strides over the rest.

#include <algorithm>
#include <cstring>

#include "common.h"

namespace scree {
namespace {

constexpr int kPadThreads = 256;

template <int U>
struct Unit;
template <>
struct Unit<16> {
  typedef uint4 type;
};
template <>
struct Unit<4> {
  typedef uint32_t type;
};
template <>
struct Unit<1> {
  typedef uint8_t type;
};

// Streaming (non-temporal) stores for to_padded's output (every byte written
// once): config-2 shape (19,758 x 4,096 bf16 into 64 x 829 rows) 112 -> 107 us
// with inputs not in the caches.  from_padded keeps plain stores: with them
// it ran 62 us against 67 from cold inputs (the non-temporal form was faster,
// 55 against 60 us, only when its input was still cached from the last call).
template <typename UT>
__device__ __forceinline__ void st_nt(UT* p, UT v) { __builtin_nontemporal_store(v, p); }
template <>
__device__ __forceinline__ void st_nt<uint4>(uint4* p, uint4 v) { st16_nt(p, v); }

// The fill value of unit c of a row: the 16-byte pattern repeats the fill
// element (16 is a multiple of every element size), so the unit starting at
// byte c*U of the row takes the pattern bytes at (c*U) % 16.
template <int U>
__device__ __forceinline__ typename Unit<U>::type fill_unit(const uint4& f, int64_t c) {
  if constexpr (U == 16) {
    return f;
  } else {
    const int w = (int)((c * U) & 15) >> 2;
    const uint32_t word = w == 0 ? f.x : w == 1 ? f.y : w == 2 ? f.z : f.w;
    if constexpr (U == 4) return word;
    else return (uint8_t)(word >> (8 * (int)(c & 3)));
  }
}

// Offsets are clamped into [0, total] and made non-decreasing per sequence,
// so malformed offsets cannot move a copy outside `values`.
__device__ __forceinline__ void seq_bounds(const int32_t* off, int b, int64_t total,
                                           int64_t& start, int64_t& len) {
  start = min<int64_t>(max<int64_t>(off[b], 0), total);
  const int64_t end = min<int64_t>(max<int64_t>(off[b + 1], start), total);
  len = end - start;
}

// padded[b, t] = values[start_b + t - lo_b] for lo_b <= t < lo_b + len_b, else
// the fill row; mask[b, t] = (row is valid).  lo_b = 0 (right padding) or
// max_len - len_b (left padding); sequences longer than max_len keep their
// first max_len rows.
template <int U>
__global__ __launch_bounds__(kPadThreads) void to_padded_kernel(
    const uint8_t* __restrict__ values, const int32_t* __restrict__ off, int64_t total,
    int64_t max_len, int64_t nrows, int64_t upr, int tpr, int left, uint4 fill,
    uint8_t* __restrict__ padded, uint8_t* __restrict__ mask) {
  typedef typename Unit<U>::type UT;
  const int rpb = kPadThreads / tpr;
  const int sub = threadIdx.x / tpr, lane = threadIdx.x % tpr;
  for (int64_t row = (int64_t)blockIdx.x * rpb + sub; row < nrows; row += (int64_t)gridDim.x * rpb) {
    const int b = (int)(row / max_len);
    const int64_t t = row - (int64_t)b * max_len;
    int64_t start, len;
    seq_bounds(off, b, total, start, len);
    len = min(len, max_len);
    const int64_t lo = left ? max_len - len : 0;
    const bool valid = t >= lo && t < lo + len;
    UT* dst = reinterpret_cast<UT*>(padded + row * upr * U);
    if (valid) {
      const UT* src = reinterpret_cast<const UT*>(values + (start + t - lo) * upr * U);
      for (int64_t c = lane; c < upr; c += tpr) st_nt(dst + c, src[c]);
    } else {
      for (int64_t c = lane; c < upr; c += tpr) st_nt(dst + c, fill_unit<U>(fill, c));
    }
    if (lane == 0 && mask) mask[row] = valid ? 1 : 0;
  }
}

// values[off[b] + t] = padded[b, t] for t < len_b (the first len_b rows of
// each batch row, the reference's right-padding convention).
template <int U>
__global__ __launch_bounds__(kPadThreads) void from_padded_kernel(
    const uint8_t* __restrict__ padded, const int32_t* __restrict__ off, int64_t total,
    int64_t max_len, int64_t nrows, int64_t upr, int tpr, uint8_t* __restrict__ values) {
  typedef typename Unit<U>::type UT;
  const int rpb = kPadThreads / tpr;
  const int sub = threadIdx.x / tpr, lane = threadIdx.x % tpr;
  for (int64_t row = (int64_t)blockIdx.x * rpb + sub; row < nrows; row += (int64_t)gridDim.x * rpb) {
    const int b = (int)(row / max_len);
    const int64_t t = row - (int64_t)b * max_len;
    int64_t start, len;
    seq_bounds(off, b, total, start, len);
    if (t >= len) continue;
    const UT* src = reinterpret_cast<const UT*>(padded + row * upr * U);
    UT* dst = reinterpret_cast<UT*>(values + (start + t) * upr * U);
    for (int64_t c = lane; c < upr; c += tpr) dst[c] = src[c];
  }
}

// counts[b] = number of nonzero bytes in mask row b (one workgroup per row).
__global__ __launch_bounds__(kPadThreads) void mask_count_kernel(const uint8_t* __restrict__ mask,
                                                                 int64_t max_len,
                                                                 int32_t* __restrict__ offsets) {
  __shared__ int part[kPadThreads / 64];
  const int b = blockIdx.x;
  const uint8_t* m = mask + (int64_t)b * max_len;
  int c = 0;
  for (int64_t t = threadIdx.x; t < max_len; t += kPadThreads) c += m[t] != 0;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) c += __shfl_xor(c, s, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int tot = 0;
    for (int w = 0; w < kPadThreads / 64; ++w) tot += part[w];
    offsets[b + 1] = tot;
  }
}

// In-place inclusive scan of offsets[1 .. batch], offsets[0] = 0 (one block);
// with `zero` set the counts are taken as 0 (an empty padded batch).
__global__ __launch_bounds__(1024) void offsets_scan_kernel(int32_t* __restrict__ offsets, int batch,
                                                            int zero) {
  __shared__ int wsum[16];
  __shared__ int carry_s;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) {
    carry_s = 0;
    offsets[0] = 0;
  }
  __syncthreads();
  for (int base = 0; base < batch; base += 1024) {
    const int i = base + tid;
    int v = i < batch && !zero ? offsets[i + 1] : 0;
    for (int d = 1; d < 64; d <<= 1) {  // wave-inclusive scan
      const int n = __shfl_up(v, d, 64);
      if (lane >= d) v += n;
    }
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    int before = carry_s;
    for (int j = 0; j < w; ++j) before += wsum[j];
    if (i < batch) offsets[i + 1] = before + v;
    __syncthreads();
    if (tid == 1023) carry_s = before + v;
    __syncthreads();
  }
}

inline bool aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int unit_bytes(int64_t row_bytes, const void* a, const void* b) {
  if (row_bytes % 16 == 0 && aligned(a, 16) && aligned(b, 16)) return 16;
  if (row_bytes % 4 == 0 && aligned(a, 4) && aligned(b, 4)) return 4;
  return 1;
}

void row_shape(int64_t upr, int64_t nrows, int& tpr, unsigned& grid) {
  tpr = 1;
  while (tpr < upr && tpr < 64) tpr <<= 1;
  const int rpb = kPadThreads / tpr;
  const int64_t need = (nrows + rpb - 1) / rpb;
  grid = (unsigned)std::min<int64_t>(need, 65536);  // the kernels stride over the rest
}

}  // namespace
}  // namespace scree

using namespace scree;

extern "C" int scree_to_padded(const void* values, const int32_t* offsets, int batch,
                               int64_t total_tokens, int64_t max_len, int64_t row_bytes,
                               int left, const void* fill_elem, int elem_bytes, void* padded,
                               void* mask, void* stream) {
  if (batch < 1 || total_tokens < 0 || max_len < 0 || row_bytes < 1)
    return set_error(SCREE_ERR_INVALID, "scree_to_padded: bad sizes");
  if (max_len == 0) return SCREE_OK;  // an empty padded batch: nothing to write
  if (!offsets || !padded || (!values && total_tokens > 0))
    return set_error(SCREE_ERR_INVALID, "scree_to_padded: null pointer");
  if (!(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8 ||
        elem_bytes == 16) || row_bytes % elem_bytes != 0 || !fill_elem)
    return set_error(SCREE_ERR_INVALID, "scree_to_padded: element size %d does not tile the row",
                     elem_bytes);
  const int64_t nrows = (int64_t)batch * max_len;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t pat[16];
  for (int i = 0; i < 16; ++i) pat[i] = static_cast<const uint8_t*>(fill_elem)[i % elem_bytes];
  const int u = unit_bytes(row_bytes, values ? values : padded, padded);
  const int64_t upr = row_bytes / u;
  int tpr;
  unsigned grid;
  row_shape(upr, nrows, tpr, grid);
  const uint8_t* v = static_cast<const uint8_t*>(values);
  uint8_t* p = static_cast<uint8_t*>(padded);
  uint8_t* m = static_cast<uint8_t*>(mask);
  uint4 f;
  std::memcpy(&f, pat, 16);
  if (u == 16)
    hipLaunchKernelGGL(to_padded_kernel<16>, dim3(grid), dim3(kPadThreads), 0, s, v, offsets,
                       total_tokens, max_len, nrows, upr, tpr, left, f, p, m);
  else if (u == 4)
    hipLaunchKernelGGL(to_padded_kernel<4>, dim3(grid), dim3(kPadThreads), 0, s, v, offsets,
                       total_tokens, max_len, nrows, upr, tpr, left, f, p, m);
  else
    hipLaunchKernelGGL(to_padded_kernel<1>, dim3(grid), dim3(kPadThreads), 0, s, v, offsets,
                       total_tokens, max_len, nrows, upr, tpr, left, f, p, m);
  return check_launch("scree_to_padded");
}

extern "C" int scree_padded_offsets(const void* mask, int batch, int64_t max_len,
                                    int32_t* offsets, void* stream) {
  if (!offsets || (!mask && max_len > 0))
    return set_error(SCREE_ERR_INVALID, "scree_padded_offsets: null pointer");
  if (batch < 1 || max_len < 0)
    return set_error(SCREE_ERR_INVALID, "scree_padded_offsets: bad sizes");
  if ((int64_t)batch * max_len > 0x7fffffff)
    return set_error(SCREE_ERR_INVALID, "scree_padded_offsets: batch * max_len must fit int32");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (max_len > 0)
    hipLaunchKernelGGL(mask_count_kernel, dim3(batch), dim3(kPadThreads), 0, s,
                       static_cast<const uint8_t*>(mask), max_len, offsets);
  hipLaunchKernelGGL(offsets_scan_kernel, dim3(1), dim3(1024), 0, s, offsets, batch,
                     max_len == 0 ? 1 : 0);
  return check_launch("scree_padded_offsets");
}

extern "C" int scree_from_padded(const void* padded, const int32_t* offsets, int batch,
                                 int64_t max_len, int64_t row_bytes, int64_t total_tokens,
                                 void* values, void* stream) {
  if (!offsets || (total_tokens > 0 && (!padded || !values)))
    return set_error(SCREE_ERR_INVALID, "scree_from_padded: null pointer");
  if (batch < 1 || max_len < 0 || row_bytes < 1 || total_tokens < 0)
    return set_error(SCREE_ERR_INVALID, "scree_from_padded: bad sizes");
  if (total_tokens == 0 || max_len == 0) return SCREE_OK;
  const int64_t nrows = (int64_t)batch * max_len;
  const int u = unit_bytes(row_bytes, padded, values);
  const int64_t upr = row_bytes / u;
  int tpr;
  unsigned grid;
  row_shape(upr, nrows, tpr, grid);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* p = static_cast<const uint8_t*>(padded);
  uint8_t* v = static_cast<uint8_t*>(values);
  if (u == 16)
    hipLaunchKernelGGL(from_padded_kernel<16>, dim3(grid), dim3(kPadThreads), 0, s, p, offsets,
                       total_tokens, max_len, nrows, upr, tpr, v);
  else if (u == 4)
    hipLaunchKernelGGL(from_padded_kernel<4>, dim3(grid), dim3(kPadThreads), 0, s, p, offsets,
                       total_tokens, max_len, nrows, upr, tpr, v);
  else
    hipLaunchKernelGGL(from_padded_kernel<1>, dim3(grid), dim3(kPadThreads), 0, s, p, offsets,
                       total_tokens, max_len, nrows, upr, tpr, v);
  return check_launch("scree_from_padded");
}
