// Varlen softmax along the ragged dimension (gfx950).
//
// Reference: src/scree/kernels/reference/varlen_softmax.py:13-63 — for every
// sequence s (rows offsets[s] .. offsets[s+1]) and every feature column c,
// y[r, c] = exp(x[r, c] - max_r x[., c]) / sum_r exp(x[r, c] - max_r x[., c]).
// The reference computes it with a Python loop over sequences (torch.softmax
// / numpy per slice); it has no GPU kernel.
//
// Layout: x, y contiguous (total_tokens, features).  One workgroup per
// (sequence, column chunk): its 256 threads (512 in the backward) are `ct`
// column lanes (each owning VEC adjacent columns, one 16-byte vector when the
// row allows it) times `threads / ct` row lanes that stride over the
// sequence's rows.  Forward pass 1 finds each column's (max, sum of
// exponentials); the row lanes merge through LDS; pass 2 writes the
// normalised values with streaming stores.  Each thread keeps its first
// kSmCache rows in registers as loaded, takes their max and then their sum,
// and writes them in pass 2 from there, so a sequence of at most
// kSmCache * (row lanes) rows reads x once.  Rows past that (long
// sequences) are streamed first with an online (max, sum), one exp per
// element, merged into the held rows' result, and re-read in pass 2 (usually
// from the L2 / MALL).  The backward holds y and dy the same way when the
// whole sequence fits, else streams every row twice.  Row lanes merge by a
// fixed tree: results are deterministic.
// Statistics are fp32 for every input dtype; y has x's dtype.

#include <type_traits>

#include "common.h"

namespace scree {
namespace {

constexpr int kSmThreadsBwd = 512;     // backward: more row lanes, so that held rows cover longer sequences
constexpr int kUnroll = 4;              // rows per thread per loop trip (loads issued together)
// Forward: rows per thread held in registers, 8 for every dtype: 80
// registers for 16-bit types (6 waves per SIMD; 16 rows took 123-151, 3-4
// waves, and ran 74 / 91 us bf16 / fp16 against 70 / 72 at 19,758 x 4,096),
// 64 for fp32 (8 waves; 131 us against 140 with 16 rows).
constexpr int kSmCache = 8;
// Forward: 512 threads per workgroup, narrowing to no fewer than 8 column
// lanes (128-byte row segments, whole cache lines).  With inputs not already
// cached (each call reading fresh data), 4 lanes of 256 threads took 94.5 us
// at the config-2 shape in bf16 against 77.7 us (the same 69 us either way
// when the input was still cached from the previous call); fp32 169 -> 140.
constexpr int kSmThreadsFwd = 512;
constexpr int kSmMinCtFwd = 8;
constexpr int kSmCacheBwd = 10;         // backward (y and dy held): 2 workgroups per CU
constexpr int64_t kSmMinBlocks = 2048;  // narrow the column lanes until the grid is this big
constexpr float kLog2eSm = 1.4426950408889634f;

// VEC columns per thread: 1 (scalar) or one 16-byte vector.
template <typename T, int VEC>
struct Vec {
  static_assert(VEC == 1 || VEC * sizeof(T) == 16, "scalar or 16-byte vectors");
  static __device__ __forceinline__ void load(const T* p, float* f) {
    if constexpr (VEC == 1) {
      f[0] = to_f32(*p);
    } else {
      const uint4 v = ld16(p);
#pragma unroll
      for (int e = 0; e < VEC; ++e) f[e] = elem<T>(v, e);
    }
  }
  static __device__ __forceinline__ void store(T* p, const float* f) {
    if constexpr (VEC == 1) {
      *p = from_f32<T>(f[0]);
    } else {
      st16_nt(p, pack16<T>(f));
    }
  }
};

// One row's VEC columns kept in registers as loaded (16 bytes, or one value).
template <typename T, int VEC>
struct Held {
  typename std::conditional<VEC == 1, float, uint4>::type v;
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (VEC == 1)
      v = to_f32(*p);
    else
      v = ld16(p);
  }
  __device__ __forceinline__ void get(float* f) const {
    if constexpr (VEC == 1) {
      f[0] = v;
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) f[e] = elem<T>(v, e);
    }
  }
};

// Online (max, sum) update with one exp per element: scale whichever of
// (sum, new term) is behind.  Non-finite input gives what the two-pass
// formula gives (and torch.softmax): a NaN, or a second +inf, makes the sum
// NaN; so does a first +inf, whose own term exp(inf - inf) is NaN.  fmaxf
// ignores a NaN operand, so the NaN is carried in the sum, not the max.
__device__ __forceinline__ void sm_update(float& m, float& l, float v) {
  const float hi = fmaxf(m, v);
  float t = hi == -__builtin_inff()
                ? 0.f  // -inf so far: nothing to add (avoids -inf - -inf)
                : __builtin_amdgcn_exp2f((fminf(m, v) - hi) * kLog2eSm);
  if (v != v) t = v;  // NaN input: poison the sum
  const float self = v == __builtin_inff() ? __builtin_nanf("") : 1.0f;  // exp(v - v)
  l = v > m ? fmaf(l, t, self) : l + t;
  m = hi;
}

// v_max3_f32 written out (fmaxf adds a canonicalising instruction per
// operand it cannot prove quiet, i.e. every loaded value).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Merge the partial (max, sum) of another row lane into (m, l).  A lane that
// has seen only -inf and NaN keeps m = -inf with a NaN sum: l * 0 carries it
// (0 * 0 = 0 otherwise), and two +inf maxima give exp(inf - inf) = NaN.
__device__ __forceinline__ void sm_merge(float& m, float& l, float m2, float l2) {
  const float hi = fmaxf(m, m2);
  const float a = m == -__builtin_inff() ? l * 0.f : l * __builtin_amdgcn_exp2f((m - hi) * kLog2eSm);
  const float b = m2 == -__builtin_inff() ? l2 * 0.f : l2 * __builtin_amdgcn_exp2f((m2 - hi) * kLog2eSm);
  l = a + b;
  m = hi;
}

// Workgroup -> (sequence, column chunk) index.  Block b runs on XCD b mod 8.
// When a chunk is narrower than a 128-byte line, the line's two halves
// (chunks 2k and 2k + 1) go to blocks b and b + 8 of each group of 16, which
// share an XCD, so its L2 fetches the line once instead of two L2s fetching
// it; blocks past the last full group of 16 keep their index.  Consecutive
// pairs still cycle over the XCDs, so every XCD gets a fair share of every
// sequence.
__device__ __forceinline__ int sm_block(bool half_lines) {
  const int b = blockIdx.x;
  if (!half_lines || b >= (int)(gridDim.x & ~15u)) return b;
  return (b & ~15) | ((b & 7) << 1) | ((b >> 3) & 1);
}

template <typename T, int VEC>
__global__ __launch_bounds__(kSmThreadsFwd) void varlen_softmax_kernel(
    const T* __restrict__ x, T* __restrict__ y, const int32_t* __restrict__ cu, int64_t total,
    int64_t features, int ct, int chunks) {
  constexpr int kSmThreads = kSmThreadsFwd;
  __shared__ float s_m[kSmThreads * VEC];
  __shared__ float s_l[kSmThreads * VEC];
  const int bsel = sm_block(ct * VEC * (int)sizeof(T) < 128);
  const int seq = bsel / chunks, chunk = bsel - seq * chunks;
  // offsets are clamped to [0, total]: malformed input cannot index outside x
  const int64_t start = min<int64_t>(max<int64_t>(cu[seq], 0), total);
  const int64_t end = min<int64_t>(max<int64_t>(cu[seq + 1], start), total);
  const int rs = kSmThreads / ct;
  const int tc = threadIdx.x % ct, tr = threadIdx.x / ct;
  const int64_t col = ((int64_t)chunk * ct + tc) * VEC;
  const bool active = col < features;  // VEC > 1 only when features % VEC == 0
  // The first kSmCache * rs rows of the sequence are held in registers
  // (kSmCache per thread).  Rows past them ("excess", only in sequences
  // longer than that) are streamed first with an online (max, sum), which is
  // parked in this thread's own LDS merge slots while the held rows load, so
  // the two never occupy registers together; pass 2 re-reads them.
  const int64_t len = end - start;
  const int64_t held_rows = (int64_t)kSmCache * rs;
  const bool excess = len > held_rows;  // uniform per workgroup

  float m[VEC], l[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    m[e] = -__builtin_inff();
    l[e] = 0.f;
  }
  Held<T, VEC> held[kSmCache];
  // rows this thread holds (0 when the sequence is shorter than tr + 1)
  const int nr = (int)min<int64_t>(kSmCache, max<int64_t>(0, (len - tr + rs - 1) / rs));
  if (active) {
    if (excess) {
      for (int64_t r = start + held_rows + tr; r < end; r += kUnroll * rs) {
        Held<T, VEC> v[kUnroll];  // kUnroll rows' loads in flight before any math, kept packed
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
          if (r + u * rs < end) v[u].load(x + (r + u * rs) * features + col);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          if (r + u * rs >= end) continue;
          float f[VEC];
          v[u].get(f);
#pragma unroll
          for (int e = 0; e < VEC; ++e) sm_update(m[e], l[e], f[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        s_m[threadIdx.x * VEC + e] = m[e];
        s_l[threadIdx.x * VEC + e] = l[e];
        m[e] = -__builtin_inff();
        l[e] = 0.f;
      }
    }
    // the held rows: every load in flight before any math; rows past the
    // end stay unread
#pragma unroll
    for (int i = 0; i < kSmCache; ++i)
      if (i < nr) held[i].load(x + (start + tr + (int64_t)i * rs) * features + col);
    // With the rows at hand, the thread's max first and then the sum of
    // exponentials against it (fewer instructions than the online update).
#pragma unroll
    for (int i = 0; i < kSmCache; i += 2) {
      if (i >= nr) continue;
      float a[VEC], b[VEC];
      held[i].get(a);
      if (i + 1 < nr)
        held[i + 1].get(b);
      else
#pragma unroll
        for (int e = 0; e < VEC; ++e) b[e] = a[e];
#pragma unroll
      for (int e = 0; e < VEC; ++e) m[e] = max3f(m[e], a[e], b[e]);
    }
    // The sum against mr = m, or 0 where m = -inf (every held value -inf or
    // NaN, as v_max3 skips NaN): -inf then adds exp2(-inf) = 0 and a NaN adds
    // NaN, as in the two-pass formula, where a guard on m = -inf would drop
    // the NaN.
    float mr[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) mr[e] = m[e] == -__builtin_inff() ? 0.f : m[e];
#pragma unroll
    for (int i = 0; i < kSmCache; ++i) {
      if (i >= nr) continue;
      float v[VEC];
      held[i].get(v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) l[e] += __builtin_amdgcn_exp2f((v[e] - mr[e]) * kLog2eSm);
    }
    if (excess) {  // fold in the streamed rows' (max, sum)
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        sm_merge(m[e], l[e], s_m[threadIdx.x * VEC + e], s_l[threadIdx.x * VEC + e]);
    }
  }
  // merge the row lanes of each column: a tree over the (power-of-two) row
  // lanes in LDS, log2(rs) steps in a fixed order (deterministic)
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    s_m[threadIdx.x * VEC + e] = m[e];
    s_l[threadIdx.x * VEC + e] = l[e];
  }
  for (int h = rs >> 1; h >= 1; h >>= 1) {
    __syncthreads();
    if (tr < h) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int o = ((tr + h) * ct + tc) * VEC + e;
        sm_merge(m[e], l[e], s_m[o], s_l[o]);
        s_m[threadIdx.x * VEC + e] = m[e];
        s_l[threadIdx.x * VEC + e] = l[e];
      }
    }
  }
  __syncthreads();
  if (tr == 0) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      s_m[tc * VEC + e] = m[e];
      s_l[tc * VEC + e] = 1.0f / l[e];
    }
  }
  __syncthreads();
  if (!active) return;
  float mm[VEC], inv[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    mm[e] = s_m[tc * VEC + e];
    inv[e] = s_l[tc * VEC + e];
  }
#pragma unroll
  for (int i = 0; i < kSmCache; ++i) {
    if (i >= nr) continue;  // (not break: a fixed trip count keeps the array in registers)
    float v[VEC];
    held[i].get(v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = __builtin_amdgcn_exp2f((v[e] - mm[e]) * kLog2eSm) * inv[e];
    Vec<T, VEC>::store(y + (start + tr + (int64_t)i * rs) * features + col, v);
  }
  for (int64_t r = start + held_rows + tr; r < end; r += kUnroll * rs) {
    Held<T, VEC> v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (r + u * rs < end) v[u].load(x + (r + u * rs) * features + col);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (r + u * rs >= end) continue;
      float f[VEC];
      v[u].get(f);
#pragma unroll
      for (int e = 0; e < VEC; ++e) f[e] = __builtin_amdgcn_exp2f((f[e] - mm[e]) * kLog2eSm) * inv[e];
      Vec<T, VEC>::store(y + (r + u * rs) * features + col, f);
    }
  }
}

// Backward: dx = y * (dy - s) with s = sum over the sequence's rows of y * dy,
// per column; same decomposition as the forward (y and dy held in registers
// when the sequence fits).
template <typename T, int VEC>
__global__ __launch_bounds__(kSmThreadsBwd) void varlen_softmax_bwd_kernel(
    const T* __restrict__ y, const T* __restrict__ dy, T* __restrict__ dx,
    const int32_t* __restrict__ cu, int64_t total, int64_t features, int ct, int chunks) {
  __shared__ float s_s[kSmThreadsBwd * VEC];
  const int bsel = sm_block(ct * VEC * (int)sizeof(T) < 128);
  const int seq = bsel / chunks, chunk = bsel - seq * chunks;
  const int64_t start = min<int64_t>(max<int64_t>(cu[seq], 0), total);
  const int64_t end = min<int64_t>(max<int64_t>(cu[seq + 1], start), total);
  const int rs = kSmThreadsBwd / ct;
  const int tc = threadIdx.x % ct, tr = threadIdx.x / ct;
  const int64_t col = ((int64_t)chunk * ct + tc) * VEC;
  const bool active = col < features;
  const bool cached = end - start <= (int64_t)kSmCacheBwd * rs;  // uniform per workgroup

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  Held<T, VEC> hy[kSmCacheBwd], hd[kSmCacheBwd];
  if (active) {
    if (cached) {
#pragma unroll
      for (int i = 0; i < kSmCacheBwd; ++i) {
        const int64_t r = start + tr + (int64_t)i * rs;
        if (r < end) {
          hy[i].load(y + r * features + col);
          hd[i].load(dy + r * features + col);
        }
      }
#pragma unroll
      for (int i = 0; i < kSmCacheBwd; ++i) {
        const int64_t r = start + tr + (int64_t)i * rs;
        if (r >= end) continue;
        float a[VEC], b[VEC];
        hy[i].get(a);
        hd[i].get(b);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = fmaf(a[e], b[e], acc[e]);
      }
    } else {
      for (int64_t r = start + tr; r < end; r += kUnroll * rs) {
        float a[kUnroll][VEC], b[kUnroll][VEC];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          if (r + u * rs < end) {
            Vec<T, VEC>::load(y + (r + u * rs) * features + col, a[u]);
            Vec<T, VEC>::load(dy + (r + u * rs) * features + col, b[u]);
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) a[u][e] = b[u][e] = 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] = fmaf(a[u][e], b[u][e], acc[e]);
      }
    }
  }
  // sum the row lanes of each column: tree over the row lanes (fixed order)
#pragma unroll
  for (int e = 0; e < VEC; ++e) s_s[threadIdx.x * VEC + e] = acc[e];
  for (int h = rs >> 1; h >= 1; h >>= 1) {
    __syncthreads();
    if (tr < h) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        acc[e] += s_s[((tr + h) * ct + tc) * VEC + e];
        s_s[threadIdx.x * VEC + e] = acc[e];
      }
    }
  }
  __syncthreads();
  if (tr == 0) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) s_s[tc * VEC + e] = acc[e];
  }
  __syncthreads();
  if (!active) return;
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = s_s[tc * VEC + e];
  if (cached) {
#pragma unroll
    for (int i = 0; i < kSmCacheBwd; ++i) {
      const int64_t r = start + tr + (int64_t)i * rs;
      if (r >= end) continue;
      float a[VEC], b[VEC];
      hy[i].get(a);
      hd[i].get(b);
#pragma unroll
      for (int e = 0; e < VEC; ++e) a[e] = a[e] * (b[e] - acc[e]);
      Vec<T, VEC>::store(dx + r * features + col, a);
    }
    return;
  }
  for (int64_t r = start + tr; r < end; r += kUnroll * rs) {
    float a[kUnroll][VEC], b[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (r + u * rs < end) {
        Vec<T, VEC>::load(y + (r + u * rs) * features + col, a[u]);
        Vec<T, VEC>::load(dy + (r + u * rs) * features + col, b[u]);
      }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (r + u * rs >= end) break;
#pragma unroll
      for (int e = 0; e < VEC; ++e) a[u][e] = a[u][e] * (b[u][e] - acc[e]);
      Vec<T, VEC>::store(dx + (r + u * rs) * features + col, a[u]);
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch shape shared by forward and backward: column lanes (a power of two,
// at most 64) and column chunks per sequence.
struct SmShape {
  bool vec;
  int ct;
  int64_t chunks;
};
template <typename T>
SmShape sm_shape(int64_t features, bool aligned, int batch, int64_t total, int threads,
                 int cache_rows, int min_ct) {
  constexpr int V = 16 / sizeof(T);
  SmShape sh;
  sh.vec = features % V == 0 && aligned;
  const int64_t units = sh.vec ? features / V : features;  // column vectors per row
  sh.ct = 1;
  while (sh.ct < units && sh.ct < 64) sh.ct <<= 1;
  // Fewer column lanes -> more chunks, more workgroups, and more row lanes,
  // i.e. longer sequences held in registers: narrow until the grid is large
  // and cache_rows rows per row lane cover twice the mean sequence length, to
  // min_ct lanes at least.  The forward goes down to 4 (64-byte row
  // segments, half-line chunks paired on one XCD by sm_block); the backward
  // keeps >= 8 x 16 bytes contiguous.
  const int64_t cover = 2 * ((total + batch - 1) / batch);
  while (sh.ct > min_ct && ((int64_t)batch * ((units + sh.ct - 1) / sh.ct) < kSmMinBlocks ||
                       (int64_t)cache_rows * (threads / sh.ct) < cover))
    sh.ct >>= 1;
  sh.chunks = (units + sh.ct - 1) / sh.ct;
  return sh;
}

template <typename T>
int launch_softmax_bwd(const void* y, const void* dy, void* dx, const int32_t* cu, int batch,
                       int64_t total, int64_t features, hipStream_t stream) {
  constexpr int V = 16 / sizeof(T);
  const SmShape sh =
      sm_shape<T>(features, aligned16(y) && aligned16(dy) && aligned16(dx), batch, total,
                  kSmThreadsBwd, kSmCacheBwd, 8);
  if ((int64_t)batch * sh.chunks > 0x7fffffff)
    return set_error(SCREE_ERR_INVALID, "scree_varlen_softmax_bwd: grid too large");
  const dim3 grid((unsigned)(batch * sh.chunks));
  if (sh.vec)
    hipLaunchKernelGGL((varlen_softmax_bwd_kernel<T, V>), grid, dim3(kSmThreadsBwd), 0, stream,
                       static_cast<const T*>(y), static_cast<const T*>(dy), static_cast<T*>(dx),
                       cu, total, features, sh.ct, (int)sh.chunks);
  else
    hipLaunchKernelGGL((varlen_softmax_bwd_kernel<T, 1>), grid, dim3(kSmThreadsBwd), 0, stream,
                       static_cast<const T*>(y), static_cast<const T*>(dy), static_cast<T*>(dx),
                       cu, total, features, sh.ct, (int)sh.chunks);
  return check_launch("scree_varlen_softmax_bwd");
}

template <typename T>
int launch_softmax(const void* x, void* y, const int32_t* cu, int batch, int64_t total,
                   int64_t features, hipStream_t stream) {
  constexpr int V = 16 / sizeof(T);
  const SmShape sh = sm_shape<T>(features, aligned16(x) && aligned16(y), batch, total,
                                 kSmThreadsFwd, kSmCache, kSmMinCtFwd);
  if ((int64_t)batch * sh.chunks > 0x7fffffff)
    return set_error(SCREE_ERR_INVALID, "scree_varlen_softmax: grid too large");
  const dim3 grid((unsigned)(batch * sh.chunks));
  if (sh.vec)
    hipLaunchKernelGGL((varlen_softmax_kernel<T, V>), grid, dim3(kSmThreadsFwd), 0, stream,
                       static_cast<const T*>(x), static_cast<T*>(y), cu, total, features, sh.ct,
                       (int)sh.chunks);
  else
    hipLaunchKernelGGL((varlen_softmax_kernel<T, 1>), grid, dim3(kSmThreadsFwd), 0, stream,
                       static_cast<const T*>(x), static_cast<T*>(y), cu, total, features, sh.ct,
                       (int)sh.chunks);
  return check_launch("scree_varlen_softmax");
}

}  // namespace
}  // namespace scree

using namespace scree;

extern "C" int scree_varlen_softmax(const void* x, void* y, const int32_t* cu_seqlens, int batch,
                                    int64_t total_tokens, int64_t features, int dtype,
                                    void* stream) {
  if (!x || !y || !cu_seqlens)
    return set_error(SCREE_ERR_INVALID, "scree_varlen_softmax: null pointer");
  if (batch < 1 || total_tokens < 0 || features < 1)
    return set_error(SCREE_ERR_INVALID,
                     "scree_varlen_softmax: need batch >= 1, total_tokens >= 0, features >= 1");
  if (total_tokens == 0) return SCREE_OK;
  if (total_tokens > ((int64_t)1 << 40) / features)
    return set_error(SCREE_ERR_INVALID, "scree_varlen_softmax: tensor too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_softmax<float>(x, y, cu_seqlens, batch, total_tokens, features, s);
    case SCREE_DTYPE_F16: return launch_softmax<f16>(x, y, cu_seqlens, batch, total_tokens, features, s);
    case SCREE_DTYPE_BF16: return launch_softmax<bf16>(x, y, cu_seqlens, batch, total_tokens, features, s);
    default: return set_error(SCREE_ERR_UNSUPPORTED, "scree_varlen_softmax: dtype %d", dtype);
  }
}

extern "C" int scree_varlen_softmax_bwd(const void* y, const void* dy, void* dx,
                                        const int32_t* cu_seqlens, int batch,
                                        int64_t total_tokens, int64_t features, int dtype,
                                        void* stream) {
  if (!y || !dy || !dx || !cu_seqlens)
    return set_error(SCREE_ERR_INVALID, "scree_varlen_softmax_bwd: null pointer");
  if (batch < 1 || total_tokens < 0 || features < 1)
    return set_error(SCREE_ERR_INVALID,
                     "scree_varlen_softmax_bwd: need batch >= 1, total_tokens >= 0, features >= 1");
  if (total_tokens == 0) return SCREE_OK;
  if (total_tokens > ((int64_t)1 << 40) / features)
    return set_error(SCREE_ERR_INVALID, "scree_varlen_softmax_bwd: tensor too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32:
      return launch_softmax_bwd<float>(y, dy, dx, cu_seqlens, batch, total_tokens, features, s);
    case SCREE_DTYPE_F16:
      return launch_softmax_bwd<f16>(y, dy, dx, cu_seqlens, batch, total_tokens, features, s);
    case SCREE_DTYPE_BF16:
      return launch_softmax_bwd<bf16>(y, dy, dx, cu_seqlens, batch, total_tokens, features, s);
    default: return set_error(SCREE_ERR_UNSUPPORTED, "scree_varlen_softmax_bwd: dtype %d", dtype);
  }
}
