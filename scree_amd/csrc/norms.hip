// Varlen RMSNorm / LayerNorm, forward and backward, for gfx950.
//
// Norms act per token row, so the packed (rows, dim) buffer is processed
// with no reference to the offsets (the reference's kernels ignore them too,
// src/scree/kernels/triton/varlen_rmsnorm.py:7-8).
//
// Fast path: one wavefront per row.  Each lane keeps CHUNKS 16-byte vectors
// of the row in registers (dim = CHUNKS * 64 lanes * 16 bytes at most), so x
// is read from HBM exactly once; the reductions are wave-wide shuffles.
// Generic path (dim not a multiple of one 16-byte vector, unaligned buffers,
// or rows longer than the fast path holds): one wavefront per row looping
// over the columns.
//
// Backward (norm_bwd_cols): each thread of a block owns fixed 16-byte column
// vectors across the block's rows, so the parameter gradients accumulate in
// its fp32 registers; the row statistics are reduced across the block through
// LDS, dx is written per row, and each block writes one partial row of
// parameter gradients, which a column-sum kernel adds in a fixed order.  No
// atomics: results are bit-identical from run to run.
#include <initializer_list>

#include "common.h"

namespace scree {
namespace {

constexpr int kWave = 64;
constexpr int kFwdWaves = 4;       // rows (waves) per forward block
constexpr int kMaxParts = 512;     // partial rows of a backward, at most
constexpr int kMaxChunks = 16;     // 16-byte vectors per lane on the fast path

// ------------------------------------------------------------------ forward
// RES (RMSNorm only): the normalised row is h = x + res, rounded to T as a
// separate addition would round it; h is written out and normalised.
template <int WAVES>
constexpr int fwd_threads() { return WAVES * kWave; }
// LayerNorm's workgroups are kLnWaves rows (waves) that stage the weight and
// bias rows in LDS once; RMSNorm's are kFwdWaves rows with the weights in
// registers.
constexpr int kLnWaves = 8;
template <bool LAYER>
constexpr int fwd_waves() { return LAYER ? kLnWaves : kFwdWaves; }

template <typename T, int CHUNKS, bool LAYER, bool RES>
__global__ __launch_bounds__(fwd_threads<fwd_waves<LAYER>()>()) void norm_fwd_vec(
    const T* __restrict__ x, const T* __restrict__ res, const T* __restrict__ w,
    const T* __restrict__ b, T* __restrict__ hout, T* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t rows, int dim, float eps) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int WAVES = fwd_waves<LAYER>();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * WAVES + (threadIdx.x / kWave);
  const bool live = row < rows;
  const int nvec = dim / VEC;
  const T* xr = x + row * (int64_t)dim;
  uint4 v[CHUNKS];
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int vi = c * kWave + lane;
    v[c] = live && vi < nvec ? ld16_nt(xr + (int64_t)vi * VEC) : make_uint4(0, 0, 0, 0);
  }
  // LayerNorm: the block copies the weight and bias rows into LDS while its
  // rows load (one L2 read per block instead of per row, and off the
  // registers); the output reads them from there.
  constexpr int NMAX = LAYER ? CHUNKS * kWave * VEC : 1;
  __shared__ __align__(16) T wb[2 * NMAX];
  if constexpr (LAYER) {
    for (int vi = threadIdx.x; vi < nvec; vi += WAVES * kWave) {
      *reinterpret_cast<uint4*>(wb + vi * VEC) = w ? ld16(w + (int64_t)vi * VEC) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(wb + NMAX + vi * VEC) = b ? ld16(b + (int64_t)vi * VEC) : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
  }
  if (!live) return;
  // RMSNorm loads its weight vectors with the row, so their (L2) latency
  // overlaps the row's instead of following the reduction.
  constexpr bool kEarlyW = !LAYER;
  uint4 wvs[kEarlyW ? CHUNKS : 1];
  if constexpr (kEarlyW) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int vi = c * kWave + lane;
      wvs[c] = (w && vi < nvec) ? ld16(w + (int64_t)vi * VEC) : make_uint4(0, 0, 0, 0);
    }
  }
  if (RES) {
    const T* rr = res + row * (int64_t)dim;
    T* hr = hout + row * (int64_t)dim;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int vi = c * kWave + lane;
      if (vi < nvec) {
        const uint4 rv = ld16_nt(rr + (int64_t)vi * VEC);
        float f[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) f[e] = elem<T>(v[c], e) + elem<T>(rv, e);
        v[c] = pack16<T>(f);
        st16_nt(hr + (int64_t)vi * VEC, v[c]);
      }
    }
  }
  const float fdim = (float)dim;
  float mu = 0.f, rstd;
  if (LAYER) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += elem<T>(v[c], e);
    mu = wave_sum(s) / fdim;
    float s2 = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      if (c * kWave + lane < nvec) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float d = elem<T>(v[c], e) - mu;
          s2 = __builtin_fmaf(d, d, s2);
        }
      }
    }
    rstd = 1.0f / sqrtf(wave_sum(s2) / fdim + eps);
  } else {
    // Explicit fused multiply-adds fix the rounding of every step, so the
    // add + RMSNorm and the plain RMSNorm instantiations (where the compiler
    // could contract a*a + b*b either way) give identical statistics.
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float t = elem<T>(v[c], e);
        s = __builtin_fmaf(t, t, s);
      }
    rstd = 1.0f / sqrtf(wave_sum(s) / fdim + eps);
  }
  T* yr = y + row * (int64_t)dim;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int vi = c * kWave + lane;
    if (vi < nvec) {
      uint4 wv = make_uint4(0, 0, 0, 0), bv = make_uint4(0, 0, 0, 0);
      if constexpr (kEarlyW) {
        wv = wvs[c];
      } else {
        wv = *reinterpret_cast<const uint4*>(wb + vi * VEC);
        bv = *reinterpret_cast<const uint4*>(wb + NMAX + vi * VEC);
      }
      float f[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float t = LAYER ? (elem<T>(v[c], e) - mu) * rstd : elem<T>(v[c], e) * rstd;
        if (w) t *= elem<T>(wv, e);
        if (LAYER && b) t += elem<T>(bv, e);
        f[e] = t;
      }
      st16_nt(yr + (int64_t)vi * VEC, pack16<T>(f));
    }
  }
  if (lane == 0) {
    if (rstd_out) rstd_out[row] = rstd;
    if (LAYER && mean_out) mean_out[row] = mu;
  }
}

template <typename T, bool LAYER, bool RES>
__global__ __launch_bounds__(kFwdWaves* kWave) void norm_fwd_generic(
    const T* __restrict__ x, const T* __restrict__ res, const T* __restrict__ w,
    const T* __restrict__ b, T* __restrict__ hout, T* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t rows, int dim, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kFwdWaves + (threadIdx.x / kWave);
  if (row >= rows) return;
  const T* xr = x + row * (int64_t)dim;
  const T* rr = RES ? res + row * (int64_t)dim : nullptr;
  // Element j of the normalised row: x, or h = x + res rounded to T (each
  // pass recomputes it rather than reading back the h it stores).
  auto at = [&](int j) -> float {
    return RES ? to_f32(from_f32<T>(to_f32(xr[j]) + to_f32(rr[j]))) : to_f32(xr[j]);
  };
  const float fdim = (float)dim;
  float mu = 0.f, rstd;
  if (LAYER) {
    float s = 0.f;
    for (int j = lane; j < dim; j += kWave) s += at(j);
    mu = wave_sum(s) / fdim;
    float s2 = 0.f;
    for (int j = lane; j < dim; j += kWave) {
      const float d = at(j) - mu;
      s2 = __builtin_fmaf(d, d, s2);
    }
    rstd = 1.0f / sqrtf(wave_sum(s2) / fdim + eps);
  } else {
    float s = 0.f;
    for (int j = lane; j < dim; j += kWave) {
      const float t = at(j);
      s = __builtin_fmaf(t, t, s);
    }
    rstd = 1.0f / sqrtf(wave_sum(s) / fdim + eps);
  }
  T* yr = y + row * (int64_t)dim;
  T* hr = RES ? hout + row * (int64_t)dim : nullptr;
  for (int j = lane; j < dim; j += kWave) {
    const float hj = at(j);
    if (RES) hr[j] = from_f32<T>(hj);
    float t = LAYER ? (hj - mu) * rstd : hj * rstd;
    if (w) t *= to_f32(w[j]);
    if (LAYER && b) t += to_f32(b[j]);
    yr[j] = from_f32<T>(t);
  }
  if (lane == 0) {
    if (rstd_out) rstd_out[row] = rstd;
    if (LAYER && mean_out) mean_out[row] = mu;
  }
}

// ----------------------------------------------------------------- backward
// Column-ownership layout.  A block of kBwdThreads threads takes every
// G-th step of R rows (G = grid size: block b takes rows b*R .. b*R+R-1,
// then those G*R rows further on, ...), so at any moment the grid works on
// one contiguous stretch of G*R rows and its reads and writes spread over
// all HBM channels; a contiguous range of rows per block put the blocks'
// concurrent streams ~40 rows apart at config 2 and ran ~10 % slower.  Thread
// t owns the 16-byte column vectors t + k*kBwdThreads (k < CPT) of every row
// the block takes.  Per step of R rows the thread loads its
// vectors of x and dy, the row statistics (sum x*g for RMS; sum g and
// sum g*xhat for LN) are reduced across the wave by shuffles and across the
// block through a double-buffered LDS array (one barrier per step), then the
// thread writes dx for its vectors and adds its parameter gradients into
// fp32 registers.  At the end each thread writes its own columns of the
// block's partial row: no intra-block reduction, and the partial rows are
// summed by norm_param_colsum in a fixed order.
// partial layout: [part][param][dim] fp32, param 0 = dweight, 1 = dbias.
constexpr int kBwdThreads = 512;
constexpr int kBwdWarps = kBwdThreads / kWave;

// One step's rows: this thread's 16-byte vectors of x, dy (and dres) for R
// rows, with the rows' statistics.  The kernel keeps two of these and loads
// the next step's rows while it reduces and writes the current one.
template <typename T, int CPT, int R, bool LAYER, bool RES>
struct BwdRows {
  uint4 xv[R][CPT], gv[R][CPT], hv[RES ? R : 1][CPT];
  float rs[R], mu[R];

  __device__ __forceinline__ void load(const T* __restrict__ x, const T* __restrict__ dy,
                                       const T* __restrict__ dres,
                                       const float* __restrict__ mean_in,
                                       const float* __restrict__ rstd_in, const bool* own,
                                       int64_t rb, int64_t r1, int dim, int tid) {
    constexpr int VEC = 16 / sizeof(T);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = rb + r;
      const bool ok = row < r1;
      rs[r] = ok ? rstd_in[row] : 0.f;
      mu[r] = (LAYER && ok) ? mean_in[row] : 0.f;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int64_t off = row * (int64_t)dim + (int64_t)(tid + k * kBwdThreads) * VEC;
        xv[r][k] = (ok && own[k]) ? ld16_nt(x + off) : make_uint4(0, 0, 0, 0);
        gv[r][k] = (ok && own[k]) ? ld16_nt(dy + off) : make_uint4(0, 0, 0, 0);
        if (RES) hv[r][k] = (ok && own[k]) ? ld16_nt(dres + off) : make_uint4(0, 0, 0, 0);
      }
    }
  }
};

// The rows of one step: row sums reduced across the wave by shuffles and
// across the block through red[buf] (one barrier), then dx written and the
// parameter gradients accumulated in aw / ab.  `wf` holds this thread's
// weights as fp32 (ones without a weight).  Per row, x-hat = x * rstd - mean
// * rstd is one FMA and the output folds its row constants into two more:
//   LayerNorm  dx = rstd * g - rstd*b * x-hat - rstd*a,  a = mean(g), b = mean(g * x-hat)
//   RMSNorm    dx = rstd * g - k * x,                    k = rstd^3 * mean(g * x)
// with g = dy * w (reference varlen_layernorm.py:64-74, varlen_rmsnorm.py:58-65).
template <typename T, int CPT, int R, bool LAYER, bool RES>
__device__ __forceinline__ void norm_bwd_step(BwdRows<T, CPT, R, LAYER, RES>& st,
                                              float (&red)[2][R][2][kBwdWarps], int buf,
                                              const float (&wf)[CPT][16 / sizeof(T)],
                                              const bool* own,
                                              float (&aw)[CPT][16 / sizeof(T)],
                                              float (&ab)[LAYER ? CPT : 1][16 / sizeof(T)],
                                              T* __restrict__ dx, int64_t rb, int64_t r1, int dim,
                                              float inv_dim, int tid) {
  constexpr int VEC = 16 / sizeof(T);
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  float s1[R], s2[R], nmr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    s1[r] = 0.f;
    s2[r] = 0.f;
    nmr[r] = -st.mu[r] * st.rs[r];
#pragma unroll
    for (int k = 0; k < CPT; ++k)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xx = elem<T>(st.xv[r][k], e);
        const float g = elem<T>(st.gv[r][k], e) * wf[k][e];
        if (LAYER) {
          s1[r] += g;
          s2[r] = fmaf(g, fmaf(xx, st.rs[r], nmr[r]), s2[r]);
        } else {
          s1[r] = fmaf(xx, g, s1[r]);
        }
      }
    s1[r] = wave_sum_last(s1[r]);
    if (LAYER) s2[r] = wave_sum_last(s2[r]);
  }
  if (lane == kWave - 1) {  // the wave's sums are complete in its last lane
#pragma unroll
    for (int r = 0; r < R; ++r) {
      red[buf][r][0][wave] = s1[r];
      red[buf][r][1][wave] = s2[r];
    }
  }
  __syncthreads();
  // Keep the rows packed across the barrier: re-derive the fp32 values
  // below instead of holding the converted floats live.
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      asm volatile("" : "+v"(st.xv[r][k].x), "+v"(st.xv[r][k].y), "+v"(st.xv[r][k].z), "+v"(st.xv[r][k].w));
      asm volatile("" : "+v"(st.gv[r][k].x), "+v"(st.gv[r][k].y), "+v"(st.gv[r][k].z), "+v"(st.gv[r][k].w));
      if (RES)
        asm volatile("" : "+v"(st.hv[RES ? r : 0][k].x), "+v"(st.hv[RES ? r : 0][k].y),
                     "+v"(st.hv[RES ? r : 0][k].z), "+v"(st.hv[RES ? r : 0][k].w));
    }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float t1 = 0.f, t2 = 0.f;
#pragma unroll
    for (int q = 0; q < kBwdWarps; ++q) {
      t1 += red[buf][r][0][q];
      if (LAYER) t2 += red[buf][r][1][q];
    }
    const int64_t row = rb + r;
    if (row >= r1) continue;
    const float rr = st.rs[r];
    // LayerNorm: c1 = -rstd * mean(g), c2 = -rstd * mean(g * x-hat);
    // RMSNorm: c2 = -rstd^3 * mean(g * x).
    const float c1 = -rr * (t1 * inv_dim);
    const float c2 = LAYER ? -rr * (t2 * inv_dim) : -(rr * rr * rr) * (t1 * inv_dim);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      if (!own[k]) continue;
      float f[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xx = elem<T>(st.xv[r][k], e);
        const float d = elem<T>(st.gv[r][k], e);
        const float g = d * wf[k][e];
        if (LAYER) {
          const float xh = fmaf(xx, rr, nmr[r]);
          f[e] = fmaf(rr, g, fmaf(c2, xh, c1));
          aw[k][e] = fmaf(d, xh, aw[k][e]);
          ab[LAYER ? k : 0][e] += d;
        } else {
          f[e] = fmaf(rr, g, c2 * xx);
          aw[k][e] = fmaf(d * rr, xx, aw[k][e]);
        }
        if (RES) f[e] += elem<T>(st.hv[RES ? r : 0][k], e);
      }
      st16_nt(dx + row * (int64_t)dim + (int64_t)(tid + k * kBwdThreads) * VEC, pack16<T>(f));
    }
  }
}

// RES: dx also receives dres (the gradient reaching the normalised input by
// another path, e.g. the residual stream of an add + RMSNorm).
template <typename T, int CPT, int R, bool LAYER, bool RES>
__global__ __launch_bounds__(kBwdThreads) void norm_bwd_cols(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
    const T* __restrict__ dres, T* __restrict__ dx, float* __restrict__ partial, int64_t rows,
    int dim, int nparam) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float red[2][R][2][kBwdWarps];
  const int tid = threadIdx.x;
  const int nvec = dim / VEC;

  float wf[CPT][VEC];  // this thread's weights as fp32, ones without a weight
  bool own[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int v = tid + k * kBwdThreads;
    own[k] = v < nvec;
    const uint4 wv = (w && own[k]) ? ld16(w + (int64_t)v * VEC) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) wf[k][e] = w ? elem<T>(wv, e) : 1.0f;
  }
  float aw[CPT][VEC], ab[LAYER ? CPT : 1][VEC];
#pragma unroll
  for (int k = 0; k < CPT; ++k)
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      aw[k][e] = 0.f;
      ab[LAYER ? k : 0][e] = 0.f;
    }

  // Two row sets: while one step reduces and writes, the next step's rows
  // load.  Steps are S rows apart; rows past the end load as zeros and are
  // not written.
  BwdRows<T, CPT, R, LAYER, RES> A, B;
  const float inv_dim = 1.0f / (float)dim;
  const int64_t S = (int64_t)gridDim.x * R;
  const int64_t first = (int64_t)blockIdx.x * R;
  if (first < rows) A.load(x, dy, dres, mean_in, rstd_in, own, first, rows, dim, tid);
  for (int64_t rb = first; rb < rows; rb += 2 * S) {
    if (rb + S < rows) B.load(x, dy, dres, mean_in, rstd_in, own, rb + S, rows, dim, tid);
    norm_bwd_step<T, CPT, R, LAYER, RES>(A, red, 0, wf, own, aw, ab, dx, rb, rows, dim, inv_dim, tid);
    if (rb + S >= rows) break;
    if (rb + 2 * S < rows) A.load(x, dy, dres, mean_in, rstd_in, own, rb + 2 * S, rows, dim, tid);
    norm_bwd_step<T, CPT, R, LAYER, RES>(B, red, 1, wf, own, aw, ab, dx, rb + S, rows, dim, inv_dim, tid);
  }
  for (int p = 0; p < nparam; ++p) {
    float* out = partial + ((int64_t)blockIdx.x * nparam + p) * dim;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      if (!own[k]) continue;
      float* o = out + (int64_t)(tid + k * kBwdThreads) * VEC;
#pragma unroll
      for (int e = 0; e < VEC; e += 4) {
        const float* src = p == 0 ? &aw[k][e] : &ab[LAYER ? k : 0][e];
        *reinterpret_cast<float4*>(o + e) = make_float4(src[0], src[1], src[2], src[3]);
      }
    }
  }
}

template <typename T, bool LAYER, bool RES>
__global__ __launch_bounds__(kFwdWaves* kWave) void norm_bwd_dx_generic(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
    const T* __restrict__ dres, T* __restrict__ dx, int64_t rows, int dim) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kFwdWaves + (threadIdx.x / kWave);
  if (row >= rows) return;
  const T* xr = x + row * (int64_t)dim;
  const T* gr = dy + row * (int64_t)dim;
  const float r = rstd_in[row];
  const float mu = LAYER ? mean_in[row] : 0.f;
  const float fdim = (float)dim;
  float s1 = 0.f, s2 = 0.f;
  for (int j = lane; j < dim; j += kWave) {
    const float xx = to_f32(xr[j]);
    const float d = to_f32(gr[j]);
    const float g = w ? d * to_f32(w[j]) : d;
    if (LAYER) {
      s1 += g;
      s2 += g * ((xx - mu) * r);
    } else {
      s1 += xx * g;
    }
  }
  s1 = wave_sum(s1);
  if (LAYER) s2 = wave_sum(s2);
  const float k_rms = r * r * r * s1 / fdim;
  const float a_ln = s1 / fdim;
  const float b_ln = s2 / fdim;
  T* dxr = dx + row * (int64_t)dim;
  for (int j = lane; j < dim; j += kWave) {
    const float xx = to_f32(xr[j]);
    const float d = to_f32(gr[j]);
    const float g = w ? d * to_f32(w[j]) : d;
    float v = LAYER ? r * (g - a_ln - ((xx - mu) * r) * b_ln) : r * g - k_rms * xx;
    if (RES) v += to_f32(dres[row * (int64_t)dim + j]);
    dxr[j] = from_f32<T>(v);
  }
}

// grid (ceil(dim/256), nparts): thread owns one column, sums rows part, part+nparts, ...
template <typename T, bool LAYER>
__global__ __launch_bounds__(256) void norm_bwd_param_generic(
    const T* __restrict__ dy, const T* __restrict__ x, const float* __restrict__ mean_in,
    const float* __restrict__ rstd_in, float* __restrict__ partial, int64_t rows, int dim,
    int nparam) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  const int part = blockIdx.y;
  const int nparts = gridDim.y;
  if (col >= dim) return;
  float aw = 0.f, ab = 0.f;
  for (int64_t row = part; row < rows; row += nparts) {
    const float xx = to_f32(x[row * (int64_t)dim + col]);
    const float d = to_f32(dy[row * (int64_t)dim + col]);
    const float r = rstd_in[row];
    if (LAYER) {
      aw += d * ((xx - mean_in[row]) * r);
      ab += d;
    } else {
      aw += d * xx * r;
    }
  }
  float* out = partial + (int64_t)part * nparam * dim;
  out[col] = aw;
  if (nparam > 1) out[dim + col] = ab;
}

// Column sums of the partial rows; output cast to out_dtype.  Scalar form
// (any dim): 64 columns x 4 row groups per block.
__device__ __forceinline__ void store_param(void* out, int col, float t, int out_dtype) {
  if (out_dtype == SCREE_DTYPE_F32) static_cast<float*>(out)[col] = t;
  else if (out_dtype == SCREE_DTYPE_F16) static_cast<f16*>(out)[col] = (f16)t;
  else static_cast<bf16*>(out)[col] = (bf16)t;
}

__global__ __launch_bounds__(256) void norm_param_colsum(const float* __restrict__ partial,
                                                         int nparts, int nparam, int dim,
                                                         void* out0, void* out1, int out_dtype) {
  __shared__ float red[4][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int grp = threadIdx.x / kWave;
  const int col = blockIdx.x * kWave + lane;
  const int p = blockIdx.y;
  float s = 0.f;
  if (col < dim) {
    for (int i = grp; i < nparts; i += 4) s += partial[((int64_t)i * nparam + p) * dim + col];
  }
  red[grp][lane] = s;
  __syncthreads();
  if (grp == 0 && col < dim) {
    const float t = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    void* out = p == 0 ? out0 : out1;
    if (out) store_param(out, col, t, out_dtype);
  }
}

// Vector form (dim % 4 == 0): 16 columns x 64 row groups per block, 16-byte
// loads, then a fixed-order tree over the row groups in LDS (deterministic).
__global__ __launch_bounds__(256) void norm_param_colsum4(const float* __restrict__ partial,
                                                          int nparts, int nparam, int dim,
                                                          void* out0, void* out1, int out_dtype) {
  __shared__ float4 red[64][4];
  const int cq = threadIdx.x & 3, rg = threadIdx.x >> 2;
  // A block reads a 64-byte strip of each partial row; block b runs on XCD
  // b mod 8, so neighbouring strips (one 128-byte line) go to blocks of the
  // same XCD, whose L2 then fetches the line once instead of once per XCD.
  int slab = blockIdx.x;
  if ((gridDim.x & 7) == 0) slab = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int col = slab * 16 + cq * 4;
  const int p = blockIdx.y;
  // Every load in flight at once (at most kMaxParts / 64 per thread), then
  // the sum in row order.
  constexpr int kIt = kMaxParts / 64;
  float4 v[kIt];
#pragma unroll
  for (int j = 0; j < kIt; ++j) {
    const int i = rg + 64 * j;
    v[j] = (col < dim && i < nparts)
               ? *reinterpret_cast<const float4*>(partial + ((int64_t)i * nparam + p) * dim + col)
               : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float4 s = v[0];
#pragma unroll
  for (int j = 1; j < kIt; ++j) {
    s.x += v[j].x; s.y += v[j].y; s.z += v[j].z; s.w += v[j].w;
  }
  red[rg][cq] = s;
  __syncthreads();
  for (int st = 32; st >= 1; st >>= 1) {
    if (rg < st) {
      const float4 o = red[rg + st][cq];
      float4 m = red[rg][cq];
      m.x += o.x; m.y += o.y; m.z += o.z; m.w += o.w;
      red[rg][cq] = m;
    }
    __syncthreads();
  }
  void* out = p == 0 ? out0 : out1;
  if (rg == 0 && col < dim && out) {
    const float4 t = red[0][cq];
    store_param(out, col + 0, t.x, out_dtype);
    store_param(out, col + 1, t.y, out_dtype);
    store_param(out, col + 2, t.z, out_dtype);
    store_param(out, col + 3, t.w, out_dtype);
  }
}

// --------------------------------------------------------------------- host
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int chunks_for(int nvec) {
  int need = (nvec + kWave - 1) / kWave;
  int c = 1;
  while (c < need) c <<= 1;
  return c;
}

inline int nparts_for(int64_t rows) {
  int64_t p = (rows + 7) / 8;
  if (p < 1) p = 1;
  if (p > kMaxParts) p = kMaxParts;
  return (int)p;
}

template <typename T>
bool fast_path_ok(int64_t dim, std::initializer_list<const void*> ptrs) {
  constexpr int VEC = 16 / sizeof(T);
  if (dim % VEC) return false;
  if (dim / VEC > (int64_t)kMaxChunks * kWave) return false;
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  return true;
}

// Backward fast path: whole 16-byte vectors, at most 2 per thread of a 512-thread block.
template <typename T>
bool bwd_fast_path_ok(int64_t dim, std::initializer_list<const void*> ptrs) {
  constexpr int VEC = 16 / sizeof(T);
  if (dim % VEC) return false;
  if (dim / VEC > 2 * (int64_t)kBwdThreads) return false;
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  return true;
}

// res / h non-null (RMSNorm only): normalise h = x + res and write h too.
template <typename T, bool LAYER, bool RES>
void launch_fwd_k(const T* xp, const T* rp, const T* wp, const T* bp, T* hp, T* yp, float* mean,
                  float* rstd, int64_t rows, int64_t dim, float eps, hipStream_t stream) {
  const dim3 grid((unsigned)((rows + kFwdWaves - 1) / kFwdWaves));
  const dim3 block(kFwdWaves * kWave);
  const int d = (int)dim;
  if (fast_path_ok<T>(dim, {xp, rp, wp, bp, hp, yp})) {
    constexpr int W = fwd_waves<LAYER>();
    const dim3 vgrid((unsigned)((rows + W - 1) / W)), vblock(W * kWave);
    const int chunks = chunks_for((int)(dim / (16 / sizeof(T))));
#define SCREE_FWD_CASE(C)                                                                      \
  case C:                                                                                      \
    hipLaunchKernelGGL((norm_fwd_vec<T, C, LAYER, RES>), vgrid, vblock, 0, stream, xp, rp, wp, bp, \
                       hp, yp, mean, rstd, rows, d, eps);                                      \
    break;
    switch (chunks) {
      SCREE_FWD_CASE(1)
      SCREE_FWD_CASE(2)
      SCREE_FWD_CASE(4)
      SCREE_FWD_CASE(8)
      SCREE_FWD_CASE(16)
      default: break;  // chunks_for never exceeds kMaxChunks on the fast path
    }
#undef SCREE_FWD_CASE
  } else {
    hipLaunchKernelGGL((norm_fwd_generic<T, LAYER, RES>), grid, block, 0, stream, xp, rp, wp, bp,
                       hp, yp, mean, rstd, rows, d, eps);
  }
}

template <typename T, bool LAYER>
int launch_fwd(const void* x, const void* res, const void* w, const void* b, void* h, void* y,
               float* mean, float* rstd, int64_t rows, int64_t dim, float eps,
               hipStream_t stream) {
  const T* xp = static_cast<const T*>(x);
  const T* rp = static_cast<const T*>(res);
  const T* wp = static_cast<const T*>(w);
  const T* bp = static_cast<const T*>(b);
  T* hp = static_cast<T*>(h);
  T* yp = static_cast<T*>(y);
  if constexpr (!LAYER) {
    if (res) {
      launch_fwd_k<T, false, true>(xp, rp, wp, bp, hp, yp, mean, rstd, rows, dim, eps, stream);
      return check_launch("scree_add_rmsnorm_fwd");
    }
  }
  launch_fwd_k<T, LAYER, false>(xp, nullptr, wp, bp, nullptr, yp, mean, rstd, rows, dim, eps,
                                stream);
  return check_launch(LAYER ? "scree_layernorm_fwd" : "scree_rmsnorm_fwd");
}

// dres non-null (RMSNorm only): dx also receives dres.
template <typename T, bool LAYER, bool RES>
void launch_bwd_k(const T* dyp, const T* xp, const T* wp, const float* mean, const float* rstd,
                  const T* dresp, T* dxp, float* partial, bool want_params, int nparts,
                  int64_t rows, int64_t dim, hipStream_t stream) {
  const int d = (int)dim;
  const int nparam = LAYER ? 2 : 1;
  if (bwd_fast_path_ok<T>(dim, {dyp, xp, wp, dresp, dxp})) {
    const int nvec = (int)(dim / (16 / sizeof(T)));
    const int cpt = (nvec + kBwdThreads - 1) / kBwdThreads;  // 1 or 2
    const dim3 grid((unsigned)nparts), block(kBwdThreads);
    const int np = want_params ? nparam : 0;
    // rows per step: two steps' rows (double-buffered) fit 4 waves per SIMD
    // (LN keeps two sums per row; the residual gradient is one more vector).
    // At one vector per thread 2 rows per step measured best for all three
    // (RMSNorm at config 2: R = 1, 2, 3, 4 -> 90.8, 87.3, 89.1, 90.5 us).
    constexpr int R1 = 2;
    constexpr int R2 = (LAYER || RES) ? 1 : 2;
    if (cpt == 1)
      hipLaunchKernelGGL((norm_bwd_cols<T, 1, R1, LAYER, RES>), grid, block, 0, stream, dyp, xp, wp,
                         mean, rstd, dresp, dxp, partial, rows, d, np);
    else
      hipLaunchKernelGGL((norm_bwd_cols<T, 2, R2, LAYER, RES>), grid, block, 0, stream, dyp, xp, wp,
                         mean, rstd, dresp, dxp, partial, rows, d, np);
  } else {
    const dim3 grid((unsigned)((rows + kFwdWaves - 1) / kFwdWaves)), block(kFwdWaves * kWave);
    if (rows > 0)
      hipLaunchKernelGGL((norm_bwd_dx_generic<T, LAYER, RES>), grid, block, 0, stream, dyp, xp, wp,
                         mean, rstd, dresp, dxp, rows, d);
    if (want_params) {
      const dim3 pgrid((unsigned)((dim + 255) / 256), (unsigned)nparts);
      hipLaunchKernelGGL((norm_bwd_param_generic<T, LAYER>), pgrid, dim3(256), 0, stream, dyp, xp,
                         mean, rstd, partial, rows, d, nparam);
    }
  }
}

template <typename T, bool LAYER>
int launch_bwd(const void* dy, const void* x, const void* w, const float* mean, const float* rstd,
               const void* dres, void* dx, void* dw, void* db, int dparam_dtype, int64_t rows,
               int64_t dim, void* workspace, hipStream_t stream) {
  const T* dyp = static_cast<const T*>(dy);
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  const T* dresp = static_cast<const T*>(dres);
  T* dxp = static_cast<T*>(dx);
  const int d = (int)dim;
  const int nparam = LAYER ? 2 : 1;
  const bool want_params = (dw != nullptr) || (db != nullptr);
  const int nparts = nparts_for(rows);
  float* partial = static_cast<float*>(workspace);
  const char* fn = LAYER ? "scree_layernorm_bwd" : (dres ? "scree_add_rmsnorm_bwd" : "scree_rmsnorm_bwd");
  bool done = false;
  if constexpr (!LAYER) {
    if (dres) {
      launch_bwd_k<T, false, true>(dyp, xp, wp, mean, rstd, dresp, dxp, partial, want_params,
                                   nparts, rows, dim, stream);
      done = true;
    }
  }
  if (!done)
    launch_bwd_k<T, LAYER, false>(dyp, xp, wp, mean, rstd, nullptr, dxp, partial, want_params,
                                  nparts, rows, dim, stream);
  int rc = check_launch(fn);
  if (rc != SCREE_OK || !want_params) return rc;
  if (dim % 4 == 0) {
    const dim3 cgrid((unsigned)((dim + 15) / 16), (unsigned)nparam);
    hipLaunchKernelGGL(norm_param_colsum4, cgrid, dim3(256), 0, stream, partial, nparts, nparam, d,
                       dw, db, dparam_dtype);
  } else {
    const dim3 cgrid((unsigned)((dim + kWave - 1) / kWave), (unsigned)nparam);
    hipLaunchKernelGGL(norm_param_colsum, cgrid, dim3(256), 0, stream, partial, nparts, nparam, d,
                       dw, db, dparam_dtype);
  }
  return check_launch(fn);
}

int validate_common(const char* fn, int64_t rows, int64_t dim, int dtype) {
  if (rows < 0 || rows >= ((int64_t)1 << 31))
    return set_error(SCREE_ERR_INVALID, "%s: rows must be in [0, 2^31), got %lld", fn, (long long)rows);
  if (dim < 1 || dim > (1 << 24))
    return set_error(SCREE_ERR_INVALID, "%s: dim must be in [1, 2^24], got %lld", fn, (long long)dim);
  if (dtype != SCREE_DTYPE_F32 && dtype != SCREE_DTYPE_F16 && dtype != SCREE_DTYPE_BF16)
    return set_error(SCREE_ERR_UNSUPPORTED, "%s: unknown dtype code %d", fn, dtype);
  if (rows * dim >= ((int64_t)1 << 40))
    return set_error(SCREE_ERR_INVALID, "%s: tensor too large", fn);
  return SCREE_OK;
}

}  // namespace
}  // namespace scree

using namespace scree;

extern "C" size_t scree_norm_bwd_workspace_bytes(int64_t rows, int64_t dim) {
  if (rows < 0 || dim < 1) return 0;
  return (size_t)nparts_for(rows) * 2u * (size_t)dim * sizeof(float);
}

extern "C" int scree_rmsnorm_fwd(const void* x, const void* weight, void* y, float* rstd,
                                 int64_t rows, int64_t dim, float eps, int dtype, void* stream) {
  const char* fn = "scree_rmsnorm_fwd";
  int rc = validate_common(fn, rows, dim, dtype);
  if (rc) return rc;
  if (rows == 0) return SCREE_OK;
  if (!x || !y) return set_error(SCREE_ERR_INVALID, "%s: x and y must be non-null", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_fwd<float, false>(x, nullptr, weight, nullptr, nullptr, y, nullptr, rstd, rows, dim, eps, s);
    case SCREE_DTYPE_F16: return launch_fwd<f16, false>(x, nullptr, weight, nullptr, nullptr, y, nullptr, rstd, rows, dim, eps, s);
    default: return launch_fwd<bf16, false>(x, nullptr, weight, nullptr, nullptr, y, nullptr, rstd, rows, dim, eps, s);
  }
}

extern "C" int scree_layernorm_fwd(const void* x, const void* weight, const void* bias, void* y,
                                   float* mean, float* rstd, int64_t rows, int64_t dim, float eps,
                                   int dtype, void* stream) {
  const char* fn = "scree_layernorm_fwd";
  int rc = validate_common(fn, rows, dim, dtype);
  if (rc) return rc;
  if (rows == 0) return SCREE_OK;
  if (!x || !y) return set_error(SCREE_ERR_INVALID, "%s: x and y must be non-null", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_fwd<float, true>(x, nullptr, weight, bias, nullptr, y, mean, rstd, rows, dim, eps, s);
    case SCREE_DTYPE_F16: return launch_fwd<f16, true>(x, nullptr, weight, bias, nullptr, y, mean, rstd, rows, dim, eps, s);
    default: return launch_fwd<bf16, true>(x, nullptr, weight, bias, nullptr, y, mean, rstd, rows, dim, eps, s);
  }
}

static int validate_bwd(const char* fn, const void* dy, const void* x, const float* rstd, void* dx,
                        bool want_params, int dparam_dtype, int64_t rows, int64_t dim,
                        void* workspace, size_t workspace_bytes) {
  // with no rows, empty row tensors may have no storage: only the parameter
  // gradients (sums over no rows: zeros) are written
  if (rows > 0 && (!dy || !x || !rstd || !dx))
    return set_error(SCREE_ERR_INVALID, "%s: dy, x, rstd and dx must be non-null", fn);
  if (want_params) {
    if (dparam_dtype != SCREE_DTYPE_F32 && dparam_dtype != SCREE_DTYPE_F16 &&
        dparam_dtype != SCREE_DTYPE_BF16)
      return set_error(SCREE_ERR_UNSUPPORTED, "%s: unknown parameter dtype code %d", fn, dparam_dtype);
    const size_t need = scree_norm_bwd_workspace_bytes(rows, dim);
    if (!workspace || workspace_bytes < need)
      return set_error(SCREE_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", fn, need,
                       workspace ? workspace_bytes : (size_t)0);
  }
  return SCREE_OK;
}

extern "C" int scree_rmsnorm_bwd(const void* dy, const void* x, const void* weight,
                                 const float* rstd, void* dx, void* dweight, int dparam_dtype,
                                 int64_t rows, int64_t dim, int dtype, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  const char* fn = "scree_rmsnorm_bwd";
  int rc = validate_common(fn, rows, dim, dtype);
  if (rc) return rc;
  if (dweight && !weight) return set_error(SCREE_ERR_INVALID, "%s: dweight requires weight", fn);
  if (rows == 0 && !dweight) return SCREE_OK;  // nothing to write; empty dweight is summed to 0 below
  rc = validate_bwd(fn, dy, x, rstd, dx, dweight != nullptr, dparam_dtype, rows, dim, workspace,
                    workspace_bytes);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_bwd<float, false>(dy, x, weight, nullptr, rstd, nullptr, dx, dweight, nullptr, dparam_dtype, rows, dim, workspace, s);
    case SCREE_DTYPE_F16: return launch_bwd<f16, false>(dy, x, weight, nullptr, rstd, nullptr, dx, dweight, nullptr, dparam_dtype, rows, dim, workspace, s);
    default: return launch_bwd<bf16, false>(dy, x, weight, nullptr, rstd, nullptr, dx, dweight, nullptr, dparam_dtype, rows, dim, workspace, s);
  }
}

extern "C" int scree_layernorm_bwd(const void* dy, const void* x, const void* weight,
                                   const float* mean, const float* rstd, void* dx, void* dweight,
                                   void* dbias, int dparam_dtype, int64_t rows, int64_t dim,
                                   int dtype, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  const char* fn = "scree_layernorm_bwd";
  int rc = validate_common(fn, rows, dim, dtype);
  if (rc) return rc;
  if (dweight && !weight) return set_error(SCREE_ERR_INVALID, "%s: dweight requires weight", fn);
  if (rows == 0 && !dweight && !dbias) return SCREE_OK;
  if (rows > 0 && !mean) return set_error(SCREE_ERR_INVALID, "%s: mean must be non-null", fn);
  rc = validate_bwd(fn, dy, x, rstd, dx, dweight != nullptr || dbias != nullptr, dparam_dtype, rows,
                    dim, workspace, workspace_bytes);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_bwd<float, true>(dy, x, weight, mean, rstd, nullptr, dx, dweight, dbias, dparam_dtype, rows, dim, workspace, s);
    case SCREE_DTYPE_F16: return launch_bwd<f16, true>(dy, x, weight, mean, rstd, nullptr, dx, dweight, dbias, dparam_dtype, rows, dim, workspace, s);
    default: return launch_bwd<bf16, true>(dy, x, weight, mean, rstd, nullptr, dx, dweight, dbias, dparam_dtype, rows, dim, workspace, s);
  }
}

extern "C" int scree_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight,
                                     void* h, void* y, float* rstd, int64_t rows, int64_t dim,
                                     float eps, int dtype, void* stream) {
  const char* fn = "scree_add_rmsnorm_fwd";
  int rc = validate_common(fn, rows, dim, dtype);
  if (rc) return rc;
  if (rows == 0) return SCREE_OK;
  if (!x || !residual || !h || !y)
    return set_error(SCREE_ERR_INVALID, "%s: x, residual, h and y must be non-null", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_fwd<float, false>(x, residual, weight, nullptr, h, y, nullptr, rstd, rows, dim, eps, s);
    case SCREE_DTYPE_F16: return launch_fwd<f16, false>(x, residual, weight, nullptr, h, y, nullptr, rstd, rows, dim, eps, s);
    default: return launch_fwd<bf16, false>(x, residual, weight, nullptr, h, y, nullptr, rstd, rows, dim, eps, s);
  }
}

extern "C" int scree_add_rmsnorm_bwd(const void* dy, const void* dh, const void* h,
                                     const void* weight, const float* rstd, void* dx,
                                     void* dweight, int dparam_dtype, int64_t rows, int64_t dim,
                                     int dtype, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  const char* fn = "scree_add_rmsnorm_bwd";
  int rc = validate_common(fn, rows, dim, dtype);
  if (rc) return rc;
  if (dweight && !weight) return set_error(SCREE_ERR_INVALID, "%s: dweight requires weight", fn);
  if (rows == 0 && !dweight) return SCREE_OK;
  rc = validate_bwd(fn, dy, h, rstd, dx, dweight != nullptr, dparam_dtype, rows, dim, workspace,
                    workspace_bytes);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case SCREE_DTYPE_F32: return launch_bwd<float, false>(dy, h, weight, nullptr, rstd, dh, dx, dweight, nullptr, dparam_dtype, rows, dim, workspace, s);
    case SCREE_DTYPE_F16: return launch_bwd<f16, false>(dy, h, weight, nullptr, rstd, dh, dx, dweight, nullptr, dparam_dtype, rows, dim, workspace, s);
    default: return launch_bwd<bf16, false>(dy, h, weight, nullptr, rstd, dh, dx, dweight, nullptr, dparam_dtype, rows, dim, workspace, s);
  }
}
