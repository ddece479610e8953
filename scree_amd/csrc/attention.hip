// Varlen causal / non-causal self-attention for gfx950: tile scheduler,
// forward (O + logsumexp) and backward (dQ with Delta, then dK/dV).
//
// Layout: q, k, v, o, do, dq, dk, dv are (total_tokens, heads, D) with the D
// axis contiguous; lse and delta are contiguous (total_tokens, heads) fp32.
//
// Work decomposition.  A sequence of length L has nblk = ceil(L / 128) row
// blocks.  The scheduler kernel writes one (seq, blk) item per row block, in
// longest-work-first order, into the workspace; every attention kernel is
// launched with grid = Tmax * heads (Tmax = ceil(N/128) + B bounds the item
// count on the host, so the host never reads the offsets) and block b takes
// item b / heads, head b % heads.  Blocks past the real item count return at
// once.  No padded grid, no host synchronisation.
//
// One workgroup = 4 wavefronts; each wavefront owns 32 rows of its item's
// 128 (queries for the forward and dQ, keys for dK/dV) and runs 32x32x16
// MFMAs.  MFMA lane layout (see mfma32 in common.h): for a 32x32 product
// C = A*B with k = 16, lane l (g = l/32, r = l%32) supplies row r of A and
// column r of B at k = 8g..8g+7, and receives C[8*(i/4) + 4g + i%4][r] in
// element i.
//
// Scores are formed transposed, S^T = K Q^T, so lane r owns one query and
// the row softmax is in-lane plus one exchange with lane r^32.  Element i of
// a 32-key tile of S^T then holds key 8*(i/4) + 4g + i%4, and elements
// 8h..8h+7 are exactly the keys {16h + 4g + 0..3, 16h + 8 + 4g + 0..3}: used
// as the k = 16 operand of the next MFMA (P^T as B, with V^T read from LDS at
// the same two 4-key runs as A), P never leaves registers.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"

namespace scree {
namespace {

constexpr int kWave = 64;
constexpr int kThreads = 256;   // 4 wavefronts
constexpr int kBM = 128;        // rows per item (4 waves x 32)
constexpr int kBN = 64;         // keys per staged block (forward, dQ)
constexpr int kMaxBatch = 2048; // sequences the sorting scheduler handles (more: natural order)
constexpr int kMaxClass = 4096; // row blocks per sequence it sorts (longer: natural order)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// ------------------------------------------------------------ workspace
// int32 header[4] = {item count T, batch, kBM, causal}, then two lists of
// int4 items[Tmax] = {seq, blk, start, len}: longest-work-first, then the same
// items sequence by sequence (attn_schedule_kernel).  start/len are the sequence's offsets clamped to
// [0, total_tokens], so attention kernels never index outside the tensors
// even for malformed offsets.  If any offset decreases (overlapping or
// negative-length sequences), or the offsets would make T exceed Tmax, the
// scheduler publishes T = 0 (no work) and header[1] = -1, and the attention
// kernels then fill their outputs with NaN (poison_rows): the device-side
// check that lets callers skip a host read of the offsets.
constexpr size_t kHeaderBytes = 16;

inline int64_t tmax_for(int batch, int64_t total) { return (total + kBM - 1) / kBM + batch; }
inline size_t schedule_bytes(int64_t tmax) { return kHeaderBytes + 2 * (size_t)tmax * sizeof(int4); }
// Past kMaxBatch the workspace also holds batch + 1 prefix sums after the lists.
inline size_t prefix_bytes(int batch) {
  return batch > kMaxBatch ? (((size_t)batch + 1) * sizeof(int32_t) + 15) & ~(size_t)15 : 0;
}

// ------------------------------------------------------------ scheduler
__device__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

// In-place exclusive scans of a[0..n) and b[0..n), held in LDS by the whole
// block, sharing their barriers; the totals go to ta / tb.  wtot holds 64
// ints.  Caller synchronises before; this synchronises after.
__device__ void block_excl_scan2(int* a, int* b, int n, int* wtot, int& ta, int& tb) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave, nw = nt / kWave;
  const int per = (n + nt - 1) / nt;
  const int beg = min(n, tid * per), end = min(n, beg + per);
  int la = 0, lb = 0;
  for (int i = beg; i < end; ++i) {
    la += a[i];
    lb += b[i];
  }
  const int ia = wave_incl_scan(la), ib = wave_incl_scan(lb);
  if (lane == kWave - 1) {
    wtot[wave] = ia;
    wtot[32 + wave] = ib;
  }
  __syncthreads();
  if (wave == 0) {  // inclusive prefixes of the wave totals
    int t = lane < nw ? wtot[lane] : 0, u = lane < nw ? wtot[32 + lane] : 0;
    t = wave_incl_scan(t);
    u = wave_incl_scan(u);
    if (lane < nw) {
      wtot[16 + lane] = t;
      wtot[48 + lane] = u;
    }
  }
  __syncthreads();
  int ra = ia - la + (wave > 0 ? wtot[16 + wave - 1] : 0);
  int rb = ib - lb + (wave > 0 ? wtot[48 + wave - 1] : 0);
  for (int i = beg; i < end; ++i) {
    const int t = a[i], u = b[i];
    a[i] = ra;
    b[i] = rb;
    ra += t;
    rb += u;
  }
  ta = wtot[16 + nw - 1];
  tb = wtot[48 + nw - 1];
  __syncthreads();
}

// One 1024-thread block.  See oracle/schedule.py for the order produced.
__global__ __launch_bounds__(1024) void attn_schedule_kernel(const int32_t* __restrict__ cu,
                                                             int batch, int total_tokens,
                                                             int causal, int tmax,
                                                             int32_t* __restrict__ header,
                                                             int4* __restrict__ items) {
  __shared__ int s_start[kMaxBatch];
  __shared__ int s_len[kMaxBatch];
  __shared__ int s_nblk[kMaxBatch];
  __shared__ int s_rank[kMaxBatch];
  __shared__ int s_sorted_scan[kMaxBatch + 1];
  __shared__ int s_nat_scan[kMaxBatch + 1];
  __shared__ int s_cls[kMaxClass + 2];
  __shared__ int s_wtot[64];
  __shared__ int s_cmax, s_bad;
  const int tid = threadIdx.x, nt = blockDim.x;
  if (tid == 0) s_cmax = s_bad = 0;
  __syncthreads();
  for (int s = tid; s < batch; s += nt) {
    if (cu[s + 1] < cu[s]) s_bad = 1;  // decreasing offsets: the schedule fails
    const int a = min(max(cu[s], 0), total_tokens);
    const int b = min(max(cu[s + 1], a), total_tokens);
    const int len = b - a;
    const int nb = (len + kBM - 1) / kBM;
    s_start[s] = a;
    s_len[s] = len;
    s_nblk[s] = nb;
    s_nat_scan[s] = nb;
    atomicMax(&s_cmax, nb);
  }
  __syncthreads();
  const int cmax = s_cmax;
  // Rank by (-nblk, seq): the longest sequences first, ties by index.
  for (int s = tid; s < batch; s += nt) {
    const int mine = s_nblk[s];
    int r = 0;
    for (int t = 0; t < batch; ++t) {
      const int o = s_nblk[t];
      r += (o > mine) || (o == mine && t < s);
    }
    s_rank[s] = r;
    s_sorted_scan[r] = mine;
  }
  __syncthreads();
  // Item bases of each sequence: in natural order (s_nat_scan), and in rank
  // order (s_sorted_scan), how the non-causal and the sequence-major lists
  // place sequences.
  int total, total_ranked;
  block_excl_scan2(s_nat_scan, s_sorted_scan, batch, s_wtot, total, total_ranked);
  (void)total_ranked;  // equals total
  if (tid == 0) s_nat_scan[batch] = total;
  const bool by_class = causal && cmax <= kMaxClass;
  if (by_class) {
    // Histogram of nblk, then two suffix passes by one wave:
    // A(c) = #{s : nblk_s >= c} and offs(c) = sum_{c' > c} A(c').
    for (int c = tid; c <= cmax + 1; c += nt) s_cls[c] = 0;
    __syncthreads();
    for (int s = tid; s < batch; s += nt) {
      const int nb = s_nblk[s];
      if (nb > 0) atomicAdd(&s_cls[nb], 1);
    }
    __syncthreads();
    if (tid < kWave) {  // lane l walks c = cmax - per*l downwards
      const int lane = tid;
      // Pass 1: A(c) = sum_{v >= c} hist(v), for c = cmax..1 (suffix scan).
      const int per = (cmax + kWave - 1) / kWave;
      const int top = cmax - per * lane;
      const int bot = max(1, top - per + 1);
      int local = 0;
      for (int c = top; c >= bot && c >= 1; --c) local += s_cls[c];
      int incl = wave_incl_scan(local);
      int run = incl - local;  // sum of hist above this lane's range
      for (int c = top; c >= bot && c >= 1; --c) {
        run += s_cls[c];
        s_cls[c] = run;  // A(c)
      }
      // Pass 2: offs(c) = sum_{c' > c} A(c').
      local = 0;
      for (int c = top; c >= bot && c >= 1; --c) local += s_cls[c];
      incl = wave_incl_scan(local);
      run = incl - local;
      for (int c = top; c >= bot && c >= 1; --c) {
        const int a = s_cls[c];
        s_cls[c] = run;  // offs(c)
        run += a;
      }
    }
    __syncthreads();
  }
  __syncthreads();
  // Emit: natural item index i -> (seq, blk) by binary search, then place.
  const bool fits = total <= tmax && !s_bad;
  for (int i = tid; fits && i < total; i += nt) {
    int lo = 0, hi = batch - 1;  // find s with nat[s] <= i < nat[s+1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_nat_scan[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    const int s = lo;
    const int b = i - s_nat_scan[s];
    int p;
    if (!causal) p = s_sorted_scan[s_rank[s]] + b;
    else if (by_class) p = s_cls[b + 1] + s_rank[s];
    else p = i;
    const int4 it = make_int4(s, b, s_start[s], s_len[s]);
    items[p] = it;
    // sequence-major: sequences in rank order, each one's blocks from the last
    items[tmax + s_sorted_scan[s_rank[s]] + s_nblk[s] - 1 - b] = it;
  }
  if (tid == 0) {
    header[0] = fits ? total : 0;
    header[1] = fits ? batch : -1;
    header[2] = kBM;
    header[3] = causal;
  }
}

// ------------------------------------------------- wave-level scheduler
// A batch of at most kWaveSched sequences fits one wavefront, lane s holding
// sequence s, and any item of either list follows from per-lane registers:
//  * causal (at most kMaxClass blocks per sequence): class c = blk + 1 from
//    the largest down, each class in sequence rank order.  Class c starts at
//    F(c) = sum_s max(0, nblk_s - c) and holds the A(c) sequences with
//    nblk >= c, which are exactly ranks 0 .. A(c) - 1;
//  * causal with a longer sequence: natural order (sequence by sequence);
//  * non-causal: sequences in rank order, blocks ascending;
//  * sequence-major (second list): rank order, blocks from the last down.
// attn_wave_schedule_kernel gives every item a wavefront of its own, which
// works it out with register and DPP operations only: no LDS, no barrier.
// The scheduler sits on the critical path of every attention step, and the
// one-block kernel above spends ~4 us there in barriers and LDS round trips.
constexpr int kWaveSched = 64;

// Wave-uniform sum / maximum of an int over the 64 lanes (all active): four
// DPP steps combine each 16-lane row (lane ^ 1, lane ^ 2, then the mirrors
// across 8 and across 16 lanes, each pairing a lane with one in the other
// half), and the four row results are read as scalars.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_i<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_i<0x141>(v);  // row_half_mirror
  v += dpp_i<0x140>(v);  // row_mirror
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp_i<0xB1>(v));
  v = max(v, dpp_i<0x4E>(v));
  v = max(v, dpp_i<0x141>(v));
  v = max(v, dpp_i<0x140>(v));
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int first_lane(bool pred) {
  const unsigned long long m = __ballot(pred);
  return m ? __builtin_ctzll(m) : 0;
}

struct WaveSched {
  int start, len, nb;  // this lane's sequence: clamped start, length, row blocks
  int total, cmax;     // item count and largest nblk (wave-uniform)
  bool bad;            // some offset decreases (wave-uniform): the schedule fails
};

// Offsets are clamped as in attn_schedule_kernel; lanes >= batch hold empty
// sequences, which rank after every real one.
__device__ __forceinline__ WaveSched wave_sched(const int32_t* __restrict__ cu, int batch,
                                                int total_tokens) {
  const int lane = threadIdx.x & (kWave - 1);
  WaveSched w;
  int a = 0, b = 0;
  bool dec = false;
  if (lane < batch) {
    const int c0 = cu[lane], c1 = cu[lane + 1];
    dec = c1 < c0;
    a = min(max(c0, 0), total_tokens);
    b = min(max(c1, a), total_tokens);
  }
  w.bad = __ballot(dec) != 0;
  w.start = a;
  w.len = b - a;
  w.nb = (w.len + kBM - 1) / kBM;
  w.total = wave_sum_i(w.nb);
  w.cmax = wave_max_i(w.nb);
  return w;
}

// The lane of the k-th (from 0, in lane order) lane where pred holds; it must exist.
__device__ __forceinline__ int nth_lane(bool pred, int k) {
  const unsigned long long m = __ballot(pred);
  const int below = (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
  return first_lane(pred && below == k);
}

// Rank order is nblk descending, ties by sequence index: the sequence of rank
// r has the largest nblk v with count(nblk >= v) > r and is the
// (r - count(nblk > v))-th of those holding v.  The caller knows that
// count(nblk >= lo) > r.  Binary search over v with one ballot a step, in
// place of comparing every pair of sequences.
__device__ __forceinline__ int lane_of_rank(const WaveSched& w, int r, int lo) {
  int hi = w.cmax;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int)__popcll(__ballot(w.nb >= mid)) > r)
      lo = mid;
    else
      hi = mid - 1;
  }
  return nth_lane(w.nb == lo, r - __popcll(__ballot(w.nb > lo)));
}

// Item p (< w.total) of the work-order list (seq_major false) or of the
// sequence-major list, as {seq, blk, start, len}.  Lanes past the batch hold
// nblk 0 and are never selected.
__device__ __forceinline__ int4 wave_item(const WaveSched& w, int batch, bool causal,
                                          bool seq_major, int p) {
  int s, b;
  if (!seq_major && causal && w.cmax <= kMaxClass) {
    int lo = 1, hi = w.cmax;  // the smallest class c with F(c) <= p (F falls with c)
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (wave_sum_i(max(0, w.nb - mid)) <= p)
        hi = mid;
      else
        lo = mid + 1;
    }
    // class lo holds the sequences of ranks 0 .. count(nblk >= lo) - 1
    s = lane_of_rank(w, p - wave_sum_i(max(0, w.nb - lo)), lo);
    b = lo - 1;
  } else if (!seq_major && causal) {
    const int lane = threadIdx.x & (kWave - 1);
    const int incl = wave_incl_scan(w.nb);
    const int nat = incl - w.nb;
    s = first_lane(lane < batch && nat <= p && p < incl);
    b = p - __builtin_amdgcn_readlane(nat, s);
  } else {
    // sequences in rank order, each nblk items long: the largest v whose
    // sequences (nblk >= v) cover position p, then p's place among the
    // sequences holding exactly v
    int lo = 1, hi = w.cmax;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (wave_sum_i(w.nb >= mid ? w.nb : 0) > p)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int q = p - wave_sum_i(w.nb > lo ? w.nb : 0);
    const int k = q / lo, j = q - k * lo;
    s = nth_lane(w.nb == lo, k);
    b = seq_major ? lo - 1 - j : j;
  }
  return make_int4(s, b, __builtin_amdgcn_readlane(w.start, s), __builtin_amdgcn_readlane(w.len, s));
}

// The two lists and the header for a batch of at most kWaveSched sequences:
// wave g of the grid writes item g of both lists (grid: tmax waves).
__global__ __launch_bounds__(256) void attn_wave_schedule_kernel(const int32_t* __restrict__ cu,
                                                                 int batch, int total_tokens,
                                                                 int causal, int tmax,
                                                                 int32_t* __restrict__ header,
                                                                 int4* __restrict__ items) {
  const WaveSched w = wave_sched(cu, batch, total_tokens);
  const bool fits = w.total <= tmax && !w.bad;
  const int p = blockIdx.x * (blockDim.x / kWave) + (int)(threadIdx.x / kWave);
  if (fits && p < w.total) {
    const int4 a = wave_item(w, batch, causal != 0, false, p);
    const int4 c = wave_item(w, batch, causal != 0, true, p);
    if ((threadIdx.x & (kWave - 1)) == 0) {
      items[p] = a;
      items[tmax + p] = c;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    header[0] = fits ? w.total : 0;
    header[1] = fits ? batch : -1;
    header[2] = kBM;
    header[3] = causal;
  }
}

// ------------------------------------------------- where items come from
// The forward of a batch of at most kWaveSched sequences in a launch of a few
// rounds of workgroups (attn_fwd_derives) needs no scheduler launch: every
// wave of every workgroup derives its own item from cu_seqlens with the code
// above (~150 instructions before its first load), and the forward leaves
// the header and its work-order list in the workspace exactly as
// attn_wave_schedule_kernel writes them (the last block the header; the
// head-0 workgroup of each item that item's entry), so the backward passes that
// follow read them.  Such a launch is head-minor, and so are both backward
// passes of the problem (the dQ grid is the forward's, the dK/dV grid at most
// that): none reads the sequence-major list, which stays as it was.  The
// backward passes always read the lists: deriving there cost more (dQ +1.9,
// dK/dV +1.5 us at config 4) than the forward does (+1.0 us), and the
// forward saves the scheduler launch (3.4 us).
struct ItemSource {
  const int32_t* header;
  const int4* items;  // the list this launch reads
  const int32_t* cu;
  int32_t* publish;   // workspace the deriving forward writes header and list into
  int batch, total_tokens;
  int seq_major;      // the sequence-major list (head-major launches)
  int derive;         // derive items from cu (the forward, batch <= kWaveSched)
};

// The schedule as this wave sees it: whether it failed (offsets that
// describe more work than tmax) and the item count.  The header and the
// listed item are loaded in both modes (the workspace always holds them;
// stale bytes when deriving) so that on the list path their loads issue
// with the kernel arguments rather than after a branch on src.derive.
// MAY_DERIVE false (the backward passes) compiles the list path alone.
struct ItemView {
  WaveSched w;
  bool failed;
  int count;
};
template <bool MAY_DERIVE>
__device__ __forceinline__ ItemView item_view(const ItemSource& src, int tmax) {
  const int listed_count = src.header[0], listed_batch = src.header[1];
  ItemView v;
  v.w = WaveSched{0, 0, 0, 0, 0, false};
  if (MAY_DERIVE && src.derive) v.w = wave_sched(src.cu, src.batch, src.total_tokens);
  const bool derive = MAY_DERIVE && src.derive;
  v.failed = derive ? (v.w.total > tmax || v.w.bad) : listed_batch < 0;
  v.count = derive ? (v.failed ? 0 : v.w.total) : min(max(listed_count, 0), tmax);
  return v;
}
// On the list path an item that no schedule can have written -- a workspace
// handed to a backward call before any schedule or forward call filled it --
// comes out empty (len 0), and the kernels skip it: wrong results for a
// misused workspace, never an access outside the tensors.
template <bool MAY_DERIVE>
__device__ __forceinline__ int4 item_at(const ItemSource& src, const ItemView& v, bool causal, int p) {
  const int4 listed = src.items[p];
  int4 it = make_int4(0, 0, 0, 0);
  if (MAY_DERIVE && src.derive) it = wave_item(v.w, src.batch, causal, src.seq_major != 0, p);
  const int4 sel = MAY_DERIVE && src.derive ? it : listed;  // a derived item always passes
  const bool ok = sel.z >= 0 && sel.w >= 1 && sel.z <= src.total_tokens - sel.w && sel.y >= 0 &&
                  (int64_t)sel.y * kBM < sel.w;
  return ok ? sel : make_int4(0, 0, 0, 0);
}

// The deriving forward's share of the schedule: the last block (the
// shortest item, or none; block 0 runs the longest) writes the header
// (failed offsets: no items and batch -1, as the scheduler publishes them),
// on whichever path it leaves the kernel.
__device__ __forceinline__ void publish_header(const ItemSource& src, const ItemView& v, int causal) {
  if (src.publish && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
    src.publish[0] = v.count;
    src.publish[1] = v.failed ? -1 : src.batch;
    src.publish[2] = kBM;
    src.publish[3] = causal;
  }
}
// Item p of the work-order list, from the head-0 workgroup of item p.
__device__ __forceinline__ void publish_item(const ItemSource& src, int p, const int4& it) {
  if (src.publish && threadIdx.x == 0)
    reinterpret_cast<int4*>(src.publish + kHeaderBytes / sizeof(int32_t))[p] = it;
}

// ------------------------------------------------- batches past kMaxBatch
// More sequences than attn_schedule_kernel's LDS arrays hold.  One
// 1024-thread block writes both lists in natural order instead: sequence by
// sequence, blocks ascending in the first list and from the last down in the
// second.  The per-sequence block prefix sums go to a tail of the workspace
// after the two lists (batch + 1 ints).  Only the balance of a launch, not its
// result, depends on the longest-first order, and batches this large are
// made of short sequences.
__global__ __launch_bounds__(1024) void attn_big_schedule_kernel(
    const int32_t* __restrict__ cu, int batch, int total_tokens, int causal, int tmax,
    int32_t* __restrict__ header, int4* __restrict__ items, int32_t* __restrict__ prefix) {
  __shared__ int s_wtot[16];
  __shared__ int s_run, s_bad;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int nw = blockDim.x / kWave;
  if (tid == 0) s_run = s_bad = 0;
  __syncthreads();
  for (int c0 = 0; c0 < batch; c0 += blockDim.x) {  // exclusive scan of nblk, chunk by chunk
    const int s = c0 + tid;
    int nb = 0;
    if (s < batch) {
      if (cu[s + 1] < cu[s]) s_bad = 1;  // decreasing offsets: the schedule fails
      const int a = min(max(cu[s], 0), total_tokens);
      const int b = min(max(cu[s + 1], a), total_tokens);
      nb = (b - a + kBM - 1) / kBM;
    }
    const int incl = wave_incl_scan(nb);
    if (lane == kWave - 1) s_wtot[wave] = incl;
    __syncthreads();
    if (wave == 0) {
      int t = lane < nw ? s_wtot[lane] : 0;
      t = wave_incl_scan(t);
      if (lane < nw) s_wtot[lane] = t;
    }
    __syncthreads();
    if (s < batch) prefix[s] = s_run + (wave > 0 ? s_wtot[wave - 1] : 0) + incl - nb;
    __syncthreads();  // every thread has read s_run and s_wtot
    if (tid == 0) s_run += s_wtot[nw - 1];
    __syncthreads();
  }
  const int total = s_run;
  if (tid == 0) prefix[batch] = total;
  __threadfence();  // the prefix sums, written by every thread, are read by any
  __syncthreads();
  const bool fits = total <= tmax && !s_bad;
  for (int i = tid; fits && i < total; i += blockDim.x) {
    int lo = 0, hi = batch - 1;  // the last sequence s with prefix[s] <= i (skips empty ones)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (prefix[mid] <= i)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int s = lo, b = i - prefix[s], nb = prefix[s + 1] - prefix[s];
    const int a = min(max(cu[s], 0), total_tokens);
    const int e = min(max(cu[s + 1], a), total_tokens);
    const int4 it = make_int4(s, b, a, e - a);
    items[i] = it;
    items[tmax + prefix[s] + nb - 1 - b] = it;
  }
  if (tid == 0) {
    header[0] = fits ? total : 0;
    header[1] = fits ? batch : -1;
    header[2] = kBM;
    header[3] = causal;
  }
}

// ------------------------------------------------------- tile staging
// Raw buffer resource for `bytes` bytes at `base` (gfx9 descriptor: stride 0,
// dword3 = 0x00020000).  Loads at offsets past `bytes` return zeros.  (Used
// only in device passes, hence maybe_unused for the host pass.)
[[maybe_unused]] __device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                                             uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <typename T>
__device__ __forceinline__ typename VecT<T>::x8 lds_frag16(const T* p) {
  return __builtin_bit_cast(typename VecT<T>::x8, *reinterpret_cast<const uint4*>(p));
}
// Transposed operand from a row-major LDS tile X[row][col].
// ds_read_tr16_b64 hands lane 16G + i, slot j, element i%4 of the 8 bytes
// addressed by lane 16G + 4j + i/4.  With each lane addressing
// X[4g + (lr%16)/4][16*(lr/16) + 4*(lr%4)] (offset `o.x` from swz_tr_off,
// which adds the tile swizzle), lane (lr, g) receives X[4g + j][lr] in slots
// j = 0..3; a second read 8 rows further (offset `o.y`) gives slots 4..7.
// That is the k-run layout {4g + 0..3, 8 + 4g + 0..3} of the MFMA operands
// here (rows of X are the k axis, columns the M axis).
template <typename T>
__device__ __forceinline__ typename VecT<T>::x8 lds_frag_tr(const T* base, int2 o) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) s4* lds_s4;
  const s4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(base + o.x));
  const s4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(base + o.y));
  const s8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(typename VecT<T>::x8, v);
}
template <typename T>
__device__ __forceinline__ typename VecT<T>::x8 gmem_frag16(const T* p) {
  return __builtin_bit_cast(typename VecT<T>::x8, ld16(p));
}
// head_dim 16 runs the 32-column kernels on rows padded with zero columns:
// they add nothing to any dot product, and the padded outputs are not stored.
// Only the 32-column kernels can see a row narrower than their D (dcols).
template <int D>
__device__ __forceinline__ bool col_live(int c0, int dcols) {
  return D > 32 || c0 < dcols;
}
// Columns [c0, c0 + 8) of a row that holds `dcols` columns; zeros past them.
template <int D, typename T>
__device__ __forceinline__ typename VecT<T>::x8 gmem_frag16_cols(const T* row, int c0, int dcols) {
  if (col_live<D>(c0, dcols)) return gmem_frag16(row + c0);
  return __builtin_bit_cast(typename VecT<T>::x8, make_uint4(0u, 0u, 0u, 0u));
}
// Elements e0..e0+7 of a 16-float accumulator, rounded to T, as an operand.
template <typename T>
__device__ __forceinline__ typename VecT<T>::x8 pack_frag(const f32x16& c, int e0) {
  const uint4 u = make_uint4(pack2<T>(c[e0 + 0], c[e0 + 1]), pack2<T>(c[e0 + 2], c[e0 + 3]),
                             pack2<T>(c[e0 + 4], c[e0 + 5]), pack2<T>(c[e0 + 6], c[e0 + 7]));
  return __builtin_bit_cast(typename VecT<T>::x8, u);
}
// Store the 16 values of one 32x32 accumulator column-slice: element i is
// D-index d0 + 8*(i/4) + 4g + i%4 of a row; scaled by `mul`.
template <typename T>
__device__ __forceinline__ void store_row_slice(T* row_ptr, int d0, int g, const f32x16& c,
                                                float mul) {
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const uint32_t lo = pack2<T>(c[4 * qd + 0] * mul, c[4 * qd + 1] * mul);
    const uint32_t hi = pack2<T>(c[4 * qd + 2] * mul, c[4 * qd + 3] * mul);
    *reinterpret_cast<uint2*>(row_ptr + d0 + 8 * qd + 4 * g) = make_uint2(lo, hi);
  }
}

// Row-contiguous stores of a wave's 32 result rows, staged through LDS.
// store_row_slice writes each lane's 4-element runs straight to memory: one
// instruction then touches 32 rows x 16 bytes, and under the attention
// kernels' load such scattered stores take microseconds just to issue.  Here
// the wave writes its accumulators (store_row_slice's layout, scaled by the
// lane's `mul`) into a wave-private LDS area of 32 rows x (D + 8) elements
// (the pad spreads the rows over the banks), then reads it back so that lane
// l holds 16-byte chunk l % CPR of row l / CPR (+ 64 / CPR per round), and
// CPR lanes store one contiguous row.  Rows >= nrows and columns >= dcols
// (head_dim 16 in the 32-column kernels) are not stored.  LDS
// accesses of one wave are processed in order, so the read-back sees the
// writes without a workgroup barrier; the caller guarantees no other wave
// uses `stage` meanwhile.
constexpr int kStagePad = 8;
template <int D>
constexpr int stage_elems() {
  return 32 * (D + kStagePad);
}
template <typename T, int D>
__device__ __forceinline__ void store_rows_staged(T* __restrict__ stage, const f32x16 (&acc)[D / 32],
                                                  float mul, T* __restrict__ dst, int64_t row_stride,
                                                  int nrows, int dcols, int lr, int g, int lane) {
  constexpr int SD = D + kStagePad;
  constexpr int CPR = D / 8;       // 16-byte chunks per row
  constexpr int RPR = 64 / CPR;    // rows per read round
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const uint32_t lo = pack2<T>(acc[dt][4 * qd + 0] * mul, acc[dt][4 * qd + 1] * mul);
      const uint32_t hi = pack2<T>(acc[dt][4 * qd + 2] * mul, acc[dt][4 * qd + 3] * mul);
      *reinterpret_cast<uint2*>(stage + lr * SD + 32 * dt + 8 * qd + 4 * g) = make_uint2(lo, hi);
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int c = lane % CPR;
#pragma unroll
  for (int j = 0; j < 32 / RPR; ++j) {
    const int r = lane / CPR + RPR * j;
    const uint4 v = *reinterpret_cast<const uint4*>(stage + r * SD + 8 * c);
    if (r < nrows && col_live<D>(8 * c, dcols))
      *reinterpret_cast<uint4*>(dst + (int64_t)r * row_stride + 8 * c) = v;
  }
}

// 2^x on the hardware unit (v_exp_f32); results below 2^-126 may flush to 0,
// which softmax weights tolerate.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row (within a 32-row MFMA tile, lane group g = 0) of accumulator element i;
// lane group g adds 4g.
constexpr int acc_row0(int i) { return 8 * (i >> 2) + (i & 3); }

// Mask (to -inf) the elements of a 32x32 tile whose row exceeds `rel`:
// element i is row acc_row0(i) + 4g, so the test is acc_row0(i) > rel - 4g.
// Callers mask only the (rare) diagonal tile, under a branch.  The empty
// volatile asm cannot be speculated, so the compiler keeps that branch:
// without it, it turned the masking into 16 v_cndmask executed on every
// tile (32 in the dK/dV pass), their 16 lane masks held in registers across
// the block loop.  The forward (OPAQUE = false) masks only in the blocks of
// its peeled diagonal loop, where the plain form needs no extra register.
template <bool OPAQUE = true>
__device__ __forceinline__ void mask_rows_above(f32x16& c, int rel_minus_4g) {
  if (OPAQUE) asm volatile("" : "+v"(rel_minus_4g));
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (acc_row0(i) > rel_minus_4g) c[i] = kNegInf;
}
// The converse: mask the elements whose row is below `rel` (acc_row0(i) <
// rel - 4g).
__device__ __forceinline__ void mask_rows_below(f32x16& c, int rel_minus_4g) {
  asm volatile("" : "+v"(rel_minus_4g));
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (acc_row0(i) < rel_minus_4g) c[i] = kNegInf;
}

// Wave index as a scalar, so per-wave tile bounds are uniform branches.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); }

// Workgroup barrier once this wave's LDS accesses have completed and at most
// its newest N vector-memory operations are still in flight.  Written without
// a fence: __syncthreads()'s release fence waits for every outstanding LDS
// write, direct-to-LDS DMA included, which would drain a DMA issued for a
// later block.  The memory clobber keeps the compiler from moving memory
// accesses across it; DMA data in LDS is visible to the workgroup once the
// issuing wave's vmcnt has counted it.
template <int N>
__device__ __forceinline__ void barrier_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate (6 bits on gfx9)");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

struct Strides {
  int64_t row, head;
};

// Workgroups are dispatched round-robin over the 8 XCDs (block b runs on XCD
// b % 8), each with its own L2.  Two block -> (item, head) orders:
//  * head-minor (block b -> item b / heads, head b % heads): every head's
//    longest items start first -- best balance when each XCD has only a few
//    rounds of work.  With heads a multiple of 8 each head still stays on one
//    XCD.
//  * head-major (heads a multiple of 8): XCD x works through heads x, x + 8,
//    ... one at a time, each in the scheduler's longest-first order, so one
//    head's K/V is the L2 working set -- best when each XCD has many rounds.
// The host picks (attn_head_major).  Returns false for blocks past the work.
//
// Grouped-query attention (group > 1 query heads per K/V head): with heads a
// multiple of 8 the head index is permuted so that XCD x serves the
// contiguous heads x*heads/8 .. (x+1)*heads/8 - 1 instead of x, x+8, ...;
// when group divides heads/8, every group then shares one XCD and its K/V
// stays in that XCD's L2.
constexpr int kXcds = 8;

// pair (sequence-major, rows of head_dim narrower than a 128-byte line, no
// grouped K/V): heads 2m and 2m + 1 of a token share a line, so the logical
// blocks 2k and 2k + 1 run as blocks b and b + 8 of each group of 16, which
// share an XCD and its L2 (block b runs on XCD b mod 8); blocks past the last
// full group of 16 keep their index.
__device__ __forceinline__ bool map_block_at(int b, int heads, int tmax, int head_major, int group,
                                             bool pair, int& item, int& head) {
  if (head_major) {
    const int x = b % kXcds, j = b / kXcds;
    const int k = j / tmax;  // k-th head of this XCD
    item = j - k * tmax;
    head = x + kXcds * k;
    if (head >= heads) return false;
  } else {
    if (pair && b < (int)(gridDim.x & ~15u)) b = (b & ~15) | ((b & 7) << 1) | ((b >> 3) & 1);
    item = b / heads;
    head = b % heads;
  }
  if (group > 1 && heads % kXcds == 0) head = (head % kXcds) * (heads / kXcds) + head / kXcds;
  return true;
}
__device__ __forceinline__ bool map_block(int heads, int tmax, int head_major, int group,
                                          bool pair, int& item, int& head) {
  return map_block_at(blockIdx.x, heads, tmax, head_major, group, pair, item, head);
}

// The scheduler publishes header[1] = -1 when some offset decreases (which is
// also the only way the offsets can describe more work than the host bound
// allows).  Every kernel then fills its outputs with NaN, block
// b taking token rows b, b + grid, ..., instead of leaving them unwritten.
template <typename T>
__device__ __forceinline__ void poison_rows(T* __restrict__ p, Strides s, int total, int heads, int d) {
  const T nan = from_f32<T>(__builtin_nanf(""));
  for (int64_t t = blockIdx.x; t < total; t += gridDim.x)
    for (int i = threadIdx.x; i < heads * d; i += blockDim.x)
      p[t * s.row + (int64_t)(i / d) * s.head + i % d] = nan;
}
__device__ __forceinline__ void poison_stats(float* __restrict__ p, int total, int heads) {
  for (int64_t t = blockIdx.x; t < total; t += gridDim.x)
    for (int i = threadIdx.x; i < heads; i += blockDim.x) p[t * heads + i] = __builtin_nanf("");
}

// The forward keeps a reference maximum m per softmax row and forms weights
// p = 2^(s*c - m*c) without first taking each tile's maximum: a lane checks
// the sum of its 16 weights of the tile instead.  The weights are >= 0, so a
// sum <= sum_limit bounds every weight by it, and fp32 sums and fp16/bf16
// operands hold such weights with the same relative precision as values
// <= 1.  Only when some lane's sum exceeds it (or is NaN) does the wave take
// the tile maximum, raise m, rescale O and the row sum, and form the weights
// again -- rarely: a wave's first tile sets m from the tile itself
// (fwd_first_weights).
//
// What the limit trades is how often a row's largest weights are exact: a
// tile that raises m gives its largest weight exactly 1, as the reference's
// per-block running maximum gives every block's (triton/varlen_attention.py
// :137-142), while weights under a lagging m sit anywhere up to the limit and
// carry their operand rounding into O.  fp16 rounds finely enough for 2^8.
// bf16 rounds 8x coarser: with 2^8 its O departed from the fp64 oracle by up
// to 2.2x what the reference kernels' own bf16 rounding gives on the same
// inputs at q, k ~ N(0, 4) (a CPU emulation of both over 6 seeds x 3
// head_dims); 2^3 keeps it within 1.5x, still rarely taking the rescale on
// unit-variance scores (the first tile's maximum is then ~2 sigma high).
template <typename T>
constexpr float sum_limit() {
  return std::is_same<T, bf16>::value ? 8.0f : 256.0f;
}

// ------------------------------------------------------- tile staging
// Direct-to-LDS tiles.  A ROWS x D tile of one head is copied from HBM into
// an unpadded row-major LDS tile by buffer loads with an LDS destination
// (no registers in between): each wave instruction fills one contiguous
// 1 KB window, lane l writing bytes [16 l, 16 l + 16), so the tile's layout is
// chosen by which global chunk each lane fetches.  The 16-byte chunk c of row
// r is stored at chunk position c ^ swz(r).
//
// gfx950's LDS serves 256 bytes (64 banks x 4 B) per pass; a 16-byte row read
// (ds_read_b128) is served 16 lanes per pass, here 16 consecutive rows at one
// logical chunk, and a transposed read (ds_read_b64_tr_b16) 32 lanes per
// pass, here 4 consecutive rows x 64 contiguous bytes.  swz makes both
// conflict-free (measured on MI355X: ~215 B/clk/CU for either read, against
// ~134 with a pattern that repeats every 8 rows):
//  * D = 64 (128-byte rows, two rows per 256 bytes): over 16 consecutive
//    rows, swz is a bijection onto 0..7 on the even and on the odd rows;
//    rows 4k and 4k+2 (and 4k+1, 4k+3) differ in bit 2, so their 64-byte
//    chunk groups are disjoint.
//  * D = 128 (256-byte rows): swz is a bijection onto 0..15 over 16 rows,
//    and swz >> 2 differs over 4 consecutive rows.
//  * D = 32 (64-byte rows, four per 256 bytes): rows r, r+4, r+8, r+12 take
//    distinct values; a transposed read covers whole rows.
// swz repeats every 16 rows, so tile offsets that are multiples of 16 rows
// keep the same lane offsets.  The buffer descriptor covers only the
// sequence's valid rows: rows past it are written as zeros by the hardware.
template <int D>
__device__ __forceinline__ int swz(int row) {
  return D >= 128 ? 4 * (row & 3) + ((row >> 2) & 3)
       : D >= 64  ? 4 * ((row >> 1) & 1) + ((row >> 2) & 3)
                  : (row >> 2) & 3;
}

template <typename T, int D, int ROWS>
struct DmaTile {
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int RPI = 1024 / (D * 2);        // rows per wave instruction
  static constexpr int INSTR = ROWS * D * 2 / 1024; // wave instructions per tile
  static_assert(INSTR % 4 == 0, "tile must split evenly over the 4 waves");
  static constexpr int PER_WAVE = INSTR / 4;
  uint32_t voff[PER_WAVE];

  // Chunks past the row's `dcols` columns (head_dim 16 in the 32-column
  // kernels) get an offset past every buffer's record count: the hardware
  // returns zeros for them, as for rows past the sequence.
  __device__ __forceinline__ void init(int64_t row_stride, int wave, int lane, int dcols) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int q = i * 4 + wave;
      const int r = q * RPI + lane / CPR;
      const int c = (lane % CPR) ^ swz<D>(r);
      voff[i] = col_live<D>(8 * c, dcols)
                    ? (uint32_t)(((int64_t)r * row_stride + c * 8) * (int64_t)sizeof(T))
                    : 0xFFFFFFF0u;
    }
  }
  // rows [row0, row0 + ROWS) of a sequence starting at `base` into `lds`
  // (ROWS * D elements); rows >= limit become zeros.
  __device__ __forceinline__ void load(T* lds, const T* __restrict__ base, int64_t row_stride,
                                       int row0, int limit, int wave) const {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS address-space cast exists only on the device side
    const int valid = min(ROWS, limit - row0);
    const uint32_t bytes = valid > 0 ? (uint32_t)((int64_t)valid * row_stride * (int64_t)sizeof(T)) : 0u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + (int64_t)row0 * row_stride, bytes);
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int q = i * 4 + wave;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(lds + q * 512), 16, voff[i], 0, 0, 0);
    }
#else
    (void)lds, (void)base, (void)row_stride, (void)row0, (void)limit, (void)wave;
#endif
  }
};

// Element offset, inside a swizzled tile, of this lane's row-read fragment
// (row `row`, logical chunk `c`).
template <int D>
__device__ __forceinline__ int swz_off(int row, int c) {
  return row * D + ((c ^ swz<D>(row)) << 3);
}
// This lane's transposed-read offsets for column block dt (32 columns): the
// lane addresses row 4g + (lr%16)/4 (.x) and 8 rows further (.y), column
// 32dt + 16(lr/16) + 4(lr%4) (see lds_frag_tr).
template <int D>
__device__ __forceinline__ int2 swz_tr_off(int lr, int g, int dt) {
  const int c = 4 * dt + 2 * (lr >> 4) + ((lr & 3) >> 1);
  int o[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int r = 4 * g + ((lr & 15) >> 2) + 8 * half;
    o[half] = r * D + ((c ^ swz<D>(r)) << 3) + 4 * (lr & 1);
  }
  return make_int2(o[0], o[1]);
}

// Reductions across the two 32-lane halves of a wave: v_permlane32_swap
// exchanges the upper 32 lanes of its first register with the lower 32 lanes
// of its second, so starting from two copies of x every lane ends up holding
// x[l % 32] and x[32 + l % 32] (no LDS round trip).  Emitted directly: the
// compiler's builtin folds the two results into one when both inputs are the
// same value.  The s_nop covers the VALU-write -> permlane read hazard.
__device__ __forceinline__ void half_pair(float x, float& a, float& b) {
  float lo = x, hi = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
  a = lo;
  b = hi;
}
__device__ __forceinline__ float halves_sum(float x) {
  float a, b;
  half_pair(x, a, b);
  return a + b;
}

// bf16 forward: O is normalised by the sum of the weights as rounded into the
// P operand, while the LSE keeps the sum of the unrounded weights (as the
// reference's l, triton/varlen_attention.py:138).  The weights here are taken
// against a reference maximum that may lag the row's true maximum (by up to
// sum_limit), so a row's dominant weight can be an arbitrary value above 1
// whose bf16 rounding (2^-9 relative) would otherwise pass straight into O;
// the reference's dominant weight is exp(0) = 1, exact.  Dividing by the
// operand sum makes O a convex combination of V rows with the rounded
// weights, in which a lone dominant weight's rounding cancels.  (fp16 rounds
// 8x finer; its budget holds without the second sum.)  Cost: 8 v_dot2 per
// tile.
template <typename T>
constexpr bool fwd_operand_sum() {
  return std::is_same<T, bf16>::value;
}
// acc + the sum of the 16 bf16 weights packed in two MFMA operands.
template <typename X8>
__device__ __forceinline__ float operand_sum(const X8& a, const X8& b, float acc) {
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
  const uint4 ua = __builtin_bit_cast(uint4, a), ub = __builtin_bit_cast(uint4, b);
  const uint32_t w[8] = {ua.x, ua.y, ua.z, ua.w, ub.x, ub.y, ub.z, ub.w};
  float x = acc, y = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    x = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[i]), one, x, false);
    y = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[i + 1]), one, y, false);
  }
  return x + y;
}

// Running max starts finite: the first tile always rescales (by exp2 of a
// huge negative number, i.e. 0), and no -inf special case is needed.
constexpr float kMaxInit = -1e30f;

// Per-wave state of the forward loop over 64-key blocks.  The workgroup's
// 4 waves hold the item's 128 queries (32 per wave) and share the K/V tiles.
template <typename T, int D>
struct FwdState {
  typedef typename VecT<T>::x8 x8;
  x8 qf[D / 16];            // this lane's query row, MFMA B fragments
  int koff[D / 16];         // swizzled K row-read offsets
  int2 voffs[D / 32];       // swizzled V transposed-read offsets
  f32x16 oacc[D / 32];      // O^T accumulators
  float m_run, l_run;       // reference max (raw scores) and row sum (this lane's keys)
  float l_op;               // bf16: row sum of the weights as rounded into the P operand
  float neg_mb;             // -m_run * scale_log2
  DmaTile<T, D, kBN> dK, dV;
  const T* kh;
  const T* vh;
  int64_t krow, vrow;
  int L, nkb, kend_wave, qw0, wave, lr, g;
  float scale_log2;
};

// v_max3_f32 written out: for fmaxf the compiler first canonicalises every
// operand it cannot prove is not a signalling NaN (each MFMA result), one
// extra instruction each.  Scores are MFMA results or -inf, never signalling.
// The compiler cannot see inside the asm: it inserts no wait states before
// it, so its operands must never come straight from an MFMA (whose results a
// VALU instruction may read only after wait states the compiler adds before
// instructions it can see).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Sum of a lane's 16 unrounded weights of a tile, in fp32 (two chains).
__device__ __forceinline__ float tile_sum(const f32x16& p) {
  float x = p[0], y = p[1];
#pragma unroll
  for (int i = 2; i < 16; i += 2) {
    x += p[i];
    y += p[i + 1];
  }
  return x + y;
}

// Maximum of a 32-key score tile for this lane's query (both wave halves).
__device__ __forceinline__ float tile_max(const f32x16& s) {
  float ma = max3f(s[0], s[1], s[2]);
  float mc = max3f(s[3], s[4], s[5]);
  ma = max3f(ma, s[6], s[7]);
  mc = max3f(mc, s[8], s[9]);
  ma = max3f(ma, s[10], s[11]);
  mc = max3f(mc, s[12], s[13]);
  ma = max3f(ma, s[14], s[15]);
  float lo, hi;
  half_pair(max3f(ma, mc, mc), lo, hi);
  return max3f(lo, hi, hi);
}

// tile_max for scores fresh from the MFMAs: the same maximum (max is exact in
// any order) from maxima the compiler emits itself, so it places the MFMA
// result wait before the first of them.
__device__ __forceinline__ float tile_max_fresh(const f32x16& s) {
  float ma = fmaxf(s[0], s[1]), mb = fmaxf(s[2], s[3]);
#pragma unroll
  for (int i = 4; i < 16; i += 2) {
    ma = fmaxf(ma, s[i]);
    mb = fmaxf(mb, s[i + 1]);
  }
  float lo, hi;
  half_pair(fmaxf(ma, mb), lo, hi);
  return fmaxf(lo, hi);
}

// Mask (to -inf) the keys of the 32-key score tile at tbase that this lane's
// query may not see: above the diagonal (causal) or past the sequence.
template <typename T, int D, bool CAUSAL>
__device__ __forceinline__ void fwd_mask(const FwdState<T, D>& st, f32x16& s, int tbase) {
  if (CAUSAL) {
    if (tbase == st.qw0) mask_rows_above<false>(s, st.lr - 4 * st.g);  // the diagonal tile
  } else if (tbase + 32 > st.L) {
    mask_rows_above<false>(s, st.L - 1 - tbase - 4 * st.g);
  }
}

// Weights p = 2^(s*c - m*c) of a score tile and this lane's fp32 sum of them.
template <typename T, int D>
__device__ __forceinline__ float fwd_weights(const FwdState<T, D>& st, const f32x16& s, f32x16& p) {
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(s[i], st.scale_log2, st.neg_mb));
  return tile_sum(p);
}

// The rare path: some lane's weights summed past sum_limit (or to NaN).
// Raise the reference maximum to the tile's, rescale O and the row sum, and
// form the tile's weights again.
template <typename T, int D>
__device__ __forceinline__ void fwd_rescale(FwdState<T, D>& st, const f32x16& s, f32x16& p, float& ls) {
  const float m_new = fmaxf(st.m_run, tile_max(s));
  const float alpha = fast_exp2((st.m_run - m_new) * st.scale_log2);
  st.l_run *= alpha;
  if constexpr (fwd_operand_sum<T>()) st.l_op *= alpha;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) st.oacc[dt][i] *= alpha;
  st.m_run = m_new;
  st.neg_mb = -m_new * st.scale_log2;
  ls = fwd_weights(st, s, p);
}

// A wave's first tile: O and the row sum are still zero, so the reference
// maximum comes from the tile directly -- the value fwd_rescale reaches after
// the sum check against the initial -1e30 fails, without forming the
// weights twice or rescaling a zero O -- and the weights are formed once.
template <typename T, int D>
__device__ __forceinline__ float fwd_first_weights(FwdState<T, D>& st, const f32x16& s, f32x16& p) {
  st.m_run = fmaxf(st.m_run, tile_max_fresh(s));
  st.neg_mb = -st.m_run * st.scale_log2;
  return fwd_weights(st, s, p);
}

// O^T += V^T P^T for one tile: the weights rounded to T as the B operand,
// V^T read transposed from the tile's 32 rows at sVt.
template <typename T, int D>
__device__ __forceinline__ void fwd_pv(FwdState<T, D>& st, const f32x16& p, const T* sVt) {
  typedef typename VecT<T>::x8 x8;
  const x8 pf0 = pack_frag<T>(p, 0), pf1 = pack_frag<T>(p, 8);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) st.oacc[dt] = mfma32(lds_frag_tr(sVt, st.voffs[dt]), pf0, st.oacc[dt]);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
    st.oacc[dt] = mfma32(lds_frag_tr(sVt + 16 * D, st.voffs[dt]), pf1, st.oacc[dt]);
  if constexpr (fwd_operand_sum<T>()) st.l_op = operand_sum(pf0, pf1, st.l_op);
}

// One 64-key block kb: start the DMA of block kb + 1 into `nxt`, then compute
// on `cur` (K tile, then V tile).  FULL: every live wave has both 32-key
// tiles of the block and none needs a mask (blocks before the item's first
// query, or before a partial last block), so the block runs without the
// per-tile checks.  Both score tiles are issued before the first tile's
// softmax, whose VALU work then overlaps the second tile's MFMAs.  The
// restrict qualifiers tell the compiler the two buffers are disjoint, so it
// keeps the DMA in flight across the reads.
template <typename T, int D, bool CAUSAL, bool FULL, bool FIRST = false>
__device__ __forceinline__ void fwd_block(FwdState<T, D>& st, int kb, const T* __restrict__ cur,
                                          T* __restrict__ nxt) {
  constexpr int TILE = kBN * D;
  const T* sK = cur;
  const T* sV = cur + TILE;
  if (kb + 1 < st.nkb) {
    st.dK.load(nxt, st.kh, st.krow, (kb + 1) * kBN, st.L, st.wave);
    st.dV.load(nxt + TILE, st.vh, st.vrow, (kb + 1) * kBN, st.L, st.wave);
  }
  const int kbase = kb * kBN;
  // (waves whose rows all lie past the sequence have kend_wave = 0: no tiles)
  const int nt = FULL ? (st.kend_wave > 0 ? 2 : 0)
                      : kbase < st.kend_wave ? (kbase + 32 < st.kend_wave ? 2 : 1) : 0;
  if (nt > 0) {
    f32x16 s0 = zero16(), s1, p0, p1;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) s0 = mfma32(lds_frag16(sK + st.koff[s]), st.qf[s], s0);
    if (FULL) {
      s1 = zero16();
#pragma unroll
      for (int s = 0; s < D / 16; ++s) s1 = mfma32(lds_frag16(sK + 32 * D + st.koff[s]), st.qf[s], s1);
      float ls0;
      if (FIRST) {
        ls0 = fwd_first_weights(st, s0, p0);
      } else {
        ls0 = fwd_weights(st, s0, p0);
        if (__any(!(ls0 <= sum_limit<T>()))) fwd_rescale(st, s0, p0, ls0);
      }
      st.l_run += ls0;
      fwd_pv(st, p0, sV);
      float ls1 = fwd_weights(st, s1, p1);
      if (__any(!(ls1 <= sum_limit<T>()))) fwd_rescale(st, s1, p1, ls1);
      st.l_run += ls1;
      fwd_pv(st, p1, sV + 32 * D);
    } else {
      if (nt > 1) {
        s1 = zero16();
#pragma unroll
        for (int s = 0; s < D / 16; ++s) s1 = mfma32(lds_frag16(sK + 32 * D + st.koff[s]), st.qf[s], s1);
      }
      fwd_mask<T, D, CAUSAL>(st, s0, kbase);
      float ls0;
      if (FIRST) {
        ls0 = fwd_first_weights(st, s0, p0);
      } else {
        ls0 = fwd_weights(st, s0, p0);
        if (__any(!(ls0 <= sum_limit<T>()))) fwd_rescale(st, s0, p0, ls0);
      }
      st.l_run += ls0;
      fwd_pv(st, p0, sV);
      if (nt > 1) {
        fwd_mask<T, D, CAUSAL>(st, s1, kbase + 32);
        float ls1 = fwd_weights(st, s1, p1);
        if (__any(!(ls1 <= sum_limit<T>()))) fwd_rescale(st, s1, p1, ls1);
        st.l_run += ls1;
        fwd_pv(st, p1, sV + 32 * D);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's share of block kb + 1 has landed
  __syncthreads();
}

// Waves per SIMD the forward is compiled for: four (128 registers) for the
// causal form up to head_dim 64, which fits them without spills; two
// otherwise (the compiler then takes what it needs: ~135 registers, three
// waves, for the non-causal form at 64).
template <int D, bool CAUSAL>
constexpr int attn_fwd_waves() {
  return D >= 256 ? 1 : CAUSAL && D <= 64 ? 4 : 2;
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, (attn_fwd_waves<D, CAUSAL>())) void attn_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ o,
    float* __restrict__ lse, ItemSource src, int tmax, int head_major, int heads, int group,
    Strides sq, Strides sk, Strides sv, Strides so, float scale, float scale_log2, int total,
    int dcols) {
  constexpr int TILE = kBN * D;  // elements per K or V tile
  constexpr int BUF = 2 * TILE;  // one buffer: K tile then V tile
  __shared__ __align__(16) T smem[2 * BUF];
  static_assert(4 * stage_elems<D>() <= 2 * BUF, "O staging must fit in the tile buffers");

  const ItemView iv = item_view<true>(src, tmax);
  if (iv.failed) {
    publish_header(src, iv, CAUSAL ? 1 : 0);
    poison_rows(o, so, total, heads, dcols);
    poison_stats(lse, total, heads);
    return;
  }
  int item, h;
  if (!map_block(heads, tmax, head_major, group, D * (int)sizeof(T) < 128 && group == 1, item, h) ||
      item >= iv.count) {
    publish_header(src, iv, CAUSAL ? 1 : 0);
    return;
  }
  const int hk = h / group;  // K/V head of this query head
  const int4 it = item_at<true>(src, iv, CAUSAL, item);
  if (it.w == 0) return;
  const int start = it.z, L = it.w, q0 = it.y * kBM;
  FwdState<T, D> st;
  st.wave = wave_id();
  const int lane = threadIdx.x & (kWave - 1);
  st.g = lane >> 5;
  st.lr = lane & 31;
  st.qw0 = q0 + 32 * st.wave;
  const int my_q = st.qw0 + st.lr;
  const bool wave_live = st.qw0 < L;
  st.L = L;
  st.kh = k + (int64_t)start * sk.row + (int64_t)hk * sk.head;
  st.vh = v + (int64_t)start * sv.row + (int64_t)hk * sv.head;
  st.krow = sk.row;
  st.vrow = sv.row;
  const int kend_wg = CAUSAL ? min(L, q0 + kBM) : L;
  st.nkb = (kend_wg + kBN - 1) / kBN;
  st.kend_wave = wave_live ? (CAUSAL ? min(L, st.qw0 + 32) : L) : 0;

  T* bufA = smem;
  T* bufB = smem + BUF;
  st.dK.init(sk.row, st.wave, lane, dcols);
  st.dV.init(sv.row, st.wave, lane, dcols);
  st.dK.load(bufA, st.kh, sk.row, 0, L, st.wave);
  st.dV.load(bufA + TILE, st.vh, sv.row, 0, L, st.wave);

  {  // rows past L read row L-1: their results are never stored
    const T* qrow = q + (int64_t)(start + min(my_q, L - 1)) * sq.row + (int64_t)h * sq.head;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) st.qf[s] = gmem_frag16_cols<D>(qrow, 16 * s + 8 * st.g, dcols);
    // Materialize the fragments before the barrier (the compiler would sink
    // the loads into the block loop, whose counter waits would then also wait
    // out the freshly issued DMA).
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" : "+v"(st.qf[s]));
  }
#pragma unroll
  for (int s = 0; s < D / 16; ++s) st.koff[s] = swz_off<D>(st.lr, 2 * s + st.g);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) st.voffs[dt] = swz_tr_off<D>(st.lr, st.g, dt);
  st.scale_log2 = scale_log2;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) st.oacc[dt] = zero16();
  st.m_run = kMaxInit;
  st.l_run = 0.f;
  st.l_op = 0.f;
  st.neg_mb = -kMaxInit * scale_log2;

  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Blocks [0, nfull) need no mask and give every wave two tiles: those
  // before the item's first query (causal) or before a partial last block.
  // Unrolled by two so that each call sees its buffers at fixed positions.
  const int nfull = CAUSAL ? min(q0, L) / kBN : L / kBN;
  // Block 0 (there is always one) holds every live wave's first tile.
  if (nfull >= 1)
    fwd_block<T, D, CAUSAL, true, true>(st, 0, bufA, bufB);
  else
    fwd_block<T, D, CAUSAL, false, true>(st, 0, bufA, bufB);
  {
    T* t = bufA;
    bufA = bufB;
    bufB = t;
  }
  int kb = 1;
  for (; kb + 1 < nfull; kb += 2) {
    fwd_block<T, D, CAUSAL, true>(st, kb, bufA, bufB);
    fwd_block<T, D, CAUSAL, true>(st, kb + 1, bufB, bufA);
  }
  if (kb < nfull) {  // odd count: the last full block, then swap the buffers
    fwd_block<T, D, CAUSAL, true>(st, kb, bufA, bufB);
    T* t = bufA;
    bufA = bufB;
    bufB = t;
    ++kb;
  }
  for (; kb < st.nkb; kb += 2) {
    fwd_block<T, D, CAUSAL, false>(st, kb, bufA, bufB);
    if (kb + 1 < st.nkb) fwd_block<T, D, CAUSAL, false>(st, kb + 1, bufB, bufA);
  }
  if (wave_live) {  // the last block's barrier freed the tile buffers: stage O there
    const float l_tot = halves_sum(st.l_run);
    const float inv_l = 1.0f / (fwd_operand_sum<T>() ? halves_sum(st.l_op) : l_tot);
    store_rows_staged<T, D>(smem + st.wave * stage_elems<D>(), st.oacc, inv_l,
                            o + (int64_t)(start + st.qw0) * so.row + (int64_t)h * so.head, so.row,
                            min(32, L - st.qw0), dcols, st.lr, st.g, lane);
    if (st.g == 0 && my_q < L)
      lse[(int64_t)(start + my_q) * heads + h] = st.m_run * scale + logf(l_tot);
  }
  // last: a store issued earlier would hold up the prologue's counter waits
  publish_header(src, iv, CAUSAL ? 1 : 0);
  if (h == 0) publish_item(src, item, it);
}

// -------------------------------------------------- backward: dQ and Delta
// Per item: 128 queries (32 per wave) loop over 64-key blocks.
//   S^T = K Q^T, dP^T = V dO^T (Q, dO operands in registers; K, V from LDS)
//   P^T = exp(S^T - LSE), dS^T = P^T (dP^T - Delta)
//   dQ^T += K^T dS^T (K^T read transposed from the K tile; dS^T in registers)
// K and V tiles arrive by DMA into swizzled LDS tiles, as in the forward.
// Delta = rowsum(O * dO) is computed here from the stored O and written out
// for the dK/dV pass.  Keys past L hold zeros in K and V, so their dS^T
// multiplies a zero row of K^T: no length mask is needed.
template <typename T, int D>
struct DqState {
  typedef typename VecT<T>::x8 x8;
  x8 qf[D / 16], df[D / 16];  // this lane's Q and dO rows, MFMA B fragments
  int koff[D / 16];           // swizzled row-read offsets (K and V tiles)
  int2 ktr[D / 32];           // swizzled transposed-read offsets (K^T)
  f32x16 dqacc[D / 32];       // dQ^T accumulators
  f32x16 neg_delta;           // dP^T accumulates onto -Delta: it comes out as dP^T - Delta
  float lse2;                 // this lane's LSE * log2(e)
  DmaTile<T, D, kBN> dK, dV;
  const T* kh;
  const T* vh;
  int64_t krow, vrow;
  int L, nkb, kend_wave, qw0, wave, lr, g;
  float scale_log2;
};

// Number of K/V tile buffers of the dQ pass: three (the DMA runs two blocks
// ahead) where the third costs no occupancy, two at D = 128.
template <int D>
constexpr int dq_nbuf() {
  return D <= 64 ? 3 : 2;
}

// One 64-key block kb on `cur` while the DMA of block kb + AHEAD fills `nxt`
// (see fwd_block for the buffer discipline).  Ends with a barrier once block
// kb + 1 has landed; block kb + 2's DMA may stay in flight across it.
template <typename T, int D, bool CAUSAL, int AHEAD>
__device__ __forceinline__ void dq_block(DqState<T, D>& st, int kb, const T* __restrict__ cur,
                                         T* __restrict__ nxt) {
  typedef typename VecT<T>::x8 x8;
  constexpr int TILE = kBN * D;
  constexpr int NL = 2 * DmaTile<T, D, kBN>::PER_WAVE;  // DMA instructions per block
  const T* sK = cur;
  const T* sV = cur + TILE;
  if (kb + AHEAD < st.nkb) {
    st.dK.load(nxt, st.kh, st.krow, (kb + AHEAD) * kBN, st.L, st.wave);
    st.dV.load(nxt + TILE, st.vh, st.vrow, (kb + AHEAD) * kBN, st.L, st.wave);
  }
  const int kbase = kb * kBN;
  const int nt = kbase < st.kend_wave ? (kbase + 32 < st.kend_wave ? 2 : 1) : 0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (t >= nt) break;
    f32x16 sacc = zero16(), pacc = st.neg_delta;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      sacc = mfma32(lds_frag16(sK + 32 * t * D + st.koff[s]), st.qf[s], sacc);
      pacc = mfma32(lds_frag16(sV + 32 * t * D + st.koff[s]), st.df[s], pacc);
    }
    if (CAUSAL && kbase + 32 * t == st.qw0) mask_rows_above(sacc, st.lr - 4 * st.g);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = fast_exp2(fmaf(sacc[i], st.scale_log2, -st.lse2));
      sacc[i] = p * pacc[i];  // dS^T = P^T (dP^T - Delta)
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const x8 sf = pack_frag<T>(sacc, 8 * hh);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
        st.dqacc[dt] = mfma32(lds_frag_tr(sK + (32 * t + 16 * hh) * D, st.ktr[dt]), sf,
                              st.dqacc[dt]);
    }
  }
  // No other vector-memory operations run in the loop, so at most NL are
  // younger than this wave's share of block kb + 1: block kb + 2's.
  if (AHEAD == 2 && kb + 2 < st.nkb)
    barrier_vm<NL>();
  else
    barrier_vm<0>();
}

// The dQ block loop over tile buffers A, B (and C): `issue` starts this
// wave's row loads, then blocks 0 (and 1) are staged, `setup` consumes the
// rows while the tiles fly, then the loop runs.  The row loads go first:
// loads retire in order, so rows requested after 32 KB of tile DMA would
// wait for all of it (microseconds under load).  Every DMA and tile read sits
// in this one function, so the compiler's alias scopes tell each pending DMA
// apart from the reads of the other buffers (a DMA pending across two calls
// of dq_block would otherwise make it wait for the DMA before every read).
template <typename T, int D, bool CAUSAL, typename Issue, typename Setup>
__device__ __forceinline__ void dq_run(DqState<T, D>& st, T* __restrict__ A, T* __restrict__ B,
                                       T* __restrict__ C, Issue issue, Setup setup) {
  constexpr int TILE = kBN * D;
  constexpr int NL = 2 * DmaTile<T, D, kBN>::PER_WAVE;
  constexpr bool three = dq_nbuf<D>() == 3;
  issue();
  st.dK.load(A, st.kh, st.krow, 0, st.L, st.wave);
  st.dV.load(A + TILE, st.vh, st.vrow, 0, st.L, st.wave);
  if (three) {  // block 1 even when unused (nkb == 1 only for L <= 64): a fixed count
    st.dK.load(B, st.kh, st.krow, kBN, st.L, st.wave);
    st.dV.load(B + TILE, st.vh, st.vrow, kBN, st.L, st.wave);
  }
  setup();
  // Block 0 has landed once at most NL operations are younger than it (block
  // 1's, or fewer when setup's own stores are among them: waiting longer is
  // only conservative).
  if (three)
    barrier_vm<NL>();
  else
    barrier_vm<0>();
  auto block = [&](int kb, const T* __restrict__ cur, T* __restrict__ nxt) {
    dq_block<T, D, CAUSAL, three ? 2 : 1>(st, kb, cur, nxt);
  };
  if constexpr (three) {
    for (int kb = 0; kb < st.nkb; kb += 3) {
      block(kb, A, C);
      if (kb + 1 >= st.nkb) break;
      block(kb + 1, B, A);
      if (kb + 2 >= st.nkb) break;
      block(kb + 2, C, B);
    }
  } else {
    for (int kb = 0; kb < st.nkb; kb += 2) {
      block(kb, A, B);
      if (kb + 1 >= st.nkb) break;
      block(kb + 1, B, A);
    }
  }
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, D >= 256 ? 1 : 2) void attn_bwd_dq_kernel(
    const T* __restrict__ dout, const T* __restrict__ q, const T* __restrict__ k,
    const T* __restrict__ v, const T* __restrict__ o, const float* __restrict__ lse,
    float* __restrict__ delta, T* __restrict__ dq, ItemSource src, int tmax, int head_major,
    int heads, int group, Strides sdo,
    Strides sq, Strides sk, Strides sv, Strides so, Strides sdq, float scale, float scale_log2,
    int total, int dcols) {
  typedef typename VecT<T>::x8 x8;
  constexpr int TILE = kBN * D;
  constexpr int BUF = 2 * TILE;  // K tile then V tile
  __shared__ __align__(16) T smem[dq_nbuf<D>() * BUF];
  static_assert(4 * stage_elems<D>() <= dq_nbuf<D>() * BUF, "dQ staging must fit in the tile buffers");

  const ItemView iv = item_view<false>(src, tmax);
  if (iv.failed) {
    poison_rows(dq, sdq, total, heads, dcols);
    poison_stats(delta, total, heads);
    return;
  }
  int item, h;
  if (!map_block(heads, tmax, head_major, group, D * (int)sizeof(T) < 128 && group == 1, item, h) ||
      item >= iv.count)
    return;
  const int hk = h / group;  // K/V head of this query head
  const int4 it = item_at<false>(src, iv, CAUSAL, item);
  if (it.w == 0) return;
  const int start = it.z, L = it.w, q0 = it.y * kBM;
  DqState<T, D> st;
  st.wave = wave_id();
  const int lane = threadIdx.x & (kWave - 1);
  st.g = lane >> 5;
  st.lr = lane & 31;
  st.qw0 = q0 + 32 * st.wave;
  const int my_q = st.qw0 + st.lr;
  const bool wave_live = st.qw0 < L;
  st.L = L;
  st.kh = k + (int64_t)start * sk.row + (int64_t)hk * sk.head;
  st.vh = v + (int64_t)start * sv.row + (int64_t)hk * sv.head;
  st.krow = sk.row;
  st.vrow = sv.row;
  const int kend_wg = CAUSAL ? min(L, q0 + kBM) : L;
  st.nkb = (kend_wg + kBN - 1) / kBN;
  st.kend_wave = wave_live ? (CAUSAL ? min(L, st.qw0 + 32) : L) : 0;

  st.dK.init(sk.row, st.wave, lane, dcols);
  st.dV.init(sv.row, st.wave, lane, dcols);

  // This wave's query rows (issued before the first K/V blocks), then Delta
  // and the fragment offsets, set up while those blocks are in flight.  Rows
  // past L read row L-1: their results are never stored.
  x8 of[D / 16];
  float lse_raw;
  auto issue = [&] {
    const int64_t tok = start + min(my_q, L - 1);
    const T* qrow = q + tok * sq.row + (int64_t)h * sq.head;
    const T* drow = dout + tok * sdo.row + (int64_t)h * sdo.head;
    const T* orow = o + tok * so.row + (int64_t)h * so.head;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      st.qf[s] = gmem_frag16_cols<D>(qrow, 16 * s + 8 * st.g, dcols);
      st.df[s] = gmem_frag16_cols<D>(drow, 16 * s + 8 * st.g, dcols);
      of[s] = gmem_frag16_cols<D>(orow, 16 * s + 8 * st.g, dcols);
    }
    lse_raw = lse[tok * heads + h];
  };
  auto setup = [&] {
    float dl = 0.f;
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) dl += (float)of[s][j] * (float)st.df[s][j];
    st.lse2 = lse_raw * kLog2e;
    // Materialize the fragments before the barrier (see the forward).
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" : "+v"(st.qf[s]), "+v"(st.df[s]));
    dl = halves_sum(dl);
    if (my_q < L && st.g == 0) delta[(int64_t)(start + my_q) * heads + h] = dl;
#pragma unroll
    for (int i = 0; i < 16; ++i) st.neg_delta[i] = -dl;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) st.koff[s] = swz_off<D>(st.lr, 2 * s + st.g);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) st.ktr[dt] = swz_tr_off<D>(st.lr, st.g, dt);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) st.dqacc[dt] = zero16();
    st.scale_log2 = scale_log2;
  };
  dq_run<T, D, CAUSAL>(st, smem, smem + BUF, dq_nbuf<D>() == 3 ? smem + 2 * BUF : nullptr, issue,
                       setup);
  if (wave_live)  // the last block's barrier freed the tile buffers: stage dQ there
    store_rows_staged<T, D>(smem + st.wave * stage_elems<D>(), st.dqacc, scale,
                            dq + (int64_t)(start + st.qw0) * sdq.row + (int64_t)h * sdq.head,
                            sdq.row, min(32, L - st.qw0), dcols, st.lr, st.g, lane);
}

// ---------------------------------------------------- backward: dK and dV
// Per item: 128 keys (32 per wave) loop over blocks of BQ queries.
//   S = Q K^T, dP = dO V^T (V operand in registers, K in registers or, at
//   D = 128, in LDS; Q, dO from LDS)
//   P = exp(S - LSE), dS = P (dP - Delta)
//   dV^T += dO^T P, dK^T += Q^T dS (dO^T, Q^T read transposed from the LDS
//   tiles; P, dS in registers)
// Q and dO tiles arrive by DMA into swizzled LDS tiles, as in the forward;
// each block's LSE and -Delta rows are staged beside them.  Queries past L
// hold zeros in Q and dO (and LSE = Delta = 0), so they add nothing to dK or
// dV: no length mask is needed.  D = 128 runs two waves per SIMD (256
// registers each); with K, V, dK and dV of its keys all in registers a few
// values spilled to scratch, and reloading them waited out the next block's
// in-flight DMA.  With each wave's K rows staged once in LDS instead (32
// registers fewer, 64 KB of LDS per workgroup: still two per CU) nothing
// spills: config 5's dK/dV pass 7.4 ms against 8.7 ms.  At D = 64 the same
// move changes nothing measurable, so K stays in registers there.
template <int D>
constexpr int dkv_bq() {
  return D >= 128 ? 32 : 64;
}
// Where the score MFMA takes its K operand from: registers (K held for the
// whole item), or, at D = 128, the wave's 32 K rows staged once in LDS.
template <int D>
constexpr bool dkv_k_lds() {
  return D >= 128;
}

template <typename T, int D>
struct DkvState {
  typedef typename VecT<T>::x8 x8;
  static constexpr int BQ = dkv_bq<D>();
  x8 kf[D / 16], vf[D / 16];      // this lane's K and V rows, MFMA B fragments
  f32x16 dkacc[D / 32], dvacc[D / 32];
  int qoff[D / 16];               // swizzled row-read offsets (Q and dO tiles)
  int2 qtr[D / 32];               // swizzled transposed-read offsets
  DmaTile<T, D, BQ> dQ, dO;
  const T* qh;
  const T* dh;
  const float* lse_h;             // lse / delta of this head at the sequence start
  const float* delta_h;
  int64_t qrow, drow;
  int heads, L, qbeg, nqb, kw0, wave, lr, g;
  int qfirst, qstep;              // query row of block 0 and the step between blocks (+-BQ)
  bool wave_live;
  float pl, pd;                   // staged LSE and Delta of one query row
  float scale_log2;
};

// LSE and Delta of query row `qq` into registers (threads < BQ own one row
// each); they are converted only when stored, so the loads stay in flight.
template <typename T, int D>
__device__ __forceinline__ void dkv_load_rows(DkvState<T, D>& st, int qq) {
  const int64_t idx = (int64_t)min(qq, st.L - 1) * st.heads;
  st.pl = qq < st.L ? st.lse_h[idx] : 0.f;
  st.pd = qq < st.L ? st.delta_h[idx] : 0.f;
}
__device__ __forceinline__ void dkv_store_rows(float* rows, int bq, float pl, float pd) {
  rows[threadIdx.x] = pl * kLog2e;
  rows[bq + threadIdx.x] = -pd;
}

// One block b of BQ queries (see fwd_block for the buffer discipline).
// `lcur` holds [LSE*log2(e) | -Delta] of the block's rows.
template <typename T, int D, bool CAUSAL>
__device__ __forceinline__ void dkv_block(DkvState<T, D>& st, int b, const T* __restrict__ cur,
                                          T* __restrict__ nxt, const float* __restrict__ lcur,
                                          const T* __restrict__ kl) {
  typedef typename VecT<T>::x8 x8;
  constexpr int BQ = DkvState<T, D>::BQ;
  constexpr int NQT = BQ / 32;
  constexpr int TILE = BQ * D;
  const T* sQ = cur;
  const T* sO = cur + TILE;
  const int qb = st.qfirst + b * st.qstep;
  if (b + 1 < st.nqb) {
    st.dQ.load(nxt, st.qh, st.qrow, qb + st.qstep, st.L, st.wave);
    st.dO.load(nxt + TILE, st.dh, st.drow, qb + st.qstep, st.L, st.wave);
  }
  if (st.wave_live) {
#pragma unroll
    for (int u = 0; u < NQT; ++u) {
      const int qt0 = qb + 32 * u;
      if (qt0 >= st.L) continue;
      if (CAUSAL && qt0 < st.kw0) continue;  // every query of the tile precedes every key
      // lane: key (column); element i: query qt0 + acc_row0(i) + 4g (row).
      // dP accumulates onto -Delta of its row, so it comes out as dP - Delta.
      f32x16 sacc = zero16(), pacc;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const float4 d4 = *reinterpret_cast<const float4*>(lcur + BQ + 32 * u + 8 * i4 + 4 * st.g);
        pacc[4 * i4 + 0] = d4.x;
        pacc[4 * i4 + 1] = d4.y;
        pacc[4 * i4 + 2] = d4.z;
        pacc[4 * i4 + 3] = d4.w;
      }
#pragma unroll
      for (int s = 0; s < D / 16; ++s) {
        x8 kfr;
        if constexpr (dkv_k_lds<D>())
          kfr = lds_frag16(kl + st.qoff[s]);
        else
          kfr = st.kf[s];
        sacc = mfma32(lds_frag16(sQ + 32 * u * D + st.qoff[s]), kfr, sacc);
        pacc = mfma32(lds_frag16(sO + 32 * u * D + st.qoff[s]), st.vf[s], pacc);
      }
      // diagonal tile: queries before the key contribute nothing (their
      // scores go to -inf, so P = 0 and dS = 0 * (dP - Delta) = 0)
      if (CAUSAL && qt0 == st.kw0) mask_rows_below(sacc, st.lr - 4 * st.g);
      f32x16 pv;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const float4 l4 = *reinterpret_cast<const float4*>(lcur + 32 * u + 8 * i4 + 4 * st.g);
        const float la[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * i4 + e;
          const float p = fast_exp2(fmaf(sacc[i], st.scale_log2, -la[e]));
          pv[i] = p;
          sacc[i] = p * pacc[i];  // dS = P (dP - Delta)
        }
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const x8 pf = pack_frag<T>(pv, 8 * hh);
        const x8 sf = pack_frag<T>(sacc, 8 * hh);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          st.dvacc[dt] = mfma32(lds_frag_tr(sO + (32 * u + 16 * hh) * D, st.qtr[dt]), pf,
                                st.dvacc[dt]);
          st.dkacc[dt] = mfma32(lds_frag_tr(sQ + (32 * u + 16 * hh) * D, st.qtr[dt]), sf,
                                st.dkacc[dt]);
        }
      }
    }
  }
}

// Block b with the row staging around it: the next block's LSE / Delta rows
// load during the block and land in `lnxt` before the closing barrier.
template <typename T, int D, bool CAUSAL>
__device__ __forceinline__ void dkv_step(DkvState<T, D>& st, int b, const T* cur, T* nxt,
                                         const float* lcur, float* lnxt, const T* kl) {
  constexpr int BQ = DkvState<T, D>::BQ;
  const bool more = b + 1 < st.nqb;
  if (more && threadIdx.x < BQ) dkv_load_rows(st, st.qfirst + (b + 1) * st.qstep + (int)threadIdx.x);
  dkv_block<T, D, CAUSAL>(st, b, cur, nxt, lcur, kl);
  if (more && threadIdx.x < BQ) dkv_store_rows(lnxt, BQ, st.pl, st.pd);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's share of block b + 1 has landed
  __syncthreads();
}

// Split-group epilogue: this part's fp32 dK / dV sums of the item's 128
// keys as rows [dK | dV][128][D] (the columns store_row_slice writes), for
// dkv_reduce_kernel to add up after the pass.
template <int D>
__device__ __forceinline__ void dkv_store_partial(const f32x16 (&dk)[D / 32],
                                                  const f32x16 (&dv)[D / 32],
                                                  float* __restrict__ rows, int key, int g) {
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int col = 32 * dt + 8 * qd + 4 * g;
      *reinterpret_cast<float4*>(rows + (int64_t)key * D + col) =
          make_float4(dk[dt][4 * qd], dk[dt][4 * qd + 1], dk[dt][4 * qd + 2], dk[dt][4 * qd + 3]);
      *reinterpret_cast<float4*>(rows + (int64_t)(kBM + key) * D + col) =
          make_float4(dv[dt][4 * qd], dv[dt][4 * qd + 1], dv[dt][4 * qd + 2], dv[dt][4 * qd + 3]);
    }
}

// Sum of the parts of one (item, K/V head) in part order (the result does not
// depend on which part ran first), scaled and rounded into dK / dV rows.  One
// workgroup per kRedRows keys of a slot, so the grid stays wide when there
// are few K/V heads.
constexpr int kRedRows = 16;
template <typename T, int D>
__global__ __launch_bounds__(256) void dkv_reduce_kernel(
    const float* __restrict__ partial, ItemSource src, int tmax, int causal, int kv_heads,
    int gsplit, T* __restrict__ dk, T* __restrict__ dv, Strides sdk, Strides sdv, float scale,
    int dcols) {
  constexpr int CHUNKS = kBM / kRedRows;
  const int slot = blockIdx.x / CHUNKS, chunk = blockIdx.x % CHUNKS;
  const int item = slot / kv_heads, hk = slot % kv_heads;
  const ItemView iv = item_view<false>(src, tmax);  // a failed schedule: the pass poisoned dk / dv
  if (item >= iv.count) return;
  const int4 it = item_at<false>(src, iv, causal != 0, item);
  if (it.w == 0) return;
  const int start = it.z, L = it.w;
  const int k0 = ((L + kBM - 1) / kBM - 1 - it.y) * kBM;
  constexpr int C4 = D / 4;
  const int64_t part_floats = 2 * kBM * D;
  const float* base = partial + (int64_t)slot * gsplit * part_floats;
  for (int idx = threadIdx.x; idx < kRedRows * C4; idx += blockDim.x) {
    const int r = chunk * kRedRows + idx / C4, c = 4 * (idx % C4);
    if (k0 + r >= L || !col_live<D>(c, dcols)) continue;
#pragma unroll
    for (int kind = 0; kind < 2; ++kind) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int p = 0; p < gsplit; ++p) {
        const float4 x = *reinterpret_cast<const float4*>(
            base + p * part_floats + (int64_t)(kind * kBM + r) * D + c);
        acc.x += x.x, acc.y += x.y, acc.z += x.z, acc.w += x.w;
      }
      const float mul = kind == 0 ? scale : 1.0f;
      const Strides sd = kind == 0 ? sdk : sdv;
      T* dst = (kind == 0 ? dk : dv) + (int64_t)(start + k0 + r) * sd.row + (int64_t)hk * sd.head + c;
      *reinterpret_cast<uint2*>(dst) =
          make_uint2(pack2<T>(acc.x * mul, acc.y * mul), pack2<T>(acc.z * mul, acc.w * mul));
    }
  }
}

// Waves per SIMD the dK/dV kernel is compiled for: three (168 registers)
// where that needs no spills -- head_dim 32, and the causal form at 64 --
// two otherwise.
template <int D, bool CAUSAL>
constexpr int dkv_waves() {
  return D >= 256 ? 1 : D <= 32 || (D == 64 && CAUSAL) ? 3 : 2;
}

template <typename T, int D, bool CAUSAL, bool SPLIT, bool REV>
__global__ __launch_bounds__(kThreads, (dkv_waves<D, CAUSAL>())) void attn_bwd_dkv_kernel(
    const T* __restrict__ dout, const T* __restrict__ q, const T* __restrict__ k,
    const T* __restrict__ v, const float* __restrict__ lse, const float* __restrict__ delta,
    T* __restrict__ dk, T* __restrict__ dv, ItemSource src, int tmax, int head_major,
    int kv_heads, int group,
    Strides sdo, Strides sq, Strides sk, Strides sv, Strides sdk, Strides sdv, float scale,
    float scale_log2, int gsplit, float* __restrict__ partial, int total, int dcols) {
  constexpr int BQ = dkv_bq<D>();
  constexpr int TILE = BQ * D;
  constexpr int BUF = 2 * TILE;  // Q tile then dO tile
  // Two [Q tile | dO tile] buffers, then two [LSE*log2(e) rows | -Delta rows]
  // buffers.  One LDS object: with several, the compiler's LDS lowering drops
  // the alias scopes that keep the DMA and the tile reads apart.
  constexpr int ROWS_T = 2 * BQ * (int)(sizeof(float) / sizeof(T));  // one row buffer, in T
  constexpr int KL = dkv_k_lds<D>() ? kBM * D : 0;  // K rows of the item's keys
  __shared__ __align__(16) T smem[2 * BUF + 2 * ROWS_T + KL];
  static_assert(4 * stage_elems<D>() <= 2 * BUF + KL, "dK/dV staging must fit in the tile buffers");
  float* sLD0 = reinterpret_cast<float*>(smem + 2 * BUF);
  float* sLD1 = reinterpret_cast<float*>(smem + 2 * BUF + ROWS_T);

  // One workgroup per (item, K/V head hk, part): the part's share of the
  // group's query heads hk*group + [g0, g1) is swept one head after another
  // and their contributions accumulate in the dK / dV registers.  With
  // gsplit > 1 parts, each part stores its fp32 sums and dkv_reduce_kernel
  // adds them up after the pass.
  const ItemView iv = item_view<false>(src, tmax);
  if (iv.failed) {
    poison_rows(dk, sdk, total, kv_heads, dcols);
    poison_rows(dv, sdv, total, kv_heads, dcols);
    return;
  }
  int item, hv;
  if (!map_block(kv_heads * gsplit, tmax, head_major, 1, D * (int)sizeof(T) < 128 && group == 1, item,
                 hv) ||
      item >= iv.count)
    return;
  const int hk = hv % kv_heads, part = hv / kv_heads;
  const int g0 = part * group / gsplit, g1 = (part + 1) * group / gsplit;
  const int heads = kv_heads * group;
  const int4 it = item_at<false>(src, iv, CAUSAL, item);
  if (it.w == 0) return;
  const int start = it.z, L = it.w;
  const int nblk = (L + kBM - 1) / kBM;
  const int k0 = (nblk - 1 - it.y) * kBM;  // key-major: the list's blk counts down
  DkvState<T, D> st;
  st.wave = wave_id();
  const int lane = threadIdx.x & (kWave - 1);
  st.g = lane >> 5;
  st.lr = lane & 31;
  st.kw0 = k0 + 32 * st.wave;
  const int my_k = st.kw0 + st.lr;
  st.wave_live = st.kw0 < L;
  st.L = L;
  st.heads = heads;
  st.qrow = sq.row;
  st.drow = sdo.row;
  st.qbeg = CAUSAL ? k0 : 0;  // k0 is a multiple of BQ
  st.nqb = (L - st.qbeg + BQ - 1) / BQ;
  st.scale_log2 = scale_log2;
  // REV (head-major launches, sequence-major list): sweep the query blocks
  // from the last down, so the resident items of one sequence all start
  // there and move together; upward sweeps start at their own key blocks.
  st.qstep = REV ? -BQ : BQ;
  st.qfirst = REV ? st.qbeg + (st.nqb - 1) * BQ : st.qbeg;

  T* bufA = smem;
  T* bufB = smem + BUF;
  st.dQ.init(sq.row, st.wave, lane, dcols);
  st.dO.init(sdo.row, st.wave, lane, dcols);
  // Query head h: point the state at it and stage its first block.
  auto start_head = [&](int h) {
    st.qh = q + (int64_t)start * sq.row + (int64_t)h * sq.head;
    st.dh = dout + (int64_t)start * sdo.row + (int64_t)h * sdo.head;
    st.lse_h = lse + (int64_t)start * heads + h;
    st.delta_h = delta + (int64_t)start * heads + h;
    st.dQ.load(bufA, st.qh, sq.row, st.qfirst, L, st.wave);
    st.dO.load(bufA + TILE, st.dh, sdo.row, st.qfirst, L, st.wave);
    if (threadIdx.x < BQ) {
      dkv_load_rows(st, st.qfirst + (int)threadIdx.x);
      dkv_store_rows(sLD0, BQ, st.pl, st.pd);
    }
  };
  start_head(hk * group + g0);
#pragma unroll
  for (int s = 0; s < D / 16; ++s) st.qoff[s] = swz_off<D>(st.lr, 2 * s + st.g);
  // This wave's K rows in LDS (D = 128): same swizzle as a Q tile, so the
  // score MFMA reads them with the Q tile's offsets.  Only this wave reads
  // them, after the barrier at the top of the head loop.
  T* kl = smem + 2 * BUF + 2 * ROWS_T + 32 * st.wave * D;
  {  // keys past L read row L-1: their results are never stored
    const int64_t tok = start + min(my_k, L - 1);
    const T* krow = k + tok * sk.row + (int64_t)hk * sk.head;
    const T* vrow = v + tok * sv.row + (int64_t)hk * sv.head;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      if constexpr (dkv_k_lds<D>())
        *reinterpret_cast<uint4*>(kl + st.qoff[s]) =
            __builtin_bit_cast(uint4, gmem_frag16_cols<D>(krow, 16 * s + 8 * st.g, dcols));
      else
        st.kf[s] = gmem_frag16_cols<D>(krow, 16 * s + 8 * st.g, dcols);
      st.vf[s] = gmem_frag16_cols<D>(vrow, 16 * s + 8 * st.g, dcols);
    }
    // Materialize the fragments here, before the barrier: left to itself the
    // compiler sinks these loads into the block loop, where their counter
    // waits then also wait out each block's freshly issued DMA.
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      if constexpr (!dkv_k_lds<D>()) asm volatile("" : "+v"(st.kf[s]));
      asm volatile("" : "+v"(st.vf[s]));
    }
  }
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) st.qtr[dt] = swz_tr_off<D>(st.lr, st.g, dt);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    st.dkacc[dt] = zero16();
    st.dvacc[dt] = zero16();
  }

  for (int gi = g0;;) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // Unrolled by two so that each call sees its buffers at fixed positions.
    for (int b = 0; b < st.nqb; b += 2) {
      dkv_step<T, D, CAUSAL>(st, b, bufA, bufB, sLD0, sLD1, kl);
      if (b + 1 < st.nqb) dkv_step<T, D, CAUSAL>(st, b + 1, bufB, bufA, sLD1, sLD0, kl);
    }
    // The last step ended with a barrier: both buffers are free again.
    if (++gi == g1) break;
    start_head(hk * group + gi);
  }
  if constexpr (SPLIT) {
    dkv_store_partial<D>(st.dkacc, st.dvacc,
                         partial + (((int64_t)item * kv_heads + hk) * gsplit + part) * (2 * kBM * D),
                         32 * st.wave + st.lr, st.g);
    return;
  }
  if (st.wave_live) {  // the last step's barrier freed the tile buffers: stage dK, then dV
    const int nrows = min(32, L - st.kw0);
    T* stage = smem + st.wave * stage_elems<D>();
    store_rows_staged<T, D>(stage, st.dkacc, scale,
                            dk + (int64_t)(start + st.kw0) * sdk.row + (int64_t)hk * sdk.head,
                            sdk.row, nrows, dcols, st.lr, st.g, lane);
    store_rows_staged<T, D>(stage, st.dvacc, 1.0f,
                            dv + (int64_t)(start + st.kw0) * sdv.row + (int64_t)hk * sdv.head,
                            sdv.row, nrows, dcols, st.lr, st.g, lane);
  }
}

// ---------------------------------------------------------- fp32 attention
// fp32 inputs, which the reference's Array-level function computes as given
// (its torch branch, reference/varlen_attention.py:90-113).  The matrix
// instructions run fp32 at a sixteenth of their 16-bit rate, so these kernels
// use FP32 FMAs instead: each row of an item (a query, or a key for dK/dV) is
// split over TPR consecutive lanes holding DPT columns each (DPT = 16, or 4-8
// for small launches, below), a dot product is DPT FMAs plus a DPP sum over
// those lanes, and K / V (or Q / dO)
// rows are staged 32 at a time in LDS, where every row group of a wave reads
// the same staged row (a broadcast); the next 32 rows are loaded into
// registers while the current ones are used.  Two workgroups share an item,
// 64 rows each (in passes of 32 rows at head_dim 256), which doubles the
// workgroups a small problem spreads over the CUs.  Scores, weights, sums and
// accumulators are fp32; the forward takes each 32-key tile's maximum before
// forming its weights, so every weight is at most 1, as in the reference's
// max-subtracted softmax.  Every sum over keys or queries is taken per
// 32-row tile first and then over the tiles, which keeps its rounding error
// near that of the blocked sums of a GEMM (a group of 4 heads over 1,000
// queries otherwise added 3x the reference's own fp32 error to dV).  Same
// work lists, item order and failure handling as the 16-bit kernels.
constexpr int kF32Split = 2;                // workgroups per item
constexpr int kF32WgRows = kBM / kF32Split;  // rows of an item per workgroup
constexpr int kF32Rows = 32;                // keys (forward, dQ) or queries (dK/dV) per LDS tile
// Columns per lane: 16 (the narrow form), or, for launches too small to
// give every SIMD a wave in that form, max(4, D / 16) (the wide form: 4 to
// 16 lanes per row, so each row's chain of keys is 2-4x shorter and a
// workgroup holds up to 4x the waves, at the price of repeating each row's
// softmax arithmetic on more lanes).  Both keep every row within 16 lanes.
// Measured (MI355X, causal): config 1's 1,980 tokens x 4 heads x 32, a
// narrow grid of 512 waves, run 56 -> 30 us forward and 182 -> 100 us
// forward + backward in the wide form (with its two key groups, below);
// 7,168 tokens x 8 heads x 64 (3,776 narrow waves) ran 13 % (forward) and
// 41 % (forward + backward) slower with the wider rows, so only launches
// below one narrow wave per SIMD take them.
constexpr int kF32NarrowDpt = 16;
template <int D>
constexpr int f32_wide_dpt() {
  return D / 16 > 4 ? D / 16 : 4;
}
template <int D, int DPT>
constexpr int f32_tpr() {
  return D / DPT;  // lanes per row
}
// KG groups per row (wide form): the row's keys (forward, dQ) or queries
// (dK/dV) are dealt out to KG groups of TPR lanes, each keeping its own
// softmax state or partial sums, merged at the end of the row pass.  Rows
// per pass: up to 512 threads per group.
template <int D, int DPT>
constexpr int f32_rows() {
  return kF32WgRows * f32_tpr<D, DPT>() <= 512 ? kF32WgRows : 512 / f32_tpr<D, DPT>();
}
template <int D, int DPT, int KG = 1>
constexpr int f32_threads() {
  return f32_rows<D, DPT>() * f32_tpr<D, DPT>() * KG;
}

// Sum over the TPR (1 to 16) consecutive lanes of one row, by the DPP steps
// of wave_sum_i (lane ^ 1, lane ^ 2, then the mirrors across 8 and 16
// lanes): VALU operations, no LDS round trip per reduction.
template <int TPR>
__device__ __forceinline__ float row_sum(float x) {
  static_assert(TPR >= 1 && TPR <= 16 && (TPR & (TPR - 1)) == 0, "TPR: a power of two <= 16");
  auto step = [](float v, auto ctrl) {
    return v + __builtin_bit_cast(float, dpp_i<decltype(ctrl)::value>(__builtin_bit_cast(int, v)));
  };
  if constexpr (TPR >= 2) x = step(x, std::integral_constant<int, 0xB1>{});
  if constexpr (TPR >= 4) x = step(x, std::integral_constant<int, 0x4E>{});
  if constexpr (TPR >= 8) x = step(x, std::integral_constant<int, 0x141>{});
  if constexpr (TPR >= 16) x = step(x, std::integral_constant<int, 0x140>{});
  return x;
}
template <int N>
__device__ __forceinline__ void load_slice(float (&dst)[N], const float* p) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const float4 t = *reinterpret_cast<const float4*>(p + i);
    dst[i] = t.x, dst[i + 1] = t.y, dst[i + 2] = t.z, dst[i + 3] = t.w;
  }
}
template <int N>
__device__ __forceinline__ void store_slice(float* __restrict__ p, const float (&src)[N], float mul) {
#pragma unroll
  for (int i = 0; i < N; i += 4)
    *reinterpret_cast<float4*>(p + i) =
        make_float4(src[i] * mul, src[i + 1] * mul, src[i + 2] * mul, src[i + 3] * mul);
}
template <int N>
__device__ __forceinline__ float dot_slice(const float (&a)[N], const float (&b)[N]) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < N; i += 2) {
    s0 = fmaf(a[i], b[i], s0);
    s1 = fmaf(a[i + 1], b[i + 1], s1);
  }
  return s0 + s1;
}
template <int N>
__device__ __forceinline__ void axpy_slice(float (&acc)[N], float a, const float (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) acc[i] = fmaf(a, x[i], acc[i]);
}

// Two (rows, D) matrices' rows [row0, row0 + kF32Rows) through registers into
// LDS (row-major, D floats per row); rows >= limit become zeros.  load()
// issues the global reads, store() writes what they returned.
template <int D, int THREADS>
struct F32Stage {
  static constexpr int C4 = D / 4;
  static constexpr int N4 = kF32Rows * C4;  // float4 per matrix
  static constexpr int PER = (N4 + THREADS - 1) / THREADS;
  float4 a[PER], b[PER];
  __device__ __forceinline__ void load(const float* __restrict__ pa, int64_t sa,
                                       const float* __restrict__ pb, int64_t sb, int row0, int limit) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = (int)threadIdx.x + j * THREADS;
      const int r = idx / C4, c = 4 * (idx % C4), row = row0 + r;
      const bool ok = idx < N4 && row < limit;
      a[j] = ok ? *reinterpret_cast<const float4*>(pa + (int64_t)row * sa + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      b[j] = ok ? *reinterpret_cast<const float4*>(pb + (int64_t)row * sb + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __device__ __forceinline__ void store(float* la, float* lb) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = (int)threadIdx.x + j * THREADS;
      if (idx < N4) {
        reinterpret_cast<float4*>(la)[idx] = a[j];
        reinterpret_cast<float4*>(lb)[idx] = b[j];
      }
    }
  }
};

template <int D, bool CAUSAL, int DPT, int KG>
__global__ __launch_bounds__((f32_threads<D, DPT, KG>())) void attn_fwd_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ o, float* __restrict__ lse, ItemSource src, int tmax, int head_major,
    int heads, int group, Strides sq, Strides sk, Strides sv, Strides so, float scale, int total) {
  constexpr int TPR = f32_tpr<D, DPT>(), RPP = f32_rows<D, DPT>(), KT = kF32Rows;
  static_assert(KT % KG == 0 && (KG == 1 || KG == 2), "one or two key groups");
  __shared__ __align__(16) float sK[KT * D];
  __shared__ __align__(16) float sV[KT * D];
  const ItemView iv = item_view<true>(src, tmax);
  if (iv.failed) {
    publish_header(src, iv, CAUSAL ? 1 : 0);
    poison_rows(o, so, total, heads, D);
    poison_stats(lse, total, heads);
    return;
  }
  const int part = blockIdx.x % kF32Split;
  int item, h;
  if (!map_block_at(blockIdx.x / kF32Split, heads, tmax, head_major, group, false, item, h) ||
      item >= iv.count) {
    publish_header(src, iv, CAUSAL ? 1 : 0);
    return;
  }
  const int4 it = item_at<true>(src, iv, CAUSAL, item);
  const int start = it.z, L = it.w, q0 = it.y * kBM + part * kF32WgRows;  // this workgroup's rows
  if (L > 0 && q0 < L) {
    const int hk = h / group;
    const int c0 = (threadIdx.x % TPR) * DPT;
    const float* kh = k + (int64_t)start * sk.row + (int64_t)hk * sk.head;
    const float* vh = v + (int64_t)start * sv.row + (int64_t)hk * sv.head;
    const int kend = CAUSAL ? min(L, q0 + kF32WgRows) : L;
    const int kg = KG > 1 ? ((int)threadIdx.x / TPR) % KG : 0;  // this lane's key group
    F32Stage<D, f32_threads<D, DPT, KG>()> stage;
    for (int r0 = 0; r0 < kF32WgRows && q0 + r0 < L; r0 += RPP) {
      const int my_q = q0 + r0 + (int)threadIdx.x / (TPR * KG);
      // rows past L compute on row L-1 and store nothing
      float qv[DPT], ov[DPT];
      load_slice(qv, q + (int64_t)(start + min(my_q, L - 1)) * sq.row + (int64_t)h * sq.head + c0);
#pragma unroll
      for (int i = 0; i < DPT; ++i) ov[i] = 0.f;
      float m = kNegInf, l = 0.f;
      const int qlim = CAUSAL ? min(my_q, L - 1) : L - 1;  // the last key this row sees
      const int kpass = CAUSAL ? min(kend, q0 + r0 + RPP) : kend;
      stage.load(kh, sk.row, vh, sv.row, 0, kend);
      for (int kb = 0; kb < kpass; kb += KT) {
        __syncthreads();  // the previous tile is consumed
        stage.store(sK, sV);
        __syncthreads();
        if (kb + KT < kpass) stage.load(kh, sk.row, vh, sv.row, kb + KT, kend);
        float s[KT / KG];  // this group's keys of the tile: kg, kg + KG, ...
        float tile_m = kNegInf;
#pragma unroll
        for (int j = 0; j < KT / KG; ++j) {
          const int i = j * KG + kg;
          float kr[DPT];
          load_slice(kr, sK + i * D + c0);
          const float dotv = row_sum<TPR>(dot_slice(qv, kr)) * scale;
          s[j] = kb + i <= qlim ? dotv : kNegInf;
          tile_m = fmaxf(tile_m, s[j]);
        }
        // key 0 is in every row's first tile, so m is finite from then on;
        // with two key groups the second may see no key of a row at all
        // (row 0, or a length-1 sequence): its m stays -inf, its weights 0
        const float m_new = fmaxf(m, tile_m);
        const float m_ref = KG > 1 && m_new == kNegInf ? 0.f : m_new;
        const float alpha = fast_exp2((m - m_ref) * kLog2e);
        float ot[DPT], lt = 0.f;
#pragma unroll
        for (int d = 0; d < DPT; ++d) ot[d] = 0.f;
#pragma unroll 4
        for (int j = 0; j < KT / KG; ++j) {
          const float p = fast_exp2((s[j] - m_ref) * kLog2e);
          float vr[DPT];
          load_slice(vr, sV + (j * KG + kg) * D + c0);
          lt += p;
          axpy_slice(ot, p, vr);
        }
        l = fmaf(l, alpha, lt);
#pragma unroll
        for (int d = 0; d < DPT; ++d) ov[d] = fmaf(ov[d], alpha, ot[d]);
        m = m_new;
      }
      if constexpr (KG > 1) {  // merge the two groups' states (lanes TPR apart)
        const float m_all = fmaxf(m, __shfl_xor(m, TPR, kWave));  // group 0 holds key 0: finite
        const float a = fast_exp2((m - m_all) * kLog2e);
        l *= a;
        l += __shfl_xor(l, TPR, kWave);
#pragma unroll
        for (int d = 0; d < DPT; ++d) {
          ov[d] *= a;
          ov[d] += __shfl_xor(ov[d], TPR, kWave);
        }
        m = m_all;
      }
      if (my_q < L && kg == 0) {
        store_slice(o + (int64_t)(start + my_q) * so.row + (int64_t)h * so.head + c0, ov, 1.0f / l);
        if (c0 == 0) lse[(int64_t)(start + my_q) * heads + h] = m + logf(l);
      }
    }
  }
  publish_header(src, iv, CAUSAL ? 1 : 0);
  if (h == 0 && part == 0 && L > 0) publish_item(src, item, it);
}

// dQ = scale * dS K with dS = P (dP - Delta), P = exp(S - LSE), dP = dO V^T;
// Delta = rowsum(O * dO) is formed here and written out for the dK/dV pass.
template <int D, bool CAUSAL, int DPT, int KG>
__global__ __launch_bounds__((f32_threads<D, DPT, KG>())) void attn_bwd_dq_f32_kernel(
    const float* __restrict__ dout, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ o, const float* __restrict__ lse,
    float* __restrict__ delta, float* __restrict__ dq, ItemSource src, int tmax, int head_major,
    int heads, int group, Strides sdo, Strides sq, Strides sk, Strides sv, Strides so,
    Strides sdq, float scale, int total) {
  constexpr int TPR = f32_tpr<D, DPT>(), RPP = f32_rows<D, DPT>(), KT = kF32Rows;
  static_assert(KT % KG == 0 && (KG == 1 || KG == 2), "one or two key groups");
  __shared__ __align__(16) float sK[KT * D];
  __shared__ __align__(16) float sV[KT * D];
  const ItemView iv = item_view<false>(src, tmax);
  if (iv.failed) {
    poison_rows(dq, sdq, total, heads, D);
    poison_stats(delta, total, heads);
    return;
  }
  const int part = blockIdx.x % kF32Split;
  int item, h;
  if (!map_block_at(blockIdx.x / kF32Split, heads, tmax, head_major, group, false, item, h) ||
      item >= iv.count)
    return;
  const int4 it = item_at<false>(src, iv, CAUSAL, item);
  const int start = it.z, L = it.w, q0 = it.y * kBM + part * kF32WgRows;
  if (L == 0 || q0 >= L) return;
  const int hk = h / group;
  const int c0 = (threadIdx.x % TPR) * DPT;
  const float* kh = k + (int64_t)start * sk.row + (int64_t)hk * sk.head;
  const float* vh = v + (int64_t)start * sv.row + (int64_t)hk * sv.head;
  const int kend = CAUSAL ? min(L, q0 + kF32WgRows) : L;
  const float c = scale * kLog2e;
  const int kg = KG > 1 ? ((int)threadIdx.x / TPR) % KG : 0;  // this lane's key group
  F32Stage<D, f32_threads<D, DPT, KG>()> stage;
  for (int r0 = 0; r0 < kF32WgRows && q0 + r0 < L; r0 += RPP) {
    const int my_q = q0 + r0 + (int)threadIdx.x / (TPR * KG);
    const int64_t tok = start + min(my_q, L - 1);
    const int kpass = CAUSAL ? min(kend, q0 + r0 + RPP) : kend;
    stage.load(kh, sk.row, vh, sv.row, 0, kend);
    float qv[DPT], dov[DPT], dqv[DPT];
    float dl;
    {
      float ov[DPT];
      load_slice(qv, q + tok * sq.row + (int64_t)h * sq.head + c0);
      load_slice(dov, dout + tok * sdo.row + (int64_t)h * sdo.head + c0);
      load_slice(ov, o + tok * so.row + (int64_t)h * so.head + c0);
      dl = row_sum<TPR>(dot_slice(ov, dov));
    }
    if (my_q < L && c0 == 0 && kg == 0) delta[(int64_t)(start + my_q) * heads + h] = dl;
    const float lse2 = lse[tok * heads + h] * kLog2e;
#pragma unroll
    for (int d = 0; d < DPT; ++d) dqv[d] = 0.f;
    const int qlim = CAUSAL ? min(my_q, L - 1) : L - 1;
    for (int kb = 0; kb < kpass; kb += KT) {
      __syncthreads();
      stage.store(sK, sV);
      __syncthreads();
      if (kb + KT < kpass) stage.load(kh, sk.row, vh, sv.row, kb + KT, kend);
      float dqt[DPT];
#pragma unroll
      for (int d = 0; d < DPT; ++d) dqt[d] = 0.f;
#pragma unroll 2
      for (int j = 0; j < KT / KG; ++j) {  // this group's keys: kg, kg + KG, ...
        const int i = j * KG + kg;
        float kr[DPT], vr[DPT];
        load_slice(kr, sK + i * D + c0);
        load_slice(vr, sV + i * D + c0);
        const float sdot = row_sum<TPR>(dot_slice(qv, kr));
        const float pdot = row_sum<TPR>(dot_slice(dov, vr));
        const float p = kb + i <= qlim ? fast_exp2(fmaf(sdot, c, -lse2)) : 0.f;
        axpy_slice(dqt, p * (pdot - dl), kr);
      }
#pragma unroll
      for (int d = 0; d < DPT; ++d) dqv[d] += dqt[d];
    }
    if constexpr (KG > 1) {  // the two groups' sums (lanes TPR apart)
#pragma unroll
      for (int d = 0; d < DPT; ++d) dqv[d] += __shfl_xor(dqv[d], TPR, kWave);
    }
    if (my_q < L && kg == 0)
      store_slice(dq + (int64_t)(start + my_q) * sdq.row + (int64_t)h * sdq.head + c0, dqv, scale);
  }
}

// dV = P^T dO and dK = scale * dS^T Q for 64 of an item's keys, summed over
// the query heads that share their K/V head.
template <int D, bool CAUSAL, int DPT, int KG>
__global__ __launch_bounds__((f32_threads<D, DPT, KG>())) void attn_bwd_dkv_f32_kernel(
    const float* __restrict__ dout, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dk, float* __restrict__ dv, ItemSource src, int tmax, int head_major,
    int kv_heads, int group, Strides sdo, Strides sq, Strides sk, Strides sv, Strides sdk,
    Strides sdv, float scale, int total) {
  constexpr int TPR = f32_tpr<D, DPT>(), RPP = f32_rows<D, DPT>(), QT = kF32Rows;
  static_assert(QT % KG == 0 && (KG == 1 || KG == 2), "one or two query groups");
  __shared__ __align__(16) float sQ[QT * D];
  __shared__ __align__(16) float sO[QT * D];  // dO rows
  __shared__ float sL[QT], sD[QT];             // LSE * log2(e) and Delta of those rows
  const ItemView iv = item_view<false>(src, tmax);
  if (iv.failed) {
    poison_rows(dk, sdk, total, kv_heads, D);
    poison_rows(dv, sdv, total, kv_heads, D);
    return;
  }
  const int part = blockIdx.x % kF32Split;
  int item, hk;
  if (!map_block_at(blockIdx.x / kF32Split, kv_heads, tmax, head_major, 1, false, item, hk) ||
      item >= iv.count)
    return;
  const int4 it = item_at<false>(src, iv, CAUSAL, item);
  const int start = it.z, L = it.w;
  const int nblk = (L + kBM - 1) / kBM;
  const int k0 = (nblk - 1 - it.y) * kBM + part * kF32WgRows;  // key-major: the list's blk counts down
  if (L == 0 || k0 >= L) return;
  const int heads = kv_heads * group;
  const int c0 = (threadIdx.x % TPR) * DPT;
  const float c = scale * kLog2e;
  const int kg = KG > 1 ? ((int)threadIdx.x / TPR) % KG : 0;  // this lane's query group
  F32Stage<D, f32_threads<D, DPT, KG>()> stage;
  for (int r0 = 0; r0 < kF32WgRows && k0 + r0 < L; r0 += RPP) {
    const int my_k = k0 + r0 + (int)threadIdx.x / (TPR * KG);
    const int64_t tok = start + min(my_k, L - 1);
    float kv[DPT], vv[DPT], dkv[DPT], dvv[DPT];
    load_slice(kv, k + tok * sk.row + (int64_t)hk * sk.head + c0);
    load_slice(vv, v + tok * sv.row + (int64_t)hk * sv.head + c0);
#pragma unroll
    for (int d = 0; d < DPT; ++d) dkv[d] = dvv[d] = 0.f;
    const int qbeg = CAUSAL ? k0 + r0 : 0;  // no earlier query sees this pass's keys
    for (int gi = 0; gi < group; ++gi) {
      const int h = hk * group + gi;
      const float* qh = q + (int64_t)start * sq.row + (int64_t)h * sq.head;
      const float* dh = dout + (int64_t)start * sdo.row + (int64_t)h * sdo.head;
      float pl = 0.f, pd = 0.f;  // the next tile's LSE and Delta (threads < QT)
      auto load_rows = [&](int qb) {
        const int qq = qb + (int)threadIdx.x;
        pl = threadIdx.x < QT && qq < L ? lse[(int64_t)(start + qq) * heads + h] * kLog2e : 0.f;
        pd = threadIdx.x < QT && qq < L ? delta[(int64_t)(start + qq) * heads + h] : 0.f;
      };
      stage.load(qh, sq.row, dh, sdo.row, qbeg, L);
      load_rows(qbeg);
      for (int qb = qbeg; qb < L; qb += QT) {
        __syncthreads();
        stage.store(sQ, sO);
        if (threadIdx.x < QT) {
          sL[threadIdx.x] = pl;
          sD[threadIdx.x] = pd;
        }
        __syncthreads();
        if (qb + QT < L) {
          stage.load(qh, sq.row, dh, sdo.row, qb + QT, L);
          load_rows(qb + QT);
        }
        float dkt[DPT], dvt[DPT];
#pragma unroll
        for (int d = 0; d < DPT; ++d) dkt[d] = dvt[d] = 0.f;
#pragma unroll 2
        for (int j = 0; j < QT / KG; ++j) {  // this group's queries: kg, kg + KG, ...
          const int i = j * KG + kg;
          const int qq = qb + i;
          float qr[DPT], orow[DPT];
          load_slice(qr, sQ + i * D + c0);
          load_slice(orow, sO + i * D + c0);
          const float sdot = row_sum<TPR>(dot_slice(kv, qr));
          const float pdot = row_sum<TPR>(dot_slice(vv, orow));
          const bool ok = qq < L && (!CAUSAL || qq >= my_k);
          const float p = ok ? fast_exp2(fmaf(sdot, c, -sL[i])) : 0.f;
          axpy_slice(dvt, p, orow);
          axpy_slice(dkt, p * (pdot - sD[i]), qr);
        }
#pragma unroll
        for (int d = 0; d < DPT; ++d) {
          dkv[d] += dkt[d];
          dvv[d] += dvt[d];
        }
      }
    }
    if constexpr (KG > 1) {  // the two groups' sums (lanes TPR apart)
#pragma unroll
      for (int d = 0; d < DPT; ++d) {
        dkv[d] += __shfl_xor(dkv[d], TPR, kWave);
        dvv[d] += __shfl_xor(dvv[d], TPR, kWave);
      }
    }
    if (my_k < L && kg == 0) {
      store_slice(dk + (int64_t)(start + my_k) * sdk.row + (int64_t)hk * sdk.head + c0, dkv, scale);
      store_slice(dv + (int64_t)(start + my_k) * sdv.row + (int64_t)hk * sdv.head + c0, dvv, 1.0f);
    }
  }
}

// ------------------------------------------------------------------- host
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_tensor(const char* fn, const char* name, const void* p, const int64_t* st, int heads,
                 int head_dim, int64_t total) {
  if (!p)  // an empty tensor (no tokens) may have no storage: nothing will be read or written
    return total == 0 ? SCREE_OK : set_error(SCREE_ERR_INVALID, "%s: %s is null", fn, name);
  if (!aligned16(p)) return set_error(SCREE_ERR_INVALID, "%s: %s is not 16-byte aligned", fn, name);
  if (st[0] % 8 || st[1] % 8 || st[0] < 0 || st[1] < 0)
    return set_error(SCREE_ERR_INVALID,
                     "%s: %s strides (%lld, %lld) must be non-negative multiples of 8 elements",
                     fn, name, (long long)st[0], (long long)st[1]);
  if (st[0] >= ((int64_t)1 << 24) || st[1] >= ((int64_t)1 << 24))
    return set_error(SCREE_ERR_INVALID, "%s: %s strides must be below 2^24 elements", fn, name);
  if (total > 1 && st[0] < head_dim)
    return set_error(SCREE_ERR_INVALID, "%s: %s row stride %lld overlaps rows", fn, name,
                     (long long)st[0]);
  (void)heads;
  return SCREE_OK;
}

// head_dim the kernels are instantiated for: every power of two from 16 to
// 256, with 16 run by the 32-column kernels on zero-padded rows (the dcols
// argument: loads past it read zeros, stores past it are skipped).
inline bool head_dim_supported(int head_dim) {
  return head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
}
inline int compute_dim(int head_dim) { return head_dim < 32 ? 32 : head_dim; }

int check_common(const char* fn, const int32_t* cu, int batch, int64_t total, int heads,
                 int head_dim, int dtype, const void* workspace, size_t workspace_bytes) {
  if (!cu) return set_error(SCREE_ERR_INVALID, "%s: cu_seqlens is null", fn);
  if (batch < 1) return set_error(SCREE_ERR_UNSUPPORTED, "%s: batch must be at least 1, got %d", fn, batch);
  if (total < 0 || total > ((int64_t)1 << 30))
    return set_error(SCREE_ERR_INVALID, "%s: total_tokens %lld out of range", fn, (long long)total);
  if (heads < 1 || heads > 4096)
    return set_error(SCREE_ERR_INVALID, "%s: heads must be in [1, 4096], got %d", fn, heads);
  if (!head_dim_supported(head_dim))
    return set_error(SCREE_ERR_UNSUPPORTED, "%s: head_dim %d unsupported (16, 32, 64, 128, 256)",
                     fn, head_dim);
  if (dtype != SCREE_DTYPE_F16 && dtype != SCREE_DTYPE_BF16 && dtype != SCREE_DTYPE_F32)
    return set_error(SCREE_ERR_UNSUPPORTED, "%s: dtype code %d unsupported (fp16, bf16, fp32)", fn,
                     dtype);
  const size_t need = scree_attn_workspace_bytes(batch, total, head_dim);
  if (!workspace || workspace_bytes < need)
    return set_error(SCREE_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", fn, need,
                     workspace ? workspace_bytes : (size_t)0);
  if (tmax_for(batch, total) * heads * (dtype == SCREE_DTYPE_F32 ? kF32Split : 1) > 0x7fffffffLL)
    return set_error(SCREE_ERR_INVALID, "%s: grid too large", fn);
  return SCREE_OK;
}

// Grouped-query dK/dV has one workgroup per (item, K/V head): group times
// fewer than the other passes.  When that leaves the GPU short of work (fewer
// than two rounds of ~3 resident workgroups per CU on 256 CUs), each head
// group is split into equal parts (a divisor of the group: unequal parts
// leave the largest as the tail) that run as workgroups of their own.
// Measured on config 4 with 16 query heads (dK/dV pass + reduce): 4 K/V
// heads in 4 parts 89 us (one part ~146 us, two parts 107 us), 2 K/V heads
// in 8 parts 86 us (7 unequal parts 131 us), 1 K/V head in 16 parts 86 us.
constexpr int64_t kDkvSlots = 1536;
inline int dkv_gsplit(int64_t tmax, int kv_heads, int group) {
  const int64_t wgs = tmax * kv_heads;
  if (group < 2 || wgs >= kDkvSlots) return 1;
  const int64_t want = (kDkvSlots + wgs - 1) / wgs;
  for (int p = 2; p < group; ++p)
    if (group % p == 0 && p >= want) return p;
  return group;
}
inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
// Bytes after the schedule for a split: fp32 dK / dV sums of 128 keys for
// every (item, K/V head, part).
inline size_t dkv_split_bytes(int64_t tmax, int kv_heads, int gsplit, int head_dim) {
  if (gsplit < 2) return 0;
  return (size_t)tmax * kv_heads * gsplit * 2 * kBM * compute_dim(head_dim) * sizeof(float);
}

// Head-major block order pays off once every XCD has many rounds of items
// (~64 resident workgroups per XCD): then L2 locality beats cross-head balance.
inline int attn_head_major(int heads, int tmax) {
  return (heads % kXcds == 0) && ((int64_t)tmax * heads / kXcds >= 512) ? 1 : 0;
}
// The item list a launch reads.  Head-major launches take the sequence-major
// list: an XCD's resident workgroups then hold row blocks of one sequence and
// head, which read the same K/V prefix (or, in the dK/dV pass, the same Q /
// dO suffix) at about the same time, so the XCD's L2 serves most of the
// re-reads; in longest-work-first order they mix sequences and drift apart.
inline const int4* schedule_list(const void* ws, int tmax, int head_major) {
  return reinterpret_cast<const int4*>(static_cast<const char*>(ws) + kHeaderBytes) +
         (head_major ? tmax : 0);
}
// The forward derives its items (and publishes its list) for batches of at
// most kWaveSched sequences in launches of a few rounds of workgroups; the
// backward passes read the lists.  Deriving costs each round of workgroups
// ~0.6 us at head_dim <= 64 (four or three workgroups per CU) and ~1.2 us at
// 128 (two): config 4's 1,776 workgroups pay +1.0 us against the scheduler's
// 3.4, config 5's 22,048 at head_dim 128 +55 us.
constexpr int64_t kFwdDeriveMaxBlocks = 2048;  // 1024 at head_dim 128, 512 at 256
static_assert(kFwdDeriveMaxBlocks < (int64_t)kXcds * 512,
              "a deriving forward's problem must have no head-major pass (attn_head_major)");
inline bool attn_fwd_derives(int batch, int64_t tmax, int heads, int head_dim) {
  return batch <= kWaveSched &&
         tmax * heads <= (head_dim <= 64    ? kFwdDeriveMaxBlocks
                          : head_dim <= 128 ? kFwdDeriveMaxBlocks / 2
                                            : kFwdDeriveMaxBlocks / 4);
}
inline ItemSource fwd_item_source(void* ws, const int32_t* cu, int batch, int total, int tmax,
                                  int heads, int head_dim, int head_major) {
  const bool derive = attn_fwd_derives(batch, tmax, heads, head_dim);
  return ItemSource{static_cast<const int32_t*>(ws), schedule_list(ws, tmax, head_major), cu,
                    derive ? static_cast<int32_t*>(ws) : nullptr, batch, total, head_major,
                    derive ? 1 : 0};
}
inline ItemSource list_item_source(const void* ws, int total, int tmax, int head_major) {
  return ItemSource{static_cast<const int32_t*>(ws), schedule_list(ws, tmax, head_major), nullptr,
                    nullptr, 0, total, head_major, 0};
}

template <typename T, int D, bool C>
void launch_fwd_t(const void* q, const void* k, const void* v, void* o, float* lse,
                  const int32_t* cu, int batch, int heads, int kv_heads, const int64_t* st,
                  float scale, int tmax, void* ws, int total, int dcols, hipStream_t stream) {
  const int64_t grid = (int64_t)tmax * heads;
  const int hm = attn_head_major(heads, tmax);
  hipLaunchKernelGGL((attn_fwd_kernel<T, D, C>), dim3((unsigned)grid), dim3(kThreads), 0, stream,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<T*>(o), lse, fwd_item_source(ws, cu, batch, total, tmax, heads, D, hm),
                     tmax, hm,
                     heads, heads / kv_heads, Strides{st[0], st[1]}, Strides{st[2], st[3]},
                     Strides{st[4], st[5]}, Strides{st[6], st[7]}, scale, scale * kLog2e, total,
                     dcols);
}

// strides: {dout, q, k, v, o, dq} x {row, head}
template <typename T, int D, bool C>
void launch_bwd_dq_t(const void* dout, const void* q, const void* k, const void* v, const void* o,
                     const float* lse, void* dq, float* delta, const int32_t* /*cu*/,
                     int /*batch*/, int heads, int kv_heads, const int64_t* st, float scale,
                     int tmax, const void* ws, int total, int dcols, hipStream_t stream) {
  const int64_t grid = (int64_t)tmax * heads;
  const int hm = attn_head_major(heads, tmax);
  hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, C>), dim3((unsigned)grid), dim3(kThreads), 0, stream,
                     static_cast<const T*>(dout), static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<const T*>(o), lse, delta, static_cast<T*>(dq),
                     list_item_source(ws, total, tmax, hm), tmax, hm, heads,
                     heads / kv_heads,
                     Strides{st[0], st[1]}, Strides{st[2], st[3]}, Strides{st[4], st[5]},
                     Strides{st[6], st[7]}, Strides{st[8], st[9]}, Strides{st[10], st[11]}, scale,
                     scale * kLog2e, total, dcols);
}

// strides: {dout, q, k, v, dk, dv} x {row, head}
template <typename T, int D, bool C>
void launch_bwd_dkv_t(const void* dout, const void* q, const void* k, const void* v,
                      const float* lse, const float* delta, void* dk, void* dv,
                      const int32_t* /*cu*/, int /*batch*/, int heads, int kv_heads,
                      const int64_t* st, float scale, int tmax,
                      const void* ws, int gsplit, float* partial, int total, int dcols,
                      hipStream_t stream) {
  // one workgroup per (item, K/V head, part of the head group)
  const int64_t grid = (int64_t)tmax * kv_heads * gsplit;
  const int hm = attn_head_major(kv_heads * gsplit, tmax);
  const ItemSource src = list_item_source(ws, total, tmax, hm);
  // the split epilogue has a kernel of its own: its registers would cost the
  // unsplit kernel a wave per SIMD at D = 64
  // (a split group never has the many rounds of a head-major launch)
  auto kern = gsplit > 1 ? attn_bwd_dkv_kernel<T, D, C, true, false>
              : hm       ? attn_bwd_dkv_kernel<T, D, C, false, true>
                         : attn_bwd_dkv_kernel<T, D, C, false, false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                     static_cast<const T*>(dout), static_cast<const T*>(q),
                     static_cast<const T*>(k), static_cast<const T*>(v), lse, delta,
                     static_cast<T*>(dk), static_cast<T*>(dv), src, tmax, hm, kv_heads,
                     heads / kv_heads,
                     Strides{st[0], st[1]}, Strides{st[2], st[3]}, Strides{st[4], st[5]},
                     Strides{st[6], st[7]}, Strides{st[8], st[9]}, Strides{st[10], st[11]}, scale,
                     scale * kLog2e, gsplit, partial, total, dcols);
  if (gsplit > 1)
    hipLaunchKernelGGL((dkv_reduce_kernel<T, D>),
                       dim3((unsigned)((int64_t)tmax * kv_heads * (kBM / kRedRows))), dim3(256), 0,
                       stream, partial, src, tmax, C ? 1 : 0, kv_heads, gsplit, static_cast<T*>(dk),
                       static_cast<T*>(dv), Strides{st[8], st[9]}, Strides{st[10], st[11]}, scale,
                       dcols);
}

// FN<T, compute_dim(head_dim), causal>(...): head_dim 16 runs the 32-column kernels.
#define SCREE_DISPATCH_T(FN, T, D, causal, ...)                                                  \
  do {                                                                                           \
    const int cd_ = compute_dim(D);                                                              \
    if (cd_ == 32) { if (causal) FN<T, 32, true>(__VA_ARGS__); else FN<T, 32, false>(__VA_ARGS__); } \
    else if (cd_ == 64) { if (causal) FN<T, 64, true>(__VA_ARGS__); else FN<T, 64, false>(__VA_ARGS__); } \
    else if (cd_ == 128) { if (causal) FN<T, 128, true>(__VA_ARGS__); else FN<T, 128, false>(__VA_ARGS__); } \
    else { if (causal) FN<T, 256, true>(__VA_ARGS__); else FN<T, 256, false>(__VA_ARGS__); }   \
  } while (0)
#define SCREE_DISPATCH(FN, dtype, D, causal, ...)                                 \
  do {                                                                            \
    if (dtype == SCREE_DTYPE_F16)                                                 \
      SCREE_DISPATCH_T(FN, f16, D, causal, __VA_ARGS__);                          \
    else                                                                          \
      SCREE_DISPATCH_T(FN, bf16, D, causal, __VA_ARGS__);                         \
  } while (0)

// fp32 kernels: FN<head_dim, causal>(...), every head_dim natively.
#define SCREE_DISPATCH_F32(FN, D, causal, ...)                                                   \
  do {                                                                                           \
    if (D == 16) { if (causal) FN<16, true>(__VA_ARGS__); else FN<16, false>(__VA_ARGS__); }     \
    else if (D == 32) { if (causal) FN<32, true>(__VA_ARGS__); else FN<32, false>(__VA_ARGS__); } \
    else if (D == 64) { if (causal) FN<64, true>(__VA_ARGS__); else FN<64, false>(__VA_ARGS__); } \
    else if (D == 128) { if (causal) FN<128, true>(__VA_ARGS__); else FN<128, false>(__VA_ARGS__); } \
    else { if (causal) FN<256, true>(__VA_ARGS__); else FN<256, false>(__VA_ARGS__); }           \
  } while (0)

// The fp32 form for a grid: wide when the narrow form would give the GPU's
// 1,024 SIMDs less than a wave each.
template <int D>
bool f32_use_wide(int64_t grid) {
  constexpr int64_t waves = (f32_threads<D, kF32NarrowDpt>() + kWave - 1) / kWave;
  return f32_wide_dpt<D>() != kF32NarrowDpt && grid * waves < 1024;
}

template <int D, bool C, int DPT, int KG>
void launch_fwd_f32_as(const void* q, const void* k, const void* v, void* o, float* lse,
                       const int32_t* cu, int batch, int heads, int kv_heads, const int64_t* st,
                       float scale, int tmax, void* ws, int total, hipStream_t stream) {
  const int64_t grid = (int64_t)tmax * heads * kF32Split;
  const int hm = attn_head_major(heads, tmax);
  hipLaunchKernelGGL((attn_fwd_f32_kernel<D, C, DPT, KG>), dim3((unsigned)grid),
                     dim3(f32_threads<D, DPT, KG>()), 0,
                     stream, static_cast<const float*>(q), static_cast<const float*>(k),
                     static_cast<const float*>(v), static_cast<float*>(o), lse,
                     fwd_item_source(ws, cu, batch, total, tmax, heads, D, hm), tmax, hm, heads,
                     heads / kv_heads, Strides{st[0], st[1]}, Strides{st[2], st[3]},
                     Strides{st[4], st[5]}, Strides{st[6], st[7]}, scale, total);
}

template <int D, bool C>
void launch_fwd_f32(const void* q, const void* k, const void* v, void* o, float* lse,
                    const int32_t* cu, int batch, int heads, int kv_heads, const int64_t* st,
                    float scale, int tmax, void* ws, int total, hipStream_t stream) {
  if constexpr (f32_wide_dpt<D>() != kF32NarrowDpt) {  // (head_dim 256 has no wide form)
    if (f32_use_wide<D>((int64_t)tmax * heads * kF32Split)) {
      launch_fwd_f32_as<D, C, f32_wide_dpt<D>(), 2>(q, k, v, o, lse, cu, batch, heads, kv_heads,
                                                    st, scale, tmax, ws, total, stream);
      return;
    }
  }
  launch_fwd_f32_as<D, C, kF32NarrowDpt, 1>(q, k, v, o, lse, cu, batch, heads, kv_heads, st, scale,
                                            tmax, ws, total, stream);
}

// strides: {dout, q, k, v, o, dq} x {row, head}
template <int D, bool C, int DPT, int KG>
void launch_bwd_dq_f32_as(const void* dout, const void* q, const void* k, const void* v,
                          const void* o, const float* lse, void* dq, float* delta, int heads,
                          int kv_heads, const int64_t* st, float scale, int tmax, const void* ws,
                          int total, hipStream_t stream) {
  const int64_t grid = (int64_t)tmax * heads * kF32Split;
  const int hm = attn_head_major(heads, tmax);
  hipLaunchKernelGGL((attn_bwd_dq_f32_kernel<D, C, DPT, KG>), dim3((unsigned)grid),
                     dim3(f32_threads<D, DPT, KG>()), 0, stream, static_cast<const float*>(dout), static_cast<const float*>(q),
                     static_cast<const float*>(k), static_cast<const float*>(v),
                     static_cast<const float*>(o), lse, delta, static_cast<float*>(dq),
                     list_item_source(ws, total, tmax, hm), tmax, hm, heads, heads / kv_heads,
                     Strides{st[0], st[1]}, Strides{st[2], st[3]}, Strides{st[4], st[5]},
                     Strides{st[6], st[7]}, Strides{st[8], st[9]}, Strides{st[10], st[11]}, scale,
                     total);
}

template <int D, bool C>
void launch_bwd_dq_f32(const void* dout, const void* q, const void* k, const void* v,
                       const void* o, const float* lse, void* dq, float* delta, int heads,
                       int kv_heads, const int64_t* st, float scale, int tmax, const void* ws,
                       int total, hipStream_t stream) {
  if constexpr (f32_wide_dpt<D>() != kF32NarrowDpt) {
    if (f32_use_wide<D>((int64_t)tmax * heads * kF32Split)) {
      launch_bwd_dq_f32_as<D, C, f32_wide_dpt<D>(), 2>(dout, q, k, v, o, lse, dq, delta, heads,
                                                       kv_heads, st, scale, tmax, ws, total, stream);
      return;
    }
  }
  launch_bwd_dq_f32_as<D, C, kF32NarrowDpt, 1>(dout, q, k, v, o, lse, dq, delta, heads, kv_heads,
                                               st, scale, tmax, ws, total, stream);
}

// strides: {dout, q, k, v, dk, dv} x {row, head}; one workgroup per (item, K/V head)
template <int D, bool C, int DPT, int KG>
void launch_bwd_dkv_f32_as(const void* dout, const void* q, const void* k, const void* v,
                           const float* lse, const float* delta, void* dk, void* dv, int heads,
                           int kv_heads, const int64_t* st, float scale, int tmax, const void* ws,
                           int total, hipStream_t stream) {
  const int64_t grid = (int64_t)tmax * kv_heads * kF32Split;
  const int hm = attn_head_major(kv_heads, tmax);
  hipLaunchKernelGGL((attn_bwd_dkv_f32_kernel<D, C, DPT, KG>), dim3((unsigned)grid),
                     dim3(f32_threads<D, DPT, KG>()), 0, stream, static_cast<const float*>(dout), static_cast<const float*>(q),
                     static_cast<const float*>(k), static_cast<const float*>(v), lse, delta,
                     static_cast<float*>(dk), static_cast<float*>(dv),
                     list_item_source(ws, total, tmax, hm), tmax, hm, kv_heads,
                     heads / kv_heads, Strides{st[0], st[1]}, Strides{st[2], st[3]},
                     Strides{st[4], st[5]}, Strides{st[6], st[7]}, Strides{st[8], st[9]},
                     Strides{st[10], st[11]}, scale, total);
}

template <int D, bool C>
void launch_bwd_dkv_f32(const void* dout, const void* q, const void* k, const void* v,
                        const float* lse, const float* delta, void* dk, void* dv, int heads,
                        int kv_heads, const int64_t* st, float scale, int tmax, const void* ws,
                        int total, hipStream_t stream) {
  if constexpr (f32_wide_dpt<D>() != kF32NarrowDpt) {
    if (f32_use_wide<D>((int64_t)tmax * kv_heads * kF32Split)) {
      // one query group at head_dim 128: two would need 1,024 threads of more
      // than the 128 registers each that allows
      constexpr int KG = D >= 128 ? 1 : 2;
      launch_bwd_dkv_f32_as<D, C, f32_wide_dpt<D>(), KG>(dout, q, k, v, lse, delta, dk, dv, heads,
                                                         kv_heads, st, scale, tmax, ws, total,
                                                         stream);
      return;
    }
  }
  launch_bwd_dkv_f32_as<D, C, kF32NarrowDpt, 1>(dout, q, k, v, lse, delta, dk, dv, heads, kv_heads,
                                                st, scale, tmax, ws, total, stream);
}

}  // namespace
}  // namespace scree

using namespace scree;

extern "C" int scree_attn_needs_schedule(int batch, int64_t total_tokens, int heads,
                                         int head_dim) {
  if (batch < 1 || total_tokens < 0 || heads < 1) return 1;
  return attn_fwd_derives(batch, tmax_for(batch, total_tokens), heads, head_dim) ? 0 : 1;
}

extern "C" size_t scree_attn_workspace_bytes(int batch, int64_t total_tokens, int head_dim) {
  (void)head_dim;
  if (batch < 1 || total_tokens < 0) return 0;
  return schedule_bytes(tmax_for(batch, total_tokens)) + prefix_bytes(batch);
}

extern "C" int scree_attn_schedule(const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                                   int head_dim, int causal, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  const char* fn = "scree_attn_schedule";
  if (!cu_seqlens) return set_error(SCREE_ERR_INVALID, "%s: cu_seqlens is null", fn);
  if (batch < 1) return set_error(SCREE_ERR_UNSUPPORTED, "%s: batch must be at least 1, got %d", fn, batch);
  if (total_tokens < 0 || total_tokens > ((int64_t)1 << 30))
    return set_error(SCREE_ERR_INVALID, "%s: total_tokens %lld out of range", fn,
                     (long long)total_tokens);
  if (!head_dim_supported(head_dim))
    return set_error(SCREE_ERR_UNSUPPORTED, "%s: head_dim %d unsupported (16, 32, 64, 128, 256)",
                     fn, head_dim);
  const size_t need = scree_attn_workspace_bytes(batch, total_tokens, head_dim);
  if (!workspace || workspace_bytes < need)
    return set_error(SCREE_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", fn, need,
                     workspace ? workspace_bytes : (size_t)0);
  int32_t* header = static_cast<int32_t*>(workspace);
  int4* items = reinterpret_cast<int4*>(static_cast<char*>(workspace) + kHeaderBytes);
  const int tmax = (int)tmax_for(batch, total_tokens);
  if (batch <= kWaveSched) {  // one wavefront per list slot
    const int waves = 256 / kWave;
    hipLaunchKernelGGL(attn_wave_schedule_kernel, dim3((unsigned)((tmax + waves - 1) / waves)),
                       dim3(256), 0, static_cast<hipStream_t>(stream), cu_seqlens, batch,
                       (int)total_tokens, causal ? 1 : 0, tmax, header, items);
  } else if (batch <= kMaxBatch) {
    hipLaunchKernelGGL(attn_schedule_kernel, dim3(1), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), cu_seqlens, batch, (int)total_tokens,
                       causal ? 1 : 0, tmax, header, items);
  } else {
    int32_t* prefix = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + schedule_bytes(tmax));
    hipLaunchKernelGGL(attn_big_schedule_kernel, dim3(1), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), cu_seqlens, batch, (int)total_tokens,
                       causal ? 1 : 0, tmax, header, items, prefix);
  }
  return check_launch(fn);
}

static int check_heads(const char* fn, int heads, int kv_heads) {
  if (kv_heads < 1 || kv_heads > heads || heads % kv_heads)
    return set_error(SCREE_ERR_INVALID,
                     "%s: kv_heads (%d) must divide heads (%d) and be at least 1", fn, kv_heads,
                     heads);
  return SCREE_OK;
}

static int check_bwd_tensors(const char* fn, const char* const* names, const void* const* ptrs,
                             int n, const int64_t* strides, int heads, int head_dim,
                             int64_t total) {
  if (!strides) return set_error(SCREE_ERR_INVALID, "%s: strides is null", fn);
  for (int i = 0; i < n; ++i) {
    int rc = check_tensor(fn, names[i], ptrs[i], strides + 2 * i, heads, head_dim, total);
    if (rc) return rc;
  }
  return SCREE_OK;
}

static int check_fwd(const char* fn, const void* q, const void* k, const void* v, const void* o,
                     const float* lse, const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                     int heads, int kv_heads, int head_dim, const int64_t* strides, int dtype,
                     const void* workspace, size_t workspace_bytes) {
  int rc = check_common(fn, cu_seqlens, batch, total_tokens, heads, head_dim, dtype, workspace,
                        workspace_bytes);
  if (rc) return rc;
  if ((rc = check_heads(fn, heads, kv_heads))) return rc;
  if (!strides) return set_error(SCREE_ERR_INVALID, "%s: strides is null", fn);
  if (total_tokens > 0 && (!lse || !aligned16(lse)))
    return set_error(SCREE_ERR_INVALID, "%s: lse null or unaligned", fn);
  const char* names[4] = {"q", "k", "v", "o"};
  const void* ptrs[4] = {q, k, v, o};
  for (int i = 0; i < 4; ++i) {
    rc = check_tensor(fn, names[i], ptrs[i], strides + 2 * i, heads, head_dim, total_tokens);
    if (rc) return rc;
  }
  return SCREE_OK;
}

static int launch_fwd(const char* fn, const void* q, const void* k, const void* v, void* o,
                      float* lse, const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                      int heads, int kv_heads, int head_dim, const int64_t* strides,
                      float softmax_scale, int causal, int dtype, void* workspace,
                      void* stream) {
  if (total_tokens == 0) return SCREE_OK;
  const int tmax = (int)tmax_for(batch, total_tokens);
  if (dtype == SCREE_DTYPE_F32)
    SCREE_DISPATCH_F32(launch_fwd_f32, head_dim, causal, q, k, v, o, lse, cu_seqlens, batch, heads,
                       kv_heads, strides, softmax_scale, tmax, workspace, (int)total_tokens,
                       static_cast<hipStream_t>(stream));
  else
    SCREE_DISPATCH(launch_fwd_t, dtype, head_dim, causal, q, k, v, o, lse, cu_seqlens, batch,
                   heads, kv_heads, strides, softmax_scale, tmax, workspace, (int)total_tokens,
                   head_dim, static_cast<hipStream_t>(stream));
  return check_launch(fn);
}

extern "C" int scree_attn_fwd_gqa(const void* q, const void* k, const void* v, void* o,
                                  float* lse, const int32_t* cu_seqlens, int batch,
                                  int64_t total_tokens, int heads, int kv_heads, int head_dim,
                                  const int64_t* strides, float softmax_scale, int causal,
                                  int dtype, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const char* fn = "scree_attn_fwd";
  int rc = check_fwd(fn, q, k, v, o, lse, cu_seqlens, batch, total_tokens, heads, kv_heads,
                     head_dim, strides, dtype, workspace, workspace_bytes);
  if (rc) return rc;
  return launch_fwd(fn, q, k, v, o, lse, cu_seqlens, batch, total_tokens, heads, kv_heads,
                    head_dim, strides, softmax_scale, causal, dtype, workspace, stream);
}

// ---------------------------------------------- allocation-free forward
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc):
// scree_attn_fwd_noalloc builds the schedule in this file-scope array
// instead of a caller's workspace.  Every GPU the library runs on holds its
// own copy until the process ends.  Host code must not use the array's name
// as an address (that is a host-side stand-in): each device's address comes
// from hipGetSymbolAddress, taken once per device with that device current,
// and only that address is passed to kernels.  The scheduler rewrites the
// header and every item it publishes on each call, so nothing needs
// clearing; two calls that overlap on one GPU race on the array.
static __device__ __align__(256) unsigned char scratch[SCREE_ATTN_NOALLOC_SCHEDULE_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

int scratch_for_current_device(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(SCREE_ERR_HIP, "%s: no usable current device (%s)", fn, hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(SCREE_ERR_HIP, "%s: hipGetSymbolAddress of the static schedule failed: %s",
                       fn, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SCREE_OK;
}
}  // namespace

extern "C" int scree_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* o,
                                      float* lse, const int32_t* cu_seqlens, int batch,
                                      int64_t total_tokens, int heads, int kv_heads, int head_dim,
                                      const int64_t* strides, float softmax_scale, int causal,
                                      int dtype, void* stream) {
  const char* fn = "scree_attn_fwd_noalloc";
  const size_t need = scree_attn_workspace_bytes(batch, total_tokens, head_dim);
  if (need > (size_t)SCREE_ATTN_NOALLOC_SCHEDULE_BYTES)
    return set_error(SCREE_ERR_UNSUPPORTED,
                     "%s: the schedule for batch %d, total_tokens %lld needs %zu bytes, more than "
                     "the %d-byte static scratch; use scree_attn_fwd with a workspace",
                     fn, batch, (long long)total_tokens, need, SCREE_ATTN_NOALLOC_SCHEDULE_BYTES);
  void* ws = nullptr;
  // validate everything before the first launch (a stand-in size: the
  // static array is checked against the schedule's need above)
  int rc = check_fwd(fn, q, k, v, o, lse, cu_seqlens, batch, total_tokens, heads, kv_heads,
                     head_dim, strides, dtype, reinterpret_cast<void*>(1),
                     SCREE_ATTN_NOALLOC_SCHEDULE_BYTES);
  if (rc) return rc;
  if (total_tokens == 0) return SCREE_OK;
  if ((rc = scratch_for_current_device(fn, &ws))) return rc;
  if (scree_attn_needs_schedule(batch, total_tokens, heads, head_dim)) {
    rc = scree_attn_schedule(cu_seqlens, batch, total_tokens, head_dim, causal, ws,
                             SCREE_ATTN_NOALLOC_SCHEDULE_BYTES, stream);
    if (rc) return rc;
  }
  return launch_fwd(fn, q, k, v, o, lse, cu_seqlens, batch, total_tokens, heads, kv_heads,
                    head_dim, strides, softmax_scale, causal, dtype, ws, stream);
}

extern "C" int scree_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                              const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                              int heads, int head_dim, const int64_t* strides, float softmax_scale,
                              int causal, int dtype, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return scree_attn_fwd_gqa(q, k, v, o, lse, cu_seqlens, batch, total_tokens, heads, heads,
                            head_dim, strides, softmax_scale, causal, dtype, workspace,
                            workspace_bytes, stream);
}

extern "C" int scree_attn_bwd_dq_gqa(const void* dout, const void* q, const void* k,
                                     const void* v, const void* o, const float* lse, void* dq,
                                     float* delta, const int32_t* cu_seqlens, int batch,
                                     int64_t total_tokens, int heads, int kv_heads, int head_dim,
                                     const int64_t* strides, float softmax_scale, int causal,
                                     int dtype, const void* workspace, size_t workspace_bytes,
                                     void* stream) {
  const char* fn = "scree_attn_bwd_dq";
  int rc = check_common(fn, cu_seqlens, batch, total_tokens, heads, head_dim, dtype, workspace,
                        workspace_bytes);
  if (rc) return rc;
  if ((rc = check_heads(fn, heads, kv_heads))) return rc;
  if (total_tokens > 0 && (!lse || !aligned16(lse)))
    return set_error(SCREE_ERR_INVALID, "%s: lse null or unaligned", fn);
  if (total_tokens > 0 && (!delta || !aligned16(delta)))
    return set_error(SCREE_ERR_INVALID, "%s: delta null or unaligned", fn);
  const char* names[6] = {"dout", "q", "k", "v", "o", "dq"};
  const void* ptrs[6] = {dout, q, k, v, o, dq};
  rc = check_bwd_tensors(fn, names, ptrs, 6, strides, heads, head_dim, total_tokens);
  if (rc) return rc;
  if (total_tokens == 0) return SCREE_OK;
  const int tmax = (int)tmax_for(batch, total_tokens);
  if (dtype == SCREE_DTYPE_F32)
    SCREE_DISPATCH_F32(launch_bwd_dq_f32, head_dim, causal, dout, q, k, v, o, lse, dq, delta,
                       heads, kv_heads, strides, softmax_scale, tmax, workspace,
                       (int)total_tokens, static_cast<hipStream_t>(stream));
  else
    SCREE_DISPATCH(launch_bwd_dq_t, dtype, head_dim, causal, dout, q, k, v, o, lse, dq, delta,
                   cu_seqlens, batch, heads, kv_heads, strides, softmax_scale, tmax, workspace,
                   (int)total_tokens, head_dim, static_cast<hipStream_t>(stream));
  return check_launch(fn);
}

extern "C" int scree_attn_bwd_dq(const void* dout, const void* q, const void* k, const void* v,
                                 const void* o, const float* lse, void* dq, float* delta,
                                 const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                                 int heads, int head_dim, const int64_t* strides,
                                 float softmax_scale, int causal, int dtype,
                                 const void* workspace, size_t workspace_bytes, void* stream) {
  return scree_attn_bwd_dq_gqa(dout, q, k, v, o, lse, dq, delta, cu_seqlens, batch, total_tokens,
                               heads, heads, head_dim, strides, softmax_scale, causal, dtype,
                               workspace, workspace_bytes, stream);
}

extern "C" int scree_attn_bwd_dkv_gqa(const void* dout, const void* q, const void* k,
                                      const void* v, const float* lse, const float* delta,
                                      void* dk, void* dv, const int32_t* cu_seqlens, int batch,
                                      int64_t total_tokens, int heads, int kv_heads,
                                      int head_dim, const int64_t* strides, float softmax_scale,
                                      int causal, int dtype, const void* workspace,
                                      size_t workspace_bytes, void* stream) {
  const char* fn = "scree_attn_bwd_dkv";
  int rc = check_common(fn, cu_seqlens, batch, total_tokens, heads, head_dim, dtype, workspace,
                        workspace_bytes);
  if (rc) return rc;
  if ((rc = check_heads(fn, heads, kv_heads))) return rc;
  if (total_tokens > 0 && (!lse || !aligned16(lse)))
    return set_error(SCREE_ERR_INVALID, "%s: lse null or unaligned", fn);
  if (total_tokens > 0 && (!delta || !aligned16(delta)))
    return set_error(SCREE_ERR_INVALID, "%s: delta null or unaligned", fn);
  const char* names[6] = {"dout", "q", "k", "v", "dk", "dv"};
  const void* ptrs[6] = {dout, q, k, v, dk, dv};
  rc = check_bwd_tensors(fn, names, ptrs, 6, strides, heads, head_dim, total_tokens);
  if (rc) return rc;
  if (total_tokens == 0) return SCREE_OK;
  const int tmax = (int)tmax_for(batch, total_tokens);
  if (dtype == SCREE_DTYPE_F32) {  // one workgroup per (item, K/V head), no split
    SCREE_DISPATCH_F32(launch_bwd_dkv_f32, head_dim, causal, dout, q, k, v, lse, delta, dk, dv,
                       heads, kv_heads, strides, softmax_scale, tmax, workspace,
                       (int)total_tokens, static_cast<hipStream_t>(stream));
    return check_launch(fn);
  }
  // Split the head groups only when the caller's workspace has room for it
  // (scree_attn_bwd_workspace_bytes_gqa); otherwise one part per group.
  int gsplit = dkv_gsplit(tmax, kv_heads, heads / kv_heads);
  const size_t base = align256(scree_attn_workspace_bytes(batch, total_tokens, head_dim));
  if (gsplit > 1 && workspace_bytes < base + dkv_split_bytes(tmax, kv_heads, gsplit, head_dim))
    gsplit = 1;
  float* partial = gsplit > 1 ? reinterpret_cast<float*>(
                                    static_cast<char*>(const_cast<void*>(workspace)) + base)
                              : nullptr;
  SCREE_DISPATCH(launch_bwd_dkv_t, dtype, head_dim, causal, dout, q, k, v, lse, delta, dk, dv,
                 cu_seqlens, batch, heads, kv_heads, strides, softmax_scale, tmax, workspace, gsplit,
                 partial, (int)total_tokens, head_dim, static_cast<hipStream_t>(stream));
  return check_launch(fn);
}

extern "C" size_t scree_attn_bwd_workspace_bytes_gqa(int batch, int64_t total_tokens, int heads,
                                                     int kv_heads, int head_dim) {
  const size_t base = scree_attn_workspace_bytes(batch, total_tokens, head_dim);
  if (!base || kv_heads < 1 || heads < kv_heads || heads % kv_heads ||
      !head_dim_supported(head_dim))
    return base;
  const int64_t tmax = tmax_for(batch, total_tokens);
  const int gsplit = dkv_gsplit(tmax, kv_heads, heads / kv_heads);
  if (gsplit < 2) return base;
  return align256(base) + dkv_split_bytes(tmax, kv_heads, gsplit, head_dim);
}

extern "C" int scree_attn_bwd_dkv(const void* dout, const void* q, const void* k, const void* v,
                                  const float* lse, const float* delta, void* dk, void* dv,
                                  const int32_t* cu_seqlens, int batch, int64_t total_tokens,
                                  int heads, int head_dim, const int64_t* strides,
                                  float softmax_scale, int causal, int dtype,
                                  const void* workspace, size_t workspace_bytes, void* stream) {
  return scree_attn_bwd_dkv_gqa(dout, q, k, v, lse, delta, dk, dv, cu_seqlens, batch,
                                total_tokens, heads, heads, head_dim, strides, softmax_scale,
                                causal, dtype, workspace, workspace_bytes, stream);
}

extern "C" int scree_attn_bwd_gqa(const void* dout, const void* q, const void* k, const void* v,
                                  const void* o, const float* lse, void* dq, void* dk, void* dv,
                                  float* delta, const int32_t* cu_seqlens, int batch,
                                  int64_t total_tokens, int heads, int kv_heads, int head_dim,
                                  const int64_t* strides, float softmax_scale, int causal,
                                  int dtype, const void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (!strides) return set_error(SCREE_ERR_INVALID, "scree_attn_bwd: strides is null");
  // strides: {dout, q, k, v, o, dq, dk, dv} x {row, head}
  const int64_t sdq[12] = {strides[0], strides[1], strides[2], strides[3], strides[4], strides[5],
                           strides[6], strides[7], strides[8], strides[9], strides[10], strides[11]};
  const int64_t sdkv[12] = {strides[0], strides[1], strides[2],  strides[3],  strides[4],  strides[5],
                            strides[6], strides[7], strides[12], strides[13], strides[14], strides[15]};
  int rc = scree_attn_bwd_dq_gqa(dout, q, k, v, o, lse, dq, delta, cu_seqlens, batch,
                                 total_tokens, heads, kv_heads, head_dim, sdq, softmax_scale,
                                 causal, dtype, workspace, workspace_bytes, stream);
  if (rc) return rc;
  return scree_attn_bwd_dkv_gqa(dout, q, k, v, lse, delta, dk, dv, cu_seqlens, batch,
                                total_tokens, heads, kv_heads, head_dim, sdkv, softmax_scale,
                                causal, dtype, workspace, workspace_bytes, stream);
}

extern "C" int scree_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                              const void* o, const float* lse, void* dq, void* dk, void* dv,
                              float* delta, const int32_t* cu_seqlens, int batch,
                              int64_t total_tokens, int heads, int head_dim,
                              const int64_t* strides, float softmax_scale, int causal, int dtype,
                              const void* workspace, size_t workspace_bytes, void* stream) {
  return scree_attn_bwd_gqa(dout, q, k, v, o, lse, dq, dk, dv, delta, cu_seqlens, batch,
                            total_tokens, heads, heads, head_dim, strides, softmax_scale, causal,
                            dtype, workspace, workspace_bytes, stream);
}
