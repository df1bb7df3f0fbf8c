// segment_reduce kernels (included once per dtype).
//
//   out[s] = red over the value rows offsets[s] .. offsets[s+1], in row order
//
// Segments are contiguous row ranges of one value block, so the work is a
// streaming read. Three kernels share it:
//
//  * seg_stage_kernel, rows of at most 32 lane vectors (16-byte chunks, or
//    elements when the width or the alignment does not allow them): a
//    wavefront owns P = 64 / G consecutive segments, G lanes each (G = the
//    power of two covering the row's vectors). It reads their rows as one
//    contiguous span, a window of 8 KB at a time, with every lane loading
//    consecutive 16-byte chunks (so each load instruction is one coalesced
//    1 KB read), stages the window in LDS and lets each lane group fold its
//    own segment's rows from there. The next window is in registers while
//    the current one is folded. Windows skip the rows of segments this
//    kernel does not reduce.
//  * seg_wide_kernel, wider rows: one wavefront per segment and 64-vector
//    slab of the row, each row read coalesced across the lanes, U rows in
//    flight.
//  * seg_split_kernel, segments longer than SEG_SPLIT_ROWS (unless the caller
//    states there are none): a workgroup per long segment; its threads are
//    row streams (rows j, j + rs, j + 2 rs, ...) times column vectors, whose
//    partials are combined in stream order through LDS.
//
// Fold order. The first two kernels fold each segment's rows one after the
// other in row order, exactly the reference's sequential fold
// (src/ported.mojo:559-647), so sum, mean, max and min are bit-identical to
// the CPU kernel in the same precision. The split kernel changes the order
// of a long segment's sum (within the rounding of the float64 tolerance);
// max and min stay exact, with the arg the first row reaching the value
// (strict comparison, the smaller row wins ties when partials combine, NaN
// never selected; -1 when no row was selected or the value was replaced
// by 0).
//
// Offsets are clamped into [0, n] and a negative length reads as empty, so
// no access leaves the value block whatever the offsets hold.
#pragma once

#include "mdgl_kernels.h"

namespace mdgl {

constexpr int SEG_WB = 8192;  // LDS bytes of one wavefront's row window
constexpr int SEG_U = 4;      // rows in flight per lane (wide and split kernels)

template <class T>
struct SegArgs {
  const int32_t* off;
  const T* val;
  T* out;
  int32_t* arg;
  int64_t S, n, d;
  int nvec, G, P, flags;
  int skip_long;  // segments longer than SEG_SPLIT_ROWS are left to seg_split_kernel
  int out_vec;    // 16-byte output stores
  int64_t slabs;  // wide kernel: 64-vector slabs per row
  int64_t spb;    // split kernel: segments scanned per workgroup
  int max_rows;   // softmax: segments of more rows are not written (0: none skipped)
};

__device__ __forceinline__ int wave_min_int(int v) {
  for (int off = 32; off >= 1; off >>= 1) {
    int o = __shfl_xor(v, off);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The row range of segment s, clamped into [0, n].
__device__ __forceinline__ void seg_range(const int32_t* __restrict__ off, int64_t s, int64_t n,
                                          int& lo, int& hi) {
  int64_t a = off[s], b = off[s + 1];
  a = a < 0 ? 0 : (a > n ? n : a);
  b = b < a ? a : (b > n ? n : b);
  lo = (int)a;
  hi = (int)b;
}

template <class T, int RED, int VEC, bool ARG>
__device__ __forceinline__ void seg_combine(T (&acc)[VEC], int (&ag)[VEC], const T (&x)[VEC],
                                            int row) {
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    if constexpr (RED == RED_MAX) {
      if (x[v] > acc[v]) { acc[v] = x[v]; if constexpr (ARG) ag[v] = row; }
    } else if constexpr (RED == RED_MIN) {
      if (x[v] < acc[v]) { acc[v] = x[v]; if constexpr (ARG) ag[v] = row; }
    } else {
      acc[v] = acc[v] + x[v];
    }
  }
}

// Mean divide, +-inf -> 0, and the stores of one lane's VEC columns
// starting at column k0 of segment s.
template <class T, int RED, int VEC, bool ARG>
__device__ __forceinline__ void seg_store(const SegArgs<T>& a, int64_t s, int64_t k0, int len,
                                          T (&acc)[VEC], int (&ag)[VEC]) {
  if ((a.flags & F_MEAN) && len > 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = acc[v] / T(len);
  }
  if (a.flags & F_REPLACE_INF) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (is_inf(acc[v])) {
        acc[v] = T(0);  // a replaced value has no row behind it
        ag[v] = -1;
      }
  }
  const int64_t o = s * a.d + k0;
  if (VEC > 1 && a.out_vec && k0 + VEC <= a.d) {
    if constexpr (VEC > 1) store_n<T, VEC>(a.out + o, acc);
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (k0 + v < a.d) a.out[o + v] = acc[v];
  }
  if constexpr (ARG) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (k0 + v < a.d) a.arg[o + v] = ag[v];
  }
}

template <class T, int RED, int VEC, bool ARG>
__global__ __launch_bounds__(BLOCK) void seg_stage_kernel(SegArgs<T> a) {
  constexpr int CH = SEG_WB / (VEC * (int)sizeof(T));  // chunks per window
  constexpr int PER = CH / WAVE;                       // chunk loads per lane per window
  __shared__ __align__(16) T buf[WAVES_PER_BLOCK][SEG_WB / sizeof(T)];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_BLOCK + w;
  const int64_t s0 = wave * a.P;
  if (s0 >= a.S) return;  // uniform per wavefront
  const int grp = lane / a.G, gl = lane % a.G;
  const int64_t seg = s0 + grp;
  const bool live = seg < a.S;
  int lo = 0, hi = 0;
  if (live) seg_range(a.off, seg, a.n, lo, hi);
  const int len = hi - lo;
  const bool mine = live && !(a.skip_long && len > SEG_SPLIT_ROWS);
  if (!mine) hi = lo;  // reduced elsewhere (or no segment): no rows needed here
  const bool col = gl < a.nvec;
  const int WR = CH / a.nvec;  // rows per window
  const int rend = wave_max_int(hi > lo ? hi : 0);

  T acc[VEC];
  int ag[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    acc[v] = seed<T>(RED);
    ag[v] = -1;  // nothing selected yet
  }
  T st[PER][VEC];
  // the window of rows [w0, w0 + WR) (clipped at rend) as chunks into st
  auto fetch = [&](int w0) {
    const int64_t e0 = (int64_t)w0 * a.d;
    const int r1 = w0 + WR < rend ? w0 + WR : rend;
    const int64_t e1 = (int64_t)r1 * a.d;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t e = e0 + (int64_t)(lane + i * WAVE) * VEC;
      if (e < e1) {
        if constexpr (VEC > 1) load_n_stream<T, VEC>(a.val + e, st[i]);
        else st[i][0] = __builtin_nontemporal_load(a.val + e);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) st[i][v] = T(0);
      }
    }
  };
  int W = wave_min_int(hi > lo ? lo : 0x7fffffff);
  if (W != 0x7fffffff) fetch(W);
  while (W != 0x7fffffff) {  // uniform per wavefront
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if constexpr (VEC > 1) store_n<T, VEC>(&buf[w][(lane + i * WAVE) * VEC], st[i]);
      else buf[w][lane + i * WAVE] = st[i][0];
    }
    wave_sync_lds();
    const int wend = W + WR;
    const int nxt = wave_min_int(hi > wend ? (lo > wend ? lo : wend) : 0x7fffffff);
    if (nxt != 0x7fffffff) fetch(nxt);
    if (col) {
      const int r0 = lo > W ? lo : W;
      const int r1 = hi < wend ? hi : wend;
      for (int r = r0; r < r1; ++r) {
        T x[VEC];
        const int c = ((r - W) * a.nvec + gl) * VEC;
        if constexpr (VEC > 1) load_n<T, VEC>(&buf[w][c], x);
        else x[0] = buf[w][c];
        seg_combine<T, RED, VEC, ARG>(acc, ag, x, r);
      }
    }
    wave_sync_lds();
    W = nxt;
  }
  if (mine && col) seg_store<T, RED, VEC, ARG>(a, seg, (int64_t)gl * VEC, len, acc, ag);
}

template <class T, int RED, int VEC, bool ARG>
__global__ __launch_bounds__(BLOCK) void seg_wide_kernel(SegArgs<T> a) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
  if (wave >= a.S * a.slabs) return;
  const int64_t seg = wave / a.slabs, slab = wave % a.slabs;
  int lo, hi;
  seg_range(a.off, seg, a.n, lo, hi);
  const int len = hi - lo;
  if (a.skip_long && len > SEG_SPLIT_ROWS) return;  // seg_split_kernel's
  const int64_t q = slab * WAVE + lane;  // this lane's vector of the row
  const bool col = q < a.nvec;
  T acc[VEC];
  int ag[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    acc[v] = seed<T>(RED);
    ag[v] = -1;  // nothing selected yet
  }
  if (col) {
    const T* p = a.val + (int64_t)lo * a.d + q * VEC;
    for (int r = lo; r < hi; r += SEG_U) {
      T x[SEG_U][VEC];
#pragma unroll
      for (int u = 0; u < SEG_U; ++u) {
        if (r + u < hi) {
          if constexpr (VEC > 1) load_n_stream<T, VEC>(p + (int64_t)u * a.d, x[u]);
          else x[u][0] = __builtin_nontemporal_load(p + (int64_t)u * a.d);
        }
      }
#pragma unroll
      for (int u = 0; u < SEG_U; ++u)
        if (r + u < hi) seg_combine<T, RED, VEC, ARG>(acc, ag, x[u], r + u);
      p += (int64_t)SEG_U * a.d;
    }
    seg_store<T, RED, VEC, ARG>(a, seg, q * VEC, len, acc, ag);
  }
}

template <class T, int RED, int VEC, bool ARG>
__global__ __launch_bounds__(BLOCK) void seg_split_kernel(SegArgs<T> a) {
  __shared__ __align__(16) T pval[BLOCK][VEC];
  __shared__ int parg[BLOCK][VEC];
  __shared__ int list[BLOCK];
  __shared__ int nlist;
  const int t = threadIdx.x;
  const int64_t first = (int64_t)blockIdx.x * a.spb;
  const int64_t last = first + a.spb < a.S ? first + a.spb : a.S;
  const int cols = a.nvec < BLOCK ? a.nvec : BLOCK;
  const int rs = BLOCK / cols;  // row streams
  const int64_t slabs = (a.nvec + cols - 1) / cols;
  for (int64_t base = first; base < last; base += BLOCK) {
    // the long segments among the next BLOCK, in any order (each is reduced
    // on its own, so the order does not change any result)
    if (t == 0) nlist = 0;
    __syncthreads();
    if (base + t < last) {
      int lo, hi;
      seg_range(a.off, base + t, a.n, lo, hi);
      if (hi - lo > SEG_SPLIT_ROWS) list[atomicAdd(&nlist, 1)] = (int)(base + t - first);
    }
    __syncthreads();
    const int count = nlist;
    for (int li = 0; li < count; ++li) {
      const int64_t seg = first + list[li];
      int lo, hi;
      seg_range(a.off, seg, a.n, lo, hi);
      for (int64_t slab = 0; slab < slabs; ++slab) {
        const int j = t / cols;
        const int64_t q = slab * cols + t % cols;
        const bool act = j < rs && q < a.nvec;
        T acc[VEC];
        int ag[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          acc[v] = seed<T>(RED);
          ag[v] = -1;  // nothing selected yet
        }
        if (act) {
          for (int r = lo + j; r < hi; r += SEG_U * rs) {
            T x[SEG_U][VEC];
#pragma unroll
            for (int u = 0; u < SEG_U; ++u) {
              const int rr = r + u * rs;
              if (rr < hi) {
                const T* p = a.val + (int64_t)rr * a.d + q * VEC;
                if constexpr (VEC > 1) load_n_stream<T, VEC>(p, x[u]);
                else x[u][0] = __builtin_nontemporal_load(p);
              }
            }
#pragma unroll
            for (int u = 0; u < SEG_U; ++u)
              if (r + u * rs < hi) seg_combine<T, RED, VEC, ARG>(acc, ag, x[u], r + u * rs);
          }
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          pval[t][v] = acc[v];
          parg[t][v] = ag[v];
        }
        __syncthreads();
        if (t < cols && q < a.nvec) {
          T res[VEC];
          int rag[VEC];
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            res[v] = seed<T>(RED);
            rag[v] = -1;
          }
          for (int jj = 0; jj < rs; ++jj) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
              const T p = pval[jj * cols + t][v];
              const int pa = parg[jj * cols + t][v];
              if constexpr (RED == RED_MAX) {
                if (p > res[v] || (p == res[v] && pa < rag[v])) { res[v] = p; rag[v] = pa; }
              } else if constexpr (RED == RED_MIN) {
                if (p < res[v] || (p == res[v] && pa < rag[v])) { res[v] = p; rag[v] = pa; }
              } else {
                res[v] = res[v] + p;
              }
            }
          }
          seg_store<T, RED, VEC, ARG>(a, seg, q * VEC, hi - lo, res, rag);
        }
        __syncthreads();
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- segment_softmax
// Per segment and column: m = max, e = exp(x - m), s = sum of e in row order,
// out = e / s (the reference's three passes, src/ported.mojo:679-768), for
// rows of at most 32 lane vectors. A wavefront owns P = 64 / G consecutive
// segments, G lanes each. A window is a run of whole segments of at most WR
// rows (8 KB): it is read with coalesced 16-byte loads into LDS; each lane
// group takes its segment's max (and records which rows are its own); then
// all 64 lanes turn the window's values into e in place, each lane group
// sums its segment's e in row order, and all lanes write e times the
// reciprocal of s with coalesced stores. The next window is in registers meanwhile. A segment
// longer than a window (which the caller's plan only hands over as chunks,
// so it does not reach this kernel) would be streamed by its lane group.
__device__ __forceinline__ float seg_exp(float x) { return expf(x); }
__device__ __forceinline__ double seg_exp(double x) { return exp(x); }

// One lane's VEC columns of a row (VEC > 1: aligned 16-byte access).
template <class T, int VEC>
__device__ __forceinline__ void seg_load_cols(const T* p, T (&x)[VEC]) {
  if constexpr (VEC > 1) load_n<T, VEC>(p, x);
  else x[0] = *p;
}
template <class T, int VEC>
__device__ __forceinline__ void seg_store_cols(T* p, const T (&x)[VEC]) {
  if constexpr (VEC > 1) store_n<T, VEC>(p, x);
  else *p = x[0];
}

template <class T, int VEC>
__global__ __launch_bounds__(BLOCK) void seg_softmax_stage_kernel(SegArgs<T> a) {
  constexpr int CH = SEG_WB / (VEC * (int)sizeof(T));  // chunks per window
  constexpr int PER = CH / WAVE;
  constexpr int SV = WAVE * 16 / (int)sizeof(T);       // m / s entries: P * nvec * VEC <= SV
  __shared__ __align__(16) T buf[WAVES_PER_BLOCK][SEG_WB / sizeof(T)];
  // per segment and column: the maximum (passes 1-2), then 1 / sum (3-4);
  // one array, so four workgroups fit a CU
  __shared__ __align__(16) T mx[WAVES_PER_BLOCK][SV];
  __shared__ unsigned char owner[WAVES_PER_BLOCK][CH];  // lane group of each window row
  constexpr unsigned char NO_OWNER = 0xff;              // lane groups are 0 .. 63
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_BLOCK + w;
  const int64_t s0 = wave * a.P;
  if (s0 >= a.S) return;  // uniform per wavefront
  const int grp = lane / a.G, gl = lane % a.G;
  const int64_t seg = s0 + grp;
  int lo = 0, hi = 0;
  if (seg < a.S) seg_range(a.off, seg, a.n, lo, hi);
  const bool col = gl < a.nvec;
  const int64_t k0 = (int64_t)gl * VEC;
  const int nv = a.nvec;
  const int WR = CH / nv;
  const int mslot = (grp * nv + gl) * VEC;  // this lane's m / s entries
  // empty segments (and lanes past the last segment) write nothing, nor do
  // segments over the row limit (the caller serves them another way)
  const bool skipped = a.max_rows > 0 && hi - lo > a.max_rows;
  bool done = hi <= lo || skipped;

  // window [w0, e0): w0 the first row of the first unfinished segment, e0
  // the end of the last unfinished segment that ends within w0 + WR (w0
  // when even the first does not fit); with a row limit it also stops at
  // the first skipped segment, whose rows it must not write
  auto window = [&](bool dn, int& w0, int& e0) {
    w0 = wave_min_int(dn ? 0x7fffffff : lo);
    if (w0 == 0x7fffffff) {
      e0 = w0;
      return;
    }
    int lim = w0 + WR;
    if (a.max_rows > 0) {
      const int sk = wave_min_int(skipped && lo >= w0 ? lo : 0x7fffffff);
      lim = sk < lim ? sk : lim;
    }
    e0 = wave_max_int(!dn && hi <= lim ? hi : w0);
  };
  T st[PER][VEC];
  auto fetch = [&](int w0, int e0) {
    const int64_t b0 = (int64_t)w0 * a.d, b1 = (int64_t)e0 * a.d;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t e = b0 + (int64_t)(lane + i * WAVE) * VEC;
      if (e < b1) {
        if constexpr (VEC > 1) load_n_stream<T, VEC>(a.val + e, st[i]);
        else st[i][0] = __builtin_nontemporal_load(a.val + e);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) st[i][v] = T(0);
      }
    }
  };
  int W, E;
  window(done, W, E);
  if (E > W) fetch(W, E);
  while (W != 0x7fffffff) {  // uniform per wavefront
    if (E > W) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if constexpr (VEC > 1) store_n<T, VEC>(&buf[w][(lane + i * WAVE) * VEC], st[i]);
        else buf[w][lane + i * WAVE] = st[i][0];
      }
      // rows of the window start unowned; offsets that run backwards can
      // leave rows inside [W, E) that no segment of this window claims, and
      // passes 2 and 4 skip those rows
      for (int r = lane; r < E - W; r += WAVE) owner[w][r] = NO_OWNER;
      wave_sync_lds();
      const bool mine = !done && lo >= W && hi <= E;
      int Wn, En;
      window(done || mine, Wn, En);
      if (En > Wn) fetch(Wn, En);
      const int nch = (E - W) * nv;  // chunks of this window
      const int base = ((lo - W) * nv + gl) * VEC, step = nv * VEC;
      // 1. max per segment and column, in the group; the group's first lane
      //    marks the rows it owns
      if (mine && col) {
        T m[VEC], x[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) m[v] = -__builtin_huge_val();
        for (int r = lo, c = base; r < hi; ++r, c += step) {
          if constexpr (VEC > 1) load_n<T, VEC>(&buf[w][c], x);
          else x[0] = buf[w][c];
#pragma unroll
          for (int v = 0; v < VEC; ++v) m[v] = x[v] > m[v] ? x[v] : m[v];
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v) mx[w][mslot + v] = m[v];
        if (gl == 0)
          for (int r = lo; r < hi; ++r) owner[w][r - W] = (unsigned char)grp;
      }
      wave_sync_lds();
      // 2. e = exp(x - m) over the whole window, every lane, in place
#pragma unroll 2
      for (int i = 0; i < PER; ++i) {
        const int c = lane + i * WAVE;
        const int r = c / nv, q = c - r * nv;
        if (c < nch && owner[w][r] != NO_OWNER) {
          const int ms = (owner[w][r] * nv + q) * VEC;
          T x[VEC];
          if constexpr (VEC > 1) load_n<T, VEC>(&buf[w][c * VEC], x);
          else x[0] = buf[w][c];
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = seg_exp(x[v] - mx[w][ms + v]);
          if constexpr (VEC > 1) store_n<T, VEC>(&buf[w][c * VEC], x);
          else buf[w][c] = x[0];
        }
      }
      wave_sync_lds();
      // 3. s = sum of e per segment and column, in row order, in the group
      if (mine && col) {
        T su[VEC], x[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) su[v] = T(0);
        for (int r = lo, c = base; r < hi; ++r, c += step) {
          if constexpr (VEC > 1) load_n<T, VEC>(&buf[w][c], x);
          else x[0] = buf[w][c];
#pragma unroll
          for (int v = 0; v < VEC; ++v) su[v] = su[v] + x[v];
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v) mx[w][mslot + v] = T(1) / su[v];
      }
      wave_sync_lds();
      // 4. out = e * (1 / s) over the whole window, every lane, coalesced
      //    stores (one correctly rounded reciprocal per segment and column
      //    instead of a divide per value: within two roundings of e / s)
      const int64_t b0 = (int64_t)W * a.d;
#pragma unroll 2
      for (int i = 0; i < PER; ++i) {
        const int c = lane + i * WAVE;
        const int r = c / nv, q = c - r * nv;
        if (c < nch && owner[w][r] != NO_OWNER) {
          const int ms = (owner[w][r] * nv + q) * VEC;
          T y[VEC];
          if constexpr (VEC > 1) load_n<T, VEC>(&buf[w][c * VEC], y);
          else y[0] = buf[w][c];
#pragma unroll
          for (int v = 0; v < VEC; ++v) y[v] = y[v] * mx[w][ms + v];
          if constexpr (VEC > 1) store_n_stream<T, VEC>(a.out + b0 + (int64_t)c * VEC, y);
          else a.out[b0 + c] = y[0];
        }
      }
      wave_sync_lds();
      done = done || mine;
      W = Wn;
      E = En;
    } else {
      // the first unfinished segment is longer than a window: its group
      // streams it from memory, three passes
      const bool mine = !done && lo == W;
      if (mine && col) {
        T m[VEC], su[VEC], x[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          m[v] = -__builtin_huge_val();
          su[v] = T(0);
        }
        for (int r = lo; r < hi; ++r) {
          seg_load_cols<T, VEC>(a.val + (int64_t)r * a.d + k0, x);
#pragma unroll
          for (int v = 0; v < VEC; ++v) m[v] = x[v] > m[v] ? x[v] : m[v];
        }
        for (int r = lo; r < hi; ++r) {
          seg_load_cols<T, VEC>(a.val + (int64_t)r * a.d + k0, x);
#pragma unroll
          for (int v = 0; v < VEC; ++v) su[v] = su[v] + seg_exp(x[v] - m[v]);
        }
        for (int r = lo; r < hi; ++r) {
          seg_load_cols<T, VEC>(a.val + (int64_t)r * a.d + k0, x);
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = seg_exp(x[v] - m[v]) / su[v];
          seg_store_cols<T, VEC>(a.out + (int64_t)r * a.d + k0, x);
        }
      }
      done = done || mine;
      window(done, W, E);
      if (E > W) fetch(W, E);
    }
  }
}

template <class T, int RED, int VEC, bool ARG>
hipError_t launch_seg(SegArgs<T> a, int passes, hipStream_t st) {
  const bool stage = a.nvec <= 32;
  if (!(passes & SEG_PASS_ROWS)) {
    // the split pass alone
  } else if (stage) {
    int G = 1;
    while (G < a.nvec) G <<= 1;
    a.G = G;
    a.P = WAVE / G;
    const int64_t waves = (a.S + a.P - 1) / a.P;
    const int64_t blocks = (waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    hipLaunchKernelGGL((seg_stage_kernel<T, RED, VEC, ARG>), dim3((unsigned)blocks), dim3(BLOCK), 0,
                       st, a);
  } else {
    a.slabs = (a.nvec + WAVE - 1) / WAVE;
    const int64_t waves = a.S * a.slabs;
    const int64_t blocks = (waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    hipLaunchKernelGGL((seg_wide_kernel<T, RED, VEC, ARG>), dim3((unsigned)blocks), dim3(BLOCK), 0,
                       st, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !a.skip_long || !(passes & SEG_PASS_SPLIT)) return e;
  int64_t blocks = 2048;
  if (blocks > a.S) blocks = a.S;
  a.spb = (a.S + blocks - 1) / blocks;
  blocks = (a.S + a.spb - 1) / a.spb;
  hipLaunchKernelGGL((seg_split_kernel<T, RED, VEC, ARG>), dim3((unsigned)blocks), dim3(BLOCK), 0,
                     st, a);
  return hipGetLastError();
}

template <class T, int RED, bool ARG>
hipError_t launch_seg_vec(const SegmentParams& p) {
  SegArgs<T> a{};
  a.off = p.offsets;
  a.val = static_cast<const T*>(p.value);
  a.out = static_cast<T*>(p.out);
  a.arg = p.arg;
  a.S = p.num_seg;
  a.n = p.n;
  a.d = p.d;
  a.flags = p.flags;
  a.skip_long = p.skip_long;
  constexpr int V = 16 / sizeof(T);
  const bool vec = p.d % V == 0 && aligned16(p.value);
  a.out_vec = vec && aligned16(p.out);
  if (vec) {
    a.nvec = (int)((p.d / V) < 0x7fffffff ? p.d / V : 0x7fffffff);
    return launch_seg<T, RED, V, ARG>(a, p.passes, p.stream);
  }
  a.nvec = (int)(p.d < 0x7fffffff ? p.d : 0x7fffffff);
  return launch_seg<T, RED, 1, ARG>(a, p.passes, p.stream);
}

template <class T>
hipError_t launch_segment_reduce(const SegmentParams& p) {
  if (p.num_seg <= 0 || p.d <= 0) return hipSuccess;
  const bool arg = p.arg != nullptr;
  switch (p.red) {
    case RED_MAX: return arg ? launch_seg_vec<T, RED_MAX, true>(p) : launch_seg_vec<T, RED_MAX, false>(p);
    case RED_MIN: return arg ? launch_seg_vec<T, RED_MIN, true>(p) : launch_seg_vec<T, RED_MIN, false>(p);
    default: return launch_seg_vec<T, RED_SUM, false>(p);
  }
}

// segment_softmax through seg_softmax_stage_kernel; hipErrorNotSupported
// when the rows are wider than 32 lane vectors (the caller then takes the
// CSR softmax kernel).
template <class T>
hipError_t launch_segment_softmax_stage(const int32_t* offsets, const void* value, void* out,
                                        int64_t num_seg, int64_t n, int64_t d, int64_t max_rows,
                                        hipStream_t st) {
  if (num_seg <= 0 || d <= 0 || n <= 0) return hipSuccess;
  constexpr int V = 16 / sizeof(T);
  const bool vec = d % V == 0 && aligned16(value) && aligned16(out);
  const int64_t nvec = vec ? d / V : d;
  if (nvec > 32) return hipErrorNotSupported;
  SegArgs<T> a{};
  a.off = offsets;
  a.val = static_cast<const T*>(value);
  a.out = static_cast<T*>(out);
  a.S = num_seg;
  a.n = n;
  a.d = d;
  a.nvec = (int)nvec;
  a.max_rows = max_rows > 0 && max_rows < n ? (int)max_rows : 0;
  int G = 1;
  while (G < a.nvec) G <<= 1;
  a.G = G;
  a.P = WAVE / G;
  const int64_t waves = (num_seg + a.P - 1) / a.P;
  const dim3 grid((unsigned)((waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK)), block(BLOCK);
  if (vec)
    hipLaunchKernelGGL((seg_softmax_stage_kernel<T, V>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((seg_softmax_stage_kernel<T, 1>), grid, block, 0, st, a);
  return hipGetLastError();
}

}  // namespace mdgl

#define MDGL_INSTANTIATE_SEGMENT(T)                                                         \
  template hipError_t mdgl::launch_segment_reduce<T>(const mdgl::SegmentParams&);          \
  template hipError_t mdgl::launch_segment_softmax_stage<T>(const int32_t*, const void*, void*, \
                                                            int64_t, int64_t, int64_t,      \
                                                            int64_t, hipStream_t);
