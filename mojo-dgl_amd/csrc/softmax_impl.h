// Row softmax over a CSR (included once per dtype). edge_softmax uses the
// in- or out-edge CSR with the edge id of every slot; segment_softmax uses
// the segment offsets with the identity edge id.
//
// For each row and each of the d columns: m = max over the row's selected
// edges, s = sum of exp(x - m), out = exp(x - m) / s -- the reference's three
// passes (src/ported.mojo:918-987, 679-768) -- but every logit is read from
// memory once: a row's values stay in registers from the max to the write.
// Only the order of the max and of the sum differs from the reference (lanes
// combine by __shfl_xor butterflies), so results agree to rounding.
//
// Lane layout. L lanes (a power of two, at most 64) cover the d columns, VEC
// per lane; a wavefront holds Pw = 64 / L edge slots; rows wider than 64 * VEC
// are cut into slabs, one wavefront per slab. Rows are served by degree:
//   * packed: rows sorted by degree; a row of at most 2^k edges gets 2^k slots
//     (one edge each), so a wavefront takes Pw / 2^k rows of one degree bin;
//   * wavefront rows: up to CPL * Pw edges, CPL per slot; in natural order
//     (no row order) R consecutive rows share a wavefront, Pw / R slots each,
//     when they fit (R from the mean degree);
//   * chunked rows (longer): chunks of CPL * Pw edges; launch 1 writes each
//     chunk's (max, sum of exp(x - max)) per column, launch 2 merges a row's
//     chunks (M = max m_c, S = sum s_c * exp(m_c - M); slot s of the wavefront
//     folds chunks s, s + Pw, ... in chunk order, the slots then combine by
//     butterflies) and writes exp(x - M) / S over the chunk.
// A packed row's slots find their edge ids in the plan's packed edge list
// when there is one (one load), else through order -> indptr -> eid.
// Launch 1 takes the chunks (their workgroups first, so the long rows start
// early) and the wavefront rows; the packed rows run in a launch of their
// own, whose kernel needs far fewer registers, each wavefront serving
// PK_U packed wavefronts' rows with its dependent loads interleaved.
//
// Two-pass form (edge_softmax with a slot-of-edge array): a random 32-byte
// write per edge costs more than the rest of the op, so the row pass then
// only writes each row's (max, sum) to a table tab[slot][2][d], and an
// edge-parallel pass in edge-id order writes out[e] = exp(x - max) / sum with
// coalesced loads and stores, reading the table row of the edge's slot. With
// a row order a row's slot is its position in the order (chunked rows follow,
// at hub_base + their first chunk), so the rows of a wavefront write
// consecutive table rows; without one the slot is the row. The values are the
// ones the one-pass form writes.
#pragma once

#include "mdgl_kernels.h"

namespace mdgl {

enum { SM_FULL = 0, SM_STATS = 1, SM_WRITE = 2 };

template <class T>
struct SoftmaxArgs {
  const int32_t* indptr;
  const int32_t* eid;
  const int8_t* mask;
  const T* logits;
  T* out;
  int64_t num_rows, d;
  int L, Pw, S, vec_io, nbins;
  const int32_t* order;          // rows sorted by degree, or null (natural order)
  int64_t bin_start[8];          // packed bin k (2^k slots): order[bin_start[k] .. bin_start[k+1])
  int64_t bin_wave[9];           // wavefronts before bin k (slabs included)
  const int32_t* peid;           // packed edge ids, or null
  int64_t bin_slot[8];           // entries of peid before bin k
  int64_t mid_start, mid_end;    // wavefront rows: order[mid_start .. mid_end) or all rows
  int nat_r;                     // rows sharing a wavefront in natural order (else 1)
  int64_t num_chunks;
  const int32_t* chunk_row;
  const int32_t* chunk_start;
  const int32_t* chunk_first;    // first chunk of the same row
  int chunk_len;
  T* pm;  // [num_chunks][d] chunk maxima
  T* ps;  // [num_chunks][d] chunk sums of exp(x - max)
  int64_t chunk_waves, chunk_blocks, light_waves, light_blocks;
  int mode2;  // launch 2: the chunk write pass
  T* tab;     // two-pass form: [slots][2][d] (max, sum), else null
  int64_t hub_base;  // table slot of the first chunked row (ordered plans)
  int row_slots;     // table slot = row id (else the order position / hub slot)
  const SoftDyn* dyn;  // device plan: figures in device memory (DYN kernels)
};

__device__ __forceinline__ float exp_t(float x) { return expf(x); }
__device__ __forceinline__ double exp_t(double x) { return exp(x); }

template <class T, int VEC>
__device__ __forceinline__ void load_cols(const T* __restrict__ p, int64_t k0, int64_t d, bool vec_io,
                                          T (&x)[VEC]) {
  if (VEC > 1 && vec_io) {
    if constexpr (VEC == VecOf<T>::n) load_vec<T>(p + k0, x);
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = (k0 + v < d) ? p[k0 + v] : T(0);
  }
}

template <class T, int VEC>
__device__ __forceinline__ void store_cols(T* __restrict__ p, int64_t k0, int64_t d, bool vec_io,
                                           const T (&x)[VEC]) {
  if (VEC > 1 && vec_io) {
    if constexpr (VEC == VecOf<T>::n) store_vec<T>(p + k0, x);
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (k0 + v < d) p[k0 + v] = x[v];
  }
}

// One row (or one chunk of a row) served by a group of Pr slots x L lanes.
// Every lane of the wavefront calls this with the same Pr, so the slot
// butterflies below always run on a full wavefront.
template <class T, int VEC, int NQ>
__device__ __forceinline__ void soft_group(const SoftmaxArgs<T>& a, int mode, bool row_ok,
                                           int64_t slot, int start, int stop, int Pr,
                                           int64_t slab, int lane, int64_t chunk) {
  const int L = a.L;
  const int s = (lane / L) % Pr, c = lane % L;
  const int64_t k0 = (slab * L + c) * VEC;
  const bool feat_ok = k0 < a.d;
  const bool vec_io = a.vec_io;

  // the two-pass chunk merge needs the partials only, not the logits
  const bool load = !(mode == SM_WRITE && a.tab);
  int64_t e[NQ];
  bool ok[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int j = start + q * Pr + s;
    ok[q] = load && row_ok && j < stop;
    e[q] = 0;
    if (ok[q]) e[q] = a.eid ? (int64_t)a.eid[j] : (int64_t)j;
  }
  if (a.mask) {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (ok[q]) ok[q] = a.mask[e[q]] == 1;
  }
  T x[NQ][VEC];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    if (ok[q] && feat_ok) load_cols<T, VEC>(a.logits + e[q] * a.d, k0, a.d, vec_io, x[q]);

  T m[VEC], sum[VEC];
  const T ninf = T(-__builtin_huge_val());
#pragma unroll
  for (int v = 0; v < VEC; ++v) m[v] = ninf;
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    if (ok[q] && feat_ok) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) m[v] = x[q][v] > m[v] ? x[q][v] : m[v];
    }
  const int span = L * Pr;
  for (int off = L; off < span; off <<= 1) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const T o = __shfl_xor(m[v], off);
      m[v] = o > m[v] ? o : m[v];
    }
  }

  if (mode == SM_WRITE) {
    // merge this row's chunk partials: slot s takes chunks s, s + Pr, ...
    // (each slot's sequence in chunk order), then the slots combine by
    // butterflies, so a row of many chunks costs ceil(chunks / Pr) rounds
    const int64_t c0 = a.chunk_first[chunk];
    const int64_t row = a.chunk_row[chunk];
    const int64_t nch = (a.indptr[row + 1] - a.indptr[row] + a.chunk_len - 1) / a.chunk_len;
    T pmv[VEC], psv[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      m[v] = ninf;
      sum[v] = T(0);
    }
    if (feat_ok) {
      for (int64_t q = c0 + s; q < c0 + nch; q += Pr)
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          if (k0 + v < a.d) {
            const T t = a.pm[q * a.d + k0 + v];
            m[v] = t > m[v] ? t : m[v];
          }
    }
    for (int off = L; off < span; off <<= 1) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const T o = __shfl_xor(m[v], off);
        m[v] = o > m[v] ? o : m[v];
      }
    }
    if (feat_ok) {
      for (int64_t q = c0 + s; q < c0 + nch; q += Pr) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          pmv[v] = k0 + v < a.d ? a.pm[q * a.d + k0 + v] : ninf;
          psv[v] = k0 + v < a.d ? a.ps[q * a.d + k0 + v] : T(0);
        }
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          if (pmv[v] != ninf) sum[v] = sum[v] + psv[v] * exp_t(pmv[v] - m[v]);
      }
    }
    for (int off = L; off < span; off <<= 1) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) sum[v] = sum[v] + __shfl_xor(sum[v], off);
    }
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) sum[v] = T(0);
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (ok[q] && feat_ok) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) sum[v] = sum[v] + exp_t(x[q][v] - m[v]);
      }
    for (int off = L; off < span; off <<= 1) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) sum[v] = sum[v] + __shfl_xor(sum[v], off);
    }
  }

  if (mode == SM_STATS) {
    if (row_ok && s == 0 && feat_ok) {
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (k0 + v < a.d) {
          a.pm[chunk * a.d + k0 + v] = m[v];
          a.ps[chunk * a.d + k0 + v] = sum[v];
        }
    }
    return;
  }
  if (!feat_ok) return;
  if (a.tab) {
    // two-pass form: the row's (max, sum) go to the node table
    const bool writer = mode == SM_WRITE ? (s == 0 && a.chunk_first[chunk] == chunk)
                                         : (row_ok && s == 0);
    if (writer) {
      // 16-byte stores when the columns allow (the table is 256-byte aligned
      // and a table row is 2d values)
      T* t = a.tab + slot * 2 * a.d;
      store_cols<T, VEC>(t, k0, a.d, vec_io, m);
      store_cols<T, VEC>(t + a.d, k0, a.d, vec_io, sum);
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (!ok[q]) continue;
    T y[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) y[v] = exp_t(x[q][v] - m[v]) / sum[v];
    store_cols<T, VEC>(a.out + e[q] * a.d, k0, a.d, vec_io, y);
  }
}

// Launch parts: the chunks and wavefront rows in one launch, the packed rows
// (one slot per edge, fewer registers) in another.
enum { PART_WIDE = 1, PART_PACKED = 2 };

constexpr int PK_U = SOFT_PK_U;

// Figures of the plan: kernel arguments, or device memory for a plan built
// on the GPU (DYN).
template <bool DYN, class T>
__device__ __forceinline__ int64_t bin_start_of(const SoftmaxArgs<T>& a, int k) {
  if constexpr (DYN) return a.dyn->bin_start[k];
  else return a.bin_start[k];
}
template <bool DYN, class T>
__device__ __forceinline__ int64_t bin_wave_of(const SoftmaxArgs<T>& a, int k) {
  if constexpr (DYN) return a.dyn->bin_wave[k];
  else return a.bin_wave[k];
}
template <bool DYN, class T>
__device__ __forceinline__ int64_t bin_slot_of(const SoftmaxArgs<T>& a, int k) {
  if constexpr (DYN) return a.dyn->bin_slot[k];
  else return a.bin_slot[k];
}

template <class T, int VEC, bool DYN>
__device__ __forceinline__ void softmax_packed_u(const SoftmaxArgs<T>& a, int64_t w, int lane);

// Wavefront w of the chunks: chunk w / S, column slab w % S (statistics in
// launch 1, the write in launch 2).
template <class T, int VEC>
__device__ __forceinline__ void softmax_chunk_task(const SoftmaxArgs<T>& a, int64_t w, int lane) {
  const int64_t chunk = w / a.S, slab = w % a.S;
  // two-pass merge: the first chunk of each row writes the row's table entry
  if (a.mode2 && a.tab && a.chunk_first[chunk] != chunk) return;
  const int64_t row = a.chunk_row[chunk];
  const int start = a.chunk_start[chunk];
  const int end = a.indptr[row + 1];
  const int stop = end - start > a.chunk_len ? start + a.chunk_len : end;
  // table slot of a chunked row: after the ordered rows, at its first chunk
  // (or the row itself)
  const int64_t slot = a.order && !a.row_slots ? a.hub_base + chunk : row;
  soft_group<T, VEC, SOFT_CPL>(a, a.mode2 ? SM_WRITE : SM_STATS, true, slot, start, stop, a.Pw,
                               slab, lane, chunk);
}

// Wavefront w of the wavefront rows (rows of up to chunk_len edges).
template <class T, int VEC, bool DYN>
__device__ __forceinline__ void softmax_light_task(const SoftmaxArgs<T>& a, int64_t w, int lane) {
  const int Pw = a.Pw;
  const int R = a.nat_r;
  int64_t mid_start, mid_end;
  if constexpr (DYN) {
    mid_start = a.dyn->mid_start;
    mid_end = a.dyn->mid_end;
  } else {
    mid_start = a.mid_start;
    mid_end = a.mid_end;
  }
  const int64_t nmid = ((mid_end - mid_start + R - 1) / R) * a.S;
  if (w >= nmid) return;
  // R consecutive rows per wavefront (R = 1 with a row order): they share
  // it, Pw / R slots each, when the longest of them fits those slots' CPL
  // rounds; otherwise each takes the whole wavefront in turn (the choice
  // is uniform per wavefront)
  const int64_t slab = w % a.S;
  const int64_t i0 = mid_start + (w / a.S) * R;
  int Pr = Pw, iters = R;
  if (R > 1) {
    const int64_t i = i0 + (lane / a.L) / (Pw / R);
    const int deg = i < mid_end ? a.indptr[i + 1] - a.indptr[i] : 0;
    if (wave_max_int(deg) <= (Pw / R) * SOFT_CPL) {
      Pr = Pw / R;
      iters = 1;
    }
  }
  for (int r = 0; r < iters; ++r) {
    if (iters > 1 && i0 + r >= mid_end) break;  // uniform
    const int64_t i = iters == 1 ? i0 + (lane / a.L) / Pr : i0 + r;
    const bool in = i < mid_end;
    const int64_t row = a.order ? (in ? (int64_t)a.order[i] : 0) : i;
    int start = 0, stop = 0;
    if (in) {
      start = a.indptr[row];
      stop = a.indptr[row + 1];
    }
    const bool ok = in && stop > start && stop - start <= a.chunk_len;
    soft_group<T, VEC, SOFT_CPL>(a, SM_FULL, ok, a.order && !a.row_slots ? i : row, start, stop,
                                 Pr, slab, lane, 0);
  }
}

template <class T, int VEC, int PART, bool DYN>
__global__ __launch_bounds__(BLOCK) void softmax_kernel(SoftmaxArgs<T> a) {
  const int lane = threadIdx.x & (WAVE - 1);
  if constexpr (DYN) {
    // a plan built on the GPU: the work counts are in device memory, and a
    // fixed grid walks the work (every wavefront's loop bound is uniform)
    const int64_t stride = (int64_t)gridDim.x * WAVES_PER_BLOCK;
    const int64_t w0 = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if constexpr (PART == PART_PACKED) {
      const int64_t tasks = a.dyn->packed_tasks;
      for (int64_t w = w0; w < tasks; w += stride) softmax_packed_u<T, VEC, true>(a, w, lane);
    } else {
      const int64_t cw = a.dyn->chunk_waves;
      const int64_t total = a.mode2 ? cw : cw + a.dyn->light_waves;
      for (int64_t w = w0; w < total; w += stride) {
        if (w < cw) softmax_chunk_task<T, VEC>(a, w, lane);
        else softmax_light_task<T, VEC, true>(a, w - cw, lane);
      }
    }
    return;
  } else {
    const int64_t b = blockIdx.x;
    if constexpr (PART == PART_PACKED) {
      // packed rows only (their own launch: one slot per edge, few registers)
      const int64_t lb = xcd_remap(b, a.light_blocks);
      const int64_t w = lb * WAVES_PER_BLOCK + (threadIdx.x >> 6);
      if (w * PK_U >= a.light_waves) return;  // uniform per wavefront
      softmax_packed_u<T, VEC, false>(a, w, lane);
      return;
    }
    if (b < a.chunk_blocks) {
      const int64_t w = b * WAVES_PER_BLOCK + (threadIdx.x >> 6);
      if (w >= a.chunk_waves) return;
      softmax_chunk_task<T, VEC>(a, w, lane);
      return;
    }
    const int64_t lb = xcd_remap(b - a.chunk_blocks, a.light_blocks);
    const int64_t w = lb * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (w >= a.light_waves) return;
    softmax_light_task<T, VEC, false>(a, w, lane);
  }
}

// The packed launch: each wavefront serves PK_U consecutive packed
// wavefronts' rows, walking the chain order -> indptr -> eid -> logits for
// all of them at once, so every dependent load has PK_U requests per lane in
// flight instead of one.
template <class T, int VEC, bool DYN>
__device__ __forceinline__ void softmax_packed_u(const SoftmaxArgs<T>& a, int64_t w, int lane) {
  const int L = a.L, Pw = a.Pw;
  const int c = lane % L;
  // every bin's wavefront count is a multiple of PK_U, so all rounds of
  // this wavefront lie in one bin k (found once, uniform)
  const int64_t pw0 = w * PK_U;
  int k = 0;
  while (k + 1 < a.nbins && bin_wave_of<DYN>(a, k + 1) <= pw0) ++k;
  const int Pr = 1 << k;
  const int per = Pw / Pr;
  const int span = L * Pr;
  const int sl = (lane / L) % Pr;
  const int64_t b0 = bin_start_of<DYN>(a, k), b1 = bin_start_of<DYN>(a, k + 1);
  const int64_t bw = bin_wave_of<DYN>(a, k);
  // indices are clamped into the bin (and rows have >= 1 edge), so every
  // load below is unconditional and in bounds; rok / ok mask the results
  int64_t slab[PK_U], ic[PK_U];
  bool rok[PK_U];
#pragma unroll
  for (int r = 0; r < PK_U; ++r) {
    const int64_t local = pw0 + r - bw;
    slab[r] = local % a.S;
    const int64_t i = b0 + (local / a.S) * per + lane / (Pr * L);
    rok[r] = i < b1;
    ic[r] = rok[r] ? i : b0;
  }
  int64_t e[PK_U];
  bool ok[PK_U];
  if (a.peid) {
    // the plan lists every packed slot's edge id: one coalesced load per
    // round instead of the chain order -> indptr -> eid (-1 past a row's
    // degree; those lanes read edge 0, which exists, and are masked)
    const int64_t bs = bin_slot_of<DYN>(a, k);
#pragma unroll
    for (int r = 0; r < PK_U; ++r) {
      const int32_t pe = a.peid[bs + (ic[r] - b0) * Pr + sl];
      ok[r] = rok[r] && pe >= 0;
      e[r] = pe >= 0 ? (int64_t)pe : 0;
    }
  } else {
    int start[PK_U], stop[PK_U];
#pragma unroll
    for (int r = 0; r < PK_U; ++r) {
      const int64_t row = a.order[ic[r]];
      start[r] = a.indptr[row];
      stop[r] = a.indptr[row + 1];
    }
#pragma unroll
    for (int r = 0; r < PK_U; ++r) {
      const int j = start[r] + sl;
      ok[r] = rok[r] && j < stop[r];
      const int jc = ok[r] ? j : start[r];
      e[r] = a.eid ? (int64_t)a.eid[jc] : (int64_t)jc;
    }
  }
  if (a.mask) {
#pragma unroll
    for (int r = 0; r < PK_U; ++r) ok[r] = ok[r] && a.mask[e[r]] == 1;
  }
  T x[PK_U][VEC];
#pragma unroll
  for (int r = 0; r < PK_U; ++r) {
    const int64_t k0 = (slab[r] * L + c) * VEC;
    const int64_t kc = k0 < a.d ? k0 : 0;
    load_cols<T, VEC>(a.logits + e[r] * a.d, kc, a.d, a.vec_io, x[r]);
  }
  const T ninf = T(-__builtin_huge_val());
#pragma unroll
  for (int r = 0; r < PK_U; ++r) {
    const int64_t k0 = (slab[r] * L + c) * VEC;
    const bool feat_ok = k0 < a.d;
    T m[VEC], sum[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) m[v] = (ok[r] && feat_ok) ? x[r][v] : ninf;
    for (int off = L; off < span; off <<= 1) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const T o = __shfl_xor(m[v], off);
        m[v] = o > m[v] ? o : m[v];
      }
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) sum[v] = (ok[r] && feat_ok) ? exp_t(x[r][v] - m[v]) : T(0);
    for (int off = L; off < span; off <<= 1) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) sum[v] = sum[v] + __shfl_xor(sum[v], off);
    }
    if (!feat_ok) continue;
    if (a.tab) {
      if (rok[r] && sl == 0) {
        // slot = position in the row order: a wavefront's rows write
        // consecutive table rows (whole lines); or the row id
        const int64_t slot = a.row_slots ? (int64_t)a.order[ic[r]] : ic[r];
        T* t = a.tab + slot * 2 * a.d;
        store_cols<T, VEC>(t, k0, a.d, a.vec_io, m);
        store_cols<T, VEC>(t + a.d, k0, a.d, a.vec_io, sum);
      }
    } else if (ok[r]) {
      T y[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) y[v] = exp_t(x[r][v] - m[v]) / sum[v];
      store_cols<T, VEC>(a.out + e[r] * a.d, k0, a.d, a.vec_io, y);
    }
  }
}

// Edge-parallel write of the two-pass form: L lanes per edge, 64 / L edges
// per wavefront, edges in id order.
template <class T, int VEC>
__global__ __launch_bounds__(BLOCK) void softmax_edge_kernel(const T* __restrict__ logits,
                                                             T* __restrict__ out,
                                                             const T* __restrict__ tab,
                                                             const int32_t* __restrict__ slot_of,
                                                             const int8_t* __restrict__ mask,
                                                             int64_t num_edges, int64_t d, int L,
                                                             int S, int vec_io, int64_t nblocks) {
  const int64_t blk = xcd_remap(blockIdx.x, nblocks);
  const int lane = threadIdx.x & (WAVE - 1);
  const int64_t w = blk * WAVES_PER_BLOCK + (threadIdx.x >> 6);
  const int64_t slab = w % S;
  const int64_t e = (w / S) * (WAVE / L) + lane / L;
  const int64_t k0 = (slab * L + lane % L) * VEC;
  if (e >= num_edges || k0 >= d) return;
  if (mask && mask[e] != 1) return;
  const int64_t r = slot_of[e];
  T x[VEC], m[VEC], s[VEC];
  if (VEC > 1 && vec_io) {
    if constexpr (VEC > 1) load_n_stream<T, VEC>(logits + e * d + k0, x);
  } else {
    load_cols<T, VEC>(logits + e * d, k0, d, vec_io, x);
  }
  load_cols<T, VEC>(tab + r * 2 * d, k0, d, vec_io, m);
  load_cols<T, VEC>(tab + r * 2 * d + d, k0, d, vec_io, s);
#pragma unroll
  for (int v = 0; v < VEC; ++v) x[v] = exp_t(x[v] - m[v]) / s[v];
  if (VEC > 1 && vec_io) {
    if constexpr (VEC > 1) store_n_stream<T, VEC>(out + e * d + k0, x);
  } else {
    store_cols<T, VEC>(out + e * d, k0, d, vec_io, x);
  }
}

// The edge-parallel write of the two-pass form over p.num_edges edges.
template <class T, int VEC>
hipError_t launch_softmax_edges(const SoftmaxParams& p, const SoftmaxArgs<T>& a) {
  const int64_t waves = ((p.num_edges + (WAVE / a.L) - 1) / (WAVE / a.L)) * a.S;
  const int64_t nb = (waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  hipLaunchKernelGGL((softmax_edge_kernel<T, VEC>), dim3((unsigned)nb), dim3(BLOCK), 0, p.stream,
                     a.logits, a.out, a.tab, p.row_of, a.mask, p.num_edges, p.d, a.L, a.S,
                     a.vec_io, nb);
  return hipGetLastError();
}

// Workgroups of a launch that walks device-counted work: 8 per CU (32
// wavefronts, the residency the kernels reach), fewer when the work cannot
// fill them.
constexpr int64_t DYN_BLOCKS = 256 * 8;

// A plan built on the GPU (p.dyn): the same three launches, on fixed grids
// whose wavefronts walk the work the device figures count; the chunk write
// pass is always launched (it finds no chunks when there are none).
template <class T, int VEC>
hipError_t launch_softmax_dyn(const SoftmaxParams& p, SoftmaxArgs<T> a) {
  a.nbins = p.nbins;
  a.peid = p.packed_eid;
  a.nat_r = 1;
  a.num_chunks = p.num_chunks;  // capacity: the partials are laid out for it
  a.chunk_row = p.chunk_row;
  a.chunk_start = p.chunk_start;
  a.chunk_first = p.chunk_first;
  a.pm = static_cast<T*>(p.part);
  a.ps = a.pm ? a.pm + p.num_chunks * p.d : nullptr;
  a.tab = static_cast<T*>(p.table);
  a.hub_base = 0;
  auto grid = [](int64_t waves) {
    const int64_t b = (waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    return (unsigned)(b < 1 ? 1 : (b > DYN_BLOCKS ? DYN_BLOCKS : b));
  };
  // upper bounds of the work, only to keep tiny plans from launching the
  // full grid: every row is packed, a wavefront row, or chunked
  const int64_t rows = p.num_rows, edges = p.num_slots;
  const int64_t wide = (p.num_chunks + rows) * a.S;
  const int64_t packed = (2 * edges / a.Pw + p.nbins + 1) * a.S / PK_U + p.nbins + 1;
  a.mode2 = 0;
  hipLaunchKernelGGL((softmax_kernel<T, VEC, PART_WIDE, true>), dim3(grid(wide)), dim3(BLOCK), 0,
                     p.stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((softmax_kernel<T, VEC, PART_PACKED, true>), dim3(grid(packed)), dim3(BLOCK),
                     0, p.stream, a);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (p.num_chunks > 0) {
    a.mode2 = 1;
    hipLaunchKernelGGL((softmax_kernel<T, VEC, PART_WIDE, true>),
                       dim3(grid(p.num_chunks * a.S)), dim3(BLOCK), 0, p.stream, a);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (a.tab && p.num_edges > 0) return launch_softmax_edges<T, VEC>(p, a);
  return hipSuccess;
}

template <class T, int VEC>
hipError_t launch_softmax_vec(const SoftmaxParams& p) {
  SoftmaxArgs<T> a{};
  a.indptr = p.indptr;
  a.eid = p.eid;
  a.mask = p.mask;
  a.logits = static_cast<const T*>(p.logits);
  a.out = static_cast<T*>(p.out);
  a.num_rows = p.num_rows;
  a.d = p.d;
  const int64_t nvec = (p.d + VEC - 1) / VEC;
  int L = 1;
  while (L < nvec && L < WAVE) L <<= 1;
  a.L = L;
  a.Pw = WAVE / L;
  a.S = (int)((nvec + L - 1) / L);
  a.vec_io = (VEC > 1) && (p.d % VEC == 0);
  a.chunk_len = SOFT_CPL * a.Pw;
  a.order = p.order;
  a.nbins = 0;
  a.row_slots = p.row_slots;
  a.dyn = p.dyn;
  if (p.dyn) return launch_softmax_dyn<T, VEC>(p, a);
  int64_t waves = 0;
  if (p.order) {
    a.nbins = p.nbins;
    for (int k = 0; k <= p.nbins; ++k) a.bin_start[k] = p.bounds[k];
    a.peid = p.packed_eid;
    int64_t slots_before = 0;
    for (int k = 0; k < p.nbins; ++k) {
      a.bin_slot[k] = slots_before;
      slots_before += (a.bin_start[k + 1] - a.bin_start[k]) << k;
    }
    for (int k = 0; k < p.nbins; ++k) {
      // padded to a multiple of PK_U: a wavefront of the packed launch
      // never straddles two bins
      const int64_t per = a.Pw >> k;
      a.bin_wave[k] = waves;
      const int64_t wk = ((a.bin_start[k + 1] - a.bin_start[k] + per - 1) / per) * a.S;
      waves += (wk + PK_U - 1) / PK_U * PK_U;
    }
    a.bin_wave[p.nbins] = waves;
    a.mid_start = p.bounds[p.nbins];
    a.mid_end = p.bounds[p.nbins + 1];
  } else {
    a.mid_start = 0;
    a.mid_end = p.num_rows;
  }
  const int64_t packed_waves = waves;
  // natural order: R rows per wavefront, Pw / R slots each, sized so the
  // mean row (slots / rows) fills at most ~60 % of its CPL rounds
  a.nat_r = 1;
  if (!p.order && p.num_slots > 0 && p.num_rows > 0) {
    const double mean = double(p.num_slots) / double(p.num_rows);
    int pr = 1;
    while (pr < a.Pw && pr * SOFT_CPL < 1.6 * mean) pr <<= 1;
    a.nat_r = a.Pw / pr;
  }
  a.light_waves = ((a.mid_end - a.mid_start + a.nat_r - 1) / a.nat_r) * a.S;
  a.light_blocks = (a.light_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  a.num_chunks = p.num_chunks;
  a.chunk_row = p.chunk_row;
  a.chunk_start = p.chunk_start;
  a.chunk_first = p.chunk_first;
  a.pm = static_cast<T*>(p.part);
  a.ps = a.pm ? a.pm + p.num_chunks * p.d : nullptr;
  a.chunk_waves = p.num_chunks * a.S;
  a.chunk_blocks = (a.chunk_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  a.mode2 = 0;
  a.tab = static_cast<T*>(p.table);
  a.hub_base = p.order ? p.bounds[p.nbins + 1] : 0;
  // chunks and wavefront rows, then the packed rows in a launch of their own
  const int64_t blocks = a.chunk_blocks + a.light_blocks;
  if (blocks > 0) {
    hipLaunchKernelGGL((softmax_kernel<T, VEC, PART_WIDE, false>), dim3((unsigned)blocks),
                       dim3(BLOCK), 0, p.stream, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (packed_waves > 0) {
    SoftmaxArgs<T> b = a;
    b.light_waves = packed_waves;
    const int64_t pk_waves = (packed_waves + PK_U - 1) / PK_U;
    b.light_blocks = (pk_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
    hipLaunchKernelGGL((softmax_kernel<T, VEC, PART_PACKED, false>),
                       dim3((unsigned)b.light_blocks), dim3(BLOCK), 0, p.stream, b);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (a.chunk_blocks > 0) {
    a.mode2 = 1;
    a.light_waves = 0;
    a.light_blocks = 0;
    hipLaunchKernelGGL((softmax_kernel<T, VEC, PART_WIDE, false>), dim3((unsigned)a.chunk_blocks),
                       dim3(BLOCK), 0, p.stream, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (a.tab && p.num_edges > 0) return launch_softmax_edges<T, VEC>(p, a);
  return hipSuccess;
}

template <class T>
hipError_t launch_softmax(const SoftmaxParams& p) {
  if (p.vec == VecOf<T>::n) return launch_softmax_vec<T, VecOf<T>::n>(p);
  return launch_softmax_vec<T, 1>(p);
}

}  // namespace mdgl

#define MDGL_INSTANTIATE_SOFTMAX(T) \
  template hipError_t mdgl::launch_softmax<T>(const mdgl::SoftmaxParams&);
