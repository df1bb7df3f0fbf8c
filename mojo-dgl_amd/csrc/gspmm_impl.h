// CSR reduce kernel behind gspmm (included once per (dtype, reducer)
// translation unit).
//
// Work list. A "unit" is either a chunk of a heavy row (written as a
// partial) or a whole row (rows longer than chunk_len are skipped there).
// The first chunk_blocks workgroups take the chunks (so they start first),
// the remaining workgroups the rows; both ranges go through the XCD remap,
// so each XCD serves a contiguous run of units and the rows of a block of
// neighbouring destinations share its L2 (a community graph's chunks dealt
// round-robin over the XCDs held its L2 hit rate at 70 %). A unit is processed
// by G consecutive lanes (G = the power of two covering the row's vectors,
// at most 64), so a wavefront packs 64 / G units; output rows wider than
// 64 * VEC are cut into S slabs, one wavefront per slab.
//
// Fold order. Each lane owns VEC output columns and folds its unit's CSR
// slots one after the other, in CSR order: for a row that is not split this
// is exactly the reference's sequential fold (src/ported.mojo:392-422), so
// sum, mean, max and min values are bit-identical to the CPU kernel in the
// same precision. Split rows fold each chunk in order and then fold the
// chunk partials in chunk order; max/min remain exact (strict comparison,
// the earlier chunk wins ties, so the arg is still the first edge in CSR
// order reaching the value).
//
// Memory. Per 64 CSR slots a lane group issues one coalesced load of the
// neighbour ids and one of the edge ids; the ids are then broadcast with
// v_readlane (whole-wavefront units, scalar registers, so the row address is
// formed on the scalar unit) or ds_bpermute (packed units). Each edge costs
// one 16-byte (float32 rows of odd multiples of 2 columns: 8-byte) gather per
// lane of the source row and one of the edge row, with U edges in flight per
// lane.
#pragma once

#include "mdgl_kernels.h"

namespace mdgl {

constexpr int M_DYN = 3;

template <class T>
struct GspmmArgs {
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* eid;
  const int32_t* deg;
  const T* lhs;
  const T* rhs;
  T* out;
  int32_t* arg_u;
  int32_t* arg_e;
  int64_t num_rows, dl, dr, dout;
  int64_t lstride;  // elements between lhs rows
  Bcast bc;
  int lmode, rmode, flags, G, S, vec;
  int64_t num_chunks;
  const int32_t* chunk_row;
  const int32_t* chunk_start;
  int chunk_len;
  T* part_val;
  int32_t* part_u;
  int32_t* part_e;
  int64_t chunk_waves, row_waves, chunk_blocks, num_blocks;
  // waves per slab (slab-major order: every unit's slab s before slab s + 1,
  // so the rows of neighbouring units share cache lines across wavefronts)
  int64_t chunk_uwaves, row_uwaves;
  int slab_major;
  const T* rowop;  // dot output (see GspmmParams), else null
  T* dot_out;
  int dot_lanes;
  const int32_t* rows;  // listed rows (see GspmmParams), else null
  int64_t row_limit;
};

template <class T, int VEC, int M>
__device__ __forceinline__ void fetch(const T* __restrict__ row, int mode_rt, const int (&off)[VEC],
                                      T (&x)[VEC]) {
  const int m = (M == M_DYN) ? mode_rt : M;
  if (VEC > 1 && m == M_CONTIG) {
    if constexpr (VEC > 1) load_n<T, VEC>(row + off[0], x);
  } else if (m == M_SPLAT) {
    const T s = row[off[0]];
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = s;
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = row[off[v]];
  }
}

// The same for the edge operand, read once per edge: non-temporal, so it
// does not displace source rows that other edges will gather.
template <class T, int VEC, int M>
__device__ __forceinline__ void fetch_stream(const T* __restrict__ row, int mode_rt,
                                             const int (&off)[VEC], T (&x)[VEC]) {
  const int m = (M == M_DYN) ? mode_rt : M;
  if (VEC > 1 && m == M_CONTIG) {
    if constexpr (VEC > 1) load_n_stream<T, VEC>(row + off[0], x);
  } else if (m == M_SPLAT) {
    const T s = __builtin_nontemporal_load(row + off[0]);
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = s;
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = __builtin_nontemporal_load(row + off[v]);
  }
}

template <class T, int OP, int RED, int VEC, int LM, int RM, bool WIDE, bool NT,
          bool DOT = false>
__device__ __forceinline__ void gspmm_body(const GspmmArgs<T>& a, bool chunk, int64_t wave,
                                           int lane) {
  // edges in flight per lane: 8 (4 in the dot pass, whose per-edge
  // butterflies already hide the loads; 8 there cost 14 %)
  constexpr int U = DOT ? 4 : 8;
  const int G = WIDE ? WAVE : a.G;
  const int grp = lane / G, gl = lane % G, gbase = grp * G;
  const int64_t uw = chunk ? a.chunk_uwaves : a.row_uwaves;
  const int64_t slab = a.slab_major ? wave / uw : wave % a.S;
  const int64_t unit = (a.slab_major ? wave % uw : wave / a.S) * (WAVE / G) + grp;

  // ---- resolve the unit to a CSR slot range
  bool ok = unit < (chunk ? a.num_chunks : a.num_rows);
  int64_t row = 0;
  int start = 0, stop = 0;
  if (ok) {
    if (chunk) {
      row = a.chunk_row[unit];
      start = a.chunk_start[unit];
      const int end = a.indptr[row + 1];
      stop = (end - start > a.chunk_len) ? start + a.chunk_len : end;
    } else {
      row = unit;
      if (a.rows) {
        row = a.rows[unit];
        if (row < 0 || row >= a.row_limit) ok = false;  // not a row of the graph: skipped
      }
      if (ok) {
        start = a.indptr[row];
        stop = a.indptr[row + 1];
        if (stop - start > a.chunk_len) ok = false;  // heavy: done by chunks + combine
      }
    }
  }

  // ---- this lane's output columns and operand offsets
  const int64_t k0 = (slab * G + gl) * VEC;
  const bool feat_ok = k0 < a.dout;
  int loff[VEC], roff[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int64_t k = (feat_ok && k0 + v < a.dout) ? k0 + v : (feat_ok ? k0 : 0);
    loff[v] = (int)bcast_off(a.bc, k, true);
    roff[v] = (int)bcast_off(a.bc, k, false);
  }

  // DOT: this row's own feature columns, dotted with every gathered lhs row
  T rowv[VEC];
  if constexpr (DOT) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) rowv[v] = T(0);
    if (ok && feat_ok) load_n<T, VEC>(a.rowop + row * a.dout + k0, rowv);
  }

  T acc[VEC];
  int au[VEC], ae[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    acc[v] = seed<T>(RED);
    au[v] = -1;  // nothing selected yet
    ae[v] = -1;
  }

  const bool ident = a.flags & F_EID_IDENTITY;
  constexpr bool ARG_OUT = (RED == RED_MAX || RED == RED_MIN);
  const int n = ok ? stop - start : 0;
  const int nmax = WIDE ? n : wave_max_int(n);
  // a scalar edge operand (one value per edge, splatted over the columns) is
  // loaded with the ids, one edge per lane, and broadcast like them
  constexpr bool SCALAR_E = RM == M_SPLAT && OP != OP_COPY_LHS;
  const bool scalar_e = SCALAR_E && a.dr == 1;
  // the edge operand may come in CSR slot order (row i of rhs for slot i)
  const bool rhs_csr = a.flags & F_RHS_CSR;
  // edge ids are read only for an arg or an edge operand in edge-id order
  // (fixed at compile time where it can be: the dot pass, whose edge operand
  // is always in edge-id order, ran 11 % slower with the load made
  // conditional at run time)
  constexpr bool E_ALWAYS = ARG_OUT || DOT;
  constexpr bool E_NEVER = !ARG_OUT && OP == OP_COPY_LHS;
  const bool need_e = E_ALWAYS || (!E_NEVER && !rhs_csr);
  for (int base = 0; base < nmax; base += G) {
    int my_s = 0, my_e = 0;
    T my_w = T(0);
    if (base + gl < n) {
      const int i = start + base + gl;
      if (a.indices) my_s = __builtin_nontemporal_load(a.indices + i);
      my_e = ident ? i : (need_e ? __builtin_nontemporal_load(a.eid + i) : 0);
      if (SCALAR_E && scalar_e) my_w = a.rhs[rhs_csr ? (int64_t)i : (int64_t)my_e];
    }
    const int cnt = n - base < G ? n - base : G;  // may be <= 0 on finished groups
    const int jmax = WIDE ? cnt : (nmax - base < G ? nmax - base : G);
    for (int j = 0; j < jmax; j += U) {
      T x[U][VEC], y[U][VEC];
      int su[U], se[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int jj = (j + u < G) ? j + u : G - 1;
        // copy_rhs needs the source only for an arg
        constexpr bool NEED_S = OP != OP_COPY_RHS || ARG_OUT;
        int s = 0, e;
        if constexpr (WIDE) {
          e = readlane_int(my_e, jj);
        } else {
          e = __shfl(my_e, gbase + jj);
        }
        if constexpr (NEED_S) {
          if constexpr (WIDE) s = readlane_int(my_s, jj);
          else s = __shfl(my_s, gbase + jj);
        }
        su[u] = s;
        se[u] = e;
        if constexpr (SCALAR_E) {
          if (scalar_e) {
            T w;
            if constexpr (WIDE) w = readlane_val(my_w, jj);
            else w = __shfl(my_w, gbase + jj);
#pragma unroll
            for (int v = 0; v < VEC; ++v) y[u][v] = w;
          }
        }
        if (j + u < cnt && feat_ok) {
          if constexpr (OP != OP_COPY_RHS)
            fetch<T, VEC, LM>(a.lhs + (int64_t)s * a.lstride, a.lmode, loff, x[u]);
          if constexpr (OP != OP_COPY_LHS) {
            if (!(SCALAR_E && scalar_e)) {
              const int64_t rrow = rhs_csr ? (int64_t)(start + base + j + u) : (int64_t)e;
              // a row gathered by a random edge id is read once: stream it
              if constexpr (NT)
                fetch_stream<T, VEC, RM>(a.rhs + rrow * a.dr, a.rmode, roff, y[u]);
              else
                fetch<T, VEC, RM>(a.rhs + rrow * a.dr, a.rmode, roff, y[u]);
            }
          }
        }
      }
      if constexpr (DOT) {
        // per slot and column group: the lanes' partial dots, then a
        // butterfly over the group's lanes; the group's first lane writes
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j + u >= jmax) break;  // uniform in the wavefront
          T pd = T(0);
          if (j + u < cnt && feat_ok) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) pd = pd + x[u][v] * rowv[v];
          }
          for (int off = 1; off < a.dot_lanes; off <<= 1) pd = pd + __shfl_xor(pd, off);
          if (j + u < cnt && feat_ok && (gl % a.dot_lanes) == 0) {
            const int64_t slot = start + base + j + u;
            a.dot_out[slot * a.dr + k0 / ((int64_t)a.dot_lanes * VEC)] = pd;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j + u < cnt && feat_ok) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            T xv = T(0), yv = T(0);
            if constexpr (OP != OP_COPY_RHS) xv = x[u][v];
            if constexpr (OP != OP_COPY_LHS) yv = y[u][v];
            const T m = message<OP>(xv, yv);
            if constexpr (RED == RED_MAX) {
              if (m > acc[v]) { acc[v] = m; au[v] = su[u]; ae[v] = se[u]; }
            } else if constexpr (RED == RED_MIN) {
              if (m < acc[v]) { acc[v] = m; au[v] = su[u]; ae[v] = se[u]; }
            } else {
              acc[v] = acc[v] + m;
            }
          }
        }
      }
    }
  }

  if (!ok || !feat_ok) return;
  constexpr bool ARG = (RED == RED_MAX || RED == RED_MIN);
  if (chunk) {
    const int64_t o = unit * a.dout + k0;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      if (k0 + v < a.dout) {
        a.part_val[o + v] = acc[v];
        if constexpr (ARG) {
          a.part_u[o + v] = au[v];
          a.part_e[o + v] = ae[v];
        }
      }
    }
    return;
  }
  if ((a.flags & F_MEAN) && n > 0) {
    T sc = a.deg ? T(a.deg[row]) : T(n);
    if (sc < T(1)) sc = T(1);
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = acc[v] / sc;
  }
  if (a.flags & F_REPLACE_INF) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (is_inf(acc[v])) {
        acc[v] = T(0);  // a replaced value has no message behind it
        au[v] = -1;
        ae[v] = -1;
      }
  }
  const int64_t o = row * a.dout + k0;
  if (VEC > 1 && (a.flags & F_OUT_VEC)) {
    if constexpr (VEC > 1) store_n_stream<T, VEC>(a.out + o, acc);
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (k0 + v < a.dout) a.out[o + v] = acc[v];
  }
  if constexpr (ARG) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      if (k0 + v < a.dout) {
        if (a.arg_u) a.arg_u[o + v] = au[v];
        if (a.arg_e) a.arg_e[o + v] = ae[v];
      }
    }
  }
}

// Kernel variants, one body each so that every launch only carries the
// registers of its own path: whole-wavefront units (G = 64) with both
// operands contiguous, with a splatted edge operand, or any modes; packed
// units likewise. A scalar edge operand (one value per edge) is loaded with
// the ids and broadcast by v_readlane or ds_bpermute in both layouts: read
// per lane and edge through the any-modes path it cost a GCN aggregation over
// 128 columns 4x the time of the same gather without the weight.
enum { P_WIDE_CC = 0, P_WIDE_CS = 1, P_WIDE_DYN = 2, P_PACK_CC = 3, P_PACK_DYN = 4,
       P_WIDE_CS_DOT = 5, P_PACK_DYN_DOT = 6, P_PACK_CS = 7 };

template <class T, int OP, int RED, int VEC, int PATH, bool NT>
__global__ __launch_bounds__(BLOCK) void gspmm_kernel(GspmmArgs<T> a) {
  const int64_t b = blockIdx.x;
  const bool chunk = b < a.chunk_blocks;
  const int64_t blk =
      chunk ? xcd_remap(b, a.chunk_blocks) : xcd_remap(b - a.chunk_blocks, a.num_blocks - a.chunk_blocks);
  const int lane = threadIdx.x & (WAVE - 1);
  // every lane of a wavefront takes the same path below, so shuffles and
  // readlanes always see a full wavefront
  const int64_t wave = blk * WAVES_PER_BLOCK + (threadIdx.x >> 6);
  if (wave >= (chunk ? a.chunk_waves : a.row_waves)) return;
  if constexpr (PATH == P_WIDE_CC)
    gspmm_body<T, OP, RED, VEC, M_CONTIG, M_CONTIG, true, NT>(a, chunk, wave, lane);
  else if constexpr (PATH == P_WIDE_CS)
    gspmm_body<T, OP, RED, VEC, M_CONTIG, M_SPLAT, true, NT>(a, chunk, wave, lane);
  else if constexpr (PATH == P_WIDE_DYN)
    gspmm_body<T, OP, RED, VEC, M_DYN, M_DYN, true, NT>(a, chunk, wave, lane);
  else if constexpr (PATH == P_PACK_CC)
    gspmm_body<T, OP, RED, VEC, M_CONTIG, M_CONTIG, false, NT>(a, chunk, wave, lane);
  else if constexpr (PATH == P_PACK_CS)
    gspmm_body<T, OP, RED, VEC, M_CONTIG, M_SPLAT, false, NT>(a, chunk, wave, lane);
  else if constexpr (PATH == P_WIDE_CS_DOT)
    gspmm_body<T, OP, RED, VEC, M_CONTIG, M_SPLAT, true, NT, true>(a, chunk, wave, lane);
  else if constexpr (PATH == P_PACK_DYN_DOT)
    gspmm_body<T, OP, RED, VEC, M_DYN, M_DYN, false, NT, true>(a, chunk, wave, lane);

  else
    gspmm_body<T, OP, RED, VEC, M_DYN, M_DYN, false, NT>(a, chunk, wave, lane);
}

// Folds the chunk partials of each heavy row in chunk (= CSR) order.
template <class T, int RED>
__global__ __launch_bounds__(BLOCK) void gspmm_combine_kernel(
    const int32_t* __restrict__ heavy_rows, const int32_t* __restrict__ heavy_ptr,
    const int32_t* __restrict__ indptr, const int32_t* __restrict__ deg,
    const T* __restrict__ part_val, const int32_t* __restrict__ part_u,
    const int32_t* __restrict__ part_e, T* __restrict__ out, int32_t* __restrict__ arg_u,
    int32_t* __restrict__ arg_e, int64_t num_heavy, int64_t dout, int flags) {
  const int64_t t = (int64_t)blockIdx.x * BLOCK + threadIdx.x;
  if (t >= num_heavy * dout) return;
  const int64_t h = t / dout, k = t % dout;
  const int64_t row = heavy_rows[h];
  T acc = seed<T>(RED);
  int au = -1, ae = -1;
  for (int c = heavy_ptr[h]; c < heavy_ptr[h + 1]; ++c) {
    const T v = part_val[(int64_t)c * dout + k];
    if constexpr (RED == RED_MAX) {
      if (v > acc) { acc = v; au = part_u[(int64_t)c * dout + k]; ae = part_e[(int64_t)c * dout + k]; }
    } else if constexpr (RED == RED_MIN) {
      if (v < acc) { acc = v; au = part_u[(int64_t)c * dout + k]; ae = part_e[(int64_t)c * dout + k]; }
    } else {
      acc = acc + v;
    }
  }
  if (flags & F_MEAN) {
    T sc = deg ? T(deg[row]) : T(indptr[row + 1] - indptr[row]);
    if (sc < T(1)) sc = T(1);
    acc = acc / sc;
  }
  if ((flags & F_REPLACE_INF) && is_inf(acc)) {
    acc = T(0);
    au = ae = -1;
  }
  out[row * dout + k] = acc;
  if constexpr (RED == RED_MAX || RED == RED_MIN) {
    if (arg_u) arg_u[row * dout + k] = au;
    if (arg_e) arg_e[row * dout + k] = ae;
  }
}

template <class T, int OP, int RED, int VEC, bool NT>
void launch_path(const GspmmArgs<T>& a, dim3 grid, dim3 block, int lm, int rm, hipStream_t st) {
  if (a.G == WAVE) {
    if (lm == M_CONTIG && rm == M_CONTIG)
      hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_WIDE_CC, NT>), grid, block, 0, st, a);
    else if (lm == M_CONTIG && rm == M_SPLAT)
      hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_WIDE_CS, NT>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_WIDE_DYN, NT>), grid, block, 0, st, a);
  } else {
    if (lm == M_CONTIG && rm == M_CONTIG)
      hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_PACK_CC, NT>), grid, block, 0, st, a);
    else if (lm == M_CONTIG && rm == M_SPLAT)
      hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_PACK_CS, NT>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_PACK_DYN, NT>), grid, block, 0, st, a);
  }
}

template <class T, int OP, int RED, int VEC>
hipError_t launch_gspmm_op(const GspmmParams& p) {
  GspmmArgs<T> a;
  a.indptr = p.indptr;
  a.indices = p.indices;
  a.eid = p.eid;
  a.deg = p.deg;
  a.lhs = static_cast<const T*>(p.lhs);
  a.rhs = static_cast<const T*>(p.rhs);
  a.out = static_cast<T*>(p.out);
  a.arg_u = p.arg_u;
  a.arg_e = p.arg_e;
  a.num_rows = p.num_rows;
  a.dl = p.dl;
  a.lstride = p.lstride > 0 ? p.lstride : p.dl;
  a.dr = p.dr;
  a.dout = p.dout;
  a.bc = p.bc;
  a.lmode = p.lmode;
  a.rmode = p.rmode;
  a.flags = p.flags;
  a.vec = VEC;
  const int64_t nvec = (p.dout + VEC - 1) / VEC;
  const int G = p.group;  // chosen by the host (gspmm_group)
  a.G = G;
  a.S = (int)((nvec + G - 1) / G);
  a.num_chunks = p.num_chunks;
  a.chunk_row = p.chunk_row;
  a.chunk_start = p.chunk_start;
  a.chunk_len = p.num_chunks > 0 ? p.chunk_len : 0x7fffffff;
  a.part_val = static_cast<T*>(p.part_val);
  a.part_u = p.part_u;
  a.part_e = p.part_e;
  const int64_t per_wave = WAVE / G;
  a.chunk_uwaves = (p.num_chunks + per_wave - 1) / per_wave;
  a.row_uwaves = (p.num_rows + per_wave - 1) / per_wave;
  a.chunk_waves = a.chunk_uwaves * a.S;
  a.row_waves = a.row_uwaves * a.S;
  a.slab_major = a.S > 1;
  a.chunk_blocks = (a.chunk_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  a.num_blocks = a.chunk_blocks + (a.row_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  a.rowop = static_cast<const T*>(p.rowop);
  a.dot_out = static_cast<T*>(p.dot_out);
  a.dot_lanes = p.dot_lanes;
  a.rows = p.rows;
  a.row_limit = p.row_limit;
  if (a.num_blocks > 0) {
    const bool copy_l = OP == OP_COPY_LHS, copy_r = OP == OP_COPY_RHS;
    const int lm = copy_r ? a.rmode : a.lmode;
    const int rm = copy_l ? a.lmode : a.rmode;
    const dim3 grid((unsigned)a.num_blocks), block(BLOCK);
    // edge rows are streamed (NT = true: every caller gathers them by edge
    // id or reads each once in CSR order)
    bool launched = false;
    if constexpr (OP == OP_MUL && RED == RED_SUM) {
      if (p.dot_out) {
        // the caller checked: contiguous lhs rows, rhs splat over the groups
        if (a.G == WAVE)
          hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_WIDE_CS_DOT, true>), grid, block, 0,
                             p.stream, a);
        else
          hipLaunchKernelGGL((gspmm_kernel<T, OP, RED, VEC, P_PACK_DYN_DOT, true>), grid, block,
                             0, p.stream, a);
        launched = true;
      }
    }
    if (!launched) launch_path<T, OP, RED, VEC, true>(a, grid, block, lm, rm, p.stream);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (p.num_heavy > 0) {
    const int64_t n = p.num_heavy * p.dout;
    hipLaunchKernelGGL((gspmm_combine_kernel<T, RED>), dim3((unsigned)((n + BLOCK - 1) / BLOCK)),
                       dim3(BLOCK), 0, p.stream, p.heavy_rows, p.heavy_ptr, p.indptr, p.deg,
                       static_cast<const T*>(p.part_val), p.part_u, p.part_e,
                       static_cast<T*>(p.out), p.arg_u, p.arg_e, p.num_heavy, p.dout, p.flags);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <class T, int RED, int VEC>
hipError_t launch_gspmm_vec(const GspmmParams& p) {
  switch (p.op) {
    case OP_ADD: return launch_gspmm_op<T, OP_ADD, RED, VEC>(p);
    case OP_SUB: return launch_gspmm_op<T, OP_SUB, RED, VEC>(p);
    case OP_MUL: return launch_gspmm_op<T, OP_MUL, RED, VEC>(p);
    case OP_DIV: return launch_gspmm_op<T, OP_DIV, RED, VEC>(p);
    case OP_COPY_LHS: return launch_gspmm_op<T, OP_COPY_LHS, RED, VEC>(p);
    case OP_COPY_RHS: return launch_gspmm_op<T, OP_COPY_RHS, RED, VEC>(p);
    default: return hipErrorInvalidValue;
  }
}

template <class T, int RED>
hipError_t launch_gspmm_red(const GspmmParams& p) {
  if (p.vec == VecOf<T>::n) return launch_gspmm_vec<T, RED, VecOf<T>::n>(p);
  if constexpr (VecOf<T>::n == 4) {
    if (p.vec == 2) return launch_gspmm_vec<T, RED, 2>(p);  // 8-byte lanes (even widths)
  } else {
    if (p.vec == 4) return launch_gspmm_vec<T, RED, 4>(p);  // 32-byte float64 lanes
  }
  return launch_gspmm_vec<T, RED, 1>(p);
}

}  // namespace mdgl

#define MDGL_INSTANTIATE_GSPMM(T, RED) \
  template hipError_t mdgl::launch_gspmm_red<T, RED>(const mdgl::GspmmParams&);
