// Edge-parallel kernel behind gsddmm (included once per dtype).
//
// Elementwise ops: G consecutive lanes (power of two covering the output
// row's vectors, at most 64) own one edge, so a wavefront writes 64 / G
// consecutive output rows with coalesced stores; each lane gathers its VEC
// columns from the two operand rows selected by the targets (u[e], v[e] or
// e itself). One IEEE operation per element, so the result is bit-identical
// to the reference's (src/ported.mojo:295-328).
//
// dot: G lanes own one (edge, output column) pair and split the contracted
// axis `red` between them (VEC consecutive elements per lane per step), then
// add the G lane partials with a butterfly of __shfl_xor; each wavefront
// serves DOT_U rounds of pairs with their loads issued together. The reference keeps
// W lane partials and reduces them once (ported.mojo:273-293), so the two
// agree to rounding, not bit for bit.
#pragma once

#include "mdgl_kernels.h"

namespace mdgl {

template <class T>
struct GsddmmArgs {
  const int32_t* uids;
  const int32_t* vids;
  const T* lhs;
  const T* rhs;
  T* out;
  int64_t num_edges, dl, dr, dout, red;
  Bcast bc;
  int lt, rt, lmode, rmode, out_vec, G, S;
  int64_t num_tasks, num_waves, num_blocks;
};

__device__ __forceinline__ int64_t target_row(int t, const int32_t* u, const int32_t* v, int64_t e) {
  return t == TGT_U ? (int64_t)u[e] : (t == TGT_V ? (int64_t)v[e] : e);
}

template <class T, int VEC>
__device__ __forceinline__ void fetch_rt(const T* __restrict__ row, int mode, const int (&off)[VEC],
                                         T (&x)[VEC]) {
  if (VEC > 1 && mode == M_CONTIG) {
    if constexpr (VEC == VecOf<T>::n) load_vec<T>(row + off[0], x);
  } else if (mode == M_SPLAT) {
    const T s = row[off[0]];
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = s;
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = row[off[v]];
  }
}

// A wavefront takes EW_U rounds of 64 / G edges (one slab of columns) and
// requests every round's operand rows before it computes, so each lane has
// 2 * EW_U row loads in flight.
constexpr int EW_U = 4;

template <class T, int OP, int VEC>
__global__ __launch_bounds__(BLOCK) void gsddmm_kernel(GsddmmArgs<T> a) {
  const int64_t blk = xcd_remap(blockIdx.x, a.num_blocks);
  const int lane = threadIdx.x & (WAVE - 1);
  const int64_t wave = blk * WAVES_PER_BLOCK + (threadIdx.x >> 6);
  if (wave >= a.num_waves) return;
  const int G = a.G;
  const int grp = lane / G, gl = lane % G;
  const int64_t slab = wave % a.S;
  const int64_t per_round = WAVE / G;
  const int64_t e0 = (wave / a.S) * EW_U * per_round + grp;
  const int64_t k0 = (slab * G + gl) * VEC;
  if (k0 >= a.dout) return;

  int loff[VEC], roff[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int64_t k = k0 + v < a.dout ? k0 + v : k0;
    loff[v] = (int)bcast_off(a.bc, k, true);
    roff[v] = (int)bcast_off(a.bc, k, false);
  }
  T x[EW_U][VEC], y[EW_U][VEC];
#pragma unroll
  for (int r = 0; r < EW_U; ++r) {
    const int64_t e = e0 + r * per_round;
    if (e < a.num_edges) {
      if constexpr (OP != OP_COPY_RHS)
        fetch_rt<T, VEC>(a.lhs + target_row(a.lt, a.uids, a.vids, e) * a.dl, a.lmode, loff, x[r]);
      if constexpr (OP != OP_COPY_LHS)
        fetch_rt<T, VEC>(a.rhs + target_row(a.rt, a.uids, a.vids, e) * a.dr, a.rmode, roff, y[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < EW_U; ++r) {
    const int64_t e = e0 + r * per_round;
    if (e >= a.num_edges) break;
    T o[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      T xv = T(0), yv = T(0);
      if constexpr (OP != OP_COPY_RHS) xv = x[r][v];
      if constexpr (OP != OP_COPY_LHS) yv = y[r][v];
      o[v] = message<OP>(xv, yv);
    }
    const int64_t base = e * a.dout + k0;
    if (VEC > 1 && a.out_vec) {
      if constexpr (VEC == VecOf<T>::n) store_n_stream<T, VEC>(a.out + base, o);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (k0 + v < a.dout) a.out[base + v] = o[v];
    }
  }
}

// dot: tasks are (edge, output column) pairs, G lanes per task. A wavefront
// takes DOT_U rounds of 64 / G tasks; when the contracted axis fits in one
// vector per lane (red <= G * VEC) the loads of all rounds are issued before
// the first product, so each lane has 2 * DOT_U row loads in flight.
constexpr int DOT_U = 4;

template <class T, int VEC>
__device__ __forceinline__ T dot_part(const T* __restrict__ l, const T* __restrict__ r,
                                      int64_t k0, int64_t red, int64_t step) {
  T part = T(0);
  for (int64_t k = k0; k < red; k += step) {
    if constexpr (VEC > 1) {
      T xv[VEC], yv[VEC];
      load_global_n<T, VEC>(l + k, xv);
      load_global_n<T, VEC>(r + k, yv);
#pragma unroll
      for (int v = 0; v < VEC; ++v) part = part + xv[v] * yv[v];
    } else {
      part = part + load_global(l + k) * load_global(r + k);
    }
  }
  return part;
}

template <class T, int VEC>
__global__ __launch_bounds__(BLOCK) void gsddmm_dot_kernel(GsddmmArgs<T> a) {
  const int64_t blk = xcd_remap(blockIdx.x, a.num_blocks);
  const int lane = threadIdx.x & (WAVE - 1);
  const int64_t wave = blk * WAVES_PER_BLOCK + (threadIdx.x >> 6);
  if (wave >= a.num_waves) return;  // uniform per wavefront
  const int G = a.G;
  const int grp = lane / G, gl = lane % G;
  const int64_t per_round = WAVE / G;
  const int64_t k0 = (int64_t)gl * VEC;
  int64_t task[DOT_U];
  const T* lp[DOT_U];
  const T* rp[DOT_U];
#pragma unroll
  for (int u = 0; u < DOT_U; ++u) {
    task[u] = (wave * DOT_U + u) * per_round + grp;
    lp[u] = rp[u] = nullptr;
    if (task[u] < a.num_tasks) {
      if (a.dout == 1) {
        // one output column per edge (u_dot_v on (n, d) rows): the task is
        // the edge and the broadcast offsets are 0 -- no 64-bit divides
        lp[u] = a.lhs + target_row(a.lt, a.uids, a.vids, task[u]) * a.dl;
        rp[u] = a.rhs + target_row(a.rt, a.uids, a.vids, task[u]) * a.dr;
      } else {
        const int64_t e = task[u] / a.dout, col = task[u] % a.dout;
        lp[u] = a.lhs + target_row(a.lt, a.uids, a.vids, e) * a.dl +
                bcast_off(a.bc, col, true) * a.red;
        rp[u] = a.rhs + target_row(a.rt, a.uids, a.vids, e) * a.dr +
                bcast_off(a.bc, col, false) * a.red;
      }
    }
  }
  T part[DOT_U];
  if (a.red <= (int64_t)G * VEC) {
    T xv[DOT_U][VEC], yv[DOT_U][VEC];
#pragma unroll
    for (int u = 0; u < DOT_U; ++u) {
      if (lp[u] && k0 < a.red) {
        if constexpr (VEC > 1) {
          load_global_n<T, VEC>(lp[u] + k0, xv[u]);
          load_global_n<T, VEC>(rp[u] + k0, yv[u]);
        } else {
          xv[u][0] = load_global(lp[u] + k0);
          yv[u][0] = load_global(rp[u] + k0);
        }
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) xv[u][v] = yv[u][v] = T(0);
      }
    }
#pragma unroll
    for (int u = 0; u < DOT_U; ++u) {
      T pu = T(0);
#pragma unroll
      for (int v = 0; v < VEC; ++v) pu = pu + xv[u][v] * yv[u][v];
      part[u] = pu;
    }
  } else {
#pragma unroll
    for (int u = 0; u < DOT_U; ++u)
      part[u] = lp[u] ? dot_part<T, VEC>(lp[u], rp[u], k0, a.red, (int64_t)G * VEC) : T(0);
  }
  // butterfly inside the lane group; every lane of the wavefront runs it
#pragma unroll
  for (int u = 0; u < DOT_U; ++u)
    for (int off = G >> 1; off >= 1; off >>= 1) part[u] = part[u] + __shfl_xor(part[u], off);
  if (G >= DOT_U) {
    // the wavefront's DOT_U * 64 / G tasks are consecutive: lane t takes
    // task wave * nt + t from its group's lanes and the results leave as one
    // coalesced store (one partial-line store per round wrote every output
    // line back about five times)
    const int pr = WAVE / G, nt = DOT_U * pr;
    const int su = lane / pr, src = (lane % pr) * G;
    T val = T(0);
#pragma unroll
    for (int u = 0; u < DOT_U; ++u) {
      const T s = __shfl(part[u], src);
      if (su == u) val = s;
    }
    const int64_t t = wave * nt + lane;
    if (lane < nt && t < a.num_tasks) a.out[t] = val;
  } else {
#pragma unroll
    for (int u = 0; u < DOT_U; ++u)
      if (lp[u] && gl == 0) __builtin_nontemporal_store(part[u], a.out + task[u]);
  }
}

template <class T, int VEC>
hipError_t launch_gsddmm_vec(const GsddmmParams& p) {
  GsddmmArgs<T> a;
  a.uids = p.uids;
  a.vids = p.vids;
  a.lhs = static_cast<const T*>(p.lhs);
  a.rhs = static_cast<const T*>(p.rhs);
  a.out = static_cast<T*>(p.out);
  a.num_edges = p.num_edges;
  a.dl = p.dl;
  a.dr = p.dr;
  a.dout = p.dout;
  a.red = p.red;
  a.bc = p.bc;
  a.lt = p.lt;
  a.rt = p.rt;
  a.lmode = p.lmode;
  a.rmode = p.rmode;
  a.out_vec = p.out_vec;
  if (p.op == OP_DOT) {
    const int64_t nvec = (p.red + VEC - 1) / VEC;
    int G = 1;
    while (G < nvec && G < WAVE) G <<= 1;
    a.G = G;
    a.S = 1;
    a.num_tasks = p.num_edges * p.dout;
    const int64_t per_wave = (WAVE / G) * DOT_U;
    a.num_waves = (a.num_tasks + per_wave - 1) / per_wave;
  } else {
    const int64_t nvec = (p.dout + VEC - 1) / VEC;
    int G = 1;
    while (G < nvec && G < WAVE) G <<= 1;
    a.G = G;
    a.S = (int)((nvec + G - 1) / G);
    a.num_tasks = p.num_edges;
    const int64_t per_wave = (WAVE / G) * EW_U;
    a.num_waves = ((p.num_edges + per_wave - 1) / per_wave) * a.S;
  }
  a.num_blocks = (a.num_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  if (a.num_blocks == 0) return hipSuccess;
  const dim3 grid((unsigned)a.num_blocks), block(BLOCK);
  switch (p.op) {
    case OP_ADD: hipLaunchKernelGGL((gsddmm_kernel<T, OP_ADD, VEC>), grid, block, 0, p.stream, a); break;
    case OP_SUB: hipLaunchKernelGGL((gsddmm_kernel<T, OP_SUB, VEC>), grid, block, 0, p.stream, a); break;
    case OP_MUL: hipLaunchKernelGGL((gsddmm_kernel<T, OP_MUL, VEC>), grid, block, 0, p.stream, a); break;
    case OP_DIV: hipLaunchKernelGGL((gsddmm_kernel<T, OP_DIV, VEC>), grid, block, 0, p.stream, a); break;
    case OP_COPY_LHS:
      hipLaunchKernelGGL((gsddmm_kernel<T, OP_COPY_LHS, VEC>), grid, block, 0, p.stream, a);
      break;
    case OP_COPY_RHS:
      hipLaunchKernelGGL((gsddmm_kernel<T, OP_COPY_RHS, VEC>), grid, block, 0, p.stream, a);
      break;
    case OP_DOT: hipLaunchKernelGGL((gsddmm_dot_kernel<T, VEC>), grid, block, 0, p.stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <class T>
hipError_t launch_gsddmm(const GsddmmParams& p) {
  if (p.vec == VecOf<T>::n) return launch_gsddmm_vec<T, VecOf<T>::n>(p);
  return launch_gsddmm_vec<T, 1>(p);
}

}  // namespace mdgl

#define MDGL_INSTANTIATE_GSDDMM(T) \
  template hipError_t mdgl::launch_gsddmm<T>(const mdgl::GsddmmParams&);
