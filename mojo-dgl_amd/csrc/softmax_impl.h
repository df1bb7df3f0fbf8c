// Row softmax over a CSR (included once per dtype). edge_softmax uses the
// in- or out-edge CSR with the edge id of every slot; segment_softmax uses
// the segment offsets with the identity edge id.
//
// For each row and each of the d columns: m = max over the row's selected
// edges, s = sum of exp(x - m), out = exp(x - m) / s, which is the
// reference's three passes (src/ported.mojo:918-987, 679-768). Only the
// order of the max and the sum differs: lanes take strided edges and the
// lane results are combined by a butterfly (and, for heavy rows, across the
// four wavefronts of a workgroup through LDS). A row with no selected edge
// writes nothing.
//
// Lane layout: L lanes cover the row's d columns (VEC per lane, L a power of
// two, at most 64) and a wavefront holds P = 64 / L edge slots. Rows wider
// than 64 * VEC are cut into slabs. Light rows: one wavefront per
// (row, slab), four per workgroup. Rows above heavy_deg: one workgroup each,
// in the first num_heavy workgroups.
#pragma once

#include "mdgl_kernels.h"

namespace mdgl {

template <class T>
struct SoftmaxArgs {
  const int32_t* indptr;
  const int32_t* eid;
  const int8_t* mask;
  const T* logits;
  T* out;
  int64_t num_rows, d;
  int L, S, vec_io;
  int64_t num_heavy;
  const int32_t* heavy_rows;
  int heavy_deg;
  int64_t light_waves, light_blocks;
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

// One (row, slab) by `nw` cooperating wavefronts (1 for light rows, 4 for
// heavy ones). `w` is this wavefront's index among them, `red` the LDS area
// for the cross-wavefront step (heavy only).
template <class T, int VEC>
__device__ __forceinline__ void softmax_row(const SoftmaxArgs<T>& a, int64_t row, int64_t slab,
                                            int w, int nw, int lane, T* red) {
  const int L = a.L, P = WAVE / L;
  const int slot = lane / L, cl = lane % L;
  const int64_t k0 = (slab * L + cl) * VEC;
  const bool feat_ok = k0 < a.d;
  const bool vec_io = a.vec_io;
  const int start = a.indptr[row], stop = a.indptr[row + 1];
  const int step = P * nw;
  const int first = start + w * P + slot;

  // pass 1: max
  T m[VEC];
  int any = 0;
#pragma unroll
  for (int v = 0; v < VEC; ++v) m[v] = T(-__builtin_huge_val());
  for (int j = first; j < stop; j += step) {
    const int64_t e = a.eid ? a.eid[j] : j;
    if (a.mask && a.mask[e] != 1) continue;
    any = 1;
    if (feat_ok) {
      T x[VEC];
      load_cols<T, VEC>(a.logits + e * a.d, k0, a.d, vec_io, x);
#pragma unroll
      for (int v = 0; v < VEC; ++v) m[v] = x[v] > m[v] ? x[v] : m[v];
    }
  }
  for (int off = L; off < WAVE; off <<= 1) {
    any |= __shfl_xor(any, off);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const T o = __shfl_xor(m[v], off);
      m[v] = o > m[v] ? o : m[v];
    }
  }
  if (nw > 1) {
    // lanes of slot 0 publish, then everyone folds the wavefronts in order
    if (slot == 0) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) red[(w * WAVE + cl) * VEC + v] = m[v];
      red[4 * WAVE * VEC + w] = T(any);
    }
    __syncthreads();
    any = 0;
    for (int q = 0; q < nw; ++q) {
      any |= red[4 * WAVE * VEC + q] != T(0);
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const T o = red[(q * WAVE + cl) * VEC + v];
        m[v] = (q == 0 || o > m[v]) ? o : m[v];
      }
    }
    __syncthreads();
  }
  if (!any) return;  // uniform across the row's wavefronts

  // pass 2: sum of exponentials
  T s[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) s[v] = T(0);
  for (int j = first; j < stop; j += step) {
    const int64_t e = a.eid ? a.eid[j] : j;
    if (a.mask && a.mask[e] != 1) continue;
    if (feat_ok) {
      T x[VEC];
      load_cols<T, VEC>(a.logits + e * a.d, k0, a.d, vec_io, x);
#pragma unroll
      for (int v = 0; v < VEC; ++v) s[v] = s[v] + exp_t(x[v] - m[v]);
    }
  }
  for (int off = L; off < WAVE; off <<= 1) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) s[v] = s[v] + __shfl_xor(s[v], off);
  }
  if (nw > 1) {
    if (slot == 0) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) red[(w * WAVE + cl) * VEC + v] = s[v];
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      T t = T(0);
      for (int q = 0; q < nw; ++q) t = t + red[(q * WAVE + cl) * VEC + v];
      s[v] = t;
    }
    __syncthreads();
  }

  // pass 3: write
  if (!feat_ok) return;
  for (int j = first; j < stop; j += step) {
    const int64_t e = a.eid ? a.eid[j] : j;
    if (a.mask && a.mask[e] != 1) continue;
    T x[VEC];
    load_cols<T, VEC>(a.logits + e * a.d, k0, a.d, vec_io, x);
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = exp_t(x[v] - m[v]) / s[v];
    store_cols<T, VEC>(a.out + e * a.d, k0, a.d, vec_io, x);
  }
}

template <class T, int VEC>
__global__ __launch_bounds__(BLOCK) void softmax_kernel(SoftmaxArgs<T> a) {
  __shared__ T red[4 * WAVE * VEC + 4];
  const int lane = threadIdx.x & (WAVE - 1);
  const int w = threadIdx.x >> 6;
  const int64_t b = blockIdx.x;
  if (b < a.num_heavy) {
    const int64_t row = a.heavy_rows[b];
    for (int64_t slab = 0; slab < a.S; ++slab)
      softmax_row<T, VEC>(a, row, slab, w, WAVES_PER_BLOCK, lane, red);
    return;
  }
  const int64_t lb = xcd_remap(b - a.num_heavy, a.light_blocks);
  const int64_t wave = lb * WAVES_PER_BLOCK + w;
  if (wave >= a.light_waves) return;
  const int64_t row = wave / a.S, slab = wave % a.S;
  if (a.num_heavy > 0 && a.indptr[row + 1] - a.indptr[row] > a.heavy_deg) return;
  softmax_row<T, VEC>(a, row, slab, 0, 1, lane, red);
}

template <class T, int VEC>
hipError_t launch_softmax_vec(const SoftmaxParams& p) {
  SoftmaxArgs<T> a;
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
  a.S = (int)((nvec + L - 1) / L);
  a.vec_io = (VEC > 1) && (p.d % VEC == 0);
  a.num_heavy = p.num_heavy;
  a.heavy_rows = p.heavy_rows;
  a.heavy_deg = p.heavy_deg;
  a.light_waves = p.num_rows * a.S;
  a.light_blocks = (a.light_waves + WAVES_PER_BLOCK - 1) / WAVES_PER_BLOCK;
  const int64_t blocks = a.num_heavy + a.light_blocks;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL((softmax_kernel<T, VEC>), dim3((unsigned)blocks), dim3(BLOCK), 0, p.stream, a);
  return hipGetLastError();
}

template <class T>
hipError_t launch_softmax(const SoftmaxParams& p) {
  if (p.vec == VecOf<T>::n) return launch_softmax_vec<T, VecOf<T>::n>(p);
  return launch_softmax_vec<T, 1>(p);
}

}  // namespace mdgl

#define MDGL_INSTANTIATE_SOFTMAX(T) \
  template hipError_t mdgl::launch_softmax<T>(const mdgl::SoftmaxParams&);
