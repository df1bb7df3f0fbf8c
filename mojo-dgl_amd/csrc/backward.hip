// Elementwise pieces of the backward passes of gspmm / gsddmm /
// edge_softmax. The reductions of those passes run through the forward
// kernels (gspmm over the in- or out-CSR, gsddmm over the edges); what they
// cannot express lives here:
//
//   edge_grad:   m[e, k] = alpha * g[v(e), k] / (mean ? max(deg v(e), 1) : 1)
//                          * (arg_e ? [arg_e[v(e), k] == e] : 1)
//                the message gradient of a max / min (only the arg edge of an
//                output element receives it) or mean reduction, per edge;
//   rows_by_degree: y[r, k] = x[r, k] / max(indptr[r + 1] - indptr[r], 1)
//                (the mean's divisor applied to a node-shaped gradient);
//   scale:       y = alpha * x (alpha = -1 for the sub / div gradients);
//   softmax_grad: dx = a * (g - s[row]) (edge_softmax, s the row sums of g * a).
//
// One multiply, divide or select per element, so the results are exact
// functions of the inputs (no order-dependent sums).
#include "mdgl_kernels.h"

namespace mdgl {

namespace {

unsigned grid_n(int64_t n) {
  int64_t b = (n + BLOCK - 1) / BLOCK;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

template <class T>
__global__ __launch_bounds__(BLOCK) void edge_grad_kernel(
    const int32_t* __restrict__ vids, const int32_t* __restrict__ indptr,
    const T* __restrict__ g, const int32_t* __restrict__ arg_e, T* __restrict__ m,
    int64_t num_edges, int64_t d, T alpha, int mean) {
  const int64_t total = num_edges * d;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t e = i / d, k = i % d;
    const int64_t v = vids[e];
    T x = g[v * d + k];
    if (mean) {
      const int32_t deg = indptr[v + 1] - indptr[v];
      x = x / T(deg > 1 ? deg : 1);
    }
    if (arg_e && arg_e[v * d + k] != (int32_t)e) x = T(0);
    m[i] = alpha * x;
  }
}

template <class T>
__global__ __launch_bounds__(BLOCK) void rows_by_degree_kernel(const int32_t* __restrict__ indptr,
                                                               const T* __restrict__ x,
                                                               T* __restrict__ y, int64_t rows,
                                                               int64_t d) {
  const int64_t total = rows * d;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t r = i / d;
    const int32_t deg = indptr[r + 1] - indptr[r];
    y[i] = x[i] / T(deg > 1 ? deg : 1);
  }
}

template <class T>
__global__ __launch_bounds__(BLOCK) void scale_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                      int64_t n, T alpha) {
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK)
    y[i] = alpha * x[i];
}

// y[i] = mask[i] != 0 ? x[i] : 0. The terms of a max / min gradient that
// come from an edge no output selected are exactly zero, even where x holds
// 0 times an infinite or NaN operand.
template <class T>
__global__ __launch_bounds__(BLOCK) void keep_where_kernel(const T* __restrict__ mask,
                                                           const T* __restrict__ x,
                                                           T* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK)
    y[i] = mask[i] != T(0) ? x[i] : T(0);
}

// dx[e, k] = a[e, k] * (g[e, k] - s[row_of[e], k]): the last two steps of
// the edge_softmax gradient in one pass (coalesced edge rows, one row of s
// per edge).
template <class T>
__global__ __launch_bounds__(BLOCK) void softmax_grad_kernel(const int32_t* __restrict__ row_of,
                                                             const T* __restrict__ a,
                                                             const T* __restrict__ g,
                                                             const T* __restrict__ s,
                                                             T* __restrict__ dx, int64_t num_edges,
                                                             int64_t d) {
  const int64_t total = num_edges * d;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t e = i / d, k = i % d;
    const T t = g[i] - s[(int64_t)row_of[e] * d + k];
    dx[i] = a[i] * t;
  }
}

// The same with 16-byte chunks (d a multiple of the chunk, buffers 16-byte
// aligned): a and g stream in and dx streams out, s is an ordinary load
// (rows of it are shared by an edge's neighbours in the same row).
template <class T, bool POW2>
__global__ __launch_bounds__(BLOCK) void softmax_grad_vec_kernel(
    const int32_t* __restrict__ row_of, const T* __restrict__ a, const T* __restrict__ g,
    const T* __restrict__ s, T* __restrict__ dx, int64_t num_edges, int64_t cpr, int shift) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t total = num_edges * cpr;
  for (int64_t t = (int64_t)blockIdx.x * BLOCK + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * BLOCK) {
    const int64_t e = POW2 ? (t >> shift) : t / cpr;
    const int64_t c = t - e * cpr;
    T av[VEC], gv[VEC], sv[VEC];
    load_n_stream<T, VEC>(a + t * VEC, av);
    load_n_stream<T, VEC>(g + t * VEC, gv);
    load_n<T, VEC>(s + ((int64_t)row_of[e] * cpr + c) * VEC, sv);
#pragma unroll
    for (int v = 0; v < VEC; ++v) av[v] = av[v] * (gv[v] - sv[v]);
    store_n_stream<T, VEC>(dx + t * VEC, av);
  }
}

template <class T>
void softmax_grad_vec(const int32_t* row_of, const T* a, const T* g, const T* s, T* dx,
                      int64_t num_edges, int64_t d, hipStream_t st) {
  const int64_t cpr = d / (16 / (int64_t)sizeof(T));
  int shift = 0;
  while (((int64_t)1 << shift) < cpr) ++shift;
  auto* f = ((int64_t)1 << shift) == cpr ? softmax_grad_vec_kernel<T, true>
                                          : softmax_grad_vec_kernel<T, false>;
  hipLaunchKernelGGL(f, dim3(grid_n(num_edges * cpr)), dim3(BLOCK), 0, st, row_of, a, g, s, dx,
                     num_edges, cpr, shift);
}

}  // namespace

hipError_t launch_softmax_grad(const int32_t* row_of, const void* a, const void* g,
                               const void* s, void* dx, int64_t num_edges, int64_t d, int dtype,
                               hipStream_t st) {
  const int64_t n = num_edges * d;
  if (n <= 0) return hipSuccess;
  if (d % (dtype == 0 ? 4 : 2) == 0 && aligned16(a) && aligned16(g) && aligned16(s) &&
      aligned16(dx)) {
    if (dtype == 0)
      softmax_grad_vec(row_of, static_cast<const float*>(a), static_cast<const float*>(g),
                       static_cast<const float*>(s), static_cast<float*>(dx), num_edges, d, st);
    else
      softmax_grad_vec(row_of, static_cast<const double*>(a), static_cast<const double*>(g),
                       static_cast<const double*>(s), static_cast<double*>(dx), num_edges, d, st);
    return hipGetLastError();
  }
  if (dtype == 0)
    hipLaunchKernelGGL(softmax_grad_kernel<float>, dim3(grid_n(n)), dim3(BLOCK), 0, st, row_of,
                       static_cast<const float*>(a), static_cast<const float*>(g),
                       static_cast<const float*>(s), static_cast<float*>(dx), num_edges, d);
  else
    hipLaunchKernelGGL(softmax_grad_kernel<double>, dim3(grid_n(n)), dim3(BLOCK), 0, st, row_of,
                       static_cast<const double*>(a), static_cast<const double*>(g),
                       static_cast<const double*>(s), static_cast<double*>(dx), num_edges, d);
  return hipGetLastError();
}

hipError_t launch_edge_grad(const int32_t* vids, const int32_t* indptr, const void* g,
                            const int32_t* arg_e, void* m, int64_t num_edges, int64_t d,
                            double alpha, int mean, int dtype, hipStream_t s) {
  const int64_t n = num_edges * d;
  if (n <= 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(edge_grad_kernel<float>, dim3(grid_n(n)), dim3(BLOCK), 0, s, vids, indptr,
                       static_cast<const float*>(g), arg_e, static_cast<float*>(m), num_edges, d,
                       (float)alpha, mean);
  else
    hipLaunchKernelGGL(edge_grad_kernel<double>, dim3(grid_n(n)), dim3(BLOCK), 0, s, vids,
                       indptr, static_cast<const double*>(g), arg_e, static_cast<double*>(m),
                       num_edges, d, alpha, mean);
  return hipGetLastError();
}

hipError_t launch_rows_by_degree(const int32_t* indptr, const void* x, void* y, int64_t rows,
                                 int64_t d, int dtype, hipStream_t s) {
  const int64_t n = rows * d;
  if (n <= 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(rows_by_degree_kernel<float>, dim3(grid_n(n)), dim3(BLOCK), 0, s, indptr,
                       static_cast<const float*>(x), static_cast<float*>(y), rows, d);
  else
    hipLaunchKernelGGL(rows_by_degree_kernel<double>, dim3(grid_n(n)), dim3(BLOCK), 0, s, indptr,
                       static_cast<const double*>(x), static_cast<double*>(y), rows, d);
  return hipGetLastError();
}

hipError_t launch_scale(const void* x, void* y, int64_t n, double alpha, int dtype,
                        hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(scale_kernel<float>, dim3(grid_n(n)), dim3(BLOCK), 0, s,
                       static_cast<const float*>(x), static_cast<float*>(y), n, (float)alpha);
  else
    hipLaunchKernelGGL(scale_kernel<double>, dim3(grid_n(n)), dim3(BLOCK), 0, s,
                       static_cast<const double*>(x), static_cast<double*>(y), n, alpha);
  return hipGetLastError();
}

hipError_t launch_keep_where(const void* mask, const void* x, void* y, int64_t n, int dtype,
                             hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(keep_where_kernel<float>, dim3(grid_n(n)), dim3(BLOCK), 0, s,
                       static_cast<const float*>(mask), static_cast<const float*>(x),
                       static_cast<float*>(y), n);
  else
    hipLaunchKernelGGL(keep_where_kernel<double>, dim3(grid_n(n)), dim3(BLOCK), 0, s,
                       static_cast<const double*>(mask), static_cast<const double*>(x),
                       static_cast<double*>(y), n);
  return hipGetLastError();
}

}  // namespace mdgl
