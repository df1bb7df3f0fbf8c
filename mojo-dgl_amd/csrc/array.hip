// Elementwise and scan helpers: replace_inf_with_zero (src/ported.mojo:157-177),
// clamp on int64 (:181-190) and the inclusive int64 prefix sum (:145-151).
#include "mdgl_kernels.h"

namespace mdgl {

template <class T>
__global__ __launch_bounds__(BLOCK) void replace_inf_kernel(const T* __restrict__ src,
                                                            T* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK) {
    const T v = src[i];
    dst[i] = is_inf(v) ? T(0) : v;
  }
}

__global__ __launch_bounds__(BLOCK) void clamp_kernel(const int64_t* __restrict__ src,
                                                      int64_t* __restrict__ dst, int64_t n,
                                                      int64_t lo, int64_t hi) {
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK) {
    int64_t v = src[i];
    v = v < lo ? lo : (v > hi ? hi : v);
    dst[i] = v;
  }
}

// One workgroup: each thread sums a contiguous span, the span totals are
// scanned in LDS, then every thread rewrites its span with its carry.
// Integer addition is exact, so this equals the sequential prefix sum.
__global__ __launch_bounds__(1024) void cumsum_kernel(const int64_t* __restrict__ src,
                                                      int64_t* __restrict__ dst, int64_t n) {
  __shared__ int64_t tot[1024];
  const int t = threadIdx.x;
  const int64_t span = (n + 1023) / 1024;
  const int64_t lo = t * span < n ? t * span : n;
  const int64_t hi = lo + span < n ? lo + span : n;
  int64_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += src[i];
  tot[t] = s;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int64_t add = t >= off ? tot[t - off] : 0;
    __syncthreads();
    tot[t] += add;
    __syncthreads();
  }
  int64_t acc = t > 0 ? tot[t - 1] : 0;
  for (int64_t i = lo; i < hi; ++i) {
    acc += src[i];
    dst[i] = acc;
  }
}

template <class T>
__global__ __launch_bounds__(BLOCK) void gather_rows_kernel(const T* __restrict__ src,
                                                            const int32_t* __restrict__ idx,
                                                            T* __restrict__ dst, int64_t n,
                                                            int64_t width) {
  const int64_t total = n * width;
  for (int64_t t = (int64_t)blockIdx.x * BLOCK + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * BLOCK) {
    const int64_t i = t / width, k = t % width;
    dst[t] = src[(int64_t)idx[i] * width + k];
  }
}

static unsigned grid_for(int64_t n) {
  int64_t b = (n + BLOCK - 1) / BLOCK;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_replace_inf(const void* src, void* dst, int64_t n, int dtype, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(replace_inf_kernel<float>, dim3(grid_for(n)), dim3(BLOCK), 0, s,
                       static_cast<const float*>(src), static_cast<float*>(dst), n);
  else
    hipLaunchKernelGGL(replace_inf_kernel<double>, dim3(grid_for(n)), dim3(BLOCK), 0, s,
                       static_cast<const double*>(src), static_cast<double*>(dst), n);
  return hipGetLastError();
}

hipError_t launch_clamp_i64(const int64_t* src, int64_t* dst, int64_t n, int64_t lo, int64_t hi,
                            hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(clamp_kernel, dim3(grid_for(n)), dim3(BLOCK), 0, s, src, dst, n, lo, hi);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const void* src, const int32_t* idx, void* dst, int64_t n,
                              int64_t width, int dtype, hipStream_t s) {
  if (n <= 0 || width <= 0) return hipSuccess;
  const int64_t total = n * width;
  if (dtype == 0)
    hipLaunchKernelGGL(gather_rows_kernel<float>, dim3(grid_for(total)), dim3(BLOCK), 0, s,
                       static_cast<const float*>(src), idx, static_cast<float*>(dst), n, width);
  else
    hipLaunchKernelGGL(gather_rows_kernel<double>, dim3(grid_for(total)), dim3(BLOCK), 0, s,
                       static_cast<const double*>(src), idx, static_cast<double*>(dst), n, width);
  return hipGetLastError();
}

hipError_t launch_cumsum_i64(const int64_t* src, int64_t* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(cumsum_kernel, dim3(1), dim3(1024), 0, s, src, dst, n);
  return hipGetLastError();
}

}  // namespace mdgl
