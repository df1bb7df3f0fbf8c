// Shared definitions of the gfx950 message-passing kernels (libmdgl.so).
//
// Layout conventions (all device memory, row-major, caller-owned):
//   * node / edge feature blocks are [rows, width] of float or double;
//   * graph index arrays (CSR row pointers, neighbour ids, edge ids, COO
//     endpoints) are int32: the host converts the reference's int64 ids once
//     per graph and refuses graphs with 2**31 or more nodes or edges;
//   * one wavefront is 64 lanes; every kernel is launched with 256-thread
//     workgroups (4 wavefronts) and maps workgroups to XCDs so that each of
//     the 8 XCDs (own L2 each) walks one contiguous range of the work list.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mdgl {

// Codes shared with the reference ABI (src/ported.mojo:44-65,
// python/mojodgl/_lib.py:65-73).
enum Target { TGT_U = 0, TGT_V = 1, TGT_E = 2 };
enum Op { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2, OP_DIV = 3, OP_DOT = 4, OP_COPY_LHS = 5, OP_COPY_RHS = 6 };
enum Red { RED_SUM = 0, RED_MAX = 1, RED_MIN = 2, RED_MEAN = 3 };

// How one lane reads the VEC output columns it owns from an operand row:
//   CONTIG  the VEC columns read VEC consecutive, VEC-aligned elements (one
//           16-byte load);
//   SPLAT   the VEC columns all read the same element (one scalar load);
//   GATHER  anything else (VEC scalar loads through the broadcast map).
enum Mode { M_CONTIG = 0, M_SPLAT = 1, M_GATHER = 2 };

constexpr int WAVE = 64;
constexpr int BLOCK = 256;
constexpr int WAVES_PER_BLOCK = BLOCK / WAVE;
constexpr int MAX_DIMS = 6;

// NumPy broadcasting of two operands against an output feature shape,
// collapsed to at most MAX_DIMS dims. Output column k (row-major over
// `shape`) reads element sum_d ((k / div[d]) % shape[d]) * stride[d] of the
// operand row; a broadcast dim has stride 0. For dot the contracted last axis
// is not part of `shape`; the strides then count `red`-long vectors.
struct Bcast {
  int nd;
  int64_t shape[MAX_DIMS];
  int64_t div[MAX_DIMS];
  int64_t lstride[MAX_DIMS];
  int64_t rstride[MAX_DIMS];
};

// Every figure here (k, the dims, strides and the offset) is below a feature
// row's width, which the C ABI keeps under 2 GiB, so the divides are 32-bit:
// a 64-bit divide is several times the instructions, and kernels form these
// offsets for every row or task.
__host__ __device__ inline int64_t bcast_off(const Bcast& b, int64_t k, bool lhs) {
  const uint32_t kk = (uint32_t)k;
  uint32_t off = 0;
  for (int d = 0; d < b.nd; ++d) {
    const uint32_t c = (kk / (uint32_t)b.div[d]) % (uint32_t)b.shape[d];
    off += c * (uint32_t)(lhs ? b.lstride[d] : b.rstride[d]);
  }
  return off;
}

template <class T> struct VecOf;
template <> struct VecOf<float> { using type = float4; static constexpr int n = 4; };
template <> struct VecOf<double> { using type = double2; static constexpr int n = 2; };

template <class T, int N> struct Frag { T v[N]; };

// 16-byte load / store of VEC consecutive elements; the host guarantees
// 16-byte alignment before selecting a mode that uses them.
template <class T>
__device__ __forceinline__ void load_vec(const T* p, T (&out)[VecOf<T>::n]) {
  using V = typename VecOf<T>::type;
  V v = *reinterpret_cast<const V*>(p);
  if constexpr (VecOf<T>::n == 4) {
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else {
    out[0] = v.x; out[1] = v.y;
  }
}

template <class T>
__device__ __forceinline__ void store_vec(T* p, const T (&in)[VecOf<T>::n]) {
  using V = typename VecOf<T>::type;
  V v;
  if constexpr (VecOf<T>::n == 4) {
    v.x = in[0]; v.y = in[1]; v.z = in[2]; v.w = in[3];
  } else {
    v.x = in[0]; v.y = in[1];
  }
  *reinterpret_cast<V*>(p) = v;
}

// N consecutive elements (N * sizeof(T) = 8 or 16 bytes) in one load / store;
// the host guarantees the alignment before selecting a mode that uses them.
template <class T, int N>
__device__ __forceinline__ void load_n(const T* p, T (&out)[N]) {
  typedef T V __attribute__((ext_vector_type(N)));
  const V v = *reinterpret_cast<const V*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = v[i];
}

// The same load from memory known to be global: pointers kept in arrays or
// captured by lambdas lose their address space, and a FLAT load would also
// hold up the LDS wait counter.
template <class T, int N>
__device__ __forceinline__ void load_global_n(const T* p, T (&out)[N]) {
  typedef T V __attribute__((ext_vector_type(N)));
  typedef const __attribute__((address_space(1))) V GV;
  const V v = *(GV*)p;
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = v[i];
}

template <class T>
__device__ __forceinline__ T load_global(const T* p) {
  typedef const __attribute__((address_space(1))) T GT;
  return *(GT*)p;
}

template <class T, int N>
__device__ __forceinline__ void store_n(T* p, const T (&in)[N]) {
  typedef T V __attribute__((ext_vector_type(N)));
  V v;
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = in[i];
  *reinterpret_cast<V*>(p) = v;
}

// True when p sits on a 16-byte boundary (the condition of the 16-byte
// vector paths).
__host__ __device__ inline bool aligned16(const void* p) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0;
}

// Streaming (non-temporal) 16-byte store / load: data written or read once,
// kept from displacing reused lines (gathered rows, node tables) in the
// caches.
template <class T, int N>
__device__ __forceinline__ void store_n_stream(T* p, const T (&in)[N]) {
  typedef T V __attribute__((ext_vector_type(N)));
  V v;
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = in[i];
  __builtin_nontemporal_store(v, reinterpret_cast<V*>(p));
}

template <class T, int N>
__device__ __forceinline__ void load_n_stream(const T* p, T (&out)[N]) {
  typedef T V __attribute__((ext_vector_type(N)));
  const V v = __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = v[i];
}

template <class T>
__device__ __forceinline__ T seed(int red) {
  if (red == RED_MAX) return -__builtin_huge_val();
  if (red == RED_MIN) return __builtin_huge_val();
  return T(0);
}

template <int OP, class T>
__device__ __forceinline__ T message(T x, T y) {
  if constexpr (OP == OP_ADD) return x + y;
  else if constexpr (OP == OP_SUB) return x - y;
  else if constexpr (OP == OP_MUL) return x * y;
  else if constexpr (OP == OP_DIV) return x / y;
  else if constexpr (OP == OP_COPY_LHS) return x;
  else return y;
}

template <class T>
__device__ __forceinline__ bool is_inf(T x) {
  return x == T(__builtin_huge_val()) || x == T(-__builtin_huge_val());
}

// Workgroup index remapped so that XCD x (which receives workgroups
// x, x + 8, x + 16, ... from the dispatcher) gets one contiguous range of
// logical indices. A bijection on [0, nb).
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nb) {
  constexpr int64_t X = 8;
  if (nb < X) return b;
  const int64_t q = nb / X, r = nb % X;
  const int64_t xcd = b % X, pos = b / X;
  return xcd < r ? xcd * (q + 1) + pos : r * (q + 1) + (xcd - r) * q + pos;
}

// Max of an int over the 64 lanes (all lanes must be active).
__device__ __forceinline__ int wave_max_int(int v) {
  for (int off = 32; off >= 1; off >>= 1) {
    int o = __shfl_xor(v, off);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int readlane_int(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

__device__ __forceinline__ float readlane_val(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ double readlane_val(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffLL), lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

}  // namespace mdgl
