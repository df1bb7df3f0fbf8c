// CPU oracle for the message-passing kernel layer.
//
// TEST INFRASTRUCTURE ONLY. This file is a restatement, in plain C++, of the
// reference's CPU kernels (src/ported.mojo) and is used as the parity checker
// by tests/, by __graft_entry__.smoke() and as the CPU-baseline leg of
// bench.py. The product library (libmdgl.so) never links, loads or calls it.
//
// What is restated, and from where:
//   * arithmetic and fold order of every kernel: src/ported.mojo (cited per
//     function below). Each output element is a sequential left fold in the
//     order the reference walks it: CSR order for gspmm / edge_softmax, row
//     order for the segment kernels, `k` order for gather_mm / segment_mm.
//   * the static split of the output axis into WORKERS contiguous chunks once
//     the axis holds PARALLEL_MIN elements (ported.mojo:34-42). The split
//     cannot change a value; it is kept so that the CPU-baseline timing uses
//     the reference's threading.
//   * the `vec` decision of src/capi.mojo:85-87: it only changes arithmetic for
//     gsddmm `dot`, whose vector path keeps W lane partials and reduces them
//     once per edge (ported.mojo:273-293). W = 4, the float64 SIMD width of the
//     AVX2 machine the reference was measured on.
//
// Extensions beyond the reference (the reference API refuses these inputs):
//   * NumPy broadcasting through per-output-column offset tables
//     (lhs_off/rhs_off, in units of `red`-long vectors), the scheme of
//     upstream DGL's BcastOff. With null tables the kernels are exactly the
//     reference's (dl == dr == dout).
//   * arg outputs for gspmm max/min: strict comparison, first in CSR order
//     wins (= smallest edge id among ties), NaN never selected, -1 when no
//     message was selected (a row with no in-edges, or only messages that
//     never beat the identity). The reference emits no arg indices at all.
//   * float32 instantiations; the reference is float64 only.
//
// Parity status of each function is listed in oracle/README.txt.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

constexpr int64_t PARALLEL_MIN = 4096;  // ported.mojo:42
constexpr int W = 4;                     // AVX2 float64 width (capi.mojo:85)

int g_workers = 32;  // ported.mojo:40

enum { SRC = 0, DST = 1, EDGE = 2 };                                   // ported.mojo:45-47
enum { OP_ADD = 0, OP_SUB, OP_MUL, OP_DIV, OP_DOT, OP_COPY_LHS, OP_COPY_RHS };  // :50-57
enum { RED_SUM = 0, RED_MAX, RED_MIN, RED_MEAN };                      // :62-65

// Runs body(lo, hi) over [0, n) split into g_workers contiguous chunks when
// n >= PARALLEL_MIN, else serially (ported.mojo:159-167 and every kernel).
template <class F>
void split(int64_t n, F body) {
  if (n >= PARALLEL_MIN && g_workers > 1) {
    std::vector<std::thread> ts;
    ts.reserve(g_workers);
    for (int t = 0; t < g_workers; ++t) {
      int64_t lo = n * t / g_workers, hi = n * (t + 1) / g_workers;
      ts.emplace_back([=] { body(lo, hi, t); });
    }
    for (auto& th : ts) th.join();
  } else {
    body(0, n, 0);
  }
}

template <class T>
inline T seed(int red) {  // ported.mojo:76-81
  if (red == RED_MAX) return -std::numeric_limits<T>::infinity();
  if (red == RED_MIN) return std::numeric_limits<T>::infinity();
  return T(0);
}

template <class T>
inline T message(int op, T x, T y) {  // ported.mojo:92-105
  switch (op) {
    case OP_ADD: return x + y;
    case OP_SUB: return x - y;
    case OP_MUL: return x * y;
    case OP_DIV: return x / y;
    case OP_COPY_LHS: return x;
    default: return y;
  }
}

// The message of one (lhs element, rhs element) pair, reading only the
// operand(s) the op uses. A copy op's missing operand aliases the present one
// (spmm.py:64-69, sddmm.py:354-361), whose row count need not fit the other
// role's index (node rows indexed by edge id), so it must not be read.
template <class T>
inline T message_at(int op, const T* lhs, int64_t li, const T* rhs, int64_t ri) {
  if (op == OP_COPY_LHS) return lhs[li];
  if (op == OP_COPY_RHS) return rhs[ri];
  return message<T>(op, lhs[li], rhs[ri]);
}

// ---------------------------------------------------------------- array ops
void cumsum(const int64_t* src, int64_t* dst, int64_t n) {  // ported.mojo:145-151
  int64_t acc = 0;
  for (int64_t i = 0; i < n; ++i) {
    acc += src[i];
    dst[i] = acc;
  }
}

template <class T>
void replace_inf_with_zero(const T* src, T* dst, int64_t n) {  // ported.mojo:157-177
  split(n, [&](int64_t lo, int64_t hi, int) {
    for (int64_t i = lo; i < hi; ++i) {
      T v = src[i];
      if (std::isinf(v)) v = T(0);
      dst[i] = v;
    }
  });
}

void clamp_i64(const int64_t* src, int64_t* dst, int64_t n, int64_t lo, int64_t hi) {  // :181-190
  for (int64_t i = 0; i < n; ++i) {
    int64_t v = src[i];
    if (v < lo) v = lo;
    else if (v > hi) v = hi;
    dst[i] = v;
  }
}

// ---------------------------------------------------------------- gsddmm
// ported.mojo:204-329. Output column o reads lhs vector lhs_off[o] and rhs
// vector rhs_off[o] of its operand rows; for every op but dot a vector is one
// element (red == 1); for dot it is `red` elements contracted with W lane
// partials when red % W == 0, then a scalar tail (ported.mojo:273-293).
template <class T>
void gsddmm(const int64_t* uids, const int64_t* vids, const T* lhs, const T* rhs, T* dst,
            int64_t num_edges, int lt, int rt, int op, int64_t dl, int64_t dr, int64_t dout,
            const int64_t* lhs_off, const int64_t* rhs_off, int64_t red) {
  const bool vec = (red % W) == 0;
  split(num_edges, [&](int64_t e0, int64_t e1, int) {
    for (int64_t e = e0; e < e1; ++e) {
      int64_t li = (lt == SRC ? uids[e] : lt == DST ? vids[e] : e) * dl;
      int64_t ri = (rt == SRC ? uids[e] : rt == DST ? vids[e] : e) * dr;
      for (int64_t o = 0; o < dout; ++o) {
        int64_t lo = li + (lhs_off ? lhs_off[o] : o) * red;
        int64_t ro = ri + (rhs_off ? rhs_off[o] : o) * red;
        if (op == OP_DOT) {
          int64_t k = 0;
          T acc = 0;
          if (vec) {
            T lane[W] = {0, 0, 0, 0};
            for (; k + W <= red; k += W)
              for (int j = 0; j < W; ++j) lane[j] = lane[j] + lhs[lo + k + j] * rhs[ro + k + j];
            acc = (lane[0] + lane[2]) + (lane[1] + lane[3]);  // halving reduce_add
          }
          for (; k < red; ++k) acc = acc + lhs[lo + k] * rhs[ro + k];
          dst[e * dout + o] = acc;
        } else {
          dst[e * dout + o] = message_at<T>(op, lhs, lo, rhs, ro);
        }
      }
    }
  });
}

// ---------------------------------------------------------------- gspmm
// ported.mojo:352-548: out[v, o] = red_{i in [indptr[v], indptr[v+1])} op(
// lhs[indices[i]], rhs[eid[i]]) folded in CSR order; mean divides the sum by
// max(deg[v], 1); a row with no in-edges keeps the reduce identity.
template <class T>
void gspmm(const int64_t* indptr, const int64_t* indices, const int64_t* eid, const T* lhs,
           const T* rhs, T* dst, int64_t num_dst, int op, int64_t dl, int64_t dr, int64_t dout,
           int reduce_op, const int64_t* deg, const int64_t* lhs_off, const int64_t* rhs_off,
           int64_t* arg_u, int64_t* arg_e) {
  const bool mean = reduce_op == RED_MEAN;
  const int red = mean ? RED_SUM : reduce_op;
  split(num_dst, [&](int64_t v0, int64_t v1, int) {
    for (int64_t v = v0; v < v1; ++v) {
      const int64_t start = indptr[v], stop = indptr[v + 1];
      T scale = 1;
      if (mean) {
        scale = T(deg[v]);
        if (scale < T(1)) scale = T(1);
      }
      for (int64_t o = 0; o < dout; ++o) {
        const int64_t lo = lhs_off ? lhs_off[o] : o;
        const int64_t ro = rhs_off ? rhs_off[o] : o;
        T acc = seed<T>(red);
        int64_t au = -1, ae = -1;
        for (int64_t i = start; i < stop; ++i) {
          T m = message_at<T>(op, lhs, indices[i] * dl + lo, rhs, eid[i] * dr + ro);
          if (red == RED_MAX) {
            if (m > acc) { acc = m; au = indices[i]; ae = eid[i]; }
          } else if (red == RED_MIN) {
            if (m < acc) { acc = m; au = indices[i]; ae = eid[i]; }
          } else {
            acc = acc + m;
          }
        }
        if (mean && start < stop) acc = acc / scale;
        dst[v * dout + o] = acc;
        if (arg_u) arg_u[v * dout + o] = au;
        if (arg_e) arg_e[v * dout + o] = ae;
      }
    }
  });
}

// ---------------------------------------------------------------- segments
// ported.mojo:559-647, offsets clamped into [0, n] as at :599-607.
template <class T>
void segment_reduce(const int64_t* offsets, const T* value, T* dst, int64_t num_seg, int64_t d,
                    int reduce_op, int64_t n) {
  split(num_seg, [&](int64_t s0, int64_t s1, int) {
    for (int64_t s = s0; s < s1; ++s) {
      int64_t start = offsets[s], stop = offsets[s + 1];
      if (start < 0) start = 0;
      if (stop > n) stop = n;
      if (stop < start) stop = start;
      for (int64_t k = 0; k < d; ++k) {
        T acc = seed<T>(reduce_op);
        for (int64_t i = start; i < stop; ++i) {
          T x = value[i * d + k];
          if (reduce_op == RED_MAX) acc = (x > acc) ? x : acc;
          else if (reduce_op == RED_MIN) acc = (x < acc) ? x : acc;
          else acc = acc + x;
        }
        dst[s * d + k] = acc;
      }
    }
  });
}

// ported.mojo:660-768: per segment and column, pass 1 max, pass 2 exp(x - max)
// written to dst and summed in row order, pass 3 divide. An empty segment
// writes nothing.
template <class T>
void segment_softmax(const int64_t* offsets, const T* value, T* dst, int64_t num_seg, int64_t d,
                     int64_t n) {
  split(num_seg, [&](int64_t s0, int64_t s1, int) {
    std::vector<T> mx(d), sm(d);
    for (int64_t s = s0; s < s1; ++s) {
      int64_t start = offsets[s], stop = offsets[s + 1];
      if (start < 0) start = 0;
      if (stop > n) stop = n;
      if (stop < start) stop = start;
      for (int64_t k = 0; k < d; ++k) mx[k] = -std::numeric_limits<T>::infinity();
      for (int64_t i = start; i < stop; ++i)
        for (int64_t k = 0; k < d; ++k) {
          T x = value[i * d + k];
          mx[k] = (x > mx[k]) ? x : mx[k];
        }
      for (int64_t k = 0; k < d; ++k) sm[k] = (start == stop) ? T(1) : T(0);
      for (int64_t i = start; i < stop; ++i)
        for (int64_t k = 0; k < d; ++k) {
          T e = std::exp(value[i * d + k] - mx[k]);
          dst[i * d + k] = e;
          sm[k] = sm[k] + e;
        }
      for (int64_t i = start; i < stop; ++i)
        for (int64_t k = 0; k < d; ++k) dst[i * d + k] = dst[i * d + k] / sm[k];
    }
  });
}

// ported.mojo:773-804: serial walk over segments; out[row] = a[row] @ b[seg]
// with the contraction summed in k order.
template <class T>
void segment_mm(const T* a, const T* b, T* dst, const int64_t* seglen, int64_t n, int64_t d1,
                int64_t r, int64_t d2) {
  (void)n;
  int64_t row = 0;
  for (int64_t seg = 0; seg < r; ++seg) {
    int64_t end = row + seglen[seg];
    for (; row < end; ++row)
      for (int64_t j = 0; j < d2; ++j) {
        T acc = 0;
        for (int64_t k = 0; k < d1; ++k) acc = acc + a[row * d1 + k] * b[(seg * d1 + k) * d2 + j];
        dst[row * d2 + j] = acc;
      }
  }
}

// ported.mojo:1089-1130: out[i] = a[i] @ b[idx_b[i]], k order.
template <class T>
void gather_mm(const T* a, const T* b, const int64_t* idx_b, T* dst, int64_t n, int64_t d1,
               int64_t d2) {
  split(n, [&](int64_t i0, int64_t i1, int) {
    for (int64_t i = i0; i < i1; ++i) {
      const int64_t o = idx_b[i] * d1 * d2;
      for (int64_t j = 0; j < d2; ++j) {
        T acc = 0;
        for (int64_t k = 0; k < d1; ++k) acc = acc + a[i * d1 + k] * b[o + k * d2 + j];
        dst[i * d2 + j] = acc;
      }
    }
  });
}

// ---------------------------------------------------------------- edge_softmax
// ported.mojo:876-1080. Per CSR row, per column: max over the selected edges,
// then exp(x - max) written and summed in CSR order, then divide; a row whose
// edges are all unselected zero-fills the selected ones (none, so nothing).
// The d == 1 register variant (:994-1080) has the same arithmetic.
template <class T>
void edge_softmax(const int64_t* indptr, const int64_t* eid, const int8_t* mask, const T* logits,
                  T* dst, int64_t num_nodes, int all_ones, int64_t d) {
  split(num_nodes, [&](int64_t i0, int64_t i1, int) {
    std::vector<T> mx(d), sm(d);
    for (int64_t i = i0; i < i1; ++i) {
      const int64_t start = indptr[i], stop = indptr[i + 1];
      if (start >= stop) continue;
      for (int64_t h = 0; h < d; ++h) mx[h] = -std::numeric_limits<T>::infinity();
      bool any = false;
      for (int64_t j = start; j < stop; ++j) {
        const int64_t e = eid[j];
        if (all_ones != 1 && mask[e] != 1) continue;
        any = true;
        for (int64_t h = 0; h < d; ++h) {
          T x = logits[e * d + h];
          mx[h] = (x > mx[h]) ? x : mx[h];
        }
      }
      if (!any) continue;  // no selected edge: nothing of this row is written
      for (int64_t h = 0; h < d; ++h) sm[h] = 0;
      for (int64_t j = start; j < stop; ++j) {
        const int64_t e = eid[j];
        if (all_ones != 1 && mask[e] != 1) continue;
        for (int64_t h = 0; h < d; ++h) {
          T v = std::exp(logits[e * d + h] - mx[h]);
          dst[e * d + h] = v;
          sm[h] = sm[h] + v;
        }
      }
      for (int64_t j = start; j < stop; ++j) {
        const int64_t e = eid[j];
        if (all_ones != 1 && mask[e] != 1) continue;
        for (int64_t h = 0; h < d; ++h) dst[e * d + h] = dst[e * d + h] / sm[h];
      }
    }
  });
}

}  // namespace

// ------------------------------------------------------------------ C ABI
// dtype: 0 = float32, 1 = float64. Index arrays are int64, as in the
// reference's ABI (capi.mojo).
#define ORACLE_DISPATCH(dtype, CALL_F, CALL_D) \
  do {                                         \
    if ((dtype) == 0) { CALL_F; } else { CALL_D; } \
  } while (0)

extern "C" {

int oracle_set_workers(int w) {
  if (w >= 1) g_workers = w;
  return g_workers;
}

int oracle_workers(void) { return g_workers; }

void oracle_cumsum(const int64_t* src, int64_t* dst, int64_t n) { cumsum(src, dst, n); }

void oracle_clamp_i64(const int64_t* src, int64_t* dst, int64_t n, int64_t lo, int64_t hi) {
  clamp_i64(src, dst, n, lo, hi);
}

void oracle_replace_inf_with_zero(const void* src, void* dst, int64_t n, int dtype) {
  ORACLE_DISPATCH(dtype, replace_inf_with_zero((const float*)src, (float*)dst, n),
                  replace_inf_with_zero((const double*)src, (double*)dst, n));
}

void oracle_gsddmm(const int64_t* uids, const int64_t* vids, const void* lhs, const void* rhs,
                   void* dst, int64_t num_edges, int lt, int rt, int op, int64_t dl, int64_t dr,
                   int64_t dout, const int64_t* lhs_off, const int64_t* rhs_off, int64_t red,
                   int dtype) {
  ORACLE_DISPATCH(dtype,
                  gsddmm(uids, vids, (const float*)lhs, (const float*)rhs, (float*)dst, num_edges,
                         lt, rt, op, dl, dr, dout, lhs_off, rhs_off, red),
                  gsddmm(uids, vids, (const double*)lhs, (const double*)rhs, (double*)dst,
                         num_edges, lt, rt, op, dl, dr, dout, lhs_off, rhs_off, red));
}

void oracle_gspmm(const int64_t* indptr, const int64_t* indices, const int64_t* eid,
                  const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op, int64_t dl,
                  int64_t dr, int64_t dout, int reduce_op, const int64_t* deg,
                  const int64_t* lhs_off, const int64_t* rhs_off, int64_t* arg_u, int64_t* arg_e,
                  int dtype) {
  ORACLE_DISPATCH(dtype,
                  gspmm(indptr, indices, eid, (const float*)lhs, (const float*)rhs, (float*)dst,
                        num_dst, op, dl, dr, dout, reduce_op, deg, lhs_off, rhs_off, arg_u, arg_e),
                  gspmm(indptr, indices, eid, (const double*)lhs, (const double*)rhs,
                        (double*)dst, num_dst, op, dl, dr, dout, reduce_op, deg, lhs_off, rhs_off,
                        arg_u, arg_e));
}

void oracle_segment_reduce(const int64_t* offsets, const void* value, void* dst, int64_t num_seg,
                           int64_t d, int reduce_op, int64_t n, int dtype) {
  ORACLE_DISPATCH(dtype,
                  segment_reduce(offsets, (const float*)value, (float*)dst, num_seg, d, reduce_op, n),
                  segment_reduce(offsets, (const double*)value, (double*)dst, num_seg, d, reduce_op,
                                 n));
}

void oracle_segment_softmax(const int64_t* offsets, const void* value, void* dst, int64_t num_seg,
                            int64_t d, int64_t n, int dtype) {
  ORACLE_DISPATCH(dtype,
                  segment_softmax(offsets, (const float*)value, (float*)dst, num_seg, d, n),
                  segment_softmax(offsets, (const double*)value, (double*)dst, num_seg, d, n));
}

void oracle_segment_mm(const void* a, const void* b, void* dst, const int64_t* seglen, int64_t n,
                       int64_t d1, int64_t r, int64_t d2, int dtype) {
  ORACLE_DISPATCH(dtype,
                  segment_mm((const float*)a, (const float*)b, (float*)dst, seglen, n, d1, r, d2),
                  segment_mm((const double*)a, (const double*)b, (double*)dst, seglen, n, d1, r,
                             d2));
}

void oracle_gather_mm(const void* a, const void* b, const int64_t* idx_b, void* dst, int64_t n,
                      int64_t d1, int64_t d2, int dtype) {
  ORACLE_DISPATCH(dtype,
                  gather_mm((const float*)a, (const float*)b, idx_b, (float*)dst, n, d1, d2),
                  gather_mm((const double*)a, (const double*)b, idx_b, (double*)dst, n, d1, d2));
}

void oracle_edge_softmax(const int64_t* indptr, const int64_t* eid, const int8_t* mask,
                         const void* logits, void* dst, int64_t num_nodes, int all_ones, int64_t d,
                         int dtype) {
  ORACLE_DISPATCH(dtype,
                  edge_softmax(indptr, eid, mask, (const float*)logits, (float*)dst, num_nodes,
                               all_ones, d),
                  edge_softmax(indptr, eid, mask, (const double*)logits, (double*)dst, num_nodes,
                               all_ones, d));
}

}  // extern "C"
