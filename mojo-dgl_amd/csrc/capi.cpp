// C ABI of libmdgl.so (declared in include/mdgl.h).
//
// This file validates arguments (before anything is launched), turns operand
// feature shapes into the collapsed broadcast descriptor, chooses per
// operand how a lane loads its columns (16-byte vector, one splatted scalar,
// or a scalar gather), and dispatches to the kernel launchers.
#include <dlfcn.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mdgl.h"
#include "mdgl_kernels.h"

using namespace mdgl;

namespace {

thread_local std::string g_last_error;

// roctx ranges around the entry points. With MDGL_ROCTX set (to anything but
// "0") when the library first needs it, the ROCm 7 roctx library is opened and
// every entry point that validates or launches pushes a range named after
// itself for the length of the call (host time: validation, workspace layout
// and launches; `rocprofv3 --marker-trace` lists them beside the kernels).
// Otherwise, or when the roctx library is not found, a range costs one load
// and one branch. Ranges are per thread and nest, as roctx's push/pop ranges
// do.
struct Roctx {
  int (*push)(const char*) = nullptr;
  int (*pop)() = nullptr;
};

const Roctx& roctx() {
  static const Roctx r = [] {
    Roctx t;
    const char* on = std::getenv("MDGL_ROCTX");
    if (!on || !*on || std::strcmp(on, "0") == 0) return t;
    void* h = dlopen("librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_LOCAL);
    if (!h) h = dlopen("/opt/rocm/lib/librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_LOCAL);
    if (!h) return t;
    auto push = reinterpret_cast<int (*)(const char*)>(dlsym(h, "roctxRangePushA"));
    auto pop = reinterpret_cast<int (*)()>(dlsym(h, "roctxRangePop"));
    if (push && pop) {
      t.push = push;
      t.pop = pop;
    }
    return t;
  }();
  return r;
}

class Range {
 public:
  explicit Range(const char* name) : pop_(roctx().pop) {
    if (pop_) roctx().push(name);
  }
  ~Range() {
    if (pop_) pop_();
  }
  Range(const Range&) = delete;
  Range& operator=(const Range&) = delete;

 private:
  int (*pop_)();
};

#define MDGL_RANGE() const Range mdgl_range_(__func__)

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MDGL_OK;
  return fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

bool dtype_ok(int dtype) { return dtype == MDGL_FLOAT32 || dtype == MDGL_FLOAT64; }
int64_t dsize(int dtype) { return dtype == MDGL_FLOAT32 ? 4 : 8; }
int vec_width(int dtype) { return dtype == MDGL_FLOAT32 ? 4 : 2; }

bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0;
}

// Workspaces hold vector-accessed arrays at 256-byte offsets: the base must
// be 256-byte aligned (hipMalloc and torch allocations are).
constexpr int64_t WS_ALIGN = 256;

// Builds the broadcast descriptor of two operands whose feature shapes are
// padded to the same rank `nd`. For dot the last axis is contracted and
// `red` receives its length. Returns 0 or a negative MDGL code.
int make_bcast(int nd, const int64_t* ls, const int64_t* rs, bool dot, Bcast* bc, int64_t* red,
               int64_t* lwidth, int64_t* rwidth, int64_t* owidth) {
  std::vector<int64_t> lsh(ls, ls + nd), rsh(rs, rs + nd);
  *red = 1;
  if (dot) {
    if (nd < 1) return fail(MDGL_EINVAL, "dot needs at least one feature axis");
    if (lsh[nd - 1] != rsh[nd - 1])
      return fail(MDGL_EINVAL, "dot needs matching last axes, got %lld and %lld",
                  (long long)lsh[nd - 1], (long long)rsh[nd - 1]);
    *red = lsh[nd - 1];
    lsh.pop_back();
    rsh.pop_back();
  }
  const int n = (int)lsh.size();
  std::vector<int64_t> out(n), lst(n), rst(n);
  int64_t lw = 1, rw = 1, ow = 1;
  for (int d = n - 1; d >= 0; --d) {
    if (lsh[d] < 0 || rsh[d] < 0) return fail(MDGL_EINVAL, "negative feature dimension");
    if (lsh[d] != rsh[d] && lsh[d] != 1 && rsh[d] != 1)
      return fail(MDGL_EINVAL, "feature shapes are not broadcastable at axis %d: %lld vs %lld",
                  d + 1, (long long)lsh[d], (long long)rsh[d]);
    out[d] = lsh[d] == 1 ? rsh[d] : lsh[d];
    lst[d] = (lsh[d] == 1 && out[d] != 1) ? 0 : lw;
    rst[d] = (rsh[d] == 1 && out[d] != 1) ? 0 : rw;
    lw *= lsh[d];
    rw *= rsh[d];
    ow *= out[d];
  }
  *lwidth = lw * *red;
  *rwidth = rw * *red;
  *owidth = ow;
  // collapse: drop size-1 axes, merge neighbours that stay contiguous in both
  std::vector<int64_t> cs, cl, cr;
  for (int d = 0; d < n; ++d) {
    if (out[d] == 1) continue;
    if (!cs.empty() && cl.back() == lst[d] * out[d] && cr.back() == rst[d] * out[d]) {
      cs.back() *= out[d];
      cl.back() = lst[d];
      cr.back() = rst[d];
    } else {
      cs.push_back(out[d]);
      cl.push_back(lst[d]);
      cr.push_back(rst[d]);
    }
  }
  if (cs.empty()) {
    cs.push_back(1);
    cl.push_back(0);
    cr.push_back(0);
  }
  if ((int)cs.size() > MAX_DIMS)
    return fail(MDGL_ENOTSUP, "broadcast needs %d axes after collapsing, at most %d supported",
                (int)cs.size(), MAX_DIMS);
  bc->nd = (int)cs.size();
  int64_t div = 1;
  for (int d = bc->nd - 1; d >= 0; --d) {
    bc->shape[d] = cs[d];
    bc->div[d] = div;
    bc->lstride[d] = cl[d];
    bc->rstride[d] = cr[d];
    div *= cs[d];
  }
  return 0;
}

void identity_bcast(int64_t width, Bcast* bc) {
  bc->nd = 1;
  bc->shape[0] = width > 0 ? width : 1;
  bc->div[0] = 1;
  bc->lstride[0] = 1;
  bc->rstride[0] = 1;
}

// Load mode of one operand for lanes owning `vec` consecutive output
// columns. Contiguous 16-byte loads need aligned rows and groups; with
// `padded` rows (a stride that is a multiple of vec, past the row's width)
// the lane holding the last columns may read a whole vector.
int pick_mode(const Bcast& bc, bool lhs, int64_t dout, int vec, int64_t width, const void* base,
              int64_t esize, bool padded = false) {
  if (vec == 1) return M_CONTIG;  // VEC = 1 kernels load one element whatever the mode
  bool contig = (padded || (dout % vec == 0 && width % vec == 0)) && aligned(base, vec * esize);
  bool splat = true;
  for (int64_t g = 0; g < dout && (contig || splat); g += vec) {
    const int64_t o0 = bcast_off(bc, g, lhs);
    if (o0 % vec != 0) contig = false;
    for (int j = 1; j < vec && g + j < dout; ++j) {
      const int64_t o = bcast_off(bc, g + j, lhs);
      if (o != o0 + j) contig = false;
      if (o != o0) splat = false;
    }
  }
  if (contig) return M_CONTIG;
  if (splat) return M_SPLAT;
  return M_GATHER;
}

bool row_widths_fit(int64_t w, int64_t esize) { return w >= 0 && w * esize < (int64_t(1) << 31); }

}  // namespace

extern "C" {

const char* mdgl_last_error(void) { return g_last_error.c_str(); }

int64_t mdgl_workers(void) { return 256; }

int mdgl_trace_ranges(void) { return roctx().pop != nullptr; }

int64_t mdgl_segment_offsets_workspace_bytes(int64_t num) {
  return num < 0 ? -1 : segment_offsets_workspace_bytes(num);
}

int mdgl_segment_offsets(const int64_t* seglen, int64_t num, int64_t chunk_len, int32_t* offsets,
                         int64_t* stats, void* workspace, int64_t workspace_bytes,
                         void* stream) {
  MDGL_RANGE();
  if (num < 0) return fail(MDGL_EINVAL, "segment_offsets: negative count");
  if (num >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "segment_offsets: 2**31 or more segments");
  if (!offsets || !stats || (num > 0 && !seglen))
    return fail(MDGL_EINVAL, "segment_offsets: null buffer");
  const int64_t need = segment_offsets_workspace_bytes(num);
  if (need > 0 && workspace && !aligned(workspace, WS_ALIGN))
    return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(MDGL_EWORKSPACE, "segment_offsets: workspace of %lld bytes needed, %lld given",
                (long long)need, (long long)workspace_bytes);
  return hip_status(launch_segment_offsets(seglen, num, chunk_len, offsets, stats, workspace,
                                           (hipStream_t)stream),
                    "segment_offsets");
}

int mdgl_cumsum(const int64_t* src, int64_t* dst, int64_t n, void* stream) {
  MDGL_RANGE();
  if (n < 0) return fail(MDGL_EINVAL, "cumsum: n must be >= 0");
  if (n > 0 && (!src || !dst)) return fail(MDGL_EINVAL, "cumsum: null buffer");
  return hip_status(launch_cumsum_i64(src, dst, n, (hipStream_t)stream), "cumsum");
}

int64_t mdgl_read_stream_sink_bytes(int64_t bytes) {
  return bytes < 0 ? -1 : read_stream_sink_bytes(bytes);
}

int64_t mdgl_read_rows_sink_bytes(int64_t n) { return n < 0 ? -1 : read_rows_sink_bytes(n); }

int mdgl_read_rows(const void* src, int64_t src_rows, int64_t row_bytes, const int32_t* idx,
                   int64_t n, void* dst, int64_t dst_rows, void* sink, void* stream) {
  MDGL_RANGE();
  if (row_bytes < 16 || row_bytes > 1024 || row_bytes % 16)
    return fail(MDGL_EINVAL, "read_rows: row_bytes must be a multiple of 16 in [16, 1024]");
  if (src_rows < 0 || n < 0 || dst_rows < 0) return fail(MDGL_EINVAL, "read_rows: negative size");
  if (n >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "read_rows: 2**31 or more indices");
  if (n == 0) return MDGL_OK;
  if (!src || !idx || !sink || (dst_rows > 0 && !dst))
    return fail(MDGL_EINVAL, "read_rows: null buffer");
  if (!aligned(src, 16) || !aligned(sink, 16) || (dst_rows > 0 && !aligned(dst, 16)))
    return fail(MDGL_EINVAL, "read_rows: buffers must be 16-byte aligned");
  return hip_status(launch_read_rows(src, src_rows, row_bytes, idx, n, dst, dst_rows, sink,
                                     (hipStream_t)stream),
                    "read_rows");
}

int mdgl_read_stream(const void* src, int64_t bytes, void* sink, void* stream) {
  MDGL_RANGE();
  if (bytes < 0 || bytes % 16) return fail(MDGL_EINVAL, "read_stream: bytes must be a multiple of 16");
  if (bytes == 0) return MDGL_OK;
  if (!src || !sink) return fail(MDGL_EINVAL, "read_stream: null buffer");
  if (!aligned(src, 16) || !aligned(sink, 16))
    return fail(MDGL_EINVAL, "read_stream: buffers must be 16-byte aligned");
  return hip_status(launch_read_stream(src, bytes, sink, (hipStream_t)stream), "read_stream");
}

int64_t mdgl_build_csr_workspace_bytes(int64_t num_edges, int64_t num_rows) {
  if (num_edges < 0 || num_rows < 0) return -1;
  return csr_workspace_bytes(num_edges, num_rows);
}

int mdgl_build_csr(const int32_t* key, const int32_t* other, int64_t num_edges, int64_t num_rows,
                   int32_t* indptr, int32_t* indices, int32_t* eid, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  MDGL_RANGE();
  if (num_edges < 0 || num_rows < 0) return fail(MDGL_EINVAL, "build_csr: negative size");
  if (num_edges >= (int64_t(1) << 31) || num_rows >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "build_csr: 2**31 or more edges or rows");
  if (num_edges > 0 && num_rows == 0)
    return fail(MDGL_EINVAL, "build_csr: edges but no rows");
  if (!indptr || (num_edges > 0 && (!key || !eid)))
    return fail(MDGL_EINVAL, "build_csr: null buffer");
  if (num_edges > 0 && !other != !indices)
    return fail(MDGL_EINVAL, "build_csr: `other` and `indices` come together or not at all");
  const int64_t need = csr_workspace_bytes(num_edges, num_rows);
  if (need > 0 && workspace && !aligned(workspace, WS_ALIGN))
    return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(MDGL_EWORKSPACE, "build_csr: workspace of %lld bytes needed, %lld given",
                (long long)need, (long long)workspace_bytes);
  return hip_status(launch_build_csr(key, other, num_edges, num_rows, indptr, indices, eid,
                                     workspace, (hipStream_t)stream),
                    "build_csr");
}

int mdgl_edge_softmax_grad(const int32_t* row_of, const void* a, const void* grad,
                           const void* row_sum, void* dst, int64_t num_edges, int64_t d, int dtype,
                           void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "edge_softmax_grad: bad dtype %d", dtype);
  if (num_edges < 0 || d < 0) return fail(MDGL_EINVAL, "edge_softmax_grad: negative size");
  if (num_edges >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "edge_softmax_grad: 2**31 or more edges");
  if (num_edges == 0 || d == 0) return MDGL_OK;
  if (!row_of || !a || !grad || !row_sum || !dst)
    return fail(MDGL_EINVAL, "edge_softmax_grad: null buffer");
  return hip_status(launch_softmax_grad(row_of, a, grad, row_sum, dst, num_edges, d, dtype,
                                        (hipStream_t)stream),
                    "edge_softmax_grad");
}

int mdgl_gspmm_edge_grad(const int32_t* vids, const int32_t* indptr, const void* grad_out,
                         const int32_t* arg_e, void* dst, int64_t num_edges, int64_t d, int mean,
                         double alpha, int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "gspmm_edge_grad: bad dtype %d", dtype);
  if (num_edges < 0 || d < 0) return fail(MDGL_EINVAL, "gspmm_edge_grad: negative size");
  if (num_edges >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "gspmm_edge_grad: 2**31 or more edges");
  if (num_edges == 0 || d == 0) return MDGL_OK;
  if (!vids || !grad_out || !dst || (mean && !indptr))
    return fail(MDGL_EINVAL, "gspmm_edge_grad: null buffer");
  return hip_status(launch_edge_grad(vids, indptr, grad_out, arg_e, dst, num_edges, d, alpha,
                                     mean, dtype, (hipStream_t)stream),
                    "gspmm_edge_grad");
}

int mdgl_rows_by_degree(const int32_t* indptr, const void* src, void* dst, int64_t rows,
                        int64_t d, int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "rows_by_degree: bad dtype %d", dtype);
  if (rows < 0 || d < 0) return fail(MDGL_EINVAL, "rows_by_degree: negative size");
  if (rows == 0 || d == 0) return MDGL_OK;
  if (!indptr || !src || !dst) return fail(MDGL_EINVAL, "rows_by_degree: null buffer");
  return hip_status(launch_rows_by_degree(indptr, src, dst, rows, d, dtype, (hipStream_t)stream),
                    "rows_by_degree");
}

int mdgl_gather_rows(const void* src, const int32_t* idx, void* dst, int64_t n, int64_t width,
                     int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "gather_rows: bad dtype %d", dtype);
  if (n < 0 || width < 0) return fail(MDGL_EINVAL, "gather_rows: negative size");
  if (n == 0 || width == 0) return MDGL_OK;
  if (!src || !idx || !dst) return fail(MDGL_EINVAL, "gather_rows: null buffer");
  return hip_status(launch_gather_rows(src, idx, dst, n, width, dtype, (hipStream_t)stream),
                    "gather_rows");
}

int mdgl_scatter_rows(const void* src, const int32_t* idx, void* dst, int64_t n, int64_t width,
                      int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "scatter_rows: bad dtype %d", dtype);
  if (n < 0 || width < 0) return fail(MDGL_EINVAL, "scatter_rows: negative size");
  if (n == 0 || width == 0) return MDGL_OK;
  if (!src || !idx || !dst) return fail(MDGL_EINVAL, "scatter_rows: null buffer");
  return hip_status(launch_gather_rows(src, idx, dst, n, width, dtype, (hipStream_t)stream, true),
                    "scatter_rows");
}

int mdgl_keep_where(const void* mask, const void* src, void* dst, int64_t n, int dtype,
                    void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "keep_where: bad dtype %d", dtype);
  if (n < 0) return fail(MDGL_EINVAL, "keep_where: n must be >= 0");
  if (n > 0 && (!mask || !src || !dst)) return fail(MDGL_EINVAL, "keep_where: null buffer");
  return hip_status(launch_keep_where(mask, src, dst, n, dtype, (hipStream_t)stream),
                    "keep_where");
}

int mdgl_scale(const void* src, void* dst, int64_t n, double alpha, int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "scale: bad dtype %d", dtype);
  if (n < 0) return fail(MDGL_EINVAL, "scale: n must be >= 0");
  if (n > 0 && (!src || !dst)) return fail(MDGL_EINVAL, "scale: null buffer");
  return hip_status(launch_scale(src, dst, n, alpha, dtype, (hipStream_t)stream), "scale");
}

int mdgl_replace_inf_with_zero(const void* src, void* dst, int64_t n, int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "replace_inf_with_zero: bad dtype %d", dtype);
  if (n < 0) return fail(MDGL_EINVAL, "replace_inf_with_zero: n must be >= 0");
  if (n > 0 && (!src || !dst)) return fail(MDGL_EINVAL, "replace_inf_with_zero: null buffer");
  return hip_status(launch_replace_inf(src, dst, n, dtype, (hipStream_t)stream),
                    "replace_inf_with_zero");
}

int mdgl_clamp_i64(const int64_t* src, int64_t* dst, int64_t n, int64_t lo, int64_t hi,
                   void* stream) {
  MDGL_RANGE();
  if (n < 0) return fail(MDGL_EINVAL, "clamp_i64: n must be >= 0");
  if (n > 0 && (!src || !dst)) return fail(MDGL_EINVAL, "clamp_i64: null buffer");
  return hip_status(launch_clamp_i64(src, dst, n, lo, hi, (hipStream_t)stream), "clamp_i64");
}

int mdgl_gsddmm(const int32_t* uids, const int32_t* vids, const void* lhs, const void* rhs,
                void* dst, int64_t num_edges, int lhs_target, int rhs_target, int op, int64_t dl,
                int64_t dr, int64_t dout, int nd, const int64_t* lhs_shape,
                const int64_t* rhs_shape, int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "gsddmm: bad dtype %d", dtype);
  if (op < OP_ADD || op > OP_COPY_RHS) return fail(MDGL_EINVAL, "gsddmm: bad op %d", op);
  if (lhs_target < 0 || lhs_target > 2 || rhs_target < 0 || rhs_target > 2)
    return fail(MDGL_EINVAL, "gsddmm: targets must be 0 (u), 1 (v) or 2 (e)");
  if (num_edges < 0 || dl < 0 || dr < 0 || dout < 0)
    return fail(MDGL_EINVAL, "gsddmm: negative size");
  if (num_edges >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "gsddmm: 2**31 or more edges");
  const int64_t es = dsize(dtype);
  if (!row_widths_fit(dl, es) || !row_widths_fit(dr, es) || !row_widths_fit(dout, es))
    return fail(MDGL_EINVAL, "gsddmm: feature rows of 2 GiB or more");
  GsddmmParams p{};
  p.uids = uids;
  p.vids = vids;
  p.lhs = lhs;
  p.rhs = rhs;
  p.out = dst;
  p.num_edges = num_edges;
  p.dl = dl;
  p.dr = dr;
  p.dout = dout;
  p.lt = lhs_target;
  p.rt = rhs_target;
  p.op = op;
  p.stream = (hipStream_t)stream;
  const bool dot = op == OP_DOT;
  const bool copy = op == OP_COPY_LHS || op == OP_COPY_RHS;
  if (copy) {
    const int64_t w = op == OP_COPY_LHS ? dl : dr;
    if (dout != w) return fail(MDGL_EINVAL, "gsddmm: copy output width %lld != operand width %lld",
                               (long long)dout, (long long)w);
    identity_bcast(dout, &p.bc);
    p.red = 1;
  } else if (nd > 0) {
    if (!lhs_shape || !rhs_shape) return fail(MDGL_EINVAL, "gsddmm: null shape");
    int64_t lw, rw, ow;
    int rc = make_bcast(nd, lhs_shape, rhs_shape, dot, &p.bc, &p.red, &lw, &rw, &ow);
    if (rc) return rc;
    if (lw != dl || rw != dr || ow != dout)
      return fail(MDGL_EINVAL, "gsddmm: widths (%lld, %lld, %lld) do not match the shapes "
                  "(%lld, %lld, %lld)", (long long)dl, (long long)dr, (long long)dout,
                  (long long)lw, (long long)rw, (long long)ow);
  } else {
    if (dot) {
      if (dl != dr || dout != 1) return fail(MDGL_EINVAL, "gsddmm: dot needs dl == dr, dout == 1");
      identity_bcast(1, &p.bc);
      p.bc.lstride[0] = p.bc.rstride[0] = 0;
      p.red = dl;
    } else {
      if (dl != dr || dl != dout)
        return fail(MDGL_EINVAL, "gsddmm: without shapes dl, dr and dout must be equal");
      identity_bcast(dout, &p.bc);
      p.red = 1;
    }
  }
  const bool need_u = (op != OP_COPY_RHS && lhs_target == TGT_U) ||
                      (op != OP_COPY_LHS && rhs_target == TGT_U);
  const bool need_v = (op != OP_COPY_RHS && lhs_target == TGT_V) ||
                      (op != OP_COPY_LHS && rhs_target == TGT_V);
  if (num_edges > 0 && dout > 0) {
    if (!dst) return fail(MDGL_EINVAL, "gsddmm: null output");
    if ((need_u && !uids) || (need_v && !vids)) return fail(MDGL_EINVAL, "gsddmm: null ids");
    if ((op != OP_COPY_RHS && !lhs) || (op != OP_COPY_LHS && !rhs))
      return fail(MDGL_EINVAL, "gsddmm: null operand");
  } else {
    return MDGL_OK;
  }
  const int vw = vec_width(dtype);
  if (dot) {
    p.vec = (p.red % vw == 0 && dl % vw == 0 && dr % vw == 0 && aligned(lhs, vw * es) &&
             aligned(rhs, vw * es)) ? vw : 1;
    p.lmode = p.rmode = M_CONTIG;
    p.out_vec = 0;
  } else {
    p.vec = dout % vw == 0 ? vw : 1;
    p.lmode = op == OP_COPY_RHS ? M_CONTIG : pick_mode(p.bc, true, dout, p.vec, dl, lhs, es);
    p.rmode = op == OP_COPY_LHS ? M_CONTIG : pick_mode(p.bc, false, dout, p.vec, dr, rhs, es);
    p.out_vec = p.vec > 1 && aligned(dst, p.vec * es);
  }
  hipError_t e = dtype == MDGL_FLOAT32 ? launch_gsddmm<float>(p) : launch_gsddmm<double>(p);
  return hip_status(e, "gsddmm");
}

int64_t mdgl_gspmm_workspace_bytes(int64_t num_chunks, int64_t dout, int reduce_op, int dtype) {
  if (num_chunks <= 0) return 0;
  const int64_t n = num_chunks * dout;
  int64_t bytes = ((n * dsize(dtype) + 255) / 256) * 256;
  if (reduce_op == RED_MAX || reduce_op == RED_MIN) bytes += 2 * (((n * 4) + 255) / 256) * 256;
  return bytes;
}

}  // extern "C"

namespace {

// Lane width and operand load modes of a gspmm (p.bc and p.lstride set):
// 16-byte lanes when the width allows (or the node rows are padded to
// lines, so the last lane may read a whole vector of them), else 8-byte
// lanes for even float32 widths, else one element per lane; a lane whose
// columns straddle broadcast groups (heads of 2, 3, 6 columns ...) would
// gather element by element through the any-layout kernel, so narrower
// lanes keep compile-time layouts (per-element offsets at one element per
// lane: on a 60M-edge graph, 48 columns as 8 heads of 6 with one weight per
// head, 12.0 -> 3.8 ms; 12 columns as 4 heads of 3, 7.4 -> 2.7 ms).
void choose_gspmm_lanes(GspmmParams& p, int op, int64_t dl, int64_t dr, int64_t dout,
                        const void* lhs, const void* rhs, int64_t es, int dtype, bool dot) {
  const int vw = vec_width(dtype);
  const bool lined = p.lstride != dl;  // node rows on 128-byte lines
  p.vec = (dout % vw == 0 || (lined && !dot)) ? vw
          : (dtype == MDGL_FLOAT32 && dout % 2 == 0 ? 2 : 1);
  p.lmode = op == OP_COPY_RHS ? M_CONTIG : pick_mode(p.bc, true, dout, p.vec, dl, lhs, es, lined);
  p.rmode = op == OP_COPY_LHS ? M_CONTIG : pick_mode(p.bc, false, dout, p.vec, dr, rhs, es);
  // float64 rows of 129-256 columns: 32-byte lanes (two 16-byte loads each)
  // make one 64-lane slab, so the row's edges are walked once instead of twice
  if (dtype == MDGL_FLOAT64 && !dot && p.vec == vw && dout > WAVE * vw && dout <= 2 * WAVE * vw &&
      dout % (2 * vw) == 0 && p.lmode != M_GATHER && p.rmode != M_GATHER) {
    const int lm = op == OP_COPY_RHS ? M_CONTIG : pick_mode(p.bc, true, dout, 2 * vw, dl, lhs, es, lined);
    const int rm = op == OP_COPY_LHS ? M_CONTIG : pick_mode(p.bc, false, dout, 2 * vw, dr, rhs, es);
    if (lm != M_GATHER && rm != M_GATHER) {
      p.vec = 2 * vw;
      p.lmode = lm;
      p.rmode = rm;
    }
  }
  if (!dot && !lined && p.vec > 1 && (p.lmode == M_GATHER || p.rmode == M_GATHER)) {
    for (int nv = p.vec / 2; nv >= 1; nv /= 2) {
      if (nv > 1 && dout % nv != 0) continue;
      const int lm = op == OP_COPY_RHS ? M_CONTIG : pick_mode(p.bc, true, dout, nv, dl, lhs, es);
      const int rm = op == OP_COPY_LHS ? M_CONTIG : pick_mode(p.bc, false, dout, nv, dr, rhs, es);
      if (lm != M_GATHER && rm != M_GATHER) {
        p.vec = nv;
        p.lmode = lm;
        p.rmode = rm;
        break;
      }
    }
  }
}

// Lanes per row slab: the power of two covering the row's vectors, at most
// 64. With MDGL_NARROW_SLABS, rows wider than 64 vectors take 32-lane slabs
// (two rows per wavefront) when that makes at most GSPMM_NARROW_MAX_SLABS of
// them: each slab walks all of a row's edges again, and on a graph whose
// sources lie near their destinations the 512-byte slabs of a block of
// neighbouring rows stay in an XCD's 4 MB L2 where 1 KB slabs do not
// (float32 602-column rows: 3 -> 5 walks, 10-14 % faster on a 50-block
// community graph; float64 ones: 5 -> 10 walks, 1-4 % slower, so excluded).
constexpr int GSPMM_NARROW_MAX_SLABS = 5;
int gspmm_group(int64_t dout, int vec, int flags, bool dot) {
  const int64_t nvec = (dout + vec - 1) / vec;
  int gmax = WAVE;
  if ((flags & MDGL_NARROW_SLABS) && !dot && nvec > WAVE &&
      (nvec + WAVE / 2 - 1) / (WAVE / 2) <= GSPMM_NARROW_MAX_SLABS)
    gmax = WAVE / 2;
  int g = 1;
  while (g < nvec && g < gmax) g <<= 1;
  return g;
}

// The broadcast descriptor of a gspmm's operands (copy ops and nd = 0: the
// identity); 0 or a failure status.
int gspmm_bcast(int op, int64_t dl, int64_t dr, int64_t dout, int nd, const int64_t* lhs_shape,
                const int64_t* rhs_shape, Bcast* bc) {
  if (op == OP_COPY_LHS || op == OP_COPY_RHS) {
    const int64_t w = op == OP_COPY_LHS ? dl : dr;
    if (dout != w) return fail(MDGL_EINVAL, "gspmm: copy output width %lld != operand width %lld",
                               (long long)dout, (long long)w);
    identity_bcast(dout, bc);
  } else if (nd > 0) {
    if (!lhs_shape || !rhs_shape) return fail(MDGL_EINVAL, "gspmm: null shape");
    int64_t red, lw, rw, ow;
    int rc = make_bcast(nd, lhs_shape, rhs_shape, false, bc, &red, &lw, &rw, &ow);
    if (rc) return rc;
    if (lw != dl || rw != dr || ow != dout)
      return fail(MDGL_EINVAL, "gspmm: widths (%lld, %lld, %lld) do not match the shapes "
                  "(%lld, %lld, %lld)", (long long)dl, (long long)dr, (long long)dout,
                  (long long)lw, (long long)rw, (long long)ow);
  } else {
    if (dl != dr || dl != dout)
      return fail(MDGL_EINVAL, "gspmm: without shapes dl, dr and dout must be equal");
    identity_bcast(dout, bc);
  }
  return MDGL_OK;
}

// gspmm proper.
int gspmm_common(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                 const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op, int64_t dl,
                 int64_t dr, int64_t dout, int reduce_op, const int32_t* deg, int nd,
                 const int64_t* lhs_shape, const int64_t* rhs_shape, int32_t* arg_u,
                 int32_t* arg_e, const int32_t* chunk_row, const int32_t* chunk_start,
                 int64_t num_chunks, int32_t chunk_len, const int32_t* heavy_rows,
                 const int32_t* heavy_ptr, int64_t num_heavy, void* workspace,
                 int64_t workspace_bytes, int flags, int dtype, void* stream,
                 const void* rowop = nullptr, void* dot_out = nullptr,
                 const int32_t* rows = nullptr, int64_t num_listed = -1) {
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "gspmm: bad dtype %d", dtype);
  if (op < OP_ADD || op > OP_COPY_RHS || op == OP_DOT)
    return fail(MDGL_EINVAL, "gspmm: bad op %d (dot is a gsddmm operator)", op);
  if (reduce_op < RED_SUM || reduce_op > RED_MEAN)
    return fail(MDGL_EINVAL, "gspmm: bad reduce_op %d", reduce_op);
  if (num_dst < 0 || dl < 0 || dr < 0 || dout < 0) return fail(MDGL_EINVAL, "gspmm: negative size");
  if (num_dst >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "gspmm: 2**31 or more rows");
  const int64_t es = dsize(dtype);
  if (!row_widths_fit(dl, es) || !row_widths_fit(dr, es) || !row_widths_fit(dout, es))
    return fail(MDGL_EINVAL, "gspmm: feature rows of 2 GiB or more");
  if (num_chunks < 0 || num_heavy < 0) return fail(MDGL_EINVAL, "gspmm: negative chunk counts");
  if (num_chunks > 0 && (chunk_len <= 0 || !chunk_row || !chunk_start || num_heavy <= 0 ||
                         !heavy_rows || !heavy_ptr))
    return fail(MDGL_EINVAL, "gspmm: incomplete heavy-row schedule");
  if (num_chunks == 0 && num_heavy != 0)
    return fail(MDGL_EINVAL, "gspmm: heavy rows without chunks");
  const bool listed = num_listed >= 0;  // mdgl_gspmm_rows
  if (listed && num_listed >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "gspmm_rows: 2**31 or more rows listed");
  if (listed && num_listed > 0 && !rows) return fail(MDGL_EINVAL, "gspmm_rows: null rows");
  GspmmParams p{};
  p.indptr = indptr;
  p.indices = indices;
  p.eid = eid;
  p.deg = deg;
  p.lhs = lhs;
  p.rhs = rhs;
  p.out = dst;
  p.num_rows = num_dst;
  p.dl = dl;
  p.lstride = dl;
  p.dr = dr;
  p.dout = dout;
  p.op = op;
  p.red = reduce_op == RED_MEAN ? RED_SUM : reduce_op;
  p.flags = (reduce_op == RED_MEAN ? F_MEAN : 0) | ((flags & MDGL_REPLACE_INF) ? F_REPLACE_INF : 0) |
            ((flags & MDGL_RHS_CSR_ORDER) ? F_RHS_CSR : 0);
  const bool arg = reduce_op == RED_MAX || reduce_op == RED_MIN;
  p.arg_u = arg ? arg_u : nullptr;
  p.arg_e = arg ? arg_e : nullptr;
  p.stream = (hipStream_t)stream;
  if (int rc = gspmm_bcast(op, dl, dr, dout, nd, lhs_shape, rhs_shape, &p.bc)) return rc;
  if (num_dst == 0 || dout == 0 || num_listed == 0) return MDGL_OK;
  if (listed) {
    p.rows = rows;
    p.row_limit = num_dst;
    p.num_rows = num_listed;
  }
  if (!indptr || !dst) return fail(MDGL_EINVAL, "gspmm: null indptr or output");
  if (op != OP_COPY_LHS && !eid) return fail(MDGL_EINVAL, "gspmm: null eid");
  if (op != OP_COPY_RHS && !indices) return fail(MDGL_EINVAL, "gspmm: null indices");
  if ((op != OP_COPY_RHS && !lhs) || (op != OP_COPY_LHS && !rhs))
    return fail(MDGL_EINVAL, "gspmm: null operand");
  if (arg && p.arg_e && !eid) return fail(MDGL_EINVAL, "gspmm: arg_e needs eid");
  if (arg && p.arg_u && !indices) return fail(MDGL_EINVAL, "gspmm: arg_u needs indices");
  // copy_lhs without edge ids never reads edge data: slot ids stand in
  if (op == OP_COPY_LHS && !eid) p.flags |= F_EID_IDENTITY;
  if (op == OP_COPY_RHS && !p.arg_u) p.indices = nullptr;
  p.num_chunks = num_chunks;
  p.chunk_row = chunk_row;
  p.chunk_start = chunk_start;
  p.chunk_len = chunk_len;
  p.num_heavy = num_heavy;
  p.heavy_rows = heavy_rows;
  p.heavy_ptr = heavy_ptr;
  if (num_chunks > 0) {
    const int64_t need = mdgl_gspmm_workspace_bytes(num_chunks, dout, reduce_op, dtype);
    if (workspace && !aligned(workspace, WS_ALIGN))
      return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
    if (!workspace || workspace_bytes < need)
      return fail(MDGL_EWORKSPACE, "gspmm: workspace of %lld bytes needed, %lld given",
                  (long long)need, (long long)workspace_bytes);
    char* w = static_cast<char*>(workspace);
    const int64_t n = num_chunks * dout;
    p.part_val = w;
    w += ((n * es + 255) / 256) * 256;
    if (arg) {
      p.part_u = reinterpret_cast<int32_t*>(w);
      w += ((n * 4 + 255) / 256) * 256;
      p.part_e = reinterpret_cast<int32_t*>(w);
    }
  }
  if ((flags & MDGL_LHS_LINE_ROWS) && op != OP_COPY_RHS) {
    if (!aligned(lhs, 128))
      return fail(MDGL_EINVAL, "gspmm: MDGL_LHS_LINE_ROWS needs lhs on a 128-byte boundary");
    p.lstride = (dl * es + 127) / 128 * 128 / es;
  }
  const int vw = vec_width(dtype);
  choose_gspmm_lanes(p, op, dl, dr, dout, lhs, rhs, es, dtype, dot_out != nullptr);
  p.group = gspmm_group(dout, p.vec, flags, dot_out != nullptr);
  if (p.vec > 1 && dout % p.vec == 0 && aligned(dst, p.vec * es)) p.flags |= F_OUT_VEC;
  if (dot_out) {
    // the fused dot: mul / sum, 16-byte lanes, lhs rows contiguous, the edge
    // operand constant over groups of D = dout / dr consecutive columns
    // (D / vec lanes, a power of two up to 64), the row operand aligned
    if (op != OP_MUL || reduce_op != RED_SUM)
      return fail(MDGL_EINVAL, "gspmm dot: mul with sum only");
    if (!rowop) return fail(MDGL_EINVAL, "gspmm dot: null row operand");
    if (dr <= 0 || dout % dr != 0)
      return fail(MDGL_EINVAL, "gspmm dot: dout %lld is not a multiple of dr %lld",
                  (long long)dout, (long long)dr);
    const int64_t D = dout / dr;
    const int64_t lanes = D / vw;
    bool ok = p.vec == vw && D % vw == 0 && lanes <= WAVE && (lanes & (lanes - 1)) == 0 &&
              p.lmode == M_CONTIG && aligned(rowop, vw * es);
    for (int64_t k = 0; ok && k < dout; ++k)
      ok = bcast_off(p.bc, k, false) == k / D && bcast_off(p.bc, k, true) == k;
    if (!ok)
      return fail(MDGL_ENOTSUP, "gspmm dot: needs contiguous aligned rows and the edge operand "
                  "splat over power-of-two groups of 16-byte lanes");
    p.rowop = rowop;
    p.dot_out = dot_out;
    p.dot_lanes = (int)lanes;
    p.rmode = M_SPLAT;
  }
  hipError_t e;
  if (dtype == MDGL_FLOAT32) {
    e = p.red == RED_MAX ? launch_gspmm_red<float, RED_MAX>(p)
        : p.red == RED_MIN ? launch_gspmm_red<float, RED_MIN>(p)
                           : launch_gspmm_red<float, RED_SUM>(p);
  } else {
    e = p.red == RED_MAX ? launch_gspmm_red<double, RED_MAX>(p)
        : p.red == RED_MIN ? launch_gspmm_red<double, RED_MIN>(p)
                           : launch_gspmm_red<double, RED_SUM>(p);
  }
  return hip_status(e, "gspmm");
}

}  // namespace

extern "C" {

int mdgl_gspmm(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
               const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op, int64_t dl,
               int64_t dr, int64_t dout, int reduce_op, const int32_t* deg, int nd,
               const int64_t* lhs_shape, const int64_t* rhs_shape, int32_t* arg_u,
               int32_t* arg_e, const int32_t* chunk_row, const int32_t* chunk_start,
               int64_t num_chunks, int32_t chunk_len, const int32_t* heavy_rows,
               const int32_t* heavy_ptr, int64_t num_heavy, void* workspace,
               int64_t workspace_bytes, int flags, int dtype, void* stream) {
  MDGL_RANGE();
  return gspmm_common(indptr, indices, eid, lhs, rhs, dst, num_dst, op, dl, dr, dout, reduce_op,
                      deg, nd, lhs_shape, rhs_shape, arg_u, arg_e, chunk_row, chunk_start,
                      num_chunks, chunk_len, heavy_rows, heavy_ptr, num_heavy, workspace,
                      workspace_bytes, flags, dtype, stream);
}

int mdgl_gspmm_rows(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                    const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op,
                    int64_t dl, int64_t dr, int64_t dout, int reduce_op, const int32_t* deg,
                    int nd, const int64_t* lhs_shape, const int64_t* rhs_shape, int32_t* arg_u,
                    int32_t* arg_e, const int32_t* rows, int64_t num_rows, int flags, int dtype,
                    void* stream) {
  MDGL_RANGE();
  if (num_rows < 0) return fail(MDGL_EINVAL, "gspmm_rows: negative row count");
  // every listed row whole, in one unit (no heavy-row schedule)
  return gspmm_common(indptr, indices, eid, lhs, rhs, dst, num_dst, op, dl, dr, dout, reduce_op,
                      deg, nd, lhs_shape, rhs_shape, arg_u, arg_e, nullptr, nullptr, 0, 0,
                      nullptr, nullptr, 0, nullptr, 0, flags, dtype, stream, nullptr, nullptr,
                      rows, num_rows);
}

int mdgl_gspmm_lanes(int op, int64_t dl, int64_t dr, int64_t dout, int nd,
                     const int64_t* lhs_shape, const int64_t* rhs_shape, const void* lhs,
                     const void* rhs, int flags, int dtype, int64_t* vec, int64_t* group) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "gspmm_lanes: bad dtype %d", dtype);
  if (op < OP_ADD || op > OP_COPY_RHS || op == OP_DOT)
    return fail(MDGL_EINVAL, "gspmm_lanes: bad op %d", op);
  if (dl < 0 || dr < 0 || dout < 0 || !vec) return fail(MDGL_EINVAL, "gspmm_lanes: bad arguments");
  GspmmParams p{};
  if (int rc = gspmm_bcast(op, dl, dr, dout, nd, lhs_shape, rhs_shape, &p.bc)) return rc;
  const int64_t es = dsize(dtype);
  p.lstride = dl;
  if ((flags & MDGL_LHS_LINE_ROWS) && op != OP_COPY_RHS) {
    if (!aligned(lhs, 128))
      return fail(MDGL_EINVAL, "gspmm_lanes: MDGL_LHS_LINE_ROWS needs lhs on a 128-byte boundary");
    p.lstride = (dl * es + 127) / 128 * 128 / es;
  }
  choose_gspmm_lanes(p, op, dl, dr, dout, lhs, rhs, es, dtype, false);
  *vec = p.vec;
  if (group) *group = gspmm_group(dout, p.vec, flags, false);
  return MDGL_OK;
}

static_assert(MDGL_COO_LOCALITY_BLOCKS == COO_LOCALITY_BLOCKS, "one count per workgroup");

int mdgl_coo_locality(const int32_t* u, const int32_t* v, int64_t num_edges, int64_t window,
                      int64_t* partial, void* stream) {
  MDGL_RANGE();
  if (num_edges < 0 || window < 0) return fail(MDGL_EINVAL, "coo_locality: negative size");
  if (!partial) return fail(MDGL_EINVAL, "coo_locality: null output");
  if (num_edges > 0 && (!u || !v)) return fail(MDGL_EINVAL, "coo_locality: null endpoints");
  return hip_status(launch_coo_locality(u, v, num_edges, window, partial, (hipStream_t)stream),
                    "coo_locality");
}

int mdgl_gspmm_mul_sum_dot(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                           const void* lhs, const void* rhs, const void* rowop, void* dst,
                           void* dot, int64_t num_dst, int64_t dl, int64_t dr, int64_t dout,
                           int nd, const int64_t* lhs_shape, const int64_t* rhs_shape,
                           const int32_t* chunk_row, const int32_t* chunk_start,
                           int64_t num_chunks, int32_t chunk_len, const int32_t* heavy_rows,
                           const int32_t* heavy_ptr, int64_t num_heavy, void* workspace,
                           int64_t workspace_bytes, int dtype, void* stream) {
  MDGL_RANGE();
  if (num_dst > 0 && dout > 0 && !dot) return fail(MDGL_EINVAL, "gspmm dot: null dot output");
  return gspmm_common(indptr, indices, eid, lhs, rhs, dst, num_dst, OP_MUL, dl, dr, dout, RED_SUM,
                      nullptr, nd, lhs_shape, rhs_shape, nullptr, nullptr, chunk_row, chunk_start,
                      num_chunks, chunk_len, heavy_rows, heavy_ptr, num_heavy, workspace,
                      workspace_bytes, 0, dtype, stream, rowop, dot);
}

namespace {

// segment_reduce and its arg form (arg null: none)
int segment_common(const char* what, const int32_t* offsets, const void* value, void* dst,
                   int32_t* arg, int64_t num_seg, int64_t d, int reduce_op, int64_t n, int flags,
                   int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "%s: bad dtype %d", what, dtype);
  if (reduce_op < RED_SUM || reduce_op > RED_MEAN)
    return fail(MDGL_EINVAL, "%s: bad reduce_op %d", what, reduce_op);
  const int pass_flags = flags & (MDGL_SEGMENTS_SHORT | MDGL_SEGMENTS_SKIP_LONG |
                                  MDGL_SEGMENTS_LONG_ONLY);
  if (pass_flags & (pass_flags - 1))
    return fail(MDGL_EINVAL, "%s: at most one of MDGL_SEGMENTS_SHORT, MDGL_SEGMENTS_SKIP_LONG "
                "and MDGL_SEGMENTS_LONG_ONLY", what);
  if (num_seg < 0 || d < 0 || n < 0) return fail(MDGL_EINVAL, "%s: negative size", what);
  if (num_seg >= (int64_t(1) << 31) || n >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "%s: 2**31 or more segments or rows", what);
  if (!row_widths_fit(d, dsize(dtype))) return fail(MDGL_EINVAL, "%s: rows too wide", what);
  if (num_seg == 0 || d == 0) return MDGL_OK;
  if (!offsets || !dst || (n > 0 && !value)) return fail(MDGL_EINVAL, "%s: null buffer", what);
  SegmentParams p{};
  p.offsets = offsets;
  p.value = value;
  p.out = dst;
  p.arg = (reduce_op == RED_MAX || reduce_op == RED_MIN) ? arg : nullptr;
  p.num_seg = num_seg;
  p.n = n;
  p.d = d;
  p.red = reduce_op == RED_MEAN ? RED_SUM : reduce_op;
  p.flags = (reduce_op == RED_MEAN ? F_MEAN : 0) | ((flags & MDGL_REPLACE_INF) ? F_REPLACE_INF : 0);
  p.skip_long = (flags & MDGL_SEGMENTS_SHORT) ? 0 : 1;
  p.passes = (flags & MDGL_SEGMENTS_SKIP_LONG)   ? SEG_PASS_ROWS
             : (flags & MDGL_SEGMENTS_LONG_ONLY) ? SEG_PASS_SPLIT
                                                 : SEG_PASS_ROWS | SEG_PASS_SPLIT;
  p.stream = (hipStream_t)stream;
  hipError_t e = dtype == MDGL_FLOAT32 ? launch_segment_reduce<float>(p)
                                       : launch_segment_reduce<double>(p);
  return hip_status(e, what);
}

}  // namespace

int mdgl_segment_reduce(const int32_t* offsets, const void* value, void* dst, int64_t num_seg,
                        int64_t d, int reduce_op, int64_t n, int flags, int dtype, void* stream) {
  MDGL_RANGE();
  return segment_common("segment_reduce", offsets, value, dst, nullptr, num_seg, d, reduce_op, n,
                        flags, dtype, stream);
}

int mdgl_segment_reduce_arg(const int32_t* offsets, const void* value, void* dst, int32_t* arg,
                            int64_t num_seg, int64_t d, int reduce_op, int64_t n, int flags,
                            int dtype, void* stream) {
  MDGL_RANGE();
  if (reduce_op != RED_MAX && reduce_op != RED_MIN)
    return fail(MDGL_EINVAL, "segment_reduce_arg: reduce_op must be max or min, got %d", reduce_op);
  if (num_seg > 0 && d > 0 && !arg) return fail(MDGL_EINVAL, "segment_reduce_arg: null buffer");
  return segment_common("segment_reduce_arg", offsets, value, dst, arg, num_seg, d, reduce_op, n,
                        flags, dtype, stream);
}

int mdgl_segment_ids(const int32_t* offsets, int64_t num_seg, int64_t n, int32_t* dst,
                     void* stream) {
  MDGL_RANGE();
  if (num_seg < 0 || n < 0) return fail(MDGL_EINVAL, "segment_ids: negative size");
  if (num_seg >= (int64_t(1) << 31) || n >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "segment_ids: 2**31 or more segments or rows");
  if (n == 0) return MDGL_OK;
  if (num_seg == 0) return fail(MDGL_EINVAL, "segment_ids: %lld rows and no segments", (long long)n);
  if (!offsets || !dst) return fail(MDGL_EINVAL, "segment_ids: null buffer");
  return hip_status(launch_segment_ids(offsets, num_seg, n, dst, (hipStream_t)stream),
                    "segment_ids");
}

// Softmax geometry for (d, dtype) and the two buffers: the vector width
// follows d and the buffers' alignment, the lane layout follows the width.
static void softmax_geom(int64_t d, int dtype, const void* logits, const void* out, int* vec,
                         int64_t* slots, int64_t* chunk_len) {
  const int vw = vec_width(dtype);
  const int64_t es = dsize(dtype);
  *vec = (d % vw == 0 && aligned(logits, vw * es) && aligned(out, vw * es)) ? vw : 1;
  const int64_t nvec = (d + *vec - 1) / *vec;
  int64_t L = 1;
  while (L < nvec && L < WAVE) L <<= 1;
  *slots = WAVE / L;
  *chunk_len = SOFT_CPL * *slots;
}

int mdgl_softmax_geometry(int64_t d, int dtype, const void* logits, const void* out,
                          int64_t* slots, int64_t* chunk_len) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "softmax_geometry: bad dtype %d", dtype);
  if (d <= 0 || !slots || !chunk_len) return fail(MDGL_EINVAL, "softmax_geometry: bad arguments");
  int vec;
  softmax_geom(d, dtype, logits, out, &vec, slots, chunk_len);
  return MDGL_OK;
}

int64_t mdgl_softmax_workspace_bytes(int64_t num_chunks, int64_t table_rows, int64_t d,
                                     int dtype) {
  if (num_chunks < 0 || table_rows < 0 || d < 0 || !dtype_ok(dtype)) return -1;
  const int64_t part = ((2 * num_chunks * d * dsize(dtype) + 255) / 256) * 256;
  return part + 2 * table_rows * d * dsize(dtype);
}

int64_t mdgl_segment_mm_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r, int dtype) {
  if (n < 0 || d1 < 0 || d2 < 0 || r < 0 || !dtype_ok(dtype)) return -1;
  return dtype == MDGL_FLOAT32 ? grouped_workspace_bytes<float>(n, d1, d2, r, false)
                               : grouped_workspace_bytes<double>(n, d1, d2, r, false);
}

int64_t mdgl_gather_mm_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r, int dtype) {
  if (n < 0 || d1 < 0 || d2 < 0 || r < 0 || !dtype_ok(dtype)) return -1;
  return dtype == MDGL_FLOAT32 ? grouped_workspace_bytes<float>(n, d1, d2, r, true)
                               : grouped_workspace_bytes<double>(n, d1, d2, r, true);
}

}  // extern "C"

namespace {

int softmax_common(const char* what, const int32_t* indptr, const int32_t* eid,
                   const int8_t* mask, const void* logits, void* dst, int64_t num_rows, int64_t d,
                   const int32_t* order, const int64_t* bounds, int nbins,
                   const int32_t* packed_eid, const int32_t* chunk_row,
                   const int32_t* chunk_start, const int32_t* chunk_first, int64_t num_chunks,
                   int64_t slots, const int32_t* row_of, int64_t num_edges,
                   int64_t num_slots, void* workspace,
                   int64_t workspace_bytes, int dtype, void* stream, bool stage = false) {
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "%s: bad dtype %d", what, dtype);
  if (num_rows < 0 || d < 0 || num_chunks < 0) return fail(MDGL_EINVAL, "%s: negative size", what);
  if (num_rows >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "%s: 2**31 or more rows", what);
  if (num_rows == 0 || d == 0) return MDGL_OK;
  if (!indptr || !logits || !dst) return fail(MDGL_EINVAL, "%s: null buffer", what);
  SoftmaxParams p{};
  int64_t want_slots, chunk_len;
  softmax_geom(d, dtype, logits, dst, &p.vec, &want_slots, &chunk_len);
  if (slots != want_slots)
    return fail(MDGL_EINVAL, "%s: plan made for %lld slots per wavefront, this call needs %lld "
                "(ask mdgl_softmax_geometry with the same buffers)", what, (long long)slots,
                (long long)want_slots);
  int want_bins = 0;
  while ((int64_t(1) << want_bins) < slots) ++want_bins;
  ++want_bins;
  if (order) {
    if (!bounds || nbins != want_bins)
      return fail(MDGL_EINVAL, "%s: a row order needs %d degree bins and their bounds", what,
                  want_bins);
    for (int k = 0; k <= nbins; ++k)
      if (bounds[k] > bounds[k + 1] || bounds[k] < 0)
        return fail(MDGL_EINVAL, "%s: bin bounds must be non-decreasing", what);
  }
  if (packed_eid && !order)
    return fail(MDGL_EINVAL, "%s: a packed edge list needs the row order it follows", what);
  if (num_chunks > 0 && (!chunk_row || !chunk_start || !chunk_first))
    return fail(MDGL_EINVAL, "%s: incomplete chunk list", what);
  if (row_of && num_edges < 0) return fail(MDGL_EINVAL, "%s: negative edge count", what);
  // table slots of the two-pass form: the ordered rows then the chunked
  // rows (one slot per chunk index), or one per row without an order
  const int64_t table_rows = !row_of ? 0 : (order ? bounds[nbins + 1] + num_chunks : num_rows);
  const int64_t need = mdgl_softmax_workspace_bytes(num_chunks, table_rows, d, dtype);
  if (need > 0 && workspace && !aligned(workspace, WS_ALIGN))
    return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(MDGL_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", what,
                (long long)need, (long long)workspace_bytes);
  p.indptr = indptr;
  p.eid = eid;
  p.mask = mask;
  p.logits = logits;
  p.out = dst;
  p.num_rows = num_rows;
  p.d = d;
  p.num_slots = num_slots;
  p.order = order;
  p.bounds = bounds;
  p.nbins = nbins;
  p.packed_eid = packed_eid;
  p.num_chunks = num_chunks;
  p.chunk_row = chunk_row;
  p.chunk_start = chunk_start;
  p.chunk_first = chunk_first;
  p.part = num_chunks > 0 ? workspace : nullptr;
  if (row_of) {
    p.row_of = row_of;
    p.num_edges = num_edges;
    p.table = static_cast<char*>(workspace) + ((2 * num_chunks * d * dsize(dtype) + 255) / 256) * 256;
  }
  p.stream = (hipStream_t)stream;
  if (stage && !order && num_chunks == 0) {
    // segments in their own order, none chunked: every one fits a staging
    // window (chunk_len rows never exceed it), so the LDS-staged kernel takes
    // them when the rows are narrow enough
    hipError_t se = dtype == MDGL_FLOAT32
                        ? launch_segment_softmax_stage<float>(indptr, logits, dst, num_rows,
                                                              num_slots, d, 0, p.stream)
                        : launch_segment_softmax_stage<double>(indptr, logits, dst, num_rows,
                                                               num_slots, d, 0, p.stream);
    if (se != hipErrorNotSupported) return hip_status(se, what);
  }
  hipError_t e = dtype == MDGL_FLOAT32 ? launch_softmax<float>(p) : launch_softmax<double>(p);
  return hip_status(e, what);
}

}  // namespace

extern "C" {

int mdgl_segment_softmax(const int32_t* offsets, const void* value, void* dst, void* scratch,
                         int64_t num_seg, int64_t d, int64_t n, const int32_t* order,
                         const int64_t* bounds, int nbins, const int32_t* packed_eid,
                         const int32_t* chunk_row, const int32_t* chunk_start,
                         const int32_t* chunk_first, int64_t num_chunks, int64_t slots,
                         void* workspace, int64_t workspace_bytes, int dtype, void* stream) {
  MDGL_RANGE();
  (void)scratch;
  if (n < 0) return fail(MDGL_EINVAL, "segment_softmax: negative size");
  if (n >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "segment_softmax: 2**31 or more rows");
  if (n == 0) return MDGL_OK;
  return softmax_common("segment_softmax", offsets, nullptr, nullptr, value, dst, num_seg, d,
                        order, bounds, nbins, packed_eid, chunk_row, chunk_start, chunk_first,
                        num_chunks, slots, nullptr, 0, n, workspace, workspace_bytes, dtype,
                        stream, true);
}

int mdgl_segment_softmax_short(const int32_t* offsets, const void* value, void* dst,
                               int64_t num_seg, int64_t d, int64_t n, int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "segment_softmax_short: bad dtype %d", dtype);
  if (num_seg < 0 || d < 0 || n < 0) return fail(MDGL_EINVAL, "segment_softmax_short: negative size");
  if (num_seg >= (int64_t(1) << 31) || n >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "segment_softmax_short: 2**31 or more segments or rows");
  if (!row_widths_fit(d, dsize(dtype)))
    return fail(MDGL_EINVAL, "segment_softmax_short: rows too wide");
  if (num_seg == 0 || d == 0 || n == 0) return MDGL_OK;
  if (!offsets || !value || !dst) return fail(MDGL_EINVAL, "segment_softmax_short: null buffer");
  int vec;
  int64_t slots, chunk_len;
  softmax_geom(d, dtype, value, dst, &vec, &slots, &chunk_len);
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e = dtype == MDGL_FLOAT32
                     ? launch_segment_softmax_stage<float>(offsets, value, dst, num_seg, n, d,
                                                           chunk_len, st)
                     : launch_segment_softmax_stage<double>(offsets, value, dst, num_seg, n, d,
                                                            chunk_len, st);
  if (e == hipErrorNotSupported)
    return fail(MDGL_ENOTSUP, "segment_softmax_short: rows of %lld values are too wide for the "
                "staged kernel", (long long)d);
  return hip_status(e, "segment_softmax_short");
}

int mdgl_edge_softmax_(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                       const int8_t* mask, const void* logits, void* dst, void* scratch,
                       int64_t num_nodes, int all_ones, int64_t d, const int32_t* order,
                       const int64_t* bounds, int nbins, const int32_t* packed_eid,
                       const int32_t* chunk_row, const int32_t* chunk_start,
                       const int32_t* chunk_first, int64_t num_chunks, int64_t slots,
                       const int32_t* slot_of_edge, int64_t num_edges, void* workspace,
                       int64_t workspace_bytes, int dtype, void* stream) {
  MDGL_RANGE();
  (void)indices;
  (void)scratch;
  if (num_nodes > 0 && d > 0 && !eid) return fail(MDGL_EINVAL, "edge_softmax: null eid");
  if (all_ones != 1 && !mask) return fail(MDGL_EINVAL, "edge_softmax: null mask");
  return softmax_common("edge_softmax", indptr, eid, all_ones == 1 ? nullptr : mask, logits, dst,
                        num_nodes, d, order, bounds, nbins, packed_eid, chunk_row, chunk_start,
                        chunk_first, num_chunks, slots, slot_of_edge, num_edges,
                        num_edges > 0 ? num_edges : 0, workspace, workspace_bytes, dtype, stream);
}

}  // extern "C"

namespace {

// Workspace layout of mdgl_edge_softmax_positional (each part 256-byte
// aligned): the launch figures, the row order, the packed position lists,
// the chunk arrays, the chunk partials and the (max, sum) table by node, then
// the plan's scratch.
struct PosLayout {
  int64_t dyn, order, packed, chunks, soft, scratch, total;
};

PosLayout pos_layout(int64_t num_sel, int64_t num_nodes, int64_t d, int dtype, int64_t max_chunks) {
  auto al = [](int64_t b) { return (b + 255) / 256 * 256; };
  PosLayout l{};
  l.dyn = 0;
  l.order = l.dyn + al(sizeof(SoftDyn));
  l.packed = l.order + al(num_nodes * 4);
  l.chunks = l.packed + al(2 * num_sel * 4);
  l.soft = l.chunks + 3 * al(max_chunks * 4);
  l.scratch = l.soft + al(mdgl_softmax_workspace_bytes(max_chunks, num_nodes, d, dtype));
  l.total = l.scratch + al(positional_scratch_bytes(num_sel, num_nodes));
  return l;
}

}  // namespace

extern "C" {

int64_t mdgl_edge_softmax_positional_workspace_bytes(int64_t num_sel, int64_t num_nodes,
                                                     int64_t d, const void* logits,
                                                     const void* dst, int dtype) {
  if (num_sel < 0 || num_nodes < 0 || d < 0 || !dtype_ok(dtype)) return -1;
  if (num_sel == 0 || d == 0) return 0;
  int vec;
  int64_t slots, chunk_len;
  softmax_geom(d, dtype, logits, dst, &vec, &slots, &chunk_len);
  return pos_layout(num_sel, num_nodes, d, dtype, positional_max_chunks(num_sel, chunk_len)).total;
}

int mdgl_edge_softmax_positional(const int32_t* ends, int64_t num_edges, const int64_t* eids,
                                 int64_t num_sel, int64_t num_nodes, const void* logits,
                                 void* dst, int64_t d, int32_t* endpoint, int32_t* group_ptr,
                                 int32_t* group_pos, int64_t* id_range, void* range_event,
                                 void* workspace, int64_t workspace_bytes, int dtype,
                                 void* stream) {
  MDGL_RANGE();
  const char* what = "edge_softmax_positional";
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "%s: bad dtype %d", what, dtype);
  if (num_edges < 0 || num_sel < 0 || num_nodes < 0 || d < 0)
    return fail(MDGL_EINVAL, "%s: negative size", what);
  if (num_edges >= (int64_t(1) << 31) || num_sel >= (int64_t(1) << 31) ||
      num_nodes >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "%s: 2**31 or more edges, positions or nodes", what);
  if (!row_widths_fit(d, dsize(dtype))) return fail(MDGL_EINVAL, "%s: rows too wide", what);
  if (num_sel == 0 || d == 0) return MDGL_OK;
  if (num_edges == 0 || num_nodes == 0)
    return fail(MDGL_EINVAL, "%s: %lld edge ids selected from a graph without edges", what,
                (long long)num_sel);
  if (!ends || !eids || !logits || !dst || !endpoint || !group_ptr || !group_pos || !id_range)
    return fail(MDGL_EINVAL, "%s: null buffer", what);
  SoftmaxParams p{};
  int64_t slots, chunk_len;
  softmax_geom(d, dtype, logits, dst, &p.vec, &slots, &chunk_len);
  const int64_t max_chunks = positional_max_chunks(num_sel, chunk_len);
  const PosLayout l = pos_layout(num_sel, num_nodes, d, dtype, max_chunks);
  if (!aligned(workspace, WS_ALIGN))
    return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
  if (!workspace || workspace_bytes < l.total)
    return fail(MDGL_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", what,
                (long long)l.total, (long long)workspace_bytes);
  char* w = static_cast<char*>(workspace);
  int nbins = 0;
  while ((int64_t(1) << nbins) < slots) ++nbins;
  ++nbins;
  const int64_t nvec = (d + p.vec - 1) / p.vec;
  int L = 1;
  while (L < nvec && L < WAVE) L <<= 1;
  PositionalPlan pp{};
  pp.ends = ends;
  pp.num_edges = num_edges;
  pp.eids = eids;
  pp.num_sel = num_sel;
  pp.num_nodes = num_nodes;
  pp.slots = (int)slots;
  pp.chunk_len = (int)chunk_len;
  pp.nbins = nbins;
  pp.Pw = WAVE / L;
  pp.S = (int)((nvec + L - 1) / L);
  pp.endpoint = endpoint;
  pp.group_ptr = group_ptr;
  pp.group_pos = group_pos;
  pp.id_range = id_range;
  pp.order = reinterpret_cast<int32_t*>(w + l.order);
  pp.packed = reinterpret_cast<int32_t*>(w + l.packed);
  const int64_t cstride = (max_chunks * 4 + 255) / 256 * 256;
  pp.chunk_row = reinterpret_cast<int32_t*>(w + l.chunks);
  pp.chunk_start = reinterpret_cast<int32_t*>(w + l.chunks + cstride);
  pp.chunk_first = reinterpret_cast<int32_t*>(w + l.chunks + 2 * cstride);
  pp.max_chunks = max_chunks;
  pp.dyn = reinterpret_cast<SoftDyn*>(w + l.dyn);
  pp.scratch = w + l.scratch;
  pp.range_event = (hipEvent_t)range_event;
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e = launch_positional_plan(pp, st);
  if (e != hipSuccess) return hip_status(e, what);
  p.indptr = group_ptr;
  p.eid = group_pos;
  p.logits = logits;
  p.out = dst;
  p.num_rows = num_nodes;
  p.d = d;
  p.num_slots = num_sel;
  p.order = pp.order;
  p.nbins = nbins;
  p.packed_eid = pp.packed;
  p.num_chunks = max_chunks;
  p.chunk_row = pp.chunk_row;
  p.chunk_start = pp.chunk_start;
  p.chunk_first = pp.chunk_first;
  p.part = w + l.soft;
  p.table = w + l.soft + ((2 * max_chunks * d * dsize(dtype) + 255) / 256) * 256;
  p.row_of = endpoint;
  p.num_edges = num_sel;
  p.row_slots = 1;
  p.dyn = pp.dyn;
  p.stream = st;
  e = dtype == MDGL_FLOAT32 ? launch_softmax<float>(p) : launch_softmax<double>(p);
  return hip_status(e, what);
}

}  // extern "C"

namespace {

constexpr int64_t MAX_GATHER_BLOCKS = 2048;  // bucketing keeps 5 * r ints in LDS

int grouped_common(const void* a, const void* b, void* dst, const int64_t* idx_b,
                   const int64_t* seglen, int64_t n, int64_t d1, int64_t d2, int64_t r,
                   void* workspace, int64_t workspace_bytes, int dtype, void* stream,
                   bool gather) {
  const char* what = gather ? "gather_mm" : "segment_mm";
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "%s: bad dtype %d", what, dtype);
  if (n < 0 || d1 < 0 || d2 < 0 || r < 0) return fail(MDGL_EINVAL, "%s: negative size", what);
  if (n >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "%s: 2**31 or more rows", what);
  if (gather && r > MAX_GATHER_BLOCKS)
    return fail(MDGL_ENOTSUP, "%s: at most %lld b blocks supported, got %lld", what,
                (long long)MAX_GATHER_BLOCKS, (long long)r);
  if (n == 0 || d2 == 0) return MDGL_OK;
  if (r == 0) return fail(MDGL_EINVAL, "%s: rows but no b blocks", what);
  if (!a || !b || !dst || (gather ? !idx_b : !seglen))
    return fail(MDGL_EINVAL, "%s: null buffer", what);
  const int64_t need = gather ? mdgl_gather_mm_workspace_bytes(n, d1, d2, r, dtype)
                              : mdgl_segment_mm_workspace_bytes(n, d1, d2, r, dtype);
  if (workspace && !aligned(workspace, WS_ALIGN))
    return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
  if (!workspace || workspace_bytes < need)
    return fail(MDGL_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", what,
                (long long)need, (long long)workspace_bytes);
  GemmLaunch L{};
  L.a = a;
  L.b = b;
  L.out = dst;
  L.idx_b = idx_b;
  L.seglen = seglen;
  L.n = n;
  L.K = d1;
  L.N = d2;
  L.R = r;
  L.workspace = workspace;
  L.stream = (hipStream_t)stream;
  hipError_t e = dtype == MDGL_FLOAT32 ? launch_grouped<float>(L, gather)
                                       : launch_grouped<double>(L, gather);
  return hip_status(e, what);
}

int grouped_grad_common(const void* a, const void* b, const void* grad, void* da, void* db,
                        const int64_t* idx_b, const int64_t* seglen, int64_t n, int64_t d1,
                        int64_t d2, int64_t r, void* workspace, int64_t workspace_bytes,
                        int dtype, void* stream, bool gather) {
  const char* what = gather ? "gather_mm_grad" : "segment_mm_grad";
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "%s: bad dtype %d", what, dtype);
  if (n < 0 || d1 < 0 || d2 < 0 || r < 0) return fail(MDGL_EINVAL, "%s: negative size", what);
  if (n >= (int64_t(1) << 31)) return fail(MDGL_EINVAL, "%s: 2**31 or more rows", what);
  if (gather && r > MAX_GATHER_BLOCKS)
    return fail(MDGL_ENOTSUP, "%s: at most %lld b blocks supported, got %lld", what,
                (long long)MAX_GATHER_BLOCKS, (long long)r);
  if (((d1 + 127) / 128) * ((d2 + 127) / 128) > 65535)
    return fail(MDGL_ENOTSUP, "%s: d1 x d2 of %lld x %lld is too large", what, (long long)d1,
                (long long)d2);
  if (n == 0 || d1 == 0 || d2 == 0 || (!da && !db)) return MDGL_OK;
  if (r == 0) return fail(MDGL_EINVAL, "%s: rows but no b blocks", what);
  if (!a || !b || !grad || (gather ? !idx_b : !seglen))
    return fail(MDGL_EINVAL, "%s: null buffer", what);
  const int64_t need = gather ? mdgl_gather_mm_grad_workspace_bytes(n, d1, d2, r, dtype)
                              : mdgl_segment_mm_grad_workspace_bytes(n, d1, d2, r, dtype);
  if (workspace && !aligned(workspace, WS_ALIGN))
    return fail(MDGL_EINVAL, "workspace must be %lld-byte aligned", (long long)WS_ALIGN);
  if (!workspace || workspace_bytes < need)
    return fail(MDGL_EWORKSPACE, "%s: workspace of %lld bytes needed, %lld given", what,
                (long long)need, (long long)workspace_bytes);
  GemmGradLaunch L{};
  L.a = a;
  L.b = b;
  L.grad = grad;
  L.da = da;
  L.db = db;
  L.idx_b = idx_b;
  L.seglen = seglen;
  L.n = n;
  L.D1 = d1;
  L.D2 = d2;
  L.R = r;
  L.workspace = workspace;
  L.stream = (hipStream_t)stream;
  hipError_t e = dtype == MDGL_FLOAT32 ? launch_grouped_grad<float>(L, gather)
                                       : launch_grouped_grad<double>(L, gather);
  return hip_status(e, what);
}

}  // namespace

extern "C" {

int64_t mdgl_segment_mm_grad_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r,
                                             int dtype) {
  if (n < 0 || d1 < 0 || d2 < 0 || r < 0 || !dtype_ok(dtype)) return -1;
  return dtype == MDGL_FLOAT32 ? grouped_grad_workspace_bytes<float>(n, d1, d2, r, false)
                               : grouped_grad_workspace_bytes<double>(n, d1, d2, r, false);
}

int64_t mdgl_gather_mm_grad_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r,
                                            int dtype) {
  if (n < 0 || d1 < 0 || d2 < 0 || r < 0 || !dtype_ok(dtype)) return -1;
  return dtype == MDGL_FLOAT32 ? grouped_grad_workspace_bytes<float>(n, d1, d2, r, true)
                               : grouped_grad_workspace_bytes<double>(n, d1, d2, r, true);
}

int mdgl_segment_mm_grad(const void* a, const void* b, const void* grad_out,
                         const int64_t* seglen_a, void* grad_a, void* grad_b, int64_t n,
                         int64_t d1, int64_t r, int64_t d2, void* workspace,
                         int64_t workspace_bytes, int dtype, void* stream) {
  MDGL_RANGE();
  return grouped_grad_common(a, b, grad_out, grad_a, grad_b, nullptr, seglen_a, n, d1, d2, r,
                             workspace, workspace_bytes, dtype, stream, false);
}

int mdgl_gather_mm_grad(const void* a, const void* b, const int64_t* idx_b, const void* grad_out,
                        void* grad_a, void* grad_b, int64_t n, int64_t d1, int64_t d2,
                        int64_t r, void* workspace, int64_t workspace_bytes, int dtype,
                        void* stream) {
  MDGL_RANGE();
  return grouped_grad_common(a, b, grad_out, grad_a, grad_b, idx_b, nullptr, n, d1, d2, r,
                             workspace, workspace_bytes, dtype, stream, true);
}

int mdgl_segment_mm(const void* a, const void* b, void* dst, const int64_t* seglen_a, int64_t n,
                    int64_t d1, int64_t r, int64_t d2, void* workspace, int64_t workspace_bytes,
                    int dtype, void* stream) {
  MDGL_RANGE();
  return grouped_common(a, b, dst, nullptr, seglen_a, n, d1, d2, r, workspace, workspace_bytes,
                        dtype, stream, false);
}

int mdgl_gather_mm(const void* a, const void* b, const int64_t* idx_b, void* dst, int64_t n,
                   int64_t d1, int64_t d2, int64_t r, void* workspace, int64_t workspace_bytes,
                   int dtype, void* stream) {
  MDGL_RANGE();
  return grouped_common(a, b, dst, idx_b, nullptr, n, d1, d2, r, workspace, workspace_bytes,
                        dtype, stream, true);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// mdgl_gspmm_noalloc: mdgl_gspmm with its heavy-row partials in a fixed device
// array instead of a caller workspace, for callers that cannot allocate.
//
// `scratch` is a host-side stand-in for the device array: host code never
// passes it to a kernel. Its device address is looked up once per device
// (hipGetSymbolAddress, with that device current, on the entry point's first
// call there) and kept in g_scratch_ptr; every use goes through that pointer.
namespace {

static __device__ __align__(256) unsigned char scratch[MDGL_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// The current device's scratch address, resolved on first use.
int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "gspmm_noalloc: hipGetDevice");
  if (dev < 0 || dev >= MAX_DEVICES)
    return fail(MDGL_ENOTSUP, "gspmm_noalloc: device %d beyond the %d supported", dev,
                MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "gspmm_noalloc: hipGetSymbolAddress(scratch)");
    if (!p) return fail(MDGL_EWORKSPACE, "gspmm_noalloc: no device address for the scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MDGL_OK;
}

}  // namespace

extern "C" int mdgl_gspmm_noalloc(const int32_t* indptr, const int32_t* indices,
                                  const int32_t* eid, const void* lhs, const void* rhs,
                                  void* dst, int64_t num_dst, int op, int64_t dl, int64_t dr,
                                  int64_t dout, int reduce_op, const int32_t* deg, int nd,
                                  const int64_t* lhs_shape, const int64_t* rhs_shape,
                                  int32_t* arg_u, int32_t* arg_e, const int32_t* chunk_row,
                                  const int32_t* chunk_start, int64_t num_chunks,
                                  int32_t chunk_len, const int32_t* heavy_rows,
                                  const int32_t* heavy_ptr, int64_t num_heavy, int flags,
                                  int dtype, void* stream) {
  MDGL_RANGE();
  if (!dtype_ok(dtype)) return fail(MDGL_EINVAL, "gspmm_noalloc: bad dtype %d", dtype);
  if (num_chunks < 0 || dout < 0) return fail(MDGL_EINVAL, "gspmm_noalloc: negative size");
  if (!row_widths_fit(dout, dsize(dtype)) || num_chunks >= (int64_t(1) << 31))
    return fail(MDGL_EINVAL, "gspmm_noalloc: rows too wide or too many chunks");
  const int64_t need = mdgl_gspmm_workspace_bytes(num_chunks, dout, reduce_op, dtype);
  if (need > MDGL_NOALLOC_SCRATCH_BYTES)
    return fail(MDGL_EWORKSPACE, "gspmm_noalloc: %lld chunks of %lld columns need %lld bytes of "
                "partials, the scratch holds %lld; use mdgl_gspmm with a workspace",
                (long long)num_chunks, (long long)dout, (long long)need,
                (long long)MDGL_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    int rc = scratch_of_current_device(&ws);
    if (rc) return rc;
  }
  return gspmm_common(indptr, indices, eid, lhs, rhs, dst, num_dst, op, dl, dr, dout, reduce_op,
                      deg, nd, lhs_shape, rhs_shape, arg_u, arg_e, chunk_row, chunk_start,
                      num_chunks, chunk_len, heavy_rows, heavy_ptr, num_heavy, ws,
                      need > 0 ? MDGL_NOALLOC_SCRATCH_BYTES : 0, flags, dtype, stream);
}
