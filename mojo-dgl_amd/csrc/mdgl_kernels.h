// Launch interfaces between the C ABI (capi.cpp) and the kernel translation
// units. Every launcher is asynchronous on `stream` and returns the launch
// status; nothing here allocates.
#pragma once

#include "mdgl_common.h"

namespace mdgl {

// Flags of the CSR-reduce kernel.
enum {
  F_MEAN = 1,          // divide the sum by max(degree, 1)
  F_REPLACE_INF = 2,   // +-inf -> 0 on the final value (update_all max/min)
  F_OUT_VEC = 4,       // output rows allow 16-byte stores
  F_EID_IDENTITY = 8,  // edge id of CSR slot i is i (copy_lhs given no edge ids)
  F_RHS_CSR = 16,      // the edge operand is in CSR slot order (rhs row i for slot i)
};

// gspmm / segment_reduce: out[row, k] = red over CSR slots of row of
// op(lhs[indices[i]], rhs[eid[i]]). Rows of degree > chunk_len are split
// into chunks (chunk_row / chunk_start, num_chunks of them) whose partials
// are reduced in CSR order by a second kernel over heavy_rows / heavy_ptr.
struct GspmmParams {
  const int32_t* indptr;
  const int32_t* indices;  // may be null when op does not read lhs and no arg_u
  const int32_t* eid;      // ignored with F_EID_IDENTITY
  const int32_t* deg;      // mean divisor; null -> row length
  const void* lhs;
  const void* rhs;
  void* out;
  int32_t* arg_u;  // optional, max/min only
  int32_t* arg_e;
  int64_t num_rows, dl, dr, dout;
  int64_t lstride;  // elements between lhs rows (dl, or more for rows on 128-byte lines)
  Bcast bc;
  int lmode, rmode;
  int op, red;  // red in {SUM, MAX, MIN}; mean is F_MEAN
  int flags;
  int vec;      // elements per lane (1 or 16 / sizeof(T))
  int group;    // lanes per row slab (a power of two, at most 64)
  int64_t num_chunks;
  const int32_t* chunk_row;
  const int32_t* chunk_start;
  int32_t chunk_len;
  int64_t num_heavy;
  const int32_t* heavy_rows;
  const int32_t* heavy_ptr;
  void* part_val;
  int32_t* part_u;
  int32_t* part_e;
  // optional (mul / sum with the edge operand splat over groups of
  // dot_lanes * vec columns): a feature row per CSR row and, per CSR slot and
  // group, dot_out[slot][group] = sum over the group of lhs[indices[slot]] *
  // rowop[row]
  const void* rowop;
  void* dot_out;
  int dot_lanes;
  // optional: the rows to reduce (num_rows of them, each in [0, row_limit));
  // null: rows 0 .. num_rows - 1
  const int32_t* rows;
  int64_t row_limit;
  hipStream_t stream;
};

template <class T, int RED>
hipError_t launch_gspmm_red(const GspmmParams& p);

// Per-block counts of the edges i with |u[i] - v[i]| < window, into
// partial[0 .. COO_LOCALITY_BLOCKS) (csr.hip).
constexpr int COO_LOCALITY_BLOCKS = 1024;
hipError_t launch_coo_locality(const int32_t* u, const int32_t* v, int64_t n, int64_t window,
                               int64_t* partial, hipStream_t s);

// segment_reduce: out[s, k] = red over value rows offsets[s] .. offsets[s+1]
// (segment_impl.h). red in {SUM, MAX, MIN}, mean is F_MEAN; arg (max / min,
// optional) receives the selected row. Unless skip_long is 0, segments
// longer than SEG_SPLIT_ROWS are left to a separate split pass. `passes`
// picks the launches: SEG_PASS_ROWS the row-order kernels, SEG_PASS_SPLIT
// the split pass (which only runs with skip_long).
constexpr int SEG_SPLIT_ROWS = 4096;
enum { SEG_PASS_ROWS = 1, SEG_PASS_SPLIT = 2 };
struct SegmentParams {
  const int32_t* offsets;
  const void* value;
  void* out;
  int32_t* arg;
  int64_t num_seg, n, d;
  int red, flags;
  int skip_long;
  int passes;
  hipStream_t stream;
};

template <class T>
hipError_t launch_segment_reduce(const SegmentParams& p);

// segment_softmax of segments that fit an 8 KB window each, rows of at most
// 32 lane vectors (segment_impl.h); hipErrorNotSupported for wider rows.
// Segments of more than max_rows rows are not written (max_rows <= 0: no
// limit).
template <class T>
hipError_t launch_segment_softmax_stage(const int32_t* offsets, const void* value, void* out,
                                        int64_t num_seg, int64_t n, int64_t d, int64_t max_rows,
                                        hipStream_t st);

// gsddmm: out[e, o] = op(lhs[t_l(e)], rhs[t_r(e)]) (or the dot over `red`).
struct GsddmmParams {
  const int32_t* uids;
  const int32_t* vids;
  const void* lhs;
  const void* rhs;
  void* out;
  int64_t num_edges, dl, dr, dout, red;
  Bcast bc;
  int lt, rt, op;
  int lmode, rmode;
  int out_vec;
  int vec;
  hipStream_t stream;
};

template <class T>
hipError_t launch_gsddmm(const GsddmmParams& p);

// CSR softmax (edge_softmax over in/out CSR, segment_softmax over offsets):
// per row and column, max, then exp(x - max) summed, then divided. Rows are
// served through a plan (see softmax_impl.h): `order` lists the rows sorted
// by degree with `bounds` (host) delimiting the packed degree bins and the
// wavefront rows, or is null for all rows in natural order; rows longer than
// the chunk length come as chunks (chunk_row / chunk_start / chunk_first)
// whose partials live in `part` (2 * num_chunks * d values).
constexpr int SOFT_CPL = 8;  // logits cached per lane in a wavefront row of the softmax
constexpr int SOFT_MAX_BINS = 7;  // packed degree bins: 1 .. 64 slots per wavefront
constexpr int SOFT_PK_U = 4;      // packed wavefronts served per wavefront of the packed launch

// A softmax plan's launch figures kept in device memory (a plan built on the
// GPU, whose sizes the host never reads): the kernels of such a launch take
// their bin bounds and work counts from here and walk their work with a
// fixed grid.
struct SoftDyn {
  int64_t bin_start[SOFT_MAX_BINS + 1];  // packed bin k: order[bin_start[k] .. bin_start[k+1])
  int64_t bin_wave[SOFT_MAX_BINS + 1];   // packed wavefronts before bin k
  int64_t bin_slot[SOFT_MAX_BINS + 1];   // packed edge-list entries before bin k
  int64_t mid_start, mid_end;            // wavefront rows: order[mid_start .. mid_end)
  int64_t light_waves;                   // wavefronts of those rows (slabs included)
  int64_t packed_tasks;                  // wavefronts of the packed launch
  int64_t num_chunks, chunk_waves;       // chunks of the long rows, their wavefronts
};

struct SoftmaxParams {
  const int32_t* indptr;
  const int32_t* eid;  // null -> identity (segment softmax)
  const int8_t* mask;  // null -> all selected
  const void* logits;
  void* out;
  int64_t num_rows, d;
  int64_t num_slots;  // CSR entries (indptr[num_rows]) when known, else 0
  int vec;            // elements per lane
  const int32_t* order;
  const int64_t* bounds;  // host: nbins + 2 entries
  int nbins;
  // null, or the edge ids of the packed rows slot by slot (2^k per row of
  // bin k, -1 past the degree, bins one after the other)
  const int32_t* packed_eid;
  int64_t num_chunks;
  const int32_t* chunk_row;
  const int32_t* chunk_start;
  const int32_t* chunk_first;
  void* part;
  // two-pass form: the table slot of every edge id's row and a
  // [slots][2][d] table
  const int32_t* row_of;
  int64_t num_edges;
  void* table;
  // the table is indexed by row id (row_of then holds each edge's row), not
  // by position in the row order
  int row_slots;
  // a plan built on the GPU: its figures (SoftDyn) in device memory, `order`,
  // the packed list and the chunk arrays device-resident and sized for
  // `num_chunks` chunks at most (the partials too); `bounds` unused
  const SoftDyn* dyn;
  hipStream_t stream;
};

template <class T>
hipError_t launch_softmax(const SoftmaxParams& p);

// Grouped GEMM behind segment_mm (groups = consecutive rows, seglen) and
// gather_mm (groups = rows with equal idx_b, bucketed on the GPU).
struct GemmLaunch {
  const void* a;
  const void* b;
  void* out;
  const int64_t* idx_b;   // gather_mm: block of each row
  const int64_t* seglen;  // segment_mm: rows per block
  int64_t n, K, N, R;
  void* workspace;
  hipStream_t stream;
  int trans_b;  // b given as [R][N][K] (multiplying by each block's transpose)
};
template <class T>
int64_t grouped_workspace_bytes(int64_t n, int64_t K, int64_t N, int64_t R, bool gather);
template <class T>
hipError_t launch_grouped(const GemmLaunch& L, bool gather);
// Gradients of out = a @ b[group] (a: n x D1, b: R x D1 x D2, grad: n x D2):
// da = grad @ b[group]^T and db[g] = sum over g's rows of a^T grad; either
// output may be null.
struct GemmGradLaunch {
  const void* a;
  const void* b;
  const void* grad;
  void* da;
  void* db;
  const int64_t* idx_b;
  const int64_t* seglen;
  int64_t n, D1, D2, R;
  void* workspace;
  hipStream_t stream;
};
template <class T>
int64_t grouped_grad_workspace_bytes(int64_t n, int64_t D1, int64_t D2, int64_t R, bool gather);
template <class T>
hipError_t launch_grouped_grad(const GemmGradLaunch& L, bool gather);

// Elementwise helpers.
hipError_t launch_replace_inf(const void* src, void* dst, int64_t n, int dtype, hipStream_t s);
hipError_t launch_clamp_i64(const int64_t* src, int64_t* dst, int64_t n, int64_t lo, int64_t hi,
                            hipStream_t s);
// dst[i, :] = src[idx[i], :] (rows of `width` elements; array.hip).
hipError_t launch_gather_rows(const void* src, const int32_t* idx, void* dst, int64_t n,
                              int64_t width, int dtype, hipStream_t s, bool scatter = false);
// dst[i] = the segment holding row i (offsets: num_seg + 1 entries; array.hip).
hipError_t launch_segment_ids(const int32_t* offsets, int64_t num_seg, int64_t n, int32_t* dst,
                              hipStream_t s);
// Backward helpers (backward.hip).
hipError_t launch_softmax_grad(const int32_t* row_of, const void* a, const void* g,
                               const void* s, void* dx, int64_t num_edges, int64_t d, int dtype,
                               hipStream_t st);
hipError_t launch_edge_grad(const int32_t* vids, const int32_t* indptr, const void* g,
                            const int32_t* arg_e, void* m, int64_t num_edges, int64_t d,
                            double alpha, int mean, int dtype, hipStream_t s);
hipError_t launch_rows_by_degree(const int32_t* indptr, const void* x, void* y, int64_t rows,
                                 int64_t d, int dtype, hipStream_t s);
hipError_t launch_keep_where(const void* mask, const void* x, void* y, int64_t n, int dtype,
                             hipStream_t s);
hipError_t launch_scale(const void* x, void* y, int64_t n, double alpha, int dtype,
                        hipStream_t s);
// COO -> CSR by `key` (csr.hip).
int64_t csr_workspace_bytes(int64_t num_edges, int64_t num_rows);
hipError_t launch_build_csr(const int32_t* key, const int32_t* other, int64_t num_edges,
                            int64_t num_rows, int32_t* indptr, int32_t* indices, int32_t* eid,
                            void* workspace, hipStream_t stream);
hipError_t launch_cumsum_i64(const int64_t* src, int64_t* dst, int64_t n, hipStream_t s);
int64_t read_stream_sink_bytes(int64_t bytes);
hipError_t launch_read_stream(const void* src, int64_t bytes, void* sink, hipStream_t s);
int64_t read_rows_sink_bytes(int64_t n);
hipError_t launch_read_rows(const void* src, int64_t src_rows, int64_t row_bytes,
                            const int32_t* idx, int64_t n, void* dst, int64_t dst_rows, void* sink,
                            hipStream_t s);
// The positional edge_softmax plan built on the GPU (softmax_plan.hip):
// positions grouped by the endpoint of their edge, rows binned by degree,
// chunks of the long rows, the packed edge lists and the SoftDyn figures.
struct PositionalPlan {
  const int32_t* ends;   // endpoint of every edge id
  int64_t num_edges;
  const int64_t* eids;   // the selected edge id of every position
  int64_t num_sel, num_nodes;
  int slots, chunk_len, nbins, S, Pw;
  // outputs
  int32_t* endpoint;     // [num_sel] endpoint of each position
  int32_t* group_ptr;    // [num_nodes + 1]
  int32_t* group_pos;    // [num_sel] positions grouped by endpoint
  int64_t* id_range;     // [2] min and max of eids
  hipEvent_t range_event;  // recorded once id_range is written (nullable)
  // plan arrays (workspace)
  int32_t* order;        // [num_nodes]
  int32_t* packed;       // [2 * num_sel]
  int32_t* chunk_row;    // [max_chunks] x3
  int32_t* chunk_start;
  int32_t* chunk_first;
  int64_t max_chunks;
  SoftDyn* dyn;
  void* scratch;         // positional_scratch_bytes(num_sel, num_nodes)
};
int64_t positional_max_chunks(int64_t num_sel, int64_t chunk_len);
int64_t positional_scratch_bytes(int64_t num_sel, int64_t num_nodes);
hipError_t launch_positional_plan(const PositionalPlan& p, hipStream_t s);
int64_t segment_offsets_workspace_bytes(int64_t num);
hipError_t launch_segment_offsets(const int64_t* len, int64_t num, int64_t chunk_len,
                                  int32_t* offsets, int64_t* stats, void* ws, hipStream_t s);

}  // namespace mdgl
