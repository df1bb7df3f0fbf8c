/* libmdgl.so -- MI355X (gfx950) message-passing kernel layer, C ABI.
 *
 * Drop-in for the reference's Mojo C ABI (src/capi.mojo), which the Python
 * host layer binds through ctypes (python/mojodgl/_lib.py:51-63). Every
 * entry point keeps the reference's symbol name and its leading arguments in
 * the reference's order and meaning, then adds what a GPU needs:
 *   - device pointers (every array argument is device memory unless stated);
 *   - int32 graph indices (CSR row pointers, neighbour ids, edge ids, COO
 *     endpoints, segment offsets); the host converts the reference's int64
 *     ids once per graph and refuses 2**31 or more nodes or edges;
 *   - a dtype code (MDGL_FLOAT32 / MDGL_FLOAT64) instead of float64 only;
 *   - NumPy broadcasting by operand feature shapes instead of materialised
 *     width-1 operands (python/mojodgl/ops/sddmm.py:62-68);
 *   - optional arg outputs for max/min, a heavy-row schedule, a caller-owned
 *     workspace, and a HIP stream (hipStream_t passed as void*; NULL is the
 *     default stream).
 *
 * Conventions (as the reference, capi.mojo:1-17): the caller owns all
 * memory, nothing here allocates or frees, and launches are asynchronous on
 * `stream`. Workspaces must be 256-byte aligned (hipMalloc's alignment). Unlike the reference every call returns a status: 0 on success,
 * a negative MDGL_E* code for an invalid argument (detected before anything
 * is launched; mdgl_last_error() names it), or a positive hipError_t from
 * the launch.
 *
 * Codes (src/ported.mojo:44-65, python/mojodgl/_lib.py:65-73):
 *   targets  u = 0, v = 1, e = 2
 *   ops      add, sub, mul, div, dot = 0..4, copy_lhs = 5, copy_rhs = 6
 *   reducers sum, max, min, mean = 0..3
 */
#ifndef MDGL_H
#define MDGL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MDGL_OK 0
#define MDGL_EINVAL (-1)     /* invalid argument */
#define MDGL_EWORKSPACE (-2) /* workspace missing or too small */
#define MDGL_ENOTSUP (-3)    /* valid but unsupported shape (e.g. > 6 broadcast dims) */

#define MDGL_FLOAT32 0
#define MDGL_FLOAT64 1

/* flags of mdgl_gspmm / mdgl_segment_reduce */
#define MDGL_REPLACE_INF 1 /* +-inf results become 0 (heterograph.py:232-239) */
#define MDGL_RHS_CSR_ORDER 2 /* mdgl_gspmm: rhs row i belongs to CSR slot i (not edge eid[i]) */
/* mdgl_gspmm: lhs rows start on 128-byte lines: row r at lhs + r * stride
 * elements, stride = dl rounded up to a multiple of 128 bytes (lhs itself
 * 128-byte aligned) */
#define MDGL_LHS_LINE_ROWS 8
/* mdgl_gspmm: rows wider than one 64-lane slab (256 float32 / 128 float64
 * columns with 16-byte lanes) are cut into 32-lane slabs, two rows to a
 * wavefront, when that makes at most 5 slabs -- for graphs whose sources lie
 * near their destinations (mdgl_coo_locality), where a narrower slab of a
 * block of neighbouring rows stays in cache. Results are the same bit for
 * bit; only the lane layout changes. */
#define MDGL_NARROW_SLABS 32
/* mdgl_segment_reduce(_arg): the caller knows that no segment has more than
 * MDGL_SEGMENT_SPLIT_ROWS rows, so the pass that splits longer segments is
 * not launched (a longer segment is then still reduced whole, in row order) */
#define MDGL_SEGMENTS_SHORT 4
#define MDGL_SEGMENT_SPLIT_ROWS 4096
/* mdgl_segment_reduce(_arg), for callers that learn the longest segment
 * only after the call (lengths on the GPU): SKIP_LONG reduces every segment
 * of at most MDGL_SEGMENT_SPLIT_ROWS rows and leaves the longer ones
 * unwritten; a second call with LONG_ONLY then reduces just those. The two
 * calls write what one call without either flag writes. At most one of
 * SHORT, SKIP_LONG and LONG_ONLY. */
#define MDGL_SEGMENTS_SKIP_LONG 8
#define MDGL_SEGMENTS_LONG_ONLY 16

/* Message of the last failed call on this thread ("" if none). */
const char* mdgl_last_error(void);

/* Replaces capi.mojo:48-50 (`mdgl_workers`). The reference returns its CPU
 * worker count; here it is the number of compute units the launches are
 * shaped for (256 on MI355X), always > 1. */
int64_t mdgl_workers(void);

/* No counterpart in the reference (it has no tracing). 1 when the library
 * pushes a roctx range named after each entry point around every call that
 * validates or launches (the environment held MDGL_ROCTX, not "0", when the
 * library first looked, and the ROCm roctx library
 * librocprofiler-sdk-roctx.so.1 was found), else 0. The ranges are host
 * time per call; `rocprofv3 --marker-trace` records them. */
int mdgl_trace_ranges(void);

/* Replaces capi.mojo:54-56. Inclusive int64 prefix sum, dst[i] = src[0..i]. */
int mdgl_cumsum(const int64_t* src, int64_t* dst, int64_t n, void* stream);

/* Segment offsets where the lengths live (the reference forms them on the
 * host: [0] + cumsum(seglen) and its checks, python/mojodgl/ops/segment.py:19-38;
 * no counterpart at its ABI): offsets[0] = 0, offsets[i + 1] = seglen[0] +
 * ... + seglen[i] (int32, valid when the total is below 2**31), and stats
 * (device, 4 int64) = (min length or 0 without segments, total, number of
 * chunk_len-row chunks of the segments longer than chunk_len, 0 when
 * chunk_len <= 0, max length or 0 without segments). The total wraps
 * around in int64 like the reference's cumsum: a caller checks min >= 0 and
 * max <= the row count before trusting it. Workspace:
 * mdgl_segment_offsets_workspace_bytes(num). */
int mdgl_segment_offsets(const int64_t* seglen, int64_t num, int64_t chunk_len, int32_t* offsets,
                         int64_t* stats, void* workspace, int64_t workspace_bytes, void* stream);
int64_t mdgl_segment_offsets_workspace_bytes(int64_t num);

/* Replaces capi.mojo:59-61. dst[i] = 0 where src[i] is +-inf, else src[i]. */
int mdgl_replace_inf_with_zero(const void* src, void* dst, int64_t n, int dtype, void* stream);

/* Replaces capi.mojo:64-66. dst[i] = min(max(src[i], lo), hi). */
int mdgl_clamp_i64(const int64_t* src, int64_t* dst, int64_t n, int64_t lo, int64_t hi,
                   void* stream);

/* Replaces capi.mojo:70-91 (`mdgl_gsddmm`): in edge-id order,
 *   dst[e] = op(lhs[t_l(e)], rhs[t_r(e)]), t = u: uids[e], v: vids[e], e: e.
 * dl / dr / dout are the operand and output row widths. `nd`, `lhs_shape`,
 * `rhs_shape` (host arrays) are the two operands' feature shapes padded to
 * the same rank (sddmm.py:24-47); nd = 0 means no broadcasting
 * (dl == dr == dout). For dot the last axis is contracted: it must be equal,
 * and dout counts the broadcast leading positions (1 for 2-D operands).
 * Copy ops read one operand and ignore the shapes. */
int mdgl_gsddmm(const int32_t* uids, const int32_t* vids, const void* lhs, const void* rhs,
                void* dst, int64_t num_edges, int lhs_target, int rhs_target, int op, int64_t dl,
                int64_t dr, int64_t dout, int nd, const int64_t* lhs_shape,
                const int64_t* rhs_shape, int dtype, void* stream);

/* Replaces capi.mojo:95-115 (`mdgl_gspmm`): over the in-edge CSR
 * (indptr, indices = source node, eid = edge id of each slot),
 *   dst[v] = reduce over slots i of row v of op(lhs[indices[i]], rhs[eid[i]]),
 * folded in CSR order; mean divides the sum by max(deg[v], 1) (deg may be
 * NULL: the row length); a row with no in-edges gets the reduce identity
 * (0, -inf, +inf) unless MDGL_REPLACE_INF is set.
 * Extensions: broadcasting as in mdgl_gsddmm; arg_u / arg_e (nullable, max
 * and min only) receive the source node and edge id of the selected message
 * (the first in CSR order among ties; -1 when no message was selected -- an
 * empty row, or only messages that never beat the identity -- and where
 * MDGL_REPLACE_INF replaced the value); rows longer than
 * chunk_len are split into the num_chunks chunks (chunk_row[c],
 * chunk_start[c]: each covers up to chunk_len slots) whose partials are
 * reduced in order per heavy row (heavy_rows[h], chunks
 * heavy_ptr[h]..heavy_ptr[h+1]) -- the chunks of every row of length
 * > chunk_len, in CSR order, and nothing else; num_chunks = 0 disables the
 * split. The partials live in `workspace` (mdgl_gspmm_workspace_bytes).
 * flags: MDGL_REPLACE_INF; MDGL_RHS_CSR_ORDER when the edge operand has been
 * put in CSR slot order (mdgl_gather_rows with eid), which turns its random
 * reads into streaming ones -- worth it for a narrow edge operand read by
 * several column slabs; arg_e still reports edge ids; MDGL_LHS_LINE_ROWS when
 * the node operand has been copied to rows that each start on a 128-byte
 * line (a row of dl elements whose size is no multiple of 128 bytes
 * otherwise starts mid-line, and every slab of its columns touches one line
 * more) -- worth it when each node row is gathered many times. */
int mdgl_gspmm(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
               const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op, int64_t dl,
               int64_t dr, int64_t dout, int reduce_op, const int32_t* deg, int nd,
               const int64_t* lhs_shape, const int64_t* rhs_shape, int32_t* arg_u,
               int32_t* arg_e, const int32_t* chunk_row, const int32_t* chunk_start,
               int64_t num_chunks, int32_t chunk_len, const int32_t* heavy_rows,
               const int32_t* heavy_ptr, int64_t num_heavy, void* workspace,
               int64_t workspace_bytes, int flags, int dtype, void* stream);

/* mdgl_gspmm over the listed rows only: dst[rows[i]] for i < num_rows, each
 * row whole (no heavy-row split: a row's messages fold in CSR order in one
 * unit), the other rows of dst left as they are. Rows outside [0, num_dst)
 * are skipped; a row listed twice is written twice with the same values.
 * Replaces the subgraph the reference builds for `pull`
 * (python/mojodgl/heterograph.py:318-347: the in-edges of the pulled nodes
 * cut out and reduced by update_all, then every other row zeroed): the
 * caller zero-fills dst and reduces the pulled rows of the graph's own CSR.
 * Same operands, flags and outputs as mdgl_gspmm. */
int mdgl_gspmm_rows(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                    const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op,
                    int64_t dl, int64_t dr, int64_t dout, int reduce_op, const int32_t* deg,
                    int nd, const int64_t* lhs_shape, const int64_t* rhs_shape, int32_t* arg_u,
                    int32_t* arg_e, const int32_t* rows, int64_t num_rows, int flags, int dtype,
                    void* stream);

/* The lane width (values per lane: 1, 2 or 4 in float32, 1 or 2 in
 * float64) and, when `group` is not null, the lanes per row slab (a power
 * of two up to 64) that mdgl_gspmm picks for these operands, shapes,
 * alignments and flags, so a caller can tell how many rows share a
 * wavefront (64 / group) and how many column slabs a row is cut into
 * (ceil(ceil(dout / vec) / group)). No counterpart in the
 * reference (its kernel is a CPU loop, src/ported.mojo:352-423); it is the
 * planning query behind the host's scheduling choices for a gspmm call. */
int mdgl_gspmm_lanes(int op, int64_t dl, int64_t dr, int64_t dout, int nd,
                     const int64_t* lhs_shape, const int64_t* rhs_shape, const void* lhs,
                     const void* rhs, int flags, int dtype, int64_t* vec, int64_t* group);

/* Locality of a graph for mdgl_gspmm's MDGL_NARROW_SLABS: partial[b]
 * (device int64, MDGL_COO_LOCALITY_BLOCKS of them) receives workgroup b's
 * count of the edges i (COO u, v on the GPU, int32) with |u[i] - v[i]| <
 * window; their sum is the count over all edges. No counterpart in the
 * reference (a scheduling statistic, computed once per graph). */
#define MDGL_COO_LOCALITY_BLOCKS 1024
int mdgl_coo_locality(const int32_t* u, const int32_t* v, int64_t num_edges, int64_t window,
                      int64_t* partial, void* stream);

/* Workspace mdgl_gspmm needs for `num_chunks` chunk partials. */
int64_t mdgl_gspmm_workspace_bytes(int64_t num_chunks, int64_t dout, int reduce_op, int dtype);

/* Bytes of the device scratch array of mdgl_gspmm_noalloc: one per GPU the
 * library runs on, held until the process ends. */
#define MDGL_NOALLOC_SCRATCH_BYTES (64ll << 20)

/* mdgl_gspmm without a workspace argument. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); nothing in
 * it allocates. Arguments and results are those of mdgl_gspmm; the heavy-row
 * partials go to a fixed device array of MDGL_NOALLOC_SCRATCH_BYTES per GPU
 * (the current device's: `stream` must belong to it). A call whose partials
 * need more (mdgl_gspmm_workspace_bytes(num_chunks, dout, reduce_op, dtype)
 * > MDGL_NOALLOC_SCRATCH_BYTES) returns MDGL_EWORKSPACE before launching.
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents (nothing in it needs to start at zero: a call writes every
 * partial it reads), so calls that overlap on one GPU -- on different
 * streams, or from threads without ordering -- race. */
int mdgl_gspmm_noalloc(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                       const void* lhs, const void* rhs, void* dst, int64_t num_dst, int op,
                       int64_t dl, int64_t dr, int64_t dout, int reduce_op, const int32_t* deg,
                       int nd, const int64_t* lhs_shape, const int64_t* rhs_shape,
                       int32_t* arg_u, int32_t* arg_e, const int32_t* chunk_row,
                       const int32_t* chunk_start, int64_t num_chunks, int32_t chunk_len,
                       const int32_t* heavy_rows, const int32_t* heavy_ptr, int64_t num_heavy,
                       int flags, int dtype, void* stream);

/* Replaces capi.mojo:119-129 (`mdgl_segment_reduce`): dst[s] = reduce of
 * value rows offsets[s]..offsets[s+1], in row order; mean divides by
 * max(length, 1) (= the reference's clamp(seglen, 1, n) divide,
 * segment.py:99-105). offsets has num_seg + 1 entries, non-decreasing, from
 * 0 to n (each is clamped into [0, n]). flags: MDGL_REPLACE_INF,
 * MDGL_SEGMENTS_SHORT. Segments longer than MDGL_SEGMENT_SPLIT_ROWS are
 * reduced by a workgroup of row streams whose partials are added in a fixed
 * order (max / min and their args unchanged, a sum to rounding); every
 * other segment is folded row by row. */
int mdgl_segment_reduce(const int32_t* offsets, const void* value, void* dst, int64_t num_seg,
                        int64_t d, int reduce_op, int64_t n, int flags, int dtype, void* stream);

/* mdgl_segment_reduce for max / min that also writes arg[s][k] (int32), the
 * row of the selected value: the first in row order among equal values, NaN
 * never selected, -1 when no row was selected (an empty segment, or only
 * values that never beat the identity) or MDGL_REPLACE_INF replaced the
 * value. No counterpart in the reference
 * (it emits no arg); the gradient of segment max / min flows to that row. */
int mdgl_segment_reduce_arg(const int32_t* offsets, const void* value, void* dst, int32_t* arg,
                            int64_t num_seg, int64_t d, int reduce_op, int64_t n, int flags,
                            int dtype, void* stream);

/* dst[i] (int32) = the segment holding row i, for the n rows of the segments
 * offsets[0..num_seg] (non-decreasing, 0 to n). No counterpart in the
 * reference: the row -> segment map of the segment gradients. */
int mdgl_segment_ids(const int32_t* offsets, int64_t num_seg, int64_t n, int32_t* dst,
                     void* stream);

/* Softmax planning. A softmax call serves rows by degree, with a lane layout
 * that depends on d, the dtype and the 16-byte alignment of the two buffers:
 * `slots` edge slots per wavefront. Rows of up to `chunk_len` (= 8 * slots)
 * edges are served whole; longer rows must be passed as chunks of chunk_len
 * edges. Call this with the buffers of the call to plan. No counterpart in the
 * reference (its split is a fixed 32-way CPU split, ported.mojo:34-42). */
int mdgl_softmax_geometry(int64_t d, int dtype, const void* logits, const void* out,
                          int64_t* slots, int64_t* chunk_len);
/* Workspace of a softmax call: partials of `num_chunks` chunks, plus a
 * (max, sum) table of `table_rows` rows for the two-pass edge_softmax:
 * bounds[nbins + 1] + num_chunks with a row order, num_nodes without. */
int64_t mdgl_softmax_workspace_bytes(int64_t num_chunks, int64_t table_rows, int64_t d,
                                     int dtype);

/* Replaces capi.mojo:132-138 (`mdgl_segment_softmax`): per segment and
 * column, softmax over the segment's rows; rows of empty segments are not
 * written. Segments are served through the plan of mdgl_edge_softmax_
 * (`order` / `bounds` / `nbins` by degree bin, or order null for every
 * segment in its own order, one wavefront each; `packed_eid` as there, with
 * the row index itself as the edge id); segments longer than
 * chunk_len come as chunks: chunk c covers rows chunk_start[c] ..
 * min(chunk_start[c] + chunk_len, offsets[chunk_row[c] + 1]) of segment
 * chunk_row[c], a segment's chunks are consecutive and chunk_first[c] is the
 * first of them. `slots` is the value mdgl_softmax_geometry returned.
 * `scratch` is accepted for signature compatibility and unused. */
int mdgl_segment_softmax(const int32_t* offsets, const void* value, void* dst, void* scratch,
                         int64_t num_seg, int64_t d, int64_t n, const int32_t* order,
                         const int64_t* bounds, int nbins, const int32_t* packed_eid,
                         const int32_t* chunk_row, const int32_t* chunk_start,
                         const int32_t* chunk_first, int64_t num_chunks, int64_t slots,
                         void* workspace, int64_t workspace_bytes, int dtype, void* stream);

/* mdgl_segment_softmax without a plan for the segments of at most
 * `chunk_len` rows (mdgl_softmax_geometry's, for these buffers): the
 * LDS-staged kernel writes their rows; the rows of longer segments are left
 * unwritten. Returns MDGL_ENOTSUP when the rows are too wide for that kernel
 * (more than 32 16-byte vectors). No counterpart in the reference: for
 * callers whose lengths are on the GPU, so the softmax can start before the
 * longest length is known on the host (a longer segment then needs the full
 * call with its chunk plan, which rewrites every row). */
int mdgl_segment_softmax_short(const int32_t* offsets, const void* value, void* dst,
                               int64_t num_seg, int64_t d, int64_t n, int dtype, void* stream);

/* Replaces capi.mojo:149-165 (`mdgl_edge_softmax_`): per CSR row, per
 * column, softmax of logits[eid[i]] over the row's slots whose edge is
 * selected (all_ones = 1, or mask[e] == 1); dst rows of the selected edges
 * are written. Plan: `order` (device) lists the rows of degree 1 .. chunk_len
 * sorted by degree, with host `bounds` (nbins + 2 entries, nbins =
 * log2(slots) + 1): bin k = order[bounds[k] .. bounds[k+1]) holds the rows of
 * degree <= 2^k (and > 2^(k-1)), order[bounds[nbins] .. bounds[nbins+1])
 * the rows of degree slots+1 .. chunk_len; or `order` = NULL: every row of
 * degree <= chunk_len in natural order. `packed_eid` (device, optional,
 * needs `order`): for the rows of bins 0 .. nbins-1 in order, 2^k entries per
 * row of bin k, the edge id eid[indptr[row] + s] of the row's slot s for
 * s < degree and -1 after it; it saves the packed rows the indptr and eid
 * lookups. Longer rows come as chunks, as in mdgl_segment_softmax. With
 * `slot_of_edge` (device, num_edges entries) the output is written by a
 * second, edge-parallel pass in edge-id order (coalesced stores) from a
 * (max, sum) table in the workspace: slot_of_edge[e] is the table slot of
 * edge e's CSR row (its destination -- or source -- node), which is the row's
 * position in `order`, bounds[nbins + 1] + the index of its first chunk for
 * a chunked row, or, with `order` NULL, the row itself. Without it every row
 * writes its own edges. `indices` and `scratch` are accepted for signature
 * compatibility and unused. */
int mdgl_edge_softmax_(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                       const int8_t* mask, const void* logits, void* dst, void* scratch,
                       int64_t num_nodes, int all_ones, int64_t d, const int32_t* order,
                       const int64_t* bounds, int nbins, const int32_t* packed_eid,
                       const int32_t* chunk_row, const int32_t* chunk_start,
                       const int32_t* chunk_first, int64_t num_chunks, int64_t slots,
                       const int32_t* slot_of_edge, int64_t num_edges, void* workspace,
                       int64_t workspace_bytes, int dtype, void* stream);

/* A streaming read of `bytes` (a multiple of 16) at `src`: a fixed grid of
 * 2,048 workgroups strides over it with 16-byte nontemporal loads, 32 KB per
 * workgroup and round; `sink` (mdgl_read_stream_sink_bytes(bytes), 16-byte
 * aligned) receives at most one 16-byte word per wavefront. No counterpart
 * in the reference: it is the measured ceiling of a one-pass read on this
 * GPU, the rate the library's bandwidth-bound kernels are judged against. */
int mdgl_read_stream(const void* src, int64_t bytes, void* sink, void* stream);
int64_t mdgl_read_stream_sink_bytes(int64_t bytes);

/* A bare read of rows by an index list: for i < n, the row idx[i] of `src`
 * (src_rows rows of row_bytes bytes, a multiple of 16 in [16, 1024]; indices
 * outside [0, src_rows) are skipped), a wavefront per 64 indices reading 16
 * bytes per lane, 8 rows in flight. Wavefront w writes the XOR of the 16-byte
 * vectors it read to sink[w] (mdgl_read_rows_sink_bytes(n) bytes, 16-byte
 * aligned); with dst_rows > 0 it also writes, to each of the rows
 * [w * dst_rows / W, (w + 1) * dst_rows / W) of `dst` (W = the wavefront
 * count, rows of row_bytes), the XOR of each vector position over its rows.
 * No counterpart in the reference: the ceiling of gspmm's source-row reads
 * (the in-CSR's sources as the index list), alone and beside its output's
 * write volume. */
int mdgl_read_rows(const void* src, int64_t src_rows, int64_t row_bytes, const int32_t* idx,
                   int64_t n, void* dst, int64_t dst_rows, void* sink, void* stream);
int64_t mdgl_read_rows_sink_bytes(int64_t n);

/* edge_softmax over a subset of edge ids, the whole call on the GPU with no
 * host read. Replaces the positional branch of the reference's host code
 * (python/mojodgl/ops/edge_softmax.py:119-158, the per-call Python grouping
 * loop before its mdgl_edge_softmax_ call, capi.mojo:149-165): position i
 * (0 <= i < num_sel) of `eids` (device, int64) belongs to the group of node
 * ends[eids[i]] (`ends`: device int32, the destination of every edge id for
 * norm_by 'dst', the source for 'src'), groups in ascending node id with
 * their positions in the order they appear, and reads logits[i]; dst rows
 * 0 .. num_sel - 1 receive the softmax of their group per column (rows past
 * num_sel are the caller's). Outputs for a backward pass: endpoint[i]
 * (num_sel), the grouping group_ptr (num_nodes + 1) / group_pos (num_sel,
 * positions grouped). id_range (device, 2 int64) receives the min and max of
 * eids: ids outside [0, num_edges) are clamped for every read (no access is
 * out of bounds) and make the results meaningless, so the caller checks
 * id_range before using them; `range_event` (a hipEvent_t, nullable) is
 * recorded on `stream` as soon as id_range is written, so the caller can copy
 * it back without waiting for the rest of the call. Needs `workspace`
 * (mdgl_edge_softmax_positional_workspace_bytes with the same d, buffers
 * and dtype). */
int mdgl_edge_softmax_positional(const int32_t* ends, int64_t num_edges, const int64_t* eids,
                                 int64_t num_sel, int64_t num_nodes, const void* logits,
                                 void* dst, int64_t d, int32_t* endpoint, int32_t* group_ptr,
                                 int32_t* group_pos, int64_t* id_range, void* range_event,
                                 void* workspace, int64_t workspace_bytes, int dtype,
                                 void* stream);

/* Workspace of mdgl_edge_softmax_positional (the logits and dst pointers
 * decide the lane width, as for mdgl_softmax_geometry); -1 for invalid
 * arguments. */
int64_t mdgl_edge_softmax_positional_workspace_bytes(int64_t num_sel, int64_t num_nodes,
                                                     int64_t d, const void* logits,
                                                     const void* dst, int dtype);

/* Replaces capi.mojo:141-145 (`mdgl_segment_mm`): out rows of segment r are
 * a[rows] @ b[r]; seglen_a (device, int64, r entries) sums to at most n and
 * rows past the sum are left as they are. Needs `workspace`
 * (mdgl_segment_mm_workspace_bytes). */
int mdgl_segment_mm(const void* a, const void* b, void* dst, const int64_t* seglen_a, int64_t n,
                    int64_t d1, int64_t r, int64_t d2, void* workspace, int64_t workspace_bytes,
                    int dtype, void* stream);
int64_t mdgl_segment_mm_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r, int dtype);

/* Replaces capi.mojo:169-173 (`mdgl_gather_mm`): dst[i] = a[i] @ b[idx_b[i]]
 * with idx_b (device, int64) in [0, r) (rows with other values are left
 * unwritten). `r` (the number of b blocks, at most 2048) is an added
 * argument; rows are bucketed by idx_b in `workspace`
 * (mdgl_gather_mm_workspace_bytes) and multiplied block by block. */
int mdgl_gather_mm(const void* a, const void* b, const int64_t* idx_b, void* dst, int64_t n,
                   int64_t d1, int64_t d2, int64_t r, void* workspace, int64_t workspace_bytes,
                   int dtype, void* stream);
int64_t mdgl_gather_mm_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r, int dtype);

/* Gradients of mdgl_segment_mm / mdgl_gather_mm (no counterpart in the
 * reference, which has no backward): with grad_out (n x d2) the gradient of
 * their output,
 *   grad_a[i] = grad_out[i] @ b[g(i)]^T            (n x d1; rows in no group
 *                                                  -- past the segments'
 *                                                  sum -- are left as they are)
 *   grad_b[g] = sum over the rows i of group g of a[i]^T grad_out[i]
 *                                                  (r x d1 x d2, 0 for an
 *                                                  empty group),
 * g(i) the segment of row i or idx_b[i]. Either output may be null; with
 * n, d1 or d2 zero nothing is written. grad_b
 * is formed per chunk of a group's rows on the matrix cores and the chunks
 * are added in order, so it is the same on every run. Workspace:
 * mdgl_*_mm_grad_workspace_bytes. */
int mdgl_segment_mm_grad(const void* a, const void* b, const void* grad_out,
                         const int64_t* seglen_a, void* grad_a, void* grad_b, int64_t n,
                         int64_t d1, int64_t r, int64_t d2, void* workspace,
                         int64_t workspace_bytes, int dtype, void* stream);
int64_t mdgl_segment_mm_grad_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r,
                                             int dtype);
int mdgl_gather_mm_grad(const void* a, const void* b, const int64_t* idx_b, const void* grad_out,
                        void* grad_a, void* grad_b, int64_t n, int64_t d1, int64_t d2,
                        int64_t r, void* workspace, int64_t workspace_bytes, int dtype,
                        void* stream);
int64_t mdgl_gather_mm_grad_workspace_bytes(int64_t n, int64_t d1, int64_t d2, int64_t r,
                                            int dtype);

/* Graph build: replaces DGLGraph._build_csr (python/mojodgl/heterograph.py:69-86),
 * which the reference runs in numpy on the host. Groups the edges 0..num_edges-1
 * (COO in edge-id order, int32 on the GPU) by `key` (v for the in-CSR, u for
 * the out-CSR; values in [0, num_rows), not checked here):
 *   indptr  (num_rows + 1) = [0] + cumsum(bincount(key)),
 *   eid     (num_edges)    = argsort(key, stable): inside a row, increasing edge id,
 *   indices (num_edges)    = other[eid].
 * Bit-identical to the numpy build. `other` and `indices` may both be null
 * (grouping only). Workspace: mdgl_build_csr_workspace_bytes (0 when
 * num_rows <= 1 or there are no edges; null is then accepted). */
int mdgl_build_csr(const int32_t* key, const int32_t* other, int64_t num_edges, int64_t num_rows,
                   int32_t* indptr, int32_t* indices, int32_t* eid, void* workspace,
                   int64_t workspace_bytes, void* stream);
int64_t mdgl_build_csr_workspace_bytes(int64_t num_edges, int64_t num_rows);

/* Backward helpers. The reference has no backward pass (README.md:110-114); these
 * are the elementwise steps of the gradients of gspmm / gsddmm / edge_softmax
 * whose reductions run through the forward entry points above.
 *
 * mdgl_gspmm_edge_grad: the gradient reaching each edge's message from
 *   grad_out (num_rows x d, rows indexed by vids[e], the destination):
 *   dst[e, k] = alpha * grad_out[v, k] / (mean ? max(indptr[v+1] - indptr[v], 1) : 1)
 *               * (arg_e ? (arg_e[v, k] == e) : 1)
 *   arg_e (num_rows x d int32, from a max / min mdgl_gspmm) may be null. */
int mdgl_gspmm_edge_grad(const int32_t* vids, const int32_t* indptr, const void* grad_out,
                         const int32_t* arg_e, void* dst, int64_t num_edges, int64_t d, int mean,
                         double alpha, int dtype, void* stream);

/* mdgl_edge_softmax_grad: dst[e][k] = a[e][k] * (grad[e][k] - row_sum[row_of[e]][k]),
 *   the last steps of the edge_softmax gradient (a the softmax output, row_sum
 *   the per-row sums of grad * a over the CSR of norm_by, row_of the
 *   destination -- or source -- node of every edge id). */
int mdgl_edge_softmax_grad(const int32_t* row_of, const void* a, const void* grad,
                           const void* row_sum, void* dst, int64_t num_edges, int64_t d, int dtype,
                           void* stream);

/* mdgl_gspmm_mul_sum_dot: one pass for both gradients of a u_mul_e_sum whose
 *   edge operand is constant over groups of D = dout / dr consecutive columns
 *   (an edge operand of shape (E, ..., 1) against node rows (N, ..., D)),
 *   run over the CSR of the reversed graph (rows = sources, indices =
 *   destinations, the arguments of mdgl_gspmm with op mul, reduce sum):
 *     dst[row][k]  = sum over the row's slots j, in CSR order, of
 *                    lhs[indices[j]][k] * rhs[eid[j]][k / D]   (as mdgl_gspmm)
 *     dot[j][c]    = sum over k in group c of lhs[indices[j]][k] * rowop[row][k]
 *   i.e. with lhs = the output gradient and rowop = the node operand, the
 *   node operand's gradient and, in CSR slot order, the edge operand's.
 *   Needs 16-byte lanes (dout a multiple of 16 / sizeof(T), lhs, rowop and
 *   the group's columns aligned) and D / (16 / sizeof(T)) a power of two up
 *   to 64; other shapes return MDGL_ENOTSUP (compute the two with
 *   mdgl_gspmm and mdgl_gsddmm then). No counterpart in the reference. */
int mdgl_gspmm_mul_sum_dot(const int32_t* indptr, const int32_t* indices, const int32_t* eid,
                           const void* lhs, const void* rhs, const void* rowop, void* dst,
                           void* dot, int64_t num_dst, int64_t dl, int64_t dr, int64_t dout,
                           int nd, const int64_t* lhs_shape, const int64_t* rhs_shape,
                           const int32_t* chunk_row, const int32_t* chunk_start,
                           int64_t num_chunks, int32_t chunk_len, const int32_t* heavy_rows,
                           const int32_t* heavy_ptr, int64_t num_heavy, void* workspace,
                           int64_t workspace_bytes, int dtype, void* stream);

/* dst[r, k] = src[r, k] / max(indptr[r+1] - indptr[r], 1): the mean's divisor on a
 * node-shaped gradient. */
int mdgl_rows_by_degree(const int32_t* indptr, const void* src, void* dst, int64_t rows,
                        int64_t d, int dtype, void* stream);

/* dst[i, :] = src[idx[i], :] for rows of `width` elements (the edge operand of a
 * gspmm put in CSR slot order with idx = eid). No counterpart in the reference. */
int mdgl_gather_rows(const void* src, const int32_t* idx, void* dst, int64_t n, int64_t width,
                     int dtype, void* stream);

/* dst[idx[i], :] = src[i, :] for rows of `width` elements, the inverse of
 * mdgl_gather_rows when idx is a permutation (rows of gather_mm's sorted
 * route put back in their original order; with repeated indices which row
 * lands is unspecified). No counterpart in the reference. */
int mdgl_scatter_rows(const void* src, const int32_t* idx, void* dst, int64_t n, int64_t width,
                      int dtype, void* stream);

/* dst[i] = mask[i] != 0 ? src[i] : 0 (mask, src and dst of one dtype): the
 * per-edge terms of a max / min gradient made exactly zero on the edges no
 * output selected, whatever the other operand holds there. No counterpart
 * in the reference. */
int mdgl_keep_where(const void* mask, const void* src, void* dst, int64_t n, int dtype,
                    void* stream);

/* dst[i] = alpha * src[i]. */
int mdgl_scale(const void* src, void* dst, int64_t n, double alpha, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MDGL_H */
