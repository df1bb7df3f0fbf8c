// The plan of edge_softmax over a subset of edge ids, built on the GPU with
// no host read: the reference's positional rule (python/mojodgl/ops/
// edge_softmax.py:119-158) groups the positions i of `eids` by the endpoint
// of edge eids[i] (groups in ascending endpoint, positions in the order they
// appear) and position i reads logits[i].
//
//   1. endpoint[i] = ends[eids[i]] (ids clamped into the edges, so nothing is
//      read out of bounds; the min and max of the ids go to id_range for the
//      caller to check), reduced per workgroup and then by one workgroup;
//   2. the stable radix grouping of the positions by endpoint (csr.hip):
//      group_ptr / group_pos, the CSR the softmax runs over;
//   3. rows binned by degree (packed bins of 1, 2, 4 .. slots edges, wavefront
//      rows up to chunk_len, chunked rows) and grouped by bin, stably, by one
//      radix pass; each long row's chunk count, scanned into chunk offsets;
//   4. one thread turns the bin bounds and the chunk total into the launch
//      figures (SoftDyn), which the softmax kernels read from device memory;
//   5. the chunk list and the packed rows' position lists are written.
// Every step counts integers, so the plan is the same on every run.
#include "mdgl_kernels.h"

namespace mdgl {

namespace {

constexpr int RANGE_BLOCKS = 1024;  // workgroups of the endpoint gather

__device__ __forceinline__ void block_min_max(int64_t& lo, int64_t& hi) {
  __shared__ int64_t s_lo[WAVES_PER_BLOCK], s_hi[WAVES_PER_BLOCK];
  for (int off = 32; off >= 1; off >>= 1) {
    const int64_t a = __shfl_xor(lo, off), b = __shfl_xor(hi, off);
    lo = a < lo ? a : lo;
    hi = b > hi ? b : hi;
  }
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  if (lane == 0) {
    s_lo[w] = lo;
    s_hi[w] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < WAVES_PER_BLOCK; ++q) {
      lo = s_lo[q] < lo ? s_lo[q] : lo;
      hi = s_hi[q] > hi ? s_hi[q] : hi;
    }
  }
}

// endpoint[i] = ends[clamp(eids[i])]; per-workgroup min / max of the ids
__global__ __launch_bounds__(BLOCK) void pos_gather_kernel(const int64_t* __restrict__ eids,
                                                           int64_t m,
                                                           const int32_t* __restrict__ ends,
                                                           int64_t num_edges,
                                                           int32_t* __restrict__ endpoint,
                                                           int64_t* __restrict__ part) {
  int64_t lo = INT64_MAX, hi = INT64_MIN;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < m;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t id = eids[i];
    lo = id < lo ? id : lo;
    hi = id > hi ? id : hi;
    const int64_t c = id < 0 ? 0 : (id >= num_edges ? num_edges - 1 : id);
    endpoint[i] = ends[c];
  }
  block_min_max(lo, hi);
  if (threadIdx.x == 0) {
    part[2 * blockIdx.x] = lo;
    part[2 * blockIdx.x + 1] = hi;
  }
}

__global__ __launch_bounds__(BLOCK) void range_final_kernel(const int64_t* __restrict__ part,
                                                            int nparts,
                                                            int64_t* __restrict__ id_range) {
  int64_t lo = INT64_MAX, hi = INT64_MIN;
  for (int b = threadIdx.x; b < nparts; b += BLOCK) {
    lo = part[2 * b] < lo ? part[2 * b] : lo;
    hi = part[2 * b + 1] > hi ? part[2 * b + 1] : hi;
  }
  block_min_max(lo, hi);
  if (threadIdx.x == 0) {
    id_range[0] = lo;
    id_range[1] = hi;
  }
}

// Bin of each row: k = ceil(log2(degree)) for 1 <= degree <= slots (packed
// bin k, 2^k slots per row), nbins for slots < degree <= chunk_len (a
// wavefront each), nbins + 1 for empty and chunked rows; and the chunk count
// of a chunked row (0 otherwise).
__global__ __launch_bounds__(BLOCK) void row_bins_kernel(const int32_t* __restrict__ ptr,
                                                         int64_t rows, int slots, int chunk_len,
                                                         int nbins, int32_t* __restrict__ key,
                                                         int64_t* __restrict__ chunks) {
  for (int64_t r = (int64_t)blockIdx.x * BLOCK + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * BLOCK) {
    const int deg = ptr[r + 1] - ptr[r];
    int k;
    if (deg == 0 || deg > chunk_len) {
      k = nbins + 1;
    } else if (deg > slots) {
      k = nbins;
    } else {
      k = 0;
      while ((1 << k) < deg) ++k;
    }
    key[r] = k;
    chunks[r] = deg > chunk_len ? (deg + chunk_len - 1) / chunk_len : 0;
  }
}

// The launch figures from the bin bounds (bptr: nbins + 3 offsets of the rows
// grouped by bin) and the chunk total (cstats[1]); one thread.
__global__ void soft_dyn_kernel(const int32_t* __restrict__ bptr,
                                const int64_t* __restrict__ cstats, int nbins, int Pw, int S,
                                int pk_u, SoftDyn* __restrict__ dyn) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  int64_t waves = 0, slots_before = 0;
  for (int k = 0; k < nbins; ++k) {
    const int64_t cnt = (int64_t)bptr[k + 1] - bptr[k];
    const int64_t per = Pw >> k;
    dyn->bin_start[k] = bptr[k];
    dyn->bin_slot[k] = slots_before;
    dyn->bin_wave[k] = waves;
    slots_before += cnt << k;
    const int64_t wk = ((cnt + per - 1) / per) * S;
    waves += (wk + pk_u - 1) / pk_u * pk_u;  // a packed wavefront never straddles two bins
  }
  dyn->bin_start[nbins] = bptr[nbins];
  dyn->bin_slot[nbins] = slots_before;
  dyn->bin_wave[nbins] = waves;
  dyn->mid_start = bptr[nbins];
  dyn->mid_end = bptr[nbins + 1];
  dyn->light_waves = ((int64_t)bptr[nbins + 1] - bptr[nbins]) * S;
  dyn->packed_tasks = waves / pk_u;
  dyn->num_chunks = cstats[1];
  dyn->chunk_waves = cstats[1] * S;
}

// Chunks of every row longer than chunk_len, at the row's scanned offset.
__global__ __launch_bounds__(BLOCK) void chunk_fill_kernel(const int32_t* __restrict__ ptr,
                                                           const int32_t* __restrict__ coff,
                                                           int64_t rows, int chunk_len,
                                                           int32_t* __restrict__ chunk_row,
                                                           int32_t* __restrict__ chunk_start,
                                                           int32_t* __restrict__ chunk_first) {
  for (int64_t r = (int64_t)blockIdx.x * BLOCK + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * BLOCK) {
    const int start = ptr[r], deg = ptr[r + 1] - start;
    if (deg <= chunk_len) continue;
    const int first = coff[r], n = coff[r + 1] - first;
    for (int j = 0; j < n; ++j) {
      chunk_row[first + j] = (int32_t)r;
      chunk_start[first + j] = start + j * chunk_len;
      chunk_first[first + j] = first;
    }
  }
}

// The packed rows' positions slot by slot: entry j of bin k (2^k per row,
// rows in bin order) holds the row's position at that slot, or -1 past its
// degree. One thread per entry, so the stores are coalesced.
__global__ __launch_bounds__(BLOCK) void packed_fill_kernel(const SoftDyn* __restrict__ dyn,
                                                            int nbins,
                                                            const int32_t* __restrict__ order,
                                                            const int32_t* __restrict__ ptr,
                                                            const int32_t* __restrict__ pos,
                                                            int32_t* __restrict__ packed) {
  const int64_t total = dyn->bin_slot[nbins];
  for (int64_t j = (int64_t)blockIdx.x * BLOCK + threadIdx.x; j < total;
       j += (int64_t)gridDim.x * BLOCK) {
    int k = 0;
    while (k + 1 < nbins && dyn->bin_slot[k + 1] <= j) ++k;
    const int64_t local = j - dyn->bin_slot[k];
    const int64_t i = dyn->bin_start[k] + (local >> k);
    const int s = (int)(local & ((int64_t(1) << k) - 1));
    const int32_t row = order[i];
    const int start = ptr[row], deg = ptr[row + 1] - start;
    packed[j] = s < deg ? pos[start + s] : -1;
  }
}

unsigned grid_rows(int64_t n) {
  int64_t b = (n + BLOCK - 1) / BLOCK;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

int64_t al256(int64_t b) { return (b + 255) / 256 * 256; }

}  // namespace

int64_t positional_max_chunks(int64_t num_sel, int64_t chunk_len) {
  // chunked rows have more than chunk_len positions each: at most
  // num_sel / (chunk_len + 1) of them, and ceil(deg / chunk_len) <=
  // deg / chunk_len + 1 chunks each
  return num_sel / chunk_len + num_sel / (chunk_len + 1) + 1;
}

int64_t positional_scratch_bytes(int64_t num_sel, int64_t num_nodes) {
  const int64_t radix = csr_workspace_bytes(num_sel, num_nodes);
  const int64_t radix_rows = csr_workspace_bytes(num_nodes, SOFT_MAX_BINS + 2);
  return al256(radix > radix_rows ? radix : radix_rows)  // radix workspace (reused)
         + al256(num_nodes * 4)                           // row bins
         + al256(num_nodes * 8)                           // chunk counts
         + al256((num_nodes + 1) * 4)                     // chunk offsets
         + al256(4 * 8)                                   // their figures
         + al256(segment_offsets_workspace_bytes(num_nodes))
         + al256((SOFT_MAX_BINS + 3) * 4)                 // bin bounds
         + al256(2 * RANGE_BLOCKS * 8);                   // partial id ranges
}

hipError_t launch_positional_plan(const PositionalPlan& p, hipStream_t s) {
  char* w = static_cast<char*>(p.scratch);
  const int64_t radix = csr_workspace_bytes(p.num_sel, p.num_nodes);
  const int64_t radix_rows = csr_workspace_bytes(p.num_nodes, SOFT_MAX_BINS + 2);
  void* rws = w;
  w += al256(radix > radix_rows ? radix : radix_rows);
  int32_t* rkey = reinterpret_cast<int32_t*>(w);
  w += al256(p.num_nodes * 4);
  int64_t* cc = reinterpret_cast<int64_t*>(w);
  w += al256(p.num_nodes * 8);
  int32_t* coff = reinterpret_cast<int32_t*>(w);
  w += al256((p.num_nodes + 1) * 4);
  int64_t* cstats = reinterpret_cast<int64_t*>(w);
  w += al256(4 * 8);
  void* segws = w;
  w += al256(segment_offsets_workspace_bytes(p.num_nodes));
  int32_t* bptr = reinterpret_cast<int32_t*>(w);
  w += al256((SOFT_MAX_BINS + 3) * 4);
  int64_t* part = reinterpret_cast<int64_t*>(w);

  // 1. endpoints and the id range
  int64_t gb = (p.num_sel + BLOCK - 1) / BLOCK;
  gb = gb < 1 ? 1 : (gb > RANGE_BLOCKS ? RANGE_BLOCKS : gb);
  hipLaunchKernelGGL(pos_gather_kernel, dim3((unsigned)gb), dim3(BLOCK), 0, s, p.eids, p.num_sel,
                     p.ends, p.num_edges, p.endpoint, part);
  hipLaunchKernelGGL(range_final_kernel, dim3(1), dim3(BLOCK), 0, s, part, (int)gb, p.id_range);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.range_event) {
    e = hipEventRecord(p.range_event, s);
    if (e != hipSuccess) return e;
  }
  // 2. positions grouped by endpoint
  e = launch_build_csr(p.endpoint, nullptr, p.num_sel, p.num_nodes, p.group_ptr, nullptr,
                       p.group_pos, rws, s);
  if (e != hipSuccess) return e;
  // 3. rows by bin, chunk offsets
  hipLaunchKernelGGL(row_bins_kernel, dim3(grid_rows(p.num_nodes)), dim3(BLOCK), 0, s,
                     p.group_ptr, p.num_nodes, p.slots, p.chunk_len, p.nbins, rkey, cc);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_build_csr(rkey, nullptr, p.num_nodes, p.nbins + 2, bptr, nullptr, p.order, rws, s);
  if (e != hipSuccess) return e;
  e = launch_segment_offsets(cc, p.num_nodes, 0, coff, cstats, segws, s);
  if (e != hipSuccess) return e;
  // 4. launch figures
  hipLaunchKernelGGL(soft_dyn_kernel, dim3(1), dim3(WAVE), 0, s, bptr, cstats, p.nbins, p.Pw,
                     p.S, SOFT_PK_U, p.dyn);
  // 5. chunk list and packed positions
  hipLaunchKernelGGL(chunk_fill_kernel, dim3(grid_rows(p.num_nodes)), dim3(BLOCK), 0, s,
                     p.group_ptr, coff, p.num_nodes, p.chunk_len, p.chunk_row, p.chunk_start,
                     p.chunk_first);
  hipLaunchKernelGGL(packed_fill_kernel, dim3(grid_rows(2 * p.num_sel)), dim3(BLOCK), 0, s, p.dyn,
                     p.nbins, p.order, p.group_ptr, p.group_pos, p.packed);
  return hipGetLastError();
}

}  // namespace mdgl
