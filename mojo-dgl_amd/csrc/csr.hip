// Graph build on the GPU: COO (edge-id order) -> CSR grouped by one endpoint,
// the reference's DGLGraph._build_csr (python/mojodgl/heterograph.py:69-86):
// indptr = [0] + cumsum(bincount(key)), order = argsort(key, stable),
// indices = other[order].
//
// The stable argsort is an LSD radix sort of (key, edge id) pairs, 8-bit
// digits, as many passes as the node count needs (3 up to 16M nodes). Each
// pass is three kernels: per-chunk digit counts (LDS histogram), a column
// scan per digit over the chunks, and a scatter in which each workgroup walks
// its chunk in order and ranks equal digits inside a wavefront with ballots,
// so equal keys keep their input order. Every step is integer counting, so
// the result is the numpy stable argsort bit for bit. indptr then comes from
// the sorted keys (row r starts at the first slot whose key is >= r) and the
// indices from one gather.
#include "mdgl_kernels.h"

namespace mdgl {

namespace {

constexpr int RADIX = 256;          // digit values; one thread each in a workgroup
constexpr int RADIX_CHUNK = 4096;   // keys per workgroup per pass
static_assert(RADIX == BLOCK, "one thread per digit value");

__device__ __forceinline__ int digit_of(int32_t key, int shift) {
  return (int)(((uint32_t)key >> shift) & (RADIX - 1));
}

// counts[b * RADIX + d] = keys of chunk b whose digit is d
__global__ __launch_bounds__(BLOCK) void radix_count_kernel(const int32_t* __restrict__ keys,
                                                            int64_t n, int shift,
                                                            int32_t* __restrict__ counts) {
  __shared__ int32_t hist[RADIX];
  hist[threadIdx.x] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * RADIX_CHUNK;
  const int64_t hi = lo + RADIX_CHUNK < n ? lo + RADIX_CHUNK : n;
  for (int64_t i = lo + threadIdx.x; i < hi; i += BLOCK)
    atomicAdd(&hist[digit_of(keys[i], shift)], 1);
  __syncthreads();
  counts[blockIdx.x * RADIX + threadIdx.x] = hist[threadIdx.x];
}

// One workgroup per digit d: counts[b * RADIX + d] becomes the exclusive
// prefix over chunks b (the digit-local position of chunk b's first key of
// digit d) and totals[d] the digit's count. Threads take contiguous spans of
// chunks; span sums are scanned in LDS.
__global__ __launch_bounds__(BLOCK) void radix_colscan_kernel(int32_t* __restrict__ counts,
                                                              int32_t* __restrict__ totals,
                                                              int64_t nchunks) {
  __shared__ int32_t part[BLOCK];
  const int64_t d = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t span = (nchunks + BLOCK - 1) / BLOCK;
  const int64_t lo = t * span < nchunks ? t * span : nchunks;
  const int64_t hi = lo + span < nchunks ? lo + span : nchunks;
  int32_t s = 0;
  for (int64_t b = lo; b < hi; ++b) s += counts[b * RADIX + d];
  part[t] = s;
  __syncthreads();
  for (int off = 1; off < BLOCK; off <<= 1) {
    const int32_t add = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += add;
    __syncthreads();
  }
  int32_t run = t > 0 ? part[t - 1] : 0;
  for (int64_t b = lo; b < hi; ++b) {
    const int32_t c = counts[b * RADIX + d];
    counts[b * RADIX + d] = run;
    run += c;
  }
  if (t == BLOCK - 1) totals[d] = part[BLOCK - 1];
}

// Stable scatter of chunk b: key i goes to digit_start[d] + counts[b][d] +
// (keys of digit d before it in the chunk). vals_in null means the edge ids
// 0..n-1 (the first pass).
//
// Wavefront w owns the chunk's quarter [w * Q, (w + 1) * Q) (Q = RADIX_PER *
// 64 keys) and loads it at once, RADIX_PER keys per lane (coalesced rows of
// 64). It ranks its keys in order, 64 at a time, with ballots (lanes whose
// digit agrees bit by bit) and a per-wavefront digit cursor in LDS, with no
// workgroup barrier. One barrier later each digit's count per wavefront is
// known: the chunk's keys are placed in LDS in digit order (digit, then
// wavefront, then rank: the input order within a digit), and the workgroup
// writes them out from there in that order, so each digit's keys leave as one
// contiguous run instead of single scattered elements.
constexpr int RADIX_PER = RADIX_CHUNK / BLOCK;  // keys per lane
static_assert(RADIX_PER * BLOCK == RADIX_CHUNK, "a chunk is RADIX_PER keys per lane");

__global__ __launch_bounds__(BLOCK) void radix_scatter_kernel(
    const int32_t* __restrict__ keys_in, const int32_t* __restrict__ vals_in,
    int32_t* __restrict__ keys_out, int32_t* __restrict__ vals_out,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ totals, int64_t n,
    int shift) {
  __shared__ int32_t scan[RADIX];
  __shared__ int32_t cur[WAVES_PER_BLOCK][RADIX];  // per wavefront: keys of each digit so far
  __shared__ int32_t gbase[RADIX];                 // output index of sorted slot 0 of digit d
  __shared__ int32_t skey[RADIX_CHUNK];
  __shared__ int32_t sval[RADIX_CHUNK];
  const int t = threadIdx.x;
  const int lane = t & (WAVE - 1), w = t >> 6;
  const uint64_t below = lane ? (~uint64_t(0) >> (64 - lane)) : 0;
  const int64_t lo = (int64_t)blockIdx.x * RADIX_CHUNK;
  const int nk = (int)(n - lo < RADIX_CHUNK ? n - lo : RADIX_CHUNK);
  // this wavefront's keys: row j of its quarter is keys [q0 + 64 j, q0 + 64 j + 64)
  const int q0 = w * (RADIX_PER * WAVE);
  int32_t key[RADIX_PER], val[RADIX_PER];
#pragma unroll
  for (int j = 0; j < RADIX_PER; ++j) {
    const int i = q0 + j * WAVE + lane;
    key[j] = 0;
    val[j] = 0;
    if (i < nk) {
      key[j] = keys_in[lo + i];
      val[j] = vals_in ? vals_in[lo + i] : (int32_t)(lo + i);
    }
  }
#pragma unroll
  for (int q = 0; q < WAVES_PER_BLOCK; ++q) cur[q][t] = 0;
  // digit starts: exclusive scan of the totals
  scan[t] = totals[t];
  __syncthreads();
  for (int off = 1; off < RADIX; off <<= 1) {
    const int32_t add = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += add;
    __syncthreads();
  }
  const int32_t dstart = scan[t] - totals[t] + counts[blockIdx.x * RADIX + t];
  // rank within the wavefront, in input order
  int32_t rank[RADIX_PER];
#pragma unroll
  for (int j = 0; j < RADIX_PER; ++j) {
    const bool ok = q0 + j * WAVE + lane < nk;
    const int dg = digit_of(key[j], shift);
    uint64_t same = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const uint64_t ones = __ballot(ok && ((dg >> bit) & 1));
      same &= ((dg >> bit) & 1) ? ones : ~ones;  // lanes whose digit agrees on this bit
    }
    const int r = __popcll(same & below);
    const int32_t base = ok ? cur[w][dg] : 0;
    rank[j] = base + r;
    __builtin_amdgcn_wave_barrier();
    if (ok && r == 0) cur[w][dg] = base + __popcll(same);
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // digit t: its keys per wavefront -> the slots of each wavefront's run in
  // the chunk's digit order, and where the digit's run goes in the output
  int32_t c[WAVES_PER_BLOCK];
  int32_t tot = 0;
#pragma unroll
  for (int q = 0; q < WAVES_PER_BLOCK; ++q) {
    c[q] = cur[q][t];
    tot += c[q];
  }
  __syncthreads();
  scan[t] = tot;
  __syncthreads();
  for (int off = 1; off < RADIX; off <<= 1) {
    const int32_t add = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += add;
    __syncthreads();
  }
  const int32_t lstart = scan[t] - tot;  // first slot of digit t in the chunk's digit order
  int32_t run = lstart;
#pragma unroll
  for (int q = 0; q < WAVES_PER_BLOCK; ++q) {
    cur[q][t] = run;  // now: the first slot of wavefront q's keys of digit t
    run += c[q];
  }
  gbase[t] = dstart - lstart;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < RADIX_PER; ++j) {
    if (q0 + j * WAVE + lane < nk) {
      const int s = cur[w][digit_of(key[j], shift)] + rank[j];
      skey[s] = key[j];
      sval[s] = val[j];
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < RADIX_PER; ++j) {
    const int s = j * BLOCK + t;
    if (s < nk) {
      const int32_t k = skey[s];
      const int32_t pos = gbase[digit_of(k, shift)] + s;
      keys_out[pos] = k;
      vals_out[pos] = sval[s];
    }
  }
}

__global__ __launch_bounds__(BLOCK) void iota_kernel(int32_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK)
    out[i] = (int32_t)i;
}

// indptr[r] = first slot whose key is >= r, for r in [0, num_rows]: slot i
// writes the rows in (key[i-1], key[i]]; the thread for i == n closes the
// rows after the last key.
__global__ __launch_bounds__(BLOCK) void indptr_kernel(const int32_t* __restrict__ skeys,
                                                       int64_t n, int64_t num_rows,
                                                       int32_t* __restrict__ indptr) {
  const int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x;
  if (i > n) return;
  int64_t k = i < n ? (int64_t)skeys[i] : num_rows;
  int64_t prev = i > 0 ? (int64_t)skeys[i - 1] : -1;
  if (k > num_rows) k = num_rows;
  if (prev > num_rows) prev = num_rows;
  for (int64_t r = prev + 1; r <= k; ++r) indptr[r] = (int32_t)i;
}

__global__ __launch_bounds__(BLOCK) void gather_i32_kernel(const int32_t* __restrict__ src,
                                                           const int32_t* __restrict__ idx,
                                                           int32_t* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK)
    out[i] = src[idx[i]];
}

// Each workgroup counts its grid-stride share of the edges whose endpoints
// differ by less than `window` and writes the count to partial[blockIdx.x]
// (no atomics: the caller adds the COO_LOCALITY_BLOCKS counts).
__global__ __launch_bounds__(BLOCK) void coo_locality_kernel(const int32_t* __restrict__ u,
                                                             const int32_t* __restrict__ v,
                                                             int64_t n, int64_t window,
                                                             int64_t* __restrict__ partial) {
  __shared__ int64_t sums[WAVES_PER_BLOCK];
  int64_t c = 0;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t d = (int64_t)u[i] - (int64_t)v[i];
    c += (d < window && -d < window) ? 1 : 0;
  }
  for (int off = WAVE / 2; off > 0; off >>= 1) c += __shfl_xor(c, off);
  const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
  if (lane == 0) sums[w] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t t = 0;
    for (int i = 0; i < WAVES_PER_BLOCK; ++i) t += sums[i];
    partial[blockIdx.x] = t;
  }
}

unsigned grid_of(int64_t n) {
  int64_t b = (n + BLOCK - 1) / BLOCK;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

int radix_passes(int64_t num_rows) {
  int bits = 0;
  while ((int64_t(1) << bits) < num_rows) ++bits;
  return (bits + 7) / 8;
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

}  // namespace

int64_t csr_workspace_bytes(int64_t num_edges, int64_t num_rows) {
  if (radix_passes(num_rows) == 0 || num_edges == 0) return 0;
  const int64_t nchunks = (num_edges + RADIX_CHUNK - 1) / RADIX_CHUNK;
  return align256(nchunks * RADIX * 4) + align256(RADIX * 4) + 3 * align256(num_edges * 4);
}

hipError_t launch_build_csr(const int32_t* key, const int32_t* other, int64_t num_edges,
                            int64_t num_rows, int32_t* indptr, int32_t* indices, int32_t* eid,
                            void* workspace, hipStream_t stream) {
  const int passes = num_edges ? radix_passes(num_rows) : 0;
  const int32_t* sorted_keys = key;
  if (passes == 0) {
    // at most one row: every key is 0, the order is the identity
    if (num_edges)
      hipLaunchKernelGGL(iota_kernel, dim3(grid_of(num_edges)), dim3(BLOCK), 0, stream, eid,
                         num_edges);
  } else {
    const int64_t nchunks = (num_edges + RADIX_CHUNK - 1) / RADIX_CHUNK;
    char* w = static_cast<char*>(workspace);
    int32_t* counts = reinterpret_cast<int32_t*>(w);
    w += align256(nchunks * RADIX * 4);
    int32_t* totals = reinterpret_cast<int32_t*>(w);
    w += align256(RADIX * 4);
    int32_t* keys_buf[2];
    keys_buf[0] = reinterpret_cast<int32_t*>(w);
    w += align256(num_edges * 4);
    keys_buf[1] = reinterpret_cast<int32_t*>(w);
    w += align256(num_edges * 4);
    int32_t* vals_tmp = reinterpret_cast<int32_t*>(w);
    const int32_t* kin = key;
    const int32_t* vin = nullptr;
    for (int p = 0; p < passes; ++p) {
      const int shift = 8 * p;
      int32_t* kout = keys_buf[p & 1];
      // the last pass lands in eid
      int32_t* vout = ((passes - 1 - p) % 2 == 0) ? eid : vals_tmp;
      hipLaunchKernelGGL(radix_count_kernel, dim3((unsigned)nchunks), dim3(BLOCK), 0, stream,
                         kin, num_edges, shift, counts);
      hipLaunchKernelGGL(radix_colscan_kernel, dim3(RADIX), dim3(BLOCK), 0, stream, counts,
                         totals, nchunks);
      hipLaunchKernelGGL(radix_scatter_kernel, dim3((unsigned)nchunks), dim3(BLOCK), 0, stream,
                         kin, vin, kout, vout, counts, totals, num_edges, shift);
      kin = kout;
      vin = vout;
    }
    sorted_keys = kin;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(indptr_kernel, dim3((unsigned)((num_edges + 1 + BLOCK - 1) / BLOCK)),
                     dim3(BLOCK), 0, stream, sorted_keys, num_edges, num_rows, indptr);
  if (num_edges && other)
    hipLaunchKernelGGL(gather_i32_kernel, dim3(grid_of(num_edges)), dim3(BLOCK), 0, stream,
                       other, eid, indices, num_edges);
  return hipGetLastError();
}

hipError_t launch_coo_locality(const int32_t* u, const int32_t* v, int64_t n, int64_t window,
                               int64_t* partial, hipStream_t s) {
  hipLaunchKernelGGL(coo_locality_kernel, dim3(COO_LOCALITY_BLOCKS), dim3(BLOCK), 0, s, u, v, n,
                     window, partial);
  return hipGetLastError();
}

}  // namespace mdgl
