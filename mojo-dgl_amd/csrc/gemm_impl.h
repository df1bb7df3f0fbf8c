// Grouped GEMM on the matrix cores behind segment_mm and gather_mm
// (included once per dtype).
//
//   out[row] = a[row] @ b[g]   for every row of group g.
//
// segment_mm's groups are consecutive row ranges (offsets from seglen);
// gather_mm's are the rows with idx_b == g, found by a stable counting sort
// on the GPU (count per block, scan, ballot-ranked scatter) into `perm`.
//
// Two forward kernels: float32 with K a multiple of 32 up to 128 and rows of
// a on a 16-byte boundary runs on the bf16 matrix cores through exact
// three-way splits (grouped_gemm_split_kernel, described where it is
// defined); every other shape, and float64, takes grouped_gemm_kernel:
//
// Tiles. A workgroup (4 wavefronts, 2 x 2) computes a 128 x 128 output tile
// of one group: 128 rows of the group x 128 columns. Wavefront (wm, wn) owns
// 64 x 64 of it as 4 x 4 blocks of v_mfma_{f32,f64}_16x16x4. The K axis is
// walked in BK-deep stages staged through LDS, double buffered: the next
// stage's global loads are in registers while the current stage multiplies.
// b is first transposed into the workspace (bt[g][n][k], k padded to a
// multiple of BK) so both LDS tiles are k-contiguous and every MFMA operand
// fragment is one 16-byte LDS read: lane l reads 4 consecutive k values
// (k = 4 * (l / 16) + s, s = 0..3) and feeds them to 4 successive MFMAs.
// Rows are padded in LDS so those reads are bank-conflict free.
//
// Arithmetic. Each output element is the sum over k of a * b in the MFMA
// units' order, in the input precision (float32 or float64); the reference
// sums in k order (src/ported.mojo:786-790, 1115-1119), so the two agree to
// rounding.
#pragma once

#include "mdgl_kernels.h"

namespace mdgl {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

template <class T> struct Mfma;
// Both instructions take A[i][k] from lane i + 16k and B[k][j] from lane
// j + 16k. They differ in where output row i lands: the f32 form keeps it in
// lane group i / 4 (register i % 4), the f64 form in lane group i % 4
// (register i / 4). `row(g, r)` is the block row held by lane group g (lanes
// 16g..16g+15) in accumulator register r; the column is the lane mod 16.
template <> struct Mfma<float> {
  using acc_t = f32x4;
  static constexpr int BK = 32;
  static constexpr int PAD = 4;
  __device__ static acc_t step(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ static int row(int g, int r) { return 4 * g + r; }
};
template <> struct Mfma<double> {
  using acc_t = f64x4;
  static constexpr int BK = 16;
  static constexpr int PAD = 2;
  __device__ static acc_t step(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  __device__ static int row(int g, int r) { return g + 4 * r; }
};

constexpr int GBM = 128, GBN = 128;
// Workspace bytes where the block-resident kernels send the stores of rows
// past a group and columns past N, so that every store is issued (see the
// float64 kernel).
constexpr int GEMM_SINK_BYTES = GBN * 8;

template <class T>
struct GemmArgs {
  const T* a;
  const T* bt;  // [R][N][Kp]
  T* out;
  const int32_t* perm;       // null: group rows are contiguous
  const int32_t* group_off;  // R + 1
  const int32_t* tile_ptr;   // R + 1, M tiles per group (prefix)
  int64_t R, K, Kp, N;
  int a_vec;    // rows of a allow 16-byte loads
  int out_vec;  // rows of out allow 16-byte stores
};

// bt[g][n][k] = b[g][k][n], zero for k in [K, Kp); with `given_t` b is
// already [g][n][k] (a product with the blocks' transposes) and is copied.
template <class T>
__global__ __launch_bounds__(BLOCK) void transpose_b_kernel(const T* __restrict__ b,
                                                            T* __restrict__ bt, int64_t R,
                                                            int64_t K, int64_t Kp, int64_t N,
                                                            int given_t) {
  const int64_t total = R * N * Kp;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t k = i % Kp, n = (i / Kp) % N, g = i / (Kp * N);
    if (k >= K) bt[i] = T(0);
    else bt[i] = given_t ? b[(g * N + n) * K + k] : b[(g * K + k) * N + n];
  }
}

template <class T>
__global__ __launch_bounds__(BLOCK) void grouped_gemm_kernel(GemmArgs<T> p) {
  using M = Mfma<T>;
  using acc_t = typename M::acc_t;
  constexpr int BK = M::BK, LD = BK + M::PAD;
  constexpr int EV = 16 / sizeof(T);          // elements per 16-byte load
  constexpr int CPR = BK / EV;                // 16-byte chunks per tile row per stage
  constexpr int RPP = BLOCK / CPR;            // tile rows covered per pass of the block
  constexpr int PASSES = GBM / RPP;           // passes to cover 128 rows
  __shared__ __align__(16) T As[2][GBM][LD];
  __shared__ __align__(16) T Bs[2][GBN][LD];
  __shared__ int rowid_s[GBM];

  const int64_t tile = blockIdx.x;
  const int64_t total = p.tile_ptr[p.R];
  if (tile >= total) return;  // uniform per workgroup
  // group of this tile: last g with tile_ptr[g] <= tile
  int64_t lo = 0, hi = p.R - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (p.tile_ptr[mid] <= tile) lo = mid; else hi = mid - 1;
  }
  const int64_t g = lo;
  const int64_t m0 = p.group_off[g] + (tile - p.tile_ptr[g]) * GBM;
  const int64_t m_end = p.group_off[g + 1];
  const int64_t n0 = (int64_t)blockIdx.y * GBN;
  const int t = threadIdx.x;
  if (t < GBM) {
    const int64_t pos = m0 + t;
    rowid_s[t] = pos < m_end ? (p.perm ? p.perm[pos] : (int32_t)pos) : -1;
  }
  __syncthreads();

  const int lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1;
  const int li = lane & 15, h = lane >> 4;
  const T* bt_g = p.bt + g * p.N * p.Kp;

  // global -> register staging of one stage
  T ra[PASSES][EV], rb[PASSES][EV];
  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int r = q * RPP + t / CPR;
      const int64_t kk = k0 + (t % CPR) * EV;
      const int rid = rowid_s[r];
      if (rid >= 0 && p.a_vec && kk + EV <= p.K) {
        load_vec<T>(p.a + (int64_t)rid * p.K + kk, ra[q]);
      } else {
#pragma unroll
        for (int v = 0; v < EV; ++v)
          ra[q][v] = (rid >= 0 && kk + v < p.K) ? p.a[(int64_t)rid * p.K + kk + v] : T(0);
      }
      const int64_t n = n0 + r;
      if (n < p.N) {
        load_vec<T>(bt_g + n * p.Kp + kk, rb[q]);  // Kp is a multiple of BK: in bounds
      } else {
#pragma unroll
        for (int v = 0; v < EV; ++v) rb[q][v] = T(0);
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int r = q * RPP + t / CPR;
      const int c = (t % CPR) * EV;
      store_vec<T>(&As[buf][r][c], ra[q]);
      store_vec<T>(&Bs[buf][r][c], rb[q]);
    }
  };

  acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = T(0);

  const int64_t nstages = p.Kp / BK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int64_t s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstages) load_stage((s + 1) * BK);
#pragma unroll
    for (int kc = 0; kc < BK; kc += 16) {
      T af[4][4], bf[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const T* pa = &As[buf][wm * 64 + i * 16 + li][kc + 4 * h];
        const T* pb = &Bs[buf][wn * 64 + i * 16 + li][kc + 4 * h];
#pragma unroll
        for (int v = 0; v < 4; v += EV) {
          T tmp[EV];
          load_vec<T>(pa + v, tmp);
#pragma unroll
          for (int e = 0; e < EV; ++e) af[i][v + e] = tmp[e];
          load_vec<T>(pb + v, tmp);
#pragma unroll
          for (int e = 0; e < EV; ++e) bf[i][v + e] = tmp[e];
        }
      }
#pragma unroll
      for (int sstep = 0; sstep < 4; ++sstep)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = M::step(af[i][sstep], bf[j][sstep], acc[i][j]);
    }
    if (s + 1 < nstages) {
      store_stage(buf ^ 1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rl = wm * 64 + i * 16 + M::row(h, r);
      const int rid = rowid_s[rl];
      if (rid < 0) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + wn * 64 + j * 16 + li;
        if (n < p.N) p.out[(int64_t)rid * p.N + n] = acc[i][j][r];
      }
    }
  }
}

// ---------------------------------------------------------------- float32 on bf16 MFMA
// float32 shapes with K a multiple of 32 up to 128 and rows of a on a 16-byte
// boundary (the host checks; other shapes and float64 take
// grouped_gemm_kernel) run on the bf16 matrix cores with float32 accuracy.
//
// Arithmetic. Each float x is cut into three bf16 values without loss,
// x = p0 + p1 + p2: p0 = x rounded to bf16 (to nearest even), p1 = the
// remainder x - p0 (exact in float32) rounded to bf16, p2 = x - p0 - p1,
// which has at most 8 significant bits and so is a bf16. |p1| <= 2^-8 |x| and
// |p2| <= 2^-17 |x|. The product a * b is the sum of the nine ai * bj, each
// exact in float32; the kernel keeps the six above 2^-25 |a b| (a0 b0, a0 b1,
// a1 b0, a1 b1, a0 b2, a2 b0) and v_mfma_f32_32x32x16_bf16 adds them into
// float32 accumulators, smallest first. The three left out sum to at most
// 2^-24 |a b| (one float32 rounding of the product) with either sign, so the
// error stays that of a float32 GEMM: against float64, rows of
// N(0, 1) x N(0, 1/128) data with K = 128 come out with a mean error of
// 1.6e-8 of sum |a b| against 2.0e-8 for v_mfma_f32_32x32x2f32 and for the
// vendor float32 GEMM (maximum 2.9e-7 against 3.3e-7 and 3.9e-7). Six bf16
// MFMAs (6 x 32 cycles) replace eight float32 ones (8 x 64) per 16-deep chunk
// of a 32 x 32 block.
// The fast path takes values that are zero or of magnitude in [2^-50, 2^60):
// there every part and every kept part product is a normal number (nothing
// lost to subnormal flushing) and no part product overflows. Others (inf and
// NaN, which do not split, since inf - inf is NaN and a zero part times an
// infinite one would make NaN where IEEE float gives inf; tiny and huge
// values) send their chunk of a, or every chunk of the group whose b block
// holds one, to v_mfma_f32_32x32x2f32 on the float32 values themselves (b read
// from the caller's array: 64 KB per block, served by L2). inf and NaN then
// propagate as in IEEE arithmetic.
//
// Work mapping. A workgroup (8 wavefronts, one per CU: the group's b block
// held in LDS as three bf16 planes of 128 columns x Kp, 104 KB, loaded once
// per group it meets) walks a contiguous range of 256-row tiles; ranges follow
// the group order, so b changes rarely. Each wavefront owns 32 rows of the
// tile and all 128 columns: four 32 x 32 blocks, so every row of a is read by
// one wavefront only, straight from global memory into registers (no LDS, no
// barrier in the K loop), half a tile ahead of the MFMAs that use it. The K
// axis goes in 16-wide chunks; in chunk c lane (lr, hf) supplies
// a[row lr][16c + 8hf .. +7] (8 consecutive floats of its row: two 16-byte
// loads, split in registers) and b[16c + 8hf .. +7][column lr] (one 16-byte
// LDS read per plane; a 272-byte row stride keeps 16 lanes on distinct
// banks). A tile's results leave after a 4 x 4 transpose in each DPP quad as
// 16-byte stores, eight rows x 128 contiguous bytes per instruction.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int SB_WAVES = 8;
constexpr int SB_TM = 32 * SB_WAVES;     // rows per tile
constexpr int SB_THREADS = 64 * SB_WAVES;
constexpr int SB_KMAX = 128;             // largest padded K held in LDS
constexpr int SB_LD = SB_KMAX + 8;       // bf16 per LDS row (272 bytes)
constexpr int SB_MAX_SLICES = 8;         // splittability flags per group of b
constexpr float SB_HI = 0x1p60f;         // fast-path values: |x| < SB_HI and
constexpr int SB_EMIN = -49;             // x == 0 or frexp exponent >= SB_EMIN

// Within each quad of lanes (s = lane % 4), x[r] = M[r][s] becomes
// x[c] = M[s][c]: two butterfly stages (partner lane s ^ 1, then s ^ 2), each
// moving the elements whose position bit and lane bit differ.
__device__ __forceinline__ int dpp_quad_xor1(int v) {
  return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
}
__device__ __forceinline__ int dpp_quad_xor2(int v) {
  return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ void quad_transpose(float (&x)[4], int s) {
  float t[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    t[r] = __int_as_float(dpp_quad_xor1(__float_as_int(x[r ^ 1])));
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if ((r & 1) != (s & 1)) x[r] = t[r];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    t[r] = __int_as_float(dpp_quad_xor2(__float_as_int(x[r ^ 2])));
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if ((r & 2) != (s & 2)) x[r] = t[r];
}

// Two floats rounded to bf16 (to nearest even), element 0 in the low half.
__device__ __forceinline__ uint32_t bf16_pair(float x0, float x1) {
  const bf16x2 v = {(__bf16)x0, (__bf16)x1};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Whether x takes the bf16 path (see above); zero has frexp exponent 0.
__device__ __forceinline__ bool splits(float x) {
  return __builtin_fabsf(x) < SB_HI && __builtin_amdgcn_frexp_expf(x) >= SB_EMIN;
}

// The three parts of two floats (|x| < 2^127), one bf16 pair per part.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& q0, uint32_t& q1,
                                           uint32_t& q2) {
  q0 = bf16_pair(x0, x1);
  const float r0 = x0 - bf16_lo(q0), r1 = x1 - bf16_hi(q0);
  q1 = bf16_pair(r0, r1);
  q2 = bf16_pair(r0 - bf16_lo(q1), r1 - bf16_hi(q1));
}

// bt3[g][q][n][k] (bf16 bit patterns): part q of b[g][k][n] (of b[g][n][k]
// with `given_t`), zero for k in [K, Kp). Workgroup (g, s) splits slice s of
// group g's N x Kp values and sets flags[g * slices + s] when the slice holds
// a value off the fast path (its parts are left zero: the group's chunks all
// take the float32 path).
static __global__ __launch_bounds__(BLOCK) void split_b_kernel(const float* __restrict__ b,
                                                               uint16_t* __restrict__ bt3,
                                                               int32_t* __restrict__ flags,
                                                               int64_t K, int64_t Kp, int64_t N,
                                                               int given_t, int slices) {
  const int64_t g = blockIdx.x / slices;
  const int s = (int)(blockIdx.x % slices);
  const int64_t per = N * Kp;
  const int64_t lo = per * s / slices, hi = per * (s + 1) / slices;
  uint16_t* o = bt3 + g * 3 * per;
  int bad = 0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += BLOCK) {
    const int64_t k = i % Kp, n = i / Kp;
    float x = 0.f;
    if (k < K) x = given_t ? b[(g * N + n) * K + k] : b[(g * K + k) * N + n];
    uint32_t q0 = 0, q1 = 0, q2 = 0;
    if (splits(x))
      split_pair(x, 0.f, q0, q1, q2);  // x's parts in the low halves
    else
      bad = 1;
    o[i] = (uint16_t)q0;
    o[per + i] = (uint16_t)q1;
    o[2 * per + i] = (uint16_t)q2;
  }
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) flags[blockIdx.x] = bad;
}

template <int NCH, bool GATHER, bool OUTV>
__global__ __launch_bounds__(SB_THREADS, 1) void grouped_gemm_split_kernel(
    GemmArgs<float> p, const uint16_t* __restrict__ bt3, const int32_t* __restrict__ bflags,
    int slices, const float* __restrict__ b, int given_t, int64_t tiles_per_wg,
    const int32_t* __restrict__ tile_ptr, const int32_t* __restrict__ group_off,
    float* __restrict__ sink) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  __shared__ __align__(16) uint16_t Bs[3][GBN][SB_LD];
  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6;
  const int lr = lane & 31, hf = lane >> 5;
  const int s4 = lane & 3, k4 = lr >> 2;
  const int64_t total = tile_ptr[p.R];
  const int64_t first = (int64_t)blockIdx.x * tiles_per_wg;
  const int64_t last = first + tiles_per_wg < total ? first + tiles_per_wg : total;
  if (first >= last) return;  // uniform per workgroup
  const int64_t n0 = (int64_t)blockIdx.y * GBN;

  // Group metadata is read with scalar loads (uniform index, read-only
  // arguments): a vector load here would be waited for with the vector
  // memory counter, i.e. behind every a load and output store in flight.
  auto uget = [](const int32_t* __restrict__ arr, int64_t i) -> int64_t {
    return arr[__builtin_amdgcn_readfirstlane((int)i)];
  };
  auto advance = [&](int64_t gg, int64_t tl) -> int64_t {
    while (uget(tile_ptr, gg + 1) <= tl) ++gg;
    return gg;
  };
  // The row of a behind tile row 32w + lr and whether there is one (rows
  // past the group load row 0 and store to the sink); gather_mm's come
  // through the permutation, requested a tile ahead. As in the float64
  // kernel, the loads and stores of the tile loop are unconditional, so each
  // wait covers only the loads it is for.
  auto row_of = [&](int64_t tl, int64_t gg, bool& ok) -> int32_t {
    const int64_t m0 = uget(group_off, gg) + (tl - uget(tile_ptr, gg)) * SB_TM;
    const int64_t pos = m0 + w * 32 + lr;
    const int64_t end = uget(group_off, gg + 1);
    ok = pos < end;
    if constexpr (GATHER) return p.perm[ok ? pos : end - 1];
    return (int32_t)pos;
  };
  auto base_of = [&](int32_t r, bool ok) -> const float* {
    return p.a + (int64_t)(ok ? r : 0) * p.K + 8 * hf;
  };
  // 8 consecutive floats (two 16-byte loads) from a row of a
  auto load_chunk = [&](const float* q, float (&d)[8]) {
    float x[4], y[4];
    load_global_n<float, 4>(q, x);
    load_global_n<float, 4>(q + 4, y);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[i] = x[i];
      d[4 + i] = y[i];
    }
  };
  // the three parts of b[k .. k + 7][column r] (one 16-byte LDS read each)
  auto lds_parts = [&](int r, int k, u32x4 (&d)[3]) {
#pragma unroll
    for (int q = 0; q < 3; ++q) d[q] = *reinterpret_cast<const u32x4*>(&Bs[q][r][k]);
  };
  int64_t tile = first;
  // group of the first tile: last g with tile_ptr[g] <= tile (uniform)
  int64_t g = 0;
  {
    int64_t lo = 0, hi = p.R - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (uget(tile_ptr, mid) <= tile) lo = mid; else hi = mid - 1;
    }
    g = lo;
  }
  // rows of this tile and of the next one (group g1; past the last tile,
  // this tile's)
  int64_t g1 = g;
  if (tile + 1 < last) g1 = advance(g, tile + 1);
  bool rok, rok1;
  int32_t rid = row_of(tile, g, rok);
  int32_t rid1 = row_of(tile + 1 < last ? tile + 1 : tile, g1, rok1);
  const float* base = base_of(rid, rok);
  // a values in a ring of RS chunks: chunk c lives in af[c % RS] and, once
  // used, its slot takes the chunk RS later (this tile's or the next one's)
  constexpr int RS = NCH >= 4 ? NCH / 2 : NCH;
  float af[RS][8];
#pragma unroll
  for (int c = 0; c < RS; ++c) load_chunk(base + 16 * c, af[c]);
  // waited for here, once: see the float64 kernel
  __builtin_amdgcn_s_waitcnt(0);

  int64_t cur_g = -1;
  bool b_whole = false;  // the group's b block has a value that does not split
  // One tile: its b block (when the group changes), the K loop with the next
  // tile's loads, the results stored.
  auto run_tile = [&]() -> bool {
    if (g != cur_g) {
      __syncthreads();  // every wavefront is done with the previous block
      const int64_t per = p.N * p.Kp;
      const uint16_t* src = bt3 + g * 3 * per;
      constexpr int CPR = NCH * 2;  // 16-byte pieces per row of a part
      for (int c = t; c < 3 * GBN * CPR; c += SB_THREADS) {
        const int q = c / (GBN * CPR), rem = c % (GBN * CPR);
        const int r = rem / CPR, k = (rem % CPR) * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (n0 + r < p.N)
          v = *(const __attribute__((address_space(1))) u32x4*)(src + q * per + (n0 + r) * p.Kp + k);
        *reinterpret_cast<u32x4*>(&Bs[q][r][k]) = v;
      }
      int bad = 0;
      for (int s = 0; s < slices; ++s) bad |= (int)uget(bflags, g * slices + s);
      b_whole = bad != 0;
      __syncthreads();
      cur_g = g;
    }
    const bool has_next = tile + 1 < last;
    const float* base_n = base_of(rid1, rok1);
    // the rows of the tile after the next (past the last tile, the next one's)
    int64_t g2 = g1;
    const int64_t t2 = tile + 2 < last ? tile + 2 : tile + 1;
    if (tile + 2 < last) g2 = advance(g1, t2);
    bool rok2;
    const int32_t rid2 = row_of(t2, g2, rok2);
    f32x16 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      int ok = 1;
#pragma unroll
      for (int s = 0; s < 8; ++s) ok &= splits(af[c % RS][s]) ? 1 : 0;
      if (!b_whole && __builtin_amdgcn_ballot_w64(!ok) == 0) {
        u32x4 A[3];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t q0, q1, q2;
          split_pair(af[c % RS][2 * i], af[c % RS][2 * i + 1], q0, q1, q2);
          A[0][i] = q0;
          A[1][i] = q1;
          A[2][i] = q2;
        }
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          u32x4 B0[3], B1[3];
          lds_parts(64 * jp + lr, 16 * c + 8 * hf, B0);
          lds_parts(64 * jp + 32 + lr, 16 * c + 8 * hf, B1);
          // the wavefront issuing MFMAs goes first while the other one on its
          // SIMD waits on memory or transposes results
          __builtin_amdgcn_s_setprio(1);
          constexpr int ORD[6][2] = {{0, 2}, {2, 0}, {1, 1}, {0, 1}, {1, 0}, {0, 0}};
#pragma unroll
          for (int o = 0; o < 6; ++o) {
            const bf16x8 av = __builtin_bit_cast(bf16x8, A[ORD[o][0]]);
            acc[2 * jp] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                av, __builtin_bit_cast(bf16x8, B0[ORD[o][1]]), acc[2 * jp], 0, 0, 0);
            acc[2 * jp + 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                av, __builtin_bit_cast(bf16x8, B1[ORD[o][1]]), acc[2 * jp + 1], 0, 0, 0);
          }
          __builtin_amdgcn_s_setprio(0);
        }
      } else {
        // float32 MFMAs on b from the caller's array (b[g][k][n], or
        // b[g][n][k] with given_t; 0 past the last column); in step s lane
        // half hf supplies k = 16c + 8hf + s
        const int64_t kb = 16 * c + 8 * hf;
        const int64_t ks = given_t ? 1 : p.N, ns = given_t ? p.K : 1;
        const float* bg = b + g * p.K * p.N + kb * ks;
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          const int64_t na = n0 + 64 * jp + lr, nb = na + 32;
          const float* pa = bg + na * ns;
          const float* pb = bg + nb * ns;
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            const float x = na < p.N ? load_global(pa + s * ks) : 0.f;
            acc[2 * jp] =
                __builtin_amdgcn_mfma_f32_32x32x2f32(af[c % RS][s], x, acc[2 * jp], 0, 0, 0);
            const float y = nb < p.N ? load_global(pb + s * ks) : 0.f;
            acc[2 * jp + 1] =
                __builtin_amdgcn_mfma_f32_32x32x2f32(af[c % RS][s], y, acc[2 * jp + 1], 0, 0, 0);
          }
        }
      }
      // chunk c's values are used: request the chunk RS later (after the
      // last tile, row 0's: loaded, never used)
      if (c + RS < NCH)
        load_chunk(base + 16 * (c + RS), af[c % RS]);
      else
        load_chunk(base_n + 16 * (c + RS - NCH), af[c % RS]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // lane (lr, hf) holds column lr of rows 8q + 4hf + r in acc[j][4q + r];
    // the quad transpose gives lane 4k4 + s4 row 8q + 4hf + s4 at columns
    // 4k4 .. 4k4 + 3. Rows past the group and columns past N go to the sink.
    // (16-byte stores with OUTV, else element by element; one form per
    // kernel: the compiler's wait counts are exact only with a single one)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int32_t orow = __shfl(rok ? rid : -1, 8 * q + 4 * hf + s4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) x[v] = acc[j][4 * q + v];
        quad_transpose(x, s4);
        const int64_t n = n0 + 32 * j + 4 * k4;
        float* o = p.out + (int64_t)(orow >= 0 ? orow : 0) * p.N + n;
        float* sk = sink + 32 * j + 4 * k4;
        if constexpr (OUTV) {
          // N is a multiple of 4: a piece is wholly inside or wholly past N
          store_n<float, 4>(orow >= 0 && n < p.N ? o : sk, x);
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) *(orow >= 0 && n + v < p.N ? o + v : sk + v) = x[v];
        }
      }
    }
    if (!has_next) return false;
    ++tile;
    g = g1;
    g1 = g2;
    rid = rid1;
    rok = rok1;
    rid1 = rid2;
    rok1 = rok2;
    base = base_n;
    return true;
  };
  while (run_tile()) {
  }
}

// ---------------------------------------------------------------- float64
// float64 shapes with K a multiple of 16 up to 128 and a on a 16-byte
// boundary (the host checks; others take grouped_gemm_kernel).
//
// Work mapping. As in the split kernel: one workgroup per CU (NW wavefronts)
// holds the group's b block in LDS (128 columns x Kp, 132 doubles per row:
// with 1,056-byte rows the reads below meet no bank conflict, where 1,040- or
// 1,072-byte rows make every read wait twice as long, as measured), loaded
// once per group it meets, and walks a contiguous range of tiles of
// 16 * RB * NW rows in group order. A wavefront owns 16 * RB rows of a tile
// and all 128 columns (RB x 8 blocks of v_mfma_f64_16x16x4f64), reads its
// rows of a straight from global memory into registers (no LDS, no barrier
// in the K loop), RS chunks of 16 ahead of the MFMAs that use them, wrapping
// into the next tile's rows.
//
// The K axis goes in 16-wide chunks, four MFMA steps each. In chunk c, lane
// (i, q) (i = lane % 16 the block row or column, q = lane / 16) supplies
// k = 16c + 2q + (s & 1) + 8 (s >> 1) in step s: a[row i][16c + 2q .. +1]
// and a[row i][16c + 8 + 2q .. +1], two 16-byte loads that cover 64
// contiguous bytes of the row per instruction, and b[k][column i] from two
// 16-byte LDS reads. The four steps of a chunk cover its 16 k exactly once.
//
// Arithmetic: each output is the sum over k of a * b, in float64, in the
// MFMA units' order (the reference sums in k order: src/ported.mojo:786-790,
// 1115-1119; the two agree to rounding).
constexpr int F64_KMAX = 128;
constexpr int F64_LD = F64_KMAX + 4;  // doubles per LDS row
constexpr int F64_RB = 1, F64_NW = 8;  // the library's shape: 128-row tiles
constexpr int F64_TM = 16 * F64_RB * F64_NW;

template <int NCH, int RB, int NW, bool GATHER>
__global__ __launch_bounds__(64 * NW, 1) void grouped_gemm_f64_kernel(
    GemmArgs<double> p, int64_t tiles_per_wg, const int32_t* __restrict__ tile_ptr,
    const int32_t* __restrict__ group_off, double* __restrict__ sink) {
  constexpr int TM = 16 * RB * NW;
  constexpr int NT = 64 * NW;
  constexpr int CB = GBN / 16;  // column blocks
  __shared__ __align__(16) double Bs[GBN][F64_LD];
  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6;
  const int li = lane & 15, q = lane >> 4;
  const int64_t total = tile_ptr[p.R];
  const int64_t first = (int64_t)blockIdx.x * tiles_per_wg;
  const int64_t last = first + tiles_per_wg < total ? first + tiles_per_wg : total;
  if (first >= last) return;  // uniform per workgroup
  const int64_t n0 = (int64_t)blockIdx.y * GBN;

  // group metadata through scalar loads (uniform index, read-only arguments)
  auto uget = [](const int32_t* __restrict__ arr, int64_t i) -> int64_t {
    return arr[__builtin_amdgcn_readfirstlane((int)i)];
  };
  // the group of tile tl, from the group of an earlier tile
  auto advance = [&](int64_t gg, int64_t tl) -> int64_t {
    while (uget(tile_ptr, gg + 1) <= tl) ++gg;
    return gg;
  };
  // The row of a behind row 16 (RB w + rb) + i of tile tl of group gg, and
  // whether there is one (none past the group: that lane's loads then read
  // row 0 and its stores go to the sink). gather_mm's rows come through the
  // permutation, a vector load that is requested a whole tile before it is
  // needed and not touched until then (its clamped index always valid), so
  // waiting for it does not also wait for the loads and stores issued just
  // before. Every global load and store in the tile loop is unconditional:
  // the compiler counts only those it knows are issued, and a skippable
  // store would make each tile's first wait cover the previous tile's
  // stores.
  auto row_of = [&](int64_t tl, int64_t gg, int rb, bool& ok) -> int32_t {
    const int64_t m0 = uget(group_off, gg) + (tl - uget(tile_ptr, gg)) * TM;
    const int64_t pos = m0 + 16 * (RB * w + rb) + li;
    const int64_t end = uget(group_off, gg + 1);
    ok = pos < end;
    if constexpr (GATHER) return p.perm[ok ? pos : end - 1];
    return (int32_t)pos;
  };
  auto base_of = [&](int32_t r, bool ok) -> const double* {
    return p.a + (int64_t)(ok ? r : 0) * p.K;
  };
  // a[row][16c + 2q .. +1] and a[row][16c + 8 + 2q .. +1] (K = 16 NCH: no
  // piece is past the row; a select of zeros past K would be placed right
  // after the loads by the compiler and wait for them there)
  auto load_chunk = [&](const double* bp, int c, double (&d)[4]) {
    double x[2], y[2];
    load_global_n<double, 2>(bp + 16 * c + 2 * q, x);
    load_global_n<double, 2>(bp + 16 * c + 8 + 2 * q, y);
    d[0] = x[0];
    d[1] = x[1];
    d[2] = y[0];
    d[3] = y[1];
  };

  int64_t tile = first;
  int64_t g = 0;
  {
    int64_t lo = 0, hi = p.R - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (uget(tile_ptr, mid) <= tile) lo = mid; else hi = mid - 1;
    }
    g = lo;
  }
  // rows of this tile (rid, rok) and of the next one (rid1, rok1, group g1;
  // past the last tile, this tile's again)
  int32_t rid[RB], rid1[RB];
  bool rok[RB], rok1[RB];
  int64_t g1 = g;
  if (tile + 1 < last) g1 = advance(g, tile + 1);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    rid[rb] = row_of(tile, g, rb, rok[rb]);
    rid1[rb] = row_of(tile + 1 < last ? tile + 1 : tile, g1, rb, rok1[rb]);
  }
  // a values in a ring of RS chunks: chunk c lives in af[c % RS] and, once
  // used, its slot takes the chunk RS later (this tile's or the next one's);
  // a whole tile ahead for one row block per wavefront, half a tile for more
  constexpr int RS = (RB > 1 && NCH % 2 == 0) ? NCH / 2 : NCH;
  static_assert(NCH % RS == 0, "a tile's chunks fill the ring evenly");
  double af[RS][RB][4];
#pragma unroll
  for (int c = 0; c < RS; ++c)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) load_chunk(base_of(rid[rb], rok[rb]), c, af[c][rb]);
  // Wait for them here, once. Otherwise the wait before each tile's first
  // MFMA is counted for the entry into the loop too (these loads only) and
  // so also waits for most of the previous tile's output stores.
  __builtin_amdgcn_s_waitcnt(0);

  int64_t cur_g = -1;
  auto run_tile = [&]() -> bool {
    if (g != cur_g) {
      __syncthreads();  // every wavefront is done with the previous block
      const double* src = p.bt + g * p.N * p.Kp;
      constexpr int CPR = NCH * 8;  // 16-byte pieces per LDS row
      for (int c = t; c < GBN * CPR; c += NT) {
        const int r = c / CPR, k = (c % CPR) * 2;
        double v[2] = {0.0, 0.0};
        if (n0 + r < p.N) load_global_n<double, 2>(src + (n0 + r) * p.Kp + k, v);
        store_n<double, 2>(&Bs[r][k], v);
      }
      __syncthreads();
      cur_g = g;
    }
    const bool has_next = tile + 1 < last;
    const double* base[RB];
    const double* base_n[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      base[rb] = base_of(rid[rb], rok[rb]);
      base_n[rb] = base_of(rid1[rb], rok1[rb]);
    }
    // the rows of the tile after the next (past the last tile, the next one's)
    int64_t g2 = g1;
    int32_t rid2[RB];
    bool rok2[RB];
    const int64_t t2 = tile + 2 < last ? tile + 2 : tile + 1;
    if (tile + 2 < last) g2 = advance(g1, t2);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) rid2[rb] = row_of(t2, g2, rb, rok2[rb]);

    f64x4 acc[RB][CB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[rb][j][r] = 0.0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // four column blocks at a time: their b values, then the four steps
      // over them (four or more independent accumulators between two MFMAs
      // that share one)
#pragma unroll
      for (int jg = 0; jg < CB; jg += 4) {
        double bv[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const double* bp = &Bs[16 * (jg + j) + li][16 * c + 2 * q];
          double x[2], y[2];
          load_n<double, 2>(bp, x);
          load_n<double, 2>(bp + 8, y);
          bv[j][0] = x[0];
          bv[j][1] = x[1];
          bv[j][2] = y[0];
          bv[j][3] = y[1];
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              acc[rb][jg + j] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                  af[c % RS][rb][s], bv[j][s], acc[rb][jg + j], 0, 0, 0);
      }
      // chunk c's values are used: request the chunk RS later (after the
      // last tile, row 0's: loaded, never used), here and not later, where
      // the scheduler would otherwise sink these loads
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if (c + RS < NCH)
          load_chunk(base[rb], c + RS, af[c % RS][rb]);
        else
          load_chunk(base_n[rb], c + RS - NCH, af[c % RS][rb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // lane (i, q) holds column i of block rows q + 4r in acc[rb][j][r];
    // rows past the group and columns past N go to the sink
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t orow = __shfl(rok[rb] ? rid[rb] : -1, q + 4 * r);
        double* o = p.out + (int64_t)(orow >= 0 ? orow : 0) * p.N + n0 + li;
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          double* d = orow >= 0 && n0 + 16 * j + li < p.N ? o + 16 * j : sink + 16 * j + li;
          *d = acc[rb][j][r];
        }
      }
    }
    if (!has_next) return false;
    ++tile;
    g = g1;
    g1 = g2;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      rid[rb] = rid1[rb];
      rok[rb] = rok1[rb];
      rid1[rb] = rid2[rb];
      rok1[rb] = rok2[rb];
    }
    return true;
  };
  while (run_tile()) {
  }
}

// ---------------------------------------------------------------- grouping
// Exclusive prefixes of the group lengths and of their tile counts
// ceil(len / tm), 1024 groups at a time by one workgroup (a scan in LDS per
// step, the running totals carried in registers). With `first` (bucketing)
// each group's first sorted position is written there too.
constexpr int PLAN_T = 1024;

__device__ __forceinline__ void plan_scan(const int64_t* len,  // may be `first`
                                          int32_t* __restrict__ group_off,
                                          int32_t* __restrict__ tile_ptr, int64_t* first,
                                          int64_t R, int tm) {
  __shared__ int64_t so[PLAN_T], st[PLAN_T];
  const int t = threadIdx.x;
  int64_t carry_o = 0, carry_t = 0;
  for (int64_t base = 0; base < R; base += PLAN_T) {
    const int64_t g = base + t;
    const int64_t l = g < R ? len[g] : 0;
    so[t] = l;
    st[t] = (l + tm - 1) / tm;
    __syncthreads();
    for (int off = 1; off < PLAN_T; off <<= 1) {  // inclusive scan
      const int64_t ao = t >= off ? so[t - off] : 0, at = t >= off ? st[t - off] : 0;
      __syncthreads();
      so[t] += ao;
      st[t] += at;
      __syncthreads();
    }
    if (g < R) {
      const int64_t eo = carry_o + so[t] - l;
      group_off[g] = (int32_t)eo;
      tile_ptr[g] = (int32_t)(carry_t + st[t] - (l + tm - 1) / tm);
      if (first) first[g] = eo;  // len[g] was read above by this thread only
    }
    carry_o += so[PLAN_T - 1];
    carry_t += st[PLAN_T - 1];
    __syncthreads();  // so / st are rewritten by the next step
  }
  if (t == 0) {
    group_off[R] = (int32_t)carry_o;
    tile_ptr[R] = (int32_t)carry_t;
  }
}

// group_off / tile_ptr from segment_mm's lengths (the host checked them).
static __global__ __launch_bounds__(PLAN_T) void seg_plan_kernel(const int64_t* __restrict__ seglen,
                                                          int32_t* __restrict__ group_off,
                                                          int32_t* __restrict__ tile_ptr, int64_t R,
                                                          int tm) {
  plan_scan(seglen, group_off, tile_ptr, nullptr, R, tm);
}

constexpr int SORT_CHUNK = 8192;  // rows per counting-sort workgroup

// counts[b * R + g] = rows of chunk b with idx == g
static __global__ __launch_bounds__(BLOCK) void bucket_count_kernel(const int64_t* __restrict__ idx,
                                                             int32_t* __restrict__ counts,
                                                             int64_t n, int64_t R) {
  extern __shared__ int32_t hist[];
  for (int64_t g = threadIdx.x; g < R; g += BLOCK) hist[g] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * SORT_CHUNK;
  const int64_t hi = lo + SORT_CHUNK < n ? lo + SORT_CHUNK : n;
  for (int64_t i = lo + threadIdx.x; i < hi; i += BLOCK) {
    const int64_t key = idx[i];
    if (key >= 0 && key < R) atomicAdd(&hist[key], 1);  // the host rejects other keys
  }
  __syncthreads();
  for (int64_t g = threadIdx.x; g < R; g += BLOCK) counts[blockIdx.x * R + g] = hist[g];
}

// Per group g (one workgroup each): counts[b * R + g] over the chunks b
// becomes the exclusive prefix (the group-local position of chunk b's first
// row of group g); the group's total goes to totals[g]. 256 threads take
// contiguous spans of chunks, their span sums are scanned in LDS.
static __global__ __launch_bounds__(BLOCK) void bucket_colscan_kernel(int32_t* __restrict__ counts,
                                                               int64_t* __restrict__ totals,
                                                               int64_t nblocks, int64_t R) {
  __shared__ int64_t part[BLOCK];
  const int64_t g = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t span = (nblocks + BLOCK - 1) / BLOCK;
  const int64_t lo = t * span < nblocks ? t * span : nblocks;
  const int64_t hi = lo + span < nblocks ? lo + span : nblocks;
  int64_t s = 0;
  for (int64_t b = lo; b < hi; ++b) s += counts[b * R + g];
  part[t] = s;
  __syncthreads();
  for (int off = 1; off < BLOCK; off <<= 1) {
    const int64_t add = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += add;
    __syncthreads();
  }
  int64_t run = t > 0 ? part[t - 1] : 0;
  for (int64_t b = lo; b < hi; ++b) {
    const int32_t c = counts[b * R + g];
    counts[b * R + g] = (int32_t)run;
    run += c;
  }
  if (t == BLOCK - 1) totals[g] = part[BLOCK - 1];
}

// group_off / tile_ptr from the group totals, and the totals turned into
// each group's first sorted position.
static __global__ __launch_bounds__(PLAN_T) void bucket_plan_kernel(int64_t* __restrict__ totals,
                                                             int32_t* __restrict__ group_off,
                                                             int32_t* __restrict__ tile_ptr,
                                                             int64_t R, int tm) {
  plan_scan(totals, group_off, tile_ptr, totals, R, tm);
}

// perm[sorted position] = row, stable: rows of a group keep their order.
// Each workgroup walks its chunk 256 rows at a time; inside a wavefront a
// row's rank among equal keys comes from ballots over the key bits, and the
// four wavefronts are ordered through per-wavefront counts in LDS.
static __global__ __launch_bounds__(BLOCK) void bucket_scatter_kernel(const int64_t* __restrict__ idx,
                                                               const int32_t* __restrict__ starts,
                                                               const int64_t* __restrict__ gstart,
                                                               int32_t* __restrict__ perm,
                                                               int64_t n, int64_t R, int bits) {
  extern __shared__ int32_t sm[];
  int32_t* cursor = sm;          // R: next position per group
  int32_t* wcount = sm + R;      // 4 x R: rows per group in each wavefront of this pass
  for (int64_t g = threadIdx.x; g < R; g += BLOCK)
    cursor[g] = (int32_t)(gstart[g] + starts[blockIdx.x * R + g]);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t lo = (int64_t)blockIdx.x * SORT_CHUNK;
  const int64_t hi = lo + SORT_CHUNK < n ? lo + SORT_CHUNK : n;
  __syncthreads();
  for (int64_t base = lo; base < hi; base += BLOCK) {
    for (int64_t g = threadIdx.x; g < 4 * R; g += BLOCK) wcount[g] = 0;
    __syncthreads();
    const int64_t i = base + threadIdx.x;
    int64_t key = i < hi ? idx[i] : -1;
    const bool ok = key >= 0 && key < R;
    if (!ok) key = 0;
    uint64_t same = __ballot(ok);
    for (int bit = 0; bit < bits; ++bit) {
      const uint64_t ones = __ballot(ok && ((key >> bit) & 1));
      same &= ((key >> bit) & 1) ? ones : ~ones;  // lanes whose key agrees on this bit
    }
    const uint64_t below = lane ? (~uint64_t(0) >> (64 - lane)) : 0;
    const int rank = __popcll(same & below);
    const int cnt = __popcll(same);
    if (ok && rank == 0) wcount[w * R + key] = cnt;
    __syncthreads();
    if (ok) {
      int32_t pos = cursor[key] + rank;
      for (int q = 0; q < w; ++q) pos += wcount[q * R + key];
      perm[pos] = (int32_t)i;
    }
    __syncthreads();
    for (int64_t g = threadIdx.x; g < R; g += BLOCK)
      cursor[g] += wcount[g] + wcount[R + g] + wcount[2 * R + g] + wcount[3 * R + g];
    __syncthreads();
  }
}

}  // namespace mdgl


namespace mdgl {

inline int64_t ws_align(int64_t b) { return ((b + 255) / 256) * 256; }

template <class T>
inline int64_t gemm_kp(int64_t K) {
  const int64_t bk = Mfma<T>::BK;
  const int64_t kp = ((K + bk - 1) / bk) * bk;
  return kp < bk ? bk : kp;
}

// Workspace of the grouping: group_off, tile_ptr and, to gather, the
// per-chunk counts, the row permutation and the group totals.
inline int64_t plan_workspace_bytes(int64_t n, int64_t R, bool gather) {
  int64_t b = 2 * ws_align((R + 1) * 4);
  if (gather) {
    const int64_t nb = (n + SORT_CHUNK - 1) / SORT_CHUNK;
    b += ws_align(nb * R * 4) + ws_align(n * 4) + ws_align(R * 8);
  }
  return b;
}

// The groups of rows: group_off[g] (first row position of group g),
// tile_ptr[g] (tiles of `tm` rows before group g) and, to gather, perm
// (row of each sorted position; null for segment_mm's consecutive groups).
inline hipError_t plan_groups(const int64_t* idx_b, const int64_t* seglen, int64_t n, int64_t R,
                              int tm, bool gather, char* w, int32_t** group_off,
                              int32_t** tile_ptr, int32_t** perm, hipStream_t s) {
  *group_off = reinterpret_cast<int32_t*>(w);
  w += ws_align((R + 1) * 4);
  *tile_ptr = reinterpret_cast<int32_t*>(w);
  w += ws_align((R + 1) * 4);
  *perm = nullptr;
  if (gather) {
    const int64_t nb = (n + SORT_CHUNK - 1) / SORT_CHUNK;
    int32_t* counts = reinterpret_cast<int32_t*>(w);
    w += ws_align(nb * R * 4);
    *perm = reinterpret_cast<int32_t*>(w);
    w += ws_align(n * 4);
    int64_t* totals = reinterpret_cast<int64_t*>(w);
    int bits = 0;
    while ((int64_t(1) << bits) < R) ++bits;
    hipLaunchKernelGGL(bucket_count_kernel, dim3((unsigned)nb), dim3(BLOCK), (size_t)(R * 4), s,
                       idx_b, counts, n, R);
    hipLaunchKernelGGL(bucket_colscan_kernel, dim3((unsigned)R), dim3(BLOCK), 0, s, counts,
                       totals, nb, R);
    hipLaunchKernelGGL(bucket_plan_kernel, dim3(1), dim3(PLAN_T), 0, s, totals, *group_off,
                       *tile_ptr, R, tm);
    hipLaunchKernelGGL(bucket_scatter_kernel, dim3((unsigned)nb), dim3(BLOCK),
                       (size_t)(5 * R * 4), s, idx_b, counts, totals, *perm, n, R, bits);
  } else {
    hipLaunchKernelGGL(seg_plan_kernel, dim3(1), dim3(PLAN_T), 0, s, seglen, *group_off, *tile_ptr,
                       R, tm);
  }
  return hipGetLastError();
}

// Slices of a group's b block that the split kernel flags separately: as
// many as keep a slice at 2,048 values or more, at most SB_MAX_SLICES.
inline int split_slices(int64_t N, int64_t Kp) {
  int64_t s = N * Kp / 2048;
  return s < 1 ? 1 : (s > SB_MAX_SLICES ? SB_MAX_SLICES : (int)s);
}

// Bytes of the b region: bt (float32 / float64 transposed) or, for float32,
// the three bf16 planes (6 bytes per value) and their finiteness flags; then
// the store sink of the block-resident kernels.
template <class T>
int64_t b_region_bytes(int64_t K, int64_t N, int64_t R) {
  const int64_t v = R * N * gemm_kp<T>(K);
  const int64_t sink = ws_align(GEMM_SINK_BYTES);
  if (sizeof(T) == 4) return ws_align(v * 6) + ws_align(R * SB_MAX_SLICES * 4) + sink;
  return ws_align(v * (int64_t)sizeof(T)) + sink;
}

// Workspace of one grouped GEMM: the b region, then the grouping.
template <class T>
int64_t grouped_workspace_bytes(int64_t n, int64_t K, int64_t N, int64_t R, bool gather) {
  return b_region_bytes<T>(K, N, R) + plan_workspace_bytes(n, R, gather);
}

template <class T>
hipError_t launch_grouped(const GemmLaunch& L, bool gather) {
  if (L.n <= 0 || L.N <= 0 || L.R <= 0) return hipSuccess;
  const int64_t Kp = gemm_kp<T>(L.K);
  constexpr int EVH = 16 / sizeof(T);
  const bool split = sizeof(T) == 4 && Kp <= SB_KMAX && Kp == L.K &&
                        reinterpret_cast<uintptr_t>(L.a) % 16 == 0 && L.K % EVH == 0;
  const bool f64 = sizeof(T) == 8 && Kp <= F64_KMAX && Kp == L.K && aligned16(L.a);
  const int tm = split ? SB_TM : (f64 ? F64_TM : GBM);
  char* w = static_cast<char*>(L.workspace);
  T* bt = reinterpret_cast<T*>(w);
  const int64_t vals = L.R * L.N * Kp;
  uint16_t* bt3 = reinterpret_cast<uint16_t*>(w);
  int32_t* bflags = reinterpret_cast<int32_t*>(w + ws_align(vals * 6));
  const int slices = split_slices(L.N, Kp);
  w += b_region_bytes<T>(L.K, L.N, L.R);
  void* sink = w - ws_align(GEMM_SINK_BYTES);

  if (split) {
    hipLaunchKernelGGL(split_b_kernel, dim3((unsigned)(L.R * slices)), dim3(BLOCK), 0, L.stream,
                       static_cast<const float*>(L.b), bt3, bflags, L.K, Kp, L.N, L.trans_b,
                       slices);
  } else {
    int64_t tb = (vals + BLOCK - 1) / BLOCK;
    if (tb > 65536) tb = 65536;
    hipLaunchKernelGGL((transpose_b_kernel<T>), dim3((unsigned)tb), dim3(BLOCK), 0, L.stream,
                       static_cast<const T*>(L.b), bt, L.R, L.K, Kp, L.N, L.trans_b);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;

  int32_t *group_off, *tile_ptr, *perm;
  e = plan_groups(L.idx_b, L.seglen, L.n, L.R, tm, gather, w, &group_off, &tile_ptr, &perm,
                  L.stream);
  if (e != hipSuccess) return e;

  GemmArgs<T> a;
  a.a = static_cast<const T*>(L.a);
  a.bt = bt;
  a.out = static_cast<T*>(L.out);
  a.perm = perm;
  a.group_off = group_off;
  a.tile_ptr = tile_ptr;
  a.R = L.R;
  a.K = L.K;
  a.Kp = Kp;
  a.N = L.N;
  constexpr int EV = 16 / sizeof(T);
  a.a_vec = (L.K % EV == 0) && (reinterpret_cast<uintptr_t>(L.a) % 16 == 0);
  a.out_vec = (L.N % EV == 0) && (reinterpret_cast<uintptr_t>(L.out) % 16 == 0);
  const int64_t nt = (L.N + GBN - 1) / GBN;
  if constexpr (sizeof(T) == 4) {
    if (split) {
      // upper bound of the tile count; one workgroup per CU (its LDS planes),
      // each a contiguous range of tiles
      const int64_t mt = (L.n + SB_TM - 1) / SB_TM + L.R;
      int64_t wgs = 256 / nt;
      if (wgs < 1) wgs = 1;
      if (wgs > mt) wgs = mt;
      const int64_t per = (mt + wgs - 1) / wgs;
      const dim3 grid((unsigned)wgs, (unsigned)nt), block(SB_THREADS);
      const float* bsrc = static_cast<const float*>(L.b);
      float* fsink = static_cast<float*>(sink);
#define MDGL_SPLIT_LAUNCH(C, G, V)                                                              \
  hipLaunchKernelGGL((grouped_gemm_split_kernel<C, G, V>), grid, block, 0, L.stream, a, bt3, \
                     bflags, slices, bsrc, L.trans_b, per, a.tile_ptr, a.group_off, fsink)
#define MDGL_SPLIT_CASE(C)                                       \
  case C:                                                      \
    if (gather) {                                              \
      if (a.out_vec) MDGL_SPLIT_LAUNCH(C, true, true);         \
      else MDGL_SPLIT_LAUNCH(C, true, false);                  \
    } else {                                                   \
      if (a.out_vec) MDGL_SPLIT_LAUNCH(C, false, true);        \
      else MDGL_SPLIT_LAUNCH(C, false, false);                 \
    }                                                          \
    break;
      switch (Kp / 16) {
        MDGL_SPLIT_CASE(2) MDGL_SPLIT_CASE(4) MDGL_SPLIT_CASE(6) MDGL_SPLIT_CASE(8)
        default: return hipErrorInvalidValue;
      }
#undef MDGL_SPLIT_CASE
#undef MDGL_SPLIT_LAUNCH
      return hipGetLastError();
    }
  }
  if constexpr (sizeof(T) == 8) {
    if (f64) {
      // as for the split kernel: one workgroup per CU (its LDS block), each a
      // contiguous range of tiles
      const int64_t mt = (L.n + F64_TM - 1) / F64_TM + L.R;
      int64_t wgs = 256 / nt;
      if (wgs < 1) wgs = 1;
      if (wgs > mt) wgs = mt;
      const int64_t per = (mt + wgs - 1) / wgs;
      const dim3 grid((unsigned)wgs, (unsigned)nt), block(64 * F64_NW);
#define MDGL_F64_CASE(C)                                                                     \
  case C:                                                                                    \
    if (gather)                                                                              \
      hipLaunchKernelGGL((grouped_gemm_f64_kernel<C, F64_RB, F64_NW, true>), grid, block, 0,  \
                         L.stream, a, per, a.tile_ptr, a.group_off, static_cast<double*>(sink)); \
    else                                                                                     \
      hipLaunchKernelGGL((grouped_gemm_f64_kernel<C, F64_RB, F64_NW, false>), grid, block, 0, \
                         L.stream, a, per, a.tile_ptr, a.group_off, static_cast<double*>(sink)); \
    break;
      switch (Kp / 16) {
        MDGL_F64_CASE(1) MDGL_F64_CASE(2) MDGL_F64_CASE(3) MDGL_F64_CASE(4)
        MDGL_F64_CASE(5) MDGL_F64_CASE(6) MDGL_F64_CASE(7) MDGL_F64_CASE(8)
        default: return hipErrorInvalidValue;
      }
#undef MDGL_F64_CASE
      return hipGetLastError();
    }
  }
  const int64_t mt = (L.n + GBM - 1) / GBM + L.R;
  hipLaunchKernelGGL((grouped_gemm_kernel<T>), dim3((unsigned)mt, (unsigned)nt), dim3(BLOCK), 0,
                     L.stream, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- gradient of b
// db[g] = sum over the rows of group g of a[row]^T grad[row] (D1 x D2 per
// group). A group's rows are cut into chunks of `ch` rows; a workgroup (4
// wavefronts, 2 x 2, each 64 x 64 of the tile as 4 x 4 MFMA blocks) forms the
// 128 x 128 tile blockIdx.y of one chunk's product. The rows are the
// contracted axis, walked BK at a time through row-major LDS tiles (double
// buffered like the forward kernel; BK rows per stage, 16 when the rows come
// through gather_mm's permutation): lane l feeds a[row k0 + l / 16][m0 + l %
// 16] as A^T and grad[row k0 + l / 16][n0 + l % 16] as B; a row stride of 144
// elements puts the four rows one 64-lane read touches in distinct banks.
// Chunk products go to partials that tn_fold_kernel adds per group in chunk
// order, so db is the same on every run.
template <class T>
struct TnArgs {
  const T* a;
  const T* g;
  T* part;                   // [chunk][D1][D2]
  const int32_t* perm;       // null: group rows are contiguous
  const int32_t* group_off;  // R + 1
  const int32_t* chunk_ptr;  // R + 1, chunks per group (prefix)
  int64_t R, D1, D2, ch;
  int a_vec, g_vec, tiles_n;
};

template <class T, int BK, bool VECT, bool GATHER>
__global__ __launch_bounds__(BLOCK) void grouped_tn_kernel(TnArgs<T> p) {
  using M = Mfma<T>;
  using acc_t = typename M::acc_t;
  constexpr int LD = GBM + 16;
  constexpr int EV = 16 / sizeof(T);   // elements per 16-byte load
  constexpr int CPR = GBM / EV;        // 16-byte chunks per 128-wide tile row
  constexpr int RPP = BLOCK / CPR;     // tile rows per pass of the block
  constexpr int PASSES = BK / RPP;
  __shared__ __align__(16) T As[2][BK][LD];
  __shared__ __align__(16) T Bs[2][BK][LD];

  const int64_t c = blockIdx.x;
  if (c >= p.chunk_ptr[p.R]) return;  // uniform per workgroup
  int64_t lo = 0, hi = p.R - 1;       // group: last g with chunk_ptr[g] <= c
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (p.chunk_ptr[mid] <= c) lo = mid; else hi = mid - 1;
  }
  const int64_t grp = lo;
  const int64_t r0 = p.group_off[grp] + (c - p.chunk_ptr[grp]) * p.ch;
  const int64_t g_end = p.group_off[grp + 1];
  const int64_t r_end = r0 + p.ch < g_end ? r0 + p.ch : g_end;
  const int64_t m0 = (int64_t)(blockIdx.y / p.tiles_n) * GBM;
  const int64_t n0 = (int64_t)(blockIdx.y % p.tiles_n) * GBN;
  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6, wm = w >> 1, wn = w & 1;
  const int li = lane & 15, h = lane >> 4;

  T ra[PASSES][EV], rb[PASSES][EV];
  // gather_mm's rows of a stage come through the permutation: they are
  // requested one stage ahead (an unconditional load of a clamped index; the
  // row test is applied where they are used), so no stage waits for them
  auto stage_rows = [&](int64_t k0, int32_t (&rid)[PASSES]) {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int64_t pos = k0 + q * RPP + t / CPR;
      if constexpr (GATHER) rid[q] = p.perm[pos < r_end ? pos : r_end - 1];
      else rid[q] = 0;
    }
  };
  // Each lane's 16-byte pieces of a stage (VECT: both operands' rows allow
  // them): rows past the chunk and pieces past the width load row 0 /
  // column 0 and are zeroed when the stage is written to LDS, at the end of
  // the stage (a test right after a load would wait for the load there);
  // otherwise element by element. The form is fixed at compile time: chosen
  // at run time, the compiler merged both into element loads.
  bool oka[PASSES], okb[PASSES];
  auto load_stage = [&](int64_t k0, const int32_t (&rids)[PASSES]) {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int r = q * RPP + t / CPR;
      const int col = (t % CPR) * EV;
      const int64_t pos = k0 + r;
      const bool ok = pos < r_end;
      const int64_t rid = ok ? (GATHER ? (int64_t)rids[q] : pos) : 0;
      const int64_t ca = m0 + col, cb = n0 + col;
      if constexpr (VECT) {
        oka[q] = ok && ca < p.D1;  // D1 and D2 are multiples of EV
        okb[q] = ok && cb < p.D2;
        load_vec<T>(p.a + rid * p.D1 + (ca < p.D1 ? ca : 0), ra[q]);
        load_vec<T>(p.g + rid * p.D2 + (cb < p.D2 ? cb : 0), rb[q]);
      } else {
        oka[q] = okb[q] = true;
#pragma unroll
        for (int v = 0; v < EV; ++v) {
          ra[q][v] = (ok && ca + v < p.D1) ? p.a[rid * p.D1 + ca + v] : T(0);
          rb[q][v] = (ok && cb + v < p.D2) ? p.g[rid * p.D2 + cb + v] : T(0);
        }
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int r = q * RPP + t / CPR;
      const int col = (t % CPR) * EV;
      T xa[EV], xb[EV];
#pragma unroll
      for (int v = 0; v < EV; ++v) {
        xa[v] = oka[q] ? ra[q][v] : T(0);
        xb[v] = okb[q] ? rb[q][v] : T(0);
      }
      store_vec<T>(&As[buf][r][col], xa);
      store_vec<T>(&Bs[buf][r][col], xb);
    }
  };

  acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = T(0);

  const int64_t nstages = (r_end - r0 + BK - 1) / BK;  // a chunk holds at least one row
  int32_t rid_a[PASSES], rid_b[PASSES];
  stage_rows(r0, rid_a);
  load_stage(r0, rid_a);
  store_stage(0);
  stage_rows(r0 + BK, rid_a);  // the next stage's rows
  __syncthreads();
  for (int64_t s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstages) load_stage(r0 + (s + 1) * BK, rid_a);
    stage_rows(r0 + (s + 2) * BK, rid_b);
#pragma unroll
    for (int q = 0; q < PASSES; ++q) rid_a[q] = rid_b[q];
    __builtin_amdgcn_s_setprio(1);  // MFMA issue first (as in the forward kernel)
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      T af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        af[i] = As[buf][kk + h][wm * 64 + i * 16 + li];
        bf[i] = Bs[buf][kk + h][wn * 64 + i * 16 + li];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = M::step(af[i], bf[j], acc[i][j]);
    }
    __builtin_amdgcn_s_setprio(0);
    if (s + 1 < nstages) {
      store_stage(buf ^ 1);
      __syncthreads();
    }
  }

  T* out = p.part + c * p.D1 * p.D2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t d1 = m0 + wm * 64 + i * 16 + M::row(h, r);
      if (d1 >= p.D1) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t d2 = n0 + wn * 64 + j * 16 + li;
        if (d2 < p.D2) out[d1 * p.D2 + d2] = acc[i][j][r];
      }
    }
  }
}

// db[g][e] = sum of part[c][e] over g's chunks in order (0 for an empty group).
template <class T>
__global__ __launch_bounds__(BLOCK) void tn_fold_kernel(const T* __restrict__ part,
                                                        const int32_t* __restrict__ chunk_ptr,
                                                        T* __restrict__ db, int64_t R, int64_t E) {
  const int64_t total = R * E;
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * BLOCK) {
    const int64_t g = i / E, e = i - g * E;
    T acc = T(0);
    for (int64_t c = chunk_ptr[g]; c < chunk_ptr[g + 1]; ++c) acc += part[c * E + e];
    db[i] = acc;
  }
}

constexpr int64_t TN_CH = 4096;                 // rows per chunk, at least
constexpr int64_t TN_PART_BYTES = 256ll << 20;  // partials kept below this when rows allow

// Rows per chunk: TN_CH, doubled until the partials of the chunks (at most
// n / ch + R of them) fit TN_PART_BYTES, and at most n (n < 2**31).
inline int64_t tn_chunk_rows(int64_t n, int64_t D1, int64_t D2, int64_t R, int64_t es) {
  int64_t ch = TN_CH;
  while (ch < n && ((n + ch - 1) / ch + R) * D1 * D2 * es > TN_PART_BYTES) ch *= 2;
  return ch < n ? ch : (n > 0 ? n : 1);
}

template <class T>
int64_t grouped_grad_workspace_bytes(int64_t n, int64_t D1, int64_t D2, int64_t R, bool gather) {
  const int64_t es = sizeof(T);
  const int64_t ch = tn_chunk_rows(n, D1, D2, R, es);
  const int64_t chunks = (n + ch - 1) / ch + R;
  // da's grouped GEMM (K = D2, N = D1), then db's grouping and partials
  return grouped_workspace_bytes<T>(n, D2, D1, R, gather) + plan_workspace_bytes(n, R, gather) +
         ws_align(chunks * D1 * D2 * es);
}

template <class T>
hipError_t launch_grouped_grad(const GemmGradLaunch& L, bool gather) {
  if (L.n <= 0 || L.R <= 0 || L.D1 <= 0 || L.D2 <= 0) return hipSuccess;
  char* w = static_cast<char*>(L.workspace);
  if (L.da) {
    GemmLaunch g{};
    g.a = L.grad;
    g.b = L.b;
    g.out = L.da;
    g.idx_b = L.idx_b;
    g.seglen = L.seglen;
    g.n = L.n;
    g.K = L.D2;
    g.N = L.D1;
    g.R = L.R;
    g.workspace = w;
    g.stream = L.stream;
    g.trans_b = 1;
    hipError_t e = launch_grouped<T>(g, gather);
    if (e != hipSuccess) return e;
  }
  w += grouped_workspace_bytes<T>(L.n, L.D2, L.D1, L.R, gather);
  if (!L.db) return hipSuccess;
  const int64_t ch = tn_chunk_rows(L.n, L.D1, L.D2, L.R, sizeof(T));
  const int64_t max_chunks = (L.n + ch - 1) / ch + L.R;
  int32_t *group_off, *chunk_ptr, *perm;
  hipError_t e = plan_groups(L.idx_b, L.seglen, L.n, L.R, (int)ch, gather, w, &group_off,
                             &chunk_ptr, &perm, L.stream);
  if (e != hipSuccess) return e;
  w += plan_workspace_bytes(L.n, L.R, gather);
  TnArgs<T> a;
  a.a = static_cast<const T*>(L.a);
  a.g = static_cast<const T*>(L.grad);
  a.part = reinterpret_cast<T*>(w);
  a.perm = perm;
  a.group_off = group_off;
  a.chunk_ptr = chunk_ptr;
  a.R = L.R;
  a.D1 = L.D1;
  a.D2 = L.D2;
  a.ch = ch;
  constexpr int EV = 16 / sizeof(T);
  a.a_vec = (L.D1 % EV == 0) && (reinterpret_cast<uintptr_t>(L.a) % 16 == 0);
  a.g_vec = (L.D2 % EV == 0) && (reinterpret_cast<uintptr_t>(L.grad) % 16 == 0);
  const int64_t tiles_m = (L.D1 + GBM - 1) / GBM;
  a.tiles_n = (int)((L.D2 + GBN - 1) / GBN);
  // rows gathered through the permutation wait longer: shallower stages,
  // half the LDS, twice the workgroups per CU to cover them
  const dim3 grid((unsigned)max_chunks, (unsigned)(tiles_m * a.tiles_n));
  const bool vect = a.a_vec && a.g_vec;
  if (perm && vect)
    hipLaunchKernelGGL((grouped_tn_kernel<T, 16, true, true>), grid, dim3(BLOCK), 0, L.stream, a);
  else if (perm)
    hipLaunchKernelGGL((grouped_tn_kernel<T, 16, false, true>), grid, dim3(BLOCK), 0, L.stream,
                       a);
  else if (vect)
    hipLaunchKernelGGL((grouped_tn_kernel<T, Mfma<T>::BK, true, false>), grid, dim3(BLOCK), 0,
                       L.stream, a);
  else
    hipLaunchKernelGGL((grouped_tn_kernel<T, Mfma<T>::BK, false, false>), grid, dim3(BLOCK), 0,
                       L.stream, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t E = L.D1 * L.D2;
  int64_t fb = (L.R * E + BLOCK - 1) / BLOCK;
  if (fb > 65536) fb = 65536;
  hipLaunchKernelGGL((tn_fold_kernel<T>), dim3((unsigned)fb), dim3(BLOCK), 0, L.stream, a.part,
                     chunk_ptr, static_cast<T*>(L.db), L.R, E);
  return hipGetLastError();
}

}  // namespace mdgl

#define MDGL_INSTANTIATE_GEMM(T)                                                               \
  template int64_t mdgl::grouped_workspace_bytes<T>(int64_t, int64_t, int64_t, int64_t, bool); \
  template hipError_t mdgl::launch_grouped<T>(const mdgl::GemmLaunch&, bool);                  \
  template int64_t mdgl::grouped_grad_workspace_bytes<T>(int64_t, int64_t, int64_t, int64_t,   \
                                                         bool);                                 \
  template hipError_t mdgl::launch_grouped_grad<T>(const mdgl::GemmGradLaunch&, bool);
