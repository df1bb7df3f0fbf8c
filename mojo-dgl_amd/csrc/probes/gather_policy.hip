// Measurement probe (not part of the library): 32-byte row gathers with each
// load cache policy (buffer loads, aux bits sc0 = 1, nt = 2, sc1 = 16, and a
// plain global load), the gather patterns of the GAT step:
//   table A: (2.5M, 8) float32 (80 MB), index = 60M random node ids
//   table B: (60M, 8) float32 (1.92 GB), index = a random permutation of 60M
// out[i] = table[idx[i]] (32 bytes, written coalesced). Median of 10 timed
// launches, each after a 512 MB write that flushes L2 and MALL.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#define CHECK(x) do { hipError_t err_ = (x); if (err_ != hipSuccess) { \
  fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(err_)); exit(1); } } while (0)

constexpr int U = 4;  // rows in flight per lane pair

template <int AUX>
__global__ __launch_bounds__(256) void gather_buf(const float* __restrict__ table, int64_t rows,
                                                  const int* __restrict__ idx, int64_t n,
                                                  float4* __restrict__ out) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      (void*)table, 0, (int)(rows * 32 > 0x7fffffff ? 0x7fffffff : rows * 32), 0x00020000);
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int half = t & 1;
  const int64_t r0 = (t >> 1) * U;  // this lane pair's first row
  int id[U];
#pragma unroll
  for (int u = 0; u < U; ++u) id[u] = idx[r0 + u < n ? r0 + u : n - 1];
  float4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const unsigned off = (unsigned)id[u] * 32u + half * 16u;
    auto x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    static_assert(sizeof(x) == 16, "16-byte load");
    __builtin_memcpy(&v[u], &x, 16);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) out[(r0 + u) * 2 + half] = v[u];  // out is padded to the grid
}

__global__ __launch_bounds__(256) void gather_glb(const float* __restrict__ table, int64_t rows,
                                                  const int* __restrict__ idx, int64_t n,
                                                  float4* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int half = t & 1;
  const int64_t r0 = (t >> 1) * U;
  int id[U];
#pragma unroll
  for (int u = 0; u < U; ++u) id[u] = idx[r0 + u < n ? r0 + u : n - 1];
  float4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    v[u] = reinterpret_cast<const float4*>(table)[(int64_t)id[u] * 2 + half];
#pragma unroll
  for (int u = 0; u < U; ++u) out[(r0 + u) * 2 + half] = v[u];  // out is padded to the grid
}

__global__ void flush_kernel(float4* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = make_float4(1.f, 2.f, 3.f, 4.f);
}

typedef void (*Kern)(const float*, int64_t, const int*, int64_t, float4*);

int main() {
  const int64_t n = 60000000;
  const int64_t rowsA = 2500000, rowsB = 60000000;
  float *tab;
  int *idxA, *idxB;
  float4 *out, *ref, *flush;
  const int64_t flush_n = (512ll << 20) / 16;
  CHECK(hipMalloc(&tab, rowsB * 32));
  CHECK(hipMalloc(&idxA, n * 4));
  CHECK(hipMalloc(&idxB, n * 4));
  const int64_t threads = (n + U - 1) / U * 2;
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  const int64_t out_rows = (int64_t)blocks * 128 * U;  // every lane pair of the grid stores U rows
  CHECK(hipMalloc(&out, out_rows * 32));
  CHECK(hipMalloc(&ref, out_rows * 32));
  CHECK(hipMalloc(&flush, flush_n * 16));
  {
    std::vector<float> h(rowsB * 8);
    for (int64_t i = 0; i < rowsB * 8; ++i) h[i] = (float)(i % 1000003);
    CHECK(hipMemcpy(tab, h.data(), rowsB * 32, hipMemcpyHostToDevice));
    std::mt19937_64 g(7);
    std::vector<int> a(n), b(n);
    for (int64_t i = 0; i < n; ++i) a[i] = (int)(g() % rowsA);
    for (int64_t i = 0; i < n; ++i) b[i] = (int)i;
    std::shuffle(b.begin(), b.end(), g);
    for (int64_t i = 0; i < n; ++i) {
      if (a[i] < 0 || a[i] >= rowsA || b[i] < 0 || b[i] >= rowsB) { fprintf(stderr, "bad idx\n"); return 1; }
    }
    CHECK(hipMemcpy(idxA, a.data(), n * 4, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(idxB, b.data(), n * 4, hipMemcpyHostToDevice));
  }
  const char* names[] = {"global", "buf", "buf_sc0", "buf_nt", "buf_sc0_nt", "buf_sc1",
                         "buf_sc0_sc1", "buf_nt_sc1", "buf_sc0_nt_sc1"};
  Kern ks[] = {gather_glb, gather_buf<0>, gather_buf<1>, gather_buf<2>, gather_buf<3>,
               gather_buf<16>, gather_buf<17>, gather_buf<18>, gather_buf<19>};
  hipEvent_t s, e;
  CHECK(hipEventCreate(&s));
  CHECK(hipEventCreate(&e));
  for (int tb = 0; tb < 2; ++tb) {
    const int* idx = tb ? idxB : idxA;
    const int64_t rows = tb ? rowsB : rowsA;
    hipLaunchKernelGGL(gather_glb, dim3(blocks), dim3(256), 0, 0, tab, rows, idx, n, ref);
    CHECK(hipDeviceSynchronize());
    for (int v = 0; v < 9; ++v) {
      std::vector<float> ms;
      for (int rep = 0; rep < 11; ++rep) {
        hipLaunchKernelGGL(flush_kernel, dim3(4096), dim3(256), 0, 0, flush, flush_n);
        CHECK(hipEventRecord(s, 0));
        hipLaunchKernelGGL(ks[v], dim3(blocks), dim3(256), 0, 0, tab, rows, idx, n, out);
        CHECK(hipEventRecord(e, 0));
        CHECK(hipEventSynchronize(e));
        float t;
        CHECK(hipEventElapsedTime(&t, s, e));
        if (rep) ms.push_back(t);
      }
      std::sort(ms.begin(), ms.end());
      // check against the plain gather
      std::vector<float> a(16), b(16);
      bool same = true;
      for (int64_t probe : {(int64_t)0, (int64_t)12345, n / 2, n - 1}) {
        CHECK(hipMemcpy(a.data(), out + probe * 2, 32, hipMemcpyDeviceToHost));
        CHECK(hipMemcpy(b.data(), ref + probe * 2, 32, hipMemcpyDeviceToHost));
        for (int j = 0; j < 8; ++j) same = same && a[j] == b[j];
      }
      printf("%s table %-16s median %.3f ms best %.3f ms  rows/s %.2f G  %s\n",
             tb ? "B(60M x 32B)" : "A(2.5M x 32B)", names[v], ms[ms.size() / 2], ms[0],
             n / ms[ms.size() / 2] / 1e6, same ? "same" : "DIFFERENT");
      fflush(stdout);
    }
  }
  return 0;
}
