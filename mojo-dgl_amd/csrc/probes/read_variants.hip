// Measurement probe (not part of the library): one-pass streaming read
// variants over 1.28 GB and 2.56 GB, each launch after a 512 MB write that
// flushes the caches; median and best of 10. 16-byte loads, 1 to 16 per lane
// per workgroup (4 to 64 KB per workgroup), nontemporal or plain, and a
// persistent grid of 2,048 or 4,096 workgroups (the form of mdgl_read_stream).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x) do { hipError_t err_ = (x); if (err_ != hipSuccess) { \
  fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(err_)); exit(1); } } while (0)

typedef unsigned int u4 __attribute__((ext_vector_type(4)));

template <int PER, bool NT>
__global__ __launch_bounds__(256) void rd(const u4* __restrict__ src, int64_t n16, u4* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * 256 * PER;
  u4 v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t i = base + j * 256 + threadIdx.x;
    if (i < n16) v[j] = NT ? __builtin_nontemporal_load(src + i) : src[i];
    else v[j] = u4{0, 0, 0, 0};
  }
  u4 x = v[0];
#pragma unroll
  for (int j = 1; j < PER; ++j) x ^= v[j];
  if ((x.x ^ x.y ^ x.z ^ x.w) == 0x12345678u) sink[blockIdx.x * 256 + threadIdx.x] = x;
}

// persistent: a fixed grid strides over chunks of 256 * PER vectors
template <int PER>
__global__ __launch_bounds__(256) void rd_persist(const u4* __restrict__ src, int64_t n16, u4* __restrict__ sink) {
  u4 x{0, 0, 0, 0};
  for (int64_t base = (int64_t)blockIdx.x * 256 * PER; base < n16; base += (int64_t)gridDim.x * 256 * PER) {
    u4 v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int64_t i = base + j * 256 + threadIdx.x;
      v[j] = i < n16 ? __builtin_nontemporal_load(src + i) : u4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) x ^= v[j];
  }
  if ((x.x ^ x.y ^ x.z ^ x.w) == 0x12345678u) sink[blockIdx.x * 256 + threadIdx.x] = x;
}

__global__ void flush_kernel(u4* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = u4{1, 2, 3, 4};
}

typedef void (*K)(const u4*, int64_t, u4*);

int main() {
  const int64_t maxb = 2560000000ll;
  u4 *src, *sink, *flush;
  const int64_t flush_n = (512ll << 20) / 16;
  CHECK(hipMalloc(&src, maxb));
  CHECK(hipMemset(src, 1, maxb));
  // the sink is written only on a value the data never produces; sized for
  // the largest grid anyway (blocks of the PER = 1 variant, 256 lanes each)
  const int64_t sink_n = (maxb / 16 / 256 + 1) * 256;
  CHECK(hipMalloc(&sink, sink_n * 16));
  CHECK(hipMalloc(&flush, flush_n * 16));
  struct V { const char* name; K k; int per; bool persist; };
  V vs[] = {{"per1_nt", rd<1, true>, 1, false},   {"per2_nt", rd<2, true>, 2, false},
            {"per4_nt", rd<4, true>, 4, false},   {"per8_nt", rd<8, true>, 8, false},
            {"per16_nt", rd<16, true>, 16, false}, {"per4_plain", rd<4, false>, 4, false},
            {"per8_plain", rd<8, false>, 8, false}, {"persist4_x2048", rd_persist<4>, 4, true},
            {"persist8_x2048", rd_persist<8>, 8, true}, {"persist8_x4096", rd_persist<8>, 8, true}};
  hipEvent_t s, e;
  CHECK(hipEventCreate(&s));
  CHECK(hipEventCreate(&e));
  for (int64_t bytes : {(int64_t)1280000000, maxb}) {
    const int64_t n16 = bytes / 16;
    for (int vi = 0; vi < 10; ++vi) {
      const V& v = vs[vi];
      int64_t blocks = v.persist ? (vi == 9 ? 4096 : 2048) : (n16 + 256 * v.per - 1) / (256 * v.per);
      if (blocks * 256 > sink_n) { fprintf(stderr, "grid too large\n"); return 1; }
      std::vector<float> ms;
      for (int rep = 0; rep < 11; ++rep) {
        hipLaunchKernelGGL(flush_kernel, dim3(4096), dim3(256), 0, 0, flush, flush_n);
        CHECK(hipEventRecord(s, 0));
        hipLaunchKernelGGL(v.k, dim3((unsigned)blocks), dim3(256), 0, 0, src, n16, sink);
        CHECK(hipEventRecord(e, 0));
        CHECK(hipEventSynchronize(e));
        float t;
        CHECK(hipEventElapsedTime(&t, s, e));
        if (rep) ms.push_back(t);
      }
      std::sort(ms.begin(), ms.end());
      printf("%.2f GB %-16s median %.4f ms best %.4f ms -> %.0f GB/s (best %.0f)\n", bytes / 1e9,
             v.name, ms[ms.size() / 2], ms[0], bytes / ms[ms.size() / 2] / 1e6, bytes / ms[0] / 1e6);
      fflush(stdout);
    }
  }
  return 0;
}
