// Host-side checks of libmdgl's C ABI under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by tests/sanitize/Makefile; the device
// code is not instrumented). Every call here returns before anything is
// launched: argument validation, broadcast descriptors, workspace sizes and
// the softmax geometry, the paths capi.cpp runs on the host for every call.
// Exit status 0 when every expectation holds; a sanitizer report fails the
// run by itself.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/mdgl.h"

static int failures = 0;

#define EXPECT(cond)                                                       \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                          \
    }                                                                      \
  } while (0)

static void gsddmm_shapes() {
  // no edges: every shape combination is validated, nothing is launched
  const int64_t shapes[][2][4] = {
      {{4, 1, 8, 0}, {1, 3, 8, 0}}, {{2, 3, 4, 0}, {2, 1, 4, 0}}, {{1, 1, 1, 0}, {5, 1, 1, 0}},
      {{7, 1, 1, 0}, {1, 6, 1, 0}}, {{3, 0, 2, 0}, {3, 1, 2, 0}},
  };
  for (auto& sh : shapes) {
    for (int nd = 1; nd <= 3; ++nd) {
      int64_t dl = 1, dr = 1, dout = 1;
      bool ok = true;
      for (int k = 0; k < nd; ++k) {
        const int64_t l = sh[0][k], r = sh[1][k];
        dl *= l;
        dr *= r;
        if (l != r && l != 1 && r != 1) ok = false;
        dout *= (l == 1 ? r : l);
      }
      for (int op = 0; op <= 3; ++op) {
        const int rc = mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 1, op, dl,
                                   dr, dout, nd, sh[0], sh[1], MDGL_FLOAT32, nullptr);
        EXPECT(rc == MDGL_OK || !ok);
      }
      // dot contracts the last axis; the rest broadcasts
      int64_t lo = 1, ro = 1, oo = 1;
      bool dok = sh[0][nd - 1] == sh[1][nd - 1];
      for (int k = 0; k < nd; ++k) {
        lo *= sh[0][k];
        ro *= sh[1][k];
        if (k < nd - 1) {
          if (sh[0][k] != sh[1][k] && sh[0][k] != 1 && sh[1][k] != 1) dok = false;
          oo *= (sh[0][k] == 1 ? sh[1][k] : sh[0][k]);
        }
      }
      const int rc = mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 1, 4, lo, ro,
                                 oo, nd, sh[0], sh[1], MDGL_FLOAT64, nullptr);
      EXPECT((rc == MDGL_OK) == dok);
    }
  }
  // mismatched widths and bad codes are refused with a message
  int64_t ls[2] = {4, 8}, rs[2] = {4, 8};
  EXPECT(mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 10, 0, 1, 0, 32, 32, 31, 2, ls,
                     rs, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  EXPECT(std::strlen(mdgl_last_error()) > 0);
  EXPECT(mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 10, 0, 5, 0, 8, 8, 8, 0,
                     nullptr, nullptr, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 10, 0, 1, 9, 8, 8, 8, 0,
                     nullptr, nullptr, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 10, 0, 1, 0, 8, 8, 8, 0,
                     nullptr, nullptr, 7, nullptr) == MDGL_EINVAL);
  int64_t deep_l[7] = {2, 1, 2, 1, 2, 1, 2}, deep_r[7] = {1, 2, 1, 2, 1, 2, 1};
  EXPECT(mdgl_gsddmm(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 1, 0, 16, 8, 128, 7,
                     deep_l, deep_r, MDGL_FLOAT32, nullptr) == MDGL_ENOTSUP);
}

static void gspmm_arguments() {
  int64_t ls[2] = {8, 32}, rs[2] = {8, 1};
  // no rows: validated, nothing launched
  EXPECT(mdgl_gspmm(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 2, 256, 8, 256, 0,
                    nullptr, 2, ls, rs, nullptr, nullptr, nullptr, nullptr, 0, 0, nullptr,
                    nullptr, 0, nullptr, 0, 0, MDGL_FLOAT32, nullptr) == MDGL_OK);
  EXPECT(mdgl_gspmm(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 5, 4, 8, 8, 8, 0,
                    nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0,
                    nullptr, nullptr, 0, nullptr, 0, 0, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_gspmm(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 5, 2, 8, 8, 8, 9,
                    nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0,
                    nullptr, nullptr, 0, nullptr, 0, 0, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  // an incomplete heavy-row schedule and a missing workspace
  int32_t dummy[4] = {0, 0, 0, 0};
  EXPECT(mdgl_gspmm(dummy, dummy, dummy, dummy, dummy, dummy, 5, 2, 8, 8, 8, 0, nullptr, 0,
                    nullptr, nullptr, nullptr, nullptr, dummy, nullptr, 3, 4, dummy, dummy, 1,
                    nullptr, 0, 0, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_gspmm(dummy, dummy, dummy, dummy, dummy, dummy, 5, 2, 8, 8, 8, 0, nullptr, 0,
                    nullptr, nullptr, nullptr, nullptr, dummy, dummy, 3, 4, dummy, dummy, 1,
                    nullptr, 0, 0, MDGL_FLOAT32, nullptr) == MDGL_EWORKSPACE);
  // the row-list form: a negative count, or a non-empty list without its rows
  EXPECT(mdgl_gspmm_rows(dummy, dummy, dummy, dummy, dummy, dummy, 5, 2, 8, 8, 8, 0, nullptr, 0,
                         nullptr, nullptr, nullptr, nullptr, nullptr, -1, 0, MDGL_FLOAT32,
                         nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_gspmm_rows(dummy, dummy, dummy, dummy, dummy, dummy, 5, 2, 8, 8, 8, 0, nullptr, 0,
                         nullptr, nullptr, nullptr, nullptr, nullptr, 3, 0, MDGL_FLOAT32,
                         nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_gspmm_rows(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 5, 2, 8, 8, 8, 0,
                         nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0,
                         MDGL_FLOAT32, nullptr) == MDGL_OK);
  // the no-allocation form refuses partials beyond its scratch before anything else
  EXPECT(mdgl_gspmm_noalloc(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 10, 2, 4096,
                            4096, 4096, 0, nullptr, 0, nullptr, nullptr, nullptr, nullptr,
                            nullptr, nullptr, 1 << 20, 8, nullptr, nullptr, 1, 0, MDGL_FLOAT32,
                            nullptr) == MDGL_EWORKSPACE);
}

static void sizes_and_geometry() {
  for (int64_t n : {0, 1, 4095, 4096, 4097, 1 << 20}) {
    EXPECT(mdgl_segment_offsets_workspace_bytes(n) >= 0);
    EXPECT(mdgl_build_csr_workspace_bytes(n, 1000) >= 0);
    for (int dt = 0; dt < 2; ++dt) {
      EXPECT(mdgl_gspmm_workspace_bytes(n, 64, 1, dt) >= 0);
      EXPECT(mdgl_softmax_workspace_bytes(n, n, 8, dt) >= 0);
      EXPECT(mdgl_segment_mm_workspace_bytes(n, 128, 128, 64, dt) >= 0);
      EXPECT(mdgl_gather_mm_workspace_bytes(n, 16, 16, 64, dt) >= 0);
      EXPECT(mdgl_segment_mm_grad_workspace_bytes(n, 33, 130, 3, dt) >= 0);
      EXPECT(mdgl_gather_mm_grad_workspace_bytes(n, 33, 130, 3, dt) >= 0);
    }
  }
  EXPECT(mdgl_build_csr_workspace_bytes(-1, 5) < 0);
  EXPECT(mdgl_softmax_workspace_bytes(1, 1, 1, 9) < 0);
  std::vector<double> buf(64);
  for (int64_t d : {1, 2, 3, 8, 16, 33, 64, 256, 1000}) {
    for (int dt = 0; dt < 2; ++dt) {
      int64_t slots = 0, chunk = 0;
      for (int off = 0; off < 2; ++off) {
        const char* p = reinterpret_cast<const char*>(buf.data()) + off * (dt ? 8 : 4);
        EXPECT(mdgl_softmax_geometry(d, dt, p, p, &slots, &chunk) == MDGL_OK);
        EXPECT(slots >= 1 && slots <= 64 && chunk >= slots);
      }
    }
  }
  EXPECT(mdgl_softmax_geometry(0, 0, nullptr, nullptr, nullptr, nullptr) == MDGL_EINVAL);
}

static void other_entry_points() {
  EXPECT(mdgl_workers() > 1);
  EXPECT(mdgl_trace_ranges() == 0 || mdgl_trace_ranges() == 1);
  EXPECT(mdgl_segment_reduce(nullptr, nullptr, nullptr, 0, 4, 0, 0, 0, MDGL_FLOAT32, nullptr) ==
         MDGL_OK);
  EXPECT(mdgl_segment_reduce(nullptr, nullptr, nullptr, 3, 4, 7, 0, 0, MDGL_FLOAT32, nullptr) ==
         MDGL_EINVAL);
  EXPECT(mdgl_segment_reduce_arg(nullptr, nullptr, nullptr, nullptr, 3, 4, 0, 10, 0, MDGL_FLOAT32,
                                 nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_build_csr(nullptr, nullptr, 10, 0, nullptr, nullptr, nullptr, nullptr, 0, nullptr) ==
         MDGL_EINVAL);
  EXPECT(mdgl_segment_mm(nullptr, nullptr, nullptr, nullptr, 0, 4, 2, 4, nullptr, 0, MDGL_FLOAT32,
                         nullptr) == MDGL_OK);
  EXPECT(mdgl_gather_mm(nullptr, nullptr, nullptr, nullptr, 10, 4, 4, 5000, nullptr, 0,
                        MDGL_FLOAT32, nullptr) == MDGL_ENOTSUP);
  EXPECT(mdgl_cumsum(nullptr, nullptr, -1, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_clamp_i64(nullptr, nullptr, 0, 1, 2, nullptr) == MDGL_OK);
  EXPECT(mdgl_replace_inf_with_zero(nullptr, nullptr, 5, MDGL_FLOAT64, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_scatter_rows(nullptr, nullptr, nullptr, 0, 8, MDGL_FLOAT32, nullptr) == MDGL_OK);
  EXPECT(mdgl_gather_rows(nullptr, nullptr, nullptr, 4, 8, MDGL_FLOAT32, nullptr) == MDGL_EINVAL);
  EXPECT(mdgl_read_rows(nullptr, 0, 64, nullptr, 0, nullptr, 0, nullptr, nullptr) == MDGL_OK);
  EXPECT(mdgl_read_rows(nullptr, 10, 24, nullptr, 64, nullptr, 0, nullptr, nullptr) ==
         MDGL_EINVAL);
  EXPECT(mdgl_read_rows(nullptr, 10, 64, nullptr, 64, nullptr, 0, nullptr, nullptr) ==
         MDGL_EINVAL);
  EXPECT(mdgl_read_rows_sink_bytes(64) == 16 && mdgl_read_rows_sink_bytes(-1) == -1);
}

int main() {
  gsddmm_shapes();
  gspmm_arguments();
  sizes_and_geometry();
  other_entry_points();
  if (failures) {
    std::fprintf(stderr, "%d expectation(s) failed\n", failures);
    return 1;
  }
  std::printf("abi host checks passed\n");
  return 0;
}
