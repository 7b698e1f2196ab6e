// Host-side checks of the C ABI's argument validation (include/zonos3_gdn.h), built with AddressSanitizer on the
// host code of every library source (zonos3-mini_amd/build.py, build_asan). Every call below is rejected by
// the library's checks before any HIP call or kernel launch, so the program needs no GPU; host arrays the ABI
// reads (the routing's source-pointer array, the status word) are heap blocks of exactly the size passed, so
// that a read or write past them is an AddressSanitizer report. Exit status: the number of failed checks.
#include <cstdio>
#include <cstring>
#include <vector>

#include "zonos3_gdn.h"

static int failures = 0;

static void expect(const char* what, int got, int want, const char* fragment) {
  const char* msg = zgdn_last_error();
  const bool ok = got == want && (fragment == nullptr || (msg != nullptr && std::strstr(msg, fragment) != nullptr));
  if (!ok) {
    ++failures;
    std::fprintf(stderr, "FAIL %s: status %d (want %d), message \"%s\" (want \"%s\")\n", what, got, want,
                 msg ? msg : "(null)", fragment ? fragment : "");
  }
}

int main() {
  std::vector<unsigned char> block(4096);
  void* p = block.data();  // stands for a device buffer: never dereferenced on the host by a rejected call
  const int32_t* tab = reinterpret_cast<const int32_t*>(p);
  float* f = reinterpret_cast<float*>(p);

  if (zgdn_abi_version() != 2) {
    ++failures;
    std::fprintf(stderr, "FAIL abi version %d\n", zgdn_abi_version());
  }

  // recurrent step / sequence
  expect("recurrent null", zgdn_recurrent_fwd(nullptr, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, 1, nullptr, 0,
                                              1, 1, 4, 4, 128, 128, 0.1f, nullptr),
         ZGDN_EINVAL, "null");
  expect("recurrent K", zgdn_recurrent_fwd(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, 1, nullptr, 0, 1, 1, 4,
                                           4, 96, 128, 0.1f, nullptr),
         ZGDN_EUNSUPPORTED, "K=96");
  expect("recurrent heads", zgdn_recurrent_fwd(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, 1, nullptr, 0, 1, 1,
                                               3, 4, 128, 128, 0.1f, nullptr),
         ZGDN_EINVAL, "multiple");
  expect("recurrent gate pair", zgdn_recurrent_fwd(p, p, p, 1, p, p, 1, f, nullptr, 1, f, f, p, 1, nullptr, 0, 1, 1, 4,
                                                   4, 128, 128, 0.1f, nullptr),
         ZGDN_EINVAL, "together");
  expect("recurrent packed B", zgdn_recurrent_fwd(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, 1, tab, 2, 2, 8,
                                                  4, 4, 128, 128, 0.1f, nullptr),
         ZGDN_EINVAL, "B == 1");

  // chunked prefill
  const size_t ws_small = 16;
  expect("chunk null", zgdn_chunk_fwd(nullptr, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, nullptr, nullptr, 0, 1,
                                      1, 64, 4, 4, 128, 128, 512, 512, 512, 4, 0, 0.1f, p, ws_small, nullptr),
         ZGDN_EINVAL, nullptr);
  expect("chunk K", zgdn_chunk_fwd(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, nullptr, nullptr, 0, 1, 1, 64, 4,
                                   4, 64, 128, 256, 256, 512, 4, 0, 0.1f, p, ws_small, nullptr),
         ZGDN_EUNSUPPORTED, "K=64");
  expect("chunk workspace", zgdn_chunk_fwd(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, nullptr, nullptr, 0, 1, 1,
                                           64, 4, 4, 128, 128, 512, 512, 512, 4, 0, 0.1f, p, ws_small, nullptr),
         ZGDN_EINVAL, "workspace");
  expect("chunk strides", zgdn_chunk_fwd(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, nullptr, nullptr, 0, 1, 1,
                                         64, 4, 4, 128, 128, 100, 512, 512, 4, 0, 0.1f, p, 1 << 30, nullptr),
         ZGDN_EINVAL, "row strides");
  const size_t cap = zgdn_chunk_noalloc_max_bytes();
  expect("chunk noalloc size", zgdn_chunk_fwd_noalloc(p, p, p, 1, p, p, 1, nullptr, nullptr, 1, f, f, p, nullptr,
                                                      nullptr, 0, 1 << 20, 1, 64 << 20, 4, 64, 128, 128, 64 * 128,
                                                      64 * 128, 64 * 128, 64, 0, 0.1f, nullptr),
         ZGDN_EINVAL, "scratch");
  if (cap == 0) {
    ++failures;
    std::fprintf(stderr, "FAIL noalloc capacity 0\n");
  }
  if (zgdn_chunk_workspace_size(0, 16) == 0 && zgdn_chunk_workspace_size(64, 16) == 0) {
    ++failures;
    std::fprintf(stderr, "FAIL chunk workspace size\n");
  }
  if (zgdn_chunk_workspace_bytes(4, 4, 96, 96, 0) != 0 || zgdn_chunk_workspace_bytes(4, 4, 64, 64, 0) == 0) {
    ++failures;
    std::fprintf(stderr, "FAIL chunk workspace bytes\n");
  }
  expect("chunk fp32 strides", zgdn_chunk_fwd(p, p, p, 0, p, p, 1, nullptr, nullptr, 1, f, f, p, nullptr, nullptr, 0, 1,
                                              1, 64, 4, 4, 64, 64, 258, 256, 256, 4, 0, 0.1f, p, 1 << 30, nullptr),
         ZGDN_EINVAL, "multiples of 4");
  expect("launch form", zgdn_chunk_set_launch_form(7), ZGDN_EINVAL, nullptr);
  expect("launch form default", zgdn_chunk_set_launch_form(-1), ZGDN_OK, nullptr);
  expect("chunk status null", zgdn_chunk_status(nullptr, 0), ZGDN_EINVAL, nullptr);
  expect("chunk status async null", zgdn_chunk_status_async(nullptr, nullptr), ZGDN_EINVAL, nullptr);
  expect("overlap queues 256/8", zgdn_chunk_overlap_queues(256, 8), 8, nullptr);
  expect("overlap queues uneven", zgdn_chunk_overlap_queues(250, 8), 0, nullptr);

  // fused decode block, serving decode step
  expect("fused K", zgdn_fused_decode_step(p, p, p, p, 1, p, p, f, f, p, f, p, 4, 8, 16, 64, 64, 4, 1e-6f, 0.1f, 0,
                                           nullptr),
         ZGDN_EUNSUPPORTED, "K=64");
  expect("fused groups", zgdn_fused_decode_step(p, p, p, p, 1, p, p, f, f, p, f, p, 4, 2, 16, 128, 128, 4, 1e-6f, 0.1f,
                                                0, nullptr),
         ZGDN_EUNSUPPORTED, "Hv/Hk=8");
  expect("serving null", zgdn_serving_decode_step(nullptr, 2056, p, 256, 1, nullptr, 1, 1, 4, 4, 128, 128, 4, p, p, p, f,
                                                  f, p, nullptr, 64, f, f, p, p, 1e-5f, 0.1f, 1, nullptr),
         ZGDN_EINVAL, "null");

  // residual routing: a source-pointer array of exactly n entries
  {
    const int n = 23;
    const void** srcs = new const void*[n];
    for (int i = 0; i < n; ++i) srcs[i] = p;
    expect("attnres dim", zgdn_attnres_route(srcs, n, 4, 1001, 1001, 1, p, 1e-5f, p, nullptr), ZGDN_EUNSUPPORTED,
           "dim=1001");
    expect("attnres stride", zgdn_attnres_route(srcs, n, 4, 1024, 1000, 1, p, 1e-5f, p, nullptr), ZGDN_EINVAL,
           "stride");
    srcs[n - 1] = nullptr;
    expect("attnres null source", zgdn_attnres_route(srcs, n, 4, 1024, 1024, 1, p, 1e-5f, p, nullptr), ZGDN_EINVAL,
           "null source 22");
    delete[] srcs;
    const void** one = new const void*[1];
    one[0] = p;
    expect("attnres count", zgdn_attnres_route(one, 65, 4, 1024, 1024, 1, p, 1e-5f, p, nullptr), ZGDN_EUNSUPPORTED,
           "65 sources");
    delete[] one;
  }

  // row operators
  expect("conv width", zgdn_causal_conv1d_fwd(p, p, nullptr, 1, nullptr, nullptr, 3, p, nullptr, nullptr, 0, 0, 1, 8,
                                              64, 5, 1, 64, nullptr),
         ZGDN_EUNSUPPORTED, "width 5");
  expect("conv packed", zgdn_causal_conv1d_fwd(p, p, nullptr, 1, nullptr, nullptr, 3, p, tab, nullptr, 1, 0, 1, 8, 64,
                                               4, 1, 64, nullptr),
         ZGDN_EINVAL, "packed");
  expect("l2norm D", zgdn_l2norm_fwd(p, 1, p, 1, f, 4, 2048, 1, 2048, 1e-6f, nullptr), ZGDN_EUNSUPPORTED, "D=2048");
  expect("sigmoid null", zgdn_sigmoid_fwd(nullptr, 1, p, 1, 16, 1.f, nullptr), ZGDN_EINVAL, "null");
  expect("gated norm group", zgdn_gated_rmsnorm_fwd(p, p, p, 1, p, f, 4, 128, 0, 128, 1e-5f, nullptr), ZGDN_EINVAL,
         "group");

  // accent shift
  expect("accent K", zgdn_accent_shift(p, 1024, p, p, p, 300, p, 2056, p, 2056, 4, 1024, 2056, 300, 1, p, 1 << 20,
                                       nullptr),
         ZGDN_EUNSUPPORTED, "K=300");
  expect("accent workspace", zgdn_accent_shift(p, 1024, p, p, p, 64, p, 2056, p, 2056, 100, 1024, 2056, 64, 1, p, 16,
                                               nullptr),
         ZGDN_EINVAL, "workspace");
  expect("accent strides", zgdn_accent_shift(p, 1000, p, p, p, 64, p, 2056, p, 2056, 100, 1024, 2056, 64, 1, p,
                                             1 << 20, nullptr),
         ZGDN_EINVAL, "row strides");

  std::fprintf(stderr, "%d failed checks\n", failures);
  return failures;
}
