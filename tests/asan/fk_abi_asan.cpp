// Host-side checks of the C ABI under AddressSanitizer (host code only; the
// device code is built as usual).  Every call below must be refused by the
// host-side validation before any HIP call, so the program needs no GPU and
// launches nothing: NULL pointers, sizes out of range, misaligned pointers,
// workspaces smaller than their header, plus the pure size and status
// functions over their whole input ranges.  A memory error in the
// validation, the size arithmetic or the message formatting stops the run
// (ASan); a call that is not refused, or that gets as far as a HIP call
// (FK_ERR_LAUNCH), fails it.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fastkernels_hip.h"

static int failures = 0;
static int checks = 0;

#define EXPECT_REFUSED(call)                                                         \
  do {                                                                               \
    ++checks;                                                                        \
    const int st_ = (call);                                                          \
    const char* d_ = fk_last_error_detail();                                         \
    if (st_ == FK_OK || st_ == FK_ERR_LAUNCH || !d_ || !d_[0]) {                     \
      ++failures;                                                                    \
      fprintf(stderr, "not refused on the host (status %d) at line %d: %s\n", st_, __LINE__, #call); \
    }                                                                                \
  } while (0)

int main() {
  // 16-byte aligned host memory, never dereferenced by a refused call
  alignas(256) static unsigned char buf[1 << 16];
  void* p = buf;
  void* mis = buf + 2;  // 2-byte offset: breaks 16-byte vector loads
  float* fp = reinterpret_cast<float*>(buf);
  int64_t* ip = reinterpret_cast<int64_t*>(buf);
  int32_t* i32 = reinterpret_cast<int32_t*>(buf);
  int32_t dts[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // status strings and the version, over and past every code
  if (fk_abi_version() != 1) ++failures;
  for (int s = -100; s < 100; ++s) {
    const char* m = fk_status_string(s);
    ++checks;
    if (!m || !m[0]) ++failures;
  }
  // size functions over edge inputs (no overflow traps, 0 for nonsense)
  const int edge[] = {-2147483647 - 1, -1, 0, 1, 2, 7, 8, 9, 16, 64, 256, 257, 512, 1024, 4096, 65536, 2147483647};
  size_t sink = 0;
  for (int a : edge)
    for (int b : edge) {
      sink += fk_moe_workspace_bytes(a, 8, b, 512, 2048);
      sink += fk_moe_workspace_bytes(16, a, 256, b, 2048);
      sink += fk_attention_workspace_bytes(a, b, 2, 256);
      sink += fk_attention_workspace_bytes(1, 16, a, b);
      sink += fk_deltanet_workspace_bytes(a, b, 128);
      sink += fk_deltanet_step_workspace_bytes(a, 16, b, 128);
      sink += fk_deltanet_step_workspace_bytes(8, a, 32, b);
    }
  if (fk_moe_workspace_bytes(0, 8, 256, 512, 2048) != 0) ++failures;

  // workspace header utilities
  EXPECT_REFUSED(fk_workspace_status(nullptr, 0, 0, nullptr));
  EXPECT_REFUSED(fk_workspace_status(p, 8, 1, nullptr));
  EXPECT_REFUSED(fk_workspace_set_poll_limit(nullptr, 0, 0, nullptr));
  EXPECT_REFUSED(fk_workspace_set_poll_limit(p, 8, 0, nullptr));
  EXPECT_REFUSED(fk_workspace_set_poll_limit(p, sizeof(buf), FK_MAX_POLL_LIMIT + 1, nullptr));
  EXPECT_REFUSED(fk_workspace_set_poll_limit(p, sizeof(buf), 1ll << 40, nullptr));

  // router
  EXPECT_REFUSED(fk_moe_router(nullptr, 1, nullptr, 1, nullptr, 1, nullptr, 1, 1, 2048, 256, 8, 1e-6f, 1.f,
                               nullptr, nullptr, nullptr, nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 1, p, 1, p, 1, nullptr, 1, 1, 2048, 256, 9, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 1, p, 1, p, 1, nullptr, 1, 1, 2047, 256, 8, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 1, p, 1, p, 1, nullptr, 1, -3, 2048, 256, 8, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 1, p, 1, p, 1, nullptr, 1, 1, 2048, 2049, 8, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 9, p, 1, p, 1, nullptr, 1, 1, 2048, 256, 8, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_router(mis, 1, p, 1, p, 1, nullptr, 1, 1, 2048, 256, 8, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 1, p, 1, p, 1, nullptr, 1, 16, 2048, 256, 8, 1e-6f, 1.f, fp, ip, fp, p, 64,
                               nullptr));
  EXPECT_REFUSED(fk_moe_router(p, 1, p, 1, p, 1, nullptr, 1, 1000, 2048, 256, 8, 1e-6f, 1.f, fp, ip, fp, p,
                               sizeof(buf), nullptr));

  // routing tables
  EXPECT_REFUSED(fk_moe_align(nullptr, 3, nullptr, 0, 1, 8, 256, nullptr, 0, nullptr, nullptr, nullptr, nullptr,
                              nullptr));
  EXPECT_REFUSED(fk_moe_align(p, 0, p, 0, 1, 8, 256, p, sizeof(buf), nullptr, nullptr, nullptr, nullptr, nullptr));
  EXPECT_REFUSED(fk_moe_align(p, 3, p, 0, 1000, 8, 256, p, sizeof(buf), i32, i32, i32, i32, nullptr));
  EXPECT_REFUSED(fk_moe_align(p, 3, p, 0, 16, 8, 256, p, 32, i32, i32, i32, i32, nullptr));
  EXPECT_REFUSED(fk_moe_align(p, 3, p, 0, 16, 0, 256, p, sizeof(buf), i32, i32, i32, i32, nullptr));

  // expert stage
  EXPECT_REFUSED(fk_moe_experts(nullptr, 1, nullptr, nullptr, 1, nullptr, nullptr, nullptr, 0, 1, 2048, 512, 256, 8,
                                nullptr, nullptr, nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_moe_experts(p, 1, p, p, 1, p, p, p, 1, 16, 2048, 510, 256, 8, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_experts(p, 1, p, p, 1, p, p, p, 1, 16, 2048, 2048, 256, 8, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_experts(p, 1, mis, p, 1, p, p, p, 1, 16, 2048, 512, 256, 8, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_experts(p, 1, p, p, 1, p, p, p, 1, 16, 2048, 512, 256, 8, fp, fp, p, 16, nullptr));

  // whole layer, with and without a workspace
  EXPECT_REFUSED(fk_moe_layer(nullptr, 1, nullptr, 1, nullptr, 1, nullptr, 1, nullptr, nullptr, 1, nullptr, nullptr,
                              nullptr, 1, 1, 2048, 512, 256, 8, 1e-6f, 1.f, nullptr, nullptr, nullptr, nullptr, nullptr,
                              nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_moe_layer(p, 1, p, 1, p, 1, nullptr, 1, p, p, 1, p, p, p, 1, 16, 2048, 512, 256, 8, 1e-6f, 1.f,
                              fp, ip, fp, fp, fp, p, 100, nullptr));
  EXPECT_REFUSED(fk_moe_layer(p, 1, p, 1, p, 1, nullptr, 1, p, p, 1, p, p, p, 1, 16, 2048, 512, 256, 9, 1e-6f, 1.f,
                              fp, ip, fp, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_moe_layer_noalloc(nullptr, 1, nullptr, 1, nullptr, 1, nullptr, 1, nullptr, nullptr, 1, nullptr,
                                      nullptr, nullptr, 1, 1, 2048, 512, 256, 8, 1e-6f, 1.f, nullptr, nullptr, nullptr,
                                      nullptr, nullptr, nullptr));
  EXPECT_REFUSED(fk_moe_layer_noalloc(p, 1, p, 1, p, 1, nullptr, 1, p, p, 1, p, p, p, 1, 4000, 2048, 512, 256, 8,
                                      1e-6f, 1.f, fp, ip, fp, fp, fp, nullptr));
  EXPECT_REFUSED(fk_moe_noalloc_workspace(nullptr, nullptr, nullptr));

  // building blocks
  EXPECT_REFUSED(fk_expert_histogram(nullptr, 3, 16, 256, nullptr, nullptr));
  EXPECT_REFUSED(fk_expert_histogram(p, 7, 16, 256, i32, nullptr));
  EXPECT_REFUSED(fk_expert_histogram(p, 3, -1, 256, i32, nullptr));
  EXPECT_REFUSED(fk_expert_histogram(p, 3, 16, 0, i32, nullptr));
  EXPECT_REFUSED(fk_fused_swiglu(nullptr, 1, 4, 512, nullptr, nullptr));
  EXPECT_REFUSED(fk_fused_swiglu(p, 9, 4, 512, p, nullptr));
  EXPECT_REFUSED(fk_fused_swiglu(p, 1, -4, 512, p, nullptr));
  EXPECT_REFUSED(fk_residual_add(nullptr, 1, nullptr, 16, nullptr, nullptr));
  EXPECT_REFUSED(fk_residual_add(p, 9, fp, 16, fp, nullptr));
  EXPECT_REFUSED(fk_stream_read(nullptr, 16, nullptr, nullptr));
  EXPECT_REFUSED(fk_stream_read(mis, 64, reinterpret_cast<uint32_t*>(p), nullptr));
  EXPECT_REFUSED(fk_stream_read(p, 15, reinterpret_cast<uint32_t*>(p), nullptr));

  // attention
  EXPECT_REFUSED(fk_attention_project(nullptr, 1, nullptr, 1, nullptr, nullptr, nullptr, 1, 1, 2048, 8192, 512,
                                      1e-6f, 1.f, nullptr, nullptr, nullptr, nullptr));
  EXPECT_REFUSED(fk_attention_project(p, 1, p, 1, p, p, p, 1, 1, 2047, 8192, 512, 1e-6f, 1.f, fp, fp, fp, nullptr));
  EXPECT_REFUSED(fk_attention_project(p, 1, p, 1, p, p, p, 9, 1, 2048, 8192, 512, 1e-6f, 1.f, fp, fp, fp, nullptr));
  EXPECT_REFUSED(fk_attention_decode(nullptr, 1, nullptr, 1, nullptr, nullptr, nullptr, nullptr, 1, nullptr, nullptr, 1,
                                     nullptr, nullptr, 0, 1024, 0, nullptr, 1, 2048, 16, 2, 256, 64, 1e7f, 1, 1e-6f,
                                     1e-6f, nullptr, nullptr, nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_attention_decode(p, 1, p, 1, p, p, p, p, 1, p, p, 1, p, p, 0, 1024, 0, nullptr, 33, 2048, 16, 2,
                                     256, 64, 1e7f, 1, 1e-6f, 1e-6f, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_attention_decode(p, 1, p, 1, p, p, p, p, 1, p, p, 1, p, p, 0, 1024, 0, nullptr, 1, 2048, 24, 2,
                                     256, 64, 1e7f, 1, 1e-6f, 1e-6f, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_attention_decode(p, 1, p, 1, p, p, p, p, 1, p, p, 1, p, p, 0, 1024, 0, nullptr, 1, 2048, 16, 2,
                                     512, 64, 1e7f, 1, 1e-6f, 1e-6f, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_attention_decode(p, 1, p, 1, p, p, p, p, 1, p, p, 1, p, p, 0, 1024, 0, nullptr, 1, 2048, 16, 2,
                                     256, -1, 1e7f, 1, 1e-6f, 1e-6f, fp, fp, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_attention_decode(p, 1, p, 1, p, p, p, p, 1, p, p, 1, p, p, 0, 1024, 0, nullptr, 1, 2048, 16, 2,
                                     256, 64, 1e7f, 1, 1e-6f, 1e-6f, fp, fp, p, 64, nullptr));

  // DeltaNet
  EXPECT_REFUSED(fk_deltanet_project(nullptr, 1, nullptr, 1, nullptr, nullptr, nullptr, nullptr, 1, 1, 2048, 8192, 4096,
                                     32, 1e-6f, 1.f, nullptr, nullptr, nullptr, nullptr, nullptr));
  EXPECT_REFUSED(fk_deltanet_project(p, 1, p, 1, p, p, p, p, 1, 0, 2048, 8192, 4096, 32, 1e-6f, 1.f, fp, fp, fp, fp,
                                     nullptr));
  EXPECT_REFUSED(fk_deltanet_project(p, 1, p, 1, p, p, p, p, 1, 1, 8192, 8192, 4096, 32, 1e-6f, 1.f, fp, fp, fp, fp,
                                     nullptr));
  EXPECT_REFUSED(fk_deltanet_conv(nullptr, 0, nullptr, 0, nullptr, 0, 1, 16, 4, nullptr, nullptr, nullptr));
  EXPECT_REFUSED(fk_deltanet_conv(p, 0, p, 0, p, 0, 1, 16, 9, fp, p, nullptr));
  EXPECT_REFUSED(fk_deltanet_conv(p, 0, p, 0, p, 0, 0, 16, 4, fp, p, nullptr));
  EXPECT_REFUSED(fk_deltanet_recurrent_output(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                              nullptr, nullptr, dts, 1, 16, 32, 128, 2048, 1e-6f, nullptr, nullptr,
                                              nullptr, nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_deltanet_recurrent_output(p, p, p, p, p, p, p, p, p, nullptr, dts, 1, 16, 32, 256, 2048, 1e-6f,
                                              fp, p, nullptr, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_deltanet_recurrent_output(p, p, p, p, p, p, p, p, p, nullptr, nullptr, 1, 16, 32, 128, 2048, 1e-6f,
                                              fp, p, nullptr, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_deltanet_recurrent_output(p, p, p, p, p, p, p, p, p, nullptr, dts, 1, 16, 33, 128, 2048, 1e-6f,
                                              fp, p, nullptr, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_deltanet_step(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                  nullptr, nullptr, nullptr, nullptr, dts, 1, 2048, 16, 32, 128, 4, 1e-6f, nullptr,
                                  nullptr, nullptr, nullptr, nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_deltanet_step(p, p, p, p, p, p, p, p, p, p, p, p, p, dts, 65, 2048, 16, 32, 128, 4, 1e-6f, fp, fp,
                                  p, p, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_deltanet_step(p, p, p, p, p, p, p, p, p, p, p, p, p, dts, 1, 2048, 16, 32, 128, 9, 1e-6f, fp, fp,
                                  p, p, p, sizeof(buf), nullptr));
  EXPECT_REFUSED(fk_deltanet_step(p, p, p, p, p, p, p, p, p, p, p, p, p, dts, 1, 2048, 16, 32, 128, 4, 1e-6f, fp, fp,
                                  p, p, p, 100, nullptr));

  // synthetic blocks
  EXPECT_REFUSED(fk_synthetic_moe(nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 16, 4, 8, 9,
                                  1e-6f, nullptr, 0, nullptr));
  EXPECT_REFUSED(fk_synthetic_moe(p, 0, p, p, p, p, p, p, 0, 0, 4, 8, 2, 1e-6f, p, 0, nullptr));
  EXPECT_REFUSED(fk_synthetic_moe(p, 0, p, p, p, p, p, p, 0, 16, 4, 8, 5, 1e-6f, p, 0, nullptr));
  EXPECT_REFUSED(fk_synthetic_deltanet(nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                                       16, 2, 8, 8, 1e-6f, nullptr, nullptr, nullptr));
  EXPECT_REFUSED(fk_synthetic_deltanet(p, 0, p, 0, p, p, p, p, p, p, 0, 4096, 2, 8, 8, 1e-6f, p, p, nullptr));
  EXPECT_REFUSED(fk_synthetic_attention(nullptr, 0, nullptr, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr,
                                        0, 16, 4, 2, 8, 4, 0, 16, 1e-6f, nullptr, nullptr));
  EXPECT_REFUSED(fk_synthetic_attention(p, 0, p, p, 0, p, p, p, p, p, 0, 16, 4, 2, 8, 4, 16, 16, 1e-6f, p, nullptr));

  printf("fk_abi_asan: %d calls checked, %d not refused (size sum %zu)\n", checks, failures, sink);
  return failures ? 1 : 0;
}
