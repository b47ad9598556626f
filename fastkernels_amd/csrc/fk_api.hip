// Library-level C-ABI functions: version, status strings, last-error text.
#include "fk_common.h"
#include "fk_host.h"

namespace fk {

static thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

// Stream-ordered header updates (kernels rather than memsets, so that a
// caller may also record them into a HIP graph).
__global__ void ws_clear_error_kernel(uint32_t* header) {
  if (header[kWorkspaceErrorWord] != 0u) {
    header[kWorkspaceErrorWord] = 0u;
    // every word written so far carries a tag <= epoch + 1: the next launch
    // (tag epoch + 2) takes none of them for its own
    header[kWorkspaceEpochWord] += 1u;
  }
}

__global__ void ws_set_word_kernel(uint32_t* header, int word, uint32_t value) { header[word] = value; }

}  // namespace fk

extern "C" {

int fk_abi_version(void) { return FK_ABI_VERSION; }

const char* fk_status_string(int status) {
  switch (status) {
    case FK_OK: return "ok";
    case FK_ERR_INVALID: return "invalid argument";
    case FK_ERR_DTYPE: return "unsupported dtype";
    case FK_ERR_WORKSPACE: return "workspace missing or too small";
    case FK_ERR_LAUNCH: return "kernel launch failed";
    case FK_ERR_UNSUPPORTED: return "shape outside kernel limits";
    case FK_ERR_ALIGNMENT: return "pointer or row length not 16-byte aligned";
    case FK_ERR_DEVICE: return "a bounded in-kernel wait ran out; outputs invalid";
    default: return "unknown status";
  }
}

const char* fk_last_error_detail(void) { return fk::g_last_error; }

int fk_workspace_status(const void* workspace, size_t workspace_bytes, int clear, void* stream) {
  using namespace fk;
  if (!workspace || workspace_bytes < (kWorkspaceErrorWord + 1) * sizeof(uint32_t))
    return fail(FK_ERR_WORKSPACE, "fk_workspace_status: workspace missing or smaller than its header");
  const hipStream_t s = as_stream(stream);
  uint32_t* word = reinterpret_cast<uint32_t*>(const_cast<void*>(workspace)) + kWorkspaceErrorWord;
  uint32_t v = 0;
  hipError_t err = hipMemcpyAsync(&v, word, sizeof(v), hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  if (err == hipSuccess && v != 0 && clear) {
    hipLaunchKernelGGL(ws_clear_error_kernel, dim3(1), dim3(1), 0, s,
                       reinterpret_cast<uint32_t*>(const_cast<void*>(workspace)));
    err = hipGetLastError();
    if (err == hipSuccess) err = hipStreamSynchronize(s);
  }
  if (err != hipSuccess) return fail(FK_ERR_LAUNCH, "fk_workspace_status: %s", hipGetErrorString(err));
  if (v != 0)
    return fail(FK_ERR_DEVICE, "device flags 0x%x:%s%s", v, (v & FK_DEVICE_ERR_BARRIER) ? " a kernel's bounded wait ran out;" : "",
                (v & FK_DEVICE_ERR_POSITION) ? " an attention step's device-held position would pass the cache;" : "");
  return FK_OK;
}

int fk_workspace_set_poll_limit(void* workspace, size_t workspace_bytes, long long limit, void* stream) {
  using namespace fk;
  if (!workspace || workspace_bytes < (kWorkspaceErrorWord + 1) * sizeof(uint32_t))
    return fail(FK_ERR_WORKSPACE, "fk_workspace_set_poll_limit: workspace missing or smaller than its header");
  // A round is one coherent read of the words not yet in (0.1-1 us), so the
  // cap keeps a wait that fails within a few seconds, like the built-in bound.
  if (limit > kMaxPollLimit)
    return fail(FK_ERR_INVALID, "poll limit must be at most %lld rounds (got %lld)", (long long)kMaxPollLimit, limit);
  const uint32_t value = limit < 0 ? 0u : (uint32_t)limit + 1u;
  hipLaunchKernelGGL(ws_set_word_kernel, dim3(1), dim3(1), 0, as_stream(stream), reinterpret_cast<uint32_t*>(workspace),
                     kWorkspacePollWord, value);
  return check_launch("ws_set_word_kernel");
}

}  // extern "C"
