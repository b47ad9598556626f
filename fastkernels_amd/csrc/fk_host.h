// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/fastkernels_hip.h"

namespace fk {

// Records a formatted reason for the calling thread's last failure and
// returns `status`, so call sites read `return fail(FK_ERR_INVALID, "...")`.
int fail(int status, const char* fmt, ...);

// Header of every polling kernel's workspace: 16 uint32 words at its start.
// Word kWorkspaceEpochWord is the launch epoch of the tagged hand-offs (a
// launch tags its words epoch + 1); kWorkspacePollWord is the host-set
// bound on every in-kernel wait plus one (0: the built-in bound);
// kWorkspaceErrorWord records a bounded wait that ran out.  While the error
// word is set, every wait of a kernel on the workspace gives up at once and
// its outputs are NaN, until fk_workspace_status(clear) resets the word and
// advances the epoch past every word written so far.
constexpr int kWorkspaceEpochWord = 8;
constexpr int kWorkspacePollWord = 14;
constexpr int kWorkspaceErrorWord = 15;
// Largest host-set wait bound (poll rounds), fk_workspace_set_poll_limit.
constexpr long long kMaxPollLimit = 1ll << 22;

// Normalized multi-matrix projection (fk_deltanet.hip), shared by the mixers.
int launch_norm_projection(const void* x, int x_dt, const void* nw, int nw_dt, const void* const (&w)[4],
                           const int (&rows)[4], float* const (&out)[4], int weight_dt, int T, int H, float eps,
                           float off, hipStream_t s);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline bool is_float_dtype(int dt) { return dt == FK_DTYPE_F32 || dt == FK_DTYPE_BF16; }
inline bool is_index_dtype(int dt) { return dt == FK_DTYPE_I32 || dt == FK_DTYPE_I64; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
  return FK_OK;
}

// Co-resident workgroup capacity of a kernel on the current device (cached
// per device); the grid-barrier kernels never launch more workgroups.
template <typename K>
inline int resident_capacity(K kernel, int block, size_t shm, int* cache) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] > 0) return cache[dev];
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, shm) != hipSuccess) return 0;
  cache[dev] = cus * per_cu;
  return cache[dev];
}

inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = cus;
  }
  return cache[dev];
}

}  // namespace fk
