// Library-level C-ABI functions: version, status strings, last-error text.
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
    default: return "unknown status";
  }
}

const char* fk_last_error_detail(void) { return fk::g_last_error; }

}  // extern "C"
