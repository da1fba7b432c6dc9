// Error reporting and version entry points of the C ABI.
#include "qsa_common.h"
#include "../../include/qsa_hip.h"

namespace qsa {

static thread_local std::string t_last_error;

void set_error(const std::string& message) { t_last_error = message; }

int fail(int status, const std::string& message) {
  set_error(message);
  return status;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(QSA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
  return QSA_OK;
}

}  // namespace qsa

extern "C" const char* qsa_last_error(void) { return qsa::t_last_error.c_str(); }

extern "C" int qsa_abi_version(void) { return 3; }
