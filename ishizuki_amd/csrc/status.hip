// Status reporting of the C ABI: the reason for the calling thread's last non-OK status.
#include <cstdio>

#include "common.h"

namespace ishz {
static thread_local std::string t_last_error;

void set_error(const std::string &msg) { t_last_error = msg; }

int fail(const char *what, hipError_t e) {
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return ISHZ_EHIP;
}

int decline(const std::string &why) {
  set_error("declined: " + why);
  return ISHZ_DECLINED;
}

int einval(const std::string &why) {
  set_error("invalid argument: " + why);
  return ISHZ_EINVAL;
}
}  // namespace ishz

extern "C" const char *ishz_last_error(void) { return ishz::t_last_error.c_str(); }
extern "C" int ishz_version(void) { return 100; }
