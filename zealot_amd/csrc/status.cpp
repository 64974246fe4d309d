// status.cpp -- thread-local last-error string of the C ABI.
#include <string>

#include "zk_common.h"

namespace zk {
namespace {
thread_local std::string g_last_error;
}
int set_error(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}
void clear_error() { g_last_error.clear(); }
const char *last_error_cstr() { return g_last_error.c_str(); }
}  // namespace zk

extern "C" const char *zk_last_error(void) { return zk::last_error_cstr(); }
extern "C" int zk_abi_version(void) { return ZK_ABI_VERSION; }
