// status.cpp -- thread-local last-error string of the C ABI.
#include <string>

#include "zk_common.h"

namespace zk {
namespace {
thread_local std::string g_last_error;
// An error whose message is built only when zk_last_error asks for it: the
// BlockManager's rejections are part of normal scheduling (a full pool, a
// stale handle) and cost a few stores this way.
struct Deferred {
    DeferredError kind = DeferredError::None;
    uint64_t a = 0, b = 0, c = 0;
};
thread_local Deferred g_deferred;
}  // namespace
int set_error(int code, const std::string &msg) {
    g_deferred.kind = DeferredError::None;
    g_last_error = msg;
    return code;
}
int set_error_deferred(int code, DeferredError kind, uint64_t a, uint64_t b, uint64_t c) {
    g_deferred = Deferred{kind, a, b, c};
    return code;
}
void clear_error() {
    g_deferred.kind = DeferredError::None;
    g_last_error.clear();
}
const char *last_error_cstr() {
    const Deferred d = g_deferred;
    switch (d.kind) {
        case DeferredError::None: break;
        case DeferredError::BlockNotAllocated:
            g_last_error = "Block " + std::to_string(d.a) + " is not allocated";
            break;
        case DeferredError::StaleHandle:
            g_last_error = "Stale handle: block " + std::to_string(d.a) + " was freed (gen " + std::to_string(d.b) +
                           ", current " + std::to_string(d.c) + ")";
            break;
        case DeferredError::OutOfBlocks:
            g_last_error = "Out of blocks: requested " + std::to_string(d.a) + ", available " + std::to_string(d.b);
            break;
    }
    g_deferred.kind = DeferredError::None;
    return g_last_error.c_str();
}
}  // namespace zk

extern "C" const char *zk_last_error(void) { return zk::last_error_cstr(); }
extern "C" int zk_abi_version(void) { return ZK_ABI_VERSION; }
