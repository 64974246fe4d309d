// status.cpp -- thread-local last error of the C ABI: status code, the typed
// fields of the reference's ZealotError variants, and the message.
#include <string>

#include "zk_error.h"

namespace zk {
namespace {
// The BlockManager's rejections are part of normal scheduling (a full pool, a
// stale handle), so a typed error stores its code and fields only; the
// message is built when zk_last_error asks for it.
thread_local ErrorSnapshot g_err;

std::string build_message(const ErrorSnapshot &e) {
    const std::string a = std::to_string(e.fields[0]), b = std::to_string(e.fields[1]),
                      c = std::to_string(e.fields[2]);
    switch (e.kind) {  // Display strings of src/error.rs:4-37
        case ErrorKind::BlockAlreadyAllocated: return "Block " + a + " is already allocated";
        case ErrorKind::BlockNotAllocated: return "Block " + a + " is not allocated";
        case ErrorKind::OutOfBlocks: return "Out of blocks: requested " + a + ", available " + b;
        case ErrorKind::InvalidBlockSize: return "Invalid block size: " + a;
        case ErrorKind::StaleHandle:
            return "Stale handle: block " + a + " was freed (gen " + b + ", current " + c + ")";
        case ErrorKind::SequenceTooLong:
            return "Sequence too long: worst case needs " + a + " blocks, pool capacity is " + b;
        case ErrorKind::None: break;
    }
    return e.message;
}
}  // namespace

int set_error(int code, const std::string &msg) {
    g_err.code = code;
    g_err.kind = ErrorKind::None;
    g_err.fields[0] = g_err.fields[1] = g_err.fields[2] = 0;
    g_err.message = msg;
    g_err.built = true;
    return code;
}
int set_error_typed(int code, ErrorKind kind, uint64_t a, uint64_t b, uint64_t c) {
    g_err.code = code;
    g_err.kind = kind;
    g_err.fields[0] = a;
    g_err.fields[1] = b;
    g_err.fields[2] = c;
    g_err.built = false;
    return code;
}
void clear_error() { set_error(ZK_OK, ""); }
ErrorSnapshot save_error() { return g_err; }
int restore_error(const ErrorSnapshot &e) {
    g_err = e;
    return e.code;
}
const char *last_error_cstr() {
    if (!g_err.built) {
        g_err.message = build_message(g_err);
        g_err.built = true;
    }
    return g_err.message.c_str();
}
}  // namespace zk

extern "C" const char *zk_last_error(void) { return zk::last_error_cstr(); }

extern "C" int zk_last_error_detail(uint64_t fields[3]) {
    const zk::ErrorSnapshot &e = zk::g_err;
    if (fields) {
        fields[0] = e.fields[0];
        fields[1] = e.fields[1];
        fields[2] = e.fields[2];
    }
    return e.code;
}

extern "C" int zk_abi_version(void) { return ZK_ABI_VERSION; }
