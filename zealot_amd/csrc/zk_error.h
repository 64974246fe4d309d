// zk_error.h -- the C ABI's thread-local last error (no HIP dependency, so
// the host-only BlockManager builds with any C++ compiler).
#pragma once

#include <cstdint>
#include <string>

#include "../../include/zealot_kv.h"

namespace zk {

// ------------------------------------------------------------------ errors
// Thread-local last error (zk_last_error / zk_last_error_detail); set_error
// returns the code so call sites read `return set_error(ZK_ERR_..., "...")`.
int set_error(int code, const std::string &msg);
// A ZealotError variant with fields (src/error.rs:4-37): the fields are kept
// for zk_last_error_detail and the Display message is built from them only
// when zk_last_error is called.  Fields: BlockAlreadyAllocated /
// BlockNotAllocated / InvalidBlockSize {value}; OutOfBlocks {requested,
// available}; StaleHandle {block_id, handle_gen, current_gen};
// SequenceTooLong {required, capacity}.
enum class ErrorKind {
    None,
    BlockAlreadyAllocated,
    BlockNotAllocated,
    OutOfBlocks,
    InvalidBlockSize,
    StaleHandle,
    SequenceTooLong
};
int set_error_typed(int code, ErrorKind kind, uint64_t a, uint64_t b = 0, uint64_t c = 0);
void clear_error();
// The whole last-error state, so a caller that must clean up (calling
// functions that may fail in turn) can re-raise the original error unchanged.
struct ErrorSnapshot {
    int code = ZK_OK;
    ErrorKind kind = ErrorKind::None;
    uint64_t fields[3] = {0, 0, 0};
    std::string message;
    bool built = true;  // message holds the text (typed errors build it lazily)
};
ErrorSnapshot save_error();
int restore_error(const ErrorSnapshot &e);  // returns e.code

}  // namespace zk
