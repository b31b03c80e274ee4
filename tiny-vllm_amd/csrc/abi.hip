// C-ABI bookkeeping: the thread-local error message and the ABI version.
#include "common.h"

namespace tvllm {

namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace tvllm

extern "C" const char* tvllm_last_error(void) { return tvllm::g_error; }

extern "C" int tvllm_abi_version(void) { return 5; }

#ifndef TVLLM_SOURCE_HASH
#define TVLLM_SOURCE_HASH "unknown"
#endif

// Digest of the kernel sources this library was compiled from (set by the
// build script), so a loader can refuse a library older than its sources.
extern "C" const char* tvllm_source_hash(void) { return TVLLM_SOURCE_HASH; }
