// tm_internal.h -- helpers shared by the library's translation units (not part of the ABI).
#ifndef TM_INTERNAL_H
#define TM_INTERNAL_H

// Records a formatted message for tm_last_error() (thread-local) and returns `code`.
__attribute__((visibility("hidden"))) int tm_internal_fail(int code, const char* fmt, ...);

#endif
