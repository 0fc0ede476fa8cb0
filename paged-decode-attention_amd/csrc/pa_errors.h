// Error reporting shared by the library's translation units: the message of
// the last failing call on this thread (returned by pa_last_error) and small
// argument checks. Hidden symbols: not part of the exported C ABI.
#ifndef PA_ERRORS_H_
#define PA_ERRORS_H_

#include <stdint.h>

#define PA_HIDDEN __attribute__((visibility("hidden")))

// Records the formatted message and returns `code`.
PA_HIDDEN int pa_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns PA_OK.
PA_HIDDEN int pa_ok();
PA_HIDDEN const char *pa_error_message();

inline bool pa_aligned(const void *ptr, int a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

#endif  // PA_ERRORS_H_
