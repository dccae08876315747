// Thread-local error text shared by libaegkv's translation units
// (read back through aegkv_last_error()). Internal to the library.
#ifndef AEGKV_ERRORS_H
#define AEGKV_ERRORS_H

// Records a printf-style message for the calling thread and returns `code`.
__attribute__((visibility("hidden"))) int aegkv_set_error(int code, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));
// Clears the calling thread's message.
__attribute__((visibility("hidden"))) void aegkv_clear_error();

#endif  // AEGKV_ERRORS_H
