// The error slot of the C ABI: every entry point returns 0 or a nonzero code and leaves a message here.
#include <stdarg.h>
#include <stdio.h>

static thread_local char message[512];

void krn_set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(message, sizeof message, fmt, args);
  va_end(args);
}

extern "C" const char* krn_amd_last_error(void) { return message; }
