// Shared helpers of the paged KV-cache library: per-thread error text.
#pragma once

#include <cstdarg>
#include <cstdio>

#include "parakeet_paged.h"

namespace pk {

// Records a message for pk_last_error() on the calling thread and returns `code`.
int fail(int code, const char* fmt, ...);
void clear_error();

}  // namespace pk
