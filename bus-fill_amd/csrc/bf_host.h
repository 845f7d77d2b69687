// Host-side helpers shared by the library's plain C++ sources (the GGUF reader)
// and its HIP sources; no HIP types, so the reader builds without the HIP
// headers (the sanitizer build of the tests).
#pragma once

#include <stddef.h>

namespace bf {

// The calling thread's text for bf_last_error().
void set_last_error(const char* text);

// Copies n bytes of host memory to device memory on `stream` (a hipStream_t)
// and waits for the copy; false, with the error text set, on failure.
bool copy_to_device(void* dst, const void* src, size_t n, void* stream);

}  // namespace bf
