#pragma once

// Symbol visibility for the library's C entry points. The definition lives in the C header so C callers
// and C++ callers agree on it.
#include <rocmkernels_attention.h>
