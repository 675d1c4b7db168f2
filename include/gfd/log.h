#pragma once
// Compile-time levelled logging to stderr (same macro names and levels as
// include/gfd/log.h:15-29 of the reference):
//   0 silent, 1 errors, 2 info + errors (default), 3 debug.
// Override with -DGFD_LOG_LEVEL=N.
#include <cstdio>

#ifndef GFD_LOG_LEVEL
#define GFD_LOG_LEVEL 2
#endif

#define GFD_LOG_ERROR(...)                                                     \
    do {                                                                       \
        if (GFD_LOG_LEVEL >= 1) std::fprintf(stderr, "[GFD ERROR] " __VA_ARGS__); \
    } while (0)

#define GFD_LOG_INFO(...)                                                      \
    do {                                                                       \
        if (GFD_LOG_LEVEL >= 2) std::fprintf(stderr, "[GFD] " __VA_ARGS__);    \
    } while (0)

#define GFD_LOG_DEBUG(...)                                                     \
    do {                                                                       \
        if (GFD_LOG_LEVEL >= 3) std::fprintf(stderr, "[GFD DBG] " __VA_ARGS__); \
    } while (0)
