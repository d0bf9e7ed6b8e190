// SPDX-License-Identifier: Apache-2.0
// log.hpp -- process-wide diagnostics of the library (reference surface:
// include/metalflat/Log.h:15-31, c/include/mflat.h:55-74).
//
// The C ABI's handler type is stored as is: the engine reports through the
// exact function pointer and user value a caller registered, so there is no
// translation layer between the two. Level values are the ABI's
// (MFLAT_LOG_INFO .. MFLAT_LOG_OFF).
#pragma once

#include "../../include/mflat.h"

namespace mflat_amd {

// Route messages to `fn(level, msg, user)`; fn == nullptr selects stderr.
void logRoute(mflat_log_handler_t fn, void* user);
void logSetThreshold(mflat_log_level_t threshold);   // clamped to [INFO, OFF]
mflat_log_level_t logThreshold();

// True when a message of `level` would be delivered (cheap: one atomic load).
bool logWants(mflat_log_level_t level);
void logEmit(mflat_log_level_t level, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace mflat_amd

// Arguments are neither evaluated nor formatted below the threshold.
#define MFLAT_LOG_AT(lvl, ...) \
    do { if (::mflat_amd::logWants(lvl)) ::mflat_amd::logEmit(lvl, __VA_ARGS__); } while (0)
#define MFLAT_LOG_ERROR(...) MFLAT_LOG_AT(MFLAT_LOG_ERROR, __VA_ARGS__)
#define MFLAT_LOG_WARN(...)  MFLAT_LOG_AT(MFLAT_LOG_WARN, __VA_ARGS__)
#define MFLAT_LOG_INFO(...)  MFLAT_LOG_AT(MFLAT_LOG_INFO, __VA_ARGS__)
