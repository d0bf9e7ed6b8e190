// SPDX-License-Identifier: Apache-2.0
// log.hpp -- process-global log sink and threshold (reference
// include/metalflat/Log.h:15-31, src/Log_internal.h:21-26).
#pragma once

namespace mflat_amd {

enum class LogLevel : int { Info = 0, Warn = 1, Error = 2, Off = 3 };
using LogHandler = void (*)(LogLevel level, const char* msg, void* user);

void setLogHandler(LogHandler handler, void* user);   // nullptr restores stderr
void setLogLevel(LogLevel threshold);
LogLevel logLevel();

bool logEnabled(LogLevel level);
void logf(LogLevel level, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace mflat_amd

// The level test runs before the arguments are evaluated or formatted.
#define MFLAT_LOG_ERROR(...) do { if (::mflat_amd::logEnabled(::mflat_amd::LogLevel::Error)) \
    ::mflat_amd::logf(::mflat_amd::LogLevel::Error, __VA_ARGS__); } while (0)
#define MFLAT_LOG_WARN(...)  do { if (::mflat_amd::logEnabled(::mflat_amd::LogLevel::Warn)) \
    ::mflat_amd::logf(::mflat_amd::LogLevel::Warn, __VA_ARGS__); } while (0)
#define MFLAT_LOG_INFO(...)  do { if (::mflat_amd::logEnabled(::mflat_amd::LogLevel::Info)) \
    ::mflat_amd::logf(::mflat_amd::LogLevel::Info, __VA_ARGS__); } while (0)
