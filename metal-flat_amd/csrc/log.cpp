// SPDX-License-Identifier: Apache-2.0
// log.cpp -- owner of the log sink and threshold. Semantics follow the
// reference's src/Log.cpp:14-59: constant-initialised atomics, threshold test
// before formatting, a 1024-byte format buffer, the handler called
// synchronously without any library lock, "Off" never delivered.
#include "log.hpp"

#include <atomic>
#include <cstdarg>
#include <cstdio>

namespace mflat_amd {
namespace {

void stderrSink(LogLevel lvl, const char* msg, void*) {
    const char* tag = lvl == LogLevel::Error ? "error" : lvl == LogLevel::Warn ? "warn" : "info";
    std::fprintf(stderr, "[mflat] %s: %s\n", tag, msg);
}

std::atomic<LogHandler> gHandler{nullptr};
std::atomic<void*> gUser{nullptr};
std::atomic<int> gThreshold{static_cast<int>(LogLevel::Info)};

}  // namespace

void setLogHandler(LogHandler h, void* user) {
    gUser.store(user, std::memory_order_release);
    gHandler.store(h, std::memory_order_release);
}
void setLogLevel(LogLevel t) { gThreshold.store(static_cast<int>(t), std::memory_order_relaxed); }
LogLevel logLevel() { return static_cast<LogLevel>(gThreshold.load(std::memory_order_relaxed)); }

bool logEnabled(LogLevel lvl) {
    const int t = gThreshold.load(std::memory_order_relaxed);
    return t != static_cast<int>(LogLevel::Off) && static_cast<int>(lvl) >= t &&
           lvl != LogLevel::Off;
}

void logf(LogLevel lvl, const char* fmt, ...) {
    if (!logEnabled(lvl)) return;
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    const int n = std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (n < 0) return;
    if (LogHandler h = gHandler.load(std::memory_order_acquire)) {
        h(lvl, buf, gUser.load(std::memory_order_acquire));
        return;
    }
    stderrSink(lvl, buf, nullptr);
}

}  // namespace mflat_amd
