// SPDX-License-Identifier: Apache-2.0
// log.cpp -- the library's message router.
//
// ABI-visible behaviour (c/include/mflat.h:55-74): one process-wide
// destination and threshold; a NULL handler means stderr; a message below the
// threshold costs one atomic load and is never formatted; MFLAT_LOG_OFF is a
// threshold, never a message level; the handler runs on the logging thread.
//
// Design: the (handler, user) pair is one record guarded by a reader/writer
// lock, so a message is always delivered to a handler together with the user
// value registered with it, even while another thread re-registers. The record
// is copied under the shared lock and the handler is called after the lock is
// released (a handler may itself log or re-register without deadlock).
// Messages are formatted to their full length: a short message uses a stack
// buffer, a longer one is measured and formatted into a heap string.
#include "log.hpp"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <shared_mutex>
#include <string>

namespace mflat_amd {
namespace {

struct Destination {
    mflat_log_handler_t fn = nullptr;
    void* user = nullptr;
};

class Router {
public:
    void route(mflat_log_handler_t fn, void* user) {
        std::unique_lock<std::shared_mutex> lk(mu_);
        dest_.fn = fn;
        dest_.user = user;
    }
    Destination destination() const {
        std::shared_lock<std::shared_mutex> lk(mu_);
        return dest_;
    }
    std::atomic<int> threshold{MFLAT_LOG_INFO};

private:
    mutable std::shared_mutex mu_;
    Destination dest_;
};

Router& router() {
    static Router r;   // constructed on first use; lives until exit
    return r;
}

const char* levelName(mflat_log_level_t l) {
    static const char* const kNames[] = {"info", "warn", "error"};
    const int i = static_cast<int>(l);
    return (i >= 0 && i < 3) ? kNames[i] : "?";
}

void deliver(mflat_log_level_t level, const char* text) {
    const Destination d = router().destination();
    if (d.fn) {
        d.fn(level, text, d.user);
        return;
    }
    // one stdio call per line, so concurrent messages do not interleave
    std::string line = "[mflat] ";
    line += levelName(level);
    line += ": ";
    line += text;
    line += '\n';
    std::fputs(line.c_str(), stderr);
}

}  // namespace

void logRoute(mflat_log_handler_t fn, void* user) { router().route(fn, user); }

void logSetThreshold(mflat_log_level_t t) {
    int v = static_cast<int>(t);
    v = v < MFLAT_LOG_INFO ? MFLAT_LOG_INFO : (v > MFLAT_LOG_OFF ? MFLAT_LOG_OFF : v);
    router().threshold.store(v, std::memory_order_relaxed);
}

mflat_log_level_t logThreshold() {
    return static_cast<mflat_log_level_t>(router().threshold.load(std::memory_order_relaxed));
}

bool logWants(mflat_log_level_t level) {
    const int lv = static_cast<int>(level);
    return lv < MFLAT_LOG_OFF && lv >= router().threshold.load(std::memory_order_relaxed);
}

void logEmit(mflat_log_level_t level, const char* fmt, ...) {
    if (!logWants(level)) return;
    char small[256];
    va_list ap, again;
    va_start(ap, fmt);
    va_copy(again, ap);
    const int len = std::vsnprintf(small, sizeof small, fmt, ap);
    va_end(ap);
    if (len < 0) {   // encoding error: nothing sensible to deliver
        va_end(again);
        return;
    }
    if (static_cast<size_t>(len) < sizeof small) {
        va_end(again);
        deliver(level, small);
        return;
    }
    std::string big(static_cast<size_t>(len) + 1, '\0');
    std::vsnprintf(&big[0], big.size(), fmt, again);
    va_end(again);
    big.resize(static_cast<size_t>(len));
    deliver(level, big.c_str());
}

}  // namespace mflat_amd
