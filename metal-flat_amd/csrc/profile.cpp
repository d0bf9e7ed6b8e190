// SPDX-License-Identifier: Apache-2.0
// profile.cpp -- optional per-kernel-family timing with HIP events recorded on
// the launch stream. Disabled by default (no events, no overhead). Pending
// event pairs are resolved lazily when totals are read.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "kernels.hpp"

namespace mflat_amd {
namespace {

struct Pending { int fam; hipEvent_t a, b; };
struct Token { int fam; hipEvent_t a; };

std::atomic<int> gOn{0};
thread_local int tSuppressed = 0;   // > 0: this thread's launches are not timed
std::mutex gMu;
std::vector<Pending> gPending;
double gMs[kFamCount] = {0};
long long gCount[kFamCount] = {0};

void resolveLocked() {
    for (auto& pe : gPending) {
        float ms = 0.0f;
        if (hipEventSynchronize(pe.b) == hipSuccess && hipEventElapsedTime(&ms, pe.a, pe.b) == hipSuccess) {
            gMs[pe.fam] += ms;
            gCount[pe.fam] += 1;
        }
        (void)hipEventDestroy(pe.a);
        (void)hipEventDestroy(pe.b);
    }
    gPending.clear();
}

}  // namespace

void prof_begin(int fam, hipStream_t s, void** token) {
    *token = nullptr;
    if (!gOn.load(std::memory_order_relaxed) || tSuppressed) return;
    hipEvent_t a;
    if (hipEventCreate(&a) != hipSuccess) return;
    if (hipEventRecord(a, s) != hipSuccess) { (void)hipEventDestroy(a); return; }
    *token = new Token{fam, a};
}

void prof_end(void* token, hipStream_t s) {
    if (!token) return;
    Token* t = static_cast<Token*>(token);
    hipEvent_t b;
    if (hipEventCreate(&b) == hipSuccess) {
        if (hipEventRecord(b, s) == hipSuccess) {
            std::lock_guard<std::mutex> lk(gMu);
            gPending.push_back({t->fam, t->a, b});
            delete t;
            return;
        }
        (void)hipEventDestroy(b);
    }
    (void)hipEventDestroy(t->a);
    delete t;
}

void prof_enable(int on) { gOn.store(on ? 1 : 0, std::memory_order_relaxed); }

// The allocation-free entry point's launches create no timer events.
void prof_suppress(bool on) { tSuppressed += on ? 1 : -1; }

void prof_reset() {
    std::lock_guard<std::mutex> lk(gMu);
    resolveLocked();
    for (int i = 0; i < kFamCount; ++i) { gMs[i] = 0.0; gCount[i] = 0; }
}

int prof_read(const char* name, double* ms, long long* n) {
    static const char* kNames[kFamCount] = {"scan_filter", "scan_sample", "scan_retry", "select", "argmin",
                                            "norms",       "prep",        "ivf_scan",   "ivf_bound"};
    int fam = -1;
    for (int i = 0; i < kFamCount; ++i)
        if (name && std::strcmp(name, kNames[i]) == 0) fam = i;
    if (fam < 0) return -1;
    std::lock_guard<std::mutex> lk(gMu);
    resolveLocked();
    if (ms) *ms = gMs[fam];
    if (n) *n = gCount[fam];
    return 0;
}

}  // namespace mflat_amd
