// Optional per-kernel timing with HIP events (g2v_profile_* in include/g2v.h).  When enabled,
// every kernel launch of the library is bracketed by two events recorded on the launch stream;
// g2v_profile_collect() waits for them and accumulates the elapsed time per kernel name.
#include <mutex>
#include <string.h>
#include <string>
#include <vector>

#include "../../include/g2v.h"
#include "g2v_internal.h"

namespace g2v {
namespace {

struct Pending {
    const char* name;
    hipEvent_t a, b;
};
struct Total {
    std::string name;
    long long launches = 0;
    double ms = 0.0;
};

std::mutex g_mu;
bool g_on = false;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_pool;
std::vector<Total> g_totals;

hipEvent_t get_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

}  // namespace

ProfMark::ProfMark(const char* name, hipStream_t s) : name_(name), s_(s), a_(nullptr) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_on) return;
    a_ = get_event();
    if (a_ && hipEventRecord(static_cast<hipEvent_t>(a_), s) != hipSuccess) {
        g_pool.push_back(static_cast<hipEvent_t>(a_));
        a_ = nullptr;
    }
}

ProfMark::~ProfMark() {
    if (!a_) return;
    std::lock_guard<std::mutex> lk(g_mu);
    hipEvent_t b = get_event();
    if (!b || hipEventRecord(b, s_) != hipSuccess) {
        g_pool.push_back(static_cast<hipEvent_t>(a_));
        if (b) g_pool.push_back(b);
        return;
    }
    g_pending.push_back(Pending{name_, static_cast<hipEvent_t>(a_), b});
}

}  // namespace g2v

using namespace g2v;

extern "C" {

int g2v_profile_enable(int on) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_on = on != 0;
    return G2V_OK;
}

int g2v_profile_reset(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& p : g_pending) {
        hipEventSynchronize(p.b);
        g_pool.push_back(p.a);
        g_pool.push_back(p.b);
    }
    g_pending.clear();
    g_totals.clear();
    return G2V_OK;
}

int g2v_profile_collect(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& p : g_pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.b) != hipSuccess || hipEventElapsedTime(&ms, p.a, p.b) != hipSuccess) ms = 0.0f;
        // a template kernel is named in parentheses at its launch: "(k<a, b>)" -> "k<a, b>"
        std::string nm(p.name);
        if (nm.size() >= 2 && nm.front() == '(' && nm.back() == ')') nm = nm.substr(1, nm.size() - 2);
        Total* t = nullptr;
        for (auto& x : g_totals)
            if (x.name == nm) { t = &x; break; }
        if (!t) {
            g_totals.push_back(Total{nm});
            t = &g_totals.back();
        }
        t->launches += 1;
        t->ms += ms;
        g_pool.push_back(p.a);
        g_pool.push_back(p.b);
    }
    g_pending.clear();
    return (int)g_totals.size();
}

int g2v_profile_entry(int i, char* name, int name_len, long long* launches, double* total_ms) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (i < 0 || i >= (int)g_totals.size()) return G2V_ERR_INVALID;
    if (name && name_len > 0) {
        strncpy(name, g_totals[i].name.c_str(), name_len - 1);
        name[name_len - 1] = 0;
    }
    if (launches) *launches = g_totals[i].launches;
    if (total_ms) *total_ms = g_totals[i].ms;
    return G2V_OK;
}

}  // extern "C"
