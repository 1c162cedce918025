// Error reporting and version query of the C ABI.
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"

namespace moe {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail_arg(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return MOE_EINVAL;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

namespace {
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRec> g_recs;
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
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

ProfScope::ProfScope(const char* name, hipStream_t s) : slot(-1), stream(s) {
  if (!g_prof_on) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  hipEvent_t a = take_event(), b = take_event();
  if (!a || !b) return;
  hipEventRecord(a, s);
  g_recs.push_back(ProfRec{name, a, b});
  slot = (int)g_recs.size() - 1;
}

ProfScope::~ProfScope() {
  if (slot < 0) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (slot < (int)g_recs.size()) hipEventRecord(g_recs[slot].b, stream);
}

}  // namespace moe

extern "C" int moe_prof_enable(int on) {
  std::lock_guard<std::mutex> lk(moe::g_prof_mu);
  if (on) {  // start a fresh recording; turning it off keeps the records for moe_prof_summary
    for (auto& r : moe::g_recs) {
      moe::g_pool.push_back(r.a);
      moe::g_pool.push_back(r.b);
    }
    moe::g_recs.clear();
  }
  moe::g_prof_on = on != 0;
  return 0;
}

extern "C" int moe_prof_summary(const char* kernel, int64_t* launches, double* total_ms) {
  std::lock_guard<std::mutex> lk(moe::g_prof_mu);
  int64_t n = 0;
  double tot = 0.0;
  for (auto& r : moe::g_recs) {
    if (kernel && strcmp(kernel, r.name) != 0) continue;
    if (hipEventSynchronize(r.b) != hipSuccess) return moe::check_launch("moe_prof_summary");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return moe::check_launch("moe_prof_summary");
    ++n;
    tot += ms;
  }
  if (launches) *launches = n;
  if (total_ms) *total_ms = tot;
  return 0;
}

extern "C" int moe_prof_kernel_name(int64_t i, char* buf, size_t len) {
  std::lock_guard<std::mutex> lk(moe::g_prof_mu);
  // i-th distinct kernel name in launch order; returns 0 when i is past the end
  std::vector<const char*> names;
  for (auto& r : moe::g_recs) {
    bool seen = false;
    for (auto* nm : names) seen = seen || strcmp(nm, r.name) == 0;
    if (!seen) names.push_back(r.name);
  }
  if (i < 0 || i >= (int64_t)names.size() || !buf || len == 0) return 0;
  strncpy(buf, names[i], len - 1);
  buf[len - 1] = '\0';
  return 1;
}

extern "C" const char* moe_version(void) { return "moe_mi355 0.1.0 (gfx950)"; }

extern "C" int moe_last_error(char* buf, size_t len) {
  if (!buf || len == 0) return (int)strlen(moe::g_last_error);
  strncpy(buf, moe::g_last_error, len - 1);
  buf[len - 1] = '\0';
  return (int)strlen(buf);
}
