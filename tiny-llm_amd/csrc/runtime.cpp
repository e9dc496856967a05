#include "runtime.h"

#include "kernels/kv_kernels.h"
#include "tiny_llm/hip_utils.h"
#include "tl_log.h"

#include <hip/hip_runtime_api.h>

#include <array>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <utility>

namespace tiny_llm {

// ------------------------------------------------------------------ log
namespace detail {
namespace log {
namespace {
Level level_from_env() {
    const char *s = std::getenv("TLLM_LOG_LEVEL");
    if (!s) return Level::WARN;
    const std::pair<const char *, Level> names[] = {
        {"trace", Level::TRACE}, {"debug", Level::DEBUG}, {"info", Level::INFO},
        {"warn", Level::WARN},   {"error", Level::ERROR}, {"critical", Level::CRITICAL},
        {"off", Level::OFF}};
    for (const auto &n : names)
        if (std::strcmp(s, n.first) == 0) return n.second;
    return Level::WARN;
}
std::atomic<int> g_level{-1};
const char      *level_name(Level l) {
    static const char *n[] = {"trace", "debug", "info", "warn", "error", "critical", "off"};
    return n[static_cast<int>(l)];
}
} // namespace

void set_level(Level level) { g_level.store(static_cast<int>(level)); }

Level level() {
    int l = g_level.load(std::memory_order_relaxed);
    if (l < 0) {
        l = static_cast<int>(level_from_env());
        g_level.store(l);
    }
    return static_cast<Level>(l);
}

void write(Level level, const char *fmt, ...) {
    char    buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    std::fprintf(stderr, "[tiny_llm] [%s] %s\n", level_name(level), buf);
}
} // namespace log
} // namespace detail

namespace detail {

int current_device() {
    int d = 0;
    HIP_CHECK(hipGetDevice(&d));
    return d;
}

int device_cus() {
    static std::mutex         mu;
    static std::map<int, int> cus;
    const int                 dev = current_device();
    std::lock_guard<std::mutex> lk(mu);
    auto                      it = cus.find(dev);
    if (it != cus.end()) return it->second;
    int v = 0;
    HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
    if (v <= 0) v = 256;
    cus[dev] = v;
    return v;
}

// ---------------------------------------------------------------- MetaRing
MetaRing::MetaRing(int slots) : slots_(static_cast<size_t>(slots)) {}

MetaRing::~MetaRing() {
    // kernels queued on callers' streams may still read the device slots
    (void)hipDeviceSynchronize();
    for (void *p : retired_dev_) (void)hipFree(p);
    for (void *p : retired_host_) (void)hipHostFree(p);
    for (auto &s : slots_) {
        if (s.ev) {
            (void)hipEventSynchronize(s.ev);
            (void)hipEventDestroy(s.ev);
        }
        if (s.host) (void)hipHostFree(s.host);
        if (s.dev) (void)hipFree(s.dev);
    }
}

void *MetaRing::begin(size_t bytes) {
    cur_ = (cur_ + 1) % static_cast<int>(slots_.size());
    Slot &s = slots_[static_cast<size_t>(cur_)];
    if (s.pending) {
        HIP_CHECK(hipEventSynchronize(s.ev));
        s.pending = false;
    }
    if (bytes == 0) bytes = 16;
    if (s.cap < bytes) grow(s, bytes);
    if (!s.ev) HIP_CHECK(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
    bytes_ = bytes;
    return s.host;
}

void MetaRing::grow(Slot &s, size_t bytes) {
    size_t cap = 4096;
    while (cap < bytes) cap <<= 1;
    void *host = nullptr, *dev = nullptr;
    HIP_CHECK(hipHostMalloc(&host, cap, hipHostMallocDefault));
    HIP_CHECK(hipMalloc(&dev, cap));
    // The old host buffer is idle (its copy completed: begin() waited on the
    // slot's event); the old device buffer may still be read by queued kernels.
    if (s.host) retired_host_.push_back(s.host);
    if (s.dev) retired_dev_.push_back(s.dev);
    s.host = host;
    s.dev = dev;
    s.cap = cap;
}

void MetaRing::reserve(size_t bytes) {
    for (auto &s : slots_) {
        if (s.pending) {
            HIP_CHECK(hipEventSynchronize(s.ev));
            s.pending = false;
        }
        if (s.cap < bytes) grow(s, bytes);
    }
}

void *MetaRing::commit(hipStream_t stream) {
    Slot &s = slots_[static_cast<size_t>(cur_)];
    HIP_CHECK(hipMemcpyAsync(s.dev, s.host, bytes_, hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipEventRecord(s.ev, stream));
    s.pending = true;
    return s.dev;
}

// --------------------------------------------------------------- Workspace
Workspace::~Workspace() {
    if (!retired_.empty() || !retired_cnt_.empty()) (void)hipDeviceSynchronize();
    for (float *p : retired_) (void)hipFree(p);
    if (ptr_) (void)hipFree(ptr_);
    for (int *p : retired_cnt_) (void)hipFree(p);
    if (cnt_) (void)hipFree(cnt_);
}

int *Workspace::counters(size_t n, hipStream_t stream) {
    if (n > cnt_cap_) {
        size_t cap = 1024;
        while (cap < n) cap <<= 1;
        int *p = nullptr;
        HIP_CHECK(hipMalloc(&p, cap * sizeof(int)));
        HIP_CHECK(hipMemsetAsync(p, 0, cap * sizeof(int), stream));
        if (cnt_) retired_cnt_.push_back(cnt_); // may still be counted in by queued kernels
        cnt_ = p;
        cnt_cap_ = cap;
    }
    return cnt_;
}

float *Workspace::get(size_t floats) {
    if (floats == 0) return ptr_;
    if (floats > cap_) {
        size_t cap = 1 << 16;
        while (cap < floats) cap <<= 1;
        float *p = nullptr;
        HIP_CHECK(hipMalloc(&p, cap * sizeof(float)));
        // kernels queued earlier may still use the old buffer: keep it until
        // the workspace goes (grow-only doubling keeps the total below 2x)
        if (ptr_) retired_.push_back(ptr_);
        ptr_ = p;
        cap_ = cap;
    }
    return ptr_;
}

// ----------------------------------------------------------- DeviceContext
void DeviceContext::claim(hipStream_t stream) {
    if (used && last_stream != stream) HIP_CHECK(hipStreamSynchronize(last_stream));
    last_stream = stream;
    used = true;
}

DeviceContext &DeviceContext::get(int device) {
    static std::mutex                                 mu;
    static std::map<int, std::unique_ptr<DeviceContext>> ctxs;
    std::lock_guard<std::mutex>                       lk(mu);
    auto                                             &p = ctxs[device];
    if (!p) p.reset(new DeviceContext());
    return *p;
}

// ---------------------------------------------------------------- profiling
namespace {
struct ProfState {
    std::mutex                                          mu;
    std::atomic<bool>                                   on{false};
    std::array<std::vector<std::pair<hipEvent_t, hipEvent_t>>, static_cast<size_t>(KernelId::Count)> done;
    std::array<hipEvent_t, static_cast<size_t>(KernelId::Count)> open{};
};
ProfState &prof() {
    static ProfState p;
    return p;
}
// Timing-only events: without the system-scope fence a record does not
// write back and invalidate the caches, which would stretch the kernel it
// brackets.
constexpr unsigned kTimingEventFlags = hipEventDisableSystemFence;
} // namespace

void profile_begin(KernelId id, hipStream_t stream) {
    ProfState &p = prof();
    if (!p.on.load(std::memory_order_relaxed)) return;
    std::lock_guard<std::mutex> lk(p.mu);
    hipEvent_t                  e;
    HIP_CHECK(hipEventCreateWithFlags(&e, kTimingEventFlags));
    HIP_CHECK(hipEventRecord(e, stream));
    p.open[static_cast<size_t>(id)] = e;
}

void profile_end(KernelId id, hipStream_t stream) {
    ProfState &p = prof();
    if (!p.on.load(std::memory_order_relaxed)) return;
    std::lock_guard<std::mutex> lk(p.mu);
    hipEvent_t                  start = p.open[static_cast<size_t>(id)];
    if (!start) return;
    hipEvent_t e;
    HIP_CHECK(hipEventCreateWithFlags(&e, kTimingEventFlags));
    HIP_CHECK(hipEventRecord(e, stream));
    p.done[static_cast<size_t>(id)].emplace_back(start, e);
    p.open[static_cast<size_t>(id)] = nullptr;
}

void profile_set(bool on) { prof().on.store(on); }

void profile_reset() {
    ProfState                  &p = prof();
    std::lock_guard<std::mutex> lk(p.mu);
    for (auto &v : p.done) {
        for (auto &pr : v) {
            (void)hipEventSynchronize(pr.second);
            (void)hipEventDestroy(pr.first);
            (void)hipEventDestroy(pr.second);
        }
        v.clear();
    }
    for (auto &o : p.open) {
        if (o) (void)hipEventDestroy(o);
        o = nullptr;
    }
}

bool profile_query(int id, double *total_ms, long long *launches) {
    if (id < 0 || id >= static_cast<int>(KernelId::Count)) return false;
    ProfState                  &p = prof();
    std::lock_guard<std::mutex> lk(p.mu);
    double                      tot = 0.0;
    for (auto &pr : p.done[static_cast<size_t>(id)]) {
        HIP_CHECK(hipEventSynchronize(pr.second));
        float ms = 0.0f;
        HIP_CHECK(hipEventElapsedTime(&ms, pr.first, pr.second));
        tot += ms;
    }
    *total_ms = tot;
    *launches = static_cast<long long>(p.done[static_cast<size_t>(id)].size());
    return true;
}

} // namespace detail
} // namespace tiny_llm
