// runtime.hip — status strings, version, the device status word, test
// hooks and launch instrumentation.
//
// Reference: runtime/core.h:35-112 (lazy JIT compile + memo, lcpp_check).
// Here every kernel is compiled ahead of time for gfx950, so there is no JIT
// cache; the C ABI returns status codes instead of asserting, and the
// debug-stream check (commit, synchronize, assert) becomes lcpp_temp_status:
// synchronize, then read the status word the call's kernels wrote.
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace lcpp {
namespace {

struct Record {
    std::string name;
    hipEvent_t start, stop;
};
struct Aggregate {
    std::string name;
    uint64_t launches;
    double total_ms;
};

std::mutex g_mu;
std::atomic<bool> g_on{false};  // read on every launch without the lock
std::vector<Record> g_pending;
std::vector<Aggregate> g_agg;

struct Open {
    std::string name;
    hipEvent_t start, stop;
    hipStream_t stream;
};

// lcpp_test_set_lookback_fault: read by every launch that waits
std::atomic<uint32_t> g_withhold{0xFFFFFFFFu};
std::atomic<uint32_t> g_spin_limit{0};

}  // namespace

WaitCtl wait_ctl(uint32_t *status)
{
    const uint32_t lim = g_spin_limit.load(std::memory_order_relaxed);
    return WaitCtl{status, lim ? lim : kSpinLimit, g_withhold.load(std::memory_order_relaxed)};
}

LaunchScope::LaunchScope(const char *name, hipStream_t s) : rec(nullptr)
{
    if (!g_on.load(std::memory_order_relaxed)) return;
    Open *o = new Open{name, nullptr, nullptr, s};
    const bool ok = hipEventCreate(&o->start) == hipSuccess && hipEventCreate(&o->stop) == hipSuccess &&
                    hipEventRecord(o->start, s) == hipSuccess;
    if (!ok) {
        if (o->start) (void)hipEventDestroy(o->start);
        if (o->stop) (void)hipEventDestroy(o->stop);
        delete o;
        return;
    }
    rec = o;
}

LaunchScope::~LaunchScope()
{
    if (!rec) return;
    Open *o = static_cast<Open *>(rec);
    (void)hipEventRecord(o->stop, o->stream);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_pending.push_back(Record{o->name, o->start, o->stop});
    }
    delete o;
}

}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_version(void) { return LCPP_AMD_VERSION; }

extern "C" const char *lcpp_status_string(int status)
{
    switch (status) {
    case LCPP_OK: return "LCPP_OK";
    case LCPP_ERR_INVALID_ARG: return "LCPP_ERR_INVALID_ARG";
    case LCPP_ERR_TEMP_TOO_SMALL: return "LCPP_ERR_TEMP_TOO_SMALL";
    case LCPP_ERR_UNSUPPORTED_DTYPE: return "LCPP_ERR_UNSUPPORTED_DTYPE";
    case LCPP_ERR_HIP: return "LCPP_ERR_HIP";
    case LCPP_ERR_LOOKBACK_TIMEOUT: return "LCPP_ERR_LOOKBACK_TIMEOUT";
    case LCPP_ERR_SIZE_LIMIT: return "LCPP_ERR_SIZE_LIMIT";
    default: return "LCPP_ERR_UNKNOWN";
    }
}

extern "C" int lcpp_device_status_decode(uint32_t word)
{
    return (word & LCPP_DEVICE_STATUS_LOOKBACK_TIMEOUT) ? LCPP_ERR_LOOKBACK_TIMEOUT : LCPP_OK;
}

extern "C" int lcpp_stream_sync(void *stream)
{
    return hipStreamSynchronize(static_cast<hipStream_t>(stream)) == hipSuccess ? LCPP_OK : LCPP_ERR_HIP;
}

extern "C" int lcpp_temp_status(const void *temp, size_t temp_bytes, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!temp || temp_bytes < kStatusBytes) return lcpp_stream_sync(stream);
    uint32_t word = 0;
    if (hipMemcpyAsync(&word, temp, sizeof(word), hipMemcpyDeviceToHost, s) != hipSuccess) return LCPP_ERR_HIP;
    if (hipStreamSynchronize(s) != hipSuccess) return LCPP_ERR_HIP;
    return lcpp_device_status_decode(word);
}

namespace {
// dst |= the status word of the call that last used the temp buffer
__global__ void status_record_kernel(const uint32_t *status, uint32_t *dst)
{
    const uint32_t w = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (w) __hip_atomic_fetch_or(dst, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
}  // namespace

extern "C" int lcpp_temp_status_record(const void *temp, size_t temp_bytes, uint32_t *dst, void *stream)
{
    if (!dst) return LCPP_ERR_INVALID_ARG;
    if (!temp || temp_bytes < kStatusBytes) return LCPP_OK;  // that call keeps no status word
    hipStream_t s = static_cast<hipStream_t>(stream);
    LCPP_LAUNCH("status_record", s,
                status_record_kernel<<<1, 1, 0, s>>>(static_cast<const uint32_t *>(temp), dst));
    return hipGetLastError() == hipSuccess ? LCPP_OK : LCPP_ERR_HIP;
}

extern "C" int lcpp_test_set_lookback_fault(uint32_t withhold_tile, uint32_t spin_limit)
{
    g_withhold.store(withhold_tile, std::memory_order_relaxed);
    g_spin_limit.store(spin_limit, std::memory_order_relaxed);
    return LCPP_OK;
}

static void drop_pending_locked()
{
    for (auto &r : g_pending) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    g_pending.clear();
}

extern "C" int lcpp_profile_enable(int on)
{
    std::lock_guard<std::mutex> lk(g_mu);
    drop_pending_locked();
    g_agg.clear();
    g_on.store(on != 0, std::memory_order_relaxed);
    return LCPP_OK;
}

extern "C" int lcpp_profile_count(void)
{
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = 0;
    for (auto &r : g_pending) {
        float ms = 0.f;
        if (hipEventSynchronize(r.stop) != hipSuccess ||
            hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) {
            rc = LCPP_ERR_HIP;
            continue;
        }
        bool found = false;
        for (auto &a : g_agg)
            if (a.name == r.name) {
                a.launches += 1;
                a.total_ms += ms;
                found = true;
                break;
            }
        if (!found) g_agg.push_back(Aggregate{r.name, 1, ms});
    }
    drop_pending_locked();
    return rc ? rc : (int)g_agg.size();
}

extern "C" int lcpp_profile_get(int i, char *name, size_t name_cap, uint64_t *launches,
                                double *total_ms)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (i < 0 || (size_t)i >= g_agg.size()) return LCPP_ERR_INVALID_ARG;
    const Aggregate &a = g_agg[(size_t)i];
    if (name && name_cap) {
        size_t n = a.name.size() < name_cap - 1 ? a.name.size() : name_cap - 1;
        a.name.copy(name, n);
        name[n] = '\0';
    }
    if (launches) *launches = a.launches;
    if (total_ms) *total_ms = a.total_ms;
    return LCPP_OK;
}
