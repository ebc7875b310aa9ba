// cm_runtime.hip -- library runtime: error reporting, per-device tables and workspace.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "cm_common.h"

namespace cm {

static thread_local char g_err[512] = "";

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(CM_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// ---------------------------------------------------------------- tables (host side)
// The activation functions in IEEE double with the C library's exp / erf / tanh, the
// formulas of vectorop_act.py:60-79 (the C++ model's act_fn, VectorOP.cpp:50-66), rounded
// half to even to Q8.8 and saturated (DataType.host_quantize, dtype.py:214-219).
static double act_value(int a, double x) {
    switch (a) {
    case 0: return x / (1.0 + std::exp(-x));
    case 1: return x * (0.5 * (1.0 + std::erf(x / std::sqrt(2.0))));
    default:
        return x * (0.5 * (1.0 + std::tanh(std::sqrt(2.0 / M_PI) * (x + 0.044715 * (x * x * x)))));
    }
}

void build_act_tables_full(int16_t (*full)[65536]) {
    for (int a = 0; a < 3; a++)
        for (int raw = -32768; raw < 32768; raw++) {
            double r = act_value(a, raw / 256.0) * 256.0;
            if (r != r) r = 0.0;
            if (r > 32767.0) r = 32767.0;
            if (r < -32768.0) r = -32768.0;
            full[a][raw + 32768] = (int16_t)std::nearbyint(r);
        }
}

// TAB[k] = round(2^16 * 2^(-k / 4096)) (vectorop_smx.py:29-34).
void build_smx_table(int32_t* tab) {
    for (int k = 0; k < 4096; k++) tab[k] = (int32_t)std::nearbyint(std::ldexp(std::exp2(-k / 4096.0), 16));
}

// The row-ops table image (rowops_spec.table_image, rowops_spec.py:605-616): words
// 0 .. 2047 two sigmoid entries {D[i] (24 bits) << 25 | T[i] (25 bits)} per 64-bit half,
// T[i] = round(2^24 / (1 + exp(-i / 256))) (rowops_spec.py:337-343); then 8192 rsqrt
// entries y0[i] = round(2^47 / sqrt((i + 0.5) 2^19)) for i >= 2048 (rowops_spec.py:92-102).
void build_rowops_table_image(uint8_t* img) {
    std::memset(img, 0, 65536);
    std::vector<int64_t> T(4097);
    for (int i = 0; i <= 4096; i++) T[i] = (int64_t)std::rint(std::ldexp(1.0, 24) / (1.0 + std::exp(-i / 256.0)));
    for (int i = 0; i < 4096; i++) {
        uint64_t d = (uint64_t)(T[i + 1] - T[i]) & 0xFFFFFF, t = (uint64_t)T[i] & 0x1FFFFFF;
        uint64_t v = (d << 25) | t;
        std::memcpy(img + 8 * i, &v, 8);
    }
    for (int i = 2048; i < 8192; i++) {
        double y = std::rint(std::ldexp(1.0, 47) / std::sqrt((i + 0.5) * 524288.0));
        uint32_t u = (uint32_t)(y > 4294967295.0 ? 4294967295.0 : y);
        std::memcpy(img + 32768 + 4 * i, &u, 4);
    }
}

// ---------------------------------------------------------------- per-device state
constexpr int kMaxDevices = 64;
static DeviceState g_states[kMaxDevices];
static std::mutex g_mu;

// Full activation tables (SiLU, GELU, GELU-tanh: f(x) at [x + 32768]) -> the compact form the
// VectorOP kernel reads, f(x) = max(x, 0) - d[|x|] with d a byte table of lens[a] entries,
// verified lossless over all 65 536 inputs; CM_EINVAL for a table without that form.
static int compact_act_tables(const int16_t (*full)[65536], uint8_t* compact, uint32_t* lens) {
    for (int a = 0; a < 3; a++) {
        uint32_t len = 0;
        for (int t = 0; t < 32768; t++) {
            int d = -(int)full[a][32768 - t];            // f(-t) = -d[t]
            if (d < 0 || d > 255) return fail(CM_EINVAL, "activation table %d: f(-%d) outside a byte", a, t);
            if (d != 0) len = (uint32_t)t + 1;
        }
        if (len > (uint32_t)kActTabBytes) return fail(CM_EINVAL, "activation table %d longer than %d", a, kActTabBytes);
        for (uint32_t t = 0; t < len; t++) compact[a * kActTabBytes + t] = (uint8_t)(-full[a][32768 - t]);
        for (int x = -32768; x < 32768; x++) {
            int ax = x < 0 ? -x : x;
            int want = (x > 0 ? x : 0) - ((uint32_t)ax < len ? compact[a * kActTabBytes + ax] : 0);
            if (want != full[a][x + 32768])
                return fail(CM_EINVAL, "activation table %d is not max(x,0) - d[|x|] at %d", a, x);
        }
        lens[a] = len;
    }
    return CM_OK;
}

static int prepare(DeviceState* st, int dev) {
    static int16_t full[3][65536];
    build_act_tables_full(full);
    std::vector<uint8_t> compact(3 * kActTabBytes, 0);
    int rc0 = compact_act_tables(full, compact.data(), st->act_len);
    if (rc0) return rc0;
    int32_t smx[4096];
    build_smx_table(smx);
    std::vector<uint8_t> img(65536);
    build_rowops_table_image(img.data());

    CM_HIP_CHECK(hipMalloc(&st->act_tab, 3 * kActTabBytes));
    CM_HIP_CHECK(hipMalloc(&st->smx_tab, sizeof(smx)));
    CM_HIP_CHECK(hipMalloc(&st->ro_tables, 65536));
    CM_HIP_CHECK(hipMalloc(&st->ro_pram, 4096 * 16));
    CM_HIP_CHECK(hipMemcpy(st->act_tab, compact.data(), compact.size(), hipMemcpyHostToDevice));
    CM_HIP_CHECK(hipMemcpy(st->smx_tab, smx, sizeof(smx), hipMemcpyHostToDevice));
    CM_HIP_CHECK(hipMemcpy(st->ro_tables, img.data(), 65536, hipMemcpyHostToDevice));
    CM_HIP_CHECK(hipMemset(st->ro_pram, 0, 4096 * 16));
    int cus = 0, lds_cu = 0, lds_blk = 0, lds_optin = 0;
    CM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    CM_HIP_CHECK(hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev));
    CM_HIP_CHECK(hipDeviceGetAttribute(&lds_blk, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    if (hipDeviceGetAttribute(&lds_optin, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess) {
        lds_optin = 0;                                   // not reported: the per-block limit stands
        (void)hipGetLastError();
    }
    st->cus = cus > 0 ? cus : 1;
    st->lds_per_cu = lds_cu > 0 ? (size_t)lds_cu : 65536;
    st->lds_per_block = std::min((size_t)std::max({lds_blk, lds_optin, 65536}), st->lds_per_cu);
    {
        int rc = prepare_softmax(st);
        if (rc) return rc;
        rc = gemm_scratch_setup(st);
        if (rc) return rc;
    }
    st->device = dev;
    st->ready = true;
    return CM_OK;
}

int state(DeviceState** out) {
    int dev = 0;
    CM_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(CM_EINVAL, "device %d beyond %d", dev, kMaxDevices);
    DeviceState* st = &g_states[dev];
    if (!st->ready) {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!st->ready) {
            int rc = prepare(st, dev);
            if (rc) return rc;
        }
    }
    *out = st;
    return CM_OK;
}

int state_ready(DeviceState** out) {
    int dev = 0;
    CM_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(CM_EINVAL, "device %d beyond %d", dev, kMaxDevices);
    DeviceState* st = &g_states[dev];
    if (!st->ready) return fail(CM_EINVAL, "device %d not initialised: call cm_init on it first", dev);
    *out = st;
    return CM_OK;
}

int workspace(DeviceState* st, size_t bytes, void** out, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes > st->ws_size) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        CM_HIP_CHECK(hipStreamIsCapturing(s, &cap));
        if (cap != hipStreamCaptureStatusNone)
            return fail(CM_EINVAL, "workspace of %zu bytes needed while the stream captures a graph (%zu held): "
                                   "run the call once before the capture", bytes, st->ws_size);
        size_t sz = round_up(bytes, (size_t)1 << 21);
        void* p = nullptr;
        if (hipMalloc(&p, sz) != hipSuccess) {
            (void)hipGetLastError();
            return fail(CM_ENOMEM, "workspace of %zu bytes", sz);
        }
        // the old buffer stays allocated: queued work and captured graphs may still use it
        if (st->ws) st->ws_retired.push_back(st->ws);
        st->ws = p;
        st->ws_size = sz;
    }
    *out = st->ws;
    return CM_OK;
}

int take_workspace(DeviceState* st, const WsRegion* fixed, size_t bytes, void** out, hipStream_t s) {
    if (fixed == nullptr) return workspace(st, bytes, out, s);
    if (bytes > fixed->cap)
        return fail(CM_EINVAL, "the call needs %zu bytes of scratch; the no-allocation maximum is %zu", bytes, fixed->cap);
    *out = fixed->base;
    return CM_OK;
}

// ---------------------------------------------------------------- kernel timing
struct TimingRecord {
    const char* name;
    hipEvent_t start, stop;
};
static std::mutex g_tmu;
static bool g_timing = false;
static std::string g_select;          // record only this kernel name (empty: all)
static std::vector<TimingRecord> g_records;
static std::vector<hipEvent_t> g_free_events;

static hipEvent_t take_event() {
    if (!g_free_events.empty()) {
        hipEvent_t e = g_free_events.back();
        g_free_events.pop_back();
        return e;
    }
    // timing only: no system-scope fence (its cache writeback and invalidation would slow
    // the launches being timed and the ones after them)
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
    return e;
}

// On a stream under capture the pair becomes two event-record nodes of the graph, so every
// replay of the graph re-records them around the launch; otherwise a plain record.  The null
// stream is never captured; a refused query's error is cleared so that the launch check after
// it does not report it.
static unsigned record_flags(hipStream_t s) {
    if (s == nullptr) return 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return cs == hipStreamCaptureStatusActive ? hipEventRecordExternal : 0;
}

// Under capture the record is an event-record node added to the captured graph by hand, after
// the stream's current dependencies, which it then replaces (the stream-capture form of an
// external record, which not every HIP runtime accepts from hipEventRecordWithFlags).
static hipError_t record_event(hipEvent_t e, hipStream_t s, unsigned flags) {
    if (!flags) return hipEventRecord(e, s);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    hipGraph_t graph = nullptr;
    const hipGraphNode_t* deps = nullptr;
    size_t nd = 0;
    hipError_t r = hipStreamGetCaptureInfo_v2(s, &cs, &id, &graph, &deps, &nd);
    if (r != hipSuccess) return r;
    if (cs != hipStreamCaptureStatusActive || graph == nullptr) return hipErrorInvalidValue;
    hipGraphNode_t node = nullptr;
    r = hipGraphAddEventRecordNode(&node, graph, deps, nd, e);
    if (r != hipSuccess) return r;
    r = hipStreamUpdateCaptureDependencies(s, &node, 1, hipStreamSetCaptureDependencies);
    return r;
}

TimedLaunch::TimedLaunch(const char* name, hipStream_t s) : s_(s) {
    std::lock_guard<std::mutex> lk(g_tmu);
    if (!g_timing || (!g_select.empty() && g_select != name)) return;
    TimingRecord r{name, take_event(), take_event()};
    if (!r.start || !r.stop) return;
    flags_ = record_flags(s);
    if (record_event(r.start, s, flags_) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    g_records.push_back(r);
    slot_ = (int)g_records.size() - 1;
}

TimedLaunch::~TimedLaunch() {
    if (slot_ < 0) return;
    std::lock_guard<std::mutex> lk(g_tmu);
    if (slot_ < (int)g_records.size() && record_event(g_records[slot_].stop, s_, flags_) != hipSuccess)
        (void)hipGetLastError();
}

}  // namespace cm

extern "C" {

int cm_timing_enable(int on) {
    std::lock_guard<std::mutex> lk(cm::g_tmu);
    cm::g_timing = on != 0;
    return CM_OK;
}

int cm_timing_select(const char* kernel) {
    std::lock_guard<std::mutex> lk(cm::g_tmu);
    cm::g_select = kernel ? kernel : "";
    return CM_OK;
}

int cm_timing_reset(void) {
    std::lock_guard<std::mutex> lk(cm::g_tmu);
    for (auto& r : cm::g_records) {
        (void)hipEventSynchronize(r.stop);
        cm::g_free_events.push_back(r.start);
        cm::g_free_events.push_back(r.stop);
    }
    cm::g_records.clear();
    return CM_OK;
}

int cm_timing_read(const char* kernel, double* total_ms, uint64_t* launches) {
    std::lock_guard<std::mutex> lk(cm::g_tmu);
    double sum = 0.0;
    uint64_t n = 0;
    for (auto& r : cm::g_records) {
        if (std::strcmp(r.name, kernel) != 0) continue;
        CM_HIP_CHECK(hipEventSynchronize(r.stop));
        float ms = 0.f;
        CM_HIP_CHECK(hipEventElapsedTime(&ms, r.start, r.stop));
        sum += ms;
        n++;
    }
    if (total_ms) *total_ms = sum;
    if (launches) *launches = n;
    return CM_OK;
}

int cm_timing_read_each(const char* kernel, double* ms, uint64_t cap, uint64_t* launches) {
    std::lock_guard<std::mutex> lk(cm::g_tmu);
    uint64_t n = 0;
    for (auto& r : cm::g_records) {
        if (std::strcmp(r.name, kernel) != 0) continue;
        if (n < cap && ms != nullptr) {
            CM_HIP_CHECK(hipEventSynchronize(r.stop));
            float e = 0.f;
            CM_HIP_CHECK(hipEventElapsedTime(&e, r.start, r.stop));
            ms[n] = e;
        }
        n++;
    }
    if (launches) *launches = n;
    return CM_OK;
}

int cm_abi_version(void) { return 100; }

const char* cm_last_error(void) { return cm::g_err; }

int cm_init(void) {
    cm::DeviceState* st;
    return cm::state(&st);
}

// Host-side tables for tests: the full activation table (act 4..6) and the row-ops image.
int cm_host_act_table(int act, int16_t* out65536) {
    if (act < 4 || act > 6) return cm::fail(CM_EINVAL, "act %d is not a unit activation", act);
    static int16_t full[3][65536];
    cm::build_act_tables_full(full);
    std::memcpy(out65536, full[act - 4], sizeof(full[0]));
    return CM_OK;
}

int cm_host_rowops_table_image(uint8_t* out65536) {
    cm::build_rowops_table_image(out65536);
    return CM_OK;
}

}  // extern "C"

extern "C" int cm_act_table_init(const int16_t* tables) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (tables == nullptr) return fail(CM_EINVAL, "act tables: null");
    std::vector<uint8_t> compact(3 * kActTabBytes, 0);
    uint32_t lens[3];
    rc = compact_act_tables(reinterpret_cast<const int16_t (*)[65536]>(tables), compact.data(), lens);
    if (rc) return rc;
    CM_HIP_CHECK(hipMemcpy(st->act_tab, compact.data(), compact.size(), hipMemcpyHostToDevice));
    for (int a = 0; a < 3; a++) st->act_len[a] = lens[a];
    return CM_OK;
}

extern "C" int cm_rowops_tables_init(const void* img64k) {
    using namespace cm;
    DeviceState* st;
    int rc = state(&st);
    if (rc) return rc;
    if (img64k == nullptr) return fail(CM_EINVAL, "row-ops tables: null");
    CM_HIP_CHECK(hipMemcpy(st->ro_tables, img64k, 65536, hipMemcpyHostToDevice));
    return CM_OK;
}
