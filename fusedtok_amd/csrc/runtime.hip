// Runtime plumbing of the C ABI: thread-local error text, device
// properties, per-device scratch pool, device probe.
#include "ft_common.hpp"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <tuple>
#include <mutex>
#include <vector>

namespace ft {

namespace {
thread_local std::string g_last_error;

struct ScratchSlot {
    void* ptr = nullptr;
    size_t bytes = 0;
};

struct DeviceState {
    bool info_ready = false;
    DevInfo info;
    ScratchSlot slots[(int)Scratch::kCount];
};

std::mutex& state_mutex() {
    static std::mutex m;
    return m;
}

std::vector<DeviceState>& states() {
    static std::vector<DeviceState> s;
    return s;
}

int current_device() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    return dev;
}

DeviceState& state_for(int dev) {
    auto& s = states();
    if ((int)s.size() <= dev) s.resize(dev + 1);
    return s[dev];
}
}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

const DevInfo& dev_info() {
    const int dev = current_device();
    std::lock_guard<std::mutex> lock(state_mutex());
    DeviceState& st = state_for(dev);
    if (!st.info_ready) {
        int cus = 0;
        hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                                        dev),
                  "hipDeviceGetAttribute(multiProcessorCount)");
        st.info.id = dev;
        st.info.cu_count = cus > 0 ? cus : 256;
        st.info_ready = true;
    }
    return st.info;
}

namespace {
constexpr const char* kTuneNames[(int)Tune::kCount] = {
    "FT_ATTN_FORCE_GENERIC", "FT_ATTN_SEGS",       "FT_ATTN_MIN_SEG",
    "FT_ATTN_CHUNK",         "FT_QGEMM_KERNEL",    "FT_QGEMM_DEC_KW",
    "FT_QGEMM_DEC_REGS",     "FT_QGEMM_KSPLIT",    "FT_QGEMM_SK_REGS",
    "FT_QGEMM_SK_WAVES",     "FT_QGEMM_SK_STAGES",
    "FT_QGEMM_BIG",          "FT_QGEMM_BAND",      "FT_RMSQ_SPLIT",
    "FT_RMSQ_GEMV_SPLIT",    "FT_PREFILL_FORCE_GENERIC", "FT_ARG_SLICES",
    "FT_SMP_SINGLE",         "FT_SMP_SLICES",      "FT_FAIL_SCRATCH",
    "FT_PREFILL_PREPASS",    "FT_GRID_SYNC"};

// value and presence per switch: the environment's (read once), then the
// run-time override, which wins while set
struct TuneState {
    int env_val[(int)Tune::kCount] = {};
    bool env_set[(int)Tune::kCount] = {};
    std::atomic<int> val[(int)Tune::kCount];
    std::atomic<bool> set[(int)Tune::kCount];
};

TuneState& tune_state() {
    static TuneState st;
    static std::once_flag once;
    std::call_once(once, [] {
        for (int i = 0; i < (int)Tune::kCount; ++i) {
            const char* v = getenv(kTuneNames[i]);
            st.env_set[i] = v && *v;
            st.env_val[i] = st.env_set[i] ? atoi(v) : 0;
            st.val[i].store(st.env_val[i]);
            st.set[i].store(st.env_set[i]);
        }
    });
    return st;
}

int tune_index(const char* name) {
    if (!name) return -1;
    for (int i = 0; i < (int)Tune::kCount; ++i)
        if (strcmp(name, kTuneNames[i]) == 0) return i;
    return -1;
}
}  // namespace

int tune(Tune which, int dflt) {
    TuneState& st = tune_state();
    const int i = (int)which;
    return st.set[i].load(std::memory_order_relaxed) ? st.val[i].load(std::memory_order_relaxed)
                                                     : dflt;
}

bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(s, &status), "hipStreamIsCapturing");
    return status != hipStreamCaptureStatusNone;
}

namespace {
void* scratch_impl(Scratch which, size_t bytes, hipStream_t s, bool zero) {
    // test hook, checked before any HIP call so that a host without a
    // device reaches it too
    if (tune(Tune::FailScratch, 0))
        throw Error{FT_EHIP, "device scratch allocation: out of memory "
                             "(simulated by FT_FAIL_SCRATCH)"};
    const int dev = current_device();
    std::lock_guard<std::mutex> lock(state_mutex());
    ScratchSlot& slot = state_for(dev).slots[(int)which];
    if (slot.bytes >= bytes && slot.ptr) return slot.ptr;
    if (stream_capturing(s))
        throw Error{FT_EHIP,
                    "device scratch must grow outside a HIP graph capture: "
                    "run the shape once before capturing it"};
    // A grown slot's old buffer is retired, never freed: in-flight kernels
    // and HIP graphs captured earlier still hold its address. Growth is
    // geometric, so a process retires at most a few dozen buffers.
    size_t want = bytes < 4096 ? 4096 : bytes;
    if (slot.ptr && want < 2 * slot.bytes) want = 2 * slot.bytes;
    want = (want + 4095) & ~(size_t)4095;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        hip_fail("device scratch allocation", e);
    }
    if (zero) {
        e = hipMemsetAsync(p, 0, want, s);
        if (e != hipSuccess) {
            (void)hipFree(p);
            hip_fail("device scratch clear", e);
        }
    }
    slot.ptr = p;
    slot.bytes = want;
    return p;
}
}  // namespace

void* scratch(Scratch which, size_t bytes, hipStream_t s) {
    return scratch_impl(which, bytes, s, false);
}

void* scratch_zeroed(Scratch which, size_t bytes, hipStream_t s) {
    return scratch_impl(which, bytes, s, true);
}

GridMax gridmax_state(int nwg, hipStream_t s) {
    // the word, then the slots from byte 256; zeroed when (re)allocated, and
    // every launch leaves the arrivals at 0 (the generation keeps counting)
    char* p = (char*)scratch_zeroed(Scratch::GridSync, 256 + 4 * (size_t)(nwg > 0 ? nwg : 1), s);
    return GridMax{(unsigned long long*)p, (unsigned*)(p + 256)};
}

bool grid_resident(const void* kernel, int nwg, int threads, GridUse use) {
    const int off = tune(Tune::GridSync, 0);
    if (nwg < 1 || (off & 1) || (off & (int)use)) return false;
    const int dev = current_device();
    const int cus = dev_info().cu_count;
    static std::mutex mu;
    static std::map<std::tuple<int, const void*, int>, int> per_cu;
    int blocks = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        const auto key = std::make_tuple(dev, kernel, threads);
        auto it = per_cu.find(key);
        if (it == per_cu.end()) {
            hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, 0),
                      "hipOccupancyMaxActiveBlocksPerMultiprocessor");
            per_cu.emplace(key, blocks);
        } else {
            blocks = it->second;
        }
    }
    return (long long)blocks * cus >= nwg;
}

}  // namespace ft

extern "C" {

const char* ft_last_error(void) { return ft::g_last_error.c_str(); }

int ft_device_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n > 0 ? 1 : 0;
}

const char* ft_version(void) { return "0.1.0"; }

int ft_host_device_address(const void* host, void** dev) {
    return ft::guarded([&] {
        if (!host || !dev) ft::inval("host_device_address: null argument");
        *dev = nullptr;
        hipPointerAttribute_t at{};
        const hipError_t e = hipPointerGetAttributes(&at, host);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            ft::inval("host_device_address: not memory the HIP runtime knows");
        }
        if (at.type != hipMemoryTypeHost || !at.devicePointer)
            ft::inval("host_device_address: not pinned host memory mapped to the device");
        // the attributes may describe the allocation's base: keep the offset
        const size_t off = at.hostPointer ? (size_t)((const char*)host - (const char*)at.hostPointer)
                                          : 0;
        *dev = (char*)at.devicePointer + off;
    });
}

int ft_set_tuning(const char* name, int value) {
    return ft::guarded([&] {
        const int i = ft::tune_index(name);
        if (i < 0) ft::inval(std::string("unknown tuning switch: ") + (name ? name : "(null)"));
        ft::TuneState& st = ft::tune_state();
        st.val[i].store(value);
        st.set[i].store(true);
    });
}

int ft_clear_tuning(const char* name) {
    return ft::guarded([&] {
        const int i = ft::tune_index(name);
        if (i < 0) ft::inval(std::string("unknown tuning switch: ") + (name ? name : "(null)"));
        ft::TuneState& st = ft::tune_state();
        st.val[i].store(st.env_val[i]);
        st.set[i].store(st.env_set[i]);
    });
}

}  // extern "C"
