// Runtime plumbing of the C ABI: thread-local error text, device
// properties, per-device scratch pool, device probe.
#include "ft_common.hpp"

#include <cstdlib>
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

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(s, &status), "hipStreamIsCapturing");
    return status != hipStreamCaptureStatusNone;
}

namespace {
void* scratch_impl(Scratch which, size_t bytes, hipStream_t s, bool zero) {
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

}  // extern "C"
