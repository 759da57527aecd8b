// common.h - host runtime helpers, the HIP counterparts of the reference's
// include/common.h:1-98: a throwing HIP_CHECK (reference CUDA_CHECK, :10-20), an
// event timer (GpuTimer, :35-63), a wall-clock timer (CpuTimer, :65-80) and scoped
// profiler ranges (NVTX_PUSH/POP, :82-98) backed by roctx, which rocprofv3
// --marker-trace records.
#pragma once

#include <hip/hip_runtime_api.h>

#include <chrono>
#include <iostream>
#include <sstream>
#include <stdexcept>

#define HIP_CHECK(call)                                                                  \
    do {                                                                                 \
        hipError_t hip_check_status_ = (call);                                           \
        if (hip_check_status_ != hipSuccess) {                                           \
            std::stringstream hip_check_ss_;                                             \
            hip_check_ss_ << "HIP error at " << __FILE__ << ":" << __LINE__ << " - "     \
                          << hipGetErrorString(hip_check_status_);                       \
            std::cerr << hip_check_ss_.str() << std::endl;                               \
            throw std::runtime_error(hip_check_ss_.str());                               \
        }                                                                                \
    } while (0)

// Event-pair timer on one stream.
struct GpuTimer {
    hipEvent_t start_event{}, stop_event{};

    GpuTimer() {
        HIP_CHECK(hipEventCreate(&start_event));
        HIP_CHECK(hipEventCreate(&stop_event));
    }
    ~GpuTimer() {
        (void)hipEventDestroy(start_event);
        (void)hipEventDestroy(stop_event);
    }
    GpuTimer(const GpuTimer&) = delete;
    GpuTimer& operator=(const GpuTimer&) = delete;

    void start(hipStream_t stream = nullptr) { HIP_CHECK(hipEventRecord(start_event, stream)); }
    void stop(hipStream_t stream = nullptr) { HIP_CHECK(hipEventRecord(stop_event, stream)); }
    float elapsed_ms() {
        HIP_CHECK(hipEventSynchronize(stop_event));
        float ms = 0.0f;
        HIP_CHECK(hipEventElapsedTime(&ms, start_event, stop_event));
        return ms;
    }
};

struct CpuTimer {
    std::chrono::high_resolution_clock::time_point t_start, t_stop;
    void start() { t_start = std::chrono::high_resolution_clock::now(); }
    void stop() { t_stop = std::chrono::high_resolution_clock::now(); }
    float elapsed_ms() const {
        return std::chrono::duration<float, std::milli>(t_stop - t_start).count();
    }
};

// Profiler ranges.  Define TCAMD_DISABLE_ROCTX to compile them out (and drop -lroctx64).
#if !defined(TCAMD_DISABLE_ROCTX)
#include <rocprofiler-sdk-roctx/roctx.h>
#define ROCTX_PUSH(name) roctxRangePushA(name)
#define ROCTX_POP() roctxRangePop()
#else
#define ROCTX_PUSH(name) ((void)0)
#define ROCTX_POP() ((void)0)
#endif

struct RoctxScopedRange {
    explicit RoctxScopedRange(const char* name) { ROCTX_PUSH(name); }
    ~RoctxScopedRange() { ROCTX_POP(); }
    RoctxScopedRange(const RoctxScopedRange&) = delete;
    RoctxScopedRange& operator=(const RoctxScopedRange&) = delete;
};
