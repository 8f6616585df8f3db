// C ABI of the measurement-aid library (include/flat_diag.h): times the probe kernels of
// diag.hip on a stream of its own. Not part of the attention library.
#include <hip/hip_runtime.h>

#include "../../include/flat_diag.h"

namespace fa {
void launch_mfma_ceiling(bool f32, float* out, int blocks, int iters, int constant,
                         hipStream_t s);
void launch_stream_read(const void* buf, int64_t n_chunks, int depth, int blocks, uint32_t* out,
                        hipStream_t s);
}  // namespace fa

namespace {
constexpr int kOk = 0, kUnavailable = 20, kDtype = 29, kNull = 50, kHip = 60;

// ms per call of `run` on `s`: `warm` untimed calls, then `reps` timed ones.
template <typename F>
int time_calls(hipStream_t s, int warm, int reps, F run, double* ms) {
    for (int i = 0; i < warm; ++i) run();
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess) return kHip;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return kHip;
    }
    int rc = kOk;
    float t = 0.0f;
    if (hipEventRecord(e0, s) != hipSuccess) rc = kHip;
    for (int i = 0; rc == kOk && i < reps; ++i) run();
    if (rc == kOk && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                      hipEventElapsedTime(&t, e0, e1) != hipSuccess ||
                      hipGetLastError() != hipSuccess))
        rc = kHip;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms = (double)t / reps;
    return rc;
}

int open_device(int device, hipStream_t* s) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
        return kUnavailable;
    if (hipSetDevice(device) != hipSuccess) return kHip;
    return hipStreamCreateWithFlags(s, hipStreamNonBlocking) == hipSuccess ? kOk : kHip;
}
}  // namespace

extern "C" {

int fad_mfma_ceiling(int32_t device, int32_t dtype, int32_t constant_operands, double* tflops) {
    if (!tflops) return kNull;
    if (dtype != 2 && dtype != 0) return kDtype;
    hipStream_t s = nullptr;
    if (int rc = open_device(device, &s)) return rc;
    const bool f32 = dtype == 0;
    // ~2.5 ms per launch on 256 CUs either way (an f32 32x32x2 MFMA takes twice the bf16 one's
    // cycles for 1/8 of its work)
    constexpr int kBlocks = 2048;
    const int iters = f32 ? 500 : 4000;
    float* out = nullptr;
    if (hipMalloc(&out, (size_t)kBlocks * 256 * sizeof(float)) != hipSuccess) {
        (void)hipStreamDestroy(s);
        return kHip;
    }
    double ms = 0.0;
    // 400 untimed launches (~1 s: the clock settles under sustained load), 200 timed (~0.5 s)
    const int rc = time_calls(s, 400, 200, [&] {
        fa::launch_mfma_ceiling(f32, out, kBlocks, iters, constant_operands != 0, s);
    }, &ms);
    (void)hipStreamSynchronize(s);
    (void)hipFree(out);
    (void)hipStreamDestroy(s);
    if (rc) return rc;
    const double per_chain = f32 ? 4.0 * 4096.0 : 32768.0;
    const double flop = (double)kBlocks * 4 /* waves */ * iters * 4 /* chains */ * per_chain;
    *tflops = flop / (ms * 1e-3) / 1e12;
    return kOk;
}

int fad_stream_read(int32_t device, int32_t loads_in_flight, double* tbps) {
    if (!tbps) return kNull;
    if (loads_in_flight != 4 && loads_in_flight != 8 && loads_in_flight != 16) return kUnavailable;
    hipStream_t s = nullptr;
    if (int rc = open_device(device, &s)) return rc;
    int cus = 0;
    constexpr size_t kBytes = (size_t)4 << 30;  // 4 GiB, far beyond every cache level
    void* buf = nullptr;
    uint32_t* out = nullptr;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        hipMalloc(&buf, kBytes) != hipSuccess) {
        (void)hipStreamDestroy(s);
        return kHip;
    }
    if (hipMalloc(&out, (size_t)cus * 512 * sizeof(uint32_t)) != hipSuccess) {
        (void)hipFree(buf);
        (void)hipStreamDestroy(s);
        return kHip;
    }
    double ms = 0.0;
    // one workgroup of 8 waves per CU (the decode's occupancy), 100 untimed and 200 timed
    // passes (~0.2 s at 7 TB/s)
    const int rc = time_calls(s, 100, 200, [&] {
        fa::launch_stream_read(buf, (int64_t)(kBytes >> 15), loads_in_flight, cus, out, s);
    }, &ms);
    (void)hipStreamSynchronize(s);
    (void)hipFree(out);
    (void)hipFree(buf);
    (void)hipStreamDestroy(s);
    if (rc) return rc;
    *tbps = (double)kBytes / (ms * 1e-3) / 1e12;
    return kOk;
}

}  // extern "C"
