// Host-side internals shared by the C-ABI glue and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/ming_hip.h"

namespace ming {
// Device memory owned by a context or model; grows on demand.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    hipError_t ensure(size_t n) {
        if (n <= bytes) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
        hipError_t e = hipMalloc(&p, n);
        if (e == hipSuccess) bytes = n;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};
}  // namespace ming

struct ming_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;     // own_stream or a borrowed one
    std::string err;
    int32_t* dev_flags = nullptr;     // [0] device-side error flag (spin timeout)
    int num_cus = 0;
    size_t max_lds = 0;
    bool alive = false;
    ming::DevBuf part;                // attention partials of ming_lm_layer
    ming::DevBuf qstage;              // staged activations of ming_qgemm
    bool timeout_seen = false;        // ming_sync saw the device error flag
};

namespace ming {

int set_err(ming_ctx* ctx, int status, const std::string& msg);
int hip_check(ming_ctx* ctx, hipError_t e, const char* what);

// ---- launchers (return hipError_t of the launch) ----
hipError_t launch_qgemv(hipStream_t st, int M, const uint16_t* x, const uint32_t* w, const uint16_t* s,
                        const uint16_t* b, int N, int K, float gscale, uint16_t* y_bf16, float* y_f32);
hipError_t launch_dequantize(hipStream_t st, const uint32_t* w, const uint16_t* s, const uint16_t* b, int64_t N,
                             int64_t K, float gscale, uint16_t* out);
hipError_t launch_quantize(hipStream_t st, const uint16_t* w, int64_t N, int64_t K, uint32_t* wq, uint16_t* s,
                           uint16_t* b);
// Batched 4-bit GEMM on MFMA: stage X [M][K] (K % 64 == 0) into xs [Mp][K/8] and
// xsum [Mp][K/64] (Mp = M rounded up to 16), then Y = g * X W^T for M <= 64.
hipError_t launch_qgemm_stage(hipStream_t st, const uint16_t* x, int M, int K, uint4* xs, float* xsum);
hipError_t launch_qgemm(hipStream_t st, const uint4* xs, const float* xsum, int M, int N, int K, const uint32_t* w,
                        const uint16_t* s, const uint16_t* b, float gscale, uint16_t* y, float* yf);

}  // namespace ming
