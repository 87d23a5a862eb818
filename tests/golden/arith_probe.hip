// Raw results of gfx950's bf16 dot and matrix instructions on host-made
// inputs (test infrastructure: it pins the oracle's restatement of their
// accumulation, or_acc_step).  Every kernel is in bounds by construction:
// grid-stride loops bounded by n, one wave per MFMA test (grid = ntests).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// d[i] = c[i] + a[i].lo b[i].lo + a[i].hi b[i].hi  (v_dot2c_f32_bf16)
__global__ void dot2_kernel(const uint32_t* a, const uint32_t* b, const float* c, float* d, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        d[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a[i]), __builtin_bit_cast(bf16x2_t, b[i]),
                                               c[i], false);
}

// chain t: acc = c[t]; for j < len: acc = dot2(a[t][j], b[t][j], acc)  (one lane's dot-product chain)
__global__ void chain_kernel(const uint32_t* a, const uint32_t* b, const float* c, float* d, int n, int len) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < n; t += gridDim.x * blockDim.x) {
        float acc = c[t];
        for (int j = 0; j < len; j++)
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a[(size_t)t * len + j]),
                                                  __builtin_bit_cast(bf16x2_t, b[(size_t)t * len + j]), acc, false);
        d[t] = acc;
    }
}

// one wave per test: A [16][32], B [32][16] bf16 row-major, C, D [16][16] f32.
// Lane l: A row l % 16 and B column l % 16 at k = 8 (l / 16) + i; D[4 (l / 16) + r][l % 16].
__global__ void mfma_kernel(const uint16_t* A, const uint16_t* B, const float* C, float* D, int ntests) {
    const int t = blockIdx.x, l = threadIdx.x;
    if (t >= ntests || l >= 64) return;
    const uint16_t* a = A + (size_t)t * 512;
    const uint16_t* b = B + (size_t)t * 512;
    uint32_t aw[4], bw[4];
    for (int i = 0; i < 4; ++i) {
        const int k = 8 * (l / 16) + 2 * i;
        aw[i] = a[(l % 16) * 32 + k] | ((uint32_t)a[(l % 16) * 32 + k + 1] << 16);
        bw[i] = b[k * 16 + l % 16] | ((uint32_t)b[(k + 1) * 16 + l % 16] << 16);
    }
    f32x4_t acc;
    for (int r = 0; r < 4; ++r) acc[r] = C[(size_t)t * 256 + (4 * (l / 16) + r) * 16 + l % 16];
    const uint4 au = {aw[0], aw[1], aw[2], aw[3]}, bu = {bw[0], bw[1], bw[2], bw[3]};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, au), __builtin_bit_cast(bf16x8_t, bu),
                                                  acc, 0, 0, 0);
    for (int r = 0; r < 4; ++r) D[(size_t)t * 256 + (4 * (l / 16) + r) * 16 + l % 16] = acc[r];
}

extern "C" {
// device pointers; returns the hipError_t of the launch and synchronisation
int arith_dot2(const void* a, const void* b, const void* c, void* d, int n) {
    hipLaunchKernelGGL(dot2_kernel, dim3(1024), dim3(256), 0, 0, (const uint32_t*)a, (const uint32_t*)b,
                       (const float*)c, (float*)d, n);
    return (int)hipDeviceSynchronize();
}
int arith_chain(const void* a, const void* b, const void* c, void* d, int n, int len) {
    hipLaunchKernelGGL(chain_kernel, dim3((n + 255) / 256), dim3(256), 0, 0, (const uint32_t*)a, (const uint32_t*)b,
                       (const float*)c, (float*)d, n, len);
    return (int)hipDeviceSynchronize();
}
int arith_mfma(const void* A, const void* B, const void* C, void* D, int ntests) {
    hipLaunchKernelGGL(mfma_kernel, dim3(ntests), dim3(64), 0, 0, (const uint16_t*)A, (const uint16_t*)B,
                       (const float*)C, (float*)D, ntests);
    return (int)hipDeviceSynchronize();
}
}
