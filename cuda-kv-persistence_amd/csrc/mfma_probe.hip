// Matrix-core ceiling probe (measurement only, not part of the attention
// API): the dense bf16 rate the MI355X sustains when every SIMD streams
// nothing but v_mfma_f32_32x32x16_bf16 with the occupancy of the attention
// kernel (two 256-thread workgroups per CU, two waves per SIMD, four
// independent accumulator chains per wave on pseudo-random operands, no
// memory traffic in the loop).
// The board's power limit lowers the shader clock under such a load, so
// this rate lies below the published peak (2.4 GHz x 4096 flop/CU/clk);
// bench.py reports the attention kernel's rate against both.
//
// Built as its own library (lib/libkvpprobe.so), loaded by bench.py only.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;

// Operands: 8 A and 8 B fragments of pseudo-random bf16 values in [-2, 2)
// per lane, cycled through so that every MFMA multiplies fresh data (the
// datapath's switching activity, and so its power, is that of real inputs,
// not of constant operands).
__device__ __forceinline__ unsigned probe_hash(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

__global__ __launch_bounds__(256, 2) void mfma_probe_kernel(float* out, int iters) {
    const unsigned id = blockIdx.x * blockDim.x + threadIdx.x;
    bf16x8 a[8], b[8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned h = probe_hash(id * 131u + (unsigned)(r * 8 + i));
            a[r][i] = (__bf16)((float)(h & 0xffffu) * (4.0f / 65536.0f) - 2.0f);
            b[r][i] = (__bf16)((float)(h >> 16) * (4.0f / 65536.0f) - 2.0f);
        }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; it += 8) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r], b[r], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[r], b[(r + 1) & 7], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(r + 2) & 7], b[r], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(r + 3) & 7], b[(r + 5) & 7], c3, 0, 0,
                                                         0);
        }
    }
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) s += c0[v] + c1[v] + c2[v] + c3[v];
    out[(size_t)id] = s;
}

}  // namespace

extern "C" {

// Runs `reps` timed launches of the probe after one warm-up launch, each
// launch `iters` loop trips on 2 x CU workgroups; returns the median rate
// in *tflops (dense bf16 TFLOP/s) and its launch time in *ms. 0 on success.
int kvpprobe_mfma_bf16(int iters, int reps, double* tflops, double* ms) {
    if (iters <= 0 || reps <= 0 || !tflops || !ms) return 1;
    iters = (iters + 7) / 8 * 8;  // the loop runs 8 trips at a time
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
        return 1;
    const int grid = 2 * prop.multiProcessorCount;
    float* out = nullptr;
    if (hipMalloc(&out, (size_t)grid * 256 * sizeof(float)) != hipSuccess) return 1;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 0;
    std::vector<double> t;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) rc = 1;
    for (int r = 0; rc == 0 && r <= reps; ++r) {
        float el = 0.f;
        if (hipEventRecord(e0, nullptr) != hipSuccess) rc = 1;
        hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)grid), dim3(256), 0, nullptr, out,
                           iters);
        if (hipGetLastError() != hipSuccess || hipEventRecord(e1, nullptr) != hipSuccess ||
            hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&el, e0, e1) != hipSuccess)
            rc = 1;
        if (r > 0) t.push_back(el);  // launch 0 warms the clock up
    }
    if (rc == 0) {
        std::sort(t.begin(), t.end());
        const double med = t[t.size() / 2];
        const double flops = (double)grid * 4 /* waves */ * iters * 4 /* chains */ * 32768.0;
        *ms = med;
        *tflops = flops / (med * 1e-3) / 1e12;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(out);
    return rc;
}

}  // extern "C"
