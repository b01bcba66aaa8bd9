// bench_native.hip -- measurement helpers for bench.py (bin/gncx_bench_native.so).
//
// Two things a Python timing loop cannot give:
//   gncx_bench_read_loop     the read ceiling of a weight matrix: plain
//                            streaming reads of the same rotated buffers the
//                            GEMV is timed on, in the GEMV's own row pattern
//                            and in the fastest pattern found (grid stride);
//   gncx_bench_matvec_loop   back-to-back gncx_xfold_universal_matvec calls
//                            issued from native code, as an integrating C/C++
//                            caller (or LuaJIT's FFI) issues them, timed by
//                            the wall clock around the loop.
// Nothing here is on the product path; it links against gncx_llm_core.so like
// any other caller of the library.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstddef>
#include <cstdint>

#include "../../include/gncx_llm_core.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// The GEMV's row pattern: work-group b of G reads rows b, b + G, ...; lane l
// of a wave reads the row's 16-byte chunks l, l + 64, ... (all J of them at
// once); one row per wave in flight.  A chunk past the row re-reads the row's
// first chunk, so every load is unconditional.
template <int J>
__global__ __launch_bounds__(1024) void read_rows_kernel(const uint8_t* __restrict w, uint32_t rb, int32_t n,
                                                          uint32_t* __restrict sink) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int32_t g = gridDim.x;
    const int32_t rows_here = (n - static_cast<int32_t>(blockIdx.x) + g - 1) / g;
    const size_t total16 = (static_cast<size_t>(rb) * static_cast<size_t>(n)) / 16;
    u32x4 acc = {0, 0, 0, 0};
    for (int32_t li = wv; li < rows_here; li += nw) {
        const size_t row = static_cast<size_t>(li) * g + blockIdx.x;
        const size_t c0 = row * rb / 16, c1 = (row * rb + rb + 15) / 16;
        u32x4 a[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            size_t c = c0 + static_cast<size_t>(lane) + 64u * j;
            if (c >= c1 || c >= total16) c = c0;
            a[j] = ld16(w + 16 * c);
        }
#pragma unroll
        for (int j = 0; j < J; ++j) acc ^= a[j];
    }
    const uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (v == 0x9e3779b9u) sink[blockIdx.x & 1023] = v;  // keeps the loads; practically never taken
}

// Grid stride: thread t reads 16-byte chunks t, t + T, ... (T = all threads).
__global__ __launch_bounds__(1024) void read_stride_kernel(const uint8_t* __restrict w, size_t bytes,
                                                            uint32_t* __restrict sink) {
    const size_t n16 = bytes / 16;
    u32x4 acc = {0, 0, 0, 0};
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        acc ^= ld16(w + 16 * i);
    const uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (v == 0x9e3779b9u) sink[blockIdx.x & 1023] = v;
}

uint32_t* g_sink = nullptr;

hipError_t launch_read(const uint8_t* w, size_t bytes, uint32_t row_bytes, int32_t pattern, hipStream_t s) {
    if (pattern == 0) {
        hipLaunchKernelGGL(read_stride_kernel, dim3(512), dim3(1024), 0, s, w, bytes, g_sink);
        return hipGetLastError();
    }
    if (row_bytes < 16 || bytes % row_bytes != 0) return hipErrorInvalidValue;
    const int32_t n = static_cast<int32_t>(bytes / row_bytes);
    const uint32_t chunks = row_bytes / 16 + 2;  // a row may straddle one more chunk at each end
    const dim3 grid(n < 256 ? n : 256), block(1024);
    if (chunks <= 192) hipLaunchKernelGGL((read_rows_kernel<3>), grid, block, 0, s, w, row_bytes, n, g_sink);
    else if (chunks <= 256) hipLaunchKernelGGL((read_rows_kernel<4>), grid, block, 0, s, w, row_bytes, n, g_sink);
    else if (chunks <= 448) hipLaunchKernelGGL((read_rows_kernel<7>), grid, block, 0, s, w, row_bytes, n, g_sink);
    else if (chunks <= 768) hipLaunchKernelGGL((read_rows_kernel<12>), grid, block, 0, s, w, row_bytes, n, g_sink);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Mean microseconds per launch of `steps` back-to-back plain reads of
// `bytes` at bufs[i % nbufs] (HIP events on `stream` around the loop, after
// 10 untimed launches).  pattern 0: grid stride (512 x 1024 threads);
// pattern 1: the GEMV's row pattern over rows of row_bytes.  Returns 0, or a
// HIP error code.
__attribute__((visibility("default"))) int gncx_bench_read_loop(const void* const* bufs, int32_t nbufs,
                                                                 size_t bytes, uint32_t row_bytes,
                                                                 int32_t pattern, int32_t steps, void* stream,
                                                                 float* us_out) {
    if (!bufs || nbufs <= 0 || steps <= 0 || !us_out) return static_cast<int>(hipErrorInvalidValue);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (!g_sink && (e = hipMalloc(&g_sink, 4096)) != hipSuccess) return static_cast<int>(e);
    for (int32_t i = 0; i < 10; ++i)
        if ((e = launch_read(static_cast<const uint8_t*>(bufs[i % nbufs]), bytes, row_bytes, pattern, s)) !=
            hipSuccess)
            return static_cast<int>(e);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) return static_cast<int>(e);
    float ms = 0.0f;
    e = hipEventRecord(e0, s);
    for (int32_t i = 0; e == hipSuccess && i < steps; ++i)
        e = launch_read(static_cast<const uint8_t*>(bufs[i % nbufs]), bytes, row_bytes, pattern, s);
    if (e == hipSuccess) e = hipEventRecord(e1, s);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (e != hipSuccess) return static_cast<int>(e);
    *us_out = ms * 1000.0f / static_cast<float>(steps);
    return 0;
}

// Wall-clock microseconds per call of `steps` back-to-back matvec calls from
// native code (weights rotated over ws[i % nw]; x, y and the weights in
// device memory), between two synchronisations of the library's stream.
// Returns 0, or the library's last status when a call failed.
__attribute__((visibility("default"))) int gncx_bench_matvec_loop(const uint8_t* const* ws, int32_t nw,
                                                                   int32_t type, const float* x, int32_t k,
                                                                   int32_t n, float* y, int32_t steps,
                                                                   double* us_out) {
    if (!ws || nw <= 0 || steps <= 0 || !us_out) return static_cast<int>(hipErrorInvalidValue);
    hipStream_t s = static_cast<hipStream_t>(gncx_hip_get_stream());
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return static_cast<int>(e);
    const auto t0 = std::chrono::steady_clock::now();
    for (int32_t i = 0; i < steps; ++i) gncx_xfold_universal_matvec(ws[i % nw], 0, type, x, nullptr, k, n, y, nullptr);
    e = hipStreamSynchronize(s);
    const auto t1 = std::chrono::steady_clock::now();
    if (e != hipSuccess) return static_cast<int>(e);
    const int st = gncx_hip_last_status();
    if (st != 0) return st;
    *us_out = std::chrono::duration<double, std::micro>(t1 - t0).count() / steps;
    return 0;
}

}  // extern "C"
