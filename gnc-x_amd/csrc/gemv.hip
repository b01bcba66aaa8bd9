// gemv.hip -- decode GEMV over GGUF blocks for gfx950.
//
// y[n] = W[n x k] . x[k] with x first quantised to per-32 int8 blocks exactly
// as the reference does (csrc/gncx_llm_kernels.cpp:955-995), then integer
// block dots (v_dot4_i32_i8) with fp32 per-block scaling:
//   Q4_0  cpp:1362-1382   Q4_K  cpp:1383-1397 (+ dot cpp:1127-1205)
//   Q6_K  cpp:1398-1412 (+ dot cpp:1211-1321)   Q8_0  cpp:1413-1431
//   BF16  cpp:1432-1461 (fp32 activations, no quantisation)
//
// Layout of the work: every work-group first quantises x into LDS (the
// activation vector is at most 40960 values, 60 KB with its block records),
// then each wave owns whole rows.  A row is split into "slots" that map one
// lane to a fixed byte range of one block:
//   Q4_K  4 lanes per 144 B super-block: 16 B header + 32 B of nibbles each
//   Q6_K  4 lanes per 210 B super-block: (half, 16-group) -> 3 x 16 B + scales
//   Q4_0  1 lane per 18 B block,  Q8_0  1 lane per 34 B block,  BF16 16 B
// so consecutive lanes read consecutive bytes of the row (coalesced 16 B
// loads) and the only cross-lane step is one wave reduction per row.
#include <hip/hip_runtime.h>

#include "gncx_device.h"
#include "gncx_launch.h"
#include "gncx_slots.h"

namespace gncx {
namespace {

using namespace dev;

constexpr int kThreads = 256;  // 4 waves per work-group

template <int TYPE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t* __restrict w, size_t rbytes,
                                                        const float* __restrict x, int32_t k, int32_t n,
                                                        float* __restrict y) {
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t* q = reinterpret_cast<int8_t*>(lds);
    ActMeta* meta = reinterpret_cast<ActMeta*>(lds + k);
    if (TYPE != kBF16) {
        dev::quantize_block8(x, k / 32, threadIdx.x, kThreads, q, meta);
        __syncthreads();
    }
    const int lane = threadIdx.x & 63;
    const int32_t wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int32_t nwaves = gridDim.x * (kThreads / 64);
    int32_t slots;
    if (TYPE == kQ4_K || TYPE == kQ6_K) slots = (k / 256) * 4;
    else if (TYPE == kBF16) slots = (k + 7) / 8;
    else slots = k / 32;
    for (int32_t r = wave; r < n; r += nwaves) {
        const uint8_t* row = w + static_cast<size_t>(r) * rbytes;
        float acc = 0.0f;
        for (int32_t s = lane; s < slots; s += 64) {
            if (TYPE == kQ4_K) acc += slot_q4_k(row, s, q, meta);
            else if (TYPE == kQ6_K) acc += slot_q6_k(row, s, q, meta);
            else if (TYPE == kQ4_0) acc += slot_q4_0(row, s, q, meta);
            else if (TYPE == kQ8_0) acc += slot_q8_0(row, s, q, meta);
            else acc += slot_bf16(row, s, k, x);
        }
        acc = wave_sum(acc);
        if (lane == 0) y[r] = acc;
    }
}

__global__ __launch_bounds__(kThreads) void act_quant_kernel(const float* __restrict x, int32_t k,
                                                             int8_t* __restrict q, ActMeta* __restrict meta) {
    const int32_t row = blockIdx.y;
    const int32_t nb = k / 32;
    // blocks of this row handled by this work-group: 32 per group
    const int32_t b0 = blockIdx.x * (kThreads / 8);
    const int32_t nb_here = min(nb - b0, kThreads / 8);
    if (nb_here <= 0) return;
    dev::quantize_block8(x + static_cast<size_t>(row) * k + static_cast<size_t>(b0) * 32, nb_here,
                         threadIdx.x, kThreads, q + static_cast<size_t>(row) * k + static_cast<size_t>(b0) * 32,
                         meta + static_cast<size_t>(row) * nb + b0);
}

template <int TYPE>
hipError_t launch_gemv_t(const uint8_t* w, const float* x, int32_t k, int32_t n, float* y,
                         hipStream_t stream) {
    const size_t rb = row_bytes(TYPE, k);
    const size_t lds = TYPE == kBF16 ? 0 : static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta);
    const int32_t rows_per_group = kThreads / 64;
    int32_t groups = (n + rows_per_group - 1) / rows_per_group;
    if (groups > 2048) groups = 2048;
    hipLaunchKernelGGL(gemv_kernel<TYPE>, dim3(groups), dim3(kThreads), lds, stream, w, rb, x, k, n, y);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n, float* y,
                       hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (k <= 0 || k > kMaxGemvK) return hipErrorInvalidValue;
    if (type != kBF16 && (k % 32) != 0) return hipErrorInvalidValue;
    if ((type == kQ4_K || type == kQ6_K) && (k % 256) != 0) return hipErrorInvalidValue;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
    if ((xa & 15u) != 0) return hipErrorInvalidValue;
    if (type == kQ4_K || type == kBF16) {
        if ((wa & 15u) != 0 || (row_bytes(type, k) & 15u) != 0) return hipErrorInvalidValue;
    } else if ((wa & 3u) != 0) {
        return hipErrorInvalidValue;
    }
    switch (type) {
    case kQ4_0: return launch_gemv_t<kQ4_0>(w, x, k, n, y, stream);
    case kQ8_0: return launch_gemv_t<kQ8_0>(w, x, k, n, y, stream);
    case kQ4_K: return launch_gemv_t<kQ4_K>(w, x, k, n, y, stream);
    case kQ6_K: return launch_gemv_t<kQ6_K>(w, x, k, n, y, stream);
    case kBF16: return launch_gemv_t<kBF16>(w, x, k, n, y, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_act_quant(const float* x, int32_t rows, int32_t k, int8_t* q, ActMeta* meta,
                            hipStream_t stream) {
    if (rows <= 0 || k <= 0) return hipSuccess;
    if ((k % 32) != 0 || (reinterpret_cast<uintptr_t>(x) & 15u) != 0) return hipErrorInvalidValue;
    const int32_t nb = k / 32;
    const int32_t gx = (nb + kThreads / 8 - 1) / (kThreads / 8);
    hipLaunchKernelGGL(act_quant_kernel, dim3(gx, rows), dim3(kThreads), 0, stream, x, k, q, meta);
    return hipGetLastError();
}

}  // namespace gncx
