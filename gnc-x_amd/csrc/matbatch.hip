// matbatch.hip -- batched prefill product Y[B x N] = Q8(X[B x K]) . W^T.
//
// Semantics of the reference's gncx_xfold_universal_matbatch
// (csrc/gncx_llm_kernels.cpp:1495-1692): every token row of X is quantised
// on its own to per-32 int8 blocks (cpp:1506-1510), then each output is the
// same integer block dot as the matvec; the output is row-major out[t*N + m].
//
// Baseline kernel: the activations are quantised once into the workspace,
// then a wave computes one (row, token) output with the GEMV slot dots.  The
// weight row is re-read per token from the caches.
#include <hip/hip_runtime.h>

#include "gncx_device.h"
#include "gncx_launch.h"
#include "gncx_slots.h"

namespace gncx {
namespace {

using namespace dev;

constexpr int kThreads = 256;

template <int TYPE>
__global__ __launch_bounds__(kThreads) void matbatch_rowtok_kernel(const uint8_t* __restrict w, size_t rbytes,
                                                                   const float* __restrict x,
                                                                   const int8_t* __restrict q,
                                                                   const ActMeta* __restrict meta, int32_t k,
                                                                   int32_t n, float* __restrict y) {
    const int lane = threadIdx.x & 63;
    const int32_t r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int32_t t = blockIdx.y;
    if (r >= n) return;
    const uint8_t* row = w + static_cast<size_t>(r) * rbytes;
    const int8_t* qt = q + static_cast<size_t>(t) * k;
    const ActMeta* mt = meta + static_cast<size_t>(t) * (k / 32);
    using S = Slot<TYPE>;
    const int32_t slots = S::slots(k);
    float acc = 0.0f;
    for (int32_t s = lane; s < slots; s += 64) {
        typename S::Frag f;
        typename S::Act a;
        S::load(f, PtrRow{row}, s);
        slot_act<TYPE>(a, s, qt, mt, x + static_cast<size_t>(t) * k);
        acc += S::dot(f, a, s);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(t) * n + r] = acc;
}

template <int TYPE>
hipError_t launch_t(const uint8_t* w, const float* x, int32_t b, int32_t k, int32_t n, float* y, int8_t* q,
                    ActMeta* meta, hipStream_t stream) {
    if (TYPE != kBF16) {
        hipError_t e = launch_act_quant(x, b, k, q, meta, stream);
        if (e != hipSuccess) return e;
    }
    dim3 grid((n + 3) / 4, b);
    hipLaunchKernelGGL(matbatch_rowtok_kernel<TYPE>, grid, dim3(kThreads), 0, stream, w, row_bytes(TYPE, k), x, q,
                       meta, k, n, y);
    return hipGetLastError();
}

}  // namespace

size_t matbatch_workspace_bytes(int32_t type, int32_t b, int32_t k) {
    if (type == kBF16) return 256;
    const size_t qbytes = (static_cast<size_t>(b) * k + 255) & ~static_cast<size_t>(255);
    return qbytes + static_cast<size_t>(b) * (k / 32) * sizeof(ActMeta) + 256;
}

hipError_t launch_matbatch(int32_t type, const uint8_t* w, const float* x, int32_t b, int32_t k, int32_t n,
                           float* y, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (b <= 0 || n <= 0) return hipSuccess;
    if (k <= 0 || b > 65535) return hipErrorInvalidValue;
    if (type != kBF16 && (k % 32) != 0) return hipErrorInvalidValue;
    if ((type == kQ4_K || type == kQ6_K) && (k % 256) != 0) return hipErrorInvalidValue;
    if (workspace_bytes < matbatch_workspace_bytes(type, b, k)) return hipErrorInvalidValue;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return hipErrorInvalidValue;
    if (type == kQ4_K || type == kBF16) {
        if ((wa & 15u) != 0 || (row_bytes(type, k) & 15u) != 0) return hipErrorInvalidValue;
    } else if ((wa & 3u) != 0) {
        return hipErrorInvalidValue;
    }
    int8_t* q = static_cast<int8_t*>(workspace);
    const size_t qbytes = (static_cast<size_t>(b) * k + 255) & ~static_cast<size_t>(255);
    ActMeta* meta = reinterpret_cast<ActMeta*>(static_cast<char*>(workspace) + qbytes);
    if (type != kBF16 && qbytes + static_cast<size_t>(b) * (k / 32) * sizeof(ActMeta) > workspace_bytes)
        return hipErrorInvalidValue;
    switch (type) {
    case kQ4_0: return launch_t<kQ4_0>(w, x, b, k, n, y, q, meta, stream);
    case kQ8_0: return launch_t<kQ8_0>(w, x, b, k, n, y, q, meta, stream);
    case kQ4_K: return launch_t<kQ4_K>(w, x, b, k, n, y, q, meta, stream);
    case kQ6_K: return launch_t<kQ6_K>(w, x, b, k, n, y, q, meta, stream);
    case kBF16: return launch_t<kBF16>(w, x, b, k, n, y, q, meta, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gncx
