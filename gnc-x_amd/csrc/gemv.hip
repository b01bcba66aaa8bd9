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

// Resident waves the grid is sized for (256 CUs x this many).
#ifndef GNCX_GEMV_WAVES_PER_CU
#define GNCX_GEMV_WAVES_PER_CU 16
#endif

// One wave owns groups of R consecutive rows.  A row's slots are consumed in
// batches of P passes (64 slots per pass).  The loads of one batch are always
// in flight while the previous batch is being reduced (double buffering in
// registers, across batches of a row and across groups), and the first batch
// is issued before the work-group quantises x into LDS, so the activation
// pass hides under the first HBM round trip.  With AREG (a row fits in one
// batch) each lane's activation slice is the same for every row, so it is
// read from LDS once into registers.
template <int TYPE, int P, int R, bool AREG>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t* __restrict w, size_t rbytes,
                                                        const float* __restrict x, int32_t k, int32_t n,
                                                        float* __restrict y) {
    using S = Slot<TYPE>;
    using Frag = typename S::Frag;
    using Act = typename S::Act;
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t* q = reinterpret_cast<int8_t*>(lds);
    ActMeta* meta = reinterpret_cast<ActMeta*>(lds + k);
    const int lane = threadIdx.x & 63;
    const int32_t wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int32_t nwaves = gridDim.x * (kThreads / 64);
    const int32_t slots = S::slots(k);
    const int32_t ngroups = (n + R - 1) / R;
    const int32_t nbatch = (slots + 64 * P - 1) / (64 * P);

    Frag cur[R][P];
    Frag nxt[R][P];
    auto issue = [&](Frag (&f)[R][P], int32_t grp, int32_t b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int32_t row = grp * R + r;
            if (row < n) {
                const uint8_t* rp = w + static_cast<size_t>(row) * rbytes;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const int s = lane + 64 * (b * P + p);
                    if (s < slots) S::load(f[r][p], rp, s);
                }
            }
        }
    };

    int32_t g = wave;
    if (g < ngroups) issue(cur, g, 0);
    if (TYPE != kBF16) {
        quantize_block8(x, k / 32, threadIdx.x, kThreads, q, meta);
        __syncthreads();
    }
    Act areg[AREG ? P : 1];
    if constexpr (AREG) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int s = lane + 64 * p;
            if (s < slots) slot_act<TYPE>(areg[p], s, q, meta, x);
        }
    }
    for (; g < ngroups; g += nwaves) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        for (int32_t b = 0; b < nbatch; ++b) {
            if (b + 1 < nbatch) issue(nxt, g, b + 1);
            else if (g + nwaves < ngroups) issue(nxt, g + nwaves, 0);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int32_t row = g * R + r;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const int s = lane + 64 * (b * P + p);
                    if (s < slots && row < n) {
                        if constexpr (AREG) {
                            acc[r] += S::dot(cur[r][p], areg[p], s);
                        } else {
                            Act a;
                            slot_act<TYPE>(a, s, q, meta, x);
                            acc[r] += S::dot(cur[r][p], a, s);
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int p = 0; p < P; ++p) cur[r][p] = nxt[r][p];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[r]);
            const int32_t row = g * R + r;
            if (lane == 0 && row < n) y[row] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Band kernel (the main path): one 1024-thread work-group per CU, so x is
// quantised into LDS only 256 times per call.  Work-group g owns rows
// g, g + G, g + 2G, ... (G = number of work-groups): at any moment the whole
// GPU is sweeping one contiguous stretch of the matrix, which keeps HBM pages
// and channels busy the way a plain streaming read does (a contiguous band
// per work-group measured 2x slower).  Waves are arranged nwk x nwr: wave
// (kw, rw) handles slots [64 kw, 64 kw + 64) (one K-slice, its activations
// kept in registers) of the work-group's local rows rw, rw + nwr, ...  Rows go
// R at a time in two register buffers used in turn; the first batches' loads
// are issued before the quantisation.  Each wave's per-row partial goes to LDS
// and the K-slices are added in a fixed order at the end (deterministic).
#ifndef GNCX_BAND_THREADS
#define GNCX_BAND_THREADS 1024
#endif
#ifndef GNCX_BAND_GROUPS
#define GNCX_BAND_GROUPS 256
#endif
#ifndef GNCX_Q4K_ROWS
#define GNCX_Q4K_ROWS 2
#endif
constexpr int kBandThreads = GNCX_BAND_THREADS;
constexpr int kBandWaves = kBandThreads / 64;
constexpr int32_t kBandGroups = GNCX_BAND_GROUPS;  // one work-group per CU of an MI355X
constexpr size_t kBandLds = 64 * 1024;

template <int TYPE, int R>
__global__ __launch_bounds__(kBandThreads) void gemv_band_kernel(const uint8_t* __restrict w, size_t rbytes,
                                                                 const float* __restrict x, int32_t k,
                                                                 int32_t n, float* __restrict y,
                                                                 int32_t rows_per_wg, int32_t nwk, int32_t nwr) {
    using S = Slot<TYPE>;
    using Frag = typename S::Frag;
    using Act = typename S::Act;
    constexpr int QU = 4;  // x tasks per thread loaded ahead (covers k <= 16384)
    extern __shared__ __align__(16) uint8_t lds[];
    const size_t qbytes = TYPE == kBF16 ? 0 : static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta);
    int8_t* q = reinterpret_cast<int8_t*>(lds);
    ActMeta* meta = reinterpret_cast<ActMeta*>(lds + k);
    float* part = reinterpret_cast<float*>(lds + qbytes);  // [rows_per_wg][nwk]

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kw = wv % nwk, rw = wv / nwk;
    const bool active = rw < nwr;
    const int32_t slots = S::slots(k);
    const int s = kw * 64 + lane;
    const bool has_slot = active && s < slots;
    const int32_t groups = gridDim.x;
    // local row li of this work-group is global row li * groups + blockIdx.x
    const int32_t rows_here = (n - static_cast<int32_t>(blockIdx.x) + groups - 1) / groups;
    const int32_t per_wave = (rows_per_wg + nwr - 1) / nwr;
    const int32_t nb = (per_wave + R - 1) / R;
    auto grow = [&](int32_t li) { return static_cast<size_t>(li) * groups + blockIdx.x; };

    // two weight buffers used in turn (no register copies: a copy would wait
    // for the loads in flight).  Loads are unconditional -- lanes without a
    // slot or row read slot 0 of row 0 and their result is masked -- so the
    // waitcnts before each use only wait for that use's loads.
    Frag fa[R], fb[R];
    auto issue = [&](Frag (&f)[R], int32_t b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int32_t li = rw + nwr * (b * R + r);
            const bool ok = has_slot && li < rows_here;
            S::load(f[r], ok ? w + grow(li) * rbytes : w, ok ? s : 0);
        }
    };
    auto reduce = [&](const Frag (&f)[R], const Act& a, int32_t b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int32_t li = rw + nwr * (b * R + r);
            if (active && li < rows_here) {  // wave-uniform
                float v = has_slot ? S::dot(f[r], a, s) : 0.0f;
                v = wave_sum_lane63(v);
                if (lane == 63) part[li * nwk + kw] = v;
            }
        }
    };

    // x first (it is waited for first), then every weight batch this wave can hold
    float4 xv[QU];
    if (TYPE != kBF16) quant_load<QU>(xv, x, k / 32, threadIdx.x, kBandThreads);
    issue(fa, 0);
    if (nb > 1) issue(fb, 1);
    if (TYPE != kBF16) quant_finish<QU>(xv, x, k / 32, threadIdx.x, kBandThreads, q, meta);
    __syncthreads();
    Act a;
    if (has_slot) slot_act<TYPE>(a, s, q, meta, x);
    for (int32_t b = 0; b < nb; b += 2) {
        reduce(fa, a, b);
        if (b + 2 < nb) issue(fa, b + 2);
        if (b + 1 < nb) {
            reduce(fb, a, b + 1);
            if (b + 3 < nb) issue(fb, b + 3);
        }
    }
    __syncthreads();
    for (int32_t li = threadIdx.x; li < rows_here; li += kBandThreads) {
        float acc = 0.0f;
        for (int j = 0; j < nwk; ++j) acc += part[li * nwk + j];
        y[grow(li)] = acc;
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

template <int TYPE, int P, int R, bool AREG>
hipError_t launch_shape(const uint8_t* w, const float* x, int32_t k, int32_t n, float* y, hipStream_t stream) {
    const size_t rb = row_bytes(TYPE, k);
    const size_t lds = TYPE == kBF16 ? 0 : static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta);
    const int32_t ngroups = (n + R - 1) / R;
    int32_t waves = 256 * GNCX_GEMV_WAVES_PER_CU;
    if (waves > ngroups) waves = ngroups;
    const int32_t groups = (waves + kThreads / 64 - 1) / (kThreads / 64);
    hipLaunchKernelGGL((gemv_kernel<TYPE, P, R, AREG>), dim3(groups), dim3(kThreads), lds, stream, w, rb, x, k, n, y);
    return hipGetLastError();
}

// Rows of one pass (<= 64 slots) go two to a wave; longer rows one to a wave,
// in batches of up to PMAX passes (register budget of the format's slot).
template <int TYPE, int PMAX>
hipError_t launch_gemv_t(const uint8_t* w, const float* x, int32_t k, int32_t n, float* y, hipStream_t stream) {
    const int32_t passes = (Slot<TYPE>::slots(k) + 63) / 64;
    if (passes <= 1) return launch_shape<TYPE, 1, 2, true>(w, x, k, n, y, stream);
    if (passes == 2) return launch_shape<TYPE, 2, 1, true>(w, x, k, n, y, stream);
    if (PMAX == 2) return launch_shape<TYPE, 2, 1, false>(w, x, k, n, y, stream);
    if (passes <= PMAX) return launch_shape<TYPE, (PMAX > 2 ? PMAX : 2), 1, true>(w, x, k, n, y, stream);
    return launch_shape<TYPE, (PMAX > 2 ? PMAX : 2), 1, false>(w, x, k, n, y, stream);
}


// Band kernel geometry for (type, k, n); false when the shape does not fit it.
bool band_plan(int32_t slots, int32_t k, int32_t n, bool quantised, int32_t& rows_per_wg, int32_t& groups,
               int32_t& nwk, int32_t& nwr, size_t& lds) {
    nwk = (slots + 63) / 64;
    if (nwk < 1 || nwk > kBandWaves) return false;
    nwr = kBandWaves / nwk;
    groups = n < kBandGroups ? n : kBandGroups;
    rows_per_wg = (n + groups - 1) / groups;
    groups = (n + rows_per_wg - 1) / rows_per_wg;
    const size_t qbytes = quantised ? static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta) : 0;
    lds = qbytes + sizeof(float) * static_cast<size_t>(rows_per_wg) * nwk;
    return lds <= kBandLds;
}

template <int TYPE, int R>
hipError_t launch_band(const uint8_t* w, const float* x, int32_t k, int32_t n, float* y, hipStream_t stream,
                       bool& used) {
    int32_t rpw, groups, nwk, nwr;
    size_t lds;
    used = band_plan(Slot<TYPE>::slots(k), k, n, TYPE != kBF16, rpw, groups, nwk, nwr, lds);
    if (!used) return hipSuccess;
    hipLaunchKernelGGL((gemv_band_kernel<TYPE, R>), dim3(groups), dim3(kBandThreads), lds, stream, w,
                       row_bytes(TYPE, k), x, k, n, y, rpw, nwk, nwr);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n, float* y,
                       hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (k <= 0 || k > kMaxGemvK) return hipErrorInvalidValue;
    if (type != kBF16 && (k % 32) != 0) return hipErrorInvalidValue;
    if ((type == kQ4_K || type == kQ6_K) && (k % 256) != 0) return hipErrorInvalidValue;
    if (type == kBF16 && (k % 8) != 0) return hipErrorInvalidValue;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
    if ((xa & 15u) != 0) return hipErrorInvalidValue;
    if (type == kQ4_K || type == kBF16) {
        if ((wa & 15u) != 0 || (row_bytes(type, k) & 15u) != 0) return hipErrorInvalidValue;
    } else if ((wa & 3u) != 0) {
        return hipErrorInvalidValue;
    }
    bool used = false;
    hipError_t e = hipSuccess;
    switch (type) {
    case kQ4_0: e = launch_band<kQ4_0, 4>(w, x, k, n, y, stream, used); break;
    case kQ8_0: e = launch_band<kQ8_0, 2>(w, x, k, n, y, stream, used); break;
    case kQ4_K: e = launch_band<kQ4_K, GNCX_Q4K_ROWS>(w, x, k, n, y, stream, used); break;
    case kQ6_K: e = launch_band<kQ6_K, 1>(w, x, k, n, y, stream, used); break;
    case kBF16: e = launch_band<kBF16, 4>(w, x, k, n, y, stream, used); break;
    default: return hipErrorInvalidValue;
    }
    if (used || e != hipSuccess) return e;
    switch (type) {
    case kQ4_0: return launch_gemv_t<kQ4_0, 4>(w, x, k, n, y, stream);
    case kQ8_0: return launch_gemv_t<kQ8_0, 2>(w, x, k, n, y, stream);
    case kQ4_K: return launch_gemv_t<kQ4_K, 2>(w, x, k, n, y, stream);
    case kQ6_K: return launch_gemv_t<kQ6_K, 2>(w, x, k, n, y, stream);
    case kBF16: return launch_gemv_t<kBF16, 4>(w, x, k, n, y, stream);
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
