// matbatch.hip -- batched prefill product Y[B x N] = Q8(X[B x K]) . W^T.
//
// Semantics of the reference's gncx_xfold_universal_matbatch
// (csrc/gncx_llm_kernels.cpp:1495-1692): every token row of X is quantised
// on its own to per-32 int8 blocks (cpp:1506-1510), then each output is the
// same integer block dot as the matvec; the output is row-major out[t*N + m].
//
// Quantised weights (Q4_0, Q8_0, Q4_K, Q6_K) go through the fp16 matrix
// cores with both operands carried as fp16 pairs (hi, lo):
//   1. act_hilo_kernel quantises each token row exactly as the reference
//      does and stores each quantised activation q * d / s as an fp16 pair
//      (s is a power-of-two row scale the MFMA epilogue multiplies back),
//   2. matbatch_mfma_kernel streams 32-wide K steps: the work-group's weight
//      rows are dequantised block by block in fp32 and split into fp16 pairs
//      in LDS, its token rows are copied into LDS, and each wave runs three
//      v_mfma_f32_32x32x16_f16 per tile and K slice (hi x hi, lo x hi,
//      hi x lo) with fp32 accumulation.
// Each product is then exact to about 2^-22, and Y lands within about 2e-7
// relative L2 of the reference's integer block dots (fp16 operands alone:
// 3e-4).  An int8 MFMA path would be exact too, but its per-32-block scales
// cost ~3 VALU operations per output and block, several times the
// matrix-core time of the three fp16 products.
// Q4_K (the layer format of the prefill workloads) and Q6_K have their own
// kernel, matbatch_qs_stream_kernel: the weights are small integers exact in
// fp16 (sc q; sc (q - 32) as two parts) with d (and dmin) fixed per
// 256-value super-block, and the activations are the quantised q as fp16
// with each block's scale, so a block's integer dot is exact in one (Q6_K:
// two) products per K slice; the block scale is applied on the VALU and d
// and the min term once per super-block.
// BF16 weights (fp32 activations, cpp:1432-1461) use the slot-dot kernel: a
// wave per (row, token).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gncx_act.h"
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

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// fp16 pair (hi, lo) of a float: hi = fp16(v) and lo = fp16(v - hi), with
// v - hi exact in fp32, so hi + lo carries 22 significant bits of v.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
    const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
    const _Float16 la = static_cast<_Float16>(a - static_cast<float>(ha));
    const _Float16 lb = static_cast<_Float16>(b - static_cast<float>(hb));
    hi = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
    lo = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, la)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lb)) << 16);
}

// act_hilo_kernel<U> holds U float4 of x per thread in registers from the
// max pass to the quantising pass (rows up to 4 kThreads U values): the
// loads of a row are issued together, and a longer row reads its tail again.
// U = 4 covers 4096-wide rows at 40-odd registers; wider rows take U = 16
// (130-odd registers, 3 waves per SIMD), or, for the SwiGLU rows of the down
// projection up to 12288 wide, 1024 threads (NT) with U = 3, which keeps more
// of a row's loads in flight (47.9 -> 45.1 us at 2048 x 12288).

// The reference's per-32 quantisation of row blockIdx.x of x (cpp:955-995),
// each quantised value a = q * d (one fp32 rounding) scaled by 1 / s, where
// s is the power of two above the row's largest |x| (stored in rscale; the
// MFMA epilogue multiplies it back, exactly), and stored as its fp16 pair
// (hi, lo): xhl holds, per 8 elements, 16 bytes of hi then 16 bytes of lo.
// The rescale keeps every value in [-1, 1], so activations far beyond fp16's
// range (SwiGLU outputs of 1e5 and more) keep the pair's relative precision.
// One work-group per row: the row maximum first, then 8 lanes per 32-block,
// 4 values per lane.
// With pq given (K a multiple of 256), also each 32-block's sum of the
// quantised activations, P = (sum q) * d / s, as an fp16 pair: per token row
// and 256-value super-block, 8 hi then 8 lo values (the Q4_K kernel's min
// term, cpp:1177-1178).
// With SW the row is the SwiGLU of two rows, x the gates and up the ups
// (the values gncx_swiglu_activation writes), formed as they are read.
// With QX (the streamed Q4_K and Q6_K kernel) the quantised values q themselves
// go out instead of the pairs, as fp16 (integers of at most 127, exact):
// xhl holds 4 of them per task, row-major [B x K], and dxs (set) each
// 32-block's d / s as fp32 [B x K / 32]; P as above.
// One task's QX outputs (4 values of row `row`, task t of k / 4, at the
// row's 1 / s = inv): q as fp16, the block's d / s from its first lane and,
// with pq, the block's P pair.  Whole 8-lane groups call it together.
__device__ __forceinline__ void emit_qx(const float4 v, int32_t t, int32_t row, int32_t k, float inv,
                                        uint2* __restrict xq, float* __restrict dxs, _Float16* __restrict pq) {
    const int32_t tasks = k / 4;
    int q0, q1, q2, q3;
    float d;
    quantize_values(v, q0, q1, q2, q3, d);
    auto h2 = [](int a, int b) {
        return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
    };
    xq[static_cast<size_t>(row) * tasks + t] = make_uint2(h2(q0, q1), h2(q2, q3));
    if ((t & 7) == 0) dxs[static_cast<size_t>(row) * (k / 32) + (t >> 3)] = d * inv;
    if (pq) {
        // the 8 lanes of block t / 8: quad sums, then lane i adds lane 7 - i
        const int s4 = quad_sum(q0 + q1 + q2 + q3);
        const int sum = s4 + __builtin_amdgcn_mov_dpp(s4, 0x141, 0xf, 0xf, false);
        if ((t & 7) == 0) {
            const int32_t blk = t >> 3;
            const float pv = (static_cast<float>(sum) * d) * inv;
            const _Float16 ph = static_cast<_Float16>(pv);
            const _Float16 pl = static_cast<_Float16>(pv - static_cast<float>(ph));
            _Float16* pr = pq + (static_cast<size_t>(row) * (k / 256) + blk / 8) * 16 + (blk & 7);
            pr[0] = ph;
            pr[8] = pl;
        }
    }
}

template <int kHiloU, bool SW = false, bool QX = false, int NT = kThreads>
__global__ __launch_bounds__(NT) void act_hilo_kernel(const float* __restrict x, int32_t k,
                                                            uint2* __restrict xhl, float* __restrict rscale,
                                                            _Float16* __restrict pq, const float* __restrict up,
                                                            float* __restrict dxs = nullptr) {
    __shared__ float red[NT / 64];
    const int32_t row = blockIdx.x, tasks = k / 4;
    const float4* xg = reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * k);
    const float4* xu = SW ? reinterpret_cast<const float4*>(up + static_cast<size_t>(row) * k) : nullptr;
    struct Row {
        const float4* g;
        const float4* u;
        __device__ float4 operator[](int32_t t) const {
            if constexpr (!SW) {
                return g[t];
            } else {
                const float4 a = g[t], b = u[t];
                return make_float4(swiglu_value(a.x, b.x), swiglu_value(a.y, b.y), swiglu_value(a.z, b.z),
                                   swiglu_value(a.w, b.w));
            }
        }
    };
    const Row xr{xg, xu};
    auto amax4 = [](const float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
    float4 xv[kHiloU];
#pragma unroll
    for (int u = 0; u < kHiloU; ++u) {
        const int32_t t = static_cast<int32_t>(threadIdx.x) + u * NT;
        xv[u] = t < tasks ? xr[t] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < kHiloU; ++u) m = fmaxf(m, amax4(xv[u]));
    for (int32_t t = threadIdx.x + kHiloU * NT; t < tasks; t += NT) m = fmaxf(m, amax4(xr[t]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) m = fmaxf(m, red[w]);
    const float sc = m > 0.0f && m <= 3.0e38f ? ldexpf(1.0f, ilogbf(m) + 1) : 1.0f;  // power of two > m
    const float inv = 1.0f / sc;                                       // exact
    if (threadIdx.x == 0) rscale[row] = sc;
    uint2* out = xhl + static_cast<size_t>(row) * tasks * 2;
    auto emit = [&](const float4 v, int32_t t) {
        if constexpr (QX) {
            emit_qx(v, t, row, k, inv, xhl, dxs, pq);
        } else {
            int q0, q1, q2, q3;
            float d;
            quantize_values(v, q0, q1, q2, q3, d);
            uint2 hi, lo;
            split2((static_cast<float>(q0) * d) * inv, (static_cast<float>(q1) * d) * inv, hi.x, lo.x);
            split2((static_cast<float>(q2) * d) * inv, (static_cast<float>(q3) * d) * inv, hi.y, lo.y);
            // task t is elements 4t .. 4t + 3: chunk t / 2 of 8, half t % 2
            uint2* c = out + 4 * (t >> 1) + (t & 1);
            c[0] = hi;
            c[2] = lo;
            if (pq) {
                // the 8 lanes of block t / 8: quad sums, then lane i adds lane 7 - i
                const int s4 = quad_sum(q0 + q1 + q2 + q3);
                const int sum = s4 + __builtin_amdgcn_mov_dpp(s4, 0x141, 0xf, 0xf, false);
                if ((t & 7) == 0) {
                    const int32_t blk = t >> 3;
                    const float pv = (static_cast<float>(sum) * d) * inv;
                    const _Float16 ph = static_cast<_Float16>(pv);
                    const _Float16 pl = static_cast<_Float16>(pv - static_cast<float>(ph));
                    _Float16* pr = pq + (static_cast<size_t>(row) * (k / 256) + blk / 8) * 16 + (blk & 7);
                    pr[0] = ph;
                    pr[8] = pl;
                }
            }
        }
    };
    // whole 8-lane groups take the same branches and trip counts (tasks and
    // NT are multiples of 8), as the group operations need
#pragma unroll
    for (int u = 0; u < kHiloU; ++u) {
        const int32_t t = static_cast<int32_t>(threadIdx.x) + u * NT;
        if (t < tasks) emit(xv[u], t);
    }
    for (int32_t t = threadIdx.x + kHiloU * NT; t < tasks; t += NT) emit(xr[t], t);
}

// the streamed kernel's activations: q as fp16 [B x K], then the blocks'
// d / s [B x K / 32] (dxs), the P pairs (Q4_K) and the row scales
void launch_act_q(const float* x, int32_t b, int32_t k, _Float16* xq, float* dxs, float* rscale, _Float16* pq,
                  hipStream_t stream, const float* up) {
    uint2* o = reinterpret_cast<uint2*>(xq);
    if (up) {
        if (k <= 4 * 4 * kThreads)
            hipLaunchKernelGGL((act_hilo_kernel<4, true, true>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale,
                               pq, up, dxs);
        else if (k <= 3 * 4 * 1024)  // up to 12288-wide rows: 16 waves, 3 float4 pairs each
            hipLaunchKernelGGL((act_hilo_kernel<3, true, true, 1024>), dim3(b), dim3(1024), 0, stream, x, k, o,
                               rscale, pq, up, dxs);
        else
            hipLaunchKernelGGL((act_hilo_kernel<16, true, true>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale,
                               pq, up, dxs);
    } else if (k <= 4 * 4 * kThreads) {
        hipLaunchKernelGGL((act_hilo_kernel<4, false, true>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale, pq,
                           nullptr, dxs);
    } else {
        hipLaunchKernelGGL((act_hilo_kernel<16, false, true>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale,
                           pq, nullptr, dxs);
    }
}

// launch_act_q of the RMSNorm of each row, after the optional residual add
// (h += r, written back), in one launch.  The norm is rmsnorm_kernel's
// (elementwise.hip) with its thread layout (1024 threads, float4 t = thread +
// 1024 j, up to 4 per thread), sum order and operation order, so the rows
// quantised are those gncx_hip_add_rmsnorm_rows / gncx_hip_rmsnorm_rows
// write; the quantisation is act_hilo_kernel's (a row maximum, then 8
// consecutive lanes per 32-block).
constexpr int kNaThreads = 1024;
constexpr int kNaRegs = 4;
template <bool ADD>
__global__ __launch_bounds__(kNaThreads) void norm_act_q_kernel(const float* x, const float* r, float* xo,
                                                               const float* __restrict g, int32_t k, float eps,
                                                               uint2* __restrict xq, float* __restrict dxs,
                                                               float* __restrict rscale, _Float16* __restrict pq) {
#pragma clang fp contract(off)
    __shared__ float part[kNaThreads / 64];
    __shared__ float red[kNaThreads / 64];
    const int32_t row = blockIdx.x, n4 = k / 4;
    const int tid = threadIdx.x;
    const float4* x4 = reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * k);
    const float4* r4 = reinterpret_cast<const float4*>(ADD ? r + static_cast<size_t>(row) * k : nullptr);
    float4* xo4 = reinterpret_cast<float4*>(ADD ? xo + static_cast<size_t>(row) * k : nullptr);
    const float4* g4 = reinterpret_cast<const float4*>(g);
    float4 xv[kNaRegs], gv[kNaRegs];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kNaRegs; ++j) {
        const int32_t t = tid + kNaThreads * j;
        if (t < n4) {
            xv[j] = x4[t];
            if (ADD) {
                const float4 b = r4[t];
                xv[j] = make_float4(xv[j].x + b.x, xv[j].y + b.y, xv[j].z + b.z, xv[j].w + b.w);
                xo4[t] = xv[j];
            }
            gv[j] = g4[t];
            s += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
        }
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kNaThreads / 64; ++w) tot += part[w];
    const float inv_rms = 1.0f / sqrtf(tot / static_cast<float>(k) + eps);
    float4 yv[kNaRegs];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kNaRegs; ++j) {
        const int32_t t = tid + kNaThreads * j;
        yv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t < n4) {
            yv[j] = make_float4(xv[j].x * inv_rms * gv[j].x, xv[j].y * inv_rms * gv[j].y,
                                xv[j].z * inv_rms * gv[j].z, xv[j].w * inv_rms * gv[j].w);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(yv[j].x), fabsf(yv[j].y)), fmaxf(fabsf(yv[j].z), fabsf(yv[j].w))));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kNaThreads / 64; ++w) m = fmaxf(m, red[w]);
    const float sc = m > 0.0f && m <= 3.0e38f ? ldexpf(1.0f, ilogbf(m) + 1) : 1.0f;  // power of two > m
    const float inv = 1.0f / sc;                                                     // exact
    if (tid == 0) rscale[row] = sc;
#pragma unroll
    for (int j = 0; j < kNaRegs; ++j) {
        const int32_t t = tid + kNaThreads * j;
        if (t < n4) emit_qx(yv[j], t, row, k, inv, xq, dxs, pq);
    }
}

// false when the fused form does not apply (then norm and quantise apart)
bool norm_act_fits(const float* h, const float* r, const float* gamma, int32_t k) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(r) |
                         reinterpret_cast<uintptr_t>(gamma);
    return k > 0 && k % 256 == 0 && k / 4 <= kNaThreads * kNaRegs && (al & 15u) == 0;
}

void launch_norm_act_q(float* h, const float* r, const float* gamma, float eps, int32_t b, int32_t k, _Float16* xq,
                       float* dxs, float* rscale, _Float16* pq, hipStream_t stream) {
    uint2* o = reinterpret_cast<uint2*>(xq);
    if (r)
        hipLaunchKernelGGL(norm_act_q_kernel<true>, dim3(b), dim3(kNaThreads), 0, stream, h, r, h, gamma, k, eps, o,
                           dxs, rscale, pq);
    else
        hipLaunchKernelGGL(norm_act_q_kernel<false>, dim3(b), dim3(kNaThreads), 0, stream, h, nullptr, nullptr,
                           gamma, k, eps, o, dxs, rscale, pq);
}

// up non-null: the rows are SwiGLU(x, up)
void launch_act_hilo(const float* x, int32_t b, int32_t k, _Float16* xhl, float* rscale, _Float16* pq,
                     hipStream_t stream, const float* up = nullptr) {
    uint2* o = reinterpret_cast<uint2*>(xhl);
    if (up) {
        if (k <= 4 * 4 * kThreads)
            hipLaunchKernelGGL((act_hilo_kernel<4, true>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale, pq, up);
        else
            hipLaunchKernelGGL((act_hilo_kernel<16, true>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale, pq,
                               up);
    } else if (k <= 4 * 4 * kThreads) {
        hipLaunchKernelGGL((act_hilo_kernel<4>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale, pq, nullptr);
    } else {
        hipLaunchKernelGGL((act_hilo_kernel<16>), dim3(b), dim3(kThreads), 0, stream, x, k, o, rscale, pq, nullptr);
    }
}

// Weights e0 .. e0 + 15 (e0 a multiple of 16) of one row: raw block bytes
// loaded into registers (WSeg::load, issued two K steps ahead of their use),
// then dequantised in fp32 (WSeg::get) and split into fp16 pairs on their way
// into LDS; an all-zero block (what a past-the-end buffer load reads)
// dequantises to zeros.  Formulas: Q4_0 d (q - 8), elements j and j + 16 in
// the low and high nibbles of byte j (cpp:1023-1030); Q8_0 d q; Q4_K
// (d sc) q - dmin m with sub-block j of chunk c in the low (j even) or high
// nibbles of bytes 32c .. 32c + 31 (cpp:1135-1178); Q6_K (d sc) (q - 32) with
// element l + 32 g of a 128-half from ql[l + 32 (g & 1)] (nibble g / 2),
// qh[l] >> 2g and scale l / 16 + 2g (cpp:742-757).
template <int TYPE>
struct WSeg;

template <>
struct WSeg<kQ4_0> {
    uint32_t d, sh;
    Raw16 qs;
    template <class Row>
    __device__ __forceinline__ void load(const Row& r, int32_t e0) {
        const uint32_t blk = static_cast<uint32_t>(e0 / 32) * 18u;
        d = r.ldu16(blk);
        sh = r.sh(blk + 2u);
        raw16_load(qs, r, blk + 2u, sh);
    }
    __device__ __forceinline__ void get(int32_t e0, float (&v)[16]) const {
        const float dv = half_bits_to_float(d);
        const uint4 q = raw16_get(qs, sh);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        const int s = 4 * ((e0 >> 4) & 1);
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = dv * static_cast<float>(static_cast<int>((w[i >> 2] >> (s + 8 * (i & 3))) & 15u) - 8);
    }
};

template <>
struct WSeg<kQ8_0> {
    uint32_t d, sh;
    Raw16 qs;
    template <class Row>
    __device__ __forceinline__ void load(const Row& r, int32_t e0) {
        const uint32_t blk = static_cast<uint32_t>(e0 / 32) * 34u;
        d = r.ldu16(blk);
        const uint32_t o = blk + 2u + 16u * static_cast<uint32_t>((e0 >> 4) & 1);
        sh = r.sh(o);
        raw16_load(qs, r, o, sh);
    }
    __device__ __forceinline__ void get(int32_t, float (&v)[16]) const {
        const float dv = half_bits_to_float(d);
        const uint4 q = raw16_get(qs, sh);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = dv * static_cast<float>(static_cast<int8_t>((w[i >> 2] >> (8 * (i & 3))) & 0xffu));
    }
};

template <>
struct WSeg<kQ4_K> {
    u32x4 hdr, q;
    template <class Row>
    __device__ __forceinline__ void load(const Row& r, int32_t e0) {
        const uint32_t blk = static_cast<uint32_t>(e0 / 256) * 144u, rr = static_cast<uint32_t>(e0 % 256);
        hdr = r.ld16(blk);
        q = r.ld16(blk + 16u + 32u * (rr / 64u) + (rr % 32u));
    }
    __device__ __forceinline__ void get(int32_t e0, float (&v)[16]) const {
        const int j = (e0 % 256) / 32, s = 4 * (j & 1);
        int sc, mn;
        k4_scale_min(j, hdr.y, hdr.z, hdr.w, sc, mn);
        const float a = half_bits_to_float(hdr.x & 0xffffu) * static_cast<float>(sc);
        const float m = half_bits_to_float(hdr.x >> 16) * static_cast<float>(mn);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = a * static_cast<float>((w[i >> 2] >> (s + 8 * (i & 3))) & 15u) - m;
    }
};

template <>
struct WSeg<kQ6_K> {
    Raw16 ql, qh;
    uint32_t scw, d, sh;
    template <class Row>
    __device__ __forceinline__ void load(const Row& r, int32_t e0) {
        const uint32_t blk = static_cast<uint32_t>(e0 / 256) * 210u;
        const uint32_t rr = static_cast<uint32_t>(e0 % 256), h = rr / 128u, g = (rr % 128u) / 32u, l0 = rr % 32u;
        sh = r.sh(blk);  // every field offset used here is even: one shift for all
        raw16_load(ql, r, blk + 64u * h + 32u * (g & 1u) + l0, sh);
        raw16_load(qh, r, blk + 128u + 32u * h + l0, sh);
        scw = r.ldu16(blk + 192u + 8u * h + 2u * g);  // scales l0 / 16 + 2g of this half
        d = r.ldu16(blk + 208u);
    }
    // sc (q - 32) as integers, |sc (q - 32)| <= 4096 (d is applied per
    // super-block); returns sc
    __device__ __forceinline__ int get_int(int32_t e0, int (&v)[16]) const {
        const int rr = e0 % 256, g = (rr % 128) / 32, l0 = rr % 32;
        const int sc = static_cast<int8_t>((scw >> (l0 >= 16 ? 8 : 0)) & 0xffu);
        const uint4 a = raw16_get(ql, sh), b = raw16_get(qh, sh);
        const uint32_t L[4] = {a.x, a.y, a.z, a.w}, H[4] = {b.x, b.y, b.z, b.w};
        const int lsh = 4 * (g >> 1), hsh = 2 * g;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int sh8 = 8 * (i & 3);
            const int q = static_cast<int>(((L[i >> 2] >> (lsh + sh8)) & 15u) | (((H[i >> 2] >> (hsh + sh8)) & 3u) << 4));
            v[i] = sc * (q - 32);
        }
        return sc;
    }
    __device__ __forceinline__ void get(int32_t e0, float (&v)[16]) const {
        const int rr = e0 % 256, g = (rr % 128) / 32, l0 = rr % 32;
        const float s = half_bits_to_float(d) * static_cast<float>(static_cast<int8_t>((scw >> (l0 >= 16 ? 8 : 0)) & 0xffu));
        const uint4 a = raw16_get(ql, sh), b = raw16_get(qh, sh);
        const uint32_t L[4] = {a.x, a.y, a.z, a.w}, H[4] = {b.x, b.y, b.z, b.w};
        const int lsh = 4 * (g >> 1), hsh = 2 * g;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int sh8 = 8 * (i & 3);
            const int q = static_cast<int>(((L[i >> 2] >> (lsh + sh8)) & 15u) | (((H[i >> 2] >> (hsh + sh8)) & 3u) << 4));
            v[i] = s * static_cast<float>(q - 32);
        }
    }
};

// Y tile of (32 WM MW) tokens x (64 WN) rows per work-group of 2 MW waves
// (MW along the tokens, 2 along the rows); each wave owns WM x WN 32x32
// accumulator tiles.  Both operands are fp16 pairs (hi, lo), and each 16-wide
// K slice runs three v_mfma_f32_32x32x16_f16 per tile: x_hi w_hi + x_lo w_hi +
// x_hi w_lo (x_lo w_lo is below 2^-22 of the product).  With fp32
// accumulation the result is within about 2e-7 relative L2 of the
// reference's integer block dots (measured on the CPU and the GPU for all
// four formats), where fp16 operands alone reach 3e-4.
// K advances 32 per step through two LDS buffers, each holding token rows
// [tokens][32 + 8 pad] and weight rows [rows][32 + 8 pad] as hi and lo
// arrays.  In step s the MFMAs consume buffer s % 2 while the loads for
// later steps are in flight, then step s + 1's registers are written to the
// other buffer; one barrier per step.  All loads are buffer loads whose
// out-of-range reads return 0 without a memory request (tokens past B, K past
// the range, rows past N), so each wave issues the same loads every step and
// each wait covers exactly the loads it needs.
// MFMA operand layouts (v_mfma_f32_32x32x16_f16): lane l holds
// A[l % 32][8 (l / 32) .. + 8] and B[8 (l / 32) .. + 8][l % 32]; accumulator
// register r of lane l is D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
// blockIdx.z selects a K range of kchunk (split K); with gridDim.z > 1 the
// tile goes to part[z][t][m] and matbatch_reduce_kernel adds the ranges in
// order.
// Q6_K weights are d (sc (q - 32)) (cpp:742-757) with sc (q - 32) an integer
// of magnitude at most 4096 and d fixed over a 256-value super-block, so the
// weight operand is that integer: exact in fp16 up to 2048 (|sc| <= 64),
// else its fp16 rounding (hi) plus an exact remainder of -1, 0 or 1 (lo).
// On the 256-token tiles (B > 128) the products of a super-block go to a
// second accumulator D, folded in as
// acc += d D at its end (d of the lane's weight row), and x_hi w_lo, the
// third product, runs only in steps where some weight of the tile has
// |sc| > 64: elsewhere w_lo is zero.  The third product's step flag is the
// step's first K index, written to LDS by any thread that dequantised such
// a scale (a stale flag never equals a later step's index).
constexpr int kMfKs = 32;
constexpr int kMfLd = kMfKs + 8;  // halves per LDS row (16-byte aligned, staggers banks)
// a buffer offset past any resource (resources here are below 2^30 bytes);
// small field offsets may still be added to it without leaving int32
constexpr int32_t kMfOob = 0x7ff00000;

template <int WM, int WN, int MW>
constexpr size_t mfma_lds_bytes() {
    return 2 * 2 * static_cast<size_t>(32 * WM * MW + 64 * WN) * kMfLd * sizeof(_Float16);
}

template <int TYPE, int WM, int WN, int MW = 2>
__global__ __launch_bounds__(128 * MW, MW == 2 ? 2 : 1) void matbatch_mfma_kernel(const uint8_t* __restrict w,
                                                                                   size_t rbytes,
                                                            const _Float16* __restrict xhl,
                                                            const float* __restrict rscale, int32_t b, int32_t k,
                                                            int32_t n, float* __restrict y, int32_t kchunk,
                                                            float* __restrict part) {
    constexpr int THREADS = 128 * MW;
    constexpr int BM = 32 * WM * MW, BN = 64 * WN;
    static_assert(2 * BN <= THREADS, "one thread per 16-value weight piece of a step");
    constexpr int XCH = BM * 4 / THREADS;  // 16-byte chunks of 8 values (hi and lo each) per thread and step
    static_assert(XCH * THREADS == BM * 4, "whole chunks per thread");
    static_assert(mfma_lds_bytes<WM, WN, MW>() <= 160 * 1024, "LDS of one CU");
    __shared__ __align__(16) _Float16 xs[2][2][BM * kMfLd];  // [buffer][hi, lo]
    __shared__ __align__(16) _Float16 ws[2][2][BN * kMfLd];
    // The tile's token scales sit in the padding of the activation rows of
    // buffer 1 (halves kMfKs .. kMfLd of row r, which no load, store or
    // product touches), so they cost no LDS: 64x64 tiles fill the CU's LDS
    // with four work-groups at exactly 40 KB each.  Read from memory at the
    // output, they were a dependent load of every wave at the moment all
    // work-groups store.
    static_assert(kMfLd - kMfKs >= 2 && BM <= THREADS, "a float of padding per row, one scale per thread");
    auto rs_at = [&](int r) -> float& { return *reinterpret_cast<float*>(&xs[1][0][r * kMfLd + kMfKs]); };
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv % MW, wn = wv / MW;
    const int32_t t0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int32_t kb = blockIdx.z * kchunk;
    const int32_t ke = min(k, kb + kchunk);
    const int32_t nsteps = (ke - kb + kMfKs - 1) / kMfKs;

    // (the 256-token tiles only: on the smaller ones D's registers cost
    // occupancy, measured 5-11% slower at B = 16 to 100)
    constexpr bool Q6 = TYPE == kQ6_K && MW == 4;
    // Q6_K: d of the tile's rows per super-block parity, the third-product flags
    __shared__ float q6d[Q6 ? 2 : 1][Q6 ? BN : 1];
    __shared__ int32_t q6big[2];
    floatx16 acc[WM][WN], D[Q6 ? WM : 1][Q6 ? WN : 1];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    if constexpr (Q6) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) D[i][j][r] = 0.0f;
    }

    // activation chunks c = tid + THREADS i: token row c / 4 of the tile,
    // values 8 (c % 4) .. + 8 of the step, hi at byte 32 j and lo at 32 j + 16
    // of chunk j = (row k + value) / 8; one resource over the tile's token rows
    const int32_t rows_here = min(BM, b - t0);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(xhl + static_cast<size_t>(t0) * k * 2), static_cast<short>(0),
        rows_here * k * 2 * static_cast<int32_t>(sizeof(_Float16)), 0x00020000);
    // weight piece tid (row tid / 2 of the tile, 16 values at 16 (tid % 2))
    // for tid < 2 BN, through one resource over the tile's rows
    const int wrow = tid >> 1, wseg = tid & 1;
    const int32_t wrows_here = min(BN, n - n0);
    TileRow wrs;
    wrs.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w + static_cast<size_t>(n0) * rbytes),
                                              static_cast<short>(0),
                                              wrows_here * static_cast<int32_t>(rbytes), 0x00020000);
    wrs.base = tid < 2 * BN && wrow < wrows_here ? wrow * static_cast<int32_t>(rbytes) : kMfOob / 2;

    uint4 xr[XCH][2];
    WSeg<TYPE> wr[2];
    // activation chunks of one step; past the range an offset past the
    // resource reads zeros
    auto gload_x = [&](int32_t k0) {
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + THREADS * i, r = c >> 2, seg = c & 3;
            const int32_t kx = k0 + 8 * seg;
            const int32_t off = kx < ke ? (r * k + kx) * 2 * static_cast<int32_t>(sizeof(_Float16)) : kMfOob;
            const u32x4 h = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
            const u32x4 l = __builtin_amdgcn_raw_buffer_load_b128(xrs, off + 16, 0, 0);
            xr[i][0] = make_uint4(h.x, h.y, h.z, h.w);
            xr[i][1] = make_uint4(l.x, l.y, l.z, l.w);
        }
    };
    // raw weight blocks of one step into register set `set`; past the range
    // (k, ke are multiples of 32) the row base moves past the resource, so
    // every field reads zeros without a memory request
    auto gload_w = [&](int set, int32_t k0) {
        const int32_t kw = k0 + 16 * wseg;
        TileRow r = wrs;
        if (kw >= ke) r.base = kMfOob / 2;
        wr[set].load(r, kw < ke ? kw : 0);
    };
    auto lstore = [&](int set, int buf, int32_t k0) {
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + THREADS * i, r = c >> 2, seg = c & 3;
            *reinterpret_cast<uint4*>(&xs[buf][0][r * kMfLd + 8 * seg]) = xr[i][0];
            *reinterpret_cast<uint4*>(&xs[buf][1][r * kMfLd + 8 * seg]) = xr[i][1];
        }
        if (tid < 2 * BN) {
            const int32_t kw = k0 + 16 * wseg;
            uint32_t hi[8], lo[8];
            if constexpr (Q6) {
                int v[16];
                const int sc = wr[set].get_int(kw < ke ? kw : 0, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const _Float16 h0 = static_cast<_Float16>(static_cast<float>(v[2 * i]));
                    const _Float16 h1 = static_cast<_Float16>(static_cast<float>(v[2 * i + 1]));
                    const _Float16 l0 = static_cast<_Float16>(static_cast<float>(v[2 * i]) - static_cast<float>(h0));
                    const _Float16 l1 =
                        static_cast<_Float16>(static_cast<float>(v[2 * i + 1]) - static_cast<float>(h1));
                    hi[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h0)) |
                            (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
                    lo[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l0)) |
                            (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
                }
                if (sc > 64 || sc < -64) q6big[buf] = k0;
                // a super-block's first step in this range stores the rows' d
                if (wseg == 0 && (k0 == kb || k0 % 256 == 0))
                    q6d[(k0 / 256) & 1][wrow] = half_bits_to_float(kw < ke ? wr[set].d : 0u);
            } else {
                float v[16];
                wr[set].get(kw < ke ? kw : 0, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) split2(v[2 * i], v[2 * i + 1], hi[i], lo[i]);
            }
            uint4* dh = reinterpret_cast<uint4*>(&ws[buf][0][wrow * kMfLd + 16 * wseg]);
            uint4* dl = reinterpret_cast<uint4*>(&ws[buf][1][wrow * kMfLd + 16 * wseg]);
            dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        }
    };

    const int li = lane & 31, lk = 8 * (lane >> 5);
    // Q6_K: products into D, the third only where a weight has |sc| > 64;
    // D folded into acc with d at a super-block's last step in the range
    auto compute_q6 = [&](int buf, int32_t k0) {
        const bool third = q6big[buf] == k0;
#pragma unroll
        for (int kk = 0; kk < kMfKs; kk += 16) {
            half8 ah[WM], al[WM], bh[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int o = (wm * 32 * WM + 32 * i + li) * kMfLd + kk + lk;
                ah[i] = *reinterpret_cast<const half8*>(&xs[buf][0][o]);
                al[i] = *reinterpret_cast<const half8*>(&xs[buf][1][o]);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j)
                bh[j] = *reinterpret_cast<const half8*>(&ws[buf][0][(wn * 32 * WN + 32 * j + li) * kMfLd + kk + lk]);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    D[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], D[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    D[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], D[i][j], 0, 0, 0);
            if (third) {
                half8 bl[WN];
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    bl[j] =
                        *reinterpret_cast<const half8*>(&ws[buf][1][(wn * 32 * WN + 32 * j + li) * kMfLd + kk + lk]);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int j = 0; j < WN; ++j)
                        D[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], D[i][j], 0, 0, 0);
            }
        }
        if ((k0 + kMfKs) % 256 == 0 || k0 + kMfKs >= ke) {
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const float dv = q6d[(k0 / 256) & 1][wn * 32 * WN + 32 * j + li];
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[i][j][r] = fmaf(D[i][j][r], dv, acc[i][j][r]);
                        D[i][j][r] = 0.0f;
                    }
            }
        }
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < kMfKs; kk += 16) {
            half8 ah[WM], al[WM], bh[WN], bl[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int o = (wm * 32 * WM + 32 * i + li) * kMfLd + kk + lk;
                ah[i] = *reinterpret_cast<const half8*>(&xs[buf][0][o]);
                al[i] = *reinterpret_cast<const half8*>(&xs[buf][1][o]);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int o = (wn * 32 * WN + 32 * j + li) * kMfLd + kk + lk;
                bh[j] = *reinterpret_cast<const half8*>(&ws[buf][0][o]);
                bl[j] = *reinterpret_cast<const half8*>(&ws[buf][1][o]);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
        }
    };

    // Activations are loaded one step ahead, raw weight blocks two steps
    // ahead in two register sets.  Each step issues the activation loads
    // before the weight loads: loads retire in order, so the wait before
    // writing step s + 1 to LDS does not cover step s + 2's weights.  Steps go
    // in pairs so that register-set and buffer indices are compile-time
    // constants; loads past the range read nothing.
    // the scale load goes first: the wait for step 0's loads covers it
    const float rsv = tid < rows_here ? rscale[t0 + tid] : 1.0f;
    gload_x(kb);
    gload_w(0, kb);
    gload_w(1, kb + kMfKs);
    lstore(0, 0, kb);
    if (tid < BM) rs_at(tid) = rsv;
    __syncthreads();
    for (int32_t s = 0; s < nsteps; s += 2) {
        const int32_t k0 = kb + s * kMfKs;
        gload_x(k0 + kMfKs);
        gload_w(0, k0 + 2 * kMfKs);
        if constexpr (Q6) compute_q6(0, k0);
        else compute(0);
        if (s + 1 < nsteps) lstore(1, 1, k0 + kMfKs);
        __syncthreads();
        if (s + 1 >= nsteps) break;
        gload_x(k0 + 2 * kMfKs);
        gload_w(1, k0 + 3 * kMfKs);
        if constexpr (Q6) compute_q6(1, k0 + kMfKs);
        else compute(1);
        if (s + 2 < nsteps) lstore(0, 0, k0 + 2 * kMfKs);
        __syncthreads();
    }
    float* dst = gridDim.z > 1 ? part + static_cast<size_t>(blockIdx.z) * b * n : y;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int32_t mm = n0 + wn * 32 * WN + 32 * j + li;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int32_t t = t0 + wm * 32 * WM + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (t < b && mm < n) dst[static_cast<size_t>(t) * n + mm] = acc[i][j][r] * rs_at(t - t0);
            }
        }
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// vmcnt(N) and lgkmcnt(0), then a work-group barrier with no memory fence.
// __syncthreads() also waits for the direct-to-LDS loads issued for later
// steps (its release fence covers every outstanding write, those included),
// which put a memory round trip on every step.  Here each wave waits only for
// the loads the next step reads (vmcnt(N)) and for its own LDS writes
// (lgkmcnt(0)) before the barrier, so after it every wave sees both; the
// empty asm statements keep the compiler from moving LDS accesses across it.
template <int N>
__device__ __forceinline__ void step_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// The matrices of one Q4_K launch (one activation batch, the same K): x-tiles
// [tile0[i], tile0[i + 1]) are matrix i, n[i] rows, output y[i] [b x n[i]].
// A work-group picks its matrix with scalar compares and selects over the
// kernel arguments.  With split K the partials of range z are one [b x ntot]
// block, matrix i's [b x n[i]] part at b npre[i] in it (npre: rows of the
// matrices before i).
constexpr int kMaxMbMats = 4;
struct MbMats {
    const uint8_t* w[kMaxMbMats];
    float* y[kMaxMbMats];
    int32_t n[kMaxMbMats];
    int32_t tile0[kMaxMbMats];
    int32_t npre[kMaxMbMats];
    int32_t ntot;
    int32_t count;
};

// The outputs of a split-K reduce: flat partial indices [end[i - 1], end[i])
// go to y[i] (end[-1] = 0), each y[i] one contiguous [b x n] block.
struct RedMats {
    float* y[kMaxMbMats];
    size_t end[kMaxMbMats];
    int32_t count;
};

// ---- Q4_K and Q6_K, weights streamed through registers ------------------------
//
// A work-group is RT row tiles of 32 weight rows (one wave each) times 64
// tokens.  Each wave streams its rows' super-blocks straight from memory
// into registers, a super-block ahead: lane l holds row l % 32 and bytes
// 16 h .. 16 h + 15 (h = l / 32) of each sub-block pair's 32 qs bytes, i.e.
// values 16 h .. 16 h + 15 of both sub-blocks, which dequantised to sc q
// are its A operands of v_mfma_f32_32x32x16_f16: K slice s of a sub-block
// is values 16 h + 8 s .. + 8 in lane half h, and the activation operand is
// read from LDS in the same order, so each slice's products pair every
// value with its own activation.  The activations (q as fp16, the blocks'
// d / s and, for the min term, the P pairs) stream through three LDS
// stages, one super-block per stage, filled by direct-to-LDS loads two
// super-blocks ahead, issued with the next super-block's weights as a
// super-block starts; one barrier per super-block.  Each block's
// integer dot is one product, scaled on the VALU by the block's d_x / s into
// a super-block accumulator, and d, dmin and the min term fold once per
// super-block.  No weight is staged in LDS and nothing is barriered per 32
// values: a work-group's weights are read once, by the wave that uses them.
// With gridDim.z > 1 the work-group's result is a split-K partial.
// The result leaves through LDS, so that each store instruction writes one
// token's contiguous row range.
// Q6_K (cpp:742-757) takes the same structure: the weights are the integers
// sc (q - 32), d folds once per super-block and there is no min term.
// sc (q - 32) can need 12 bits (|sc| up to 128), so each is taken as two
// fp16 integers that are always exact, sc (l - 16) and 16 sc (u - 1) (q = l
// + 16 u, l the 4 bits from ql, u the 2 from qh), and a block's dot is two
// products per K slice (integers below 2^24: exact).  Lane half h takes
// values 16 h .. 16 h + 15 of each 32-value group of both 128-value halves:
// per half the 16 bytes of ql at 16 h and at 32 + 16 h and of qh at 16 h
// (all four groups' values), so a group's two K slices are again values
// 16 h + 8 s .. + 8.  Its blocks are only 2-byte aligned: each 16-byte piece
// is read as a dwordx4 from the dword at or below it plus one dword, and
// realigned.
constexpr int kQsTok = 64;            // tokens per work-group
constexpr int kQsXHalves = 64 * 260;  // halves per q stage: 64 x 256 of q, or 32 x (256 + 4) floats of output

// one super-block of a lane's weight row in registers
template <int TYPE>
struct QsW;
template <>
struct QsW<kQ4_K> {
    static constexpr int32_t kBytes = 144;
    u32x4 h, q[4];  // header; 16 bytes of each sub-block pair's qs
    __device__ __forceinline__ void load(const __amdgpu_buffer_rsrc_t& rs, int32_t off, int lh) {
        h = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
#pragma unroll
        for (int p = 0; p < 4; ++p) q[p] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 + 32 * p + 16 * lh, 0, 0);
    }
};
template <>
struct QsW<kQ6_K> {
    static constexpr int32_t kBytes = 210;
    // pieces: ql of half 0 at 16 h and 32 + 16 h, of half 1 at 64 + 16 h and
    // 96 + 16 h, qh at 128 + 16 h and 160 + 16 h, the scales and d at 192;
    // each as the 20 bytes from the dword at or below it
    u32x4 p[7];
    uint32_t e[7];
    static __device__ __forceinline__ int32_t piece(int i, int lh) {
        return i < 6 ? 32 * i + 16 * lh : 192;
    }
    __device__ __forceinline__ void load(const __amdgpu_buffer_rsrc_t& rs, int32_t off, int lh) {
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            const int32_t o = (off + piece(i, lh)) & ~3;
            p[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
            e[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, o + 16, 0, 0);
        }
    }
};

template <int TYPE, int RT>
__global__ __launch_bounds__(64 * RT, 1) void matbatch_qs_stream_kernel(
    MbMats mats, size_t rbytes, const _Float16* __restrict xq, const float* __restrict dxs,
    const _Float16* __restrict pq, const float* __restrict rscale, int32_t b, int32_t k, int32_t kchunk,
    float* __restrict part, int32_t xmap_tg) {
    constexpr int WAVES = RT, BM = kQsTok, BN = 32 * RT;
    static_assert(RT == 8, "one d / s row and one P slice per wave and stage");
    // stage s: q [token][256] with the 16-byte segments of token t at
    // positions c ^ (t % 16) (conflict-free reads of one segment by 16
    // tokens), d_x / s [block][token], P [token][8 hi, 8 lo]; separate
    // arrays, so that a load into one stage does not make the compiler wait
    // before reads of another
    __shared__ __align__(16) _Float16 xs0[kQsXHalves], xs1[kQsXHalves], xs2[kQsXHalves];
    __shared__ __align__(16) float sd0[8 * BM], sd1[8 * BM], sd2[8 * BM];
    __shared__ __align__(16) _Float16 sp0[16 * BM], sp1[16 * BM], sp2[16 * BM];
    __shared__ __align__(16) float srs[BM];
    __shared__ __align__(16) float sdm[WAVES][2][32];  // per wave: its rows' d and dmin

    // the work-group's row group, token group and K range.  Without a split
    // the 1-D grid can be dealt over the XCDs (work-group i runs on XCD i %
    // 8, each with its own L2): xmap > 0 (token groups, a multiple of 8):
    // each XCD keeps one eighth of the token groups and walks the row
    // groups, its concurrent work-groups sharing row groups' weights and its
    // token groups' activations; xmap < 0 (-row groups, a multiple of 8):
    // each XCD keeps one eighth of the row groups, token groups fastest, so
    // every weight is read by one XCD and the activations by all
    int bx, by, bz;
    if (xmap_tg > 0) {
        const int lin = static_cast<int>(blockIdx.x), xcd = lin & 7, slot = lin >> 3, tpx = xmap_tg / 8;
        bx = slot / tpx;
        by = xcd * tpx + slot % tpx;
        bz = 0;
    } else if (xmap_tg < 0) {
        const int lin = static_cast<int>(blockIdx.x), xcd = lin & 7, slot = lin >> 3;
        const int rgs = -xmap_tg, tgs = static_cast<int>(gridDim.x) / rgs;
        bx = xcd * (rgs / 8) + slot / tgs;
        by = slot % tgs;
        bz = 0;
    } else {
        bx = static_cast<int>(blockIdx.x);
        by = static_cast<int>(blockIdx.y);
        bz = static_cast<int>(blockIdx.z);
    }
    const uint8_t* __restrict w = mats.w[0];
    float* __restrict y = mats.y[0];
    int32_t n = mats.n[0], tile0 = 0, npre = 0;
#pragma unroll
    for (int i = 1; i < kMaxMbMats; ++i) {
        if (mats.count > i && bx >= mats.tile0[i]) {
            w = mats.w[i];
            y = mats.y[i];
            n = mats.n[i];
            tile0 = mats.tile0[i];
            npre = mats.npre[i];
        }
    }
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int32_t t0 = by * BM, n0 = (bx - tile0) * BN;
    const int32_t kb = bz * kchunk;
    const int32_t nsb = (min(k, kb + kchunk) - kb) / 256;  // super-blocks of the range
    const int32_t rows_here = min(BM, b - t0);

    // this lane's weight row, 32 wv + l % 32; rows past N and super-blocks
    // past the range read zeros (offsets past the resource)
    const int32_t wrows_here = min(BN, n - n0);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w + static_cast<size_t>(n0) * rbytes), static_cast<short>(0),
        wrows_here * static_cast<int32_t>(rbytes), 0x00020000);
    constexpr int32_t kWB = QsW<TYPE>::kBytes;
    const int32_t wbase = (32 * wv + li) * static_cast<int32_t>(rbytes) + (kb / 256) * kWB;
    using SbRegs = QsW<TYPE>;
    auto wload = [&](SbRegs& r, int32_t s) { r.load(wrs, s < nsb ? wbase + s * kWB : kMfOob, lh); };
    // the activations of super-block s into a stage: 4 q loads, one d / s
    // row and one P slice per wave (token rows past B read zeros)
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(xq + static_cast<size_t>(t0) * k), static_cast<short>(0),
        rows_here * k * static_cast<int32_t>(sizeof(_Float16)), 0x00020000);
    const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(dxs + static_cast<size_t>(t0) * (k / 32)), static_cast<short>(0),
        rows_here * (k / 32) * static_cast<int32_t>(sizeof(float)), 0x00020000);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(TYPE == kQ4_K ? pq + static_cast<size_t>(t0) * (k / 256) * 16 : xq), static_cast<short>(0),
        TYPE == kQ4_K ? rows_here * (k / 256) * 16 * static_cast<int32_t>(sizeof(_Float16)) : 0, 0x00020000);
    auto xload = [&](_Float16* xst, float* sdt, _Float16* spt, int32_t s) {
        const bool in = s < nsb;
        const int32_t k0 = kb + 256 * s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = i * WAVES + wv;  // token rows 2 q, 2 q + 1
            const int t = 2 * q + (lane >> 5), c = (lane & 31) ^ (t & 15);
            const int32_t off = in ? (t * k + k0 + 8 * c) * static_cast<int32_t>(sizeof(_Float16)) : kMfOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_ptr)(xst + 512 * q), 16, off, 0, 0, 0);
        }
        {
            const int32_t off = in ? (lane * (k / 32) + k0 / 32 + wv) * static_cast<int32_t>(sizeof(float)) : kMfOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(drs, (lds_ptr)(sdt + 64 * wv), 4, off, 0, 0, 0);
        }
        if constexpr (TYPE == kQ4_K) {
            const int dw = 64 * wv + lane, t = dw >> 3;
            const int32_t off =
                in ? ((t * (k / 256) + k0 / 256) * 16 + 2 * (dw & 7)) * static_cast<int32_t>(sizeof(_Float16)) : kMfOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(prs, (lds_ptr)(spt + 128 * wv), 4, off, 0, 0, 0);
        }
    };
    // activation loads per wave and super-block (q; d / s; Q4_K: P)
    constexpr int kXLoads = TYPE == kQ4_K ? 6 : 5;
    if (tid < BM) srs[tid] = tid < rows_here ? rscale[t0 + tid] : 0.0f;
    SbRegs R0, R1;
    wload(R0, 0);
    xload(xs0, sd0, sp0, 0);
    xload(xs1, sd1, sp1, 1);
    step_barrier<kXLoads>();

    floatx16 acc[2], S[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[tt][r] = S[tt][r] = 0.0f;

    // one Q4_K super-block from its registers and stage
    auto process_q4k = [&](const QsW<kQ4_K>& R, const _Float16* xst, const float* sdt, const _Float16* spt) {
        if (lh == 0) {
            sdm[wv][0][li] = half_bits_to_float(R.h.x & 0xffffu);
            sdm[wv][1][li] = half_bits_to_float(R.h.x >> 16);
        }
        int sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) k4_scale_min(j, R.h.y, R.h.z, R.h.w, sc[j], mn[j]);
        const uint32_t qd[4][4] = {{R.q[0].x, R.q[0].y, R.q[0].z, R.q[0].w},
                                   {R.q[1].x, R.q[1].y, R.q[1].z, R.q[1].w},
                                   {R.q[2].x, R.q[2].y, R.q[2].z, R.q[2].w},
                                   {R.q[3].x, R.q[3].y, R.q[3].z, R.q[3].w}};
        // block j's operands: activations of both token tiles and K slices,
        // their block scales, and the weights as sc q, two codes per
        // instruction: a byte permute puts codes a and c under the exponent
        // of 1024 (fp16 bits 0x6400 | a are 1024 + a), and one packed fma
        // gives (1024 + a) sc - 1024 sc = a sc with a single rounding of an
        // exact value (a sc <= 945)
        auto operands = [&](int j, half8 (&xo)[2][2], float (&dvv)[2], half8 (&wq)[2]) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int tr = 32 * tt + li;
#pragma unroll
                for (int sl = 0; sl < 2; ++sl) {
                    const int c = (4 * j + 2 * lh + sl) ^ (tr & 15);
                    xo[tt][sl] = *reinterpret_cast<const half8*>(&xst[256 * tr + 8 * c]);
                }
                dvv[tt] = sdt[64 * j + tr];
            }
            const _Float16 scf = static_cast<_Float16>(static_cast<float>(sc[j]));
            const _Float16 off = static_cast<_Float16>(-1024.0f * static_cast<float>(sc[j]));
            const half2 s2 = {scf, scf}, m2 = {off, off};
            uint32_t o[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t x = (qd[j >> 1][d] >> (4 * (j & 1))) & 0x0f0f0f0fu;
                const half2 p0 = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u));
                const half2 p1 = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u));
                o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p0, s2, m2));
                o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(p1, s2, m2));
            }
            wq[0] = __builtin_bit_cast(half8, make_uint4(o[0], o[1], o[2], o[3]));
            wq[1] = __builtin_bit_cast(half8, make_uint4(o[4], o[5], o[6], o[7]));
        };
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            half8 xo[2][2], wq[2];
            float dvv[2];
            operands(j, xo, dvv, wq);
            floatx16 blk[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const floatx16 zero = {};
                blk[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq[0], xo[tt][0], zero, 0, 0, 0);
                blk[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wq[1], xo[tt][1], blk[tt], 0, 0, 0);
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) S[tt][r] = j == 0 ? dvv[tt] * blk[tt][r] : fmaf(dvv[tt], blk[tt][r], S[tt][r]);
        }
        // acc += d S - dmin (m . P); the mins of sub-blocks 4 h .. + 3 are
        // the min product's A operand (K = the super-block's 8 sub-blocks)
        half4 mn4;
#pragma unroll
        for (int q = 0; q < 4; ++q) mn4[q] = static_cast<_Float16>(static_cast<float>(lh ? mn[4 + q] : mn[q]));
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int tr = 32 * tt + li;
            const half4 ph = *reinterpret_cast<const half4*>(&spt[16 * tr + 4 * lh]);
            const half4 pl = *reinterpret_cast<const half4*>(&spt[16 * tr + 8 + 4 * lh]);
            const floatx16 zero = {};
            floatx16 M = __builtin_amdgcn_mfma_f32_32x32x8f16(mn4, ph, zero, 0, 0, 0);
            M = __builtin_amdgcn_mfma_f32_32x32x8f16(mn4, pl, M, 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 d4 = *reinterpret_cast<const float4*>(&sdm[wv][0][8 * g + 4 * lh]);
                const float4 m4 = *reinterpret_cast<const float4*>(&sdm[wv][1][8 * g + 4 * lh]);
                const float dq[4] = {d4.x, d4.y, d4.z, d4.w}, mq[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 4 * g + q;
                    acc[tt][r] = fmaf(S[tt][r], dq[q], acc[tt][r]);
                    acc[tt][r] = fmaf(M[r], -mq[q], acc[tt][r]);
                }
            }
        }
    };

    // one Q6_K super-block (index sidx of the range) from its registers and stage
    auto process_q6k = [&](const QsW<kQ6_K>& R, const _Float16* xst, const float* sdt, int32_t sidx) {
        // pieces realigned as they are used (blocks are 2-byte aligned: the shift is 0 or 2)
        const int sh = (wbase + sidx * kWB) & 3;
        auto piece = [&](int i, int d) {
            const uint32_t lo = d == 0 ? R.p[i].x : d == 1 ? R.p[i].y : d == 2 ? R.p[i].z : R.p[i].w;
            const uint32_t hi = d == 0 ? R.p[i].y : d == 1 ? R.p[i].z : d == 2 ? R.p[i].w : R.e[i];
            return __builtin_amdgcn_alignbyte(hi, lo, sh);
        };
        if (lh == 0) sdm[wv][0][li] = half_bits_to_float((R.e[6] >> (8 * sh)) & 0xffffu);
        // the lane's scales: group g of half hf uses byte 8 hf + 2 g + h of the 16
        int sc[2][4];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t wd = piece(6, 2 * hf + (g >> 1));
                sc[hf][g] = static_cast<int>(static_cast<int8_t>((wd >> (8 * (2 * (g & 1) + lh))) & 0xffu));
            }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int jb = 4 * hf + g;  // the 32-value block of the super-block
                half8 xo[2][2];
                float dvv[2];
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int tr = 32 * tt + li;
#pragma unroll
                    for (int sl = 0; sl < 2; ++sl) {
                        const int c = (4 * jb + 2 * lh + sl) ^ (tr & 15);
                        xo[tt][sl] = *reinterpret_cast<const half8*>(&xst[256 * tr + 8 * c]);
                    }
                    dvv[tt] = sdt[64 * jb + tr];
                }
                // sc (q - 32) = sc (l - 16) + 16 sc (u - 1) with q = l + 16 u
                // (l the ql nibble, u the qh pair): |sc (l - 16)| <= 2048 and
                // 16 sc (u - 1) = 16 x an integer of at most 256, both exact in
                // fp16 for every int8 scale; from the fp16 integers 1024 + l and
                // 1024 + u, one exact add and one exact multiply each
                const _Float16 scf = static_cast<_Float16>(static_cast<float>(sc[hf][g]));
                const _Float16 sc16 = static_cast<_Float16>(16.0f * static_cast<float>(sc[hf][g]));
                const half2 s1 = {scf, scf}, s2 = {sc16, sc16};
                const half2 o1 = {static_cast<_Float16>(-1040.0f), static_cast<_Float16>(-1040.0f)};
                const half2 o2 = {static_cast<_Float16>(-1025.0f), static_cast<_Float16>(-1025.0f)};
                uint32_t a1[8], a2[8];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t l4 = (piece(2 * hf + (g & 1), d) >> (4 * (g >> 1))) & 0x0f0f0f0fu;
                    const uint32_t u4 = (piece(4 + hf, d) >> (2 * g)) & 0x03030303u;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const uint32_t sel = e == 0 ? 0x04010400u : 0x04030402u;
                        const half2 pl = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, l4, sel));
                        const half2 pu = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, u4, sel));
                        a1[2 * d + e] = __builtin_bit_cast(uint32_t, (pl + o1) * s1);
                        a2[2 * d + e] = __builtin_bit_cast(uint32_t, (pu + o2) * s2);
                    }
                }
                const half8 w10 = __builtin_bit_cast(half8, make_uint4(a1[0], a1[1], a1[2], a1[3]));
                const half8 w11 = __builtin_bit_cast(half8, make_uint4(a1[4], a1[5], a1[6], a1[7]));
                const half8 w20 = __builtin_bit_cast(half8, make_uint4(a2[0], a2[1], a2[2], a2[3]));
                const half8 w21 = __builtin_bit_cast(half8, make_uint4(a2[4], a2[5], a2[6], a2[7]));
                floatx16 blk[2];
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const floatx16 zero = {};
                    blk[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w10, xo[tt][0], zero, 0, 0, 0);
                    blk[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w11, xo[tt][1], blk[tt], 0, 0, 0);
                    blk[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w20, xo[tt][0], blk[tt], 0, 0, 0);
                    blk[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w21, xo[tt][1], blk[tt], 0, 0, 0);
                }
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        S[tt][r] = jb == 0 ? dvv[tt] * blk[tt][r] : fmaf(dvv[tt], blk[tt][r], S[tt][r]);
            }
        // acc += d S (d of the accumulator's rows, from the wave's exchange slots)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 d4 = *reinterpret_cast<const float4*>(&sdm[wv][0][8 * g + 4 * lh]);
                acc[tt][4 * g] = fmaf(S[tt][4 * g], d4.x, acc[tt][4 * g]);
                acc[tt][4 * g + 1] = fmaf(S[tt][4 * g + 1], d4.y, acc[tt][4 * g + 1]);
                acc[tt][4 * g + 2] = fmaf(S[tt][4 * g + 2], d4.z, acc[tt][4 * g + 2]);
                acc[tt][4 * g + 3] = fmaf(S[tt][4 * g + 3], d4.w, acc[tt][4 * g + 3]);
            }
    };
    auto process = [&](const SbRegs& R, const _Float16* xst, const float* sdt, const _Float16* spt, int32_t sidx) {
        if constexpr (TYPE == kQ4_K) {
            (void)sidx;
            process_q4k(R, xst, sdt, spt);
        } else {
            (void)spt;
            process_q6k(R, xst, sdt, sidx);
        }
    };

    // super-block s in register set s % 2 and stage s % 3: each starts
    // the loads of the next super-block's weights and of the activations two
    // ahead (into the stage the one before it left), and ends with the
    // barrier after which the next is in place for every wave (only the
    // activations two ahead may still be in flight) and its own stage may be
    // refilled
#define GNCX_QS_STEP(RA, RB, XA, DA, PA, XC, DC, PC, OFF) \
    wload(RB, s + (OFF) + 1);                        \
    xload(XC, DC, PC, s + (OFF) + 2);                \
    process(RA, XA, DA, PA, s + (OFF));              \
    step_barrier<kXLoads>();                         \
    if (s + (OFF) + 1 >= nsb) break;
    for (int32_t s = 0; s < nsb; s += 6) {
        GNCX_QS_STEP(R0, R1, xs0, sd0, sp0, xs2, sd2, sp2, 0)
        GNCX_QS_STEP(R1, R0, xs1, sd1, sp1, xs0, sd0, sp0, 1)
        GNCX_QS_STEP(R0, R1, xs2, sd2, sp2, xs1, sd1, sp1, 2)
        GNCX_QS_STEP(R1, R0, xs0, sd0, sp0, xs2, sd2, sp2, 3)
        GNCX_QS_STEP(R0, R1, xs1, sd1, sp1, xs0, sd0, sp0, 4)
        GNCX_QS_STEP(R1, R0, xs2, sd2, sp2, xs1, sd1, sp1, 5)
    }
#undef GNCX_QS_STEP

    // the tile of token tile tt in stage tt's q array as [32 tokens][BN + 4]
    // floats (rows padded: conflict-free), then whole token rows out
    constexpr int OLD = BN + 4;
    static_assert(32 * OLD * 2 <= kQsXHalves, "an output tile fits in a stage");
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        float* ost = reinterpret_cast<float*>(tt == 0 ? xs0 : xs1);
        const float rs = srs[32 * tt + li];
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<float4*>(&ost[li * OLD + 32 * wv + 8 * g + 4 * lh]) =
                make_float4(acc[tt][4 * g] * rs, acc[tt][4 * g + 1] * rs, acc[tt][4 * g + 2] * rs,
                            acc[tt][4 * g + 3] * rs);
    }
    __syncthreads();
    float* dst = gridDim.z > 1 ? part + (static_cast<size_t>(bz) * mats.ntot + npre) * b : y;
    const int32_t rows = min(BN, n - n0);
    if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        // 4 rows per lane, BN / 4 lanes per token
        constexpr int LPT = BN / 4, TPI = 64 * WAVES / LPT;
        const int c = 4 * (tid % LPT);
        for (int tl = tid / LPT; tl < rows_here; tl += TPI) {
            const float* ost = reinterpret_cast<const float*>(tl < 32 ? xs0 : xs1);
            if (c < rows)
                *reinterpret_cast<float4*>(&dst[static_cast<size_t>(t0 + tl) * n + n0 + c]) =
                    *reinterpret_cast<const float4*>(&ost[(tl & 31) * OLD + c]);
        }
    } else {
        for (int e = tid; e < rows_here * BN; e += 64 * WAVES) {
            const int tl = e / BN, c = e % BN;
            const float* ost = reinterpret_cast<const float*>(tl < 32 ? xs0 : xs1);
            if (c < rows) dst[static_cast<size_t>(t0 + tl) * n + n0 + c] = ost[(tl & 31) * OLD + c];
        }
    }
}

// y = sum over the split K ranges, added in range order (deterministic);
// range z's partials are the flat block [z count, (z + 1) count).  The
// first kRedU ranges are loaded together before the adds (a loop of
// load-then-add waited on memory once per range).
constexpr int kRedU = 16;

__global__ __launch_bounds__(kThreads) void matbatch_reduce_kernel(const float* __restrict part, int32_t splits,
                                                                   RedMats r) {
    const size_t count = r.end[r.count - 1];
    for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * kThreads) {
        float v[kRedU];
#pragma unroll
        for (int u = 0; u < kRedU; ++u) v[u] = u < splits ? part[static_cast<size_t>(u) * count + i] : 0.0f;
        float acc = v[0];
#pragma unroll
        for (int u = 1; u < kRedU; ++u)
            if (u < splits) acc += v[u];
        for (int32_t z = kRedU; z < splits; ++z) acc += part[static_cast<size_t>(z) * count + i];
        float* y = r.y[0];
        size_t first = 0;
#pragma unroll
        for (int m = 1; m < kMaxMbMats; ++m) {
            if (r.count > m && i >= r.end[m - 1]) {
                y = r.y[m];
                first = r.end[m - 1];
            }
        }
        y[i - first] = acc;
    }
}

hipError_t launch_reduce(const float* part, int32_t splits, const RedMats& r, hipStream_t stream) {
    size_t g = (r.end[r.count - 1] + kThreads - 1) / kThreads;
    if (g > 4096) g = 4096;
    hipLaunchKernelGGL(matbatch_reduce_kernel, dim3(static_cast<unsigned>(g)), dim3(kThreads), 0, stream, part,
                       splits, r);
    return hipGetLastError();
}

struct MfmaPlan {
    int wm, wn;
    int32_t splits, kchunk;
    int mw = 2;  // waves along the tokens (4: 512-thread work-groups)
};

// From 129 tokens, 256-token tiles of 8 waves (one work-group per CU, 111 KB
// of LDS): 256 x 128 when that gives at least 192 tiles, else 256 x 64 when
// that does, else 256 x 128 with K split until about 256 work-groups run.
// Twice the tokens per dequantised weight step, with the dequantising waves
// and MFMA-only waves sharing each SIMD, measured 1.1-1.4x the 128 x 128 tile
// (Q4_K 4096 x 14336 at B = 512: 111 vs 141 us; 4096 x 4096 at B = 2048: 116
// vs 149 us) with bit-identical results (same K order); with K split, Q6_K
// 14336 -> 4096 at B = 200 / 256 / 512 took 139 / 144 / 258 us against 266 /
// 268 / 480 us for 64 x 64 tiles with K split.  From 65 to 128 tokens,
// 128 x 128 tiles of 4 waves with K split until about 512 work-groups run
// (Q6_K 14336 -> 4096 at B = 128: 108 against 157 us).  Up to 64 tokens, the
// largest tile whose grid fills every CU with as many work-groups as its LDS
// lets one CU hold (2 for 128 x 128 and 128 x 64, 4 for 64 x 64), else 64 x 64
// tiles with K split until it does (ranges of at least 256).
MfmaPlan mfma_plan(int32_t b, int32_t k, int32_t n) {
    auto tiles = [&](int wm, int wn) {
        return static_cast<int64_t>((n + 64 * wn - 1) / (64 * wn)) * ((b + 64 * wm - 1) / (64 * wm));
    };
    if (b > 128) {
        const int64_t mt = (b + 255) / 256;
        const int64_t t = static_cast<int64_t>((n + 127) / 128) * mt;
        if (t >= 192) return {2, 2, 1, k, 4};
        if (static_cast<int64_t>((n + 63) / 64) * mt >= 192) return {2, 1, 1, k, 4};
        // fewer tiles: 256 x 128 with K split (ranges of whole 256-value
        // blocks) until about 256 work-groups run
        int32_t splits = static_cast<int32_t>(256 / t);
        if (splits > k / 256) splits = k / 256;
        if (splits <= 1) return {2, 2, 1, k, 4};
        const int32_t kchunk = (k / 256 + splits - 1) / splits * 256;
        return {2, 2, (k + kchunk - 1) / kchunk, kchunk, 4};
    }
    if (b > 64) {
        // 128 x 128 tiles of 4 waves, with K split until about 512 work-groups run
        const int64_t t = tiles(2, 2);
        int32_t splits = static_cast<int32_t>(512 / t);
        if (splits > k / 256) splits = k / 256;
        if (splits <= 1) return {2, 2, 1, k};
        const int32_t kchunk = (k / 256 + splits - 1) / splits * 256;
        return {2, 2, (k + kchunk - 1) / kchunk, kchunk};
    }
    const int cand[3][3] = {{2, 2, 2}, {2, 1, 2}, {1, 1, 4}};
    for (const auto& c : cand)
        if (tiles(c[0], c[1]) >= 256 * c[2]) return {c[0], c[1], 1, k};
    const int64_t t = tiles(1, 1);
    int32_t splits = static_cast<int32_t>((1024 + t - 1) / t);
    const int32_t max_splits = k / 256 > 0 ? k / 256 : 1;
    if (splits > max_splits) splits = max_splits;
    int32_t kchunk = (k + splits - 1) / splits;
    kchunk = (kchunk + kMfKs - 1) / kMfKs * kMfKs;
    splits = (k + kchunk - 1) / kchunk;
    return {1, 1, splits, kchunk};
}

template <int TYPE, int WM, int WN, int MW = 2>
hipError_t launch_mfma_t(const uint8_t* w, const _Float16* xhl, const float* rscale, int32_t b, int32_t k,
                         int32_t n, float* y, const MfmaPlan& p, float* part, hipStream_t stream) {
    constexpr int BM = 32 * WM * MW;
    const dim3 grid((n + 64 * WN - 1) / (64 * WN), (b + BM - 1) / BM, p.splits);
    hipLaunchKernelGGL((matbatch_mfma_kernel<TYPE, WM, WN, MW>), grid, dim3(128 * MW), 0, stream, w,
                       row_bytes(TYPE, k), xhl, rscale, b, k, n, y, p.kchunk, part);
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_mfma(const uint8_t* w, const float* x, int32_t b, int32_t k, int32_t n, float* y, _Float16* xhl,
                       float* rscale, float* part, hipStream_t stream, const float* up) {
    launch_act_hilo(x, b, k, xhl, rscale, nullptr, stream, up);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const MfmaPlan p = mfma_plan(b, k, n);
    if (p.mw == 4 && p.wn == 2) e = launch_mfma_t<TYPE, 2, 2, 4>(w, xhl, rscale, b, k, n, y, p, part, stream);
    else if (p.mw == 4) e = launch_mfma_t<TYPE, 2, 1, 4>(w, xhl, rscale, b, k, n, y, p, part, stream);
    else if (p.wn == 2) e = launch_mfma_t<TYPE, 2, 2>(w, xhl, rscale, b, k, n, y, p, part, stream);
    else if (p.wm == 2) e = launch_mfma_t<TYPE, 2, 1>(w, xhl, rscale, b, k, n, y, p, part, stream);
    else e = launch_mfma_t<TYPE, 1, 1>(w, xhl, rscale, b, k, n, y, p, part, stream);
    if (e != hipSuccess || p.splits == 1) return e;
    RedMats r{};
    r.y[0] = y;
    r.end[0] = static_cast<size_t>(b) * n;
    r.count = 1;
    return launch_reduce(part, p.splits, r, stream);
}

// A launch plan of matbatch_qs_stream_kernel: K ranges and the XCD order
struct Q4kPlan {
    int32_t splits, kchunk;
    int32_t xmap = 0;  // token groups of the XCD-aware order (> 0), minus row groups (< 0), 0: grid order
};

// Row groups of 256 x 64 tokens, K split in ranges of whole super-blocks
// until about 256 work-groups run (one per CU).
Q4kPlan q4k_stream_plan(int32_t b, int32_t k, int32_t n) {
    Q4kPlan p{1, k};
    const int32_t nsb = k / 256;
    const int64_t rg = (n + 255) / 256, tg = (b + kQsTok - 1) / kQsTok, wgs = rg * tg;
    int32_t splits = wgs >= 256 ? 1 : static_cast<int32_t>(256 / wgs);
    splits = std::max(1, std::min(splits, nsb));
    const int32_t csb = (nsb + splits - 1) / splits;
    p.kchunk = csb * 256;
    p.splits = (nsb + csb - 1) / csb;
    // the XCD order with the least L2-miss traffic, counting each XCD's own
    // reads: by token groups every XCD reads all weights W and its share of
    // the activations X; by row groups one XCD reads each weight and every
    // XCD the activations once per round of 32 work-groups (rg tg / 256)
    p.xmap = 0;
    if (p.splits == 1) {
        const double w = static_cast<double>(n) * (k / 256) * 210.0, x = static_cast<double>(b) * k * 2.2;
        const double by_tok = 8.0 * w + x, by_row = w + 8.0 * x * std::max(1.0, static_cast<double>(wgs) / 256.0);
        if (rg % 8 == 0 && (tg % 8 != 0 || by_row < by_tok)) p.xmap = -static_cast<int32_t>(rg);
        else if (tg % 8 == 0) p.xmap = static_cast<int32_t>(tg);
    }
    return p;
}

Q4kPlan q4k_plan(int32_t b, int32_t k, int32_t n) { return q4k_stream_plan(b, k, n); }

// rows per row group of the streamed kernel (8 waves x 32 rows)
constexpr int32_t kQ4kTileRows = 256;

// the streamed kernel's activations: q as fp16 in xhl's first B K halves and
// the blocks' d / s after them (the pairs' space holds both)
float* q4k_dxs(_Float16* xhl, int32_t b, int32_t k) { return reinterpret_cast<float*>(xhl + static_cast<size_t>(b) * k); }

void launch_q4k_act(const float* x, int32_t b, int32_t k, _Float16* xhl, float* rscale, _Float16* pq,
                    hipStream_t stream, const float* up) {
    launch_act_q(x, b, k, xhl, q4k_dxs(xhl, b, k), rscale, pq, stream, up);
}

template <int TYPE>
hipError_t launch_qs(const MbMats& m, const _Float16* xq, const float* dxs, const _Float16* pq,
                     const float* rscale, int32_t b, int32_t k, const Q4kPlan& p, float* part, hipStream_t stream) {
    constexpr int BN = 256;
    if (p.kchunk % 256 != 0) return hipErrorInvalidValue;
    const int32_t rg = m.tile0[m.count - 1] + (m.n[m.count - 1] + BN - 1) / BN, tg = (b + kQsTok - 1) / kQsTok;
    if (p.xmap > 0 && (p.xmap != tg || tg % 8 != 0 || p.splits != 1)) return hipErrorInvalidValue;
    if (p.xmap < 0 && (-p.xmap != rg || rg % 8 != 0 || p.splits != 1)) return hipErrorInvalidValue;
    const dim3 grid = p.xmap != 0 ? dim3(rg * tg) : dim3(rg, tg, p.splits);
    hipLaunchKernelGGL((matbatch_qs_stream_kernel<TYPE, 8>), grid, dim3(512), 0, stream, m, row_bytes(TYPE, k), xq,
                       dxs, pq, rscale, b, k, p.kchunk, part, p.xmap);
    return hipGetLastError();
}

#ifndef GNCX_Q6K_STREAM
#define GNCX_Q6K_STREAM 1
#endif
// Q6_K through matbatch_qs_stream_kernel (plan as q4k_stream_plan): the
// activations as q, d / s and row scales, the product, with split K the
// reduce
hipError_t launch_q6ks(const uint8_t* w, const float* x, int32_t b, int32_t k, int32_t n, float* y, _Float16* xhl,
                       float* rscale, float* part, hipStream_t stream, const float* up) {
    const Q4kPlan p = q4k_stream_plan(b, k, n);
    launch_act_q(x, b, k, xhl, q4k_dxs(xhl, b, k), rscale, nullptr, stream, up);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MbMats m{};
    m.w[0] = w;
    m.y[0] = y;
    m.n[0] = n;
    m.ntot = n;
    m.count = 1;
    e = launch_qs<kQ6_K>(m, xhl, q4k_dxs(xhl, b, k), nullptr, rscale, b, k, p, part, stream);
    if (e != hipSuccess || p.splits == 1) return e;
    RedMats r{};
    r.y[0] = y;
    r.end[0] = static_cast<size_t>(b) * n;
    r.count = 1;
    return launch_reduce(part, p.splits, r, stream);
}

// The product of plan p over the matrices of m (w, y, n and count set), then
// with split K the reduce of the partials into each y
hipError_t launch_q4k_mats(MbMats& m, _Float16* xhl, const _Float16* pq, const float* rscale, int32_t b,
                           int32_t k, const Q4kPlan& p, float* part, hipStream_t stream) {
    const int32_t bn = kQ4kTileRows;
    int32_t t = 0, rows = 0;
    RedMats r{};
    for (int32_t i = 0; i < m.count; ++i) {
        m.tile0[i] = t;
        m.npre[i] = rows;
        t += (m.n[i] + bn - 1) / bn;
        rows += m.n[i];
        r.y[i] = m.y[i];
        r.end[i] = static_cast<size_t>(b) * rows;
    }
    m.ntot = rows;
    r.count = m.count;
    const hipError_t e = launch_qs<kQ4_K>(m, xhl, q4k_dxs(xhl, b, k), pq, rscale, b, k, p, part, stream);
    if (e != hipSuccess || p.splits == 1) return e;
    return launch_reduce(part, p.splits, r, stream);
}

hipError_t launch_q4k(const uint8_t* w, const float* x, int32_t b, int32_t k, int32_t n, float* y, _Float16* xhl,
                      _Float16* pq, float* rscale, float* part, hipStream_t stream, const float* up) {
    const Q4kPlan p = q4k_plan(b, k, n);
    launch_q4k_act(x, b, k, xhl, rscale, pq, stream, up);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MbMats m{};
    m.w[0] = w;
    m.y[0] = y;
    m.n[0] = n;
    m.count = 1;
    return launch_q4k_mats(m, xhl, pq, rscale, b, k, p, part, stream);
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

// fp16 pairs of the quantised activations [B x K x 2] (or, for the
// streamed Q4_K / Q6_K kernel, q [B x K] and the blocks' d / s [B x K / 32]),
// their row scales [B], then the split-K partials [splits x B x N]
static size_t xh_bytes(int32_t b, int32_t k) {
    return (static_cast<size_t>(b) * k * 2 * sizeof(_Float16) + 255) & ~static_cast<size_t>(255);
}
static size_t rscale_bytes(int32_t b) { return (static_cast<size_t>(b) * sizeof(float) + 255) & ~static_cast<size_t>(255); }

// Q4_K: the activation sums of each 32-block as fp16 pairs [B x K/256 x 16]
static size_t pq_bytes(int32_t type, int32_t b, int32_t k) {
    return type == kQ4_K ? (static_cast<size_t>(b) * (k / 256) * 16 * sizeof(_Float16) + 255) & ~static_cast<size_t>(255)
                         : 0;
}

size_t matbatch_workspace_bytes(int32_t type, int32_t b, int32_t k, int32_t n) {
    if (type == kBF16) return 256;
    const int32_t splits = type == kQ4_K                     ? q4k_plan(b, k, n).splits
                           : type == kQ6_K && GNCX_Q6K_STREAM ? q4k_stream_plan(b, k, n).splits
                                                              : mfma_plan(b, k, n).splits;
    const size_t parts = splits > 1 ? static_cast<size_t>(splits) * b * n * sizeof(float) : 0;
    return xh_bytes(b, k) + pq_bytes(type, b, k) + rscale_bytes(b) + parts + 256;
}

hipError_t launch_matbatch(int32_t type, const uint8_t* w, const float* x, int32_t b, int32_t k, int32_t n,
                           float* y, void* workspace, size_t workspace_bytes, hipStream_t stream, const float* up) {
    if (b <= 0 || n <= 0) return hipSuccess;
    if (k <= 0 || k > (1 << 20) || b > 65535) return hipErrorInvalidValue;  // keeps buffer offsets in int32
    if (type != kBF16 && (k % 32) != 0) return hipErrorInvalidValue;
    if ((type == kQ4_K || type == kQ6_K) && (k % 256) != 0) return hipErrorInvalidValue;
    if (workspace_bytes < matbatch_workspace_bytes(type, b, k, n)) return hipErrorInvalidValue;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return hipErrorInvalidValue;
    if (type == kQ4_K || type == kBF16) {
        if ((wa & 15u) != 0 || (row_bytes(type, k) & 15u) != 0) return hipErrorInvalidValue;
    } else if ((wa & 3u) != 0) {
        return hipErrorInvalidValue;
    }
    char* ws = static_cast<char*>(workspace);
    _Float16* xhl = reinterpret_cast<_Float16*>(ws);
    _Float16* pq = reinterpret_cast<_Float16*>(ws + xh_bytes(b, k));
    float* rscale = reinterpret_cast<float*>(ws + xh_bytes(b, k) + pq_bytes(type, b, k));
    float* part = reinterpret_cast<float*>(ws + xh_bytes(b, k) + pq_bytes(type, b, k) + rscale_bytes(b));
    if ((reinterpret_cast<uintptr_t>(xhl) & 255u) != 0) return hipErrorInvalidValue;
    switch (type) {
    case kQ4_0: return launch_mfma<kQ4_0>(w, x, b, k, n, y, xhl, rscale, part, stream, up);
    case kQ8_0: return launch_mfma<kQ8_0>(w, x, b, k, n, y, xhl, rscale, part, stream, up);
    case kQ4_K: return launch_q4k(w, x, b, k, n, y, xhl, pq, rscale, part, stream, up);
    case kQ6_K:
        return GNCX_Q6K_STREAM ? launch_q6ks(w, x, b, k, n, y, xhl, rscale, part, stream, up)
                               : launch_mfma<kQ6_K>(w, x, b, k, n, y, xhl, rscale, part, stream, up);
    case kBF16: return up ? hipErrorNotSupported : launch_t<kBF16>(w, x, b, k, n, y, nullptr, nullptr, stream);
    default: return hipErrorInvalidValue;
    }
}


namespace {

// One launch over count Q4_K matrices sharing the activation batch (and with
// split K one reduce over all of them): when every matrix is whole x-tiles of
// the plan for the summed rows (false otherwise, and the matrices go one call
// each).
bool multi_fused(int32_t type, int32_t count, const int32_t* ns, int32_t b, int32_t k, Q4kPlan& p, int64_t& total) {
    if (type != kQ4_K || count < 2 || count > kMaxMbMats || b <= 0 || k <= 0 || (k % 256) != 0) return false;
    total = 0;
    for (int32_t i = 0; i < count; ++i) total += ns[i];
    if (total > INT32_MAX) return false;
    p = q4k_plan(b, k, static_cast<int32_t>(total));
    const int32_t bn = kQ4kTileRows;
    for (int32_t i = 0; i < count; ++i)
        if (ns[i] % bn != 0) return false;
    return true;
}

}  // namespace

size_t matbatch_multi_workspace_bytes(int32_t type, int32_t count, const int32_t* ns, int32_t b, int32_t k) {
    size_t need = 256;
    for (int32_t i = 0; i < count; ++i) need = std::max(need, matbatch_workspace_bytes(type, b, k, ns[i]));
    Q4kPlan p;
    int64_t total;
    if (multi_fused(type, count, ns, b, k, p, total)) {
        const size_t parts = p.splits > 1 ? static_cast<size_t>(p.splits) * b * total * sizeof(float) : 0;
        need = std::max(need, xh_bytes(b, k) + pq_bytes(type, b, k) + rscale_bytes(b) + parts + 256);
    }
    return need;
}

hipError_t launch_matbatch_multi(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns,
                                 const float* x, int32_t b, int32_t k, float* const* ys, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
    if (count <= 0 || count > kMaxMbMats || !ws || !ns || !ys) return hipErrorInvalidValue;
    for (int32_t i = 0; i < count; ++i)
        if (ns[i] <= 0 || !ws[i] || !ys[i]) return hipErrorInvalidValue;
    if (workspace_bytes < matbatch_multi_workspace_bytes(type, count, ns, b, k)) return hipErrorInvalidValue;
    Q4kPlan p;
    int64_t total;
    if (!multi_fused(type, count, ns, b, k, p, total)) {
        for (int32_t i = 0; i < count; ++i) {
            const hipError_t e = launch_matbatch(type, ws[i], x, b, k, ns[i], ys[i], workspace, workspace_bytes, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // the checks of launch_matbatch for Q4_K
    if (k > (1 << 20) || b > 65535) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (row_bytes(kQ4_K, k) & 15u) != 0) return hipErrorInvalidValue;
    for (int32_t i = 0; i < count; ++i)
        if ((reinterpret_cast<uintptr_t>(ws[i]) & 15u) != 0) return hipErrorInvalidValue;
    char* wsp = static_cast<char*>(workspace);
    _Float16* xhl = reinterpret_cast<_Float16*>(wsp);
    _Float16* pq = reinterpret_cast<_Float16*>(wsp + xh_bytes(b, k));
    float* rscale = reinterpret_cast<float*>(wsp + xh_bytes(b, k) + pq_bytes(kQ4_K, b, k));
    float* part = reinterpret_cast<float*>(wsp + xh_bytes(b, k) + pq_bytes(kQ4_K, b, k) + rscale_bytes(b));
    if ((reinterpret_cast<uintptr_t>(xhl) & 255u) != 0) return hipErrorInvalidValue;
    launch_q4k_act(x, b, k, xhl, rscale, pq, stream, nullptr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MbMats m{};
    for (int32_t i = 0; i < count; ++i) {
        m.w[i] = ws[i];
        m.y[i] = ys[i];
        m.n[i] = ns[i];
    }
    m.count = count;
    return launch_q4k_mats(m, xhl, pq, rscale, b, k, p, part, stream);
}

hipError_t launch_matbatch_multi_norm(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns,
                                      float* h, const float* r, const float* gamma, float eps, int32_t b, int32_t k,
                                      float* const* ys, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
    if (count <= 0 || count > kMaxMbMats || !ws || !ns || !ys || !h || !gamma) return hipErrorInvalidValue;
    for (int32_t i = 0; i < count; ++i)
        if (ns[i] <= 0 || !ws[i] || !ys[i]) return hipErrorInvalidValue;
    Q4kPlan p;
    int64_t total;
    if (!multi_fused(type, count, ns, b, k, p, total) || !norm_act_fits(h, r, gamma, k)) return hipErrorNotSupported;
    if (workspace_bytes < matbatch_multi_workspace_bytes(type, count, ns, b, k)) return hipErrorInvalidValue;
    if (k > (1 << 20) || b > 65535 || (row_bytes(kQ4_K, k) & 15u) != 0) return hipErrorInvalidValue;
    for (int32_t i = 0; i < count; ++i)
        if ((reinterpret_cast<uintptr_t>(ws[i]) & 15u) != 0) return hipErrorInvalidValue;
    char* wsp = static_cast<char*>(workspace);
    _Float16* xhl = reinterpret_cast<_Float16*>(wsp);
    _Float16* pq = reinterpret_cast<_Float16*>(wsp + xh_bytes(b, k));
    float* rscale = reinterpret_cast<float*>(wsp + xh_bytes(b, k) + pq_bytes(kQ4_K, b, k));
    float* part = reinterpret_cast<float*>(wsp + xh_bytes(b, k) + pq_bytes(kQ4_K, b, k) + rscale_bytes(b));
    if ((reinterpret_cast<uintptr_t>(xhl) & 255u) != 0) return hipErrorInvalidValue;
    launch_norm_act_q(h, r, gamma, eps, b, k, xhl, q4k_dxs(xhl, b, k), rscale, pq, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    MbMats m{};
    for (int32_t i = 0; i < count; ++i) {
        m.w[i] = ws[i];
        m.y[i] = ys[i];
        m.n[i] = ns[i];
    }
    m.count = count;
    return launch_q4k_mats(m, xhl, pq, rscale, b, k, p, part, stream);
}

}  // namespace gncx
