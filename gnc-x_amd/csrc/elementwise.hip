// elementwise.hip -- the small per-token kernels around the hot path, plus
// the block dequantiser used to prove the decoders bit-exact.
//   per-head RMSNorm      cpp:895-953    RMSNorm (fast path)  cpp:789-833
//   NEOX RoPE             cpp:1797-1862  SwiGLU               cpp:2038-2052
//   lm_head softcap       cpp:1726-1731  embedding row fetch  cpp:693-780
//   block decoders        cpp:85-112, 707-714, 734-759 and the dots' implicit
//                         Q4_0/Q4_K decoders (cpp:1023-1030, 1127-1178)
#include <hip/hip_runtime.h>

#include "gncx_act.h"
#include "gncx_device.h"
#include "gncx_launch.h"

namespace gncx {
namespace {

using namespace dev;

// One wave per head: the head is copied into LDS with coalesced loads, then
// head_inv_rms forms the reference's four sequential fp32 lane sums from the
// LDS copy (bit-exact with cpp:905-926) and the wave writes the result.  Heads
// longer than kHeadsMaxHd (whole-vector norms, n_heads = 1) read global memory.
constexpr int kHeadsMaxHd = 512;

__global__ __launch_bounds__(256) void rmsnorm_heads_kernel(float* __restrict v, const float* __restrict g,
                                                            int32_t n_heads, int32_t hd, float eps) {
#pragma clang fp contract(off)
    __shared__ float buf[4][kHeadsMaxHd];
    const int w = threadIdx.x >> 6;
    const int h = blockIdx.x * 4 + w;
    const int lane = threadIdx.x & 63;
    const bool active = h < n_heads;
    float* x = v + static_cast<size_t>(active ? h : 0) * hd;
    float* lx = buf[w];
    if (active)
        for (int i = lane; i < hd; i += 64) lx[i] = x[i];
    __syncthreads();
    if (!active) return;
    const float inv = head_inv_rms(lx, hd, eps, lane);
    for (int i = lane; i < hd; i += 64) {
        const float y = lx[i] * inv;
        x[i] = g ? y * g[i] : y;
    }
}

__global__ __launch_bounds__(256) void rmsnorm_heads_long_kernel(float* __restrict v, const float* __restrict g,
                                                                 int32_t n_heads, int32_t hd, float eps) {
#pragma clang fp contract(off)
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (h >= n_heads) return;
    float* x = v + static_cast<size_t>(h) * hd;
    const float inv = head_inv_rms(x, hd, eps, lane);
    for (int i = lane; i < hd; i += 64) {
        const float y = x[i] * inv;
        x[i] = g ? y * g[i] : y;
    }
}

// The 4-phase telemetry encode of one vector (reference cpp:842-889) by one
// work-group of kNormThreads: the largest |v| (at least 1e-9), the scale to
// the layer's integer range 9 R_k (R_k the repunit of k ones), then per
// element the rounded integer, its diagonal digit d (nearest multiple of R_k,
// at most 9), the residual from d R_k and the two sign bits, packed as the
// 4-byte token {phase, d, |residual| mod 2^16}.  Every float step is the
// reference's, correctly rounded and uncontracted, so the tokens are
// bit-exact.  qscale[0] receives the quant scale and qscale[1] (as a
// uint32) the cancellation count sum_d min(#positive, #negative) over the
// digits d (cpp:882-887).  red: kNormThreads / 64 floats of LDS.
// One element of the encode: the token, and the counter of its (sign, digit)
// pair (0-9: val >= 0, 10-19: val < 0) for the cancellation count.
struct EncScale {
    int64_t r_k;
    float to_int, inv_rk, half_rk;
};
template <class I>
__device__ __forceinline__ uint32_t encode_value(float v, const EncScale& e, uint32_t& ctr) {
#pragma clang fp contract(off)
    const I val = static_cast<I>(rintf(__fmul_rn(v, e.to_int)));
    const I av = val >= 0 ? val : -val;
    int32_t d = static_cast<int32_t>(__fmul_rn(__fadd_rn(static_cast<float>(av), e.half_rk), e.inv_rk));
    if (d > 9) d = 9;
    const I anchor = static_cast<I>(d) * static_cast<I>(e.r_k);
    const I res = val - (val >= 0 ? anchor : -anchor);
    const uint32_t ares = static_cast<uint32_t>(static_cast<uint16_t>(res >= 0 ? res : -res));
    const uint32_t phase = (val >= 0 ? 2u : 0u) | (res >= 0 ? 1u : 0u);
    ctr = static_cast<uint32_t>(d) + (val >= 0 ? 0u : 10u);
    return phase | (static_cast<uint32_t>(d) << 8) | (ares << 16);
}
// Up to k = 8 every integer of the encode (|val| <= 9 R_k < 10^9, the residual
// below 2 x 10^9) fits 32 bits, and the 32-bit steps give the 64-bit results.
constexpr int32_t kEnc32MaxK = 8;

// the scale of the layer's range from the largest |v| m (qscale[0] = m / 9 R_k)
__device__ __forceinline__ EncScale encode_scale(float m, int32_t lay_k, float* __restrict qscale) {
#pragma clang fp contract(off)
    EncScale e;
    e.r_k = 1;
    for (int i = 0; i < lay_k; ++i) e.r_k = e.r_k * 10 + 1;
    const float target = static_cast<float>(9 * e.r_k);
    e.to_int = __fdiv_rn(target, m);
    if (threadIdx.x == 0) *qscale = __fdiv_rn(m, target);
    e.inv_rk = __fdiv_rn(1.0f, static_cast<float>(e.r_k));
    e.half_rk = static_cast<float>(e.r_k >> 1);
    return e;
}

__device__ void encode_row(const float* v, int32_t dim, int32_t lay_k, uint32_t* __restrict tokens,
                           float* __restrict qscale, float* red) {
    __shared__ uint32_t signs[20];
    if (threadIdx.x < 20) signs[threadIdx.x] = 0;
    float m = 1e-9f;
    for (int32_t i = threadIdx.x; i < dim; i += blockDim.x) {
        const float a = fabsf(v[i]);
        m = a > m ? a : m;
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < static_cast<int>(blockDim.x / 64); ++w) m = red[w] > m ? red[w] : m;
    const EncScale e = encode_scale(m, lay_k, qscale);
    for (int32_t i = threadIdx.x; i < dim; i += blockDim.x) {
        uint32_t ctr;
        tokens[i] = lay_k <= kEnc32MaxK ? encode_value<int32_t>(v[i], e, ctr) : encode_value<int64_t>(v[i], e, ctr);
        __hip_atomic_fetch_add(&signs[ctr], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t c = 0;
        for (int d = 0; d < 10; ++d) c += signs[d] < signs[10 + d] ? signs[d] : signs[10 + d];
        reinterpret_cast<uint32_t*>(qscale)[1] = c;
    }
}

// RMSNorm of one row per work-group (cpp:789-833): x and gamma are read once
// as float4 (kept in registers for rows up to 16384 values), the sum of
// squares is a fp32 tree over the work-group, y = (x * inv) * gamma.
constexpr int kNormThreads = 1024;
constexpr int kNormRegs = 4;  // float4 per thread held in registers

// The encode of a row whose normalised values a work-group of kNormThreads
// holds in registers (y[j]: float4 t = threadIdx.x + kNormThreads j, t < n4):
// no second pass over memory, tokens stored as uint4 (16-byte aligned), and
// the (sign, digit) counts formed per wave with ballots instead of LDS
// atomics on 20 addresses.  Max, tokens and counts are those of encode_row
// (a max and integer counts do not depend on the order).
__device__ void encode_regs(const float4 (&y)[kNormRegs], int32_t n4, int32_t lay_k, uint32_t* __restrict tokens,
                            float* __restrict qscale) {
    __shared__ float red[kNormThreads / 64];
    __shared__ uint32_t cnt[kNormThreads / 64][20];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float m = 1e-9f;
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
        if (tid + kNormThreads * j < n4) {
            const float a0 = fabsf(y[j].x), a1 = fabsf(y[j].y), a2 = fabsf(y[j].z), a3 = fabsf(y[j].w);
            m = a0 > m ? a0 : m;
            m = a1 > m ? a1 : m;
            m = a2 > m ? a2 : m;
            m = a3 > m ? a3 : m;
        }
    }
    m = wave_max(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < kNormThreads / 64; ++i) m = red[i] > m ? red[i] : m;
    const EncScale e = encode_scale(m, lay_k, qscale);
    uint4* t4 = reinterpret_cast<uint4*>(tokens);
    const bool small = lay_k <= kEnc32MaxK;
    uint32_t n[20] = {};
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
        if (kNormThreads * j >= n4) break;  // no thread holds float4 j
        const int32_t t = tid + kNormThreads * j;
        uint32_t ctr[4] = {20u, 20u, 20u, 20u};  // 20: counted nowhere
        if (t < n4) {
            uint4 tk;
            const float* yj = &y[j].x;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                (&tk.x)[q] = small ? encode_value<int32_t>(yj[q], e, ctr[q]) : encode_value<int64_t>(yj[q], e, ctr[q]);
            t4[t] = tk;
        }
#pragma unroll
        for (uint32_t c = 0; c < 20; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) n[c] += static_cast<uint32_t>(__popcll(__ballot(ctr[q] == c)));
    }
    if (lane == 0)
#pragma unroll
        for (int c = 0; c < 20; ++c) cnt[w][c] = n[c];
    __syncthreads();
    if (w == 0) {
        // lane d < 10 sums digit d's two counts over the waves; the ten
        // minima meet in one wave sum (integers below 2^24: exact in fp32)
        float mn = 0.0f;
        if (lane < 10) {
            uint32_t pos = 0, neg = 0;
#pragma unroll
            for (int i = 0; i < kNormThreads / 64; ++i) {
                pos += cnt[i][lane];
                neg += cnt[i][10 + lane];
            }
            mn = static_cast<float>(pos < neg ? pos : neg);
        }
        mn = wave_sum(mn);
        if (lane == 0) reinterpret_cast<uint32_t*>(qscale)[1] = static_cast<uint32_t>(mn);
    }
}

// ADD: x is the residual stream h (row blockIdx.x), updated in place to h + r
// before it is normalised -- the fp32 add of the separate vec_add kernel, so
// the result is the same bit for bit.  ENC: the 4-phase encode of the
// normalised row follows in the same work-group (one row).
template <bool ADD, bool ENC = false>
// (x and xo are the same row under ADD: no __restrict on the row pointers)
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* x, const float* __restrict g,
                                                               int32_t dim, float eps, float* out, int32_t vec4,
                                                               const float* r, float* xo, int32_t lay_k = 0,
                                                               uint32_t* tokens = nullptr, float* qscale = nullptr) {
#pragma clang fp contract(off)
    __shared__ float part[kNormThreads / 64];
    const float* xr = x + static_cast<size_t>(blockIdx.x) * dim;
    float* yr = out + static_cast<size_t>(blockIdx.x) * dim;
    if (ADD) {  // one row per work-group: its residual row and delta row
        r += static_cast<size_t>(blockIdx.x) * dim;
        xo += static_cast<size_t>(blockIdx.x) * dim;
    }
    const int tid = threadIdx.x;
    float s = 0.0f;
    float4 xv[kNormRegs], gv[kNormRegs];
    const int32_t n4 = vec4 ? dim / 4 : 0;
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const float4* g4 = reinterpret_cast<const float4*>(g);
    const float4* r4 = reinterpret_cast<const float4*>(r);
    float4* xo4 = reinterpret_cast<float4*>(xo);
    auto add4 = [](float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); };
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
        const int32_t t = tid + kNormThreads * j;
        if (t < n4) {
            xv[j] = x4[t];
            if (ADD) {
                xv[j] = add4(xv[j], r4[t]);
                xo4[t] = xv[j];
            }
            gv[j] = g4[t];
            s += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
        }
    }
    for (int32_t t = tid + kNormThreads * kNormRegs; t < n4; t += kNormThreads) {
        float4 a = x4[t];
        if (ADD) {
            a = add4(a, r4[t]);
            xo4[t] = a;
        }
        s += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    for (int32_t i = 4 * n4 + tid; i < dim; i += kNormThreads) {
        float a = xr[i];
        if (ADD) {
            a = a + r[i];
            xo[i] = a;
        }
        s += a * a;
    }
    // rows past the registers are read again below: from xo, which now holds h + r
    if (ADD) {
        xr = xo;
        x4 = reinterpret_cast<const float4*>(xo);
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) tot += part[w];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
    float4* y4 = reinterpret_cast<float4*>(yr);
    float4 yv[kNormRegs];
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
        const int32_t t = tid + kNormThreads * j;
        yv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t < n4) {
            yv[j] = make_float4(xv[j].x * inv * gv[j].x, xv[j].y * inv * gv[j].y, xv[j].z * inv * gv[j].z,
                                xv[j].w * inv * gv[j].w);
            y4[t] = yv[j];
        }
    }
    for (int32_t t = tid + kNormThreads * kNormRegs; t < n4; t += kNormThreads) {
        const float4 a = x4[t], b = g4[t];
        y4[t] = make_float4(a.x * inv * b.x, a.y * inv * b.y, a.z * inv * b.z, a.w * inv * b.w);
    }
    for (int32_t i = 4 * n4 + tid; i < dim; i += kNormThreads) yr[i] = xr[i] * inv * g[i];
    if constexpr (ENC) {
        // the whole row in registers and 16-byte token stores: encode from
        // the registers; otherwise from the row just stored
        if (4 * n4 == dim && n4 <= kNormThreads * kNormRegs && (reinterpret_cast<uintptr_t>(tokens) & 15u) == 0) {
            encode_regs(yv, n4, lay_k, tokens, qscale);
            return;
        }
        __threadfence_block();
        __syncthreads();
        encode_row(yr, dim, lay_k, tokens, qscale, part);
    }
}

__global__ void rope_kernel(float* __restrict q, float* __restrict k, RopeTable t, int32_t n_heads,
                            int32_t n_kv, int32_t hd) {
#pragma clang fp contract(off)
    const int half = hd / 2;
    const int total = (n_heads + n_kv) * half;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int h = idx / half, i = idx % half;
        float* v = h < n_heads ? (q ? q + static_cast<size_t>(h) * hd : nullptr)
                               : (k ? k + static_cast<size_t>(h - n_heads) * hd : nullptr);
        if (!v) continue;
        const float x1 = v[i], x2 = v[i + half];
        v[i] = x1 * t.c[i] - x2 * t.s[i];
        v[i + half] = x2 * t.c[i] + x1 * t.s[i];
    }
}

__global__ void swiglu_kernel(const float* __restrict g, const float* __restrict u, int32_t n,
                              float* __restrict out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = swiglu_value(g[i], u[i]);
}

// tanh-approximated GELU of the gate times up, in the reference's order of
// operations (cpp:2024-2030) with no contraction into fused multiply-adds.
__global__ void geglu_kernel(const float* __restrict g, const float* __restrict u, int32_t n,
                             float* __restrict out) {
    constexpr float kSqrt2OverPi = 0.7978845608028654f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float x = g[i];
        const float cube = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x);
        const float t = tanhf(__fmul_rn(kSqrt2OverPi, __fadd_rn(x, cube)));
        out[i] = __fmul_rn(__fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, t)), u[i]);
    }
}

__global__ void vec_add_kernel(float* __restrict y, const float* __restrict x, int32_t n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) y[i] += x[i];
}

__global__ void softcap_kernel(float* __restrict y, int32_t n, float cap) {
    const float inv = __fdiv_rn(1.0f, cap);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        y[i] = __fmul_rn(tanhf(__fmul_rn(y[i], inv)), cap);
}

// Decode element e of a row (all decoders are exact: every product below is
// representable in fp32, except where the reference also rounds).
__device__ __forceinline__ float decode_elem(int32_t type, const uint8_t* __restrict row, int32_t e, float scale) {
    if (type == kQ4_0) {
        const uint8_t* blk = row + static_cast<size_t>(e / 32) * 18;
        const int j = e % 32;
        const float d = half_bits_to_float(ld_u16(blk));
        const int b = blk[2 + (j & 15)];
        const int qv = (j < 16 ? (b & 15) : (b >> 4)) - 8;
        return __fmul_rn(d, static_cast<float>(qv));
    }
    if (type == kQ8_0) {
        const uint8_t* blk = row + static_cast<size_t>(e / 32) * 34;
        const float d = __fmul_rn(half_bits_to_float(ld_u16(blk)), scale);
        return __fmul_rn(static_cast<float>(static_cast<int8_t>(blk[2 + e % 32])), d);
    }
    if (type == kQ4_K) {
        const uint8_t* blk = row + static_cast<size_t>(e / 256) * 144;
        const int r = e % 256, c = r / 64, hi = (r % 64) / 32, l = r % 32;
        const uint32_t s0 = blk[4] | (blk[5] << 8) | (blk[6] << 16) | (static_cast<uint32_t>(blk[7]) << 24);
        const uint32_t s1 = blk[8] | (blk[9] << 8) | (blk[10] << 16) | (static_cast<uint32_t>(blk[11]) << 24);
        const uint32_t s2 = blk[12] | (blk[13] << 8) | (blk[14] << 16) | (static_cast<uint32_t>(blk[15]) << 24);
        int sc, mn;
        k4_scale_min(2 * c + hi, s0, s1, s2, sc, mn);
        const float d = half_bits_to_float(ld_u16(blk)), dmin = half_bits_to_float(ld_u16(blk + 2));
        const int b = blk[16 + 32 * c + l];
        const int qv = hi ? (b >> 4) : (b & 15);
        return __fsub_rn(__fmul_rn(__fmul_rn(d, static_cast<float>(sc)), static_cast<float>(qv)),
                         __fmul_rn(dmin, static_cast<float>(mn)));
    }
    if (type == kQ6_K) {
        const uint8_t* blk = row + static_cast<size_t>(e / 256) * 210;
        const int r = e % 256, h = r / 128, rr = r % 128, grp = rr / 32, l = rr % 32;
        const uint8_t* ql = blk + 64 * h;
        const uint8_t* qh = blk + 128 + 32 * h;
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * h);
        const int lo4 = (grp & 1) ? ql[l + 32] : ql[l];
        const int low = (grp >= 2) ? (lo4 >> 4) : (lo4 & 15);
        const int qv = (low | (((qh[l] >> (2 * grp)) & 3) << 4)) - 32;
        const float d = __fmul_rn(half_bits_to_float(ld_u16(blk + 208)), scale);
        return __fmul_rn(__fmul_rn(d, static_cast<float>(sc[l / 16 + 2 * grp])), static_cast<float>(qv));
    }
    // BF16
    return __fmul_rn(__uint_as_float(ld_u16(row + static_cast<size_t>(e) * 2) << 16), scale);
}

__global__ void dequant_kernel(int32_t type, const uint8_t* __restrict w, size_t rb, int32_t k, int32_t n,
                               float* __restrict out) {
    const size_t total = static_cast<size_t>(k) * n;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int32_t r = static_cast<int32_t>(i / k), e = static_cast<int32_t>(i % k);
        out[i] = decode_elem(type, w + static_cast<size_t>(r) * rb, e, 1.0f);
    }
}

__global__ void fetch_embedding_kernel(int32_t type, const uint8_t* __restrict row, int32_t dim, float scale,
                                       float* __restrict out) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < dim; e += gridDim.x * blockDim.x)
        out[e] = decode_elem(type, row, e, scale);
}

// The row of a token read from device memory (a decode loop that feeds its
// own argmax back without a host round trip).  Rows of tokens outside
// [0, vocab) are not read: the output is left as it is.
__global__ void fetch_embedding_dev_kernel(int32_t type, const uint8_t* __restrict table, const int32_t* token,
                                           int32_t vocab, size_t rbytes, int32_t dim, float scale,
                                           float* __restrict out) {
    const int32_t t = *token;
    if (t < 0 || t >= vocab) return;
    const uint8_t* row = table + static_cast<size_t>(t) * rbytes;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < dim; e += gridDim.x * blockDim.x)
        out[e] = decode_elem(type, row, e, scale);
}

// Rows of `count` tokens (ids already checked against the table's rows), one
// y-block of the grid per token.
__global__ void fetch_embedding_rows_kernel(int32_t type, const uint8_t* __restrict table, const int32_t* tokens,
                                            size_t rbytes, int32_t dim, float scale, float* __restrict out) {
    const uint8_t* row = table + static_cast<size_t>(tokens[blockIdx.y]) * rbytes;
    float* o = out + static_cast<size_t>(blockIdx.y) * dim;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < dim; e += gridDim.x * blockDim.x)
        o[e] = decode_elem(type, row, e, scale);
}

// Index of the largest value (the first one among equal maxima; NaN never
// wins), as torch.argmax and the greedy pick of the streamer's sampler take
// it.  Two launches: argmax_part_kernel reduces contiguous chunks of
// kArgmaxChunk values (coalesced float4 loads, several in flight per thread)
// to (value, index) pairs, argmax_final_kernel reduces the pairs.
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxChunk = 4096;
constexpr int kArgmaxMaxParts = 1024;

struct ArgBest {
    float v;
    int32_t i;  // INT32_MAX: no candidate
};
__device__ __forceinline__ ArgBest arg_better(ArgBest a, ArgBest b) {
    // b replaces a when it is larger, or equal with a smaller index; NaN never wins
    const bool take = b.i != INT32_MAX && (a.i == INT32_MAX || b.v > a.v || (b.v == a.v && b.i < a.i));
    return take ? b : a;
}
__device__ ArgBest block_argmax(ArgBest b) {
    __shared__ float sv[kArgmaxThreads];
    __shared__ int32_t si[kArgmaxThreads];
    sv[threadIdx.x] = b.v;
    si[threadIdx.x] = b.i;
    __syncthreads();
    for (int h = kArgmaxThreads / 2; h > 0; h >>= 1) {
        if (static_cast<int>(threadIdx.x) < h) {
            const ArgBest r = arg_better({sv[threadIdx.x], si[threadIdx.x]}, {sv[threadIdx.x + h], si[threadIdx.x + h]});
            sv[threadIdx.x] = r.v;
            si[threadIdx.x] = r.i;
        }
        __syncthreads();
    }
    return {sv[0], si[0]};
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_part_kernel(const float* __restrict x, int32_t n,
                                                                     float* __restrict pv, int32_t* __restrict pi) {
    const int32_t base = blockIdx.x * kArgmaxChunk;
    const int32_t end = min(n, base + kArgmaxChunk);
    ArgBest b{-INFINITY, INT32_MAX};
    // 4 values per thread per step, 4 steps: the whole chunk in flight at once
    float vals[kArgmaxChunk / kArgmaxThreads];
#pragma unroll
    for (int s = 0; s < kArgmaxChunk / (4 * kArgmaxThreads); ++s) {
        const int32_t i = base + 4 * (s * kArgmaxThreads + static_cast<int32_t>(threadIdx.x));
        if (i + 3 < end && (n & 3) == 0) {
            const float4 v = *reinterpret_cast<const float4*>(x + i);
            vals[4 * s] = v.x;
            vals[4 * s + 1] = v.y;
            vals[4 * s + 2] = v.z;
            vals[4 * s + 3] = v.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) vals[4 * s + c] = i + c < end ? x[i + c] : NAN;
        }
    }
#pragma unroll
    for (int s = 0; s < kArgmaxChunk / (4 * kArgmaxThreads); ++s)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int32_t i = base + 4 * (s * kArgmaxThreads + static_cast<int32_t>(threadIdx.x)) + c;
            const float v = vals[4 * s + c];
            if (v == v) b = arg_better(b, {v, i});
        }
    b = block_argmax(b);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = b.v;
        pi[blockIdx.x] = b.i;
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(const float* __restrict pv,
                                                                      const int32_t* __restrict pi, int32_t parts,
                                                                      int32_t* __restrict out, int32_t* __restrict log) {
    ArgBest b{-INFINITY, INT32_MAX};
    for (int32_t p = threadIdx.x; p < parts; p += kArgmaxThreads) b = arg_better(b, {pv[p], pi[p]});
    b = block_argmax(b);
    if (threadIdx.x == 0) {
        const int32_t r = b.i == INT32_MAX ? 0 : b.i;
        *out = r;
        if (log) *log = r;
    }
}

int grid_for(size_t n, int threads) {
    size_t g = (n + threads - 1) / threads;
    if (g > 4096) g = 4096;
    return g < 1 ? 1 : static_cast<int>(g);
}

}  // namespace

hipError_t launch_rmsnorm_heads(float* v, const float* gamma, int32_t n_heads, int32_t head_dim, float eps,
                                hipStream_t stream) {
    if (n_heads <= 0 || head_dim <= 0) return hipSuccess;
    if (head_dim <= kHeadsMaxHd)
        hipLaunchKernelGGL(rmsnorm_heads_kernel, dim3((n_heads + 3) / 4), dim3(256), 0, stream, v, gamma, n_heads,
                           head_dim, eps);
    else
        hipLaunchKernelGGL(rmsnorm_heads_long_kernel, dim3((n_heads + 3) / 4), dim3(256), 0, stream, v, gamma,
                           n_heads, head_dim, eps);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* gamma, int32_t rows, int32_t dim, float eps, float* out,
                          hipStream_t stream) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma) |
                         reinterpret_cast<uintptr_t>(out);
    const int32_t vec4 = (dim % 4 == 0 && (al & 15u) == 0) ? 1 : 0;
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(kNormThreads), 0, stream, x, gamma, dim, eps, out,
                       vec4, nullptr, nullptr);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm_rows(float* h, const float* r, const float* gamma, int32_t rows, int32_t dim, float eps,
                                   float* out, hipStream_t stream) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    const uintptr_t al = reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(r) |
                         reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(out);
    const int32_t vec4 = (dim % 4 == 0 && (al & 15u) == 0) ? 1 : 0;
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(kNormThreads), 0, stream, h, gamma, dim, eps, out, vec4,
                       r, h);
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(float* h, const float* r, const float* gamma, int32_t dim, float eps, float* out,
                              hipStream_t stream) {
    if (dim <= 0) return hipSuccess;
    const uintptr_t al = reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(r) |
                         reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(out);
    const int32_t vec4 = (dim % 4 == 0 && (al & 15u) == 0) ? 1 : 0;
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(1), dim3(kNormThreads), 0, stream, h, gamma, dim, eps, out, vec4, r,
                       h);
    return hipGetLastError();
}

hipError_t launch_rope(float* q, float* k, const RopeTable& table, int32_t n_heads, int32_t n_kv_heads,
                       int32_t head_dim, hipStream_t stream) {
    if (head_dim / 2 > kMaxRopeHalf || table.half * 2 != head_dim) return hipErrorInvalidValue;
    const size_t work = static_cast<size_t>(n_heads + n_kv_heads) * (head_dim / 2);
    if (work == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(work, 256)), dim3(256), 0, stream, q, k, table, n_heads,
                       n_kv_heads, head_dim);
    return hipGetLastError();
}

hipError_t launch_vec_add(float* y, const float* x, int32_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(vec_add_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, y, x, n);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* gate, const float* up, int32_t n, float* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, gate, up, n, out);
    return hipGetLastError();
}

hipError_t launch_geglu(const float* gate, const float* up, int32_t n, float* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(geglu_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, gate, up, n, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_encode(const float* x, const float* gamma, int32_t dim, float eps, float* out,
                                 int32_t layer_k, uint32_t* tokens, float* qscale, hipStream_t stream) {
    if (dim <= 0) return hipSuccess;
    const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma) |
                         reinterpret_cast<uintptr_t>(out);
    const int32_t vec4 = (dim % 4 == 0 && (al & 15u) == 0) ? 1 : 0;
    const int32_t k = layer_k < 0 ? 0 : (layer_k > 17 ? 17 : layer_k);
    hipLaunchKernelGGL((rmsnorm_kernel<false, true>), dim3(1), dim3(kNormThreads), 0, stream, x, gamma, dim, eps, out,
                       vec4, nullptr, nullptr, k, tokens, qscale);
    return hipGetLastError();
}

hipError_t launch_softcap(float* y, int32_t n, float softcap, hipStream_t stream) {
    if (n <= 0 || !(softcap > 0.0f)) return hipSuccess;
    hipLaunchKernelGGL(softcap_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, y, n, softcap);
    return hipGetLastError();
}

hipError_t launch_dequant(int32_t type, const uint8_t* w, int32_t k, int32_t n, float* out, hipStream_t stream) {
    if (!type_supported(type)) return hipErrorInvalidValue;
    if (k <= 0 || n <= 0) return hipSuccess;
    if (k % block_elems(type) != 0 || (reinterpret_cast<uintptr_t>(w) & 1u)) return hipErrorInvalidValue;
    const size_t total = static_cast<size_t>(k) * n;
    hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream, type, w,
                       row_bytes(type, k), k, n, out);
    return hipGetLastError();
}

hipError_t launch_fetch_embedding(int32_t type, const uint8_t* table, int32_t token, int32_t dim, float scale,
                                  float* out, hipStream_t stream) {
    if (type != kQ8_0 && type != kQ6_K && type != kBF16) return hipErrorInvalidValue;
    if (dim <= 0) return hipSuccess;
    const uint8_t* row = table + static_cast<size_t>(token) * row_bytes(type, dim);
    hipLaunchKernelGGL(fetch_embedding_kernel, dim3(grid_for(dim, 256)), dim3(256), 0, stream, type, row, dim,
                       scale, out);
    return hipGetLastError();
}

hipError_t launch_fetch_embedding_rows(int32_t type, const uint8_t* table, const int32_t* tokens, int32_t count,
                                       int32_t dim, float scale, float* out, hipStream_t stream) {
    if (type != kQ8_0 && type != kQ6_K && type != kBF16) return hipErrorInvalidValue;
    if (dim <= 0 || count <= 0) return hipSuccess;
    if (count > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fetch_embedding_rows_kernel, dim3(grid_for(dim, 256), count), dim3(256), 0, stream, type,
                       table, tokens, row_bytes(type, dim), dim, scale, out);
    return hipGetLastError();
}

hipError_t launch_fetch_embedding_dev(int32_t type, const uint8_t* table, const int32_t* token, int32_t vocab,
                                      int32_t dim, float scale, float* out, hipStream_t stream) {
    if (dim <= 0 || vocab <= 0) return hipSuccess;
    hipLaunchKernelGGL(fetch_embedding_dev_kernel, dim3(grid_for(dim, 256)), dim3(256), 0, stream, type, table, token,
                       vocab, row_bytes(type, dim), dim, scale, out);
    return hipGetLastError();
}

size_t argmax_workspace_bytes(int32_t n) {
    const size_t parts = n > 0 ? (static_cast<size_t>(n) + kArgmaxChunk - 1) / kArgmaxChunk : 0;
    return parts * (sizeof(float) + sizeof(int32_t));
}

hipError_t launch_argmax(const float* x, int32_t n, int32_t* out, int32_t* log, void* workspace, size_t ws_bytes,
                         hipStream_t stream) {
    if (n <= 0 || (reinterpret_cast<uintptr_t>(x) & 15u) != 0) return hipErrorInvalidValue;
    const int32_t parts = (n + kArgmaxChunk - 1) / kArgmaxChunk;
    if (parts > kArgmaxMaxParts || ws_bytes < argmax_workspace_bytes(n)) return hipErrorInvalidValue;
    float* pv = static_cast<float*>(workspace);
    int32_t* pi = reinterpret_cast<int32_t*>(pv + parts);
    hipLaunchKernelGGL(argmax_part_kernel, dim3(parts), dim3(kArgmaxThreads), 0, stream, x, n, pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, stream, pv, pi, parts, out, log);
    return hipGetLastError();
}

}  // namespace gncx
