// gncx_device.h -- device helpers shared by the HIP kernels (gfx950).
//
// Loads: GGUF blocks other than Q4_K are only 2-byte aligned (18, 34 and 210
// byte blocks).  A 16-byte field at a 2-aligned address is read as one
// dword-aligned dwordx4 plus one extra 16-bit load, and realigned with
// v_alignbyte_b32; no load ever reaches outside the block it belongs to.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gncx_formats.h"

namespace gncx {
namespace dev {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

__device__ __forceinline__ uint4 ld16_aligned(const uint8_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// 16 bytes at a 2-aligned address p.  Reads [p - sh, p - sh + 16) and
// [p + 14, p + 16) with sh = p mod 4 in {0, 2}: nothing past the field, and
// the 2 bytes before p only when p is not 4-aligned (then p - 2 is still
// inside a tensor whose base is 4-aligned).
__device__ __forceinline__ uint4 ld16_a2(const uint8_t* p) {
    const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint8_t* a = p - sh;
    const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(a);
    const uint32_t tail = ld_u16(p + 14);  // == a[16], a[17] when sh == 2
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    r.w = __builtin_amdgcn_alignbyte(tail, v.w, sh);
    return r;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    // v_cvt_f32_f16: exact IEEE conversion (subnormal halves are normal floats)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// v + (v of another lane) through DPP; lanes the masks leave out add 0
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_ZERO = false>
__device__ __forceinline__ float dpp_add(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO);
    return v + __builtin_bit_cast(float, o);
}

// Sum over the 64 lanes of a wave, left in lane 63 (and every lane of the
// last 16-lane row).  Row butterflies (xor 1, xor 2, half-mirror, mirror),
// then row_bcast:15 / row_bcast:31 carry the row totals up: six DPP adds, no
// LDS traffic.
__device__ __forceinline__ float wave_sum_lane63(float v) {
    v = dpp_add<0xb1>(v);          // quad_perm [1,0,3,2]
    v = dpp_add<0x4e>(v);          // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);         // row_half_mirror
    v = dpp_add<0x140>(v);         // row_mirror: every lane holds its row's sum
    v = dpp_add<0x142, 0xa>(v);    // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);    // row_bcast:31 into rows 2 and 3
    return v;
}

// Sum over the wave, returned in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v = wave_sum_lane63(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over aligned groups of N = 4, 8 or 16 lanes (the first N / 4 + 1 steps
// of wave_sum_lane63); every lane of a group ends with the same sum.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 4 || N == 8 || N == 16, "groups of 4, 8 or 16 lanes");
    v = dpp_add<0xb1>(v);
    v = dpp_add<0x4e>(v);
    if constexpr (N >= 8) v = dpp_add<0x141>(v);
    if constexpr (N >= 16) v = dpp_add<0x140>(v);
    return v;
}

// max(v, v of another lane) through DPP; lanes the masks leave out keep v
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_max(float v) {
    const int o = __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -__builtin_inff()), __builtin_bit_cast(int, v),
                                              CTRL, ROW_MASK, BANK_MASK, false);
    return fmaxf(v, __builtin_bit_cast(float, o));
}

// Max over the wave, returned in every lane: the steps of wave_sum_lane63
// with max for add (no LDS round trips, unlike a shuffle butterfly).
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max<0xb1>(v);
    v = dpp_max<0x4e>(v);
    v = dpp_max<0x141>(v);
    v = dpp_max<0x140>(v);
    v = dpp_max<0x142, 0xa>(v);
    v = dpp_max<0x143, 0xc>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Q4_K 6-bit (scale, min) of sub-block j (reference cpp:1112-1120) from the
// three little-endian dwords of the 12 scale bytes.
__device__ __forceinline__ void k4_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             int& sc, int& mn) {
    const int jj = j & 3;
    const uint32_t a = byte_of(s0, jj), b = byte_of(s1, jj), c = byte_of(s2, jj);
    // both forms computed and selected: j varies across lanes, a branch would diverge
    const uint32_t sc_lo = a & 63u, mn_lo = b & 63u;
    const uint32_t sc_hi = (c & 15u) | ((a >> 6) << 4), mn_hi = (c >> 4) | ((b >> 6) << 4);
    sc = static_cast<int>(j < 4 ? sc_lo : sc_hi);
    mn = static_cast<int>(j < 4 ? mn_lo : mn_hi);
}

// 1/rms of one head of hd values, formed as the reference does
// (cpp:905-926): four fp32 lane sums over i mod 4 for the multiple-of-4
// prefix, the lanes added in double, a double tail, then
// 1 / sqrtf((float)(sum/hd) + eps).  No contraction; IEEE division and
// sqrtf (correctly rounded here, unlike the 1-ulp __fsqrt_rn).
// Called by a whole wave; every lane returns the same value.
__device__ __forceinline__ float head_inv_rms(const float* v, int hd, float eps, int lane) {
#pragma clang fp contract(off)
    const int full = hd & ~3;
    float part = 0.0f;
    if (lane < 4) {
        // 32 loads in flight ahead of the ordered adds (the order is the sum's):
        // a 128-wide head waits for LDS once
        int i = lane;
        for (; i + 124 < full; i += 128) {
            float a[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) a[u] = v[i + 4 * u];
#pragma unroll
            for (int u = 0; u < 32; ++u) part += a[u] * a[u];
        }
        for (; i + 28 < full; i += 32) {
            float a[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) a[u] = v[i + 4 * u];
#pragma unroll
            for (int u = 0; u < 8; ++u) part += a[u] * a[u];
        }
        for (; i < full; i += 4) part += v[i] * v[i];
    }
    auto lane_val = [](float v, int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    };
    const float p0 = lane_val(part, 0), p1 = lane_val(part, 1);
    const float p2 = lane_val(part, 2), p3 = lane_val(part, 3);
    double s = static_cast<double>(p0) + static_cast<double>(p1) + static_cast<double>(p2) + static_cast<double>(p3);
    for (int i = full; i < hd; ++i) s += static_cast<double>(v[i]) * static_cast<double>(v[i]);
    const float mean = static_cast<float>(s / static_cast<double>(hd));
    return 1.0f / sqrtf(mean + eps);
}

// max / sum over aligned groups of 8 lanes with DPP (no LDS traffic):
// half-mirror (lane i <-> 7-i), then quad xor 2, then quad xor 1; every lane
// of the group ends with the group's result.
__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false)));
    return v;
}
// sum over aligned groups of 4 lanes (quad xor 2, xor 1)
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false);
    v += __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false);
    return v;
}

// Per-32 Q8 quantisation of x[k] (reference cpp:955-995), done by the whole
// work-group: 8 lanes per 32-block, 4 values per lane, up to four tasks per
// thread with their loads issued together.  Writes int8 values to q[k] and
// one ActMeta per block.  blockDim.x must be a multiple of 64.  Bit-exact with
// the reference: IEEE 127/amax and amax/127, one rounding for x*inv,
// round-half-even.
// The four int8 values and the block scale of one task (8 lanes per block).
__device__ __forceinline__ void quantize_values(const float4 v, int& q0, int& q1, int& q2, int& q3, float& d) {
    const float a = group8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    q0 = q1 = q2 = q3 = 0;
    d = 0.0f;
    if (a != 0.0f) {
        const float inv = 127.0f / a;
        d = a / 127.0f;
        q0 = static_cast<int>(rintf(v.x * inv));
        q1 = static_cast<int>(rintf(v.y * inv));
        q2 = static_cast<int>(rintf(v.z * inv));
        q3 = static_cast<int>(rintf(v.w * inv));
    }
}

__device__ __forceinline__ void quantize_task(const float4 v, int32_t b, int j, int8_t* __restrict q,
                                              ActMeta* __restrict meta) {
    int q0, q1, q2, q3;
    float d;
    quantize_values(v, q0, q1, q2, q3, d);
    const uint32_t packed = (static_cast<uint32_t>(q0) & 0xffu) | ((static_cast<uint32_t>(q1) & 0xffu) << 8) |
                            ((static_cast<uint32_t>(q2) & 0xffu) << 16) | (static_cast<uint32_t>(q3) << 24);
    *reinterpret_cast<uint32_t*>(q + static_cast<size_t>(b) * 32 + j * 4) = packed;
    // lanes 0-3 of the group: sum of q[0:16]; lanes 4-7: q[16:32]
    const int s = quad_sum(q0 + q1 + q2 + q3);
    const int other = __builtin_amdgcn_mov_dpp(s, 0x141, 0xf, 0xf, false);  // lane i <- lane 7-i
    if (j == 0) {
        ActMeta m;
        m.d = d;
        m.sum_lo16 = s;
        m.sum_hi16 = other;
        m.sum = s + other;
        meta[b] = m;
    }
}

// Split form for kernels that must order their loads: quant_load issues the
// first U tasks' x loads (call it before issuing other global loads, since
// vmcnt retires loads in order), quant_finish quantises them and any tasks
// beyond U * nthr.
// Loads are unconditional (tasks past the end re-read the last one), so the
// number of loads in flight is static and the waitcnt for x does not wait for
// the weight loads issued after it.
template <int U>
__device__ __forceinline__ void quant_load(float4 (&v)[U], const float* __restrict x, int32_t nb, int tid,
                                           int nthr) {
    const int32_t ntask = nb * 8;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int32_t t = min(tid + u * nthr, ntask - 1);
        v[u] = *reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * 4);
    }
}

template <int U>
__device__ __forceinline__ void quant_finish(const float4 (&v)[U], const float* __restrict x, int32_t nb, int tid,
                                             int nthr, int8_t* __restrict q, ActMeta* __restrict meta) {
    const int32_t ntask = nb * 8;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int32_t t = tid + u * nthr;
        if (t < ntask) quantize_task(v[u], t >> 3, t & 7, q, meta);
    }
    for (int32_t t = tid + U * nthr; t < ntask; t += nthr) {
        const float4 w = *reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * 4);
        quantize_task(w, t >> 3, t & 7, q, meta);
    }
}

__device__ __forceinline__ void quantize_block8(const float* __restrict x, int32_t nb, int tid, int nthr,
                                                int8_t* __restrict q, ActMeta* __restrict meta) {
    constexpr int U = 4;
    const int32_t ntask = nb * 8;
    for (int32_t base = tid; base < ntask; base += U * nthr) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int32_t t = base + u * nthr;
            if (t < ntask) v[u] = *reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * 4);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int32_t t = base + u * nthr;
            if (t < ntask) quantize_task(v[u], t >> 3, t & 7, q, meta);
        }
    }
}

}  // namespace dev
}  // namespace gncx
