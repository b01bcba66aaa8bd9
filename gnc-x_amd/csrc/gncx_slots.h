// gncx_slots.h -- per-lane block dots shared by the GEMV and the small-batch
// matbatch kernels.  A "slot" maps one lane to a fixed byte range of one
// block of a weight row; each function returns that slot's fp32 share of the
// row sum, using Q8 activations (int8 values q + ActMeta per 32-block):
//   Q4_K  4 slots per 144 B super-block (16 B header + 32 B of nibbles each),
//         reference dot cpp:1127-1205
//   Q6_K  4 slots per 210 B super-block, (128-half, 16-group) each,
//         reference dot cpp:1211-1321
//   Q4_0  1 slot per 18 B block (cpp:1362-1382), Q8_0 1 per 34 B block
//         (cpp:1413-1431), BF16 16 bytes of weights with fp32 x (cpp:1432-1461)
#pragma once
#include <hip/hip_runtime.h>

#include "gncx_device.h"

namespace gncx {
namespace dev {

__device__ __forceinline__ float slot_q4_k(const uint8_t* __restrict row, int s,
                                           const int8_t* __restrict q, const ActMeta* __restrict meta) {
    const int sb = s >> 2, c = s & 3;
    const uint8_t* blk = row + static_cast<size_t>(sb) * 144;
    const uint4 hdr = ld16_aligned(blk);
    const uint4 w0 = ld16_aligned(blk + 16 + 32 * c);
    const uint4 w1 = ld16_aligned(blk + 32 + 32 * c);
    const int ab = sb * 8 + 2 * c;
    const uint4* xq = reinterpret_cast<const uint4*>(q + static_cast<size_t>(ab) * 32);
    const uint4 xl0 = xq[0], xl1 = xq[1], xh0 = xq[2], xh1 = xq[3];
    const ActMeta ml = meta[ab], mh = meta[ab + 1];
    const uint32_t M = 0x0f0f0f0fu;
    int dl = 0, dh = 0;
    dl = sdot4(w0.x & M, xl0.x, dl); dh = sdot4((w0.x >> 4) & M, xh0.x, dh);
    dl = sdot4(w0.y & M, xl0.y, dl); dh = sdot4((w0.y >> 4) & M, xh0.y, dh);
    dl = sdot4(w0.z & M, xl0.z, dl); dh = sdot4((w0.z >> 4) & M, xh0.z, dh);
    dl = sdot4(w0.w & M, xl0.w, dl); dh = sdot4((w0.w >> 4) & M, xh0.w, dh);
    dl = sdot4(w1.x & M, xl1.x, dl); dh = sdot4((w1.x >> 4) & M, xh1.x, dh);
    dl = sdot4(w1.y & M, xl1.y, dl); dh = sdot4((w1.y >> 4) & M, xh1.y, dh);
    dl = sdot4(w1.z & M, xl1.z, dl); dh = sdot4((w1.z >> 4) & M, xh1.z, dh);
    dl = sdot4(w1.w & M, xl1.w, dl); dh = sdot4((w1.w >> 4) & M, xh1.w, dh);
    int s1, m1, s2, m2;
    k4_scale_min(2 * c, hdr.y, hdr.z, hdr.w, s1, m1);
    k4_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, s2, m2);
    const float d = half_bits_to_float(hdr.x & 0xffffu);
    const float dmin = half_bits_to_float(hdr.x >> 16);
    const float d1 = d * static_cast<float>(s1), dm1 = dmin * static_cast<float>(m1);
    const float d2 = d * static_cast<float>(s2), dm2 = dmin * static_cast<float>(m2);
    return ml.d * (d1 * static_cast<float>(dl) - dm1 * static_cast<float>(ml.sum)) +
           mh.d * (d2 * static_cast<float>(dh) - dm2 * static_cast<float>(mh.sum));
}

__device__ __forceinline__ float slot_q6_k(const uint8_t* __restrict row, int s,
                                           const int8_t* __restrict q, const ActMeta* __restrict meta) {
    const int sb = s >> 2, n = (s >> 1) & 1, g = s & 1;
    const uint8_t* blk = row + static_cast<size_t>(sb) * 210;
    const uint4 pa = ld16_a2(blk + 64 * n + 16 * g);
    const uint4 pb = ld16_a2(blk + 64 * n + 32 + 16 * g);
    const uint4 ph = ld16_a2(blk + 128 + 32 * n + 16 * g);
    // scales sc[8n .. 8n+7] (2-aligned 8 bytes)
    const uint8_t* ps = blk + 192 + 8 * n;
    const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ps) & 3u);
    const u32x2a4 sv = *reinterpret_cast<const u32x2a4*>(ps - sh);
    const uint32_t st = ld_u16(ps + 6);
    const uint32_t sc_lo = __builtin_amdgcn_alignbyte(sv.y, sv.x, sh);  // sc[8n+0..3]
    const uint32_t sc_hi = __builtin_amdgcn_alignbyte(st, sv.y, sh);    // sc[8n+4..7]
    const float d = half_bits_to_float(ld_u16(blk + 208));

    const int ab = sb * 8 + 4 * n;
    const uint32_t M4 = 0x0f0f0f0fu, M2 = 0x03030303u;
    const uint32_t wa[4] = {pa.x, pa.y, pa.z, pa.w};
    const uint32_t wb[4] = {pb.x, pb.y, pb.z, pb.w};
    const uint32_t wh[4] = {ph.x, ph.y, ph.z, ph.w};
    int dot[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 xv = *reinterpret_cast<const uint4*>(q + static_cast<size_t>(ab + k) * 32 + 16 * g);
        const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t v;
            if (k == 0) v = (wa[i] & M4) | ((wh[i] & M2) << 4);
            else if (k == 1) v = (wb[i] & M4) | (((wh[i] >> 2) & M2) << 4);
            else if (k == 2) v = ((wa[i] >> 4) & M4) | (((wh[i] >> 4) & M2) << 4);
            else v = ((wb[i] >> 4) & M4) | (((wh[i] >> 6) & M2) << 4);
            dot[k] = sdot4(v, xs[i], dot[k]);
        }
    }
    float p = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const ActMeta m = meta[ab + k];
        const int sidx = g + 2 * k;  // 0..7 within sc[8n..8n+7]
        const uint32_t word = sidx < 4 ? sc_lo : sc_hi;
        const int scv = static_cast<int>(static_cast<int8_t>(byte_of(word, sidx & 3)));
        const int ssum = g == 0 ? m.sum_lo16 : m.sum_hi16;
        p += static_cast<float>(dot[k] - 32 * ssum) * (m.d * static_cast<float>(scv));
    }
    return d * p;
}

__device__ __forceinline__ float slot_q4_0(const uint8_t* __restrict row, int b,
                                           const int8_t* __restrict q, const ActMeta* __restrict meta) {
    const ActMeta m = meta[b];
    const uint8_t* blk = row + static_cast<size_t>(b) * 18;
    const float wd = half_bits_to_float(ld_u16(blk));
    const uint4 qs = ld16_a2(blk + 2);
    const uint4* xq = reinterpret_cast<const uint4*>(q + static_cast<size_t>(b) * 32);
    const uint4 xl = xq[0], xh = xq[1];
    const uint32_t M = 0x0f0f0f0fu;
    int dot = 0;
    dot = sdot4(qs.x & M, xl.x, dot); dot = sdot4((qs.x >> 4) & M, xh.x, dot);
    dot = sdot4(qs.y & M, xl.y, dot); dot = sdot4((qs.y >> 4) & M, xh.y, dot);
    dot = sdot4(qs.z & M, xl.z, dot); dot = sdot4((qs.z >> 4) & M, xh.z, dot);
    dot = sdot4(qs.w & M, xl.w, dot); dot = sdot4((qs.w >> 4) & M, xh.w, dot);
    const int folded = dot - 8 * m.sum;
    // cpp:1371: blocks with a zero activation scale are skipped
    return m.d != 0.0f ? static_cast<float>(folded) * (wd * m.d) : 0.0f;
}

__device__ __forceinline__ float slot_q8_0(const uint8_t* __restrict row, int b,
                                           const int8_t* __restrict q, const ActMeta* __restrict meta) {
    const ActMeta m = meta[b];
    const uint8_t* blk = row + static_cast<size_t>(b) * 34;
    const float wd = half_bits_to_float(ld_u16(blk));
    const uint4 w0 = ld16_a2(blk + 2);
    const uint4 w1 = ld16_a2(blk + 18);
    const uint4* xq = reinterpret_cast<const uint4*>(q + static_cast<size_t>(b) * 32);
    const uint4 x0 = xq[0], x1 = xq[1];
    int dot = 0;
    dot = sdot4(w0.x, x0.x, dot); dot = sdot4(w0.y, x0.y, dot);
    dot = sdot4(w0.z, x0.z, dot); dot = sdot4(w0.w, x0.w, dot);
    dot = sdot4(w1.x, x1.x, dot); dot = sdot4(w1.y, x1.y, dot);
    dot = sdot4(w1.z, x1.z, dot); dot = sdot4(w1.w, x1.w, dot);
    return static_cast<float>(dot) * (wd * m.d);
}

__device__ __forceinline__ float bf16_bits(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float slot_bf16(const uint8_t* __restrict row, int s, int32_t k,
                                           const float* __restrict x) {
    const int32_t e0 = s * 8;
    float acc = 0.0f;
    if (e0 + 8 <= k) {
        const uint4 w = ld16_aligned(row + static_cast<size_t>(e0) * 2);
        const float4 xa = *reinterpret_cast<const float4*>(x + e0);
        const float4 xb = *reinterpret_cast<const float4*>(x + e0 + 4);
        acc = bf16_bits(w.x & 0xffffu) * xa.x + bf16_bits(w.x >> 16) * xa.y +
              bf16_bits(w.y & 0xffffu) * xa.z + bf16_bits(w.y >> 16) * xa.w +
              bf16_bits(w.z & 0xffffu) * xb.x + bf16_bits(w.z >> 16) * xb.y +
              bf16_bits(w.w & 0xffffu) * xb.z + bf16_bits(w.w >> 16) * xb.w;
    } else {
        for (int32_t e = e0; e < k; ++e) acc += bf16_bits(ld_u16(row + static_cast<size_t>(e) * 2)) * x[e];
    }
    return acc;
}

}  // namespace dev
}  // namespace gncx
