// gncx_slots.h -- per-lane block dots shared by the GEMV and the small-batch
// matbatch kernels.  A "slot" maps one lane to a fixed byte range of one
// block of a weight row.  Each format has
//   Frag                 the raw weight registers one slot needs from HBM,
//   load(f, row, s)      issues those loads from a row source (PtrRow or
//                        BufRow below),
//   Act                  the Q8 activation registers the slot multiplies,
//   load_act(a, s, ...)  reads them (LDS q + ActMeta, or fp32 x for BF16),
//   dot(f, a, s)         the slot's fp32 share of the row sum (no contraction, so
//                        every inlined copy rounds alike and a row's result does
//                        not depend on which loop of a kernel computed it),
// so kernels can put several slots' weight loads in flight before touching
// any, and keep a slot's activations in registers across rows.
//   Q4_K  4 slots per 144 B super-block: 16 B header + 32 B of nibbles each
//         (reference dot cpp:1127-1205)
//   Q6_K  4 slots per 210 B super-block, one (128-half, 16-group) each
//         (reference dot cpp:1211-1321)
//   Q4_0  1 slot per 18 B block (cpp:1362-1382)
//   Q8_0  1 slot per 34 B block (cpp:1413-1431)
//   BF16  8 weights (16 B) per slot, fp32 x (cpp:1432-1461)
#pragma once
#include <hip/hip_runtime.h>

#include "gncx_device.h"

namespace gncx {
namespace dev {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2a2 __attribute__((ext_vector_type(2), aligned(2)));

// Row sources: a slot reads its fields by byte offset within one weight row.
//   PtrRow  global loads from a row pointer (plain loads: non-temporal ones
//           measured up to 2.3x slower on these 2-aligned, partly overlapping
//           fields and fetched 1.5x the bytes),
//   BufRow  buffer loads through a resource whose base (4-aligned, delta
//           bytes before the row) sits in scalar registers; an offset at or
//           past num_records reads 0 and makes no memory request, so a
//           resource with num_records 0 is a free dummy row.
// Offsets are signed: a realigned field read starts up to 2 bytes before the
// field (o - sh), which is before the row itself for a row that starts 2 bytes
// past a 4-byte boundary (still inside the tensor, whose base is 4-aligned).
// Offsets passed to ld16 are 16-aligned from a 16-aligned row; ld16a4 and
// ld8a4 take 4-aligned addresses (sh() gives a field's address mod 4); ld16u
// and ld8u take any 2-aligned address (one dwordx4 / dwordx2 at that byte
// address: the memory model runs in unaligned-access mode).
struct PtrRow {
    const uint8_t* p;
    __device__ __forceinline__ u32x4 ld16(int32_t o) const { return *reinterpret_cast<const u32x4*>(p + o); }
    __device__ __forceinline__ u32x4a4 ld16a4(int32_t o) const {
        return *reinterpret_cast<const u32x4a4*>(p + o);
    }
    __device__ __forceinline__ u32x2a4 ld8a4(int32_t o) const {
        return *reinterpret_cast<const u32x2a4*>(p + o);
    }
    __device__ __forceinline__ uint32_t ldu16(int32_t o) const {
        return *reinterpret_cast<const uint16_t*>(p + o);
    }
    __device__ __forceinline__ u32x4 ld16u(int32_t o) const { return *reinterpret_cast<const u32x4a2*>(p + o); }
    __device__ __forceinline__ u32x2 ld8u(int32_t o) const { return *reinterpret_cast<const u32x2a2*>(p + o); }
    __device__ __forceinline__ uint32_t sh(int32_t o) const {
        return static_cast<uint32_t>((reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(o)) & 3u);
    }
};

struct BufRow {
    __amdgpu_buffer_rsrc_t r;
    uint32_t delta;
    // rows start 2-aligned; the resource starts at the 4-aligned address at
    // or before the row and covers exactly the row (0 bytes when !valid)
    __device__ __forceinline__ BufRow(const uint8_t* row, uint32_t bytes, bool valid) {
        const uint32_t dl = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(row) & 3u);
        r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(row - dl), static_cast<short>(0),
                                              valid ? static_cast<int>(bytes + dl) : 0, 0x00020000);
        delta = dl;
    }
    __device__ __forceinline__ u32x4 ld16(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int32_t>(delta) + o, 0, 0);
    }
    __device__ __forceinline__ u32x4a4 ld16a4(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int32_t>(delta) + o, 0, 0);
    }
    __device__ __forceinline__ u32x2a4 ld8a4(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int32_t>(delta) + o, 0, 0);
    }
    __device__ __forceinline__ uint32_t ldu16(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int32_t>(delta) + o, 0, 0);
    }
    __device__ __forceinline__ u32x4 ld16u(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int32_t>(delta) + o, 0, 0);
    }
    __device__ __forceinline__ u32x2 ld8u(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int32_t>(delta) + o, 0, 0);
    }
    __device__ __forceinline__ uint32_t sh(int32_t o) const { return (delta + static_cast<uint32_t>(o)) & 3u; }
};

// Rows of a tile read through one wave-uniform resource over the tile's rows
// (4-aligned base); each lane adds the byte offset of its own row.  A lane
// with no row uses an offset past the resource and reads zeros.
struct TileRow {
    __amdgpu_buffer_rsrc_t r;
    int32_t base;
    __device__ __forceinline__ u32x4 ld16(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b128(r, base + o, 0, 0);
    }
    __device__ __forceinline__ u32x4a4 ld16a4(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b128(r, base + o, 0, 0);
    }
    __device__ __forceinline__ u32x2a4 ld8a4(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b64(r, base + o, 0, 0);
    }
    __device__ __forceinline__ uint32_t ldu16(int32_t o) const {
        return __builtin_amdgcn_raw_buffer_load_b16(r, base + o, 0, 0);
    }
    __device__ __forceinline__ u32x4 ld16u(int32_t o) const { return __builtin_amdgcn_raw_buffer_load_b128(r, base + o, 0, 0); }
    __device__ __forceinline__ u32x2 ld8u(int32_t o) const { return __builtin_amdgcn_raw_buffer_load_b64(r, base + o, 0, 0); }
    __device__ __forceinline__ uint32_t sh(int32_t o) const { return static_cast<uint32_t>(base + o) & 3u; }
};

// raw 16-byte field at a 2-aligned row offset o: the dword-aligned dwordx4 at
// o - sh and the 2 bytes at o + 14 (see ld16_a2); sh = field address mod 4 is
// kept by the caller (all fields of one block share it) and the field is
// realigned only when used
struct Raw16 {
    u32x4a4 v;
    uint32_t tail;
};

template <class Row>
__device__ __forceinline__ void raw16_load(Raw16& r, const Row& row, uint32_t o, uint32_t sh) {
    r.v = row.ld16a4(static_cast<int32_t>(o) - static_cast<int32_t>(sh));
    r.tail = row.ldu16(static_cast<int32_t>(o) + 14);
}

__device__ __forceinline__ uint4 raw16_get(const Raw16& r, uint32_t sh) {
    uint4 o;
    o.x = __builtin_amdgcn_alignbyte(r.v.y, r.v.x, sh);
    o.y = __builtin_amdgcn_alignbyte(r.v.z, r.v.y, sh);
    o.z = __builtin_amdgcn_alignbyte(r.v.w, r.v.z, sh);
    o.w = __builtin_amdgcn_alignbyte(r.tail, r.v.w, sh);
    return o;
}

__device__ __forceinline__ uint4 lds16(const int8_t* p) { return *reinterpret_cast<const uint4*>(p); }

template <int TYPE>
struct Slot;

// ---------------------------------------------------------------- Q4_K
template <>
struct Slot<kQ4_K> {
    struct Frag {
        u32x4 hdr, w0, w1;
    };
    struct Act {
        uint4 xl0, xl1, xh0, xh1;  // q of sub-blocks 2c (low nibbles) and 2c+1 (high)
        float dl, dh;              // their block scales
        float bl, bh;              // block scale x sum of q
        uint32_t sel;              // byte selector of sub-blocks 2c, 2c+1
    };
    static constexpr int32_t slots(int32_t k) { return (k / 256) * 4; }
    template <class Row>
    __device__ static __forceinline__ void load(Frag& f, const Row& row, int s) {
        const uint32_t sb = static_cast<uint32_t>(s) >> 2, c = static_cast<uint32_t>(s) & 3u;
        const uint32_t blk = sb * 144u;
        f.hdr = row.ld16(blk);
        f.w0 = row.ld16(blk + 16u + 32u * c);
        f.w1 = row.ld16(blk + 32u + 32u * c);
    }
    __device__ static __forceinline__ void load_act(Act& a, int s, const int8_t* __restrict q,
                                                    const ActMeta* __restrict meta) {
#pragma clang fp contract(off)
        const int c = s & 3;
        const int ab = (s >> 2) * 8 + 2 * c;
        const int8_t* xq = q + static_cast<size_t>(ab) * 32;
        a.xl0 = lds16(xq);
        a.xl1 = lds16(xq + 16);
        a.xh0 = lds16(xq + 32);
        a.xh1 = lds16(xq + 48);
        const ActMeta ml = meta[ab], mh = meta[ab + 1];
        a.dl = ml.d;
        a.dh = mh.d;
        a.bl = ml.d * static_cast<float>(ml.sum);
        a.bh = mh.d * static_cast<float>(mh.sum);
        a.sel = 0x0c0c0000u | static_cast<uint32_t>(2 * c) | (static_cast<uint32_t>(2 * c + 1) << 8);
    }
    __device__ static __forceinline__ float dot(const Frag& f, const Act& a, int) {
#pragma clang fp contract(off)
        const uint32_t M = 0x0f0f0f0fu;
        int dl = 0, dh = 0;
        dl = sdot4(f.w0.x & M, a.xl0.x, dl); dh = sdot4((f.w0.x >> 4) & M, a.xh0.x, dh);
        dl = sdot4(f.w0.y & M, a.xl0.y, dl); dh = sdot4((f.w0.y >> 4) & M, a.xh0.y, dh);
        dl = sdot4(f.w0.z & M, a.xl0.z, dl); dh = sdot4((f.w0.z >> 4) & M, a.xh0.z, dh);
        dl = sdot4(f.w0.w & M, a.xl0.w, dl); dh = sdot4((f.w0.w >> 4) & M, a.xh0.w, dh);
        dl = sdot4(f.w1.x & M, a.xl1.x, dl); dh = sdot4((f.w1.x >> 4) & M, a.xh1.x, dh);
        dl = sdot4(f.w1.y & M, a.xl1.y, dl); dh = sdot4((f.w1.y >> 4) & M, a.xh1.y, dh);
        dl = sdot4(f.w1.z & M, a.xl1.z, dl); dh = sdot4((f.w1.z >> 4) & M, a.xh1.z, dh);
        dl = sdot4(f.w1.w & M, a.xl1.w, dl); dh = sdot4((f.w1.w >> 4) & M, a.xh1.w, dh);
        // The eight 6-bit scales and mins of the super-block (get_scale_min_k4,
        // cpp:1112-1120), one per byte with sub-block j in byte j of {lo, hi}
        // -- sub-blocks 0-3 take the low 6 bits of bytes 0-3 / 4-7, sub-blocks
        // 4-7 a nibble of bytes 8-11 plus the top 2 bits of bytes 0-3 / 4-7 --
        // then the two of this slot picked by one byte permute.  The slot's
        // share is regrouped from the reference's per-block
        //   dx_j (d sc_j isum_j - dmin m_j sum_j)
        // as d (sc_1 dx_1 isum_1 + sc_2 dx_2 isum_2) - dmin (m_1 b_1 + m_2 b_2)
        // with b_j = dx_j sum_j formed once per launch: every term stays exact
        // up to its fp32 roundings, and the VALU work per row drops by a quarter.
        const uint32_t y = f.hdr.y, z = f.hdr.z, w = f.hdr.w;
        const uint32_t sc_lo = y & 0x3f3f3f3fu, mn_lo = z & 0x3f3f3f3fu;
        const uint32_t sc_hi = (w & M) | ((y >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((w >> 4) & M) | ((z >> 2) & 0x30303030u);
        const uint32_t sc = __builtin_amdgcn_perm(sc_hi, sc_lo, a.sel);
        const uint32_t mn = __builtin_amdgcn_perm(mn_hi, mn_lo, a.sel);
        const float d = half_bits_to_float(f.hdr.x & 0xffffu);
        const float dmin = half_bits_to_float(f.hdr.x >> 16);
        const float s1 = static_cast<float>(sc & 0xffu), s2 = static_cast<float>((sc >> 8) & 0xffu);
        const float m1 = static_cast<float>(mn & 0xffu), m2 = static_cast<float>((mn >> 8) & 0xffu);
        const float sum = __builtin_fmaf(s2 * a.dh, static_cast<float>(dh), (s1 * a.dl) * static_cast<float>(dl));
        const float mins = __builtin_fmaf(m2, a.bh, m1 * a.bl);
        return __builtin_fmaf(-dmin, mins, d * sum);
    }
};

// ---------------------------------------------------------------- Q6_K
template <>
struct Slot<kQ6_K> {
    // Fields of the 2-aligned 210-byte block are read where they lie with
    // unaligned loads: 5 loads per slot instead of 9 and no realignment
    // (Q6_K 14336 x 4096: 13.2 against 13.9 us).  Q4_0 and Q8_0 keep the
    // aligned form (Raw16), which measured faster for their 18 / 34-byte blocks.
    struct Frag {
        u32x4 pa, pb, ph;
        u32x2 sv;        // scales sc[8n..8n+7]
        uint32_t d;      // fp16 bits
    };
    struct Act {
        uint4 x[4];   // bytes [16g, 16g+16) of the four 32-blocks of this 128-half
        float d[4];
        int s[4];     // sum of those 16 q
    };
    static constexpr int32_t slots(int32_t k) { return (k / 256) * 4; }
    template <class Row>
    __device__ static __forceinline__ void load(Frag& f, const Row& row, int s) {
        const uint32_t sb = static_cast<uint32_t>(s) >> 2, n = (static_cast<uint32_t>(s) >> 1) & 1u,
                       g = static_cast<uint32_t>(s) & 1u;
        const int32_t blk = static_cast<int32_t>(sb * 210u);
        f.pa = row.ld16u(blk + static_cast<int32_t>(64u * n + 16u * g));
        f.pb = row.ld16u(blk + static_cast<int32_t>(64u * n + 32u + 16u * g));
        f.ph = row.ld16u(blk + static_cast<int32_t>(128u + 32u * n + 16u * g));
        f.sv = row.ld8u(blk + static_cast<int32_t>(192u + 8u * n));
        f.d = row.ldu16(blk + 208);
    }
    __device__ static __forceinline__ void load_act(Act& a, int s, const int8_t* __restrict q,
                                                    const ActMeta* __restrict meta) {
        const int sb = s >> 2, n = (s >> 1) & 1, g = s & 1;
        const int ab = sb * 8 + 4 * n;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a.x[k] = lds16(q + static_cast<size_t>(ab + k) * 32 + 16 * g);
            const ActMeta m = meta[ab + k];
            a.d[k] = m.d;
            a.s[k] = g == 0 ? m.sum_lo16 : m.sum_hi16;
        }
    }
    __device__ static __forceinline__ float dot(const Frag& f, const Act& a, int s) {
#pragma clang fp contract(off)
        const int g = s & 1;
        const uint32_t sc_lo = f.sv.x;  // sc[8n+0..3]
        const uint32_t sc_hi = f.sv.y;  // sc[8n+4..7]
        const uint32_t M4 = 0x0f0f0f0fu, M2 = 0x03030303u;
        const uint32_t wa[4] = {f.pa.x, f.pa.y, f.pa.z, f.pa.w};
        const uint32_t wb[4] = {f.pb.x, f.pb.y, f.pb.z, f.pb.w};
        const uint32_t wh[4] = {f.ph.x, f.ph.y, f.ph.z, f.ph.w};
        float p = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t xs[4] = {a.x[k].x, a.x[k].y, a.x[k].z, a.x[k].w};
            int dot = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t v;
                if (k == 0) v = (wa[i] & M4) | ((wh[i] & M2) << 4);
                else if (k == 1) v = (wb[i] & M4) | (((wh[i] >> 2) & M2) << 4);
                else if (k == 2) v = ((wa[i] >> 4) & M4) | (((wh[i] >> 4) & M2) << 4);
                else v = ((wb[i] >> 4) & M4) | (((wh[i] >> 6) & M2) << 4);
                dot = sdot4(v, xs[i], dot);
            }
            const int sidx = g + 2 * k;  // 0..7 within sc[8n..8n+7]
            const uint32_t word = sidx < 4 ? sc_lo : sc_hi;
            const int scv = static_cast<int>(static_cast<int8_t>(byte_of(word, sidx & 3)));
            p += static_cast<float>(dot - 32 * a.s[k]) * (a.d[k] * static_cast<float>(scv));
        }
        return half_bits_to_float(f.d) * p;
    }
};

// ---------------------------------------------------------------- Q4_0
template <>
struct Slot<kQ4_0> {
    struct Frag {
        uint32_t d, sh;
        Raw16 qs;
    };
    struct Act {
        uint4 xl, xh;
        float d;
        int sum;
    };
    static constexpr int32_t slots(int32_t k) { return k / 32; }
    template <class Row>
    __device__ static __forceinline__ void load(Frag& f, const Row& row, int b) {
        const uint32_t blk = static_cast<uint32_t>(b) * 18u;
        f.d = row.ldu16(blk);
        f.sh = row.sh(blk + 2u);
        raw16_load(f.qs, row, blk + 2u, f.sh);
    }
    __device__ static __forceinline__ void load_act(Act& a, int b, const int8_t* __restrict q,
                                                    const ActMeta* __restrict meta) {
        a.xl = lds16(q + static_cast<size_t>(b) * 32);
        a.xh = lds16(q + static_cast<size_t>(b) * 32 + 16);
        const ActMeta m = meta[b];
        a.d = m.d;
        a.sum = m.sum;
    }
    __device__ static __forceinline__ float dot(const Frag& f, const Act& a, int) {
#pragma clang fp contract(off)
        const uint4 qs = raw16_get(f.qs, f.sh);
        const uint32_t M = 0x0f0f0f0fu;
        int dot = 0;
        dot = sdot4(qs.x & M, a.xl.x, dot); dot = sdot4((qs.x >> 4) & M, a.xh.x, dot);
        dot = sdot4(qs.y & M, a.xl.y, dot); dot = sdot4((qs.y >> 4) & M, a.xh.y, dot);
        dot = sdot4(qs.z & M, a.xl.z, dot); dot = sdot4((qs.z >> 4) & M, a.xh.z, dot);
        dot = sdot4(qs.w & M, a.xl.w, dot); dot = sdot4((qs.w >> 4) & M, a.xh.w, dot);
        const int folded = dot - 8 * a.sum;
        // cpp:1371: blocks with a zero activation scale are skipped
        return a.d != 0.0f ? static_cast<float>(folded) * (half_bits_to_float(f.d) * a.d) : 0.0f;
    }
};

// ---------------------------------------------------------------- Q8_0
template <>
struct Slot<kQ8_0> {
    struct Frag {
        uint32_t d, sh;
        Raw16 lo, hi;
    };
    struct Act {
        uint4 x0, x1;
        float d;
    };
    static constexpr int32_t slots(int32_t k) { return k / 32; }
    template <class Row>
    __device__ static __forceinline__ void load(Frag& f, const Row& row, int b) {
        const uint32_t blk = static_cast<uint32_t>(b) * 34u;
        f.d = row.ldu16(blk);
        f.sh = row.sh(blk + 2u);
        raw16_load(f.lo, row, blk + 2u, f.sh);
        raw16_load(f.hi, row, blk + 18u, f.sh);
    }
    __device__ static __forceinline__ void load_act(Act& a, int b, const int8_t* __restrict q,
                                                    const ActMeta* __restrict meta) {
        a.x0 = lds16(q + static_cast<size_t>(b) * 32);
        a.x1 = lds16(q + static_cast<size_t>(b) * 32 + 16);
        a.d = meta[b].d;
    }
    __device__ static __forceinline__ float dot(const Frag& f, const Act& a, int) {
#pragma clang fp contract(off)
        const uint4 w0 = raw16_get(f.lo, f.sh), w1 = raw16_get(f.hi, f.sh);
        int dot = 0;
        dot = sdot4(w0.x, a.x0.x, dot); dot = sdot4(w0.y, a.x0.y, dot);
        dot = sdot4(w0.z, a.x0.z, dot); dot = sdot4(w0.w, a.x0.w, dot);
        dot = sdot4(w1.x, a.x1.x, dot); dot = sdot4(w1.y, a.x1.y, dot);
        dot = sdot4(w1.z, a.x1.z, dot); dot = sdot4(w1.w, a.x1.w, dot);
        return static_cast<float>(dot) * (half_bits_to_float(f.d) * a.d);
    }
};

// ---------------------------------------------------------------- BF16
__device__ __forceinline__ float bf16_bits(uint32_t b) { return __uint_as_float(b << 16); }

template <>
struct Slot<kBF16> {
    struct Frag {
        u32x4 w;
    };
    struct Act {
        float4 a, b;
    };
    static constexpr int32_t slots(int32_t k) { return k / 8; }  // launchers require k % 8 == 0
    template <class Row>
    __device__ static __forceinline__ void load(Frag& f, const Row& row, int s) {
        f.w = row.ld16(static_cast<uint32_t>(s) * 16u);
    }
    // BF16 multiplies the fp32 vector itself (global memory)
    __device__ static __forceinline__ void load_act_x(Act& a, int s, const float* __restrict x) {
        a.a = *reinterpret_cast<const float4*>(x + 8 * s);
        a.b = *reinterpret_cast<const float4*>(x + 8 * s + 4);
    }
    __device__ static __forceinline__ float dot(const Frag& f, const Act& x, int) {
#pragma clang fp contract(off)
        return bf16_bits(f.w.x & 0xffffu) * x.a.x + bf16_bits(f.w.x >> 16) * x.a.y +
               bf16_bits(f.w.y & 0xffffu) * x.a.z + bf16_bits(f.w.y >> 16) * x.a.w +
               bf16_bits(f.w.z & 0xffffu) * x.b.x + bf16_bits(f.w.z >> 16) * x.b.y +
               bf16_bits(f.w.w & 0xffffu) * x.b.z + bf16_bits(f.w.w >> 16) * x.b.w;
    }
};

// activations of slot s from the quantised vector (LDS or global) or, for
// BF16, from the fp32 vector
template <int TYPE>
__device__ __forceinline__ void slot_act(typename Slot<TYPE>::Act& a, int s, const int8_t* __restrict q,
                                         const ActMeta* __restrict meta, const float* __restrict x) {
    if constexpr (TYPE == kBF16) Slot<TYPE>::load_act_x(a, s, x);
    else Slot<TYPE>::load_act(a, s, q, meta);
}

}  // namespace dev
}  // namespace gncx
