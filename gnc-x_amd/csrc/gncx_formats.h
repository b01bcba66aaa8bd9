// gncx_formats.h -- GGUF block geometry shared by the host shim and the HIP
// kernels.  The byte layouts are the ones the reference declares packed in
// csrc/gncx_llm_kernels.cpp:266-297 (they are the ggml on-disk formats, so
// they must match byte for byte):
//
//   Q4_0  18 B / 32 w   {fp16 d; u8 qs[16]}            w = d*(nibble-8)
//   Q8_0  34 B / 32 w   {fp16 d; i8 qs[32]}            w = d*q
//   Q4_K 144 B / 256 w  {fp16 d, dmin; u8 sc[12]; u8 qs[128]}
//   Q6_K 210 B / 256 w  {u8 ql[128]; u8 qh[64]; i8 sc[16]; fp16 d}
//   BF16   2 B / 1 w
#pragma once
#include <cstddef>
#include <cstdint>

namespace gncx {

enum GgmlType : int32_t { kQ4_0 = 2, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kBF16 = 30 };

constexpr int32_t block_elems(int32_t t) {
    return (t == kQ4_K || t == kQ6_K) ? 256 : (t == kBF16 ? 1 : 32);
}
constexpr int32_t block_bytes(int32_t t) {
    return t == kQ4_0 ? 18 : t == kQ8_0 ? 34 : t == kQ4_K ? 144 : t == kQ6_K ? 210 : t == kBF16 ? 2 : 0;
}
constexpr bool type_supported(int32_t t) {
    return t == kQ4_0 || t == kQ8_0 || t == kQ4_K || t == kQ6_K || t == kBF16;
}
// Bytes of one row of k weights (k is truncated to whole blocks, as the
// reference does with in_dim / 32 and in_dim / 256).
constexpr size_t row_bytes(int32_t t, int32_t k) {
    return static_cast<size_t>(k / block_elems(t)) * static_cast<size_t>(block_bytes(t));
}

// Quantised activations kept in device memory: int8 values in element order
// and one 16-byte record per 32-block {d, sum of q[0:16], sum of q[16:32],
// sum of q[0:32]} (the fields of the reference's BlockActQ8, cpp:299-306).
struct ActMeta {
    float d;
    int32_t sum_lo16;
    int32_t sum_hi16;
    int32_t sum;
};
static_assert(sizeof(ActMeta) == 16, "ActMeta is one 16-byte record");

}  // namespace gncx
