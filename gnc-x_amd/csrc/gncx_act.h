// gncx_act.h -- activation functions shared by the kernels that apply them,
// so every path computes the same bits.
#pragma once

#include <hip/hip_runtime.h>

namespace gncx {
namespace dev {

// SwiGLU of one gate / up pair: (g / (1 + e^-g)) u with each operation
// rounded on its own (no contraction), as the reference's loop
// (cpp:2038-2052) computes it.
__device__ __forceinline__ float swiglu_value(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

}  // namespace dev
}  // namespace gncx
