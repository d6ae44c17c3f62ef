// mfma.h -- fp32 matrix-core helpers for gfx950 (CDNA4).
//
// All tiles in this library are built from v_mfma_f32_32x32x2f32: one wave
// (64 lanes) multiplies a 32x2 A slice by a 2x32 B slice into a 32x32 fp32
// accumulator held as 16 floats per lane.  Operand and result placement
// (checked on the device with an in-bounds probe):
//   A[m][k]  : lane l supplies m = l % 32, k = l / 32
//   B[k][n]  : lane l supplies n = l % 32, k = l / 32
//   C[m][n]  : lane l, register i holds n = l % 32,
//              m = acc_row(i, l / 32) = 8*(i/4) + 4*(l/32) + i%4
// Because the contraction index k only has to agree between A and B, every
// kernel is free to map (k-step, lane half) to any element of the contracted
// dimension; the kernels use that freedom to make each lane read contiguous
// memory (128-bit LDS reads).  Because C's row index m lives in (register,
// lane half) exactly like a contraction index, an accumulator can be fed
// back as the A or B operand of a product that contracts over m with no data
// movement: register i is the operand of k-step i.
#pragma once

#include <hip/hip_runtime.h>

namespace ember {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma_32x32x2(float a, float b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row of the 32x32 accumulator that register i of lane half h holds.
__device__ __forceinline__ constexpr int acc_row(int i, int h)
{
    return ((i >> 2) << 3) + (h << 2) + (i & 3);
}

__device__ __forceinline__ f32x16 zero16()
{
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.0f;
    return z;
}

// Loads DB consecutive floats (DB in {1, 2, 4}) as one LDS/global vector.
template <int DB>
struct VecN;
template <>
struct VecN<1> {
    typedef float T;
};
template <>
struct VecN<2> {
    typedef f32x2 T;
};
template <>
struct VecN<4> {
    typedef f32x4 T;
};

template <int DB>
__device__ __forceinline__ float vget(const typename VecN<DB>::T &v, int j)
{
    if constexpr (DB == 1)
        return v;
    else
        return v[j];
}

}  // namespace ember
