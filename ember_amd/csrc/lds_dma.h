// lds_dma.h -- buffer-descriptor memory helpers on gfx950 (not part of the
// public ABI): direct HBM -> LDS copies, wait counts, and bounds-checked
// stores.
#pragma once

#include <hip/hip_runtime.h>

namespace ember {

// 16 bytes per lane from global memory straight into LDS, bypassing
// registers: lane l's data lands at lds + 16*l bytes
// (global_load_lds_dwordx4; `lds` must be wave-uniform).  Completion is
// tracked by the wave's vmcnt like any vector-memory load.
__device__ __forceinline__ void dma16(const float *src, float *lds)
{
    typedef __attribute__((address_space(1))) void gvoid;
    typedef __attribute__((address_space(3))) void lvoid;
    __builtin_amdgcn_global_load_lds((gvoid *)src, (lvoid *)lds, 16, 0, 0);
}

// The same copy in buffer form (buffer_load_dwordx4 ... lds): the base
// address lives in a scalar buffer descriptor and each lane supplies a
// 32-bit byte offset, so a copy needs one offset register and no per-lane
// 64-bit address arithmetic.  The descriptor's range is the full 4 GiB
// (no clamping); its format word is the raw-buffer setting for gfx9 parts.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_rsrc(const float *base)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, -1, 0x00020000);
}

__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, unsigned byte_off, float *lds)
{
    typedef __attribute__((address_space(3))) void lvoid;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lvoid *)lds, 16, byte_off, 0, 0, 0);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// and lgkmcnt left at their maxima): at most N of this wave's vector-memory
// operations, including LDS-bound copies, are still in flight.
template <int N>
__device__ __forceinline__ void wait_vmem_n()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void wait_vmem()
{
    wait_vmem_n<0>();
}

// s_waitcnt lgkmcnt(0): this wave's LDS reads (and scalar loads) are done.
__device__ __forceinline__ void wait_lds()
{
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// Bounds-checked stores through a buffer descriptor (raw buffer_store): the
// hardware drops a store whose byte offset (plus its size) passes the
// descriptor's range.  A lane that must not store passes kStoreNone as its
// offset, so a masked store needs no branch and every wave issues the same
// stores on every path.  That matters in the persistent kernels, which load
// the next head's rows, then store this head's results, then wait for the
// rows: with the stores under per-row branches the compiler's wait count
// there can only be vmcnt(0), which waits for the stores as well; with one
// path it is vmcnt(number of stores).  Ranges stay below kStoreNone: the
// kernels that use these stores cover at most 64 rows of a head, so a range
// is at most 4 * (63 * (2^24 - 1) + 128) bytes (row strides are below 2^24
// floats, checked on the host), 4227858692 < 0xFFFFFF00.
constexpr unsigned kStoreNone = 0xFFFFFF00u;

// A descriptor over `bytes` bytes from `base` (bytes <= kStoreNone).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t store_rsrc(float *base, unsigned bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void store1_bounded(__amdgpu_buffer_rsrc_t rsrc, unsigned byte_off, float v)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), rsrc, byte_off, 0, 0);
}

}  // namespace ember
