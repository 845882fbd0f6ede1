// Global → LDS transfers without VGPR staging (buffer_load … lds), shared by
// the ring GEMM (gemm_ring.hip) and the fused feed-forward kernel (mlp.hip).
#pragma once

#include "fh_common.h"

namespace fh_dma {

// Buffer resource for raw loads and stores of `bytes` bytes at p: offsets
// at or beyond `bytes` read as zero and are not written.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from rs + voff + soff into LDS at lds_addr + lane·16
// (buffer_load_dwordx4 … lds).  Callers order these against their LDS reads
// themselves (s_waitcnt vmcnt + barrier); the compiler counts them in vmcnt.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(uintptr_t)lds_addr, 16,
                                             voff, soff, 0, 0);
}

}  // namespace fh_dma
