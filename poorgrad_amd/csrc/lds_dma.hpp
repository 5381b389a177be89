// LDS-DMA primitives shared by the f32 and bf16 matrix-core products:
// global_load_lds_dwordx4 issued as inline assembly, the waits and barrier
// that order it, and the row swizzle of the k-contiguous slab layout.
//
// A wave-wide global_load_lds_dwordx4 writes 1 KB: each lane's 16 bytes land
// at LDS position 16 * lane from the wave's base address (held in M0), so an
// operand's LDS layout is chosen through which global address each lane
// loads. A k-contiguous slab keeps 16 rows of 64 bytes per KB (16 f32 k
// values, or 32 bf16 ones): the 16-byte quad q of local row r sits at
// position 4r + (q ^ dma_swizzle(r)), so the fragment reads of 16 rows by one
// lane group (the same quad of each row) fall on different banks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace topos_hip {
namespace lds_dma {

__device__ __forceinline__ int dma_swizzle(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

#define TOPOS_COMPILER_FENCE() __atomic_signal_fence(__ATOMIC_SEQ_CST)

// One wave-wide global_load_lds_dwordx4: each lane's 16 bytes at `src` land
// in LDS at `lds_byte` + 16 * lane (M0 holds the wave's LDS byte address).
// Issued as inline assembly: the compiler's wait insertion treats a DMA
// issued through the builtin as a pending LDS write that every later LDS
// read must wait for, which put a vmcnt(0) before each slab's fragment reads
// and so waited for the slab two ahead as well; the kernels order their DMA
// themselves (dma_wait, then a barrier). `src` needs 4-byte alignment.
__device__ __forceinline__ void dma_load16(const void *src, uint32_t lds_byte) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_byte)
               : "memory", "m0");
}

// The LDS byte address of an LDS location.
__device__ __forceinline__ uint32_t lds_byte_address(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

// Waits until at most N of this lane's vector-memory operations are
// outstanding and its LDS operations are done (s_waitcnt vmcnt(N)
// lgkmcnt(0); expcnt left at its maximum). Vector-memory operations complete
// in issue order for this count, so a wait for a later load (the compiler's
// own, before a register-staged slab's LDS store) also covers every earlier
// DMA.
template <int N>
__device__ __forceinline__ void dma_wait() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  TOPOS_COMPILER_FENCE();
  __builtin_amdgcn_s_waitcnt(0x070 | N);
  TOPOS_COMPILER_FENCE();
}

// A barrier without the workgroup fence of __syncthreads(), which would also
// wait for the DMA loads kept in flight across it.
__device__ __forceinline__ void dma_barrier() {
  TOPOS_COMPILER_FENCE();
  __builtin_amdgcn_s_barrier();
  TOPOS_COMPILER_FENCE();
}

}  // namespace lds_dma
}  // namespace topos_hip
