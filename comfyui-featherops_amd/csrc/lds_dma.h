// gfx950 global -> LDS copy helpers (LDS DMA) shared by the GEMM kernels.
#pragma once

#include "feather_common.h"

namespace feather {

// s_waitcnt with only vmcnt limited (expcnt / lgkmcnt left at their maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// vmcnt(N) and lgkmcnt(0) in one s_waitcnt.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// Workgroup barrier that neither waits for outstanding LDS-DMA copies (the
// caller waits for exactly the ones it needs) nor lets the compiler move
// memory accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Orders a wave's LDS writes before its own later LDS reads of them (by any
// lane of the same wave): the writes are waited for (lgkmcnt(0)) and the
// compiler may not move LDS accesses across. Enough when each wave stages
// through its own LDS region; no workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef __attribute__((address_space(3))) void lds_void;

// A rows are 128 bytes (8 chunks of 16 B); chunk c of row r sits at c ^ swz(r).
// An A-operand ds_read_b128 has lanes 0-15 on 16 consecutive rows (one
// logical chunk) and lanes 16-31 / 32-47 / 48-63 on the same rows at other
// chunks. Measured on gfx950 with SQ_LDS_BANK_CONFLICT: r & 7 and
// (r >> 1) & 7 both take 8 LDS cycles per instruction (2-way conflicts), while
// (r & 7) ^ ((r >> 3) & 1) takes the conflict-free 4.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// 16 bytes per lane from sbase + voff into LDS at lds_addr + 16 * lane
// (sbase and lds_addr wave-uniform; lds_addr a byte address in LDS, e.g. a
// __shared__ array's address plus a constant). Inline asm so that the
// compiler's wait-count tracking does not treat the copy as an LDS write that
// every later ds_read might alias (it would put a vmcnt(0) in front of the
// current stage's reads, draining the copies of the next stages); the
// kernels wait with explicit vmcnt counts instead. M0 is an operand of the
// asm, so the compiler sets it (often to an immediate) and keeps no copy of
// it, and no generic-to-LDS pointer conversion (with its null check) is needed.
__device__ __forceinline__ void dma16_lds(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile(
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(sbase), "{m0}"(lds_addr)
        : "memory");
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

}  // namespace feather
