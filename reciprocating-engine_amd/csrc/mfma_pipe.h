// mfma_pipe.h - pieces shared by the LDS-staged MFMA GEMM kernels
// (gemm_fp8.hip, gemm_tiles.hip): the LDS row swizzle, explicit vmcnt waits,
// global -> LDS copies, a barrier without the vmcnt(0) of __syncthreads and an
// MFMA / LDS-read / copy interleave for the scheduler.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace reng {
namespace pipe {

constexpr int XCDS = 8;    // MI355X: 8 XCDs, workgroups dispatched round-robin over them

// The scale an unscaled operand reads, so that epilogues load a scale through
// (pointer, stride) without branching on the scale form.
static __device__ const float one_f32 = 1.0f;

// Slot permutation of an LDS row of CH 16-byte chunks: chunk c of tile row r
// sits in slot c ^ swz(r). A fragment read takes 32 consecutive rows at one
// chunk; with these permutations any 8 consecutive rows use 8 distinct slots
// modulo 128 bytes and any 16 use 16 distinct slots modulo 256 bytes, so the
// ds_read_b128 phases are free of bank conflicts for 32 or 64 four-byte banks.
// swz depends on the low five bits of r only: the reader knows its row as
// (32-row tile base) + lane % 32.
template <int CH>
__device__ __forceinline__ uint32_t swz(uint32_t r) {
    if constexpr (CH == 4) return ((r >> 1) ^ (r >> 3)) & 3;
    else return (r ^ ((r >> 3) & 3)) & 7;
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 0xf) | (7 << 4) | (0xf << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0): the wave's LDS reads (and scalar loads) are done.
__device__ __forceinline__ void wait_lgkm0() {
    asm volatile("" ::: "memory");   // LDS accesses before the wait stay before it
    __builtin_amdgcn_s_waitcnt(0xf | (7 << 4) | (0 << 8) | (3 << 14));
    asm volatile("" ::: "memory");
}

// One global_load_lds_dwordx4: 16 bytes per lane from
// g into LDS at l + 16 * lane (l is wave-uniform). A __device__ function
// rather than code in the kernel's lambdas, whose host-side instantiation
// cannot form the LDS address-space cast.
__device__ __forceinline__ void copy16_to_lds(const uint8_t *g, uint8_t *l) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 16, 0, 0);
}

// A workgroup barrier that orders LDS traffic for the compiler (the memory
// clobbers) without the vmcnt(0) that __syncthreads' fence would add.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Scheduling pattern for one region of the stage: NM MFMAs, with NDS LDS
// reads and NVM vector-memory instructions spread evenly between them, so the
// MFMA pipe keeps receiving work while the wave issues its copies and
// fragment reads (a wave issues in order, one wave per SIMD).
template <int NM, int NDS, int NVM, int I = 0>
__device__ __forceinline__ void interleave() {
    if constexpr (I < NM) {
        constexpr int ds = (NDS * (I + 1)) / NM - (NDS * I) / NM;
        constexpr int vm = (NVM * (I + 1)) / NM - (NVM * I) / NM;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        if constexpr (ds > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds, 0);   // DS read
        if constexpr (vm > 0) __builtin_amdgcn_sched_group_barrier(0x060, vm, 0);   // VMEM
        interleave<NM, NDS, NVM, I + 1>();
    }
}

}  // namespace pipe
}  // namespace reng
