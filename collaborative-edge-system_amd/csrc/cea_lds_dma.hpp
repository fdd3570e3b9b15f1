// Buffer loads straight into LDS, explicit memory waits and a fence-free barrier, shared by
// the matrix-core attention kernels.
#pragma once

#include "cea_common.hpp"

namespace cea {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int kRsrcFlags = 0x00020000;  // raw buffer resource word 3 (gfx9 family)

// Raw buffer resource: base, stride 0, num_records = bytes (reads at or past it return 0).
// base and bytes must be wave-uniform; they are moved to scalar registers here.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int32_t)((uint32_t)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int32_t)bytes);
  r[3] = kRsrcFlags;
  return r;
}

// LDS byte address of a wave-uniform pointer, in an SGPR (M0 takes scalar operands only)
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_ptr)p);
}

// Buffer loads straight into LDS (M0 = LDS base, lane l writes base + l*size).  Issued as
// inline assembly: the kernels wait for them explicitly with vmcnt, and the compiler, which
// cannot tell which LDS bytes they write, would otherwise drain every load in flight before
// each LDS read.  A load the compiler does not see can only make its own waits stricter.
__device__ __forceinline__ void buffer_load_lds16(i32x4 rs, const char* lds_base, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(lds_addr(lds_base)), "v"(voffset), "s"(rs) : "memory", "m0");
}
// Streaming variant (non-temporal): for data read once, such as a KV cache during decoding.
__device__ __forceinline__ void buffer_load_lds16_nt(i32x4 rs, const char* lds_base, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               ::"s"(lds_addr(lds_base)), "v"(voffset), "s"(rs) : "memory", "m0");
}
// 4 bytes per lane (exact per-dword range check)
__device__ __forceinline__ void buffer_load_lds4(i32x4 rs, const char* lds_base, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               ::"s"(lds_addr(lds_base)), "v"(voffset), "s"(rs) : "memory", "m0");
}

// The same loads with the LDS destination given as an LDS byte address (wave-uniform).
__device__ __forceinline__ void buffer_load_lds16_m0(i32x4 rs, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(rs) : "memory", "m0");
}
__device__ __forceinline__ void buffer_load_lds4_m0(i32x4 rs, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(rs) : "memory", "m0");
}

// 16-byte load with a wave-uniform byte offset (soffset) added to the per-lane offset.
__device__ __forceinline__ void buffer_load_lds16_m0_so(i32x4 rs, uint32_t lds, uint32_t voffset,
                                                        uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(rs),
                 "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
}

// Waits until at most N of this wave's vector-memory loads are outstanding.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until this wave's LDS reads have returned their data.
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier that keeps the compiler from moving memory operations across it without
// forcing outstanding buffer loads to complete (the kernels wait for them explicitly).
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

}  // namespace cea
