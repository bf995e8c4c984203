// Device helpers shared by the persistent attention kernels (attn_pp.hip,
// attn_wide.hip): buffer descriptors, direct global -> LDS loads, LDS access
// at integer addresses and the LDS-only barrier.
#pragma once

#include "attn_kernels.hpp"

namespace inl {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

#define PP_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pp_rsrc(const void* base, uint32_t bytes) {
  // word3 0x00020000: raw (untyped) 32-bit data, the gfx9 buffer format.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The same buffer descriptor as four SGPR words, for inline asm.
__device__ __forceinline__ i32x4 pp_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// Direct global -> LDS load of 16 bytes per lane: lane l's bytes land at LDS
// address lds + 16 * l; the global address is the descriptor base + voff
// (bytes past the descriptor's range read as zero). Issued from inline asm so
// that the compiler does not treat every later LDS read as a possible alias
// of the load and wait for all loads in flight; the kernel waits for these
// loads itself (vmcnt) before their data is used.
__device__ __forceinline__ void dma_b128(i32x4 rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}

// LDS access at an integer byte address: with a per-lane base register and a
// compile-time offset the offset lands in the instruction's offset field.
template <typename T>
__device__ __forceinline__ T lds_load(uint32_t a) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>((size_t)a);
}
template <typename T>
__device__ __forceinline__ void lds_store(uint32_t a, const T& v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>((size_t)a) = v;
}

// Hides a value's provenance from the optimizer, so that base + constant is
// not reassociated into constant + base (which would cost an add per use).
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(size_t)PP_LDS_PTR(p));
}

// Workgroup barrier that orders LDS only. __syncthreads() would also wait
// for every outstanding global -> LDS load (vmcnt(0)), which the pipeline
// keeps in flight across barriers on purpose.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace

}  // namespace inl
