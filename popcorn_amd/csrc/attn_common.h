// Pieces shared by the attention kernels: matrix-core fragment types, the
// 32x32x16 MFMA for each 16-bit element type, and 16-byte buffer loads.
#pragma once

#include "common.h"

namespace pk {
namespace attn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s4;

// D[32x32] += A[32x16] B[16x32]: lane l holds row l%32 of A (K elements
// 8*(l/32) .. +8) and column l%32 of B (the same K elements); the result
// lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + r%4 for r = 0..15.
template <typename T> struct Mma;
template <> struct Mma<bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma<f16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// 16 bytes at voffset + soffset of a buffer resource (zeros past its range)
__device__ __forceinline__ uint4 ld_buf(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes at voffset + soffset of a buffer resource written straight to LDS:
// lane i's bytes land at lds + 16 * i (lds must be the same for the whole
// wave); zeros past the resource's range. Completion is counted by vmcnt.
__device__ __forceinline__ void ld_buf_lds(__amdgpu_buffer_rsrc_t r, void* lds, int voffset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0, 0);
}

// 4 bytes per lane, as ld_buf_lds (lane i's word at lds + 4 * i).
__device__ __forceinline__ void ld_buf_lds4(__amdgpu_buffer_rsrc_t r, void* lds, int voffset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voffset, soffset, 0, 0);
}

// A buffer resource as its four words (base, 32-bit range, raw-buffer flags),
// made wave-uniform, for the inline-assembly loads below.
typedef unsigned rsrc_words __attribute__((ext_vector_type(4)));
__device__ __forceinline__ rsrc_words make_rsrc_words(const void* base, int nrec) {
  const uint64_t p = (uint64_t)base;
  rsrc_words r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)p);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32) & 0xffffu);
  r.z = __builtin_amdgcn_readfirstlane((uint32_t)nrec);
  r.w = 0x00020000u;
  return r;
}

// ld_buf_lds and ld_buf_lds4 as inline assembly (M0 = the wave's LDS base).
// The compiler does not see these LDS writes, so it waits for none of them
// before later LDS reads, which it must do for the builtin whenever it cannot
// tell the written buffer from the one read (one array indexed by stage). The
// caller waits (lds_loads_landed) before any barrier after which a wave may
// read what it wrote. It must also let the compiler finish its own vector
// loads before issuing these: its waits count loads by number, and loads it
// does not know of would make them wait for more than they mean to.
// (A generic pointer into LDS holds the LDS address in its low 32 bits.)
__device__ __forceinline__ uint32_t lds_base(const void* lds) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
}
__device__ __forceinline__ void ld_lds16_asm(rsrc_words r, const void* lds, int voffset, int soffset) {
  asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lds_base(lds)), "v"(voffset), "s"(r),
               "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory");
}
__device__ __forceinline__ void ld_lds4_asm(rsrc_words r, const void* lds, int voffset, int soffset) {
  asm volatile("buffer_load_dword %1, %2, %3 offen lds" ::"{m0}"(lds_base(lds)), "v"(voffset), "s"(r),
               "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory");
}

// Wait until this wave's LDS-bound buffer loads have landed.
__device__ __forceinline__ void lds_loads_landed() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N of this wave's vector memory loads are still in flight
// (they complete in issue order).
template <int N> __device__ __forceinline__ void loads_landed_but() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Four 16-bit values as two packed 32-bit words
template <typename T> __device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
  return make_uint2((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(a)) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(b)) << 16),
                    (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(c)) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(d)) << 16));
}

}  // namespace attn
}  // namespace pk
