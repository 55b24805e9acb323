// Shared device helpers for the gfx950 kernels: element types, 16-byte vector
// access, wavefront reductions and the thread-local error slot of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pk {

// Element-type codes of the C ABI (include/popcorn_amd.h: PK_F32/PK_BF16/PK_F16).
enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

typedef __bf16 bf16;
typedef _Float16 f16;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }

// Round-to-nearest-even narrowing, the rounding torch applies on every cast.
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }

// Value as it reads back after a round trip through T: models one torch op
// whose result tensor has dtype T.
template <typename T> __device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }

// Sixteen bytes of T: the unit of every coalesced load and store here.
template <typename T> struct alignas(16) Vec {
  static constexpr int N = 16 / sizeof(T);
  T v[N];
};

template <typename T> __device__ __forceinline__ Vec<T> ld16(const T* p) {
  Vec<T> r;
  *reinterpret_cast<uint4*>(&r) = *reinterpret_cast<const uint4*>(p);
  return r;
}

template <typename T> __device__ __forceinline__ void st16(T* p, const Vec<T>& r) {
  *reinterpret_cast<uint4*>(p) = *reinterpret_cast<const uint4*>(&r);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming variants: data touched exactly once is marked non-temporal so it
// does not evict reusable lines from L2 / MALL.
template <typename T> __device__ __forceinline__ Vec<T> ld16_stream(const T* p) {
  Vec<T> r;
  *reinterpret_cast<u32x4*>(&r) = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return r;
}

template <typename T> __device__ __forceinline__ void st16_stream(T* p, const Vec<T>& r) {
  __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&r), reinterpret_cast<u32x4*>(p));
}

// N elements of E whose bytes are a whole number of 16-byte vectors: the pack
// of a wider type that lines up with one Vec of a narrower one (8 fp32 beside
// 8 bf16 values, say), moved as one or more 16-byte accesses.
template <typename E, int N> struct alignas(16) Lane {
  static_assert(N * sizeof(E) % 16 == 0, "a lane pack is whole 16-byte vectors");
  static constexpr int kVectors = N * (int)sizeof(E) / 16;
  E v[N];
};

template <typename E, int N> __device__ __forceinline__ Lane<E, N> ld_lane(const E* p) {
  Lane<E, N> r;
#pragma unroll
  for (int i = 0; i < Lane<E, N>::kVectors; ++i)
    reinterpret_cast<uint4*>(r.v)[i] = reinterpret_cast<const uint4*>(p)[i];
  return r;
}

template <typename E, int N> __device__ __forceinline__ Lane<E, N> ld_lane_stream(const E* p) {
  Lane<E, N> r;
#pragma unroll
  for (int i = 0; i < Lane<E, N>::kVectors; ++i)
    reinterpret_cast<u32x4*>(r.v)[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
  return r;
}

template <typename E, int N> __device__ __forceinline__ void st_lane_stream(E* p, const Lane<E, N>& r) {
#pragma unroll
  for (int i = 0; i < Lane<E, N>::kVectors; ++i)
    __builtin_nontemporal_store(reinterpret_cast<const u32x4*>(r.v)[i], reinterpret_cast<u32x4*>(p) + i);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace pk
