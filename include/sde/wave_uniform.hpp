// Wave-uniform values for buffer resource descriptors and device-function
// arguments (gfx950).
//
// A raw buffer access takes its resource descriptor in scalar registers.
// When the compiler cannot prove the base pointer or the range uniform --
// a device function compiled on its own receives its arguments in vector
// registers, and values carried around a persistent kernel's loops can lose
// their uniformity -- it wraps every access in a loop over the distinct
// descriptors of the wave, and keeps every value derived from the arguments
// in vector registers.  The device functions here take arguments and build
// descriptors that are the same in every lane of a wave, so lane 0's copy,
// read into a scalar register, is the value itself (a no-op where the value
// already sits in a scalar register).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sde {

template <class T>
__device__ __forceinline__ T* wave_uniform(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint32_t wave_uniform(uint32_t x) {
  return __builtin_amdgcn_readfirstlane(x);
}

__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ size_t wave_uniform(size_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (size_t)(((uint64_t)hi << 32) | lo);
}

}  // namespace sde
