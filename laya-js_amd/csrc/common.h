// Shared device/host helpers for libhipbackend (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <atomic>
#include <string>

#include "../../include/laya_hip.h"

namespace hb {

// ------------------------------------------------------------------ errors

void set_error(const std::string& msg);
#define HB_CHECK_HIP(expr)                                                           \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess) {                                                          \
      throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(_e));   \
    }                                                                                \
  } while (0)
#define HB_REQUIRE(cond, msg)                                        \
  do {                                                               \
    if (!(cond)) throw std::runtime_error(std::string(msg));         \
  } while (0)
void check_launch(const char* what);

// Runs `set` (a kernel attribute setting, which applies to the current
// device) once per device: bit d of `done` records device d.  Concurrent
// first calls may both run `set`, which is idempotent.
template <class Set>
inline void once_per_device(std::atomic<uint64_t>& done, Set&& set) {
  int dev = 0;
  HB_CHECK_HIP(hipGetDevice(&dev));
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return;
  set();
  done.fetch_or(bit, std::memory_order_acq_rel);
}

struct Context;
hipStream_t stream_of(uintptr_t ctx);
int device_of(uintptr_t ctx);
int cu_count(uintptr_t ctx);
// finds the device address of hb_sdpa_noalloc's scratch on `device` (current)
void sdpa_scratch_init(int device);
// scratch memory from the context's stream-ordered pool (freed with pool_free)
void* pool_alloc(uintptr_t ctx, size_t bytes);
void pool_free(uintptr_t ctx, void* p);

// ------------------------------------------------------------------ dtypes

typedef _Float16 f16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short short8 __attribute__((ext_vector_type(8)));
typedef short short4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef unsigned int uint4v __attribute__((ext_vector_type(4)));
typedef unsigned int uint2v __attribute__((ext_vector_type(2)));

struct bf16s {  // bf16 storage: raw bits
  uint16_t bits;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  f16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  f16 h = (f16)x;  // v_cvt_f16_f32: round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Generic element load/store by runtime dtype code (HB_F32 ...).
__device__ __forceinline__ float load_f(const void* p, int64_t i, int dt) {
  switch (dt) {
    case HB_F32: return ((const float*)p)[i];
    case HB_F16: return f16_bits_to_f32(((const uint16_t*)p)[i]);
    case HB_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case HB_I32: return (float)((const int32_t*)p)[i];
    case HB_BOOL: return ((const uint8_t*)p)[i] ? 1.0f : 0.0f;
    case HB_U8: return (float)((const uint8_t*)p)[i];
    case HB_I8: return (float)((const int8_t*)p)[i];
    case HB_U16: return (float)((const uint16_t*)p)[i];
    case HB_I16: return (float)((const int16_t*)p)[i];
    case HB_U32: return (float)((const uint32_t*)p)[i];
    default: return 0.0f;
  }
}
__device__ __forceinline__ int32_t load_i(const void* p, int64_t i, int dt) {
  switch (dt) {
    case HB_I32: return ((const int32_t*)p)[i];
    case HB_BOOL: return ((const uint8_t*)p)[i] ? 1 : 0;
    case HB_U8: return ((const uint8_t*)p)[i];
    case HB_I8: return ((const int8_t*)p)[i];
    case HB_U16: return ((const uint16_t*)p)[i];
    case HB_I16: return ((const int16_t*)p)[i];
    case HB_U32: return (int32_t)((const uint32_t*)p)[i];
    default: return (int32_t)load_f(p, i, dt);
  }
}
__device__ __forceinline__ void store_f(void* p, int64_t i, int dt, float v) {
  switch (dt) {
    case HB_F32: ((float*)p)[i] = v; break;
    case HB_F16: ((uint16_t*)p)[i] = f32_to_f16_bits(v); break;
    case HB_BF16: ((uint16_t*)p)[i] = f32_to_bf16(v); break;
    case HB_I32: ((int32_t*)p)[i] = (int32_t)v; break;
    case HB_BOOL: ((uint8_t*)p)[i] = v != 0.0f ? 1 : 0; break;
    case HB_U8: ((uint8_t*)p)[i] = (uint8_t)(int32_t)v; break;
    case HB_I8: ((int8_t*)p)[i] = (int8_t)(int32_t)v; break;
    case HB_U16: ((uint16_t*)p)[i] = (uint16_t)(int32_t)v; break;
    case HB_I16: ((int16_t*)p)[i] = (int16_t)(int32_t)v; break;
    case HB_U32: ((uint32_t*)p)[i] = (uint32_t)(int64_t)v; break;
    default: break;
  }
}
__device__ __forceinline__ void store_i(void* p, int64_t i, int dt, int32_t v) {
  switch (dt) {
    case HB_I32: ((int32_t*)p)[i] = v; break;
    case HB_BOOL: ((uint8_t*)p)[i] = v != 0 ? 1 : 0; break;
    case HB_U8: ((uint8_t*)p)[i] = (uint8_t)v; break;
    case HB_I8: ((int8_t*)p)[i] = (int8_t)v; break;
    case HB_U16: ((uint16_t*)p)[i] = (uint16_t)v; break;
    case HB_I16: ((int16_t*)p)[i] = (int16_t)v; break;
    case HB_U32: ((uint32_t*)p)[i] = (uint32_t)v; break;
    default: store_f(p, i, dt, (float)v); break;
  }
}
// Rounds an f32 value through the storage dtype (f16/bf16 round; f32 as is).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == HB_F16) return (float)(f16)v;
  if (dt == HB_BF16) return bf16_to_f32(f32_to_bf16(v));
  return v;
}

// Keeps an f32 value as computed (no contraction of the producing op with a
// following f16 conversion into one mixed-precision instruction), so fused
// kernels round exactly like the separate op they replace.
__device__ __forceinline__ float pin_f32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// GELU for 16-bit outputs (the fused GeGLU epilogue of the GEMMs): erf by
// Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26,
// erf(z) = 1 - t(a1 + t(a2 + t(a3 + t(a4 + t a5)))) exp(-z^2), t = 1/(1 + p z),
// |error| <= 1.5e-7 for z >= 0.  For x < 0, 1 + erf = t(...)exp(-z^2) is used
// directly, so the left tail keeps its relative accuracy.  The result is well
// inside half a unit of f16 / bf16 precision of gelu.
__device__ __forceinline__ float gelu_fast(float x) {
  const float z = fabsf(x) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
  float p = fmaf(t, 1.061405429f, -1.453152027f);
  p = fmaf(t, p, 1.421413741f);
  p = fmaf(t, p, -0.284496736f);
  p = fmaf(t, p, 0.254829592f);
  float pe = p * t * __expf(-z * z);  // 1 - erf(z)
  // pinned: no contraction of p*t*e into the subtraction below, so every
  // caller rounds the same way whatever code surrounds it
  pe = pin_f32(pe);
  return 0.5f * x * (x >= 0.f ? 2.0f - pe : pe);
}

// ------------------------------------------------------------------ wave reductions (wave64)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ------------------------------------------------------------------ strided N-d indexing

constexpr int kMaxRank = 8;
struct Strided {
  int rank;
  int64_t shape[kMaxRank];
  int64_t st[3][kMaxRank];  // element strides of up to three operands
};
// Offsets of linear (row-major over shape) index `i` in up to three operands.
__device__ __forceinline__ void strided_offsets(const Strided& s, int64_t i, int64_t* o0, int64_t* o1, int64_t* o2) {
  int64_t a = 0, b = 0, c = 0;
  for (int d = s.rank - 1; d >= 0; --d) {
    int64_t n = s.shape[d];
    int64_t idx = i % n;
    i /= n;
    a += idx * s.st[0][d];
    b += idx * s.st[1][d];
    c += idx * s.st[2][d];
  }
  *o0 = a;
  *o1 = b;
  *o2 = c;
}

inline int64_t numel(const int64_t* shape, int rank) {
  int64_t n = 1;
  for (int i = 0; i < rank; i++) n *= shape[i];
  return n;
}

inline unsigned grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  if (g > (1 << 30)) g = 1 << 30;
  return (unsigned)(g < 1 ? 1 : g);
}

// Blocks are dealt to the 8 XCDs in turn (block b runs on XCD b % 8, each
// XCD with its own L2).  This maps block `bid` of `nb` to a work index so
// that every XCD takes one contiguous run of indices, in order: work items
// next to each other in the index run at the same time on one XCD and share
// what they read in its L2.
__device__ __forceinline__ int xcd_tile(int bid, int nb) {
  int xcd = bid & 7, idx = bid >> 3;
  int q = nb >> 3, rem = nb & 7;
  return xcd * q + (xcd < rem ? xcd : rem) + idx;
}

}  // namespace hb

// Every exported entry point: catch, record the message, return -1.
#define HB_API_BEGIN try {
#define HB_API_END                        \
  }                                       \
  catch (const std::exception& e) {       \
    hb::set_error(e.what());              \
    return -1;                            \
  }                                       \
  catch (...) {                           \
    hb::set_error("unknown error");       \
    return -1;                            \
  }                                       \
  return 0;
