// Shared helpers for the usaf_hip C-ABI library (gfx950 / CDNA4).
//
// Every exported entry point validates its arguments on the host, launches on
// the caller's stream and returns a status code; it never throws across the
// ABI.  The message for the last failure on the calling thread is kept in a
// thread-local buffer read back through usaf_hip_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>

#include "../../include/usaf_hip.h"

namespace usaf {

// Records a formatted message as the calling thread's last error; returns `code`.
int set_error(int code, const char* fmt, ...);
// Clears the calling thread's last error; returns USAF_OK.
int clear_error();
// Number of compute units of the current device (cached per device).
int device_cu_count();
// One-time host set-up of the GEMM kernels (dynamic-LDS limits) and of the
// sampled-gradient kernels (occupancy queries); safe to call from any thread,
// run by usaf_hip_init() and otherwise on first use.
void prepare_gemm_kernels();
void prepare_sparse_kernels();
// Resolves the current device's address of the no-alloc bucketing scratch
// array (usaf_hip_bucket_by_expert_noalloc); returns a status code.
int prepare_noalloc_scratch();

// 16-bit float types used in device code.
typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just issued; returns a status code.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(USAF_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return clear_error();
}

// ---- device-side conversions -------------------------------------------------

// fp32 -> bf16 with round-to-nearest-even (NaN stays NaN).  Bit-level form so
// the result does not depend on the compiler's choice of instruction.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load one element of a 16-bit or 32-bit float array as fp32.
template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == USAF_F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (DT == USAF_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}
// Store an fp32 value into a float array of type DT with round-to-nearest-even.
template <int DT>
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v) {
  if constexpr (DT == USAF_F32) reinterpret_cast<float*>(p)[i] = v;
  else if constexpr (DT == USAF_F16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
}
// Round an fp32 value to the storage type DT and back (models a tensor of type DT).
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == USAF_F32) return v;
  else if constexpr (DT == USAF_F16) return (float)(_Float16)v;
  else return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// Conversions on pairs: fp32 -> two 16-bit values of DT (round to nearest
// even, as round_to; one v_cvt_pk_bf16_f32 for bf16) packed low/high, and back.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == USAF_BF16) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    const f16x2 h = {(f16)a, (f16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
}
template <int DT>
__device__ __forceinline__ f32x2 unpack2(uint32_t w) {
  if constexpr (DT == USAF_BF16) return f32x2{__uint_as_float(w << 16), __uint_as_float(w & 0xFFFF0000u)};
  else {
    const f16x2 h = __builtin_bit_cast(f16x2, w);
    return f32x2{(float)h.x, (float)h.y};
  }
}
// ---- 64-slot x 64-feature transposes through LDS ---------------------------------
// The tile is stored feature-major, 32 dwords (64 slots) per feature row; a dword
// holds two consecutive slots.  Writer thread (sp, cg) = (tid >> 3, tid & 7) has
// the 16-byte chunks of features [8 cg, 8 cg + 8) of slots 2 sp and 2 sp + 1 and
// writes 8 dwords, one per feature; reader (cl, sg) fetches the 16 bytes of
// feature cl, slots [8 sg, 8 sg + 8).  The 16-byte groups of a row are XOR
// swizzled by the feature's group of 8 (cl >> 3), which keeps the writes of a
// wave at two lanes per bank and the reads at full 16-byte vectors.
constexpr int TT_DWORDS = 64 * 32;
__device__ __forceinline__ int tt_index(int col, int slot_pair) {
  return col * 32 + ((((slot_pair >> 2) ^ (col >> 3)) & 7) << 2) + (slot_pair & 3);
}
__device__ __forceinline__ void tt_write(uint32_t* tile, int sp, int cg, uint4 a, uint4 b) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    tile[tt_index(8 * cg + 2 * q, sp)] = __builtin_amdgcn_perm(bw[q], aw[q], 0x05040100u);      // low halves
    tile[tt_index(8 * cg + 2 * q + 1, sp)] = __builtin_amdgcn_perm(bw[q], aw[q], 0x07060302u);  // high halves
  }
}
__device__ __forceinline__ uint4 tt_read(const uint32_t* tile, int cl, int sg) {
  return *reinterpret_cast<const uint4*>(&tile[tt_index(cl, 4 * sg)]);
}

}  // namespace usaf

// Dispatch a runtime dtype code onto a template parameter.
#define USAF_DISPATCH_DT(dt, DTNAME, ...)                                        \
  switch (dt) {                                                                \
    case USAF_F32: { constexpr int DTNAME = USAF_F32; __VA_ARGS__; } break;    \
    case USAF_F16: { constexpr int DTNAME = USAF_F16; __VA_ARGS__; } break;    \
    case USAF_BF16: { constexpr int DTNAME = USAF_BF16; __VA_ARGS__; } break;  \
    default: return usaf::set_error(USAF_ERR_INVALID, "unknown dtype code %d", (int)(dt)); \
  }
