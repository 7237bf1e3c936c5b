// 4-bit group codec: unpack+dequant (kernel a) and quantize.
//
// Dequant reproduces usaf/quantization.py:107-132 bit for bit:
//   nibble i of the flat code bytes (low nibble first)  -> q in [0, 15]
//   x = fp16( fp16(q * scale) + zero )                    (two fp16 roundings)
// The fast kernel serves the production layout (group_size 128 -> 64 code
// bytes per group): each lane turns one 32-bit code word into 8 outputs,
// unpacking nibbles in registers with the 0x6400 magic (fp16 1024 + q),
// running packed fp16 mul and add and writing one 128-bit store; a wave's
// loads and stores are contiguous across lanes.  Contraction is disabled so mul+add never fuse into an FMA (an FMA
// rounds once and would not match the reference's two roundings).
#include "common.h"


namespace usaf {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Eight codes of one 32-bit word (bytes b0..b3 hold elements e0..e7 as
// lo(b0), hi(b0), lo(b1), ...) -> four fp16 pairs in natural element order,
// each element fp16(fp16(q*s)+z).
__device__ __forceinline__ void dequant_word_f16(uint32_t w, f16x2 s2, f16x2 z2, uint32_t out[4]) {
#pragma clang fp contract(off)
  const f16x2 magic = {(f16)1024.0f, (f16)1024.0f};
  f16x2 p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // nibble i -> e_i (low half), nibble 4+i -> e_{4+i} (high half), each as 1024+q
    uint32_t bits = ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
    f16x2 q = __builtin_bit_cast(f16x2, bits) - magic;  // exact
    f16x2 m = q * s2;                                    // fp16 round #1
    p[i] = m + z2;                                       // fp16 round #2
  }
  // p[i] = (e_i, e_{i+4}); reorder to (e0,e1) (e2,e3) (e4,e5) (e6,e7)
  uint32_t u0 = __builtin_bit_cast(uint32_t, p[0]);
  uint32_t u1 = __builtin_bit_cast(uint32_t, p[1]);
  uint32_t u2 = __builtin_bit_cast(uint32_t, p[2]);
  uint32_t u3 = __builtin_bit_cast(uint32_t, p[3]);
  out[0] = (u0 & 0xFFFFu) | (u1 << 16);
  out[1] = (u2 & 0xFFFFu) | (u3 << 16);
  out[2] = (u0 >> 16) | (u1 & 0xFFFF0000u);
  out[3] = (u2 >> 16) | (u3 & 0xFFFF0000u);
}

// fp16 pair (as bits) -> bf16 pair (as bits), round-to-nearest-even.  Only
// called for finite scale/zero (no NaN can arise then); NaN-capable groups
// take f16bits_to_bf16bits.
__device__ __forceinline__ uint32_t f16pair_to_bf16pair(uint32_t h2) {
  f16x2 h = __builtin_bit_cast(f16x2, h2);
  f32x2 f = {(float)h.x, (float)h.y};
  bf16x2 b = __builtin_convertvector(f, bf16x2);  // v_cvt_pk_bf16_f32 on gfx950
  return __builtin_bit_cast(uint32_t, b);
}

// Scalar fp16 -> bf16 bits with torch's NaN convention (canonical 0x7FC0).
__device__ __forceinline__ uint16_t f16bits_to_bf16bits(uint16_t h) {
  if ((h & 0x7FFFu) > 0x7C00u) return 0x7FC0u;
  return f32_to_bf16_bits(f16_bits_to_f32(h));
}

// One reference dequant element: fp16(fp16(q*s)+z).
__device__ __forceinline__ uint16_t dequant_one_f16(uint32_t q, uint16_t s_bits, uint16_t z_bits) {
#pragma clang fp contract(off)
  f16 qh = (f16)(float)q;
  f16 s = __builtin_bit_cast(f16, s_bits);
  f16 z = __builtin_bit_cast(f16, z_bits);
  f16 m = qh * s;
  f16 r = m + z;
  return __builtin_bit_cast(uint16_t, r);
}

// Fast path: group_size 128 (64 code bytes per group), 16-byte aligned output.
// Work is cut into wave tiles of 2048 elements (1 KiB of codes, 16 groups).
// Lane l of a wave owns the 8-element units u = l + 64k (k = 0..3) of its
// tile: one 32-bit code word in, one 128-bit store out, so every load and
// store instruction of the wave touches one contiguous 256 B / 1 KiB span.
// UNR tiles are loaded before any is converted to keep more bytes in flight.
// SLICES: the tiles come from a job list instead of one linear range.  Tile t
// belongs to job j = t / tps (tps tiles per slice); it reads tile t % tps of
// source slice src[j] and writes the same tile of destination slice dst[j]
// (slices of tps * 2048 elements).  Jobs naming a slice outside
// [0, n_src) / [0, n_dst) are skipped.
template <int OUT_DT, int UNR, bool SLICES>
__global__ __launch_bounds__(256) void dequant_g128_kernel(const uint32_t* __restrict__ packed,
                                                           const uint16_t* __restrict__ scale,
                                                           const uint16_t* __restrict__ zero,
                                                           u32x4* __restrict__ out, int64_t n_tiles,
                                                           const int64_t* __restrict__ src,
                                                           const int64_t* __restrict__ dst, int64_t tps,
                                                           int64_t n_src, int64_t n_dst) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  // first code word of a tile in the source and first output vector in the destination (-1: skip)
  auto tile_src = [&](int64_t t) -> int64_t {
    if constexpr (SLICES) {
      const int64_t j = t / tps, s0 = src[j], d0 = dst[j];
      if (s0 < 0 || s0 >= n_src || d0 < 0 || d0 >= n_dst) return -1;
      return (s0 * tps + (t - j * tps)) * 256;
    } else {
      return t * 256;
    }
  };
  auto tile_dst = [&](int64_t t) -> int64_t {
    if constexpr (SLICES) {
      const int64_t j = t / tps;
      return (dst[j] * tps + (t - j * tps)) * 256;
    } else {
      return t * 256;
    }
  };
  for (int64_t t0 = wave * UNR; t0 < n_tiles; t0 += n_waves * UNR) {
    uint32_t w[UNR][4];
    uint16_t sb[UNR][4], zb[UNR][4];
    int64_t us[UNR];
#pragma unroll
    for (int r = 0; r < UNR; ++r) {
      us[r] = t0 + r < n_tiles ? tile_src(t0 + r) : -1;
      if (us[r] >= 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t u = us[r] + lane + 64 * k;
          w[r][k] = __builtin_nontemporal_load(packed + u);
          sb[r][k] = scale[u >> 4];
          zb[r][k] = zero[u >> 4];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < UNR; ++r) {
      if (us[r] >= 0) {
        const int64_t ud = tile_dst(t0 + r);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t u = ud + lane + 64 * k;
          const f16 s = __builtin_bit_cast(f16, sb[r][k]);
          const f16 z = __builtin_bit_cast(f16, zb[r][k]);
          const f16x2 s2 = {s, s};
          const f16x2 z2 = {z, z};
          uint32_t h[4];
          dequant_word_f16(w[r][k], s2, z2, h);
          u32x4 v;
          if constexpr (OUT_DT == USAF_F16) {
            v = u32x4{h[0], h[1], h[2], h[3]};
          } else {
            // Non-finite scale or zero can produce NaN; those groups take the
            // scalar conversion that yields torch's canonical bf16 NaN.
            const bool finite = ((sb[r][k] & 0x7C00u) != 0x7C00u) && ((zb[r][k] & 0x7C00u) != 0x7C00u);
            if (finite) {
              v = u32x4{f16pair_to_bf16pair(h[0]), f16pair_to_bf16pair(h[1]), f16pair_to_bf16pair(h[2]),
                        f16pair_to_bf16pair(h[3])};
            } else {
              uint32_t b[4];
#pragma unroll
              for (int j = 0; j < 4; ++j)
                b[j] = (uint32_t)f16bits_to_bf16bits((uint16_t)(h[j] & 0xFFFFu)) |
                       ((uint32_t)f16bits_to_bf16bits((uint16_t)(h[j] >> 16)) << 16);
              v = u32x4{b[0], b[1], b[2], b[3]};
            }
          }
          __builtin_nontemporal_store(v, out + u);
        }
      }
    }
  }
}

// General path: any group size / code-row width, one thread per element.
// Element i reads nibble i of the flat code array (the reference interleaves
// low/high nibbles of the flattened [G, packed_cols] bytes and then slices the
// first G*eff_gs of them, quantization.py:115-127) and group i / eff_gs.
template <int OUT_DT>
__global__ __launch_bounds__(256) void dequant_generic_kernel(const uint8_t* __restrict__ packed,
                                                              const uint16_t* __restrict__ scale,
                                                              const uint16_t* __restrict__ zero,
                                                              uint16_t* __restrict__ out, int64_t begin,
                                                              int64_t numel, int64_t eff_gs) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += stride) {
    const uint32_t byte = packed[i >> 1];
    const uint32_t q = (i & 1) ? (byte >> 4) : (byte & 0xFu);
    const int64_t g = i / eff_gs;
    const uint16_t h = dequant_one_f16(q, scale[g], zero[g]);
    if constexpr (OUT_DT == USAF_F16) out[i] = h;
    else out[i] = f16bits_to_bf16bits(h);
  }
}

// Dequantized values at a list of flat positions, fp32 of the fp16 result:
// the reference's dequantize_4bit(...).reshape(-1)[idx].float() without the
// full tensor (masters of new active positions, train.py:456-465, 589-595).
// Element i takes nibble i of the flat code bytes and group i / eff_gs, as the
// generic kernel; positions outside [0, numel) give NaN and set *bad.
__global__ __launch_bounds__(256) void dequant_at_kernel(const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scale,
                                                         const uint16_t* __restrict__ zero,
                                                         const int64_t* __restrict__ idx, int64_t n, int64_t numel,
                                                         int64_t eff_gs, float* __restrict__ out,
                                                         int32_t* __restrict__ bad) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) {
    const int64_t i = idx[j];
    if (i < 0 || i >= numel) {
      out[j] = __builtin_nanf("");
      if (bad) bad[0] = 1;
      continue;
    }
    const uint32_t byte = packed[i >> 1];
    const uint32_t q = (i & 1) ? (byte >> 4) : (byte & 0xFu);
    const int64_t g = i / eff_gs;
    out[j] = f16_bits_to_f32(dequant_one_f16(q, scale[g], zero[g]));
  }
}

// ---- quantize ------------------------------------------------------------------

__device__ __forceinline__ float nan_min(float a, float b) { return (a != a) ? a : ((b != b) ? b : fminf(a, b)); }
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a) ? a : ((b != b) ? b : fmaxf(a, b)); }

// One wavefront per group.  Lane l owns code bytes j = l, l+64, ... of the
// group, i.e. elements 2j and 2j+1.  Elements past numel are the reference's
// zero padding and take part in min/max (quantization.py:54-60).
template <int IN_DT>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ x, int64_t numel, int64_t eff_gs,
                                                       int64_t n_groups, uint8_t* __restrict__ packed,
                                                       uint16_t* __restrict__ scale, uint16_t* __restrict__ zero) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t g = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (g >= n_groups) return;
  const int64_t base = g * eff_gs;
  const int64_t pb = (eff_gs + 1) >> 1;

  float mn = INFINITY, mx = -INFINITY;
  for (int64_t e = lane; e < eff_gs; e += 64) {
    const int64_t i = base + e;
    const float v = (i < numel) ? load_as_f32<IN_DT>(x, i) : 0.0f;
    mn = nan_min(mn, v);
    mx = nan_max(mx, v);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mn = nan_min(mn, __shfl_xor(mn, off, 64));
    mx = nan_max(mx, __shfl_xor(mx, off, 64));
  }
  float sc = (mx - mn) / 15.0f;
  sc = fmaxf(sc, 1e-12f);
  if (mx != mx || mn != mn) sc = NAN;  // torch.clamp_min propagates NaN

  for (int64_t j = lane; j < pb; j += 64) {
    uint32_t qq[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t e = 2 * j + h;
      uint32_t q = 0;
      if (e < eff_gs) {
        const int64_t i = base + e;
        const float v = (i < numel) ? load_as_f32<IN_DT>(x, i) : 0.0f;
        float r = rintf((v - mn) / sc);
        r = fminf(fmaxf(r, 0.0f), 15.0f);
        q = (uint32_t)r;
      }
      qq[h] = q;
    }
    packed[g * pb + j] = (uint8_t)(qq[0] | (qq[1] << 4));
  }
  if (lane == 0) {
    scale[g] = f32_to_f16_bits(sc);
    zero[g] = f32_to_f16_bits(mn);
  }
}

int launch_blocks(int64_t work_items, int per_block, int max_blocks_per_cu) {
  int64_t blocks = (work_items + per_block - 1) / per_block;
  const int64_t cap = (int64_t)device_cu_count() * max_blocks_per_cu;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

}  // namespace
}  // namespace usaf

using namespace usaf;

namespace usaf {
namespace {
__global__ __launch_bounds__(256) void pack_scale_zero_kernel(const uint16_t* __restrict__ s, const uint16_t* __restrict__ z,
                                                              int64_t n, uint32_t* __restrict__ sz) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    sz[i] = (uint32_t)s[i] | ((uint32_t)z[i] << 16);
}

// Transposed copy of a [E, rows, cols] 4-bit tensor (groups of 128 along cols)
// for the grad-input GEMMs, which contract over rows:
//   qT[e][c][r]        the code of element (r, c); two per byte along r, even r
//                      in the low nibble (the reference's nibble order, on W^T)
//   szT[e][c/128][r/2] = { s(r) | s(r+1) << 16, z(r) | z(r+1) << 16 }
// with s(r), z(r) the fp16 scale/zero of the group holding (r, c).  Codes and
// scale/zero bits are copied unchanged, so W^T dequantizes to exactly the
// transposed values of W.  One block: 64 rows x 128 columns of one expert.
__global__ __launch_bounds__(256) void q4_transpose_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ z, int64_t rows, int64_t cols,
                                                           uint8_t* __restrict__ qT, uint32_t* __restrict__ szT) {
  __shared__ __align__(16) uint8_t tile[64][80];  // 64 rows x 64 code bytes (128 columns), padded
  const int64_t e = blockIdx.z, r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 128;
  const int t = threadIdx.x;
  {
    const int row = t >> 2, part = t & 3;
    const uint4 v = *reinterpret_cast<const uint4*>(q + (((e * rows + r0 + row) * cols + c0) >> 1) + part * 16);
    *reinterpret_cast<uint4*>(&tile[row][part * 16]) = v;
  }
  __syncthreads();
  {
    // column c0 + c, rows r0 + 32 half + [0, 32): 16 output bytes
    const int c = t >> 1, half = t & 1, sh = (c & 1) * 4;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = 32 * half + 8 * k + 2 * b;
        const uint32_t lo = (tile[r][c >> 1] >> sh) & 0xFu, hi = (tile[r + 1][c >> 1] >> sh) & 0xFu;
        acc |= (lo | (hi << 4)) << (8 * b);
      }
      w[k] = acc;
    }
    *reinterpret_cast<uint4*>(qT + (((e * cols + c0 + c) * rows + r0) >> 1) + half * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (t < 32) {
    const int64_t gpr = cols / 128, gc = c0 / 128;
    const int64_t ga = (e * rows + r0 + 2 * t) * gpr + gc, gb = ga + gpr;  // groups of rows r, r + 1
    uint32_t* dst = szT + ((e * gpr + gc) * (rows / 2) + r0 / 2 + t) * 2;
    dst[0] = (uint32_t)s[ga] | ((uint32_t)s[gb] << 16);
    dst[1] = (uint32_t)z[ga] | ((uint32_t)z[gb] << 16);
  }
}
}  // namespace
}  // namespace usaf

extern "C" int usaf_hip_q4_transpose(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                                     int64_t E, int64_t rows, int64_t cols, int8_t* packed_t, uint32_t* sz_t,
                                     void* stream) {
  if (E <= 0 || rows <= 0 || cols <= 0) return set_error(USAF_ERR_INVALID, "q4_transpose: need E, rows, cols > 0");
  if (cols % 128 != 0 || rows % 64 != 0)
    return set_error(USAF_ERR_UNSUPPORTED, "q4_transpose: needs cols %% 128 == 0 and rows %% 64 == 0 (rows=%lld, cols=%lld)",
                     (long long)rows, (long long)cols);
  if (!packed || !scale_f16 || !zero_f16 || !packed_t || !sz_t) return set_error(USAF_ERR_INVALID, "q4_transpose: null pointer");
  if (((uintptr_t)packed & 15) || ((uintptr_t)packed_t & 15))
    return set_error(USAF_ERR_INVALID, "q4_transpose: code buffers must be 16-byte aligned");
  if (E > 65535 || rows / 64 > 65535) return set_error(USAF_ERR_INVALID, "q4_transpose: too large");
  const dim3 grid((unsigned)(cols / 128), (unsigned)(rows / 64), (unsigned)E);
  q4_transpose_kernel<<<grid, 256, 0, as_stream(stream)>>>((const uint8_t*)packed, scale_f16, zero_f16, rows, cols,
                                                          (uint8_t*)packed_t, sz_t);
  return check_launch("q4_transpose");
}

extern "C" int usaf_hip_dequant_q4(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                                   int64_t n_groups, int64_t packed_cols, int64_t group_size, int64_t numel,
                                   void* out, int32_t out_dtype, void* stream) {
  if (numel < 0 || n_groups < 0 || packed_cols < 0 || group_size <= 0)
    return set_error(USAF_ERR_INVALID, "dequant_q4: negative size or non-positive group_size");
  if (out_dtype != USAF_F16 && out_dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "dequant_q4: out_dtype must be fp16 or bf16, got %d", (int)out_dtype);
  if (numel == 0) return clear_error();
  if (!packed || !scale_f16 || !zero_f16 || !out) return set_error(USAF_ERR_INVALID, "dequant_q4: null pointer");
  const int64_t eff_gs = group_size < numel ? group_size : numel;
  const int64_t actual = n_groups * eff_gs;
  if (actual > 2 * n_groups * packed_cols)
    return set_error(USAF_ERR_INVALID, "dequant_q4: %lld groups of %lld elements exceed %lld code nibbles",
                     (long long)n_groups, (long long)eff_gs, (long long)(2 * n_groups * packed_cols));
  if (actual < numel)
    return set_error(USAF_ERR_INVALID, "dequant_q4: %lld groups of %lld elements cannot hold %lld elements",
                     (long long)n_groups, (long long)eff_gs, (long long)numel);
  hipStream_t st = as_stream(stream);

  int64_t done = 0;
  const bool fast = eff_gs == 128 && packed_cols == 64 && (((uintptr_t)packed & 3) == 0) &&
                    (((uintptr_t)out & 15) == 0);
  if (fast) {
    constexpr int UNR = 2;
    const int64_t n_tiles = numel / 2048;
    if (n_tiles > 0) {
      int64_t blocks = (n_tiles + 4 * UNR - 1) / (4 * UNR);  // 4 waves per block, UNR tiles per wave
      if (blocks > 65536) blocks = 65536;
      if (out_dtype == USAF_F16)
        dequant_g128_kernel<USAF_F16, UNR, false><<<(unsigned)blocks, 256, 0, st>>>(
            (const uint32_t*)packed, scale_f16, zero_f16, (u32x4*)out, n_tiles, nullptr, nullptr, 1, 0, 0);
      else
        dequant_g128_kernel<USAF_BF16, UNR, false><<<(unsigned)blocks, 256, 0, st>>>(
            (const uint32_t*)packed, scale_f16, zero_f16, (u32x4*)out, n_tiles, nullptr, nullptr, 1, 0, 0);
      int rc = check_launch("dequant_q4");
      if (rc) return rc;
    }
    done = n_tiles * 2048;
  }
  if (done < numel) {
    const int blocks = launch_blocks(numel - done, 256, 16);
    if (out_dtype == USAF_F16)
      dequant_generic_kernel<USAF_F16><<<blocks, 256, 0, st>>>((const uint8_t*)packed, scale_f16, zero_f16,
                                                               (uint16_t*)out, done, numel, eff_gs);
    else
      dequant_generic_kernel<USAF_BF16><<<blocks, 256, 0, st>>>((const uint8_t*)packed, scale_f16, zero_f16,
                                                                (uint16_t*)out, done, numel, eff_gs);
    return check_launch("dequant_q4");
  }
  return clear_error();
}

extern "C" int usaf_hip_dequant_q4_at(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                                      int64_t n_groups, int64_t packed_cols, int64_t group_size, int64_t numel,
                                      const int64_t* idx, int64_t n, float* out, int32_t* bad_flag, void* stream) {
  if (numel < 0 || n_groups < 0 || packed_cols < 0 || group_size <= 0 || n < 0)
    return set_error(USAF_ERR_INVALID, "dequant_q4_at: negative size or non-positive group_size");
  if (n == 0) return clear_error();
  if (!packed || !scale_f16 || !zero_f16 || !idx || !out) return set_error(USAF_ERR_INVALID, "dequant_q4_at: null pointer");
  const int64_t eff_gs = group_size < numel ? group_size : numel;
  if (numel > 0 && (n_groups * eff_gs > 2 * n_groups * packed_cols || n_groups * eff_gs < numel))
    return set_error(USAF_ERR_INVALID, "dequant_q4_at: %lld groups of %lld elements do not fit %lld elements",
                     (long long)n_groups, (long long)eff_gs, (long long)numel);
  dequant_at_kernel<<<launch_blocks(n, 256, 8), 256, 0, as_stream(stream)>>>(
      (const uint8_t*)packed, scale_f16, zero_f16, idx, n, numel, eff_gs > 0 ? eff_gs : 1, out, bad_flag);
  return check_launch("dequant_q4_at");
}

extern "C" int usaf_hip_dequant_q4_slices(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                                          int64_t n_groups, int64_t slice_elems, int64_t n_jobs,
                                          const int64_t* src_slice, const int64_t* dst_slice, int64_t n_dst_slices,
                                          void* out, int32_t out_dtype, void* stream) {
  if (n_groups < 0 || slice_elems <= 0 || n_jobs < 0 || n_dst_slices < 0)
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices: bad sizes");
  if (out_dtype != USAF_F16 && out_dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices: out_dtype must be fp16 or bf16");
  if (slice_elems % 2048 != 0)
    return set_error(USAF_ERR_UNSUPPORTED, "dequant_q4_slices: slice_elems must be a multiple of 2048");
  if (n_jobs == 0) return clear_error();
  if (!packed || !scale_f16 || !zero_f16 || !src_slice || !dst_slice || !out)
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices: null pointer");
  if ((((uintptr_t)packed) & 3) || (((uintptr_t)out) & 15))
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices: codes must be 4-byte and out 16-byte aligned");
  const int64_t tps = slice_elems / 2048;
  const int64_t n_src = n_groups * 128 / slice_elems;
  const int64_t n_tiles = n_jobs * tps;
  constexpr int UNR = 2;
  int64_t blocks = (n_tiles + 4 * UNR - 1) / (4 * UNR);
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = as_stream(stream);
  if (out_dtype == USAF_F16)
    dequant_g128_kernel<USAF_F16, UNR, true><<<(unsigned)blocks, 256, 0, st>>>(
        (const uint32_t*)packed, scale_f16, zero_f16, (u32x4*)out, n_tiles, src_slice, dst_slice, tps, n_src,
        n_dst_slices);
  else
    dequant_g128_kernel<USAF_BF16, UNR, true><<<(unsigned)blocks, 256, 0, st>>>(
        (const uint32_t*)packed, scale_f16, zero_f16, (u32x4*)out, n_tiles, src_slice, dst_slice, tps, n_src,
        n_dst_slices);
  return check_launch("dequant_q4_slices");
}

namespace usaf {
namespace {

// Expert copies in the fragment order of the dense-weight grouped GEMM: the
// 16-byte chunk c of a slot is (n-tile nt, wave w, k-step ks, fragment
// register j, lane l) with c = (((nt * 8 + w) * nk + ks) * 4 + j) * 64 + l,
// and holds weight row wrow(nt, 32 w + (l & 31)), elements k = 64 ks + 32 (l >> 5)
// + 8 j + [0, 8): what lane l of wave w loads into register j at k-step ks.
// Rows: inter > 0 pairs gate row n = 128 nt + 16 w + (l & 15) with up row
// inter + n (the SwiGLU tile); inter == 0 takes row 256 nt + 32 w + (l & 31).
// Rows past the matrix are zero.  One thread per (tile row, k-step): it reads
// the row's 32 code bytes of the k-step (two 16-byte loads) and its
// scale/zero, and writes the 64 weights as the 8 chunks (j, l >> 5) of lane
// l & 31; the 32 rows of a wave's unit sit in neighbouring threads, so each
// chunk store of 32 threads covers 512 contiguous bytes.
template <int OUT_DT>
__global__ __launch_bounds__(256) void dequant_frag_kernel(const uint8_t* __restrict__ packed,
                                                           const uint16_t* __restrict__ scale,
                                                           const uint16_t* __restrict__ zero, u32x4* __restrict__ out,
                                                           int64_t n_items, int64_t ips, int64_t cps, int64_t w_rows,
                                                           int64_t K, int64_t inter, const int64_t* __restrict__ src,
                                                           const int64_t* __restrict__ dst, int64_t n_src,
                                                           int64_t n_dst) {
  const int64_t nk = K / 64;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < n_items; it += stride) {
    const int64_t job = it / ips, r = it - job * ips;
    const int64_t e = src[job], d = dst[job];
    if (e < 0 || e >= n_src || d < 0 || d >= n_dst) continue;
    const int l32 = (int)(r & 31);
    const int64_t t = r >> 5;
    const int64_t ks = t % nk, unit = t / nk;  // unit = nt * 8 + w
    const int w = (int)(unit & 7);
    const int64_t nt = unit >> 3;
    int64_t row;
    bool valid;
    if (inter > 0) {
      const int64_t n = nt * 128 + 16 * w + (l32 & 15);
      valid = n < inter;
      row = ((l32 & 16) ? inter : 0) + n;
    } else {
      row = nt * 256 + 32 * w + l32;
      valid = row < w_rows;
    }
    u32x4 v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = u32x4{0u, 0u, 0u, 0u};
    if (valid) {
      const int64_t el = (e * w_rows + row) * K + ks * 64;  // multiple of 64: the k-step's first element
      const uint4 c0 = *reinterpret_cast<const uint4*>(packed + (el >> 1));
      const uint4 c1 = *reinterpret_cast<const uint4*>(packed + (el >> 1) + 16);
      const uint32_t words[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const uint16_t sb = scale[el >> 7], zb = zero[el >> 7];
      const f16 sh = __builtin_bit_cast(f16, sb), zh = __builtin_bit_cast(f16, zb);
      const bool finite_sz = ((sb & 0x7C00u) != 0x7C00u) && ((zb & 0x7C00u) != 0x7C00u);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        uint32_t h[4];
        dequant_word_f16(words[q], f16x2{sh, sh}, f16x2{zh, zh}, h);
        if constexpr (OUT_DT == USAF_F16) {
          v[q] = u32x4{h[0], h[1], h[2], h[3]};
        } else if (finite_sz) {
          v[q] = u32x4{f16pair_to_bf16pair(h[0]), f16pair_to_bf16pair(h[1]), f16pair_to_bf16pair(h[2]),
                       f16pair_to_bf16pair(h[3])};
        } else {
          uint32_t b2[4];
#pragma unroll
          for (int u = 0; u < 4; ++u)
            b2[u] = (uint32_t)f16bits_to_bf16bits((uint16_t)(h[u] & 0xFFFFu)) |
                    ((uint32_t)f16bits_to_bf16bits((uint16_t)(h[u] >> 16)) << 16);
          v[q] = u32x4{b2[0], b2[1], b2[2], b2[3]};
        }
      }
    }
    // word q: elements 8 q + [0, 8) of the k-step = register q & 3 of lane l32 + 32 (q >> 2)
    u32x4* o = out + d * cps + (unit * nk + ks) * 256 + l32;
#pragma unroll
    for (int q = 0; q < 8; ++q) o[(q & 3) * 64 + 32 * (q >> 2)] = v[q];
  }
}

}  // namespace
}  // namespace usaf

extern "C" int64_t usaf_hip_frag_slot_elems(int64_t w_rows, int64_t K, int64_t inter) {
  if (w_rows <= 0 || K <= 0 || K % 128 != 0 || inter < 0 || (inter > 0 && w_rows != 2 * inter)) return -1;
  const int64_t n_nt = inter > 0 ? (inter + 127) / 128 : (w_rows + 255) / 256;
  return n_nt * 256 * K;
}

extern "C" int usaf_hip_dequant_q4_slices_frag(const int8_t* packed, const uint16_t* scale_f16,
                                               const uint16_t* zero_f16, int64_t n_experts, int64_t w_rows, int64_t K,
                                               int64_t inter, int64_t n_jobs, const int64_t* src_expert,
                                               const int64_t* dst_slot, int64_t n_slots, void* out,
                                               int32_t out_dtype, void* stream) {
  const int64_t slot_elems = usaf_hip_frag_slot_elems(w_rows, K, inter);
  if (slot_elems < 0 || n_experts < 0 || n_jobs < 0 || n_slots < 0)
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices_frag: needs K %% 128 == 0, w_rows = 2 inter (or inter 0), "
                                       "non-negative counts");
  if (out_dtype != USAF_F16 && out_dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices_frag: out_dtype must be fp16 or bf16");
  if (n_jobs == 0) return clear_error();
  if (!packed || !scale_f16 || !zero_f16 || !src_expert || !dst_slot || !out)
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices_frag: null pointer");
  if ((((uintptr_t)packed) & 15) || (((uintptr_t)out) & 15))
    return set_error(USAF_ERR_INVALID, "dequant_q4_slices_frag: codes and out must be 16-byte aligned");
  const int64_t cps = slot_elems / 8;    // 16-byte chunks per slot
  const int64_t ips = slot_elems / 64;   // (tile row, k-step) items per slot
  const int64_t n_items = n_jobs * ips;
  int64_t blocks = (n_items + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * 16;
  if (blocks > cap) blocks = cap;
  hipStream_t st = as_stream(stream);
  if (out_dtype == USAF_F16)
    dequant_frag_kernel<USAF_F16><<<(unsigned)blocks, 256, 0, st>>>((const uint8_t*)packed, scale_f16, zero_f16,
                                                                    (u32x4*)out, n_items, ips, cps, w_rows, K, inter,
                                                                    src_expert, dst_slot, n_experts, n_slots);
  else
    dequant_frag_kernel<USAF_BF16><<<(unsigned)blocks, 256, 0, st>>>((const uint8_t*)packed, scale_f16, zero_f16,
                                                                     (u32x4*)out, n_items, ips, cps, w_rows, K, inter,
                                                                     src_expert, dst_slot, n_experts, n_slots);
  return check_launch("dequant_q4_slices_frag");
}

extern "C" int usaf_hip_quantize_q4(const void* x, int32_t x_dtype, int64_t numel, int64_t group_size,
                                    int8_t* packed, uint16_t* scale_f16, uint16_t* zero_f16, void* stream) {
  if (numel <= 0) return set_error(USAF_ERR_INVALID, "quantize_q4: Scalar tensors cannot be quantized; numel must be > 0");
  if (group_size <= 0) return set_error(USAF_ERR_INVALID, "quantize_q4: group_size must be positive");
  if (!x || !packed || !scale_f16 || !zero_f16) return set_error(USAF_ERR_INVALID, "quantize_q4: null pointer");
  const int64_t eff_gs = group_size < numel ? group_size : numel;
  const int64_t n_groups = (numel + eff_gs - 1) / eff_gs;
  hipStream_t st = as_stream(stream);
  const int64_t blocks = (n_groups + 3) / 4;  // 4 wavefronts (groups) per 256-thread block
  if (blocks > 0x7fffffffLL) return set_error(USAF_ERR_INVALID, "quantize_q4: too many groups");
  USAF_DISPATCH_DT(x_dtype, DT,
                   quantize_kernel<DT><<<(unsigned)blocks, 256, 0, st>>>(x, numel, eff_gs, n_groups,
                                                                        (uint8_t*)packed, scale_f16, zero_f16));
  return check_launch("quantize_q4");
}

extern "C" int usaf_hip_pack_scale_zero(const uint16_t* scale_f16, const uint16_t* zero_f16, int64_t n_groups,
                                        uint32_t* scale_zero, void* stream) {
  if (n_groups < 0) return set_error(USAF_ERR_INVALID, "pack_scale_zero: negative group count");
  if (n_groups == 0) return clear_error();
  if (!scale_f16 || !zero_f16 || !scale_zero) return set_error(USAF_ERR_INVALID, "pack_scale_zero: null pointer");
  int64_t blocks = (n_groups + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * 8;
  if (blocks > cap) blocks = cap;
  pack_scale_zero_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(scale_f16, zero_f16, n_groups, scale_zero);
  return check_launch("pack_scale_zero");
}
