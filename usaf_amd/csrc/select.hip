// Top-k by magnitude on the GPU: the selection steps of the importance pass
// (usaf/moe_loader.py:584-631 TopKImportanceStore: per-expert top |grad|
// candidates, then a global top-k over the candidates).
//
// Radix select over the magnitude's bit pattern, which orders like the value
// for non-negative floats (NaN above +inf, as torch.topk ranks NaN first):
//   key = bits & 0x7FFF       for fp16 / bf16 input (2 digits of 8 bits)
//   key = bits & 0x7FFFFFFF   for fp32 input        (4 digits)
// Each digit takes one histogram pass over the keys that match the digits
// fixed so far and one single-block pick that fixes the digit holding the
// k-th largest key.  The state (prefix, remaining k, histogram) lives in the
// workspace, so no value goes back to the host.  The threshold key T and the
// number of T-valued keys still needed then drive an ordered compaction:
// every key > T and the first `need` keys == T, in position order.
#include "common.h"

namespace usaf {
namespace {

constexpr int SEL_THREADS = 256;
constexpr int SEL_ITEMS = 16;                           // elements per thread per block chunk
constexpr int SEL_CHUNK = SEL_THREADS * SEL_ITEMS;      // 4096 positions per block
constexpr int SEL_HDR = 4;                              // prefix, k remaining, digit shift, spare
constexpr int SEL_BINS = 256;

template <int DT>
__device__ __forceinline__ uint32_t mag_key(const void* x, int64_t i) {
  if constexpr (DT == USAF_F32) return reinterpret_cast<const uint32_t*>(x)[i] & 0x7FFFFFFFu;
  else return (uint32_t)(reinterpret_cast<const uint16_t*>(x)[i] & 0x7FFFu);
}

template <int DT>
__device__ __forceinline__ float mag_value(const void* x, int64_t i) {
  return fabsf(load_as_f32<DT>(x, i));
}

template <int DT>
constexpr int key_bits() {
  return DT == USAF_F32 ? 32 : 16;
}

__global__ void select_init_kernel(int32_t* __restrict__ ws, int64_t k) {
  const int t = threadIdx.x;
  if (t == 0) {
    ws[0] = 0;        // key prefix fixed so far
    ws[1] = (int32_t)k;  // keys still to select at or below the prefix
  }
  for (int b = t; b < SEL_BINS; b += blockDim.x) ws[SEL_HDR + b] = 0;
}

// Histogram of digit `shift` over the keys whose bits above it equal the prefix.
template <int DT>
__global__ __launch_bounds__(SEL_THREADS) void select_hist_kernel(const void* __restrict__ x, int64_t n, int shift,
                                                                  int32_t* __restrict__ ws) {
  __shared__ int32_t hist[SEL_BINS];
  const int t = threadIdx.x;
  hist[t] = 0;
  __syncthreads();
  const uint32_t prefix = (uint32_t)ws[0];
  const uint32_t hi_mask = shift + 8 >= 32 ? 0u : ~((1u << (shift + 8)) - 1u);
  const int64_t stride = (int64_t)gridDim.x * SEL_THREADS;
  for (int64_t i = (int64_t)blockIdx.x * SEL_THREADS + t; i < n; i += stride) {
    const uint32_t key = mag_key<DT>(x, i);
    if ((key & hi_mask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFFu], 1);
  }
  __syncthreads();
  const int32_t c = hist[t];
  if (c) atomicAdd(&ws[SEL_HDR + t], c);
}

// Fixes digit `shift`: the bin holding the k-th largest matching key, counted
// from the top bin down; clears the histogram for the next digit.
__global__ __launch_bounds__(SEL_BINS) void select_pick_kernel(int shift, int32_t* __restrict__ ws) {
  __shared__ int32_t suffix[SEL_BINS];  // suffix[b] = keys in bins > b
  const int t = threadIdx.x;
  const int32_t c = ws[SEL_HDR + t];
  suffix[t] = c;
  __syncthreads();
  // inclusive suffix sum (Hillis-Steele from the top)
  for (int off = 1; off < SEL_BINS; off <<= 1) {
    const int32_t v = t + off < SEL_BINS ? suffix[t + off] : 0;
    __syncthreads();
    suffix[t] += v;
    __syncthreads();
  }
  const int32_t k = ws[1];
  const int32_t above = suffix[t] - c;  // keys in bins > t
  __syncthreads();
  if (above < k && above + c >= k) {  // exactly one bin qualifies (k >= 1, sum >= k)
    ws[0] = ws[0] | (int32_t)((uint32_t)t << shift);
    ws[1] = k - above;
  }
  ws[SEL_HDR + t] = 0;
}

// Per-block counts of keys > T and == T (T = the full prefix).
template <int DT>
__global__ __launch_bounds__(SEL_THREADS) void select_count_kernel(const void* __restrict__ x, int64_t n,
                                                                   const int32_t* __restrict__ ws,
                                                                   int32_t* __restrict__ blk) {
  __shared__ int32_t s_gt[SEL_THREADS / 64], s_eq[SEL_THREADS / 64];
  const uint32_t thr = (uint32_t)ws[0];
  const int t = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * SEL_CHUNK;
  int gt = 0, eq = 0;
#pragma unroll 4
  for (int j = 0; j < SEL_ITEMS; ++j) {
    const int64_t i = base + (int64_t)j * SEL_THREADS + t;
    if (i < n) {
      const uint32_t key = mag_key<DT>(x, i);
      gt += key > thr;
      eq += key == thr;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    gt += __shfl_down(gt, off);
    eq += __shfl_down(eq, off);
  }
  if ((t & 63) == 0) {
    s_gt[t >> 6] = gt;
    s_eq[t >> 6] = eq;
  }
  __syncthreads();
  if (t == 0) {
    int a = 0, b = 0;
    for (int w = 0; w < SEL_THREADS / 64; ++w) {
      a += s_gt[w];
      b += s_eq[w];
    }
    blk[2 * blockIdx.x] = a;
    blk[2 * blockIdx.x + 1] = b;
  }
}

// Exclusive scan of the per-block (gt, eq) counts, in place, one block.
__global__ __launch_bounds__(1024) void select_scan_kernel(int32_t* __restrict__ blk, int64_t nblk) {
  __shared__ int32_t s_gt[1024], s_eq[1024];
  __shared__ int32_t carry_gt, carry_eq;
  const int t = threadIdx.x;
  if (t == 0) carry_gt = carry_eq = 0;
  __syncthreads();
  for (int64_t b0 = 0; b0 < nblk; b0 += 1024) {
    const int64_t b = b0 + t;
    const int32_t g = b < nblk ? blk[2 * b] : 0, e = b < nblk ? blk[2 * b + 1] : 0;
    s_gt[t] = g;
    s_eq[t] = e;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int32_t vg = t >= off ? s_gt[t - off] : 0, ve = t >= off ? s_eq[t - off] : 0;
      __syncthreads();
      s_gt[t] += vg;
      s_eq[t] += ve;
      __syncthreads();
    }
    if (b < nblk) {
      blk[2 * b] = carry_gt + s_gt[t] - g;
      blk[2 * b + 1] = carry_eq + s_eq[t] - e;
    }
    __syncthreads();
    if (t == 1023) {
      carry_gt += s_gt[t];
      carry_eq += s_eq[t];
    }
    __syncthreads();
  }
}

// Ordered compaction: the selected positions of a block's chunk go out in
// position order at (keys > T before it) + min(keys == T before it, need).
template <int DT>
__global__ __launch_bounds__(SEL_THREADS) void select_write_kernel(const void* __restrict__ x, int64_t n,
                                                                   const int32_t* __restrict__ ws,
                                                                   const int32_t* __restrict__ blk,
                                                                   int64_t* __restrict__ pos, float* __restrict__ vals) {
  __shared__ int32_t w_gt[SEL_THREADS / 64], w_eq[SEL_THREADS / 64];
  const uint32_t thr = (uint32_t)ws[0];
  const int32_t need = ws[1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t base = (int64_t)blockIdx.x * SEL_CHUNK;
  int32_t run_gt = blk[2 * blockIdx.x], run_eq = blk[2 * blockIdx.x + 1];
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  for (int j = 0; j < SEL_ITEMS; ++j) {
    const int64_t i = base + (int64_t)j * SEL_THREADS + t;
    const uint32_t key = i < n ? mag_key<DT>(x, i) : 0u;
    const bool gt = i < n && key > thr, eq = i < n && key == thr;
    const uint64_t bg = __ballot(gt), be = __ballot(eq);
    if (lane == 0) {
      w_gt[wave] = __popcll(bg);
      w_eq[wave] = __popcll(be);
    }
    __syncthreads();
    int32_t pre_gt = run_gt + __popcll(bg & below), pre_eq = run_eq + __popcll(be & below);
    int32_t tot_gt = 0, tot_eq = 0;
#pragma unroll
    for (int w = 0; w < SEL_THREADS / 64; ++w) {
      if (w < wave) {
        pre_gt += w_gt[w];
        pre_eq += w_eq[w];
      }
      tot_gt += w_gt[w];
      tot_eq += w_eq[w];
    }
    if (gt || (eq && pre_eq < need)) {
      const int64_t o = (int64_t)pre_gt + (pre_eq < need ? pre_eq : need);
      pos[o] = i;
      if (vals) vals[o] = mag_value<DT>(x, i);
    }
    run_gt += tot_gt;
    run_eq += tot_eq;
    __syncthreads();
  }
}

template <int DT>
int launch_select(const void* x, int64_t n, int64_t k, int64_t* pos, float* vals, int32_t* ws, hipStream_t st) {
  const int64_t nblk = (n + SEL_CHUNK - 1) / SEL_CHUNK;
  int32_t* blk = ws + SEL_HDR + SEL_BINS;
  int64_t hist_blocks = (n + SEL_THREADS * 8 - 1) / (SEL_THREADS * 8);
  const int64_t cap = (int64_t)device_cu_count() * 8;
  if (hist_blocks > cap) hist_blocks = cap;
  if (hist_blocks < 1) hist_blocks = 1;
  select_init_kernel<<<1, SEL_THREADS, 0, st>>>(ws, k);
  for (int shift = key_bits<DT>() - 8; shift >= 0; shift -= 8) {
    select_hist_kernel<DT><<<(unsigned)hist_blocks, SEL_THREADS, 0, st>>>(x, n, shift, ws);
    select_pick_kernel<<<1, SEL_BINS, 0, st>>>(shift, ws);
  }
  select_count_kernel<DT><<<(unsigned)nblk, SEL_THREADS, 0, st>>>(x, n, ws, blk);
  select_scan_kernel<<<1, 1024, 0, st>>>(blk, nblk);
  select_write_kernel<DT><<<(unsigned)nblk, SEL_THREADS, 0, st>>>(x, n, ws, blk, pos, vals);
  return check_launch("topk_abs");
}

}  // namespace
}  // namespace usaf

using namespace usaf;

extern "C" int64_t usaf_hip_topk_abs_ws_ints(int64_t n) {
  if (n < 0) return -1;
  return SEL_HDR + SEL_BINS + 2 * ((n + SEL_CHUNK - 1) / SEL_CHUNK);
}

extern "C" int usaf_hip_topk_abs(const void* x, int32_t dtype, int64_t n, int64_t k, int64_t* pos, float* vals,
                                 int32_t* workspace, void* stream) {
  if (n < 0 || k < 0) return set_error(USAF_ERR_INVALID, "topk_abs: negative size");
  if (n >= ((int64_t)1 << 31)) return set_error(USAF_ERR_UNSUPPORTED, "topk_abs: needs n < 2^31");
  if (dtype != USAF_F32 && dtype != USAF_F16 && dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "topk_abs: dtype must be fp32, fp16 or bf16");
  if (k > n) k = n;
  if (k == 0) return clear_error();
  if (!x || !pos || !workspace) return set_error(USAF_ERR_INVALID, "topk_abs: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_F32) return launch_select<USAF_F32>(x, n, k, pos, vals, workspace, st);
  if (dtype == USAF_F16) return launch_select<USAF_F16>(x, n, k, pos, vals, workspace, st);
  return launch_select<USAF_BF16>(x, n, k, pos, vals, workspace, st);
}
