// Routing (softmax + top-k threshold), bucketing of tokens by expert, and the
// expert-ordered combine, with their backward passes.
//
//  route_topk        usaf/qwen3moe_dml.py:73-83
//  bucket_by_expert  benchmarks/kaggle_t4_bench.py:293-306 (nonzero -> bincount
//                    -> stable argsort by expert -> offsets)
//  moe_combine       usaf/qwen3moe_dml.py:62-64 (fp32 accumulation in expert order)
#include "common.h"

#include <atomic>
#include <mutex>

namespace usaf {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// k-th largest value (counting repeats, as torch.topk(...).values[:, -1]) of
// the valid entries held by the wave: VPL values per lane, element e = lane + 64*j.
template <int VPL>
__device__ __forceinline__ float kth_largest(const float (&p)[VPL], const bool (&valid)[VPL], int k, int lane) {
  bool taken[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) taken[j] = !valid[j];
  float thr = -INFINITY;
  for (int r = 0; r < k; ++r) {
    // lane-local best (largest value, lowest element index on ties)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = lane + kWave * j;
      if (!taken[j] && (p[j] > bv || (p[j] == bv && e < bi))) { bv = p[j]; bi = e; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, kWave);
      const int oi = __shfl_xor(bi, off, kWave);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    thr = bv;
    if (bi == 0x7fffffff) break;  // fewer valid entries than k
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (lane + kWave * j == bi) taken[j] = true;
  }
  return thr;
}

// Softmax over the row (fp32), as F.softmax(logits, dtype=float).
template <int VPL>
__device__ __forceinline__ void row_softmax(float (&p)[VPL], const bool (&valid)[VPL]) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPL; ++j) if (valid[j]) m = fmaxf(m, p[j]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    p[j] = valid[j] ? expf(p[j] - m) : 0.f;
    s += p[j];
  }
  s = wave_sum(s);
#pragma unroll
  for (int j = 0; j < VPL; ++j) p[j] = p[j] / s;
}

// Routing of one token by one wavefront, from its logits (VPL per lane,
// element e = lane + 64 j; invalid entries ignored): softmax, top-k threshold
// mask, optional renormalisation; writes weights[t, :] and probs[t, :].
template <int VPL, int WDT>
__device__ __forceinline__ void route_token(float (&p)[VPL], const bool (&valid)[VPL], int64_t t, int E, int k,
                                            int norm, void* __restrict__ weights, float* __restrict__ probs,
                                            int lane) {
  row_softmax<VPL>(p, valid);
  const float thr = kth_largest<VPL>(p, valid, k, lane);
  float w[VPL];
  float ws = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    w[j] = (valid[j] && p[j] >= thr) ? p[j] : 0.f;  // probs * mask
    ws += w[j];
  }
  if (norm) {
    ws = fmaxf(wave_sum(ws), 1e-9f);
#pragma unroll
    for (int j = 0; j < VPL; ++j) w[j] = w[j] / ws;
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    if (!valid[j]) continue;
    const int64_t i = t * E + lane + kWave * j;
    store_from_f32<WDT>(weights, i, w[j]);
    if (probs) probs[i] = p[j];
  }
}

// One wavefront per token.
template <int VPL, int LDT, int WDT>
__global__ __launch_bounds__(256) void route_topk_kernel(const void* __restrict__ logits, int64_t T, int E, int k,
                                                         int norm, void* __restrict__ weights,
                                                         float* __restrict__ probs) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  float p[VPL];
  bool valid[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + kWave * j;
    valid[j] = e < E;
    p[j] = valid[j] ? load_as_f32<LDT>(logits, t * E + e) : -INFINITY;
  }
  route_token<VPL, WDT>(p, valid, t, E, k, norm, weights, probs, lane);
}

// Backward of route_topk: d(weights) -> d(logits) through the mask, the
// optional renormalisation and the fp32 softmax (probs saved by the forward).
template <int VPL, int WDT, int LDT>
__global__ __launch_bounds__(256) void route_topk_bwd_kernel(const void* __restrict__ dweights,
                                                             const float* __restrict__ probs, int64_t T, int E, int k,
                                                             int norm, void* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  float p[VPL], g[VPL];
  bool valid[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + kWave * j;
    valid[j] = e < E;
    p[j] = valid[j] ? probs[t * E + e] : -INFINITY;
    g[j] = valid[j] ? load_as_f32<WDT>(dweights, t * E + e) : 0.f;
  }
  const float thr = kth_largest<VPL>(p, valid, k, lane);
  bool sel[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) sel[j] = valid[j] && p[j] >= thr;
  if (norm) {
    // w = w0 / s, s = max(sum(w0), 1e-9), w0 = p * mask
    float s = 0.f, gw = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) if (sel[j]) s += p[j];
    s = wave_sum(s);
    const bool clamped = s < 1e-9f;
    const float sc = clamped ? 1e-9f : s;
#pragma unroll
    for (int j = 0; j < VPL; ++j) if (sel[j]) gw += g[j] * p[j];
    gw = wave_sum(gw);
#pragma unroll
    for (int j = 0; j < VPL; ++j) g[j] = clamped ? g[j] / sc : g[j] / sc - gw / (sc * sc);
  }
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    g[j] = sel[j] ? g[j] : 0.f;  // d(probs) = d(w0) * mask
    if (valid[j]) dot += g[j] * p[j];
  }
  dot = wave_sum(dot);
#pragma unroll
  for (int j = 0; j < VPL; ++j)
    if (valid[j]) store_from_f32<LDT>(dlogits, t * E + lane + kWave * j, p[j] * (g[j] - dot));
}

// ---- bucketing ------------------------------------------------------------------
// Three passes over the [T, E] routing weights, chunked by kChunk tokens:
//  count: per (chunk, expert) number of nonzero weights
//  scan : per-expert totals -> counts, offsets; per (chunk, expert) base slot
//  fill : token ids in ascending order within each expert (a stable sort by
//         expert), slot weights, and the [T, E] token/expert -> slot map.
// Count and fill issue a chunk's kChunk loads per thread before using them;
// the scan splits each expert's chunk list over 1024 / E threads.
constexpr int kChunk = 16;

template <int WDT>
__global__ __launch_bounds__(256) void bucket_count_kernel(const void* __restrict__ w, int64_t T, int E,
                                                           int32_t* __restrict__ chunk_cnt) {
  const int64_t c = blockIdx.x;
  const int64_t t0 = c * kChunk;
  const int nt = (T - t0 < kChunk) ? (int)(T - t0) : kChunk;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float v[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) v[j] = j < nt ? load_as_f32<WDT>(w, (t0 + j) * E + e) : 0.f;
    int n = 0;
#pragma unroll
    for (int j = 0; j < kChunk; ++j) n += v[j] != 0.f;
    chunk_cnt[c * E + e] = n;
  }
}

// Single block of 1024 threads; E <= 1024.  Thread (e, seg) owns expert e's
// chunks [seg * per, (seg + 1) * per).  Offsets are clamped to `capacity`;
// with `overflow` set (capacity mode) the slots [offsets[E], capacity) get
// token 0 and weight 0, and *overflow becomes 1 when the pairs exceed capacity.
__global__ __launch_bounds__(1024) void bucket_scan_kernel(int32_t* __restrict__ chunk_cnt, int64_t n_chunks, int E,
                                                           int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                           int64_t capacity, int32_t* __restrict__ token_idx,
                                                           float* __restrict__ slot_w, int32_t* __restrict__ overflow) {
  __shared__ int32_t s_seg[1024];
  __shared__ int32_t s_tot[1024];
  const int tid = threadIdx.x;
  const int nseg = 1024 / E;
  const int e = tid % E, seg = tid / E;
  const bool active = seg < nseg;
  const int64_t per = (n_chunks + nseg - 1) / nseg;
  const int64_t c0 = active ? (int64_t)seg * per : 0;
  const int64_t c1 = active ? (c0 + per < n_chunks ? c0 + per : n_chunks) : 0;
  int sum = 0;
  for (int64_t c = c0; c < c1; c += 8) {
    int v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c + j < c1 ? chunk_cnt[(c + j) * E + e] : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[j];
  }
  s_seg[tid] = sum;
  __syncthreads();
  int tot = 0;
  if (tid < E) {  // exclusive prefix over the expert's segments, in place
    for (int q = 0; q < nseg; ++q) {
      const int v = s_seg[q * E + tid];
      s_seg[q * E + tid] = tot;
      tot += v;
    }
    counts[tid] = tot;
  }
  s_tot[tid] = tid < E ? tot : 0;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scan over the experts
    const int v = (tid >= off) ? s_tot[tid - off] : 0;
    __syncthreads();
    s_tot[tid] += v;
    __syncthreads();
  }
  const int64_t total = s_tot[E - 1];
  const int64_t s_end = total < capacity ? total : capacity;
  __shared__ int32_t s_base[1024];
  if (tid < E) {
    const int64_t base = s_tot[tid] - tot;
    s_base[tid] = (int32_t)base;
    offsets[tid] = (int32_t)(base < capacity ? base : capacity);
  }
  if (tid == 0) {
    offsets[E] = (int32_t)s_end;
    if (overflow && total > capacity) overflow[0] = 1;
  }
  __syncthreads();
  // chunk bases (unclamped: the fill stores only slots below capacity)
  int run = active ? s_base[e] + s_seg[seg * E + e] : 0;
  for (int64_t c = c0; c < c1; c += 8) {
    int v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c + j < c1 ? chunk_cnt[(c + j) * E + e] : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (c + j < c1) chunk_cnt[(c + j) * E + e] = run;
      run += v[j];
    }
  }
  if (overflow)
    for (int64_t i = s_end + tid; i < capacity; i += 1024) {
      token_idx[i] = 0;
      slot_w[i] = 0.f;
    }
}

template <int WDT>
__global__ __launch_bounds__(256) void bucket_fill_kernel(const void* __restrict__ w, int64_t T, int E,
                                                          const int32_t* __restrict__ chunk_base,
                                                          int64_t capacity, int32_t* __restrict__ token_idx,
                                                          float* __restrict__ slot_w, int32_t* __restrict__ pair_slot) {
  const int64_t c = blockIdx.x;
  const int64_t t0 = c * kChunk;
  const int nt = (T - t0 < kChunk) ? (int)(T - t0) : kChunk;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float v[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) v[j] = j < nt ? load_as_f32<WDT>(w, (t0 + j) * E + e) : 0.f;
    int64_t pos = chunk_base[c * E + e];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      if (j < nt) {
        int32_t sl = -1;
        if (v[j] != 0.f) {
          if (pos < capacity) {
            token_idx[pos] = (int32_t)(t0 + j);
            slot_w[pos] = v[j];
            sl = (int32_t)pos;
          }
          ++pos;
        }
        pair_slot[(t0 + j) * E + e] = sl;
      }
    }
  }
}

// ---- combine ---------------------------------------------------------------------
// out[t] = dtype( sum over experts e ascending of float(y[slot(t,e)]) * float(w[t,e]) )
// with the sum in fp32 and each product rounded before it is added (no FMA),
// which is the reference's `final = final + cur.float() * w.float()` sequence.
// w == nullptr: unweighted sum (the backward's gradient accumulation over experts).
template <int DT>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y, const void* __restrict__ w,
                                                      const int32_t* __restrict__ pair_slot, int64_t T, int E,
                                                      int64_t H, uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
  // The token's routed slots, in expert order, are listed in LDS first (wave 0,
  // ballot-compacted), so the row loads of up to 8 experts are issued together
  // instead of one expert's load at a time behind the scan of pair_slot.
  __shared__ int32_t s_slot[1024];
  __shared__ float s_w[1024];
  __shared__ int32_t s_n;
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid < 64) {
    int base = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + tid;
      const int32_t sl = e < E ? pair_slot[t * E + e] : -1;
      const uint64_t mask = __ballot(sl >= 0);
      if (sl >= 0) {
        const int pos = base + __popcll(mask & ((1ull << tid) - 1ull));
        s_slot[pos] = sl;
        s_w[pos] = w ? load_as_f32<DT>(w, t * E + e) : 1.0f;
      }
      base += __popcll(mask);
    }
    if (tid == 0) s_n = base;
  }
  __syncthreads();
  const int n = s_n;
  // 8 consecutive features per thread per pass (one 128-bit load of each row)
  for (int64_t h0 = (int64_t)tid * 8; h0 < H; h0 += (int64_t)blockDim.x * 8) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    const bool vec = h0 + 8 <= H && H % 8 == 0 && (((uintptr_t)y & 15) == 0);
    for (int i0 = 0; i0 < n; i0 += 8) {
      uint4 q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        q[i] = make_uint4(0, 0, 0, 0);
        if (i0 + i < n) {
          const uint16_t* yr = y + (int64_t)s_slot[i0 + i] * H + h0;
          if (vec) {
            q[i] = *reinterpret_cast<const uint4*>(yr);
          } else {
            uint16_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (h0 + j < H) ? yr[j] : 0;
            q[i] = make_uint4(v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16),
                              v[4] | ((uint32_t)v[5] << 16), v[6] | ((uint32_t)v[7] << 16));
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i0 + i < n) {
          const float we = s_w[i0 + i];
          const uint16_t v[8] = {(uint16_t)q[i].x, (uint16_t)(q[i].x >> 16), (uint16_t)q[i].y,
                                 (uint16_t)(q[i].y >> 16), (uint16_t)q[i].z, (uint16_t)(q[i].z >> 16),
                                 (uint16_t)q[i].w, (uint16_t)(q[i].w >> 16)};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float yv = load_as_f32<DT>(v, j);
            const float prod = w ? yv * we : yv;
            acc[j] = acc[j] + prod;
          }
        }
      }
    }
    uint16_t* const orow = out + t * H + h0;
    if (vec && (((uintptr_t)out & 15) == 0)) {
      uint16_t b[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) store_from_f32<DT>(b, j, acc[j]);
      *reinterpret_cast<uint4*>(orow) = make_uint4(b[0] | ((uint32_t)b[1] << 16), b[2] | ((uint32_t)b[3] << 16),
                                                   b[4] | ((uint32_t)b[5] << 16), b[6] | ((uint32_t)b[7] << 16));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (h0 + j < H) store_from_f32<DT>(out, t * H + h0 + j, acc[j]);
    }
  }
}

// Backward of the weighted combine, one block per slot m (token t = token_idx[m],
// expert e): dcur[m] = dtype(float(dout[t]) * w_m) and
// dweights[t, e] = dtype(sum_h float(dout[t,h]) * float(y[m,h])).
template <int DT>
__global__ __launch_bounds__(256) void combine_bwd_kernel(const uint16_t* __restrict__ dout,
                                                          const uint16_t* __restrict__ y,
                                                          const int32_t* __restrict__ token_idx,
                                                          const float* __restrict__ slot_w,
                                                          const int32_t* __restrict__ offsets, int E, int64_t H,
                                                          uint16_t* __restrict__ dcur, void* __restrict__ dweights) {
#pragma clang fp contract(off)
  __shared__ float s_part[4];
  const int64_t m = blockIdx.x;
  if (m >= offsets[E]) return;  // padding slots of a capacity-mode bucketing (block-uniform)
  const int64_t t = token_idx[m];
  const float wm = slot_w[m];
  float part = 0.f;
  if (H % 8 == 0 && ((((uintptr_t)dout | (uintptr_t)y | (uintptr_t)dcur) & 15) == 0)) {
    // 8 consecutive features per thread per pass: 16-byte loads of dout and y, one 16-byte store of dcur
    for (int64_t h = (int64_t)threadIdx.x * 8; h < H; h += (int64_t)blockDim.x * 8) {
      const uint4 gq = *reinterpret_cast<const uint4*>(dout + t * H + h);
      const uint4 yq = *reinterpret_cast<const uint4*>(y + m * H + h);
      const uint16_t gv[8] = {(uint16_t)gq.x, (uint16_t)(gq.x >> 16), (uint16_t)gq.y, (uint16_t)(gq.y >> 16),
                              (uint16_t)gq.z, (uint16_t)(gq.z >> 16), (uint16_t)gq.w, (uint16_t)(gq.w >> 16)};
      const uint16_t yv[8] = {(uint16_t)yq.x, (uint16_t)(yq.x >> 16), (uint16_t)yq.y, (uint16_t)(yq.y >> 16),
                              (uint16_t)yq.z, (uint16_t)(yq.z >> 16), (uint16_t)yq.w, (uint16_t)(yq.w >> 16)};
      uint16_t dv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g = load_as_f32<DT>(gv, j);
        store_from_f32<DT>(dv, j, g * wm);
        part += g * load_as_f32<DT>(yv, j);
      }
      *reinterpret_cast<uint4*>(dcur + m * H + h) =
          make_uint4(dv[0] | ((uint32_t)dv[1] << 16), dv[2] | ((uint32_t)dv[3] << 16), dv[4] | ((uint32_t)dv[5] << 16),
                     dv[6] | ((uint32_t)dv[7] << 16));
    }
  } else {
    for (int64_t h = threadIdx.x; h < H; h += blockDim.x) {
      const float g = load_as_f32<DT>(dout, t * H + h);
      store_from_f32<DT>(dcur, m * H + h, g * wm);
      part += g * load_as_f32<DT>(y, m * H + h);
    }
  }
  part = wave_sum(part);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = part;
  __syncthreads();
  if (threadIdx.x == 0) {
    float tot = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += s_part[i];
    // expert of slot m: largest e with offsets[e] <= m (offsets ascending)
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (offsets[mid] <= m) lo = mid; else hi = mid - 1;
    }
    store_from_f32<DT>(dweights, t * E + lo, tot);
  }
}

template <int VPL>
int launch_route(const void* logits, int ldt, int64_t T, int E, int k, int norm, void* weights, int wdt, float* probs,
                 hipStream_t st) {
  const unsigned blocks = (unsigned)((T + 3) / 4);
  USAF_DISPATCH_DT(ldt, LDT, USAF_DISPATCH_DT(wdt, WDT, route_topk_kernel<VPL, LDT, WDT><<<blocks, 256, 0, st>>>(
                                                            logits, T, E, k, norm, weights, probs)));
  return check_launch("route_topk");
}

template <int VPL>
int launch_route_bwd(const void* dw, int wdt, const float* probs, int64_t T, int E, int k, int norm, void* dlogits,
                     int ldt, hipStream_t st) {
  const unsigned blocks = (unsigned)((T + 3) / 4);
  USAF_DISPATCH_DT(wdt, WDT, USAF_DISPATCH_DT(ldt, LDT, route_topk_bwd_kernel<VPL, WDT, LDT><<<blocks, 256, 0, st>>>(
                                                            dw, probs, T, E, k, norm, dlogits)));
  return check_launch("route_topk_bwd");
}

int check_route_args(const char* what, int64_t T, int64_t E, int64_t k) {
  if (T < 0 || E <= 0 || E > 1024) return set_error(USAF_ERR_INVALID, "%s: need 0 < E <= 1024, got E=%lld", what, (long long)E);
  if (k <= 0 || k > E) return set_error(USAF_ERR_INVALID, "%s: need 0 < top_k <= E, got top_k=%lld", what, (long long)k);
  if (T > (int64_t)0x7fffffff * 4) return set_error(USAF_ERR_INVALID, "%s: too many tokens", what);
  return USAF_OK;
}

// ---- router weight gradient ---------------------------------------------------------
// dW[e, h] = dtype( sum_t fp32(dl[t, e]) * fp32(x[t, h]) ): the weight gradient of
// the router's F.linear (qwen3moe_dml.py:72), a GEMM whose contraction runs over
// the tokens -- the slow index of both operands.  A block computes a 128 (e) x
// 128 (h) tile over one split of the tokens with v_mfma_f32_32x32x16; 64-token
// chunks of both operands are transposed through LDS (tt_write) so that each
// MFMA fragment (8 consecutive tokens) is one 16-byte LDS read.  The fp32 tile
// goes to ws[split]; router_dw_reduce_kernel adds the splits in order and rounds.
// Wave w owns experts [32 w, 32 w + 32) x all 128 columns (4 accumulator blocks).
typedef float rdw_f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 rdw_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 rdw_f16x8 __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ rdw_f32x16 rdw_mfma(uint4 a, uint4 b, rdw_f32x16 c) {
  if constexpr (DT == USAF_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(rdw_bf16x8, a), __builtin_bit_cast(rdw_bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(rdw_f16x8, a), __builtin_bit_cast(rdw_f16x8, b),
                                                  c, 0, 0, 0);
}

template <int DT>
__global__ __launch_bounds__(256) void router_dw_kernel(const uint16_t* __restrict__ dl, const uint16_t* __restrict__ x,
                                                        int64_t T, int E, int64_t H, int64_t t_per_split,
                                                        float* __restrict__ ws) {
  __shared__ __align__(16) uint32_t sA[2][TT_DWORDS];  // experts e0 + [0, 64), e0 + [64, 128)
  __shared__ __align__(16) uint32_t sB[2][TT_DWORDS];  // columns h0 + [0, 64), h0 + [64, 128)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t h0 = (int64_t)blockIdx.x * 128;
  const int e0 = (int)blockIdx.y * 128;
  const int64_t t_beg = (int64_t)blockIdx.z * t_per_split;
  const int64_t t_end = t_beg + t_per_split < T ? t_beg + t_per_split : T;
  const int sp = tid >> 3, cg = tid & 7;  // writer cell: tokens 2 sp, 2 sp + 1; 8 columns at 8 cg
  rdw_f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = rdw_f32x16{};
  uint4 ra[2][2], rb[2][2];  // [half][token of the pair]
  auto load = [&](int64_t c0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int64_t t = c0 + 2 * sp + u;
        const int e = e0 + 64 * q + 8 * cg;
        const int64_t h = h0 + 64 * q + 8 * cg;
        ra[q][u] = (t < t_end && e < E) ? *reinterpret_cast<const uint4*>(dl + t * E + e) : make_uint4(0, 0, 0, 0);
        rb[q][u] = (t < t_end && h < H) ? *reinterpret_cast<const uint4*>(x + t * H + h) : make_uint4(0, 0, 0, 0);
      }
  };
  load(t_beg);
  for (int64_t c0 = t_beg; c0 < t_end; c0 += 64) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      tt_write(sA[q], sp, cg, ra[q][0], ra[q][1]);
      tt_write(sB[q], sp, cg, rb[q][0], rb[q][1]);
    }
    __syncthreads();
    if (c0 + 64 < t_end) load(c0 + 64);  // next chunk in flight during this chunk's MFMAs
    const int ea = 32 * wave + (lane & 31);  // this lane's A row (expert within the tile)
#pragma unroll
    for (int kb = 0; kb < 64; kb += 16) {
      const int sg = (kb >> 3) + (lane >> 5);
      const uint4 a = tt_read(sA[ea >> 6], ea & 63, sg);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int hb = 32 * j + (lane & 31);
        const uint4 b = tt_read(sB[hb >> 6], hb & 63, sg);
        acc[j] = rdw_mfma<DT>(a, b, acc[j]);
      }
    }
    __syncthreads();
  }
  // acc[j][r]: expert e0 + 32 wave + 8 (r >> 2) + 4 (lane >> 5) + (r & 3), column h0 + 32 j + (lane & 31)
  float* const out = ws + (int64_t)blockIdx.z * E * H;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t h = h0 + 32 * j + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int e = e0 + 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (e < E && h < H) out[(int64_t)e * H + h] = acc[j][r];
    }
  }
}

// ---- router grad-input ------------------------------------------------------------
// dx[t, h] = dtype( dtype(sum_e fp32(dl[t, e]) * fp32(W[e, h])) + fp32(dx[t, h]) )
// (accumulate) or dtype(sum ...) (no accumulate): the grad-input of the router's
// F.linear (qwen3moe_dml.py:72) -- autograd's matmul, rounded to the dtype --
// plus, when accumulating, the gradient the experts' branch gave the same hidden
// states, added and rounded once more as autograd's accumulation of the two.
// A block computes 128 tokens x 128 columns with v_mfma_f32_32x32x16; wave w
// owns tokens [32 w, 32 w + 32) x all 128 columns (4 accumulator blocks).  The
// A fragments (8 consecutive experts of a token row) come straight from global
// memory; W's 64-expert chunks are transposed through LDS (tt_write) so that a
// B fragment (8 consecutive experts of one column) is one 16-byte LDS read.
template <int DT>
__global__ __launch_bounds__(256) void router_dx_kernel(const uint16_t* __restrict__ dl, const uint16_t* __restrict__ w,
                                                        int64_t T, int E, int64_t H, uint16_t* __restrict__ dx,
                                                        int accumulate) {
#pragma clang fp contract(off)
  __shared__ __align__(16) uint32_t sB[2][TT_DWORDS];  // columns h0 + [0, 64), h0 + [64, 128)
  __shared__ __align__(16) uint16_t sC[128 * 136];      // the rounded tile, 128 tokens x 128 columns (+8 pad)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t h0 = (int64_t)blockIdx.x * 128;
  const int64_t t0 = (int64_t)blockIdx.y * 128;
  const int sp = tid >> 3, cg = tid & 7;  // writer cell: experts 2 sp, 2 sp + 1 of the chunk; 8 columns at 8 cg
  const int64_t ta = t0 + 32 * wave + (lane & 31);  // this lane's A row (token)
  const bool t_ok = ta < T;
  rdw_f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = rdw_f32x16{};
  uint4 rb[2][2];  // W rows of the next chunk: [column half][expert of the pair]
  auto load_w = [&](int e0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int e = e0 + 2 * sp + u;
        const int64_t h = h0 + 64 * q + 8 * cg;
        rb[q][u] = (e < E && h < H) ? *reinterpret_cast<const uint4*>(w + (int64_t)e * H + h) : make_uint4(0, 0, 0, 0);
      }
  };
  load_w(0);
  for (int e0 = 0; e0 < E; e0 += 64) {
    __syncthreads();  // the previous chunk's fragment reads are done
#pragma unroll
    for (int q = 0; q < 2; ++q) tt_write(sB[q], sp, cg, rb[q][0], rb[q][1]);
    // the chunk's four A fragments (E % 16 == 0: e < E implies e + 8 <= E)
    uint4 a[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int e = e0 + 16 * s4 + 8 * (lane >> 5);
      a[s4] = (t_ok && e < E) ? *reinterpret_cast<const uint4*>(dl + ta * E + e) : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    if (e0 + 64 < E) load_w(e0 + 64);  // the next chunk's W rows in flight during these MFMAs
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int sg = 2 * s4 + (lane >> 5);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int hb = 32 * j + (lane & 31);
        acc[j] = rdw_mfma<DT>(a[s4], tt_read(sB[hb >> 6], hb & 63, sg), acc[j]);
      }
    }
  }
  // acc[j][r]: token 32 wave + 8 (r >> 2) + 4 (lane >> 5) + (r & 3), column 32 j + (lane & 31) of
  // the tile; rounded to the dtype into LDS, then out (and, accumulating, dx in)
  // as 16-byte row chunks
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tl = 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), hl = 32 * j + (lane & 31);
      sC[tl * 136 + hl] = DT == USAF_F16 ? f32_to_f16_bits(acc[j][r]) : f32_to_bf16_bits(acc[j][r]);
    }
  __syncthreads();
  for (int c = tid; c < 128 * 16; c += 256) {
    const int tl = c >> 4, hc = 8 * (c & 15);
    const int64_t t = t0 + tl, h = h0 + hc;
    if (t >= T || h >= H) continue;  // H % 8 == 0: a chunk is inside or outside
    const uint4 g = *reinterpret_cast<const uint4*>(&sC[tl * 136 + hc]);
    uint4* const o = reinterpret_cast<uint4*>(dx + t * H + h);
    if (accumulate) {
      const uint4 d = *o;
      const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, dw[4] = {d.x, d.y, d.z, d.w};
      uint32_t ow[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x2 a = unpack2<DT>(gw[q]), b = unpack2<DT>(dw[q]);
        ow[q] = pack2<DT>(a.x + b.x, a.y + b.y);
      }
      *o = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    } else {
      *o = g;
    }
  }
}

// ---- router forward: the logits GEMM ------------------------------------------------
// logits[t, e] = dtype( sum_h x[t, h] * W[e, h] ), the router's F.linear
// (qwen3moe_dml.py:72).  A block computes 32 tokens x 32 experts with
// v_mfma_f32_32x32x16; its four waves split the contraction into quarters and
// add their partial tiles in LDS in wave order.  Both operand fragments (8
// consecutive h of one token / one expert) come straight from global memory
// through a ring of RING register slots, the loads of step s + RING issued before
// the MFMA of step s.
template <int DT>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w, int64_t T, int E,
                                                            int64_t H, uint16_t* __restrict__ logits) {
#pragma clang fp contract(off)
  __shared__ float s_part[4][32 * 33];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Blocks go round-robin over the 8 dies (block b on die b % 8).  The
  // expert tiles of one token tile get blocks b, b + 8, b + 16, ... of one die,
  // dispatched together, so that die's L2 serves the token rows to all of them.
  const int n_et = (E + 31) / 32;
  const int64_t r = (int64_t)blockIdx.x / 8;
  const int64_t t0 = ((r / n_et) * 8 + (int64_t)(blockIdx.x % 8)) * 32;
  const int e0 = (int)(r % n_et) * 32;
  if (t0 >= T) return;  // block-uniform: the last token tiles of the padded grid
  // rows past T or E read row 0: their results are never stored, and the loads
  // stay unpredicated (a conditional load joins its branch with a wait)
  const int64_t ta = t0 + (lane & 31) < T ? t0 + (lane & 31) : 0;
  const int eb = e0 + (lane & 31) < E ? e0 + (lane & 31) : 0;
  // A wave's quarter of the contraction goes in 64-wide chunks.  Within a chunk,
  // lane half c reads 32 consecutive elements [32 c, 32 c + 32) of its row as
  // four 16-byte vectors and feeds vector q to MFMA step q: A and B use the same
  // assignment, so the four steps cover the chunk's 64 products exactly once.
  const int64_t chunks = H / 256;  // 64-wide chunks per wave quarter
  const int64_t h0 = (int64_t)wave * chunks * 64 + 32 * (lane >> 5);
  const uint16_t* xa = x + ta * H + h0;
  const uint16_t* wb = w + (int64_t)eb * H + h0;
  rdw_f32x16 acc = rdw_f32x16{};
  constexpr int RING = 2;  // chunks in flight
  uint4 ra[RING][4], rb[RING][4];
#pragma unroll
  for (int c = 0; c < RING; ++c) {
    const int64_t cq = c < chunks ? c : chunks - 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ra[c][q] = *reinterpret_cast<const uint4*>(xa + 64 * cq + 8 * q);
      rb[c][q] = *reinterpret_cast<const uint4*>(wb + 64 * cq + 8 * q);
    }
  }
  for (int64_t c0 = 0; c0 < chunks; c0 += RING) {
#pragma unroll
    for (int c = 0; c < RING; ++c) {
      uint4 a[4], b[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a[q] = ra[c][q];
        b[q] = rb[c][q];
      }
      const int64_t cn = c0 + RING + c < chunks ? c0 + RING + c : chunks - 1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ra[c][q] = *reinterpret_cast<const uint4*>(xa + 64 * cn + 8 * q);
        rb[c][q] = *reinterpret_cast<const uint4*>(wb + 64 * cn + 8 * q);
      }
      if (c0 + c < chunks)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = rdw_mfma<DT>(a[q], b[q], acc);
    }
  }
  // acc[r]: token 8 (r >> 2) + 4 (lane >> 5) + (r & 3), expert e0 + (lane & 31)
#pragma unroll
  for (int r = 0; r < 16; ++r) s_part[wave][(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * 33 + (lane & 31)] = acc[r];
  __syncthreads();
  for (int i = tid; i < 32 * 32; i += 256) {
    const int tl = i >> 5, el = i & 31;
    const int64_t t = t0 + tl;
    const int e = e0 + el;
    if (t < T && e < E) {
      const int j = tl * 33 + el;
      const float v = ((s_part[0][j] + s_part[1][j]) + s_part[2][j]) + s_part[3][j];
      store_from_f32<DT>(logits, t * E + e, v);
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void router_dw_reduce_kernel(const float* __restrict__ ws, int n_split, int64_t n,
                                                               uint16_t* __restrict__ dw) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float a = 0.f;
  for (int q = 0; q < n_split; ++q) a += ws[(int64_t)q * n + i];
  store_from_f32<DT>(dw, i, a);
}

}  // namespace
}  // namespace usaf

using namespace usaf;

extern "C" int usaf_hip_route_topk(const void* logits, int32_t logits_dtype, int64_t T, int64_t E, int64_t top_k,
                                   int32_t norm_topk_prob, void* weights, int32_t weights_dtype, float* probs,
                                   void* stream) {
  if (int rc = check_route_args("route_topk", T, E, top_k)) return rc;
  if (T == 0) return clear_error();
  if (!logits || !weights) return set_error(USAF_ERR_INVALID, "route_topk: null pointer");
  hipStream_t st = as_stream(stream);
  const int e = (int)E, k = (int)top_k, n = norm_topk_prob ? 1 : 0;
  if (E <= 64) return launch_route<1>(logits, logits_dtype, T, e, k, n, weights, weights_dtype, probs, st);
  if (E <= 128) return launch_route<2>(logits, logits_dtype, T, e, k, n, weights, weights_dtype, probs, st);
  if (E <= 256) return launch_route<4>(logits, logits_dtype, T, e, k, n, weights, weights_dtype, probs, st);
  if (E <= 512) return launch_route<8>(logits, logits_dtype, T, e, k, n, weights, weights_dtype, probs, st);
  return launch_route<16>(logits, logits_dtype, T, e, k, n, weights, weights_dtype, probs, st);
}

extern "C" int usaf_hip_route_topk_bwd(const void* dweights, int32_t weights_dtype, const float* probs, int64_t T,
                                       int64_t E, int64_t top_k, int32_t norm_topk_prob, void* dlogits,
                                       int32_t logits_dtype, void* stream) {
  if (int rc = check_route_args("route_topk_bwd", T, E, top_k)) return rc;
  if (T == 0) return clear_error();
  if (!dweights || !probs || !dlogits) return set_error(USAF_ERR_INVALID, "route_topk_bwd: null pointer");
  hipStream_t st = as_stream(stream);
  const int e = (int)E, k = (int)top_k, n = norm_topk_prob ? 1 : 0;
  if (E <= 64) return launch_route_bwd<1>(dweights, weights_dtype, probs, T, e, k, n, dlogits, logits_dtype, st);
  if (E <= 128) return launch_route_bwd<2>(dweights, weights_dtype, probs, T, e, k, n, dlogits, logits_dtype, st);
  if (E <= 256) return launch_route_bwd<4>(dweights, weights_dtype, probs, T, e, k, n, dlogits, logits_dtype, st);
  if (E <= 512) return launch_route_bwd<8>(dweights, weights_dtype, probs, T, e, k, n, dlogits, logits_dtype, st);
  return launch_route_bwd<16>(dweights, weights_dtype, probs, T, e, k, n, dlogits, logits_dtype, st);
}

extern "C" int64_t usaf_hip_bucket_workspace_ints(int64_t T, int64_t E) {
  if (T < 0 || E < 0) return -1;
  return ((T + kChunk - 1) / kChunk) * E;
}

extern "C" int usaf_hip_bucket_by_expert(const void* weights, int32_t weights_dtype, int64_t T, int64_t E,
                                         int32_t* workspace, int32_t* counts, int32_t* offsets, int32_t* token_idx,
                                         float* slot_w, int32_t* pair_slot, int64_t capacity, int32_t* overflow,
                                         void* stream) {
  if (T < 0 || E <= 0 || E > 1024) return set_error(USAF_ERR_INVALID, "bucket_by_expert: need 0 < E <= 1024");
  if (T > 0x7fffffff) return set_error(USAF_ERR_INVALID, "bucket_by_expert: token ids must fit int32");
  if (!counts || !offsets) return set_error(USAF_ERR_INVALID, "bucket_by_expert: null counts/offsets");
  if (T > 0 && (!weights || !workspace || !pair_slot || (capacity > 0 && (!token_idx || !slot_w))))
    return set_error(USAF_ERR_INVALID, "bucket_by_expert: null pointer");
  if (capacity < 0 || capacity > 0x7fffffff) return set_error(USAF_ERR_INVALID, "bucket_by_expert: bad capacity");
  if (overflow && capacity > 0 && (!token_idx || !slot_w))
    return set_error(USAF_ERR_INVALID, "bucket_by_expert: capacity mode needs token_idx and slot_w");
  hipStream_t st = as_stream(stream);
  const int64_t n_chunks = (T + kChunk - 1) / kChunk;
  const int e = (int)E;
  if (n_chunks > 0) {
    USAF_DISPATCH_DT(weights_dtype, WDT,
                     bucket_count_kernel<WDT><<<(unsigned)n_chunks, 256, 0, st>>>(weights, T, e, workspace));
    if (int rc = check_launch("bucket_by_expert/count")) return rc;
  }
  bucket_scan_kernel<<<1, 1024, 0, st>>>(workspace, n_chunks, e, counts, offsets, capacity, token_idx, slot_w,
                                          overflow);
  if (int rc = check_launch("bucket_by_expert/scan")) return rc;
  if (n_chunks > 0) {
    USAF_DISPATCH_DT(weights_dtype, WDT,
                     bucket_fill_kernel<WDT><<<(unsigned)n_chunks, 256, 0, st>>>(
                         weights, T, e, workspace, capacity, token_idx, slot_w, pair_slot));
    if (int rc = check_launch("bucket_by_expert/fill")) return rc;
  }
  return clear_error();
}

// ---- bucketing without an allocation ---------------------------------------------
// The workspace of usaf_hip_bucket_by_expert (per chunk of 16 tokens and expert:
// the pair count, then that chunk's first slot) lives in this file-scope device
// array instead of caller memory, for callers that cannot allocate device
// memory.  Each GPU the library runs on holds its own copy until the process
// ends.  The count pass writes every entry the scan and fill passes read, so
// nothing has to start at zero, and the array keeps the last call's contents.
// Calls that overlap on one GPU (other streams, other threads) share the array
// and race.
constexpr int64_t kBucketScratchInts = int64_t(1) << 20;  // 4 MiB: ceil(T / 16) * E <= 2^20
static __device__ __align__(256) int32_t scratch[kBucketScratchInts];

namespace {
// Device address of `scratch` per device, resolved once per device with that
// device current.  In host code the array's name only stands in for the symbol:
// kernels, copies and fills get this address.
std::mutex g_scratch_mu;
std::atomic<int32_t*> g_scratch_ptr[64];

int bucket_scratch(int32_t** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(USAF_ERR_RUNTIME, "bucket_by_expert_noalloc: no current HIP device");
  }
  if (dev < 0 || dev >= 64) return set_error(USAF_ERR_UNSUPPORTED, "bucket_by_expert_noalloc: device %d >= 64", dev);
  int32_t* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr) {
        (void)hipGetLastError();
        return set_error(USAF_ERR_RUNTIME, "bucket_by_expert_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                         hipGetErrorString(e));
      }
      p = static_cast<int32_t*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return USAF_OK;
}
}  // namespace

int usaf::prepare_noalloc_scratch() {
  int32_t* p = nullptr;
  return bucket_scratch(&p);
}

extern "C" int64_t usaf_hip_bucket_noalloc_max_ints(void) { return kBucketScratchInts; }

extern "C" int usaf_hip_bucket_by_expert_noalloc(const void* weights, int32_t weights_dtype, int64_t T, int64_t E,
                                                 int32_t* counts, int32_t* offsets, int32_t* token_idx,
                                                 float* slot_w, int32_t* pair_slot, int64_t capacity,
                                                 int32_t* overflow, void* stream) {
  if (T < 0 || E <= 0 || E > 1024) return set_error(USAF_ERR_INVALID, "bucket_by_expert_noalloc: need 0 < E <= 1024");
  const int64_t need = usaf_hip_bucket_workspace_ints(T, E);
  if (need > kBucketScratchInts)
    return set_error(USAF_ERR_UNSUPPORTED,
                     "bucket_by_expert_noalloc: T=%lld, E=%lld need %lld workspace ints; the static scratch holds "
                     "%lld (ceil(T/16) * E <= 2^20): use usaf_hip_bucket_by_expert with a workspace",
                     (long long)T, (long long)E, (long long)need, (long long)kBucketScratchInts);
  int32_t* ws = nullptr;
  if (int rc = bucket_scratch(&ws)) return rc;
  return usaf_hip_bucket_by_expert(weights, weights_dtype, T, E, ws, counts, offsets, token_idx, slot_w, pair_slot,
                                   capacity, overflow, stream);
}

extern "C" int usaf_hip_moe_combine(const void* y_slots, const void* weights, const int32_t* pair_slot, int64_t T,
                                    int64_t E, int64_t H, int32_t dtype, void* out, void* stream) {
  if (T < 0 || E <= 0 || H <= 0) return set_error(USAF_ERR_INVALID, "moe_combine: bad sizes");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "moe_combine: dtype must be fp16/bf16");
  if (T == 0) return clear_error();
  if (!y_slots || !pair_slot || !out) return set_error(USAF_ERR_INVALID, "moe_combine: null pointer");
  if (T > 0x7fffffff) return set_error(USAF_ERR_INVALID, "moe_combine: too many tokens");
  if (E > 1024) return set_error(USAF_ERR_UNSUPPORTED, "moe_combine: needs E <= 1024");
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_F16)
    combine_kernel<USAF_F16><<<(unsigned)T, 256, 0, st>>>((const uint16_t*)y_slots, weights, pair_slot, T, (int)E, H,
                                                         (uint16_t*)out);
  else
    combine_kernel<USAF_BF16><<<(unsigned)T, 256, 0, st>>>((const uint16_t*)y_slots, weights, pair_slot, T, (int)E, H,
                                                          (uint16_t*)out);
  return check_launch("moe_combine");
}

extern "C" int usaf_hip_moe_combine_bwd(const void* dout, const void* y_slots, const int32_t* token_idx,
                                        const float* slot_w, const int32_t* offsets, int64_t S, int64_t E, int64_t H,
                                        int32_t dtype, void* dcur, void* dweights, void* stream) {
  if (S < 0 || E <= 0 || H <= 0) return set_error(USAF_ERR_INVALID, "moe_combine_bwd: bad sizes");
  if (dtype != USAF_F16 && dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "moe_combine_bwd: dtype must be fp16/bf16");
  if (S == 0) return clear_error();
  if (!dout || !y_slots || !token_idx || !slot_w || !offsets || !dcur || !dweights)
    return set_error(USAF_ERR_INVALID, "moe_combine_bwd: null pointer");
  if (S > 0x7fffffff) return set_error(USAF_ERR_INVALID, "moe_combine_bwd: too many slots");
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_F16)
    combine_bwd_kernel<USAF_F16><<<(unsigned)S, 256, 0, st>>>((const uint16_t*)dout, (const uint16_t*)y_slots,
                                                             token_idx, slot_w, offsets, (int)E, H, (uint16_t*)dcur,
                                                             dweights);
  else
    combine_bwd_kernel<USAF_BF16><<<(unsigned)S, 256, 0, st>>>((const uint16_t*)dout, (const uint16_t*)y_slots,
                                                              token_idx, slot_w, offsets, (int)E, H, (uint16_t*)dcur,
                                                              dweights);
  return check_launch("moe_combine_bwd");
}

extern "C" int64_t usaf_hip_router_dw_ws_floats(int64_t T, int64_t E, int64_t H) {
  if (T < 0 || E <= 0 || H <= 0) return -1;
  const int64_t tiles = ((H + 127) / 128) * ((E + 127) / 128);
  const int64_t chunks = (T + 63) / 64;
  int64_t ks = (256 + tiles - 1) / tiles;
  if (ks > chunks) ks = chunks;
  if (ks < 1) ks = 1;
  return ks * E * H;
}

extern "C" int usaf_hip_router_dw(const void* dlogits, const void* x, int64_t T, int64_t E, int64_t H, int32_t dtype,
                                  void* dw, float* workspace, void* stream) {
  if (T < 0 || E <= 0 || H <= 0) return set_error(USAF_ERR_INVALID, "router_dw: bad sizes");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "router_dw: dtype must be fp16/bf16");
  if (!dw || !workspace || (T > 0 && (!dlogits || !x))) return set_error(USAF_ERR_INVALID, "router_dw: null pointer");
  if (E % 8 != 0 || H % 8 != 0 || (((uintptr_t)dlogits | (uintptr_t)x) & 15))
    return set_error(USAF_ERR_UNSUPPORTED, "router_dw: needs E, H %% 8 == 0 and 16-byte aligned operands");
  if (E > 0x7fffffff || H > 0x7fffffff || T > 0x7fffffff) return set_error(USAF_ERR_INVALID, "router_dw: too large");
  const int64_t tiles_h = (H + 127) / 128, tiles_e = (E + 127) / 128, chunks = (T + 63) / 64;
  int64_t ks = (256 + tiles_h * tiles_e - 1) / (tiles_h * tiles_e);
  if (ks > chunks) ks = chunks;
  if (ks < 1) ks = 1;
  const int64_t t_per_split = ((chunks + ks - 1) / ks) * 64;
  ks = T > 0 ? (T + t_per_split - 1) / t_per_split : 1;  // splits actually holding tokens (<= workspace count)
  if (tiles_h > 0x7fffffff || tiles_e > 65535 || ks > 65535) return set_error(USAF_ERR_INVALID, "router_dw: too large");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)tiles_h, (unsigned)tiles_e, (unsigned)ks);
  const int64_t n = E * H;
  const unsigned rb = (unsigned)((n + 255) / 256);
  if (dtype == USAF_BF16) {
    router_dw_kernel<USAF_BF16><<<grid, 256, 0, st>>>((const uint16_t*)dlogits, (const uint16_t*)x, T, (int)E, H,
                                                      t_per_split, workspace);
    router_dw_reduce_kernel<USAF_BF16><<<rb, 256, 0, st>>>(workspace, (int)ks, n, (uint16_t*)dw);
  } else {
    router_dw_kernel<USAF_F16><<<grid, 256, 0, st>>>((const uint16_t*)dlogits, (const uint16_t*)x, T, (int)E, H,
                                                     t_per_split, workspace);
    router_dw_reduce_kernel<USAF_F16><<<rb, 256, 0, st>>>(workspace, (int)ks, n, (uint16_t*)dw);
  }
  return check_launch("router_dw");
}

extern "C" int usaf_hip_router_dx(const void* dlogits, const void* w, int64_t T, int64_t E, int64_t H, int32_t dtype,
                                  void* dx, int32_t accumulate, void* stream) {
  if (T < 0 || E <= 0 || H <= 0) return set_error(USAF_ERR_INVALID, "router_dx: bad sizes");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "router_dx: dtype must be fp16/bf16");
  if (T == 0) return clear_error();
  if (!dlogits || !w || !dx) return set_error(USAF_ERR_INVALID, "router_dx: null pointer");
  if (E % 16 != 0 || H % 8 != 0 || (((uintptr_t)dlogits | (uintptr_t)w | (uintptr_t)dx) & 15))
    return set_error(USAF_ERR_UNSUPPORTED, "router_dx: needs E %% 16 == 0, H %% 8 == 0 and 16-byte aligned operands");
  if (E > 0x7fffffff || H > 0x7fffffff) return set_error(USAF_ERR_INVALID, "router_dx: too large");
  const int64_t tiles_h = (H + 127) / 128, tiles_t = (T + 127) / 128;
  if (tiles_h > 0x7fffffff || tiles_t > 65535) return set_error(USAF_ERR_INVALID, "router_dx: too large");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)tiles_h, (unsigned)tiles_t);
  if (dtype == USAF_BF16)
    router_dx_kernel<USAF_BF16><<<grid, 256, 0, st>>>((const uint16_t*)dlogits, (const uint16_t*)w, T, (int)E, H,
                                                      (uint16_t*)dx, accumulate ? 1 : 0);
  else
    router_dx_kernel<USAF_F16><<<grid, 256, 0, st>>>((const uint16_t*)dlogits, (const uint16_t*)w, T, (int)E, H,
                                                     (uint16_t*)dx, accumulate ? 1 : 0);
  return check_launch("router_dx");
}

extern "C" int usaf_hip_router_fwd(const void* x, const void* w, int64_t T, int64_t E, int64_t H, int32_t dtype,
                                   int64_t top_k, int32_t norm_topk_prob, void* logits, void* weights,
                                   int32_t weights_dtype, float* probs, void* stream) {
  if (int rc = check_route_args("router_fwd", T, E, top_k)) return rc;
  if (H <= 0) return set_error(USAF_ERR_INVALID, "router_fwd: bad sizes");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "router_fwd: dtype must be fp16/bf16");
  if (T == 0) return clear_error();
  if (!x || !w || !logits || !weights) return set_error(USAF_ERR_INVALID, "router_fwd: null pointer");
  if (H % 256 != 0 || (((uintptr_t)x | (uintptr_t)w) & 15))
    return set_error(USAF_ERR_UNSUPPORTED, "router_fwd: needs H %% 256 == 0 and 16-byte aligned operands");
  if (((T + 31) / 32 + 7) / 8 * 8 * ((E + 31) / 32) > 0x7fffffff)
    return set_error(USAF_ERR_INVALID, "router_fwd: too many tokens");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)(((T + 31) / 32 + 7) / 8 * 8 * ((E + 31) / 32)));
  if (dtype == USAF_BF16)
    router_logits_kernel<USAF_BF16><<<grid, 256, 0, st>>>((const uint16_t*)x, (const uint16_t*)w, T, (int)E, H,
                                                          (uint16_t*)logits);
  else
    router_logits_kernel<USAF_F16><<<grid, 256, 0, st>>>((const uint16_t*)x, (const uint16_t*)w, T, (int)E, H,
                                                         (uint16_t*)logits);
  if (int rc = check_launch("router_fwd/logits")) return rc;
  return usaf_hip_route_topk(logits, dtype, T, E, top_k, norm_topk_prob, weights, weights_dtype, probs, stream);
}
