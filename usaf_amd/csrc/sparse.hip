// Sparse gradient path and optimizer, all in HBM:
//   gather_transpose   slot-major operands for the sampled products
//   sddmm_masked       dW at the active positions only (SparseGradStore.add,
//                      moe_loader.py:564-578, fed by F.linear's weight grad)
//   sparse_adam_step   SparseAdam.step, compact_params path (sparse_optim.py:86-134)
//   scale_check        cg = compact / denom + finite flag (train.py:661-663)
//   overlay_scatter    base.flat[idx] = dtype(vals) (moe_loader.py:218-221, 411-443)
#include "common.h"

namespace usaf {
namespace {

// out[c, s] = in[rows ? rows[s] : s, c] for c < C, s < S; 16-bit elements.
// A 64 (s) x 64 (c) tile goes through LDS stored column-major, so that the row
// reads and the column writes are both 16-byte vectors over contiguous runs.
// VEC: C, ld_in and ld_out are multiples of 8 and both bases 16-byte aligned;
// the writes then also cover out[c, S .. round_up(S, 8)) with zeros.
template <bool VEC>
__global__ __launch_bounds__(256) void gather_transpose_kernel(const uint16_t* __restrict__ in, int64_t ld_in,
                                                               const int32_t* __restrict__ rows, int64_t S, int64_t C,
                                                               uint16_t* __restrict__ out, int64_t ld_out) {
  constexpr int LDT = 72;  // scalar path: 64 slots + 8, 64 * 72 halfwords
  __shared__ __align__(16) uint32_t tile32[64 * LDT / 2 > TT_DWORDS ? 64 * LDT / 2 : TT_DWORDS];
  uint16_t* const tile = reinterpret_cast<uint16_t*>(tile32);
  const int64_t s0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;
  if constexpr (VEC) {
    {
      const int sp = threadIdx.x >> 3, cg = threadIdx.x & 7;
      const int64_t sa = s0 + 2 * sp, c = c0 + 8 * cg;
      uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
      if (c < C) {
        if (sa < S) a = *reinterpret_cast<const uint4*>(in + (rows ? (int64_t)rows[sa] : sa) * ld_in + c);
        if (sa + 1 < S) b = *reinterpret_cast<const uint4*>(in + (rows ? (int64_t)rows[sa + 1] : sa + 1) * ld_in + c);
      }
      tt_write(tile32, sp, cg, a, b);
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int v = threadIdx.x + 256 * it;
      const int cl = v >> 3, sg = v & 7;
      const int64_t c = c0 + cl, s = s0 + 8 * sg;
      if (c < C && s < S) *reinterpret_cast<uint4*>(out + c * ld_out + s) = tt_read(tile32, cl, sg);
    }
  } else {
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
    for (int r = ty; r < 64; r += 4) {
      const int64_t s = s0 + r, c = c0 + tx;
      uint16_t v = 0;
      if (s < S && c < C) {
        const int64_t row = rows ? (int64_t)rows[s] : s;
        v = in[row * ld_in + c];
      }
      tile[tx * LDT + r] = v;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
      const int64_t c = c0 + r, s = s0 + tx;
      if (c < C && s < S) out[c * ld_out + s] = tile[r * LDT + tx];
    }
  }
}

// Value of lane (l + R) mod 16 of the lane's 16-lane row (DPP row_ror), so that
// four adds with R = 8, 4, 2, 1 leave the row's sum in every lane of it: one
// VALU instruction per step instead of an LDS-routed ds_bpermute.
template <int R>
__device__ __forceinline__ float row_ror_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + R, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += row_ror_f32<8>(v);
  v += row_ror_f32<4>(v);
  v += row_ror_f32<2>(v);
  v += row_ror_f32<1>(v);
  return v;
}

// Products of two 16-bit pairs accumulated in fp32 (v_dot2_f32_bf16 / _f16).
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == USAF_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// Sixteen lanes per active position p: row code rcode[p] = e << 21 | o (expert
// e, weight row o < 2^21), column col_idx[p] = i:
//   compact[pos(p)] += fp32(DT( sum_{s0 <= s < s1} rowT[o, s] * colT[i, s] ))
// over expert e's slots [s0, s1) = [offsets[e], offsets[e + 1]).  Lane l of a
// group reads slots [b + 8l, b + 8l + 8) of each 128-slot window starting at
// b = s0 rounded down to 8, as one 16-byte load per operand, and accumulates
// them with v_dot2 in fp32; elements outside [s0, s1) (neighbouring experts,
// row padding) are masked to zero in both operands.  Every load stays inside
// the operand rows: w < s1 <= ldT and ldT % 8 == 0, so w + 7 < ldT.  Positions of one weight
// row are adjacent, so the groups of a wave mostly read the same rowT line.
// Rows >= R, experts >= E and columns >= C are skipped.
template <int DT>
__global__ __launch_bounds__(256) void sddmm_kernel(const uint16_t* __restrict__ rowT, const uint16_t* __restrict__ colT,
                                                    int64_t ldT, const int32_t* __restrict__ offsets, int32_t E,
                                                    int32_t R, int32_t C, int64_t n_pos,
                                                    const int32_t* __restrict__ rcode,
                                                    const int32_t* __restrict__ col_idx,
                                                    const int64_t* __restrict__ pos_map, float* __restrict__ compact) {
  const int gl = threadIdx.x & 15;
  // The position list is cut into one contiguous slice per accelerator die
  // (blocks are dispatched round-robin over the dies: block b runs on die
  // b % dies).  Positions come sorted by expert, so the groups of a die work
  // through one expert at a time and its operand rows stay in that die's L2.
  const int dies = gridDim.x < 8 ? (int)gridDim.x : 8;
  const int die = (int)(blockIdx.x % dies);
  const int64_t die_blocks = ((int64_t)gridDim.x + dies - 1 - die) / dies;
  const int64_t lo = n_pos * die / dies, hi = n_pos * (die + 1) / dies;
  const int64_t n_grp = die_blocks * (blockDim.x >> 4);
  for (int64_t p = lo + (int64_t)(blockIdx.x / dies) * (blockDim.x >> 4) + (threadIdx.x >> 4); p < hi; p += n_grp) {
    const uint32_t code = (uint32_t)rcode[p];
    const uint32_t i = (uint32_t)col_idx[p];
    const uint32_t e = code >> 21, o = code & 0x1FFFFFu;
    if (e >= (uint32_t)E || o >= (uint32_t)R || i >= (uint32_t)C) continue;
    int s0 = offsets[e], s1 = offsets[e + 1];
    s0 = s0 < 0 ? 0 : s0;
    s1 = s1 > (int)ldT ? (int)ldT : s1;
    const uint16_t* rv = rowT + (int64_t)o * ldT;
    const uint16_t* cv = colT + (int64_t)i * ldT;
    const unsigned span = (unsigned)(s1 - s0);
    float acc = 0.f;
    for (int w = (s0 & ~7) + 8 * gl; w < s1; w += 128) {
      const uint4 a = *reinterpret_cast<const uint4*>(rv + w);
      const uint4 c = *reinterpret_cast<const uint4*>(cv + w);
      if ((unsigned)(w - s0) < span && (unsigned)(w + 7 - s0) < span) {  // interior: no masking
        acc = dot2<DT>(a.x, c.x, acc);
        acc = dot2<DT>(a.y, c.y, acc);
        acc = dot2<DT>(a.z, c.z, acc);
        acc = dot2<DT>(a.w, c.w, acc);
      } else {
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t m = (((unsigned)(w + 2 * q - s0) < span) ? 0x0000FFFFu : 0u) |
                             (((unsigned)(w + 2 * q + 1 - s0) < span) ? 0xFFFF0000u : 0u);
          acc = dot2<DT>(aw[q] & m, cw[q] & m, acc);
        }
      }
    }
    acc = row16_sum(acc);
    if (gl == 0) {
      const int64_t pos = pos_map ? pos_map[p] : p;
      compact[pos] += round_to<DT>(acc);
    }
  }
}


// ---- per-expert blocked slot-major operands -------------------------------------
// Expert e's slots [s0_e, s0_e + S_e) form a contiguous block of C rows of
// ld_e = round_up(S_e, BLK_PAD) elements at element offset C * P[e], P[e] = sum of
// ld_e' over e' < e; the padding columns [S_e, ld_e) are zero.  A weight
// position's dot product then reads one contiguous, zero-padded run of its
// expert, and one expert's operands are one contiguous region (TLB and L2
// friendly).  P and the per-expert 64-slot chunk counts come from a layout
// table built once per bucketing (blocked_layout_kernel).
constexpr int BLK_MAX_E = 1024;

// Number of 64-slot chunks the blocked layout of S slots over E experts can
// need: sum_e ceil(blk_ld(S_e) / 64) <= (S + (BLK_PAD - 1) E) / 64 + E.
// Expert blocks are padded to BLK_PAD slots: a block row then starts on a 32-byte
// boundary, so the transposes' 128-byte row segments cover whole 32-byte
// sectors and no write of theirs is a partial-sector read-modify-write.
constexpr int BLK_PAD = 16;
constexpr int GT_TILES = 4;  // 64-column tiles per block of the blocked gather-transpose
constexpr int CB_STEPS = 4;  // 64-feature steps per load batch of the blocked combine backward
__host__ __device__ inline int blk_ld(int se) { return (se + BLK_PAD - 1) & ~(BLK_PAD - 1); }
__host__ __device__ inline int64_t blk_chunk_bound(int64_t S, int64_t E) { return (S + BLK_PAD * E) / 64 + E + 1; }

// table[e] = P[e] (padded slots before expert e), table[E + 1 + e] = 64-slot
// chunks before expert e (e <= E), table[2(E + 1) + k] = the expert that owns
// chunk k, -1 past the last (k < n_map); one block of 256 threads.
__global__ __launch_bounds__(256) void blocked_layout_kernel(const int32_t* __restrict__ offsets, int E,
                                                             int32_t* __restrict__ table, int64_t S, int64_t n_map) {
  __shared__ int32_t s_tmp[512];
  const int tid = threadIdx.x;
  const int per = (E + 255) / 256;
  int sp = 0, sc = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      const int ld = blk_ld(offsets[e + 1] - offsets[e]);
      sp += ld;
      sc += (ld + 63) >> 6;
    }
  }
  s_tmp[tid] = sp;
  s_tmp[256 + tid] = sc;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int a = tid >= off ? s_tmp[tid - off] : 0, b = tid >= off ? s_tmp[256 + tid - off] : 0;
    __syncthreads();
    s_tmp[tid] += a;
    s_tmp[256 + tid] += b;
    __syncthreads();
  }
  int rp = s_tmp[tid] - sp, rc = s_tmp[256 + tid] - sc;
  int32_t* const map = table + 2 * (E + 1);
  // offsets[E] above the S the table was sized for: map no chunk, so no
  // blocked transpose writes past a buffer of usaf_hip_blocked_elems(S, E)
  const bool fits = offsets[0] == 0 && offsets[E] <= S;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      const int ld = blk_ld(offsets[e + 1] - offsets[e]);
      const int nc = (ld + 63) >> 6;
      table[e] = rp;
      table[E + 1 + e] = rc;
      for (int k = 0; k < nc && rc + k < n_map; ++k) map[rc + k] = fits ? e : -1;
      rp += ld;
      rc += nc;
    }
  }
  for (int64_t k = (int64_t)s_tmp[511] + tid; k < n_map; k += 256) map[k] = -1;
  if (tid == 255) {
    table[E] = s_tmp[255];
    table[2 * E + 1] = s_tmp[511];
  }
}

// out (blocked) from in[rows ? rows[s] : s, c]: a block transposes 64 slots of
// one expert x 64 columns through LDS; grid.x enumerates the (expert, 64-slot
// chunk) pairs (surplus blocks exit), grid.y the 64-column chunks.  16-byte
// loads and stores: C, ld_in multiples of 8, bases 16-byte aligned.
__global__ __launch_bounds__(256) void gather_transpose_blocked_kernel(const uint16_t* __restrict__ in, int64_t ld_in,
                                                                       const int32_t* __restrict__ rows,
                                                                       const int32_t* __restrict__ offsets,
                                                                       const int32_t* __restrict__ table, int E,
                                                                       int64_t C, uint16_t* __restrict__ out) {
  // A block covers one 64-slot chunk and GT_TILES 64-column tiles: the chunk
  // lookup and the row indices are read once, and all the tiles' loads are in
  // flight before the first store.
  __shared__ __align__(16) uint32_t tile32[GT_TILES][TT_DWORDS];
  const int64_t chunk = blockIdx.x;
  const int e = table[2 * (E + 1) + chunk];
  if (e < 0) return;  // block-uniform
  const int s0 = offsets[e], se = offsets[e + 1] - s0, ld = blk_ld(se);
  const int j0 = (int)(chunk - table[E + 1 + e]) * 64;  // first slot of the chunk within the expert
  const int64_t c0 = (int64_t)blockIdx.y * 64 * GT_TILES;
  {
    const int sp = threadIdx.x >> 3, cg = threadIdx.x & 7;
    const int ja = j0 + 2 * sp;
    const int64_t ra = ja < se ? (rows ? (int64_t)rows[s0 + ja] : (int64_t)(s0 + ja)) : -1;
    const int64_t rb = ja + 1 < se ? (rows ? (int64_t)rows[s0 + ja + 1] : (int64_t)(s0 + ja + 1)) : -1;
    uint4 a[GT_TILES], b[GT_TILES];
#pragma unroll
    for (int t = 0; t < GT_TILES; ++t) {
      const int64_t c = c0 + 64 * t + 8 * cg;
      a[t] = make_uint4(0, 0, 0, 0);
      b[t] = make_uint4(0, 0, 0, 0);
      if (c < C) {
        if (ra >= 0) a[t] = *reinterpret_cast<const uint4*>(in + ra * ld_in + c);
        if (rb >= 0) b[t] = *reinterpret_cast<const uint4*>(in + rb * ld_in + c);
      }
    }
#pragma unroll
    for (int t = 0; t < GT_TILES; ++t) tt_write(tile32[t], sp, cg, a[t], b[t]);
  }
  __syncthreads();
  uint16_t* const blk = out + C * (int64_t)table[e];
#pragma unroll
  for (int t = 0; t < GT_TILES; ++t) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int v = threadIdx.x + 256 * it;
      const int cl = v >> 3, sg = v & 7;
      const int64_t c = c0 + 64 * t + cl;
      const int j = j0 + 8 * sg;
      if (c < C && j < ld) *reinterpret_cast<uint4*>(blk + c * ld + j) = tt_read(tile32[t], cl, sg);
    }
  }
}

// Backward of the weighted combine (route.hip's combine_bwd_kernel) fused with
// the blocked transpose of its output.  A block covers one 64-slot chunk of one
// expert (the layout table's chunk map) and a 512-feature range (blockIdx.y):
//   dcur[s, h]   = dtype(fp32(dout[t_s, h]) * w_s)            row-major [S, H]
//   dcurB        = the same values in the blocked slot-major layout (H rows per
//                  expert block, zero padding up to round_up(S_e, BLK_PAD))
//   part[y][s]   = sum over the range of fp32(dout[t_s, h]) * fp32(y[s, h])
// combine_bwd_finish_kernel adds the ranges: dweights[t_s, e] = dtype(sum_y part).
// Needs H % 8 == 0 and 16-byte aligned rows.
template <int DT>
__global__ __launch_bounds__(256) void combine_bwd_blocked_kernel(
    const uint16_t* __restrict__ dout, const uint16_t* __restrict__ y, const int32_t* __restrict__ token_idx,
    const float* __restrict__ slot_w, const int32_t* __restrict__ offsets, const int32_t* __restrict__ table, int E,
    int64_t H, int64_t S_cap, uint16_t* __restrict__ dcur, uint16_t* __restrict__ dcurB, float* __restrict__ part) {
#pragma clang fp contract(off)
  // the 512 features go in batches of CB_STEPS 64-feature steps: every load of
  // a batch is issued before its first product, and one barrier pair serves
  // the batch's transposed stores
  __shared__ __align__(16) uint32_t tile32[CB_STEPS][TT_DWORDS];
  const int64_t chunk = blockIdx.x;
  const int e = table[2 * (E + 1) + chunk];
  if (e < 0) return;  // block-uniform
  const int s0 = offsets[e], se = offsets[e + 1] - s0, ld = blk_ld(se);
  const int j0 = (int)(chunk - table[E + 1 + e]) * 64;  // first slot of the chunk within the expert
  uint16_t* const blk = dcurB + H * (int64_t)table[e];
  const int64_t hbeg = (int64_t)blockIdx.y * 512;
  const int64_t hend = hbeg + 512 < H ? hbeg + 512 : H;
  const int tid = threadIdx.x;
  // this thread's cell: slots 2 sp, 2 sp + 1, features [8 cg, 8 cg + 8) of each 64-feature step
  const int sp = tid >> 3, cg = tid & 7;
  bool ok[2];
  int64_t srow[2], trow[2];
  float wv[2], acc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int j = j0 + 2 * sp + u;
    ok[u] = j < se;
    srow[u] = (int64_t)(s0 + j);
    trow[u] = ok[u] ? (int64_t)token_idx[s0 + j] : 0;
    wv[u] = ok[u] ? slot_w[s0 + j] : 0.f;
    acc[u] = 0.f;
  }
  for (int64_t cb0 = hbeg; cb0 < hend; cb0 += 64 * CB_STEPS) {
    uint4 gq[CB_STEPS][2], yq[CB_STEPS][2];
#pragma unroll
    for (int st = 0; st < CB_STEPS; ++st) {
      const int64_t c = cb0 + 64 * st + 8 * cg;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        gq[st][u] = make_uint4(0, 0, 0, 0);
        yq[st][u] = make_uint4(0, 0, 0, 0);
        if (ok[u] && c < hend) {
          gq[st][u] = *reinterpret_cast<const uint4*>(dout + trow[u] * H + c);
          yq[st][u] = *reinterpret_cast<const uint4*>(y + srow[u] * H + c);
        }
      }
    }
#pragma unroll
    for (int st = 0; st < CB_STEPS; ++st) {
      const int64_t c = cb0 + 64 * st + 8 * cg;
      uint4 d[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        d[u] = make_uint4(0, 0, 0, 0);
        if (ok[u] && c < hend) {
          const uint32_t gw[4] = {gq[st][u].x, gq[st][u].y, gq[st][u].z, gq[st][u].w};
          const uint32_t yw[4] = {yq[st][u].x, yq[st][u].y, yq[st][u].z, yq[st][u].w};
          uint32_t dw[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x2 g = unpack2<DT>(gw[q]), yv = unpack2<DT>(yw[q]);
            dw[q] = pack2<DT>(g.x * wv[u], g.y * wv[u]);
            acc[u] += g.x * yv.x;
            acc[u] += g.y * yv.y;
          }
          d[u] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
          *reinterpret_cast<uint4*>(dcur + srow[u] * H + c) = d[u];
        }
      }
      tt_write(tile32[st], sp, cg, d[0], d[1]);
    }
    __syncthreads();
#pragma unroll
    for (int st = 0; st < CB_STEPS; ++st) {
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int v = tid + 256 * it;
        const int cl = v >> 3, sg = v & 7;
        const int64_t cc = cb0 + 64 * st + cl;
        const int j = j0 + 8 * sg;
        if (cc < hend && j < ld) *reinterpret_cast<uint4*>(blk + cc * ld + j) = tt_read(tile32[st], cl, sg);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float a = acc[u];
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) a += __shfl_xor(a, off, 8);
    if (cg == 0 && ok[u]) part[(int64_t)blockIdx.y * S_cap + srow[u]] = a;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void combine_bwd_finish_kernel(const float* __restrict__ part, int n_split,
                                                                 int64_t S_cap, const int32_t* __restrict__ token_idx,
                                                                 const int32_t* __restrict__ offsets, int E,
                                                                 void* __restrict__ dweights) {
#pragma clang fp contract(off)
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= S_cap || s >= offsets[E]) return;
  float a = 0.f;
  for (int q = 0; q < n_split; ++q) a += part[(int64_t)q * S_cap + s];
  int lo = 0, hi = E - 1;  // expert of slot s: largest e with offsets[e] <= s
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= s) lo = mid; else hi = mid - 1;
  }
  store_from_f32<DT>(dweights, (int64_t)token_idx[s] * E + lo, a);
}

// Sampled gradient on blocked operands: as sddmm_kernel, with expert e's rows
// rowB[e][o] and colB[e][i] contiguous, zero-padded runs of ld_e elements, so
// no masking is needed; the position list is cut into one contiguous slice
// per die, positions sorted by expert keep a die on one expert's operands.
template <int DT>
__global__ __launch_bounds__(256) void sddmm_blocked_kernel(const uint16_t* __restrict__ rowB,
                                                            const uint16_t* __restrict__ colB,
                                                            const int32_t* __restrict__ table, int32_t E,
                                                            int32_t R, int32_t C, int64_t n_pos,
                                                            const int32_t* __restrict__ rcode,
                                                            const int32_t* __restrict__ col_idx,
                                                            const int64_t* __restrict__ pos_map,
                                                            float* __restrict__ compact, int accumulate) {
  __shared__ int32_t s_pre[BLK_MAX_E + 1];
  for (int e = threadIdx.x; e <= E; e += blockDim.x) s_pre[e] = table[e];
  __syncthreads();
  const int gl = threadIdx.x & 15;
  const int dies = gridDim.x < 8 ? (int)gridDim.x : 8;
  const int die = (int)(blockIdx.x % dies);
  const int64_t die_blocks = ((int64_t)gridDim.x + dies - 1 - die) / dies;
  const int64_t lo = n_pos * die / dies, hi = n_pos * (die + 1) / dies;
  const int64_t n_grp = die_blocks * (blockDim.x >> 4);
  // Each group takes runs of RUN consecutive positions; the runs of a die's
  // groups sweep its slice together (run r of group g starts at
  // lo + (r * n_grp + g) * RUN), so the die's L2 holds about one expert's
  // operands at a time.  Positions of one weight row are adjacent, so a run
  // mostly repeats its row: the row operand's first two 128-slot windows stay
  // in registers while the row does not change, halving the loads per position.
  constexpr int RUN = 8;
  const int64_t gi = (int64_t)(blockIdx.x / dies) * (blockDim.x >> 4) + (threadIdx.x >> 4);
  // A run's position data is fetched once: lane j of the group loads position
  // base + j's row code, column and compact slot (and the old compact value),
  // the group takes them from lane j by shuffles, and lane j stores position
  // j's sum at the end -- a handful of memory instructions per run instead of
  // five per position, which the address units were spending most of their time on.
  for (int64_t base = lo + gi * RUN; base < hi; base += n_grp * RUN) {
    const int nrun = (int)(base + RUN < hi ? RUN : hi - base);  // uniform across the group
    uint32_t my_code = 0xFFFFFFFFu, my_i = 0;
    int64_t my_pos = 0;
    float my_old = 0.f, my_sum = 0.f;
    bool my_ok = false;
    if (gl < nrun) {
      my_code = (uint32_t)rcode[base + gl];
      my_i = (uint32_t)col_idx[base + gl];
      my_ok = (my_code >> 21) < (uint32_t)E && (my_code & 0x1FFFFFu) < (uint32_t)R && my_i < (uint32_t)C;
      my_pos = pos_map ? pos_map[base + gl] : base + gl;
      if (my_ok && accumulate) my_old = compact[my_pos];  // else 0 + sum: a zeroed buffer's first add
    }
    uint32_t cached = 0xFFFFFFFFu;
    int ld = 0;
    const uint16_t* rv = rowB;
    uint4 r0 = make_uint4(0, 0, 0, 0), r1 = make_uint4(0, 0, 0, 0);
    for (int j = 0; j < nrun; ++j) {
      const uint32_t code = (uint32_t)__shfl((int)my_code, j, 16);
      const uint32_t i = (uint32_t)__shfl((int)my_i, j, 16);
      const uint32_t e = code >> 21, o = code & 0x1FFFFFu;
      if (e >= (uint32_t)E || o >= (uint32_t)R || i >= (uint32_t)C) continue;  // uniform across the group
      const int pe = s_pre[e];
      if (code != cached) {  // uniform across the group
        cached = code;
        ld = s_pre[e + 1] - pe;
        rv = rowB + (int64_t)R * pe + (int64_t)o * ld;
        r0 = 8 * gl < ld ? *reinterpret_cast<const uint4*>(rv + 8 * gl) : make_uint4(0, 0, 0, 0);
        r1 = 8 * gl + 128 < ld ? *reinterpret_cast<const uint4*>(rv + 8 * gl + 128) : make_uint4(0, 0, 0, 0);
      }
      const uint16_t* cv = colB + (int64_t)C * pe + (int64_t)i * ld;
      float acc = 0.f;
      if (8 * gl < ld) {
        const uint4 c = *reinterpret_cast<const uint4*>(cv + 8 * gl);
        acc = dot2<DT>(r0.x, c.x, acc);
        acc = dot2<DT>(r0.y, c.y, acc);
        acc = dot2<DT>(r0.z, c.z, acc);
        acc = dot2<DT>(r0.w, c.w, acc);
      }
      if (8 * gl + 128 < ld) {
        const uint4 c = *reinterpret_cast<const uint4*>(cv + 8 * gl + 128);
        acc = dot2<DT>(r1.x, c.x, acc);
        acc = dot2<DT>(r1.y, c.y, acc);
        acc = dot2<DT>(r1.z, c.z, acc);
        acc = dot2<DT>(r1.w, c.w, acc);
      }
      for (int w = 8 * gl + 256; w < ld; w += 128) {  // experts past 256 slots
        const uint4 a = *reinterpret_cast<const uint4*>(rv + w);
        const uint4 c = *reinterpret_cast<const uint4*>(cv + w);
        acc = dot2<DT>(a.x, c.x, acc);
        acc = dot2<DT>(a.y, c.y, acc);
        acc = dot2<DT>(a.z, c.z, acc);
        acc = dot2<DT>(a.w, c.w, acc);
      }
      acc = row16_sum(acc);
      if (gl == j) my_sum = round_to<DT>(acc);
    }
    // positions with an invalid row code or column: left alone when accumulating, 0 otherwise
    if (gl < nrun && (my_ok || !accumulate)) compact[my_pos] = my_old + my_sum;
  }
}

// SparseAdam.step for one compact vector (sparse_optim.py:96-130), with the
// rounding of torch's vectorized CPU kernels the reference runs:
//   g = g + wd*p                       mul, add
//   m = fma(1-b1, g, m*b1)             mul_; add_(alpha=) is one fused multiply-add
//   v = v*b2 + ((1-b2)*g)*g            mul_; addcmul_ multiplies then adds
//   p = p + (-lr) * ((m/bias1) / (sqrt(v/bias2) + eps))
// One element of SparseAdam.step (sparse_optim.py:113-134): L2 decay folded into
// the gradient, m/v moving averages, bias-corrected update, in the reference's
// fp32 operation order.
__device__ __forceinline__ void adam_element(float* __restrict__ p, const float* __restrict__ grad,
                                             float* __restrict__ m, float* __restrict__ v, int64_t i, float lr,
                                             float b1, float omb1, float b2, float omb2, float eps, float wd,
                                             float bias1, float bias2) {
#pragma clang fp contract(off)
  float gi = grad[i];
  const float pi = p[i];
  if (wd > 0.f) gi = gi + wd * pi;
  const float mi = __builtin_fmaf(omb1, gi, m[i] * b1);
  const float vi = v[i] * b2 + (omb2 * gi) * gi;
  m[i] = mi;
  v[i] = vi;
  const float upd = (mi / bias1) / (sqrtf(vi / bias2) + eps);
  p[i] = pi + (-lr) * upd;
}

__global__ __launch_bounds__(256) void sparse_adam_kernel(float* __restrict__ p, const float* __restrict__ grad,
                                                          float* __restrict__ m, float* __restrict__ v, int64_t n,
                                                          float lr, float b1, float omb1, float b2, float omb2,
                                                          float eps, float wd, float bias1, float bias2) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    adam_element(p, grad, m, v, i, lr, b1, omb1, b2, omb2, eps, wd, bias1, bias2);
}

// The same step gated on the device: skipped unless finite[0] != 0 and
// halt[0] == 0 (the trainer's finite gate, train.py:649-672, decided without a
// host read); the step number is count[0] + 1 (count = steps applied so far,
// advanced by count_step_kernel after the step's launches) and its bias
// corrections come from the host-computed table bias[2 (t - 1) + {0, 1}].
__global__ __launch_bounds__(256) void sparse_adam_gated_kernel(
    float* __restrict__ p, const float* __restrict__ grad, float* __restrict__ m, float* __restrict__ v, int64_t n,
    float lr, float b1, float omb1, float b2, float omb2, float eps, float wd, const int32_t* __restrict__ finite,
    const int32_t* __restrict__ halt, const int32_t* __restrict__ count, const float* __restrict__ bias,
    int64_t bias_steps, int32_t* __restrict__ bad) {
  if ((finite && *finite == 0) || (halt && *halt != 0)) return;
  const int64_t t = (int64_t)count[0] + 1;
  if (t < 1 || t > bias_steps) {
    if (bad && blockIdx.x == 0 && threadIdx.x == 0) bad[0] = 1;
    return;
  }
  const float bias1 = bias[2 * (t - 1)], bias2 = bias[2 * (t - 1) + 1];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    adam_element(p, grad, m, v, i, lr, b1, omb1, b2, omb2, eps, wd, bias1, bias2);
}

// count[0] += 1 when the step's gate is open (one thread).
__global__ void count_step_kernel(const int32_t* __restrict__ finite, const int32_t* __restrict__ halt,
                                  int32_t* __restrict__ count) {
  if ((finite && *finite == 0) || (halt && *halt != 0)) return;
  count[0] = count[0] + 1;
}

// torch.optim.SGD's single-tensor step with momentum (dampening 0, no Nesterov)
// for the router weight (train.py:493-498, 667-672), in one pass:
//   d = grad + wd * p; buf = d (first step) or buf * momentum + d; p = p - lr * buf
// with torch's per-op rounding to the tensor dtype: each `a + alpha * b` is one
// fp32 fused multiply-add, rounded once; mul_ multiplies by the fp32 factor and
// rounds before the add.
template <int DT>
__global__ __launch_bounds__(256) void sgd_momentum_kernel(void* __restrict__ p, const void* __restrict__ grad,
                                                           void* __restrict__ buf, int64_t n, float lr,
                                                           float momentum, float wd, int first,
                                                           const int32_t* __restrict__ finite,
                                                           const int32_t* __restrict__ halt,
                                                           const int32_t* __restrict__ scale_state, float accum) {
#pragma clang fp contract(off)
  // the step's gate, read on the device (no host read): skipped unless the
  // finite flag is set and the halt flag is clear
  if ((finite && *finite == 0) || (halt && *halt != 0)) return;
  // the loss-scaled gradient is first divided by loss_scale * ACCUM and rounded
  // to the dtype (train.py:669-670 grad.div_); the gradient buffer is not written
  const float denom = scale_state ? __int_as_float(scale_state[0]) * accum : 1.f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  // Each fp32 result is pinned (asm) before its conversion: otherwise the
  // compiler folds product-then-fp16 into v_fma_mix, which rounds once from the
  // exact product instead of rounding to fp32 first as torch's kernels do.
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float pf = load_as_f32<DT>(p, i);
    float g = load_as_f32<DT>(grad, i);
    if (scale_state) {
      float gs = g / denom;
      asm volatile("" : "+v"(gs));
      g = round_to<DT>(gs);
    }
    float d32 = __builtin_fmaf(wd, pf, g);
    asm volatile("" : "+v"(d32));
    const float d = round_to<DT>(d32);
    float b;
    if (first) {
      b = d;
    } else {
      float bm32 = load_as_f32<DT>(buf, i) * momentum;
      asm volatile("" : "+v"(bm32));
      float b32 = round_to<DT>(bm32) + d;
      asm volatile("" : "+v"(b32));
      b = round_to<DT>(b32);
    }
    store_from_f32<DT>(buf, i, b);
    float p32 = __builtin_fmaf(-lr, b, pf);
    asm volatile("" : "+v"(p32));
    store_from_f32<DT>(p, i, p32);
  }
}

__global__ __launch_bounds__(256) void scale_check_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                          int64_t n, float denom, int32_t* __restrict__ finite) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  bool ok = true;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = in[i] / denom;
    out[i] = v;
    ok = ok && isfinite(v);
  }
  if (!ok) finite[0] = 0;  // benign race: every writer stores the same value
}

// ---- dynamic loss scale with its state on the device ------------------------------
// The trainer's loss scaling (train.py:31, 351-353, 661-677) for loops that launch
// step n + 1 before the host has read step n's finite flag.  State, int32[4]:
//   [0] the loss scale (fp32 bits), [1] good steps (train.py's good_streak, never
//   reset by a skipped step), [2] skipped steps, [3] unused.
__device__ __forceinline__ float loss_scale_of(const int32_t* state) { return __int_as_float(state[0]); }

// out = DT(x * scale): the gradient seed of the scaled loss.  VEC: 8 elements per
// 16-byte vector (n % 8 == 0, both bases 16-byte aligned).
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void loss_scale_mul_kernel(const uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ out, int64_t n,
                                                             const int32_t* __restrict__ state) {
  const float sc = loss_scale_of(state);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if constexpr (VEC) {
    const int64_t nv = n / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
      const uint4 a = reinterpret_cast<const uint4*>(x)[i];
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x2 v = unpack2<DT>(w[q]);
        o[q] = pack2<DT>(v.x * sc, v.y * sc);
      }
      reinterpret_cast<uint4*>(out)[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
      store_from_f32<DT>(out, i, load_as_f32<DT>(x, i) * sc);
  }
}

// out = in / (scale * accum) and finite[0] = 0 if any result is inf/NaN
// (train.py:661-663 with denom = loss_scale * ACCUM read from the state).
__global__ __launch_bounds__(256) void scale_check_state_kernel(const float* __restrict__ in,
                                                                float* __restrict__ out, int64_t n,
                                                                const int32_t* __restrict__ state, float accum,
                                                                int32_t* __restrict__ finite) {
  const float denom = loss_scale_of(state) * accum;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  bool ok = true;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = in[i] / denom;
    out[i] = v;
    ok = ok && isfinite(v);
  }
  if (!ok) finite[0] = 0;  // benign race: every writer stores the same value
}

// The schedule of train.py:673-677, one thread, after the step's gated updates:
// a finite step counts as good and doubles the scale on every `every`-th good
// step (capped at hi); a non-finite one counts as skipped and halves it (floored
// at lo).  A halted step (halt[0] != 0) changes nothing.
__global__ void loss_scale_update_kernel(int32_t* __restrict__ state, const int32_t* __restrict__ finite,
                                         const int32_t* __restrict__ halt, int32_t every, float lo, float hi) {
  if (halt && *halt != 0) return;
  float sc = loss_scale_of(state);
  if (!finite || *finite != 0) {
    const int32_t good = state[1] + 1;
    state[1] = good;
    if (good % every == 0) sc = fminf(sc * 2.f, hi);
  } else {
    state[2] = state[2] + 1;
    sc = fmaxf(sc * 0.5f, lo);
  }
  state[0] = __float_as_int(sc);
}

template <int DT>
__global__ __launch_bounds__(256) void overlay_scatter_kernel(uint16_t* __restrict__ base, int64_t numel,
                                                              const int64_t* __restrict__ idx,
                                                              const float* __restrict__ vals, int64_t n,
                                                              int32_t* __restrict__ bad) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) {
    const int64_t k = idx[j];
    if (k < 0 || k >= numel) {
      bad[0] = 1;
      continue;
    }
    store_from_f32<DT>(base, k, vals[j]);
  }
}

// Trained values into the overlay entries of the fused 4-bit GEMMs: entry word
// wa[j] of table ta takes DT(fp16(p[ia[j]])) in its high half (likewise wb, ib,
// tb) -- the reference's fp16 weight after the overlay scatter
// (moe_loader.py:218-221), then the activation dtype, as the GEMMs convert every
// dequantized weight.  The caller orders j by word, so that neighbouring
// threads write neighbouring words and each cache line of a table is written
// by one burst; ia / ib NULL read p[j].  Words outside a table or indices
// outside [0, n) set *bad and are skipped.
template <int DT>
__device__ __forceinline__ void overlay_put(const float* __restrict__ p, int64_t n, int64_t j,
                                            const int32_t* __restrict__ w, const int32_t* __restrict__ idx,
                                            uint16_t* __restrict__ t, int64_t nw, int32_t* __restrict__ bad) {
  const int64_t i = idx ? (int64_t)idx[j] : j;
  const int64_t wd = w[j];
  if (i < 0 || i >= n || wd < 0 || wd >= nw) {
    if (bad) bad[0] = 1;
    return;
  }
  const uint16_t h = f32_to_f16_bits(p[i]);
  t[2 * wd + 1] = DT == USAF_F16 ? h : f32_to_bf16_bits(f16_bits_to_f32(h));
}

template <int DT>
__global__ __launch_bounds__(256) void overlay_refresh_kernel(const float* __restrict__ p, int64_t n,
                                                              const int32_t* __restrict__ wa,
                                                              const int32_t* __restrict__ ia, uint16_t* __restrict__ ta,
                                                              int64_t na, const int32_t* __restrict__ wb,
                                                              const int32_t* __restrict__ ib, uint16_t* __restrict__ tb,
                                                              int64_t nb, int32_t* __restrict__ bad) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) {
    if (ta) overlay_put<DT>(p, n, j, wa, ia, ta, na, bad);
    if (tb) overlay_put<DT>(p, n, j, wb, ib, tb, nb, bad);
  }
}

int grid_for(int64_t n, int per_cu = 8) {
  int64_t b = (n + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  if (b > cap) b = cap;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace
}  // namespace usaf

using namespace usaf;

namespace {
// Blocks of 256 threads of `kernel` that stay resident on one CU (at least 1).
// The position-list kernels launch exactly that many per CU: a second round of
// blocks would walk the per-die slices of the list again from the start and
// fetch every expert's operands into L2 a second time.
int resident_blocks_per_cu(const void* kernel) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 1;
  }
  return n;
}

// Resident blocks per CU of the four sampled-gradient kernel instantiations,
// queried once per process (a function-local static: C++11 runs its
// initializer exactly once, also under concurrent first calls).
struct SddmmOccupancy {
  int masked_bf16, masked_f16, blocked_bf16, blocked_f16;
};
const SddmmOccupancy& sddmm_occupancy() {
  static const SddmmOccupancy occ = {
      resident_blocks_per_cu(reinterpret_cast<const void*>(&sddmm_kernel<USAF_BF16>)),
      resident_blocks_per_cu(reinterpret_cast<const void*>(&sddmm_kernel<USAF_F16>)),
      resident_blocks_per_cu(reinterpret_cast<const void*>(&sddmm_blocked_kernel<USAF_BF16>)),
      resident_blocks_per_cu(reinterpret_cast<const void*>(&sddmm_blocked_kernel<USAF_F16>))};
  return occ;
}
}  // namespace

void usaf::prepare_sparse_kernels() { (void)sddmm_occupancy(); }

extern "C" int usaf_hip_gather_transpose(const void* in, int64_t ld_in, const int32_t* rows, int64_t S, int64_t C,
                                         void* out, int64_t ld_out, void* stream) {
  if (S < 0 || C < 0 || ld_in < C || ld_out < S) return set_error(USAF_ERR_INVALID, "gather_transpose: bad sizes");
  if (S == 0 || C == 0) return clear_error();
  if (!in || !out) return set_error(USAF_ERR_INVALID, "gather_transpose: null pointer");
  const int64_t gx = (S + 63) / 64, gy = (C + 63) / 64;
  if (gx > 0x7fffffff || gy > 65535) return set_error(USAF_ERR_INVALID, "gather_transpose: too large");
  const bool vec = C % 8 == 0 && ld_in % 8 == 0 && ld_out % 8 == 0 && ((uintptr_t)in & 15) == 0 &&
                   ((uintptr_t)out & 15) == 0;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  if (vec)
    gather_transpose_kernel<true><<<grid, 256, 0, as_stream(stream)>>>((const uint16_t*)in, ld_in, rows, S, C,
                                                                       (uint16_t*)out, ld_out);
  else
    gather_transpose_kernel<false><<<grid, 256, 0, as_stream(stream)>>>((const uint16_t*)in, ld_in, rows, S, C,
                                                                        (uint16_t*)out, ld_out);
  return check_launch("gather_transpose");
}

extern "C" int usaf_hip_sddmm_masked(const void* rowT, const void* colT, int64_t ldT, const int32_t* offsets,
                                     int64_t E, int64_t R, int64_t C, int64_t n_pos, const int32_t* row_code,
                                     const int32_t* col_idx, const int64_t* pos_map, int32_t dtype, float* compact,
                                     void* stream) {
  if (E <= 0 || R <= 0 || C <= 0 || n_pos < 0 || ldT < 0) return set_error(USAF_ERR_INVALID, "sddmm_masked: bad sizes");
  if (E > 1024 || R >= (1 << 21) || C > 0x7fffffff || ldT > 0x7fffffff)
    return set_error(USAF_ERR_INVALID, "sddmm_masked: needs E <= 1024, R < 2^21, C and ldT < 2^31");
  if (ldT % 8 != 0) return set_error(USAF_ERR_INVALID, "sddmm_masked: ldT must be a multiple of 8");
  if (n_pos == 0) return clear_error();
  if (!rowT || !colT || !offsets || !row_code || !col_idx || !compact)
    return set_error(USAF_ERR_INVALID, "sddmm_masked: null pointer");
  if (((uintptr_t)rowT & 15) || ((uintptr_t)colT & 15))
    return set_error(USAF_ERR_INVALID, "sddmm_masked: rowT and colT must be 16-byte aligned");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "sddmm_masked: dtype must be 16-bit");
  const SddmmOccupancy& occ = sddmm_occupancy();
  int64_t blocks = (n_pos + 15) / 16;
  const int64_t cap = (int64_t)device_cu_count() * (dtype == USAF_BF16 ? occ.masked_bf16 : occ.masked_f16);
  if (blocks > cap) blocks = cap;
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_BF16)
    sddmm_kernel<USAF_BF16><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)rowT, (const uint16_t*)colT, ldT,
                                                              offsets, (int32_t)E, (int32_t)R, (int32_t)C, n_pos,
                                                              row_code, col_idx, pos_map, compact);
  else
    sddmm_kernel<USAF_F16><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)rowT, (const uint16_t*)colT, ldT,
                                                             offsets, (int32_t)E, (int32_t)R, (int32_t)C, n_pos,
                                                             row_code, col_idx, pos_map, compact);
  return check_launch("sddmm_masked");
}

extern "C" int64_t usaf_hip_blocked_elems(int64_t S, int64_t E, int64_t C) { return C * (S + (BLK_PAD - 1) * E); }

extern "C" int64_t usaf_hip_blocked_table_elems(int64_t S, int64_t E) { return 2 * (E + 1) + blk_chunk_bound(S, E); }

extern "C" int usaf_hip_blocked_layout(const int32_t* offsets, int64_t E, int64_t S, int32_t* table, void* stream) {
  if (E <= 0 || E > BLK_MAX_E) return set_error(USAF_ERR_INVALID, "blocked_layout: needs 0 < E <= %d", BLK_MAX_E);
  if (S < 0 || blk_chunk_bound(S, E) > 0x7fffffff) return set_error(USAF_ERR_INVALID, "blocked_layout: bad S");
  if (!offsets || !table) return set_error(USAF_ERR_INVALID, "blocked_layout: null pointer");
  blocked_layout_kernel<<<1, 256, 0, as_stream(stream)>>>(offsets, (int)E, table, S, blk_chunk_bound(S, E));
  return check_launch("blocked_layout");
}

extern "C" int usaf_hip_gather_transpose_blocked(const void* in, int64_t ld_in, const int32_t* rows,
                                                 const int32_t* offsets, const int32_t* table, int64_t S, int64_t E,
                                                 int64_t C, void* out, void* stream) {
  if (S < 0 || C < 0 || E <= 0 || ld_in < C) return set_error(USAF_ERR_INVALID, "gather_transpose_blocked: bad sizes");
  if (E > BLK_MAX_E) return set_error(USAF_ERR_UNSUPPORTED, "gather_transpose_blocked: needs E <= %d", BLK_MAX_E);
  if (S == 0 || C == 0) return clear_error();
  if (!in || !out || !offsets || !table) return set_error(USAF_ERR_INVALID, "gather_transpose_blocked: null pointer");
  if (C % 8 != 0 || ld_in % 8 != 0 || ((uintptr_t)in & 15) || ((uintptr_t)out & 15))
    return set_error(USAF_ERR_UNSUPPORTED, "gather_transpose_blocked: needs C, ld_in %% 8 == 0 and 16-byte aligned bases");
  const int64_t gx = blk_chunk_bound(S, E), gy = (C + 64 * GT_TILES - 1) / (64 * GT_TILES);
  if (gx > 0x7fffffff || gy > 65535) return set_error(USAF_ERR_INVALID, "gather_transpose_blocked: too large");
  gather_transpose_blocked_kernel<<<dim3((unsigned)gx, (unsigned)gy), 256, 0, as_stream(stream)>>>(
      (const uint16_t*)in, ld_in, rows, offsets, table, (int)E, C, (uint16_t*)out);
  return check_launch("gather_transpose_blocked");
}

extern "C" int64_t usaf_hip_combine_bwd_blocked_ws_floats(int64_t S, int64_t H) {
  if (S < 0 || H <= 0) return -1;
  return ((H + 511) / 512) * S;
}

extern "C" int usaf_hip_moe_combine_bwd_blocked(const void* dout, const void* y_slots, const int32_t* token_idx,
                                                const float* slot_w, const int32_t* offsets, const int32_t* table,
                                                int64_t S, int64_t E, int64_t H, int32_t dtype, void* dcur,
                                                void* dcur_blk, void* dweights, float* workspace, void* stream) {
  if (S < 0 || E <= 0 || H <= 0) return set_error(USAF_ERR_INVALID, "moe_combine_bwd_blocked: bad sizes");
  if (E > BLK_MAX_E) return set_error(USAF_ERR_UNSUPPORTED, "moe_combine_bwd_blocked: needs E <= %d", BLK_MAX_E);
  if (dtype != USAF_F16 && dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "moe_combine_bwd_blocked: dtype must be fp16/bf16");
  if (S == 0) return clear_error();
  if (!dout || !y_slots || !token_idx || !slot_w || !offsets || !table || !dcur || !dcur_blk || !dweights || !workspace)
    return set_error(USAF_ERR_INVALID, "moe_combine_bwd_blocked: null pointer");
  if (H % 8 != 0 || (((uintptr_t)dout | (uintptr_t)y_slots | (uintptr_t)dcur | (uintptr_t)dcur_blk) & 15))
    return set_error(USAF_ERR_UNSUPPORTED, "moe_combine_bwd_blocked: needs H %% 8 == 0 and 16-byte aligned buffers");
  const int64_t gx = blk_chunk_bound(S, E), gy = (H + 511) / 512;
  if (gx > 0x7fffffff || gy > 65535 || S > 0x7fffffff)
    return set_error(USAF_ERR_INVALID, "moe_combine_bwd_blocked: too large");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)gx, (unsigned)gy);
  const unsigned fin = (unsigned)((S + 255) / 256);
  if (dtype == USAF_BF16) {
    combine_bwd_blocked_kernel<USAF_BF16><<<grid, 256, 0, st>>>(
        (const uint16_t*)dout, (const uint16_t*)y_slots, token_idx, slot_w, offsets, table, (int)E, H, S,
        (uint16_t*)dcur, (uint16_t*)dcur_blk, workspace);
    combine_bwd_finish_kernel<USAF_BF16><<<fin, 256, 0, st>>>(workspace, (int)gy, S, token_idx, offsets, (int)E,
                                                              dweights);
  } else {
    combine_bwd_blocked_kernel<USAF_F16><<<grid, 256, 0, st>>>(
        (const uint16_t*)dout, (const uint16_t*)y_slots, token_idx, slot_w, offsets, table, (int)E, H, S,
        (uint16_t*)dcur, (uint16_t*)dcur_blk, workspace);
    combine_bwd_finish_kernel<USAF_F16><<<fin, 256, 0, st>>>(workspace, (int)gy, S, token_idx, offsets, (int)E,
                                                             dweights);
  }
  return check_launch("moe_combine_bwd_blocked");
}

extern "C" int usaf_hip_sddmm_blocked(const void* row_blk, const void* col_blk, const int32_t* table, int64_t E,
                                      int64_t R, int64_t C, int64_t n_pos, const int32_t* row_code,
                                      const int32_t* col_idx, const int64_t* pos_map, int32_t dtype, float* compact,
                                      int32_t accumulate, void* stream) {
  if (E <= 0 || R <= 0 || C <= 0 || n_pos < 0) return set_error(USAF_ERR_INVALID, "sddmm_blocked: bad sizes");
  if (E > BLK_MAX_E || R >= (1 << 21) || C > 0x7fffffff)
    return set_error(USAF_ERR_INVALID, "sddmm_blocked: needs E <= %d, R < 2^21, C < 2^31", BLK_MAX_E);
  if (n_pos == 0) return clear_error();
  if (!row_blk || !col_blk || !table || !row_code || !col_idx || !compact)
    return set_error(USAF_ERR_INVALID, "sddmm_blocked: null pointer");
  if (((uintptr_t)row_blk & 15) || ((uintptr_t)col_blk & 15))
    return set_error(USAF_ERR_INVALID, "sddmm_blocked: operands must be 16-byte aligned");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "sddmm_blocked: dtype must be 16-bit");
  const SddmmOccupancy& occ = sddmm_occupancy();
  int64_t blocks = (n_pos + 15) / 16;
  const int64_t cap = (int64_t)device_cu_count() * (dtype == USAF_BF16 ? occ.blocked_bf16 : occ.blocked_f16);
  if (blocks > cap) blocks = cap;
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_BF16)
    sddmm_blocked_kernel<USAF_BF16><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)row_blk, (const uint16_t*)col_blk,
                                                                      table, (int32_t)E, (int32_t)R, (int32_t)C, n_pos,
                                                                      row_code, col_idx, pos_map, compact,
                                                                      accumulate ? 1 : 0);
  else
    sddmm_blocked_kernel<USAF_F16><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)row_blk, (const uint16_t*)col_blk,
                                                                     table, (int32_t)E, (int32_t)R, (int32_t)C, n_pos,
                                                                     row_code, col_idx, pos_map, compact,
                                                                     accumulate ? 1 : 0);
  return check_launch("sddmm_blocked");
}

extern "C" int usaf_hip_sparse_adam_step(float* p, const float* grad, float* m, float* v, int64_t n, double lr,
                                         double beta1, double beta2, double eps, double weight_decay, int64_t step,
                                         void* stream) {
  if (n < 0 || step <= 0) return set_error(USAF_ERR_INVALID, "sparse_adam_step: need n >= 0 and step >= 1");
  if (n == 0) return clear_error();
  if (!p || !grad || !m || !v) return set_error(USAF_ERR_INVALID, "sparse_adam_step: null pointer");
  // Python-float (double) scalars of the reference, used by fp32 tensor ops as fp32
  const float bias1 = (float)(1.0 - pow(beta1, (double)step));
  const float bias2 = (float)(1.0 - pow(beta2, (double)step));
  sparse_adam_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(
      p, grad, m, v, n, (float)lr, (float)beta1, (float)(1.0 - beta1), (float)beta2, (float)(1.0 - beta2),
      (float)eps, (float)weight_decay, bias1, bias2);
  return check_launch("sparse_adam_step");
}

extern "C" int usaf_hip_sparse_adam_step_gated(float* p, const float* grad, float* m, float* v, int64_t n,
                                               double lr, double beta1, double beta2, double eps,
                                               double weight_decay, const int32_t* finite, const int32_t* halt,
                                               const int32_t* step_count, const float* bias_table,
                                               int64_t table_steps, int32_t* bad_flag, void* stream) {
  if (n < 0 || table_steps < 0) return set_error(USAF_ERR_INVALID, "sparse_adam_step_gated: negative size");
  if (n == 0) return clear_error();
  if (!p || !grad || !m || !v || !step_count || !bias_table)
    return set_error(USAF_ERR_INVALID, "sparse_adam_step_gated: null pointer");
  sparse_adam_gated_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(
      p, grad, m, v, n, (float)lr, (float)beta1, (float)(1.0 - beta1), (float)beta2, (float)(1.0 - beta2),
      (float)eps, (float)weight_decay, finite, halt, step_count, bias_table, table_steps, bad_flag);
  return check_launch("sparse_adam_step_gated");
}

extern "C" int usaf_hip_count_step(const int32_t* finite, const int32_t* halt, int32_t* step_count, void* stream) {
  if (!step_count) return set_error(USAF_ERR_INVALID, "count_step: null pointer");
  count_step_kernel<<<1, 1, 0, as_stream(stream)>>>(finite, halt, step_count);
  return check_launch("count_step");
}

extern "C" int usaf_hip_sgd_momentum_step(void* p, const void* grad, void* momentum_buf, int64_t n, int32_t dtype,
                                          double lr, double momentum, double weight_decay, int32_t first_step,
                                          const int32_t* finite, const int32_t* halt, const int32_t* scale_state,
                                          double accum, void* stream) {
  if (n < 0) return set_error(USAF_ERR_INVALID, "sgd_momentum_step: negative n");
  if (first_step && (finite || halt))
    return set_error(USAF_ERR_INVALID, "sgd_momentum_step: the first step (momentum buffer = d) cannot be gated");
  if (scale_state && !(accum >= 1.0)) return set_error(USAF_ERR_INVALID, "sgd_momentum_step: accum must be >= 1");
  if (n == 0) return clear_error();
  if (!p || !grad || !momentum_buf) return set_error(USAF_ERR_INVALID, "sgd_momentum_step: null pointer");
  hipStream_t st = as_stream(stream);
  const float lr_f = (float)lr, m_f = (float)momentum, wd_f = (float)weight_decay;
  const int first = first_step ? 1 : 0;
  switch (dtype) {
    case USAF_F32:
      sgd_momentum_kernel<USAF_F32><<<grid_for(n), 256, 0, st>>>(p, grad, momentum_buf, n, lr_f, m_f, wd_f, first,
                                                                                  finite, halt, scale_state,
                                                                                  (float)accum);
      break;
    case USAF_F16:
      sgd_momentum_kernel<USAF_F16><<<grid_for(n), 256, 0, st>>>(p, grad, momentum_buf, n, lr_f, m_f, wd_f, first,
                                                                                  finite, halt, scale_state,
                                                                                  (float)accum);
      break;
    case USAF_BF16:
      sgd_momentum_kernel<USAF_BF16><<<grid_for(n), 256, 0, st>>>(p, grad, momentum_buf, n, lr_f, m_f, wd_f, first,
                                                                                  finite, halt, scale_state,
                                                                                  (float)accum);
      break;
    default:
      return set_error(USAF_ERR_INVALID, "sgd_momentum_step: dtype must be fp32, fp16 or bf16");
  }
  return check_launch("sgd_momentum_step");
}

extern "C" int usaf_hip_scale_check(const float* in, float* out, int64_t n, float denom, int32_t* finite_flag,
                                    void* stream) {
  if (n < 0) return set_error(USAF_ERR_INVALID, "scale_check: negative n");
  if (n == 0) return clear_error();
  if (!in || !out || !finite_flag) return set_error(USAF_ERR_INVALID, "scale_check: null pointer");
  scale_check_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(in, out, n, denom, finite_flag);
  return check_launch("scale_check");
}

extern "C" int usaf_hip_loss_scale_apply(const void* x, void* out, int64_t n, int32_t dtype,
                                         const int32_t* scale_state, void* stream) {
  if (n < 0) return set_error(USAF_ERR_INVALID, "loss_scale_apply: negative n");
  if (dtype != USAF_F16 && dtype != USAF_BF16)
    return set_error(USAF_ERR_INVALID, "loss_scale_apply: dtype must be fp16 or bf16");
  if (n == 0) return clear_error();
  if (!x || !out || !scale_state) return set_error(USAF_ERR_INVALID, "loss_scale_apply: null pointer");
  hipStream_t st = as_stream(stream);
  const bool vec = n % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0;
  const uint16_t* xi = static_cast<const uint16_t*>(x);
  uint16_t* oi = static_cast<uint16_t*>(out);
  if (dtype == USAF_BF16) {
    if (vec) loss_scale_mul_kernel<USAF_BF16, true><<<grid_for(n / 8), 256, 0, st>>>(xi, oi, n, scale_state);
    else loss_scale_mul_kernel<USAF_BF16, false><<<grid_for(n), 256, 0, st>>>(xi, oi, n, scale_state);
  } else {
    if (vec) loss_scale_mul_kernel<USAF_F16, true><<<grid_for(n / 8), 256, 0, st>>>(xi, oi, n, scale_state);
    else loss_scale_mul_kernel<USAF_F16, false><<<grid_for(n), 256, 0, st>>>(xi, oi, n, scale_state);
  }
  return check_launch("loss_scale_apply");
}

extern "C" int usaf_hip_scale_check_state(const float* in, float* out, int64_t n, const int32_t* scale_state,
                                          double accum, int32_t* finite_flag, void* stream) {
  if (n < 0) return set_error(USAF_ERR_INVALID, "scale_check_state: negative n");
  if (!(accum >= 1.0)) return set_error(USAF_ERR_INVALID, "scale_check_state: accum must be >= 1");
  if (n == 0) return clear_error();
  if (!in || !out || !scale_state || !finite_flag)
    return set_error(USAF_ERR_INVALID, "scale_check_state: null pointer");
  scale_check_state_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(in, out, n, scale_state, (float)accum,
                                                                       finite_flag);
  return check_launch("scale_check_state");
}

extern "C" int usaf_hip_loss_scale_update(int32_t* scale_state, const int32_t* finite, const int32_t* halt,
                                          int32_t scale_up_every, double min_scale, double max_scale, void* stream) {
  if (!scale_state) return set_error(USAF_ERR_INVALID, "loss_scale_update: null pointer");
  if (scale_up_every < 1 || !(min_scale > 0.0) || !(max_scale >= min_scale))
    return set_error(USAF_ERR_INVALID, "loss_scale_update: need scale_up_every >= 1 and 0 < min_scale <= max_scale");
  loss_scale_update_kernel<<<1, 1, 0, as_stream(stream)>>>(scale_state, finite, halt, scale_up_every,
                                                           (float)min_scale, (float)max_scale);
  return check_launch("loss_scale_update");
}

extern "C" int usaf_hip_overlay_refresh(const float* p, int64_t n, const int32_t* words_a, const int32_t* index_a,
                                        uint32_t* table_a, int64_t n_words_a, const int32_t* words_b,
                                        const int32_t* index_b, uint32_t* table_b, int64_t n_words_b, int32_t dtype,
                                        int32_t* bad_flag, void* stream) {
  if (n < 0 || n_words_a < 0 || n_words_b < 0) return set_error(USAF_ERR_INVALID, "overlay_refresh: negative size");
  if (n == 0) return clear_error();
  if (!p || (table_a && !words_a) || (table_b && !words_b))
    return set_error(USAF_ERR_INVALID, "overlay_refresh: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_F16)
    overlay_refresh_kernel<USAF_F16><<<grid_for(n), 256, 0, st>>>(p, n, words_a, index_a, (uint16_t*)table_a, n_words_a,
                                                                   words_b, index_b, (uint16_t*)table_b, n_words_b,
                                                                   bad_flag);
  else if (dtype == USAF_BF16)
    overlay_refresh_kernel<USAF_BF16><<<grid_for(n), 256, 0, st>>>(p, n, words_a, index_a, (uint16_t*)table_a,
                                                                    n_words_a, words_b, index_b, (uint16_t*)table_b,
                                                                    n_words_b, bad_flag);
  else
    return set_error(USAF_ERR_INVALID, "overlay_refresh: dtype must be fp16 or bf16");
  return check_launch("overlay_refresh");
}

extern "C" int usaf_hip_overlay_scatter(void* base, int32_t dtype, int64_t numel, const int64_t* idx,
                                        const float* vals, int64_t n, int32_t* bad_flag, void* stream) {
  if (n < 0 || numel < 0) return set_error(USAF_ERR_INVALID, "overlay_scatter: negative size");
  if (n == 0) return clear_error();
  if (!base || !idx || !vals || !bad_flag) return set_error(USAF_ERR_INVALID, "overlay_scatter: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_F16)
    overlay_scatter_kernel<USAF_F16><<<grid_for(n), 256, 0, st>>>((uint16_t*)base, numel, idx, vals, n, bad_flag);
  else if (dtype == USAF_BF16)
    overlay_scatter_kernel<USAF_BF16><<<grid_for(n), 256, 0, st>>>((uint16_t*)base, numel, idx, vals, n, bad_flag);
  else
    return set_error(USAF_ERR_INVALID, "overlay_scatter: dtype must be fp16 or bf16");
  return check_launch("overlay_scatter");
}
