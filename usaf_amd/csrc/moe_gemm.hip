// Grouped (per-expert) GEMM with 4-bit weights dequantized on the fly, on
// gfx950 MFMA (v_mfma_f32_32x32x16_{bf16,f16}).
//
//   C[m, n] = sum_k A[row(m), k] * W_e[n, k]      (slots m of expert e)
//
// Slots are the token/expert pairs bucketed by expert (route.hip): expert e
// owns slots [offsets[e], offsets[e+1]).  The weight of expert e is the e-th
// [rows, cols] slice of a [E, rows, cols] tensor in the reference's 4-bit
// format (groups of 128 consecutive elements of a row, fp16 scale/zero).
// Each B tile is loaded as packed codes, dequantized in registers exactly as
// dequantize_4bit does (fp16(fp16(q*s)+z), then bf16 for bf16 activations)
// and staged in LDS; A tiles are gathered rows of the activations.
//
// The weight operand (BQ) is either 4-bit codes or a dense 16-bit tensor of
// the activation dtype (the reference's fp16 expert weights, e.g. resident
// copies with trained overlays).
// Weight layouts (BMODE):
//   NK  W_e is [N, K] with K contiguous (forward: x @ W^T, reference F.linear)
//   KN  W_e is [K, N] with N contiguous (backward grad-input: dY @ W)
// Epilogues (EPI):
//   STORE       out[m, n] = dtype(acc)
//   SWIGLU_FWD  tile columns pair gate row n with up row I+n of gate_up;
//               stores gu[m, n], gu[m, I+n] (pre-activation, dtype) and
//               act[m, n] = dtype(dtype(silu(g)) * u)  (qwen3moe_dml.py:58-60)
//   SWIGLU_BWD  acc = d(act); with the saved gu: d(up) = dtype(dact * silu(g)),
//               d(gate) = dtype(dtype(dact * u) * silu'(g)) -> dgu[m, n], dgu[m, I+n]
//
// Block: 512 threads, one block per CU, warp-specialised: 4 multiply waves
// (2 (M) x 2 (N) over the tile, LDS fragments -> MFMA only) and 4 producer
// waves (global loads, 4-bit dequant, LDS stores), one of each per SIMD, so
// the dequant and memory work overlaps the matrix cores instead of
// serialising with them in one instruction stream.
// Tile: up to BM = 320 slots of one expert x BN = 128 columns x BK = 64, so a
// typical expert (~256 routed tokens of 4096 x top-8 over 128 experts) is one
// m-tile and each dequantized weight tile feeds all of its tokens.  Each
// multiply wave owns 5 x 2 MFMA 32x32 accumulators (160 registers).  Two LDS
// stages (129 KB); the producers load two k-tiles ahead.
// The grid is persistent: tiles (expert m-tile x n-tile) come from a
// device-side list, walked per die so one expert's n-tiles share an L2; no
// host sync is needed.
#include "common.h"

#include <type_traits>

namespace usaf {
namespace {

// Tile: up to BM slots of one expert (10 MFMA row blocks of 32; empty blocks
// are skipped) x BN output columns x BK contraction per LDS stage.
constexpr int BM = 320, BN = 128, BK = 64;
constexpr int WM_SUB = BM / 32 / 2;    // 32-row blocks per M-wave (2 M-waves x 2 N-waves)
constexpr int kThreads = 512;                // 4 multiply waves + 4 producer waves
constexpr int A_CHUNKS = BM * BK / 8 / 256;  // 16-byte A chunks per producer thread per k-tile
constexpr int LDSW = BK + 8;  // LDS row stride in 16-bit elements (16 B pad: conflict-free 128-bit reads)
constexpr int LDSC = BN + 8; // epilogue tile row stride (16-bit elements)
constexpr int MAX_E = 1024;
constexpr int kXcds = 8;      // MI355X: 8 accelerator dies, blocks dispatched round-robin over them
constexpr size_t kSmemBytes = (size_t)2 * (BM + BN) * LDSW * 2 + (2 * (MAX_E + 1) + kThreads) * 4;

enum { BMODE_NK = 0, BMODE_KN = 1 };
enum { BQ_Q4 = 0, BQ_DENSE16 = 1 };
enum { EPI_STORE = 0, EPI_SWIGLU_FWD = 1, EPI_SWIGLU_BWD = 2 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

struct GemmArgs {
  const uint16_t* A;       // activations, 16-bit, row stride lda
  int64_t lda;
  const int32_t* a_rows;   // A row of slot m (nullptr: row m)
  const uint8_t* wq;       // packed codes of the whole [E, w_rows, w_cols] weight
  const uint32_t* wsz;     // per 128-element group: fp16 scale bits | fp16 zero bits << 16
  const uint16_t* w16;     // dense 16-bit weight [E, w_rows, w_cols] (BQ == BQ_DENSE16)
  const int32_t* w_slot;   // dense weights in an arena: expert e's [w_rows, w_cols] block is
  int64_t n_slots;         //   block w_slot[e] (clamped to [0, n_slots)) of w16; nullptr: block e
  int64_t w_rows, w_cols;  // per-expert weight matrix
  int64_t N, K;            // output columns, contraction length
  int64_t inter;           // I (SwiGLU epilogues)
  const int32_t* offsets;  // [E+1]
  int E;
  uint16_t* out;  int64_t ldo;   // STORE: C; SWIGLU_FWD: act; SWIGLU_BWD: dgu
  uint16_t* out2; int64_t ldo2;  // SWIGLU_FWD: gu
  const uint16_t* aux; int64_t ld_aux;  // SWIGLU_BWD: saved gu
  uint16_t* out_t;                // SWIGLU_FWD (4-bit DMA kernel): act also in the blocked slot-major
  const int32_t* blk_table;       //   layout of blk_table (usaf_hip_blocked_layout), or nullptr
  const uint32_t* ovl;            // 4-bit DMA kernel: overlay entries (usaf_hip_overlay_* layout), or nullptr
  int64_t ovl_words;              //   and their count (checked against what the GEMM reads)
  int w_frag;                     // dense weights (DW): 1 = each expert block in the GEMM's fragment order
  int64_t w_blk_elems;            //   (usaf_hip_dequant_q4_slices_frag) of w_blk_elems elements; 0: w_rows * w_cols
};

// Workgroup barrier ordering LDS accesses only.  __syncthreads() also orders
// global memory, which makes every wave drain its outstanding global loads
// (s_waitcnt vmcnt(0)) at each barrier and exposes the full memory latency of
// the prefetched k-steps; no thread here communicates through global memory.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block of the dense weight operand that holds expert e: e itself, or its
// arena slot (clamped, so a stale table can give wrong weights but never an
// access outside the arena).
__device__ __forceinline__ int64_t weight_block(const GemmArgs& g, int e) {
  if (g.w_slot == nullptr) return e;
  const int64_t s = g.w_slot[e];
  return s < 0 ? 0 : (s >= g.n_slots ? g.n_slots - 1 : s);
}

// ---- 4-bit -> 16-bit conversion (bit-identical to dequantize_4bit) ----------

__device__ __forceinline__ void dq_word(uint32_t w, f16x2 s2, f16x2 z2, uint32_t out[4]) {
#pragma clang fp contract(off)
  const f16x2 magic = {(f16)1024.0f, (f16)1024.0f};
  f16x2 p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t bits = ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
    const f16x2 q = __builtin_bit_cast(f16x2, bits) - magic;
    const f16x2 m = q * s2;
    p[i] = m + z2;
  }
  const uint32_t u0 = __builtin_bit_cast(uint32_t, p[0]), u1 = __builtin_bit_cast(uint32_t, p[1]);
  const uint32_t u2 = __builtin_bit_cast(uint32_t, p[2]), u3 = __builtin_bit_cast(uint32_t, p[3]);
  out[0] = (u0 & 0xFFFFu) | (u1 << 16);
  out[1] = (u2 & 0xFFFFu) | (u3 << 16);
  out[2] = (u0 >> 16) | (u1 & 0xFFFF0000u);
  out[3] = (u2 >> 16) | (u3 & 0xFFFF0000u);
}

__device__ __forceinline__ uint32_t h2_to_bf2(uint32_t h2) {
  const f16x2 h = __builtin_bit_cast(f16x2, h2);
  const f32x2 f = {(float)h.x, (float)h.y};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// 32 codes (16 bytes, one group) -> 32 16-bit operands in natural order.
template <int DT>
__device__ __forceinline__ void dequant32(const u32x4 w, uint16_t sb, uint16_t zb, uint32_t o[16]) {
  const f16 s = __builtin_bit_cast(f16, sb), z = __builtin_bit_cast(f16, zb);
  const f16x2 s2 = {s, s}, z2 = {z, z};
  dq_word(w.x, s2, z2, o + 0);
  dq_word(w.y, s2, z2, o + 4);
  dq_word(w.z, s2, z2, o + 8);
  dq_word(w.w, s2, z2, o + 12);
  if constexpr (DT == USAF_BF16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = h2_to_bf2(o[i]);
  }
}

// ---- small helpers -------------------------------------------------------------

// fp32 -> 16-bit bits of dtype DT (round to nearest even) and back.
template <int DT>
__device__ __forceinline__ uint16_t round_bits(float v) {
  if constexpr (DT == USAF_F16) return f32_to_f16_bits(v);
  else return f32_to_bf16_bits(v);
}
template <int DT>
__device__ __forceinline__ float bits_to_f32(uint16_t b) {
  if constexpr (DT == USAF_F16) return f16_bits_to_f32(b);
  else return bf16_bits_to_f32(b);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// silu(x) = x / (1 + e^-x) with the hardware exp2 and reciprocal (about 1 ulp
// of fp32 each, far below the 16-bit rounding that follows)
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

template <int DT>
__device__ __forceinline__ f32x16 mfma32(const u32x4 a, const u32x4 b, f32x16 c) {
  if constexpr (DT == USAF_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
}

// Weight row r of expert e (NK, SWIGLU_FWD): tile row b of n-tile nt pairs gate
// and up rows so that each wave holds 32 gate and the matching 32 up columns.
template <int EPI>
__device__ __forceinline__ int64_t nk_weight_row(int b, int64_t n0, int64_t inter) {
  if constexpr (EPI == EPI_SWIGLU_FWD) {
    const int wn = b >> 6, within = b & 63;
    return ((within >= 32) ? inter : 0) + n0 + wn * 32 + (within & 31);
  } else {
    return n0 + b;
  }
}

// ---- producer waves: global -> registers -> LDS, 4-bit B dequantized on the way ----
// Called by the 256 threads of waves 4-7 for one tile; executes exactly the
// barriers the multiply waves do (one after the prologue, one per k-tile, one
// after the accumulators are parked).
template <int BMODE, int EPI, int BQ, int DT>
__device__ __forceinline__ void produce_tile(const GemmArgs& g, uint16_t* sA0, uint16_t* sB0, const int ptid,
                                             const int e, const int64_t m_beg, const int valid, const int64_t n0,
                                             const int nk) {
  const int64_t w_base = weight_block(g, e) * g.w_rows * g.w_cols;  // element offset of expert e's weight
  // A: chunks c = ptid + 256*i (i < A_CHUNKS) of 16 B: row c>>3, 8-element k block c&7.
  // Rows past the expert's last slot re-read its first row into LDS rows that
  // are never used: loads and stores stay unconditional, which keeps the
  // producer loop one basic block and its memory waits precise.
  int32_t a_off[A_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = ptid + 256 * i;
    const int row = c >> 3;
    const int64_t m = m_beg + (row < valid ? row : 0);
    const int64_t arow = g.a_rows ? (int64_t)g.a_rows[m] : m;
    a_off[i] = (int32_t)(arow * g.lda + (c & 7) * 8);
  }
  // B (4-bit NK): 16 code bytes (32 elements of one group) of tile row ptid>>1.
  // B (4-bit KN): 4 contraction rows 4*(ptid&15)+r, 8 columns 8*(ptid>>4): one code word per row.
  // B (dense NK): 4 chunks of 8 elements; (dense KN): 4 rows x 8 columns.
  int64_t b_off[4] = {0, 0, 0, 0};
  int64_t b_kstep;
  if constexpr (BMODE == BMODE_NK) {
    b_kstep = BK;
    if constexpr (BQ == BQ_Q4) {
      b_off[0] = w_base + nk_weight_row<EPI>(ptid >> 1, n0, g.inter) * g.w_cols + (ptid & 1) * 32;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = ptid + 256 * i;
        b_off[i] = w_base + nk_weight_row<EPI>(c >> 3, n0, g.inter) * g.w_cols + (c & 7) * 8;
      }
    }
  } else {
    b_kstep = (int64_t)BK * g.w_cols;
    const int kb = ptid & 15, nb = ptid >> 4;
    b_off[0] = w_base + (int64_t)(4 * kb) * g.w_cols + n0 + nb * 8;  // row r adds r * w_cols
  }

  // Register ring: tile kt lives in slot kt % RING; with RING = 3 loads are
  // issued two k-tiles before their LDS store, covering L2/HBM latency (the
  // dense-weight and transposed-weight variants need more registers per tile
  // and use RING = 2).
  constexpr int RING = (BQ == BQ_Q4 && BMODE == BMODE_NK) ? 3 : 2;
  u32x4 ra[RING][A_CHUNKS];
  u32x4 rb4[RING][(BQ == BQ_Q4) ? 1 : 4];
  uint32_t rw[RING][4];
  uint32_t rsz[RING][4];  // scale | zero << 16 of each row's group
  auto load_tile = [&](auto slot_c, int kt) {
    constexpr int S = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) ra[S][i] = *reinterpret_cast<const u32x4*>(g.A + a_off[i] + kt * BK);
    const int64_t ks = (int64_t)kt * b_kstep;
    if constexpr (BQ == BQ_Q4) {
      if constexpr (BMODE == BMODE_NK) {
        const int64_t el = b_off[0] + ks;
        rb4[S][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g.wq + (el >> 1)));
        rsz[S][0] = g.wsz[el >> 7];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t el = b_off[0] + r * g.w_cols + ks;
          rw[S][r] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(g.wq + (el >> 1)));
          rsz[S][r] = g.wsz[el >> 7];
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t off = (BMODE == BMODE_NK) ? b_off[r] : b_off[0] + r * g.w_cols;
        rb4[S][r] = *reinterpret_cast<const u32x4*>(g.w16 + off + ks);
      }
    }
  };
  auto store_tile = [&](auto slot_c, int st) {
    constexpr int S = decltype(slot_c)::value;
    uint16_t* sA = sA0 + st * (BM * LDSW);
    uint16_t* sB = sB0 + st * (BN * LDSW);
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = ptid + 256 * i;
      *reinterpret_cast<u32x4*>(&sA[(c >> 3) * LDSW + (c & 7) * 8]) = ra[S][i];
    }
    if constexpr (BMODE == BMODE_NK) {
      if constexpr (BQ == BQ_Q4) {
        uint32_t o[16];
        dequant32<DT>(rb4[S][0], (uint16_t)(rsz[S][0] & 0xFFFFu), (uint16_t)(rsz[S][0] >> 16), o);
        u32x4* dst = reinterpret_cast<u32x4*>(&sB[(ptid >> 1) * LDSW + (ptid & 1) * 32]);
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[j] = u32x4{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = ptid + 256 * i;
          *reinterpret_cast<u32x4*>(&sB[(c >> 3) * LDSW + (c & 7) * 8]) = rb4[S][i];
        }
      }
    } else {
      // rows r = 0..3 hold 8 consecutive columns each as 4 pairs (col 2p, 2p+1);
      // write column-major: 4 consecutive contraction values per column (8 bytes)
      uint32_t v[4][4];
      if constexpr (BQ == BQ_Q4) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f16 sv = __builtin_bit_cast(f16, (uint16_t)(rsz[S][r] & 0xFFFFu));
          const f16 zv = __builtin_bit_cast(f16, (uint16_t)(rsz[S][r] >> 16));
          const f16x2 s2 = {sv, sv}, z2 = {zv, zv};
          dq_word(rw[S][r], s2, z2, v[r]);
          if constexpr (DT == USAF_BF16) {
#pragma unroll
            for (int p = 0; p < 4; ++p) v[r][p] = h2_to_bf2(v[r][p]);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r][0] = rb4[S][r].x; v[r][1] = rb4[S][r].y; v[r][2] = rb4[S][r].z; v[r][3] = rb4[S][r].w;
        }
      }
      const int kb = ptid & 15, nb = ptid >> 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint2 even, odd;
        even.x = __builtin_amdgcn_perm(v[1][p], v[0][p], 0x05040100u);  // lo halves of rows 0,1
        even.y = __builtin_amdgcn_perm(v[3][p], v[2][p], 0x05040100u);  // lo halves of rows 2,3
        odd.x = __builtin_amdgcn_perm(v[1][p], v[0][p], 0x07060302u);   // hi halves of rows 0,1
        odd.y = __builtin_amdgcn_perm(v[3][p], v[2][p], 0x07060302u);
        *reinterpret_cast<uint2*>(&sB[(nb * 8 + 2 * p) * LDSW + 4 * kb]) = even;
        *reinterpret_cast<uint2*>(&sB[(nb * 8 + 2 * p + 1) * LDSW + 4 * kb]) = odd;
      }
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;

  // Steady-state loops are branch-free (every store and load of a step exists);
  // the guarded tail finishes the remaining steps.  One barrier per step k
  // (store tile k+1 into stage (k+1)&1, load tile k+RING into the slot tile k left).
  if constexpr (RING == 3) {
    load_tile(S0{}, 0);
    if (nk > 1) load_tile(S1{}, 1);
    if (nk > 2) load_tile(S2{}, 2);
    store_tile(S0{}, 0);
    lds_barrier();
    int k = 0;
    for (; k + 5 < nk; k += 3) {
      store_tile(S1{}, (k + 1) & 1); load_tile(S0{}, k + 3); lds_barrier();
      store_tile(S2{}, (k + 2) & 1); load_tile(S1{}, k + 4); lds_barrier();
      store_tile(S0{}, (k + 3) & 1); load_tile(S2{}, k + 5); lds_barrier();
    }
    auto step = [&](auto store_c, auto load_c, int kk) {
      if (kk + 1 < nk) store_tile(store_c, (kk + 1) & 1);
      if (kk + 3 < nk) load_tile(load_c, kk + 3);
      lds_barrier();
    };
    for (; k < nk; k += 3) {
      step(S1{}, S0{}, k);
      if (k + 1 < nk) step(S2{}, S1{}, k + 1);
      if (k + 2 < nk) step(S0{}, S2{}, k + 2);
    }
  } else {
    load_tile(S0{}, 0);
    if (nk > 1) load_tile(S1{}, 1);
    store_tile(S0{}, 0);
    lds_barrier();
    int k = 0;
    for (; k + 3 < nk; k += 2) {
      store_tile(S1{}, (k + 1) & 1); load_tile(S0{}, k + 2); lds_barrier();
      store_tile(S0{}, (k + 2) & 1); load_tile(S1{}, k + 3); lds_barrier();
    }
    auto step = [&](auto store_c, auto load_c, int kk) {
      if (kk + 1 < nk) store_tile(store_c, (kk + 1) & 1);
      if (kk + 2 < nk) load_tile(load_c, kk + 2);
      lds_barrier();
    };
    for (; k < nk; k += 2) {
      step(S1{}, S0{}, k);
      if (k + 1 < nk) step(S0{}, S1{}, k + 1);
    }
  }
  lds_barrier();  // the multiply waves park their accumulators
}

// ---- multiply waves: LDS fragments -> MFMA, accumulators parked in LDS ----
// Waves 0-3 as 2 (M) x 2 (N); each owns WM_SUB x 2 MFMA 32x32 accumulators.
// A fragments are re-read one k16 step ahead and B fragments double-buffered
// so LDS latency hides behind the MFMAs.  Row blocks past the expert's last
// slot multiply stale rows whose results are never stored.
template <int DT>
__device__ __forceinline__ void consume_tile(const uint16_t* sA0, const uint16_t* sB0, const int lane, const int wm,
                                             const int wn, const int nk, const int nrb, uint16_t* sC) {
  f32x16 acc[WM_SUB][2];
#pragma unroll
  for (int i = 0; i < WM_SUB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  auto frag_a = [&](int st, int i, int kk) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(
        &sA0[st * (BM * LDSW) + ((wm * WM_SUB + i) * 32 + (lane & 31)) * LDSW + kk * 16 + (lane >> 5) * 8]);
  };
  auto frag_b = [&](int st, int j, int kk) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(
        &sB0[st * (BN * LDSW) + (wn * 64 + j * 32 + (lane & 31)) * LDSW + kk * 16 + (lane >> 5) * 8]);
  };
  lds_barrier();  // stage 0 filled
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    u32x4 fa[WM_SUB], fb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) fb[j] = frag_b(cur, j, 0);
#pragma unroll
    for (int i = 0; i < WM_SUB; ++i) fa[i] = frag_a(cur, i, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      u32x4 fbn[2];
      if (kk + 1 < BK / 16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) fbn[j] = frag_b(cur, j, kk + 1);
      }
#pragma unroll
      for (int i = 0; i < WM_SUB; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
        if (kk + 1 < BK / 16) fa[i] = frag_a(cur, i, kk + 1);
      }
      if (kk + 1 < BK / 16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) fb[j] = fbn[j];
      }
    }
    lds_barrier();
  }
  // park dtype(acc) as the [BM][BN] tile; acc[i][j][r] is tile row
  // 32*(wm*WM_SUB+i) + 8*(r/4) + 4*(lane/32) + r%4, column wn*64 + j*32 + lane%32
  if (wm * WM_SUB < nrb) {
#pragma unroll
    for (int i = 0; i < WM_SUB; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * (wm * WM_SUB + i) + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          const int col = wn * 64 + j * 32 + (lane & 31);
          sC[row * LDSC + col] = round_bits<DT>(acc[i][j][r]);
        }
  }
  lds_barrier();
}

// ---- tile list ------------------------------------------------------------------
// Expert e's slots form ceil(S_e / BMV) m-tiles of BMV rows; the last one is
// "light" when it holds fewer than BMV / 2 rows.  The list puts every heavy
// m-tile (expert-major) before every light one, so tiles of equal cost run in
// the same rounds and the blocks sharing an m-tile stay in step.
// s_h[e] / s_l[e]: prefix counts of heavy / light m-tiles before expert e
// (s_h[E], s_l[E] the totals).  All THREADS threads call it.
template <int THREADS>
__device__ __forceinline__ void block_scan(int32_t* s_part, int tid, int local) {
  s_part[tid] = local;
  lds_barrier();
  for (int off = 1; off < THREADS; off <<= 1) {
    const int v = (tid >= off) ? s_part[tid - off] : 0;
    lds_barrier();
    s_part[tid] += v;
    lds_barrier();
  }
}

template <int THREADS, int BMV>
__device__ __forceinline__ void mtile_prefix(const GemmArgs& g, int32_t* s_h, int32_t* s_l, int32_t* s_part,
                                             int tid) {
  const int E = g.E;
  const int per = (E + THREADS - 1) / THREADS;
  const int e0 = tid * per;
  auto counts = [&](int e, int& h, int& l) {
    const int S = g.offsets[e + 1] - g.offsets[e];
    const int c = (S + BMV - 1) / BMV;
    l = (c > 0 && S - (c - 1) * BMV < BMV / 2) ? 1 : 0;
    h = c - l;
  };
  int hl = 0, ll = 0;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      int h, l;
      counts(e, h, l);
      hl += h;
      ll += l;
    }
  }
  block_scan<THREADS>(s_part, tid, hl);
  int run = s_part[tid] - hl;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      int h, l;
      counts(e, h, l);
      s_h[e] = run;
      run += h;
    }
  }
  if (tid == THREADS - 1) s_h[E] = s_part[THREADS - 1];
  lds_barrier();
  block_scan<THREADS>(s_part, tid, ll);
  run = s_part[tid] - ll;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      int h, l;
      counts(e, h, l);
      s_l[e] = run;
      run += l;
    }
  }
  if (tid == THREADS - 1) s_l[E] = s_part[THREADS - 1];
  lds_barrier();
}

// mtile_prefix from expert offsets already in LDS (s_off[0..E]), by one wave:
// lane l takes experts 4l .. 4l + 3 (E <= 256) and the prefixes come from
// shuffle scans, with no block barrier.  Called by the 64 lanes of one wave.
template <int BMV>
__device__ __forceinline__ void mtile_prefix_wave(const int32_t* s_off, int E, int32_t* s_h, int32_t* s_l, int lane) {
  int h[4], l[4], hs = 0, ls = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = 4 * lane + k;
    h[k] = l[k] = 0;
    if (e < E) {
      const int S = s_off[e + 1] - s_off[e];
      const int c = (S + BMV - 1) / BMV;
      l[k] = (c > 0 && S - (c - 1) * BMV < BMV / 2) ? 1 : 0;
      h[k] = c - l[k];
    }
    hs += h[k];
    ls += l[k];
  }
  int hi = hs, li = ls;  // inclusive scans over the lanes
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int ho = __shfl_up(hi, d, 64), lo = __shfl_up(li, d, 64);
    if (lane >= d) {
      hi += ho;
      li += lo;
    }
  }
  int hr = hi - hs, lr = li - ls;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = 4 * lane + k;
    if (e < E) {
      s_h[e] = hr;
      s_l[e] = lr;
    }
    hr += h[k];
    lr += l[k];
  }
  if (lane == 63) {
    s_h[E] = hi;
    s_l[E] = li;
  }
}

// largest e with pre[e] <= x (pre non-decreasing, pre[0] = 0 <= x)
__device__ __forceinline__ int prefix_owner(const int32_t* pre, int E, int64_t x) {
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// m-tile mt of the list -> expert, first slot, rows
template <int BMV>
__device__ __forceinline__ void mtile_decode(const GemmArgs& g, const int32_t* s_h, const int32_t* s_l, int64_t mt,
                                             int& e, int64_t& m_beg, int& valid) {
  const int E = g.E;
  int64_t j;
  if (mt < s_h[E]) {
    e = prefix_owner(s_h, E, mt);
    j = mt - s_h[e];
  } else {
    e = prefix_owner(s_l, E, mt - s_h[E]);
    const int S = g.offsets[e + 1] - g.offsets[e];
    j = (S + BMV - 1) / BMV - 1;
  }
  m_beg = g.offsets[e] + j * BMV;
  const int64_t rem = g.offsets[e + 1] - m_beg;
  valid = (int)(rem < BMV ? rem : BMV);
}

// XCD-aware tile walk: blocks are dispatched round-robin over kXcds dies
// (block b on die b % dies), and die d takes the m-tiles mt = d, d + dies, ...
// with all their n-tiles, spread over the die's blocks; the n-tiles of one
// m-tile -- which read the same activation rows -- run together on one die
// and share its L2, and every die gets the same mix of heavy and light tiles.
struct TileWalk {
  // counts of blocks, tiles and units: 32-bit (a 64-bit division is a long
  // emulated sequence; these run in every prologue and tile decode)
  int n_mt, n_nt;
  int dies, xcd;
  int per_xcd, local_b, count;  // blocks on this die, this block's rank, m-tiles of this die
  __device__ TileWalk(int64_t n_mt_, int64_t n_nt_) : n_mt((int)n_mt_), n_nt((int)n_nt_) {
    const int nblk = (int)gridDim.x;
    dies = nblk < kXcds ? nblk : kXcds;
    xcd = (int)(blockIdx.x % (unsigned)dies);
    per_xcd = (nblk + dies - 1 - xcd) / dies;
    local_b = (int)(blockIdx.x / (unsigned)dies);
    count = n_mt > xcd ? (n_mt - xcd + dies - 1) / dies : 0;
  }
  __device__ int64_t first() const { return local_b; }
  __device__ int64_t end() const { return (int64_t)count * n_nt; }
  __device__ int64_t step() const { return per_xcd; }
  __device__ void decode(int64_t u, int64_t& mt, int64_t& nt) const {
    const int q = (int)u / n_nt;
    mt = xcd + (int64_t)dies * q;
    nt = (int)u - q * n_nt;
  }
  // Pass p hands units [p * per_xcd, (p + 1) * per_xcd) to the die's blocks,
  // upward (block b takes position b), as a plain round-robin does.  When the
  // heavy units do not fill whole passes, the passes after the one holding the
  // last heavy unit alternate downward and upward: the unit list runs heavy
  // tiles before light remainders, so the blocks left one heavy tile short
  // take the light ones first, and a second round of light units starts again
  // from them instead of from the blocks that ran the extra heavy tile.
  int pass_turn = INT32_MAX;  // first pass that runs downward (set by set_heavy)
  __device__ void set_heavy(int64_t n_heavy_mt) {
    const int nh = (int)n_heavy_mt;
    const int hd = nh > xcd ? (nh - xcd + dies - 1) / dies : 0;
    const int uh = hd * n_nt;
    pass_turn = uh % per_xcd == 0 ? INT32_MAX : uh / per_xcd + 1;
  }
  __device__ bool down(int64_t p) const { return p >= pass_turn && ((p - pass_turn) & 1) == 0; }
  __device__ int64_t snake_unit(int64_t p) const {
    return (int)p * per_xcd + (down(p) ? per_xcd - 1 - local_b : local_b);
  }
  __device__ int snake_count() const {
    const int tot = count * n_nt, full = tot / per_xcd, rem = tot % per_xcd;
    const int pos = down(full) ? per_xcd - 1 - local_b : local_b;
    return full + (pos < rem ? 1 : 0);
  }
};

template <int BMODE, int EPI, int BQ, int DT>
__global__ __launch_bounds__(kThreads) void moe_gemm_kernel(const GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* const sA0 = smem;                      // [2][BM * LDSW]
  uint16_t* const sB0 = smem + 2 * BM * LDSW;      // [2][BN * LDSW]
  int32_t* const s_h = reinterpret_cast<int32_t*>(smem + 2 * (BM + BN) * LDSW);  // [MAX_E + 1]
  int32_t* const s_l = s_h + MAX_E + 1;                                           // [MAX_E + 1]
  int32_t* const s_part = s_l + MAX_E + 1;                                        // [kThreads]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  // Waves 0-3 multiply (2 x 2 over the tile), waves 4-7 feed the LDS stages.
  // Waves are placed round-robin on the 4 SIMDs, so every SIMD runs one of each.
  const bool producer = wave >= 4;
  const int ptid = tid - 256;  // producer thread index 0..255
  const int wm = (wave & 3) >> 1, wn = wave & 1;
  const int E = g.E;

  mtile_prefix<kThreads, BM>(g, s_h, s_l, s_part, tid);
  const int64_t n_nt = (EPI == EPI_SWIGLU_FWD) ? g.N / 64 : g.N / BN;
  const int nk = (int)(g.K / BK);
  const TileWalk walk(s_h[E] + s_l[E], n_nt);
  for (int64_t u = walk.first(); u < walk.end(); u += walk.step()) {
    int64_t mt, nt;
    walk.decode(u, mt, nt);
    int e, valid;
    int64_t m_beg;
    mtile_decode<BM>(g, s_h, s_l, mt, e, m_beg, valid);
    const int nrb = (valid + 31) >> 5;  // 32-row blocks holding slots
    const int64_t n0 = (EPI == EPI_SWIGLU_FWD) ? nt * 64 : nt * BN;

    if (producer) {
      produce_tile<BMODE, EPI, BQ, DT>(g, sA0, sB0, ptid, e, m_beg, valid, n0, nk);
    } else {
      consume_tile<DT>(sA0, sB0, lane, wm, wn, nk, nrb, sA0);
    }

    // ---- epilogue: all waves walk the valid rows in 8-column chunks of the
    //      [BM][BN] dtype tile the multiply waves parked in LDS (sA0) ----
    const uint16_t* sC = sA0;
    constexpr int CPR = (EPI == EPI_SWIGLU_FWD) ? 8 : 16;  // 8-column chunks per row
    for (int c = tid; c < valid * CPR; c += kThreads) {
      const int row = c / CPR, ch = c % CPR;
      const int64_t m = m_beg + row;
      if constexpr (EPI == EPI_STORE) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(&sC[row * LDSC + ch * 8]);
        *reinterpret_cast<u32x4*>(g.out + m * g.ldo + n0 + ch * 8) = v;
      } else if constexpr (EPI == EPI_SWIGLU_FWD) {
        // output columns o..o+7 (o = 8*ch): gate at tile column (o/32)*64 + o%32, up 32 further
        const int o = ch * 8;
        const int cg = (o >> 5) * 64 + (o & 31);
        const u32x4 gv = *reinterpret_cast<const u32x4*>(&sC[row * LDSC + cg]);
        const u32x4 uv = *reinterpret_cast<const u32x4*>(&sC[row * LDSC + cg + 32]);
        const int64_t n = n0 + o;
        *reinterpret_cast<u32x4*>(g.out2 + m * g.ldo2 + n) = gv;
        *reinterpret_cast<u32x4*>(g.out2 + m * g.ldo2 + g.inter + n) = uv;
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
        uint32_t aw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t h2 = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float gt = bits_to_f32<DT>((uint16_t)(gw[q] >> (16 * h)));
            const float up = bits_to_f32<DT>((uint16_t)(uw[q] >> (16 * h)));
            const float sg = round_to<DT>(silu_f(gt));
            h2 |= (uint32_t)round_bits<DT>(sg * up) << (16 * h);
          }
          aw[q] = h2;
        }
        *reinterpret_cast<u32x4*>(g.out + m * g.ldo + n) = u32x4{aw[0], aw[1], aw[2], aw[3]};
      } else {  // EPI_SWIGLU_BWD
        const int64_t n = n0 + ch * 8;
        const u32x4 dv = *reinterpret_cast<const u32x4*>(&sC[row * LDSC + ch * 8]);
        const u32x4 gv = *reinterpret_cast<const u32x4*>(g.aux + m * g.ld_aux + n);
        const u32x4 uv = *reinterpret_cast<const u32x4*>(g.aux + m * g.ld_aux + g.inter + n);
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w},
                       uw[4] = {uv.x, uv.y, uv.z, uv.w};
        uint32_t dg_w[4], du_w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t a = 0, b = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float da = bits_to_f32<DT>((uint16_t)(dw[q] >> (16 * h)));
            const float gt = bits_to_f32<DT>((uint16_t)(gw[q] >> (16 * h)));
            const float up = bits_to_f32<DT>((uint16_t)(uw[q] >> (16 * h)));
            const float sig = 1.0f / (1.0f + expf(-gt));
            const float sg = round_to<DT>(gt * sig);
            const float dsil = round_to<DT>(da * up);
            const float dg = (dsil * sig) * (1.0f + gt * (1.0f - sig));
            a |= (uint32_t)round_bits<DT>(dg) << (16 * h);
            b |= (uint32_t)round_bits<DT>(da * sg) << (16 * h);
          }
          dg_w[q] = a;
          du_w[q] = b;
        }
        *reinterpret_cast<u32x4*>(g.out + m * g.ldo + n) = u32x4{dg_w[0], dg_w[1], dg_w[2], dg_w[3]};
        *reinterpret_cast<u32x4*>(g.out + m * g.ldo + g.inter + n) = u32x4{du_w[0], du_w[1], du_w[2], du_w[3]};
      }
    }
    lds_barrier();  // sC aliases the stage buffers the next tile fills
  }
}

// =====================================================================================
// Forward (NK) kernel: weight fragments dequantized straight into MFMA registers.
//
// 256 threads = 4 waves, one per SIMD, one block per CU.  Tile: up to 320 slots
// of one expert (10 row blocks of 32) x 256 output columns; wave w owns tile
// columns [64w, 64w + 64) (two 32-column blocks) for every row.  Per k-step of 64:
//   * the block stages the 320 x 64 activation tile in LDS (two stages), loaded
//     one k-step ahead into registers;
//   * each lane loads the 16 code bytes (32 k-values of one group) of its weight
//     row per column block and dequantizes them in registers into the k-step's
//     four MFMA B fragments: lane half h takes k = 32h + 8j + [0, 8) at sub-step
//     j, and the activation fragments read the same k from LDS.
// The weight tile never touches LDS and every weight element is dequantized
// once; the activation tile is read from global memory once per 256 columns.
// SwiGLU: column block 0 of wave w holds gate rows n, block 1 the up rows I + n
// of the same 32 n, so silu(gate) * up is formed in registers.
// =====================================================================================
constexpr int NK_BM = 256, NK_BN = 256, NK_THREADS = 256;
constexpr int NK_A_CHUNKS = NK_BM * BK / 8 / NK_THREADS;  // 16-byte A chunks per thread per k-step
constexpr int NK_EPW = 40;      // epilogue staging row stride (16-bit elements; rows stay 16-byte aligned)
constexpr int NK_EPI_ARR = 3;   // 32 x 32 blocks a wave stages per row block (gate, up, act)
constexpr int NK_EPI_ELEMS = NK_EPI_ARR * 32 * NK_EPW;
constexpr size_t kNkSmemBytes =
    (size_t)2 * NK_BM * LDSW * 2 + (size_t)4 * NK_EPI_ELEMS * 2 + (size_t)(2 * (MAX_E + 1) + NK_THREADS) * 4;

// 8 codes of one 32-bit word (code 2i in the low nibble of byte i) -> 8 16-bit
// weights in natural order, bit-identical to dequantize_4bit:
// fp16(fp16(q * s) + z), then RNE bf16 for bf16 operands.
template <int DT>
__device__ __forceinline__ u32x4 dq8(uint32_t w, f16x2 s2, f16x2 z2) {
#pragma clang fp contract(off)
  const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
  const f16x2 sub = {(f16)-1024.0f, (f16)-64.0f};
  uint32_t o[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // byte p in both halves: the low half keeps code 2p (bits 0-3), the high half
    // code 2p+1 (bits 20-23), as fp16 1024 + q and 1024 + 16 q
    const uint32_t t = __builtin_amdgcn_perm(w, w, 0x0C000C00u | ((uint32_t)p << 16) | (uint32_t)p);
    const uint32_t bits = (t & 0x00F0000Fu) | 0x64006400u;
    const f16x2 q = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, bits), mul, sub);  // exact codes
    const f16x2 m = q * s2;
    const f16x2 v = m + z2;
    o[p] = __builtin_bit_cast(uint32_t, v);
    if constexpr (DT == USAF_BF16) o[p] = h2_to_bf2(o[p]);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// Codes 2p, 2p+1 of a 32-bit code word (byte p) -> their two 16-bit weights
// (dq8 for one pair).  v_perm places byte p under the fp16 exponent byte 0x64 in
// both halves; the mask keeps code 2p in the low half (1024 + q) and code 2p+1
// in the high half (1024 + 16 q).
template <int DT>
__device__ __forceinline__ uint32_t dq_pair(uint32_t w, int p, f16x2 s2, f16x2 z2) {
#pragma clang fp contract(off)
  const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
  const f16x2 sub = {(f16)-1024.0f, (f16)-64.0f};
  const uint32_t t = __builtin_amdgcn_perm(0x64646464u, w, 0x04000400u | ((uint32_t)p << 16) | (uint32_t)p) & 0xFFF0FF0Fu;
  const f16x2 q = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, t), mul, sub);  // exact codes
  const f16x2 m = q * s2;
  const f16x2 v = m + z2;
  uint32_t o = __builtin_bit_cast(uint32_t, v);
  if constexpr (DT == USAF_BF16) o = h2_to_bf2(o);
  return o;
}

// One tile of the NK kernel with NRB (>= the tile's occupied row blocks) row
// blocks computed.  Row blocks past the expert's slots multiply rows of the
// staged tile that are never stored.
template <int NRB, int EPI, int BQ, int DT>
__device__ __forceinline__ void nk_tile(const GemmArgs& g, uint16_t* sA0, uint16_t* sE, const int tid, const int e,
                                        const int64_t m_beg, const int valid, const int64_t nt, const int nk) {
  const int lane = tid & 63, wave = tid >> 6, l32 = lane & 31, half = lane >> 5;
  const int64_t K = g.K;
  // this wave's weight rows (one per column block) and whether it has columns at all;
  // a wave without columns (last n-tile of a ragged N) multiplies row 0's weights
  // and stores nothing, so the k-loop has no wave-dependent branches
  int64_t nbase;  // first output column of the wave (gate column for SwiGLU)
  bool wave_on;
  int64_t wrow[2];
  if constexpr (EPI == EPI_SWIGLU_FWD) {
    nbase = nt * 128 + wave * 32;
    wave_on = nbase < g.inter;
    wrow[0] = nbase + l32;
    wrow[1] = g.inter + nbase + l32;
  } else {
    nbase = nt * NK_BN + wave * 64;
    wave_on = nbase < g.N;
    wrow[0] = nbase + l32;
    wrow[1] = nbase + 32 + l32;
  }
  // element offset of (weight row, k = 32 * half) in the [E, w_rows, K] weight
  int64_t woff[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
    woff[cb] = ((BQ == BQ_DENSE16 ? weight_block(g, e) : (int64_t)e) * g.w_rows + (wave_on ? wrow[cb] : 0)) * K +
               32 * half;

  // A: chunk c = tid + 256 i is row (tid >> 3) + 32 i (row block i), k block tid & 7
  int32_t a_off[NRB];
#pragma unroll
  for (int i = 0; i < NRB; ++i) {
    const int row = (tid >> 3) + 32 * i;
    const int64_t m = m_beg + (row < valid ? row : valid - 1);
    const int64_t arow = g.a_rows ? (int64_t)g.a_rows[m] : m;
    a_off[i] = (int32_t)(arow * g.lda + (tid & 7) * 8);
  }
  const int a_lds = (tid >> 3) * LDSW + (tid & 7) * 8;

  using std::integral_constant;
  // Regions per k-step: each covers sub-step j and G consecutive row blocks
  // (2G MFMAs); with G = 2 a region also holds two weight pairs whose
  // dependent dequant chains interleave instead of stalling on each other.
  constexpr int G = NRB >= 2 ? 2 : 1;
  constexpr int RPJ = NRB / G;   // regions per sub-step
  constexpr int R = 4 * RPJ;     // regions per k-step
  constexpr int NF = 4 * NRB;    // A fragments per k-step, f = j * NRB + i
  constexpr int PF = 4 * G;      // A-fragment prefetch distance (fragments)
  constexpr int NPAIR = (BQ == BQ_Q4) ? 32 : 0;  // weight pairs per k-step per lane
  constexpr int PPR = (NPAIR + R - 1) / R;       // pairs dequantized per region
  const int frag = l32 * LDSW + 32 * half;  // lane's A fragment: row l32 of a row block, k = 32 half + 8 j

  u32x4 ra[NRB];            // A chunks of the next stage, in flight between global and LDS
  u32x4 bfs[2][2][4];       // B fragments [slot][column block][sub-step j]
  u32x4 cq[3][2];           // 4-bit codes of three k-steps (ring) [slot][column block]
  uint32_t csz[3][2];       // their scale/zero pairs
  f32x16 acc[NRB][2];
#pragma unroll
  for (int i = 0; i < NRB; ++i) acc[i][0] = acc[i][1] = f32x16{};

  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < NRB; ++i) ra[i] = *reinterpret_cast<const u32x4*>(g.A + a_off[i] + kt * BK);
  };
  auto store_a = [&](int st) {
#pragma unroll
    for (int i = 0; i < NRB; ++i) *reinterpret_cast<u32x4*>(&sA0[st * (NK_BM * LDSW) + a_lds + 32 * i * LDSW]) = ra[i];
  };
  // codes + scale/zero pairs of k-step kk (clamped to the last one) into ring slot CS
  auto load_codes = [&](auto CSc, int kk) {
    constexpr int CS = decltype(CSc)::value;
    kk = kk < nk ? kk : nk - 1;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int64_t el = woff[cb] + (int64_t)kk * BK;
      cq[CS][cb] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g.wq + (el >> 1)));
      csz[CS][cb] = g.wsz[el >> 7];
    }
  };
  // dense 16-bit weight fragments of k-step kk into B slot BS
  auto load_dense = [&](auto BSc, int kk) {
    constexpr int BS = decltype(BSc)::value;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int64_t el = woff[cb] + (int64_t)kk * BK;
#pragma unroll
      for (int j = 0; j < 4; ++j) bfs[BS][cb][j] = *reinterpret_cast<const u32x4*>(g.w16 + el + 8 * j);
    }
  };
  // whole-k-step dequant of ring slot CS into B slot BS (prologue and tail)
  auto dequant_all = [&](auto BSc, auto CSc) {
    constexpr int BS = decltype(BSc)::value, CS = decltype(CSc)::value;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const f16x2 s2 = __builtin_bit_cast(f16x2, (csz[CS][cb] & 0xFFFFu) * 0x10001u);
      const f16x2 z2 = __builtin_bit_cast(f16x2, (csz[CS][cb] >> 16) * 0x10001u);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfs[BS][cb][j] = dq8<DT>(cq[CS][cb][j], s2, z2);
    }
  };
  // the MFMAs of k-step kt alone (last two k-steps), in the same regions
  auto mma = [&](auto BSc, int kt) {
    constexpr int BS = decltype(BSc)::value;
    const uint16_t* sA = sA0 + (kt & 1) * (NK_BM * LDSW);
    u32x4 af[NF];
#pragma unroll
    for (int f = 0; f < PF && f < NF; ++f)
      af[f] = *reinterpret_cast<const u32x4*>(&sA[(f % NRB) * 32 * LDSW + frag + 8 * (f / NRB)]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = r / RPJ;
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const int f = j * NRB + (r % RPJ) * G + gg, i = f % NRB;
        if (f + PF < NF)
          af[f + PF] = *reinterpret_cast<const u32x4*>(&sA[((f + PF) % NRB) * 32 * LDSW + frag + 8 * ((f + PF) / NRB)]);
        acc[i][0] = mfma32<DT>(af[f], bfs[BS][0][j], acc[i][0]);
        acc[i][1] = mfma32<DT>(af[f], bfs[BS][1][j], acc[i][1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One steady k-step kt (kt + 2 < nk), software-pipelined in source order: the
  // 8 * NRB MFMAs form R regions of two; every region also reads the A
  // fragment of region r + PF from LDS and dequantizes its share of the next
  // k-step's weights (ring slot CS -> B slot BS ^ 1), and every other region
  // stages one A chunk of kt + 1 into LDS or refills it with kt + 2.  The codes
  // of kt + 3 are fetched at the top, two k-steps before they are needed.
  // sched_barrier keeps the regions in this order, so the matrix pipe has
  // independent VALU, LDS and memory work issued between its MFMAs.
  auto step = [&](auto BSc, auto CSc, int kt) {
    constexpr int BS = decltype(BSc)::value, CS = decltype(CSc)::value;
    const uint16_t* sA = sA0 + (kt & 1) * (NK_BM * LDSW);
    uint16_t* sAn = sA0 + ((kt + 1) & 1) * (NK_BM * LDSW);
    u32x4 af[NF];
    f16x2 s2[2], z2[2];
#pragma unroll
    for (int f = 0; f < PF && f < NF; ++f)
      af[f] = *reinterpret_cast<const u32x4*>(&sA[(f % NRB) * 32 * LDSW + frag + 8 * (f / NRB)]);
    if constexpr (BQ == BQ_Q4) load_codes(integral_constant<int, (CS + 2) % 3>{}, kt + 3);
    else load_dense(integral_constant<int, BS ^ 1>{}, kt + 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = r / RPJ;
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const int f = j * NRB + (r % RPJ) * G + gg, i = f % NRB;
        if (f + PF < NF)
          af[f + PF] = *reinterpret_cast<const u32x4*>(&sA[((f + PF) % NRB) * 32 * LDSW + frag + 8 * ((f + PF) / NRB)]);
        acc[i][0] = mfma32<DT>(af[f], bfs[BS][0][j], acc[i][0]);
        acc[i][1] = mfma32<DT>(af[f], bfs[BS][1][j], acc[i][1]);
      }
      if constexpr (BQ == BQ_Q4) {
#pragma unroll
        for (int pp = 0; pp < PPR; ++pp) {
          const int p = r * PPR + pp;
          if (p < NPAIR) {
            const int cb = p >> 4, wd = (p >> 2) & 3, q = p & 3;
            if ((p & 15) == 0) {
              s2[cb] = __builtin_bit_cast(f16x2, (csz[CS][cb] & 0xFFFFu) * 0x10001u);
              z2[cb] = __builtin_bit_cast(f16x2, (csz[CS][cb] >> 16) * 0x10001u);
            }
            bfs[BS ^ 1][cb][wd][q] = dq_pair<DT>(cq[CS][cb][wd], q, s2[cb], z2[cb]);
          }
        }
      }
      // stage the A chunks of k-step kt + 1 and refill them with kt + 2, CPR chunks per region
      constexpr int CPR = (NRB + R - 1) / R;
#pragma unroll
      for (int cc = 0; cc < CPR; ++cc) {
        const int c = r * CPR + cc;
        if (c < NRB) {
          *reinterpret_cast<u32x4*>(&sAn[a_lds + 32 * c * LDSW]) = ra[c];
          ra[c] = *reinterpret_cast<const u32x4*>(g.A + a_off[c] + (kt + 2) * BK);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();
  };

  // prologue: A of k-step 0 staged in LDS and k-step 1 in flight; B of k-step 0
  // in slot 0; codes of k-steps 1 and 2 in ring slots 0 and 1
  using I0 = integral_constant<int, 0>;
  using I1 = integral_constant<int, 1>;
  using I2 = integral_constant<int, 2>;
  load_a(0);
  if constexpr (BQ == BQ_Q4) {
    load_codes(I2{}, 0);
    load_codes(I0{}, 1);
    load_codes(I1{}, 2);
  } else {
    load_dense(I0{}, 0);
  }
  store_a(0);
  if constexpr (BQ == BQ_Q4) dequant_all(I0{}, I2{});
  load_a(1);
  lds_barrier();

  // steady state, unrolled by six so that the B slots (period 2) and the code
  // ring (period 3) are addressed statically: no register moves of data whose
  // loads may still be in flight
  int kt = 0;
  for (; kt + 7 < nk; kt += 6) {
    step(I0{}, I0{}, kt);
    step(I1{}, I1{}, kt + 1);
    step(I0{}, I2{}, kt + 2);
    step(I1{}, I0{}, kt + 3);
    step(I0{}, I1{}, kt + 4);
    step(I1{}, I2{}, kt + 5);
  }
  // remaining steady steps (fewer than six) rotate the slots back to the same
  // positions after each step
  for (; kt + 2 < nk; ++kt) {
    step(I0{}, I0{}, kt);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) bfs[0][cb][j] = bfs[1][cb][j];
      cq[0][cb] = cq[1][cb];
      csz[0][cb] = csz[1][cb];
      cq[1][cb] = cq[2][cb];
      csz[1][cb] = csz[2][cb];
    }
  }
  // the last two k-steps (nk >= 2: the entry points require K % 128 == 0)
  mma(I0{}, kt);
  store_a((kt + 1) & 1);
  if constexpr (BQ == BQ_Q4) dequant_all(I1{}, I0{});
  else load_dense(I1{}, kt + 1);
  lds_barrier();
  mma(I1{}, kt + 1);
  lds_barrier();  // every wave is done with the staged tiles

  // ---- epilogue: per row block, the wave's dtype results go through its own LDS
  //      area (C-fragment layout -> rows) and out as 16-byte row stores ----
  if (!wave_on) return;
  const int nrb = (valid + 31) >> 5;
#pragma unroll
  for (int i = 0; i < NRB; ++i) {
    if (i >= nrb) continue;
    const int rows = valid - 32 * i;  // valid rows in this row block (may exceed 32)
    if constexpr (EPI == EPI_SWIGLU_FWD) {
      // gate, up rounded to DT; act = DT(DT(silu(gate)) * up), two rows at a time
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const int row = 8 * (r >> 2) + 4 * half + (r & 3);
        const uint32_t gb = pack2<DT>(acc[i][0][r], acc[i][0][r + 1]);
        const uint32_t ub = pack2<DT>(acc[i][1][r], acc[i][1][r + 1]);
        const f32x2 gf = unpack2<DT>(gb), uf = unpack2<DT>(ub);
        const f32x2 sf = unpack2<DT>(pack2<DT>(silu_fast(gf.x), silu_fast(gf.y)));
        const uint32_t ab = pack2<DT>(sf.x * uf.x, sf.y * uf.y);
        sE[row * NK_EPW + l32] = (uint16_t)gb;
        sE[(row + 1) * NK_EPW + l32] = (uint16_t)(gb >> 16);
        sE[32 * NK_EPW + row * NK_EPW + l32] = (uint16_t)ub;
        sE[32 * NK_EPW + (row + 1) * NK_EPW + l32] = (uint16_t)(ub >> 16);
        sE[64 * NK_EPW + row * NK_EPW + l32] = (uint16_t)ab;
        sE[64 * NK_EPW + (row + 1) * NK_EPW + l32] = (uint16_t)(ab >> 16);
      }
#pragma unroll
      for (int q = 0; q < 6; ++q) {
        const int c = lane + 64 * q;
        const int arr = c >> 7, rr = (c & 127) >> 2, part = c & 3;
        if (rr < rows) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(&sE[arr * 32 * NK_EPW + rr * NK_EPW + part * 8]);
          const int64_t m = m_beg + 32 * i + rr;
          const int64_t n = nbase + part * 8;
          uint16_t* dst = (arr == 2) ? g.out + m * g.ldo + n : g.out2 + m * g.ldo2 + (arr == 1 ? g.inter : 0) + n;
          *reinterpret_cast<u32x4*>(dst) = v;
        }
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const int row = 8 * (r >> 2) + 4 * half + (r & 3);
          const uint32_t v = pack2<DT>(acc[i][cb][r], acc[i][cb][r + 1]);
          sE[cb * 32 * NK_EPW + row * NK_EPW + l32] = (uint16_t)v;
          sE[cb * 32 * NK_EPW + (row + 1) * NK_EPW + l32] = (uint16_t)(v >> 16);
        }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = lane + 64 * q;
        const int cb = c >> 7, rr = (c & 127) >> 2, part = c & 3;
        if (rr < rows) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(&sE[cb * 32 * NK_EPW + rr * NK_EPW + part * 8]);
          const int64_t m = m_beg + 32 * i + rr;
          *reinterpret_cast<u32x4*>(g.out + m * g.ldo + nbase + cb * 32 + part * 8) = v;
        }
      }
    }
  }
}

template <int EPI, int BQ, int DT>
__global__ __launch_bounds__(NK_THREADS) void moe_gemm_nk_kernel(const GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* const sA0 = smem;                           // [2][NK_BM * LDSW]
  uint16_t* const sE0 = smem + 2 * NK_BM * LDSW;        // [4 waves][NK_EPI_ELEMS]
  int32_t* const s_h = reinterpret_cast<int32_t*>(sE0 + 4 * NK_EPI_ELEMS);  // [MAX_E + 1]
  int32_t* const s_l = s_h + MAX_E + 1;                                     // [MAX_E + 1]
  int32_t* const s_part = s_l + MAX_E + 1;                                  // [NK_THREADS]
  const int tid = threadIdx.x;
  uint16_t* const sE = sE0 + (tid >> 6) * NK_EPI_ELEMS;
  const int E = g.E;
  mtile_prefix<NK_THREADS, NK_BM>(g, s_h, s_l, s_part, tid);
  const int64_t n_nt = (EPI == EPI_SWIGLU_FWD) ? (g.inter + 127) / 128 : (g.N + NK_BN - 1) / NK_BN;
  const int nk = (int)(g.K / BK);
  const TileWalk walk(s_h[E] + s_l[E], n_nt);
  for (int64_t u = walk.first(); u < walk.end(); u += walk.step()) {
    int64_t mt, nt;
    walk.decode(u, mt, nt);
    int e, valid;
    int64_t m_beg;
    mtile_decode<NK_BM>(g, s_h, s_l, mt, e, m_beg, valid);
    const int nrb = (valid + 31) >> 5;
    if (nrb > 4) nk_tile<8, EPI, BQ, DT>(g, sA0, sE, tid, e, m_beg, valid, nt, nk);
    else if (nrb > 2) nk_tile<4, EPI, BQ, DT>(g, sA0, sE, tid, e, m_beg, valid, nt, nk);
    else nk_tile<2, EPI, BQ, DT>(g, sA0, sE, tid, e, m_beg, valid, nt, nk);
  }
}

// =====================================================================================
// Forward (NK) kernel for 4-bit weights with LDS-DMA staging.
//
//   C[m, n] = sum_k A[row(m), k] * W_e[n, k]
//
// 512 threads = 8 waves, two per SIMD, one block per CU, persistent over a
// per-die tile list.  Tile: up to 256 slots of one expert (8 blocks of 32) x
// 256 weight rows; wave w owns weight rows [32w, 32w + 32) for every slot, so
// each weight element is dequantized once per tile.  The two waves of a SIMD
// fill each other's stalls (barrier, LDS and DMA counters) and share the
// issue cycles the matrix core leaves: one wave per SIMD cannot issue the
// dequant VALU work under its own MFMAs.
// The MFMA takes the weights as its A operand (32 n x 16 k) and the slots as
// its B operand (32 m x 16 k): a lane's accumulator then holds 4 consecutive
// output columns of one slot.
// Every global read is a global_load_lds (DMA into LDS, no VGPR staging)
// into a 3-stage ring, stage s = k-step % 3:
//   activations  256 rows x 128 B (16-byte chunks XOR-swizzled by row)
//   codes        256 weight rows x 32 B, scale|zero 256 x 4 B
//   (OVL) overlay entries, 64 words per wave
// At k-step gs a thread issues the codes of gs + 3 and the activations of
// gs + 2 (6 or 7 DMA instructions), multiplies k-step gs, and dequantizes the
// codes of gs + 1 into the other register set of weight fragments; the step
// ends with a vmcnt wait (everything older than this step's DMAs has landed)
// and a workgroup barrier.  The load streams run straight across tile
// boundaries, so the next tile's first k-steps are in flight during this
// tile's last steps and epilogue.
// =====================================================================================
constexpr int Q_BM = 256, Q_BN = 256, Q_THREADS = 512, Q_WAVES = Q_THREADS / 64;
constexpr int Q_MAX_E = 255;
constexpr int Q_A_BYTES = Q_BM * BK * 2;                 // activation rows of one k-step
constexpr int Q_C_BYTES = Q_BN * BK / 2;                 // codes of one k-step
constexpr int Q_Z_BYTES = Q_BN * 4;                      // scale|zero words of one k-step
constexpr int Q_OVL_WORDS = 64;                          // overlay entries per wave and k-step
constexpr int Q_O_BYTES = Q_WAVES * Q_OVL_WORDS * 4;     // overlay entries of one k-step
constexpr int Q_STAGE = Q_A_BYTES + Q_C_BYTES + Q_Z_BYTES + Q_O_BYTES;
constexpr int Q_A_LOADS = Q_A_BYTES / (16 * Q_THREADS);  // 4 x 16 B per thread
// DMA instructions per thread and k-step: d = 0 the scale|zero word, d = 1
// the code chunk, d = 2.. the activation chunks;
// OVL: d = Q_DMAS the wave's overlay entries of the code stream's k-step
constexpr int Q_DMAS = 2 + Q_A_LOADS;
// Overlay (trained values over the 4-bit weights): per wave and k-step one
// group of 64 entries, each a 32-bit word {byte offset | value << 16}.  Lane l
// holds word l, an entry of fragment register j = l / 16 whose offset points
// into that register's 1 KiB image (lane l' at byte 16 l'); unused words point
// into [1024, 2048) of the wave's epilogue tile, which the k-steps do not read.
// The entries travel with the codes of their k-step, in the same stage.
constexpr int Q_IMG = 64 * 16;                           // one fragment register of the wave
// Dynamic LDS (the DMA targets): 3 stages | s_h, s_l, s_off tables | token rows [2][Q_BM].
// A stage: activations | codes | scale|zero words | overlay entries.
// The epilogue tiles are a separate static array: the compiler then knows that
// their stores cannot collide with DMA writes still in flight and does not
// drain the DMAs before them.
constexpr int Q_TAB_OFF = 3 * Q_STAGE;
constexpr int Q_TOK_OFF = Q_TAB_OFF + 3 * (Q_MAX_E + 1) * 4;
constexpr size_t kQSmemBytes = (size_t)Q_TOK_OFF + 2 * Q_BM * 4;
constexpr int Q_EPW = 48;                       // staging row stride, 16-bit elements (48 or 32 columns)
constexpr int Q_EP_ELEMS = 32 * Q_EPW;          // one wave's 32-slot staging tile
static_assert(kQSmemBytes + Q_WAVES * Q_EP_ELEMS * 2 <= 160 * 1024, "LDS budget");
static_assert(Q_WAVES * Q_EP_ELEMS * 2 >= Q_THREADS * 4, "the prefix scratch lives in the epilogue tiles");
static_assert(Q_EP_ELEMS * 2 >= 2 * Q_IMG, "the overlay's fragment image and dummy area live in the wave's epilogue tile");

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// 16-byte chunk of an activation row: logical chunk c of row r sits at physical
// chunk c ^ ((r >> 1) & 7).  A fragment read takes 16 consecutive rows (one
// 16-byte chunk each) per 256-byte LDS cycle; two 128-byte rows share the 64
// banks, so the 16 chunks hit distinct banks when the even rows and the odd
// rows each take 8 distinct chunks.  (c ^ (r & 7) gives rows r and r + 8 the
// same chunk: a 2-way conflict in every cycle.)
__device__ __forceinline__ int q_swz(int r) { return (r >> 1) & 7; }

// LDS DMA (global_load_lds): lane l's 16 (4) bytes at base + off land at
// lds_dst + 16 l (4 l); base and lds_dst are wave-uniform.  Issued as inline
// asm: with the compiler's own LDS-DMA intrinsic in the code it stops counting
// the wave's LDS reads and waits for all of them (lgkmcnt(0)) before every use
// of a fragment, which drains the fragment prefetches several times a k-step.
// The DMAs count in vmcnt only; the k-step's explicit vmcnt wait covers them,
// and any wait the compiler places for its own loads is at least as strict
// with them in flight (vector memory loads complete in order).  M0 takes the
// LDS address; one wait state separates the M0 write from the DMA.
// lds: LDS byte address (uniform); base: uniform global pointer.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off), "s"(base) : "m0");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(off), "s"(base) : "m0");
}
// dma4 for a base that may come straight out of readfirstlane: 5 wait states
// between that VALU write of the SGPRs and the DMA reading them (s_mov + s_nop 3)
__device__ __forceinline__ void dma4_vb(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 3\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(off), "s"(base) : "m0");
}
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
// A wave-uniform 64-bit pointer in scalar registers: each 32-bit half passes
// readfirstlane as an unsigned word and the halves are joined zero-extended.
__device__ __forceinline__ const uint8_t* uni_ptr(const uint8_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)hi << 32) | (uint64_t)lo));
}

constexpr int Q_MTE_CAP = 1024;  // m-tiles covered by the m-tile -> expert table

struct QTile {
  int e, valid, m_beg, nt;  // all wave-uniform
};

// BT: the weight is a transposed copy (usaf_hip_q4_transpose): codes along k as
// usual, but every k has its own scale/zero, read as {s(k) | s(k+1) << 16,
// z(k) | z(k+1) << 16} pairs from wsz (one 128-column group of n per 256 B per k-step).
// OVL: trained values replace some of the dequantized weights (the reference's
// overlay scatter into the fp16 weights, usaf/moe_loader.py:218-221, 425-443).
// The entries of a k-step ride the code stream (one more DMA per thread and
// step, into the code stage).  As soon as a wave has dequantized fragment
// register j of the next k-step, it writes the register to a 1 KiB image in
// its epilogue tile, stores over it the values of its entries that fall in
// register j (one 16-bit LDS store by each of 16 lanes) and reads the register
// back, four such round trips spread over the k-step's MFMA regions: every
// weight the MFMAs see is then the trained value where an entry names it.
// SwiGLU forward: wave w holds gate rows n = 16 w + [0, 16) of the n-tile as
// its rows 0-15 and the up rows I + n as rows 16-31, so accumulator registers
// r and r + 8 of a lane are gate and up of the same column and slot.
// DW: dense 16-bit weights of the activation dtype instead of codes (the
// dequantized copies of the per-expert cache, expert e's [w_rows, w_cols]
// matrix at block weight_block(e) of w16).  Each weight element feeds exactly
// one lane, so the weights skip LDS: a lane loads its four fragment registers
// of k-step gs + 1 straight from global memory during k-step gs (one 16-byte
// load each), and the code stream's DMA slot instead touches the wave's
// weight lines of k-step gs + 3 (4 bytes per lane into a scratch word), which
// brings them into the cache hierarchy ahead of the register loads.
template <int EPI, int DT, bool BT, bool OVL, bool DW = false>
__global__ __launch_bounds__(Q_THREADS) void moe_gemm_q4_kernel(const GemmArgs g) {
  static_assert(!DW || (!BT && !OVL && EPI != EPI_SWIGLU_BWD), "dense weights: forward GEMMs without overlays");
  extern __shared__ __attribute__((aligned(16))) uint8_t qsm[];
  __shared__ __attribute__((aligned(16))) uint16_t q_ep[Q_WAVES * Q_EP_ELEMS];
  __shared__ uint8_t q_mte[Q_MTE_CAP];  // expert of m-tile mt (when the list fits)
  int32_t* const s_h = reinterpret_cast<int32_t*>(qsm + Q_TAB_OFF);  // [Q_MAX_E + 1] heavy m-tile prefix
  int32_t* const s_l = s_h + Q_MAX_E + 1;                             // [Q_MAX_E + 1] light m-tile prefix
  int32_t* const s_off = s_l + Q_MAX_E + 1;                           // [Q_MAX_E + 1] expert offsets
  int32_t* const s_tok = reinterpret_cast<int32_t*>(qsm + Q_TOK_OFF); // [2][Q_BM] activation rows
  const uint32_t qsm_lds = (uint32_t)(uintptr_t)(lds_void_ptr)qsm;   // LDS address of the dynamic area (DMA targets)
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, half = lane >> 5;
  const int wave = uni(tid >> 6);
  const int E = g.E;
  const int nk = (int)(g.K / BK);  // even and >= 2: K % 128 == 0
  for (int e = tid; e <= E; e += Q_THREADS) s_off[e] = g.offsets[e];  // one global read of the offsets
  lds_barrier();
  if (wave == 0) mtile_prefix_wave<Q_BM>(s_off, E, s_h, s_l, lane);
  lds_barrier();
  const int64_t n_nt = (EPI == EPI_SWIGLU_FWD) ? (g.inter + 127) / 128 : (g.N + Q_BN - 1) / Q_BN;
  // the tile counts come from LDS: readfirstlane tells the compiler they are
  // uniform, so that the stream state below lives in scalar registers
  const int n_heavy = uni(s_h[E]);
  const int n_mt = n_heavy + uni(s_l[E]);
  TileWalk walk(n_mt, n_nt);
  walk.set_heavy(n_heavy);
  const int n_grp = (int)(g.N / 128);  // BT: 128-column groups of n
  const int n_my = uni(walk.snake_count());
  if (n_my == 0) return;  // block-uniform
  // m-tile -> expert as a table (one LDS read per tile instead of a binary
  // search over the prefix tables, about seven dependent LDS reads), built
  // once; longer lists keep the search
  const bool mte = n_mt <= Q_MTE_CAP;
  if (mte) {  // expert e owns heavy m-tiles [s_h[e], s_h[e + 1]) and at most one light one
    for (int e = tid; e < E; e += Q_THREADS) {
      for (int mt = s_h[e]; mt < s_h[e + 1]; ++mt) q_mte[mt] = (uint8_t)e;
      if (s_l[e + 1] > s_l[e]) q_mte[n_heavy + s_l[e]] = (uint8_t)e;
    }
    lds_barrier();
  }
  const int nnt = (int)n_nt;  // n-tiles per m-tile (the unit arithmetic below is 32-bit)

  // tile ordinal -> expert, first slot, rows, n-tile (the m-tile list of
  // mtile_decode: every full-size tile before every light remainder; tables in LDS)
  // Odd blocks of a die walk their tiles in reverse, light remainders first: the
  // die's blocks then leave their tiles at two phases instead of all at once,
  // which halves the write burst of the epilogues.
  const bool rev = (walk.local_b & 1) != 0;
  auto decode = [&](int ord) {
    const int u = (int)walk.snake_unit(rev ? n_my - 1 - ord : ord);
    const int mi = u / nnt, nt = u - mi * nnt;
    const int mt = walk.xcd + walk.dies * mi;  // TileWalk::decode in 32 bits
    int e, j;
    if (mt < n_heavy) {
      e = mte ? (int)q_mte[mt] : prefix_owner(s_h, E, mt);
      j = mt - s_h[e];
    } else {
      e = mte ? (int)q_mte[mt] : prefix_owner(s_l, E, mt - n_heavy);
      j = (s_off[e + 1] - s_off[e] + Q_BM - 1) / Q_BM - 1;
    }
    QTile t;
    t.e = uni(e);
    t.m_beg = uni(s_off[t.e] + j * Q_BM);
    const int rem = s_off[t.e + 1] - t.m_beg;
    t.valid = uni(rem < Q_BM ? rem : Q_BM);
    t.nt = uni((int)nt);
    return t;
  };
  // weight row of tile row b (0..255); columns past N (or I) read row 0 and are never stored
  auto wrow = [&](const QTile& t, int b) -> int64_t {
    if constexpr (EPI == EPI_SWIGLU_FWD) {
      const int64_t n = (int64_t)t.nt * 128 + (b >> 5) * 16 + (b & 15);
      return n < g.inter ? ((b & 16) ? g.inter : 0) + n : 0;
    } else {
      const int64_t n = (int64_t)t.nt * Q_BN + b;
      return n < g.N ? n : 0;
    }
  };

  // ---- load streams.  Each DMA address is a wave-uniform base plus a 32-bit
  //      per-lane byte offset (the host checks that the operands fit) ----
  // scale|zero words of a k-step: one per weight row (4 waves' worth), or (BT)
  // 64 per 128-row group of n (two groups per tile: 2 waves' worth)
  constexpr int Z_WAVES = BT ? 2 : 4;
  // code stream: the codes of a k-step run one k-step ahead of its activations
  int c_ord = 0, c_kt = 0;
  uint32_t c_off = 0, z_off = 0;  // byte offsets of this thread's code chunk / scale|zero word at k-step 0
  QTile c_next;                   // the tile the code stream enters next
  // activation stream
  int a_ord = 0, a_kt = 0;
  bool a_enter = false;           // entered a new tile at the last advance: refresh a_off
  uint32_t a_off[Q_A_LOADS];      // byte offsets of this thread's chunks at k-step 0
  uint32_t o_off = 0;             // OVL: byte offset of this lane's entry word at k-step 0 of the code stream's tile
  const int a_lc = (tid & 7) ^ q_swz(tid >> 3);  // logical chunk of this thread's DMA slot
  const uint32_t lda_b = (uint32_t)g.lda * 2;
  // DW: expert blocks of the dense weight; within one block the offsets are 32-bit
  const uint64_t w_blk_bytes = (g.w_blk_elems ? (uint64_t)g.w_blk_elems : (uint64_t)g.w_rows * (uint64_t)g.w_cols) * 2u;
  // fragment order: the wave's four registers of one k-step are 4 KiB in a row
  // (register j at 1 KiB j, lane l at 16 l), its k-steps follow each other
  const uint32_t w_kstep_bytes = g.w_frag ? 4096u : (uint32_t)(BK * 2);
  auto w_block_base = [&](const QTile& t) -> const uint8_t* {
    const uint32_t blk = (uint32_t)uni((int)weight_block(g, t.e));  // clamped to [0, n_slots)
    return reinterpret_cast<const uint8_t*>(g.w16) + (uint64_t)blk * w_blk_bytes;
  };
  const uint8_t* c_wbase = nullptr;  // DW: weight block of the code stream's tile
  auto c_setup = [&](const QTile& t) {
    if constexpr (DW) {
      c_wbase = w_block_base(t);
      if (g.w_frag)  // lane l touches bytes [64 l, 64 l + 4) of the wave's 4 KiB
        c_off = (uint32_t)((((int64_t)t.nt * Q_WAVES + wave) * nk) * 4096) + 64u * (uint32_t)lane;
      else  // lane l touches row 32 wave + (l >> 1) of the wave, 64-byte half l & 1
        c_off = (uint32_t)(wrow(t, 32 * wave + (lane >> 1)) * g.K * 2) + 64u * (uint32_t)(lane & 1);
      return;
    }
    const int64_t base = (int64_t)t.e * g.w_rows;
    c_off = (uint32_t)((((base + wrow(t, tid >> 1)) * g.K) >> 1) + 16 * (tid & 1));
    if constexpr (OVL) {
      // entries of tile unit ((e * n_nt + nt) * 8 + wave): nk groups of 64 words
      const uint32_t unit = (uint32_t)(((int64_t)t.e * n_nt + t.nt) * Q_WAVES + wave);
      o_off = unit * (uint32_t)nk * (Q_OVL_WORDS * 4) + (uint32_t)lane * 4;
    }
    if constexpr (BT) {
      // thread t fetches word t & 63 of group (tile's first group + ((t >> 6) & 1))
      int grp = t.nt * (Q_BN / 128) + ((tid >> 6) & 1);
      grp = grp < n_grp ? grp : n_grp - 1;
      z_off = (uint32_t)((((int64_t)t.e * n_grp + grp) * (g.K / 2) * 2 + (tid & 63)) * 4);
    } else {
      z_off = (uint32_t)((((base + wrow(t, tid & 255)) * g.K) >> 7) * 4);
    }
  };
  // with a row map, the activation rows of tile t are fetched into token buffer
  // buf by a DMA of waves 0-3 (visible to all threads after the next barrier);
  // without one the row is the slot itself
  auto tok_fill = [&](const QTile& t, int buf) {
    if (g.a_rows && wave < 4) {
      const int r = tid < t.valid ? tid : t.valid - 1;
      // (buf can come out of a vector register: readfirstlane puts the address in a scalar one)
      dma4(g.a_rows + t.m_beg, (uint32_t)r * 4, (uint32_t)uni((int)(qsm_lds + Q_TOK_OFF + (buf * Q_BM + wave * 64) * 4)));
    }
  };
  auto a_refresh = [&](int ord) {
    if (g.a_rows) {
      const int32_t* src = s_tok + (ord & 1) * Q_BM;
#pragma unroll
      for (int c = 0; c < Q_A_LOADS; ++c) a_off[c] = (uint32_t)src[64 * c + (tid >> 3)] * lda_b + a_lc * 16;
    } else {
      const QTile t = decode(ord);
#pragma unroll
      for (int c = 0; c < Q_A_LOADS; ++c) {
        const int r = 64 * c + (tid >> 3);
        a_off[c] = (uint32_t)(t.m_beg + (r < t.valid ? r : t.valid - 1)) * lda_b + a_lc * 16;
      }
    }
  };
  // one DMA instruction of a k-step (d as for Q_DMAS): codes, scale|zero and
  // entries into stage sc_stage, activations into stage sa_stage
  auto dma_one = [&](int d, int sc_stage, int sa_stage) {
    sc_stage = uni(sc_stage);
    sa_stage = uni(sa_stage);
    const int c_kt_u = uni(c_kt), a_kt_u = uni(a_kt);
    const uint32_t sc = qsm_lds + sc_stage * Q_STAGE + Q_A_BYTES;
    if constexpr (DW) {
      // d = 0: the weight lines of the code stream's k-step, into the wave's
      // scratch words in the (unused) code area; d = 1..: activation chunks
      if (d == 0) {
        dma4_vb(uni_ptr(c_wbase + (uint32_t)c_kt_u * w_kstep_bytes), c_off, sc + wave * 256);
      } else {
        const int c = d - 1;
        const uint8_t* base = reinterpret_cast<const uint8_t*>(g.A) + a_kt_u * (BK * 2);
        dma16(base, a_off[c], qsm_lds + sa_stage * Q_STAGE + (c * Q_THREADS + wave * 64) * 16);
      }
      return;
    }
    if (OVL && d == Q_DMAS) {
      const uint8_t* base = reinterpret_cast<const uint8_t*>(g.ovl) + c_kt_u * (Q_OVL_WORDS * 4);
      dma4(base, o_off, sc + Q_C_BYTES + Q_Z_BYTES + wave * (Q_OVL_WORDS * 4));
    } else if (d == 0) {
      // per k-step: one scale|zero word per weight row, or (BT) 32 k-pairs x 2 words
      // per group; the waves past Z_WAVES fetch the same words to the same place
      // (a branch here would split the step's schedule)
      const uint8_t* base = reinterpret_cast<const uint8_t*>(g.wsz) + (BT ? c_kt_u * 256 : (c_kt_u >> 1) * 4);
      dma4(base, z_off, sc + Q_C_BYTES + (wave & (Z_WAVES - 1)) * 256);
    } else if (d == 1) {
      const uint8_t* base = reinterpret_cast<const uint8_t*>(g.wq) + c_kt_u * 32;
      dma16(base, c_off, sc + wave * 64 * 16);
    } else {
      const int c = d - 2;
      const uint8_t* base = reinterpret_cast<const uint8_t*>(g.A) + a_kt_u * (BK * 2);
      dma16(base, a_off[c], qsm_lds + sa_stage * Q_STAGE + (c * Q_THREADS + wave * 64) * 16);
    }
  };
  // start of a k-step: the activation stream picks up the rows of the tile it
  // entered (their DMA landed before the last barrier); when the code stream is
  // about to enter a new tile, fetch that tile's activation rows now, ahead of
  // this k-step's DMAs
  auto pre_step = [&]() {
    if (a_enter) {
      a_refresh(a_ord);
      a_enter = false;
    }
    if (c_kt == nk - 1 && c_ord + 1 < n_my) {
      c_next = decode(c_ord + 1);
      tok_fill(c_next, (c_ord + 1) & 1);
    }
  };
  // DW register-load stream: the weight fragments of k-step r_kt of tile
  // r_ord, one k-step ahead of the MFMAs (r_base: the tile's weight block;
  // r_off: this lane's row and half within it)
  int r_ord = 0, r_kt = 0;
  const uint8_t* r_base = nullptr;
  uint32_t r_off = 0;
  auto r_setup = [&](const QTile& t) {
    r_base = w_block_base(t);
    if (g.w_frag)
      r_off = (uint32_t)((((int64_t)t.nt * Q_WAVES + wave) * nk) * 4096) + 16u * (uint32_t)lane;
    else
      r_off = (uint32_t)(wrow(t, 32 * wave + l32) * g.K * 2) + 64u * (uint32_t)half;
  };
  // end of a k-step: advance both streams (past the last tile they repeat the
  // last k-step into a stage nobody reads).  The stream state goes through
  // readfirstlane: it is uniform, and the compiler then keeps it in scalar
  // registers and branches on it with scalar branches.
  // DW: the r stream moves one k-step per k-step of the MFMAs (and once in the
  // prologue, after k-step 0's load), independently of the DMA streams
  auto r_advance = [&]() {
    r_kt = uni(r_kt + 1);
    if (r_kt == nk) {
      if (r_ord + 1 < n_my) {
        r_ord = uni(r_ord + 1);
        r_kt = 0;
        r_setup(decode(r_ord));
      } else {
        r_kt = nk - 1;
      }
    }
  };
  auto advance = [&]() {
    c_kt = uni(c_kt + 1);
    if (c_kt == nk) {
      if (c_ord + 1 < n_my) {
        c_ord = uni(c_ord + 1);
        c_kt = 0;
        c_setup(c_next);
      } else {
        c_kt = nk - 1;
      }
    }
    a_kt = uni(a_kt + 1);
    if (a_kt == nk) {
      if (a_ord + 1 < n_my) {
        a_ord = uni(a_ord + 1);
        a_kt = 0;
        a_enter = true;
      } else {
        a_kt = nk - 1;
      }
    }
  };

  // ---- weight fragments: wf[set][sub-step j]; lane half h holds
  //      k = 32h + 8j + [0, 8) of weight row 32 wave + l32 ----
  u32x4 wf[2][4];
  // DW: the four fragment registers of the r stream's k-step into set BSX (one
  // 16-byte global load each, issued as asm so that no compiler wait drains
  // the DMAs in flight); the step's closing vmcnt wait covers them, and that
  // wait takes the registers as operands, so no use can move above it.  The
  // base comes out of readfirstlane (a VALU write of the SGPRs) and a VMEM
  // instruction may read such an SGPR only 5 wait states later; the compiler
  // does not look into the asm, so the asm supplies them (s_nop 4).
#define USAF_WLOAD(X, O1, O2, O3)                                                              \
  asm volatile("s_nop 4\n\t"                                                                    \
               "global_load_dwordx4 %0, %4, %5\n\t"                                             \
               "global_load_dwordx4 %1, %4, %5 offset:" #O1 "\n\t"                              \
               "global_load_dwordx4 %2, %4, %5 offset:" #O2 "\n\t"                              \
               "global_load_dwordx4 %3, %4, %5 offset:" #O3                                      \
               : "=&v"(wf[X][0]), "=&v"(wf[X][1]), "=&v"(wf[X][2]), "=&v"(wf[X][3])              \
               : "v"(woff), "s"(wbase))
#define USAF_WWAIT(X, N)                                                                       \
  asm volatile("s_waitcnt vmcnt(" #N ")\n\ts_barrier"                                          \
               : "+v"(wf[X][0]), "+v"(wf[X][1]), "+v"(wf[X][2]), "+v"(wf[X][3])::"memory")
  auto wload = [&](int set) {
    const uint8_t* wbase = uni_ptr(r_base + (uint32_t)uni(r_kt) * w_kstep_bytes);
    const uint32_t woff = r_off;
    if (g.w_frag) {  // registers 1 KiB apart
      if (set == 0) USAF_WLOAD(0, 1024, 2048, 3072);
      else USAF_WLOAD(1, 1024, 2048, 3072);
    } else {  // 16 bytes apart within the row's k-step
      if (set == 0) USAF_WLOAD(0, 16, 32, 48);
      else USAF_WLOAD(1, 16, 32, 48);
    }
  };
  // the step's closing wait (vmcnt(5): all but its 5 DMAs) and barrier, with set `set` as operands
  auto wwait5 = [&](int set) {
    if (set == 0) USAF_WWAIT(0, 5);
    else USAF_WWAIT(1, 5);
  };
  auto wwait0 = [&](int set) {
    if (set == 0) USAF_WWAIT(0, 0);
    else USAF_WWAIT(1, 0);
  };
#undef USAF_WLOAD
#undef USAF_WWAIT
  // per-lane LDS byte offsets within a stage (the stage offset is uniform):
  // activation fragment j of slot block i at fb_j + 4096 i (the swizzle of row
  // 32 i + l32 does not depend on i), the lane's codes, its scale|zero word
  uint32_t fb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) fb[j] = (uint32_t)(128 * l32 + 16 * ((4 * half + j) ^ q_swz(l32)));
  const uint32_t cb_off = (uint32_t)(Q_A_BYTES + (2 * (32 * wave + l32) + half) * 16);
  const uint32_t zb_off = (uint32_t)(Q_A_BYTES + Q_C_BYTES + (32 * wave + l32) * 4);
  // codes of the lane's weight row and its scale|zero: one pair per row, or
  // (BT) the 16 k-pairs {s2, z2} of k = 32 half + [0, 32) of the wave's group
  // (a wave's 32 rows never straddle a 128-row group)
  auto codes_read = [&](int stage, u32x4& cq, uint32_t& csz) {
    const uint8_t* st = qsm + stage * Q_STAGE;
    cq = *reinterpret_cast<const u32x4*>(st + cb_off);
    if constexpr (!BT) csz = *reinterpret_cast<const uint32_t*>(st + zb_off);
  };
  // BT: the k-pair words of fragment register wd (kz[2 wd], kz[2 wd + 1])
  auto kz_read = [&](int stage, int wd, u32x4 (&kz)[8]) {
    const uint8_t* zg = qsm + stage * Q_STAGE + Q_A_BYTES + Q_C_BYTES + ((wave >> 2) * 64 + 32 * half) * 4;
    kz[2 * wd] = *reinterpret_cast<const u32x4*>(zg + 32 * wd);
    kz[2 * wd + 1] = *reinterpret_cast<const u32x4*>(zg + 32 * wd + 16);
  };
  // k-pair p4 (= 4 wd + q, k = 32 half + 2 p4) of the BT words: {s2, z2}
  auto kz_pair = [&](const u32x4 (&kz)[8], int p4, f16x2& s2, f16x2& z2) {
    const u32x4 w = kz[p4 >> 1];
    s2 = __builtin_bit_cast(f16x2, (p4 & 1) ? w.z : w.x);
    z2 = __builtin_bit_cast(f16x2, (p4 & 1) ? w.w : w.y);
  };
  auto dequant_all = [&](auto bs_c, int stage) {
    constexpr int BS = decltype(bs_c)::value;
    u32x4 cq, kz[8];
    uint32_t csz = 0;
    codes_read(stage, cq, csz);
    if constexpr (BT) {
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) kz_read(stage, wd, kz);
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        f16x2 s2, z2;
        kz_pair(kz, p, s2, z2);
        wf[BS][p >> 2][p & 3] = dq_pair<DT>(cq[p >> 2], p & 3, s2, z2);
      }
    } else {
      const f16x2 s2 = __builtin_bit_cast(f16x2, (csz & 0xFFFFu) * 0x10001u);
      const f16x2 z2 = __builtin_bit_cast(f16x2, (csz >> 16) * 0x10001u);
#pragma unroll
      for (int j = 0; j < 4; ++j) wf[BS][j] = dq8<DT>(cq[j], s2, z2);
    }
  };

  // the wave's epilogue tile (also the overlay's fragment image during the k-steps)
  uint16_t* const sEp = q_ep + wave * Q_EP_ELEMS;
  const uint32_t sEp_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)sEp;

  // OVL: this lane's entry word of the wave's next k-step (stage `stage`)
  auto ovl_entry = [&](int stage) -> uint32_t {
    const uint8_t* ent = qsm + uni(stage) * Q_STAGE + Q_A_BYTES + Q_C_BYTES + Q_Z_BYTES + wave * (Q_OVL_WORDS * 4);
    return *reinterpret_cast<const uint32_t*>(ent + lane * 4);
  };
  // OVL: fragment register j of set BSX through the image: lane l's 16 bytes
  // at l * 16; lanes 16 j..16 j + 15 store their entry over it, the other lanes
  // store into the dummy area (a lane-mask select of the address, no exec
  // change), and the register is read back.  The stores are explicit ds_write
  // instructions (a compiler-visible LDS store would make it drain the DMAs in
  // flight first); the LDS operations of one wave complete in order, so the
  // read sees the stores before it.  a: LDS address of the lane's entry, d: its value.
  const uint32_t img_lds = sEp_lds + (uint32_t)lane * 16;
  const uint32_t dummy_lds = sEp_lds + Q_IMG + (uint32_t)lane * 2;
  const int my_j = lane >> 4;
  auto ovl_patch_j = [&](auto bsx_c, auto j_c, uint32_t a, uint32_t d) {
    constexpr int BSX = decltype(bsx_c)::value, J = decltype(j_c)::value;
    const uint32_t addr = my_j == J ? a : dummy_lds;
    asm volatile("ds_write_b128 %0, %1\n\tds_write_b16 %2, %3" ::"v"(img_lds), "v"(wf[BSX][J]), "v"(addr), "v"(d)
                 : "memory");
    wf[BSX][J] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(sEp) + lane * 16);
  };
  auto ovl_patch_wd = [&](auto bsx_c, int wd, uint32_t a, uint32_t d) {
    switch (wd) {  // wd is a constant after unrolling: one case survives
      case 0: ovl_patch_j(bsx_c, std::integral_constant<int, 0>{}, a, d); break;
      case 1: ovl_patch_j(bsx_c, std::integral_constant<int, 1>{}, a, d); break;
      case 2: ovl_patch_j(bsx_c, std::integral_constant<int, 2>{}, a, d); break;
      default: ovl_patch_j(bsx_c, std::integral_constant<int, 3>{}, a, d); break;
    }
  };

  // ---- one k-step: MFMAs of k-step gs (activations in stage s0, weights in
  //      set BS) with the dequant of k-step gs + 1 (codes in stage s1) into
  //      set BS ^ 1; the k-step's DMAs (codes of gs + 3 into stage s0,
  //      activations of gs + 2 into stage s2) are spread over its regions ----
  constexpr int QD = DW ? 1 + Q_A_LOADS : Q_DMAS + (OVL ? 1 : 0);  // DMA instructions of a full step
  auto step = [&](auto bs_c, auto nrb_c, f32x16 (&acc)[decltype(nrb_c)::value], int s0, int s1, int s2) {
    constexpr int BS = decltype(bs_c)::value, NRB = decltype(nrb_c)::value;
    constexpr int NF = 4 * NRB;   // activation fragments = MFMAs, f = j * NRB + i
    constexpr int R = NF / 2;     // regions of two MFMAs
    constexpr int PF = 4;         // fragment prefetch distance
    constexpr int NP = 16;        // weight pairs per lane and k-step
    // Pair p goes to region 1 + p (R - 1) / NP and DMA d to region d R / QD:
    // spread evenly, so that every region holds about the same MFMA, VALU and
    // memory work and the two waves of a SIMD overlap them in any phase.
    auto rp = [](int p) { return 1 + p * (R - 1) / NP; };
    auto rd = [](int d) { return d * R / QD; };
    pre_step();
    // DW: next k-step's weight fragments, first of the step's memory operations
    if constexpr (DW) wload(BS ^ 1);
    u32x4 cq, kz[8];
    uint32_t csz = 0;
    if constexpr (!DW) codes_read(s1, cq, csz);
    // BT: the words of register wd are read one region before its first pair
    if constexpr (BT) kz_read(s1, 0, kz);
    uint32_t oa = 0, od = 0;
    if constexpr (OVL) {
      const uint32_t e = ovl_entry(s1);
      oa = sEp_lds + (e & 0xFFFFu);
      od = e >> 16;
    }
    const uint8_t* sa = qsm + s0 * Q_STAGE;
    auto frag = [&](int f) -> u32x4 {
      const int i = f % NRB, j = f / NRB;
      return *reinterpret_cast<const u32x4*>(sa + fb[j] + 4096 * i);
    };
    u32x4 af[NF];
#pragma unroll
    for (int f = 0; f < PF; ++f) af[f] = frag(f);
    f16x2 s2v = {}, z2v = {};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // The two waves of a SIMD run the same step; the older one wins every
      // issue tie and would finish the step far ahead, leaving the younger to
      // run the step's tail alone.  Each wave lowers its priority as it passes
      // the quarter marks of the step, so the leader yields to the other.
      if (r * 4 % R == 0) {
        switch (r * 4 / R) {  // a constant after unrolling
          case 0: __builtin_amdgcn_s_setprio(3); break;
          case 1: __builtin_amdgcn_s_setprio(2); break;
          case 2: __builtin_amdgcn_s_setprio(1); break;
          default: __builtin_amdgcn_s_setprio(0); break;
        }
      }
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int f = 2 * r + gg, i = f % NRB, j = f / NRB;
        if (f + PF < NF) af[f + PF] = frag(f + PF);
        acc[i] = mfma32<DT>(wf[BS][j], af[f], acc[i]);
      }
#pragma unroll
      for (int d = 0; d < QD; ++d)
        if (rd(d) == r) dma_one(d, s0, s2);
      if constexpr (BT) {
#pragma unroll
        for (int wd = 1; wd < 4; ++wd)
          if (rp(4 * wd) - 1 == r) kz_read(s1, wd, kz);
      }
      if (!DW && r >= 1) {
        // this region's pairs p (half-word pair q = p & 3 of fragment register
        // wd = p >> 2), computed together (independent chains) and pinned here
        uint32_t v[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (rp(p) == r) {
            const int wd = p >> 2, q = p & 3;
            // the code word passes an empty asm here, so the pair's arithmetic
            // cannot be hoisted into an earlier region
            uint32_t cw = cq[wd];
            asm volatile("" : "+v"(cw));
            if constexpr (BT) {
              f16x2 s2, z2;
              kz_pair(kz, p, s2, z2);
              v[p] = dq_pair<DT>(cw, q, s2, z2);
            } else {
              if (p == 0) {
                s2v = __builtin_bit_cast(f16x2, (csz & 0xFFFFu) * 0x10001u);
                z2v = __builtin_bit_cast(f16x2, (csz >> 16) * 0x10001u);
              }
              v[p] = dq_pair<DT>(cw, q, s2v, z2v);
            }
          }
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (rp(p) == r) {
            const int wd = p >> 2, q = p & 3;
            asm volatile("" : "+v"(v[p]));  // computed here, next to the MFMAs, not sunk to its first use
            wf[BS ^ 1][wd][q] = v[p];
            // register wd complete: its trained values, now
            if constexpr (OVL) {
              if (q == 3) ovl_patch_wd(std::integral_constant<int, BS ^ 1>{}, wd, oa, od);
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    advance();
    if constexpr (DW) r_advance();
    // this step's QD DMAs may stay in flight; everything older (the stages the
    // next step reads, the token rows) has landed in this wave, and after the
    // barrier in all waves.  sched_barrier keeps the step's register work on
    // its side of the barrier.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DW) wwait5(BS ^ 1);  // the weight loads were issued before the step's 5 DMAs
    else if constexpr (OVL) asm volatile("s_waitcnt vmcnt(7)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(QD == (DW ? 5 : OVL ? 7 : 6), "the step's vmcnt wait counts its DMAs");

  // ---- epilogue: per 32-slot block, the wave's dtype results go through its
  //      own LDS tile ([32 slots][Q_EPW]) and out as 16-byte row stores ----
  // lane's accumulator values r = 4q..4q+3 -> columns 8q + 4half + [0,4) of slot l32.
  // Written with an explicit ds_write_b64: the compiler would otherwise drain
  // every DMA in flight (the next tile's first k-steps) before an LDS store.
  // The wave's own LDS operations complete in order, so the reads below see it.
  auto stage4 = [&](int col, uint32_t lo, uint32_t hi) {
    const uint32_t addr = sEp_lds + (uint32_t)(l32 * Q_EPW + col) * 2;
    const uint64_t v = (uint64_t)lo | ((uint64_t)hi << 32);
    asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(v) : "memory");
  };
  auto epilogue = [&](auto nrb_c, f32x16 (&acc)[decltype(nrb_c)::value], const QTile& t) {
    constexpr int NRB = decltype(nrb_c)::value;
    if constexpr (EPI == EPI_SWIGLU_FWD) {
      // staging columns: gate [0, 16), up [16, 32), act [32, 48) of the wave's 16 n
      const int64_t n0 = (int64_t)t.nt * 128 + wave * 16;
      if (n0 >= g.inter) return;  // I % 16 == 0
      // blocked act^T: the expert's block holds, per feature n, ld = round_up(se, 16)
      // slots (zero past se); tblk points at feature n0's row of it
      uint16_t* tblk = nullptr;
      int jt = 0, se = 0, ld = 0;
      if (g.out_t) {  // wave-uniform
        const int s0 = s_off[t.e];
        se = s_off[t.e + 1] - s0;
        ld = (se + 15) & ~15;
        jt = t.m_beg - s0;
        tblk = g.out_t + g.inter * (int64_t)g.blk_table[t.e] + n0 * (int64_t)ld;
      }
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        if (32 * i >= t.valid) break;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          uint32_t gb[2], ub[2], ab[2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            gb[h2] = pack2<DT>(acc[i][4 * q + 2 * h2], acc[i][4 * q + 2 * h2 + 1]);
            ub[h2] = pack2<DT>(acc[i][8 + 4 * q + 2 * h2], acc[i][8 + 4 * q + 2 * h2 + 1]);
            const f32x2 gf = unpack2<DT>(gb[h2]), uf = unpack2<DT>(ub[h2]);
            const f32x2 sf = unpack2<DT>(pack2<DT>(silu_fast(gf.x), silu_fast(gf.y)));
            ab[h2] = pack2<DT>(sf.x * uf.x, sf.y * uf.y);
          }
          const int col = 8 * q + 4 * half;
          stage4(col, gb[0], gb[1]);
          stage4(16 + col, ub[0], ub[1]);
          stage4(32 + col, ab[0], ab[1]);
        }
        // gate and up: 32 rows x 2 x 32 B; lane l takes row (l >> 2) + 16p,
        // gate or up by bit 1, 16-byte chunk l & 1
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int rr = (lane >> 2) + 16 * p;
          if (32 * i + rr < t.valid) {
            const int64_t m = t.m_beg + 32 * i + rr;
            const int part = (lane >> 1) & 1, ch = (lane & 1) * 8;
            const u32x4 v = *reinterpret_cast<const u32x4*>(sEp + rr * Q_EPW + 16 * part + ch);
            *reinterpret_cast<u32x4*>(g.out2 + m * g.ldo2 + (part ? g.inter : 0) + n0 + ch) = v;
          }
        }
        // act: 32 rows x 32 B; lane l takes row l >> 1, chunk l & 1
        {
          const int rr = lane >> 1;
          if (32 * i + rr < t.valid) {
            const int64_t m = t.m_beg + 32 * i + rr;
            const int ch = (lane & 1) * 8;
            *reinterpret_cast<u32x4*>(g.out + m * g.ldo + n0 + ch) =
                *reinterpret_cast<const u32x4*>(sEp + rr * Q_EPW + 32 + ch);
          }
        }
        if (tblk) {
          // the staged act columns read down the slots: lane l is feature l >> 2,
          // slots 8 (l & 3) + [0, 8) of block i, one 16-byte store; slots at or
          // past se (padding up to ld) are zero
          const int f = lane >> 2, sg = lane & 3;
          const int j = jt + 32 * i + 8 * sg;
          if (j < ld) {
            // all eight staged values are read (rows 8 sg .. 8 sg + 7 of the
            // 32-row tile: in bounds), back to back under one wait; the slots
            // past se become zero by selects, not by skipped reads
            uint32_t v[8], w[4];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = sEp[(8 * sg + k) * Q_EPW + 32 + f];
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
              const uint32_t lo = j + 2 * k2 < se ? v[2 * k2] : 0u;
              const uint32_t hi = j + 2 * k2 + 1 < se ? v[2 * k2 + 1] : 0u;
              w[k2] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x4*>(tblk + f * (int64_t)ld + j) = u32x4{w[0], w[1], w[2], w[3]};
          }
        }
      }
    } else if constexpr (EPI == EPI_SWIGLU_BWD) {
      // acc = d(act) for columns n of [0, I): with the saved gu (g = gate, u = up),
      //   d(up)   = DT(da * DT(silu(g)))
      //   d(gate) = DT(DT(da * u) * sig * (1 + g (1 - sig))),  da = DT(acc), sig = sigmoid(g)
      // into dgu[m, n] and dgu[m, I + n].  da goes through the LDS tile; the
      // math then runs on 16-byte row chunks (8 columns) next to coalesced gu
      // loads and dgu stores, in a loop that is not unrolled (code size).  The
      // units (row block i, half p) run in order, and the gu chunks of the next
      // unit are loaded before the current unit's math, so that their latency
      // hides behind it.
      const int64_t n0 = (int64_t)t.nt * Q_BN + wave * 32;
      if (n0 >= g.N) return;  // N % 32 == 0
      const int ch = (lane & 3) * 8;
      auto gu_row = [&](int u) -> const uint16_t* {  // this lane's gate chunk of unit u, or null
        const int rr = 32 * (u >> 1) + (lane >> 2) + 16 * (u & 1);
        return rr < t.valid ? g.aux + ((int64_t)t.m_beg + rr) * g.ld_aux + n0 + ch : nullptr;
      };
      u32x4 gn = {}, un = {};
      if (const uint16_t* r0 = gu_row(0)) {
        gn = *reinterpret_cast<const u32x4*>(r0);
        un = *reinterpret_cast<const u32x4*>(r0 + g.inter);
      }
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        if (32 * i >= t.valid) break;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          stage4(8 * q + 4 * half, pack2<DT>(acc[i][4 * q], acc[i][4 * q + 1]),
                 pack2<DT>(acc[i][4 * q + 2], acc[i][4 * q + 3]));
#pragma unroll 1
        for (int p = 0; p < 2; ++p) {
          const int u = 2 * i + p;
          const u32x4 gv = gn, uv = un;
          if (u + 1 < 2 * NRB) {
            if (const uint16_t* rn = gu_row(u + 1)) {
              gn = *reinterpret_cast<const u32x4*>(rn);
              un = *reinterpret_cast<const u32x4*>(rn + g.inter);
            }
          }
          const int rr = (lane >> 2) + 16 * p;
          if (32 * i + rr < t.valid) {
            const int64_t m = t.m_beg + 32 * i + rr;
            const u32x4 dv = *reinterpret_cast<const u32x4*>(sEp + rr * Q_EPW + ch);
            uint32_t dgw[4], duw[4];
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) {
              // the two roundings to DT per element go through the pair
              // conversion (round to nearest even, as round_to) and back
              const f32x2 da = unpack2<DT>(dv[w2]), gt = unpack2<DT>(gv[w2]), up = unpack2<DT>(uv[w2]);
              const float s0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * gt.x));
              const float s1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * gt.y));
              const f32x2 sg = unpack2<DT>(pack2<DT>(gt.x * s0, gt.y * s1));
              const f32x2 dsil = unpack2<DT>(pack2<DT>(da.x * up.x, da.y * up.y));
              dgw[w2] = pack2<DT>((dsil.x * s0) * (1.0f + gt.x * (1.0f - s0)), (dsil.y * s1) * (1.0f + gt.y * (1.0f - s1)));
              duw[w2] = pack2<DT>(da.x * sg.x, da.y * sg.y);
            }
            *reinterpret_cast<u32x4*>(g.out + m * g.ldo + n0 + ch) = u32x4{dgw[0], dgw[1], dgw[2], dgw[3]};
            *reinterpret_cast<u32x4*>(g.out + m * g.ldo + g.inter + n0 + ch) = u32x4{duw[0], duw[1], duw[2], duw[3]};
          }
        }
      }
    } else {
      const int64_t n0 = (int64_t)t.nt * Q_BN + wave * 32;
      if (n0 >= g.N) return;  // N % 32 == 0: a wave's 32 columns are all valid or none
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        if (32 * i >= t.valid) break;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          stage4(8 * q + 4 * half, pack2<DT>(acc[i][4 * q], acc[i][4 * q + 1]),
                 pack2<DT>(acc[i][4 * q + 2], acc[i][4 * q + 3]));
        // 32 rows x 64 B: lane l takes 16-byte chunk l & 3 of row (l >> 2) + 16p
        // (a wave-uniform row base plus one 32-bit lane offset)
        uint8_t* const rowbase = reinterpret_cast<uint8_t*>(g.out + ((int64_t)t.m_beg + 32 * i) * g.ldo + n0);
        const uint32_t loff = (uint32_t)(((lane >> 2) * g.ldo + (lane & 3) * 8) * 2);
        const int rows_left = t.valid - 32 * i;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int rr = (lane >> 2) + 16 * p;
          if (rr < rows_left)
            *reinterpret_cast<u32x4*>(rowbase + (size_t)p * 32 * g.ldo + loff) =
                *reinterpret_cast<const u32x4*>(sEp + rr * Q_EPW + (lane & 3) * 8);
        }
      }
    }
  };

  using std::integral_constant;
  using I0 = integral_constant<int, 0>;
  using I1 = integral_constant<int, 1>;

  // ---- prologue: rows of tile 0, codes of k-steps 0..2, activations of k-steps 0..1;
  //      afterwards the code stream stands at k-step 3 and the activation stream at 2 ----
  {
    const QTile t0 = decode(0);
    c_setup(t0);
    if constexpr (DW) r_setup(t0);
    tok_fill(t0, 0);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    a_refresh(0);
  }
  dma_one(0, 0, 0);                            // codes 0: scale|zero (DW: the weight lines of k-step 0)
  if constexpr (!DW) dma_one(1, 0, 0);         // codes 0
  if constexpr (OVL) dma_one(Q_DMAS, 0, 0);    // their entries
  if (nk == 2 && n_my > 1) {                   // the code stream enters tile 1 after codes 1
    c_next = decode(1);
    tok_fill(c_next, 1);
  }
  if (++c_kt == nk) {
    if (c_ord + 1 < n_my) {
      ++c_ord;
      c_kt = 0;
      c_setup(c_next);
    } else {
      c_kt = nk - 1;
    }
  }
  for (int d = 0; d < QD; ++d) dma_one(d, 1, 0);  // codes (and entries) 1, activations 0
  advance();
  pre_step();
  for (int d = 0; d < QD; ++d) dma_one(d, 2, 1);  // codes (and entries) 2, activations 1
  advance();
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (DW) {
    // k-step 0's weight fragments; the r stream then stands at k-step 1
    wload(0);
    wwait0(0);
    r_advance();
  } else {
    dequant_all(I0{}, 0);
  }
  if constexpr (OVL) {  // k-step 0: its entries are in stage 0
    const uint32_t e = ovl_entry(0);
    const uint32_t a = sEp_lds + (e & 0xFFFFu), d = e >> 16;
    ovl_patch_j(I0{}, integral_constant<int, 0>{}, a, d);
    ovl_patch_j(I0{}, integral_constant<int, 1>{}, a, d);
    ovl_patch_j(I0{}, integral_constant<int, 2>{}, a, d);
    ovl_patch_j(I0{}, integral_constant<int, 3>{}, a, d);
  }
  asm volatile("s_barrier" ::: "memory");  // stage 0's codes are refilled by k-step 0

  // ---- tiles ----
  int s0 = 0;  // stage of the current k-step
  for (int ord = 0; ord < n_my; ++ord) {
    const QTile t = decode(ord);
    const int nrb = (t.valid + 31) >> 5;
    auto run = [&](auto nrb_c) {
      constexpr int NRB = decltype(nrb_c)::value;
      f32x16 acc[NRB];
#pragma unroll
      for (int i = 0; i < NRB; ++i) acc[i] = f32x16{};
      for (int kt = 0; kt < nk; kt += 2) {
        int s1 = uni(s0 == 2 ? 0 : s0 + 1), s2 = uni(s1 == 2 ? 0 : s1 + 1);
        step(I0{}, nrb_c, acc, s0, s1, s2);
        s0 = s1;
        s1 = s2;
        s2 = uni(s2 == 2 ? 0 : s2 + 1);
        step(I1{}, nrb_c, acc, s0, s1, s2);
        s0 = s1;
      }
      epilogue(nrb_c, acc, t);
    };
    if (nrb > 6) run(integral_constant<int, 8>{});
    else if (nrb > 4) run(integral_constant<int, 6>{});
    else if (nrb > 2) run(integral_constant<int, 4>{});
    else run(integral_constant<int, 2>{});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // drain the trailing DMAs before the wave ends
}

// The dynamic-LDS limit of each kernel instantiation is raised once per
// process, before its first launch: each *_prepare() holds a function-local
// static whose initializer C++11 runs exactly once even under concurrent first
// calls (the reference's prefetch thread), and usaf_hip_init() runs them all
// up front for callers that must not make such calls later (stream capture).
// A runtime that does not need (or know) the attribute may refuse it; the
// launch reports any real problem.
bool raise_lds_limit(const void* kernel, size_t bytes) {
  (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  (void)hipGetLastError();
  return true;
}

template <int EPI, int BQ, int DT>
void nk_prepare() {
  static const bool done = raise_lds_limit(reinterpret_cast<const void*>(&moe_gemm_nk_kernel<EPI, BQ, DT>), kNkSmemBytes);
  (void)done;
}

template <int EPI, int BQ, int DT>
int launch_nk_one(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  nk_prepare<EPI, BQ, DT>();
  moe_gemm_nk_kernel<EPI, BQ, DT><<<blocks, NK_THREADS, kNkSmemBytes, st>>>(g);
  return USAF_OK;
}

template <int EPI, int DT, bool BT, bool OVL, bool DW = false>
void q4_prepare() {
  static const bool done =
      raise_lds_limit(reinterpret_cast<const void*>(&moe_gemm_q4_kernel<EPI, DT, BT, OVL, DW>), kQSmemBytes);
  (void)done;
}

// dense 16-bit weights on the LDS-DMA kernel (DW)
template <int EPI, int DT>
int launch_dw_one(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  q4_prepare<EPI, DT, false, false, true>();
  moe_gemm_q4_kernel<EPI, DT, false, false, true><<<blocks, Q_THREADS, kQSmemBytes, st>>>(g);
  return USAF_OK;
}

template <int EPI, int DT, bool BT = false>
int launch_q4_one(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  if (g.ovl) {
    q4_prepare<EPI, DT, BT, true>();
    moe_gemm_q4_kernel<EPI, DT, BT, true><<<blocks, Q_THREADS, kQSmemBytes, st>>>(g);
  } else {
    q4_prepare<EPI, DT, BT, false>();
    moe_gemm_q4_kernel<EPI, DT, BT, false><<<blocks, Q_THREADS, kQSmemBytes, st>>>(g);
  }
  return USAF_OK;
}

// Entry words of an overlay for this GEMM: 8 waves x (K / 64) k-steps x 64 per
// (expert, n-tile); the kernel addresses them with 32-bit byte offsets.
int64_t ovl_words(const GemmArgs& g, int epi) {
  const int64_t n_nt = epi == EPI_SWIGLU_FWD ? (g.inter + 127) / 128 : (g.N + Q_BN - 1) / Q_BN;
  return (int64_t)g.E * n_nt * Q_WAVES * (g.K / BK) * Q_OVL_WORDS;
}

int check_ovl(const GemmArgs& g, int epi, const char* what) {
  if (!g.ovl) return USAF_OK;
  if ((uintptr_t)g.ovl & 3) return set_error(USAF_ERR_INVALID, "%s: overlay entries must be 4-byte aligned", what);
  const int64_t need = ovl_words(g, epi);
  if (g.ovl_words < need)
    return set_error(USAF_ERR_INVALID, "%s: overlay table of %lld words, this GEMM reads %lld", what,
                     (long long)g.ovl_words, (long long)need);
  if (need * 4 >= ((int64_t)1 << 32)) return set_error(USAF_ERR_UNSUPPORTED, "%s: overlay table beyond 4 GiB", what);
  return USAF_OK;
}

// grad-input GEMMs on transposed 4-bit weights (always the LDS-DMA kernel)
template <int EPI>
int launch_q4t(const GemmArgs& g, int dt, int64_t max_tiles, int64_t a_rows_total, hipStream_t st, const char* what) {
  if (g.E > Q_MAX_E) return set_error(USAF_ERR_UNSUPPORTED, "%s: needs E <= %d", what, Q_MAX_E);
  if (((uintptr_t)g.A & 15) || g.lda % 8 != 0)
    return set_error(USAF_ERR_INVALID, "%s: activations must be 16-byte aligned rows", what);
  if (a_rows_total * g.lda * 2 >= ((int64_t)1 << 32) || (int64_t)g.E * g.w_rows * g.w_cols / 2 >= ((int64_t)1 << 32))
    return set_error(USAF_ERR_UNSUPPORTED, "%s: operands beyond 4 GiB", what);
  if (int rc = check_ovl(g, EPI, what)) return rc;
  int64_t blocks = (int64_t)device_cu_count();
  if (blocks > max_tiles) blocks = max_tiles;
  if (blocks < 1) blocks = 1;
  int rc;
  if (dt == USAF_BF16) rc = launch_q4_one<EPI, USAF_BF16, true>(g, (unsigned)blocks, st);
  else if (dt == USAF_F16) rc = launch_q4_one<EPI, USAF_F16, true>(g, (unsigned)blocks, st);
  else return set_error(USAF_ERR_INVALID, "%s: dtype must be fp16 or bf16", what);
  if (rc) return rc;
  return check_launch(what);
}

// 4-bit weights go to the LDS-DMA kernel when the activation rows are 16-byte
// aligned and the row and code offsets within one operand fit 32-bit byte offsets
bool q4_dma_ok(const GemmArgs& g, int64_t a_rows_total) {
  return g.w16 == nullptr && ((uintptr_t)g.A & 15) == 0 && g.lda % 8 == 0 && g.K % 128 == 0 && g.E <= Q_MAX_E &&
         a_rows_total * g.lda * 2 < ((int64_t)1 << 32) && (int64_t)g.E * g.w_rows * g.w_cols / 2 < ((int64_t)1 << 32);
}

// dense weights (one expert's block below 4 GiB, 16-byte aligned) on the same kernel (DW)
bool dw_dma_ok(const GemmArgs& g, int64_t a_rows_total) {
  const int64_t blk = g.w_blk_elems ? g.w_blk_elems : g.w_rows * g.w_cols;
  return g.w16 != nullptr && ((uintptr_t)g.w16 & 15) == 0 && ((uintptr_t)g.A & 15) == 0 && g.lda % 8 == 0 &&
         g.K % 128 == 0 && g.E <= Q_MAX_E && a_rows_total * g.lda * 2 < ((int64_t)1 << 32) && blk > 0 &&
         blk * 2 < ((int64_t)1 << 32) && g.w_cols == g.K;
}

template <int EPI>
int launch_gemm_nk(const GemmArgs& g, int dt, int64_t max_tiles, int64_t a_rows_total, hipStream_t st,
                   const char* what) {
  if (a_rows_total * g.lda >= ((int64_t)1 << 31))
    return set_error(USAF_ERR_UNSUPPORTED, "%s: activation operand of %lld x %lld elements exceeds 2^31", what,
                     (long long)a_rows_total, (long long)g.lda);
  int64_t blocks = (int64_t)device_cu_count();
  if (blocks > max_tiles) blocks = max_tiles;
  if (blocks < 1) blocks = 1;
  const bool dense = g.w16 != nullptr;
  const bool dma = q4_dma_ok(g, a_rows_total);
  if (g.ovl && !dma)
    return set_error(USAF_ERR_UNSUPPORTED,
                     "%s: an overlay needs the 4-bit LDS-DMA kernel (4-bit weights, 16-byte aligned activation rows, "
                     "K %% 128 == 0, E <= %d, operands below 4 GiB)", what, Q_MAX_E);
  if (int rc = check_ovl(g, EPI, what)) return rc;
  const bool dw = dense && dw_dma_ok(g, a_rows_total);
  int rc;
  if (dt == USAF_BF16)
    rc = dw ? launch_dw_one<EPI, USAF_BF16>(g, (unsigned)blocks, st)
         : dense ? launch_nk_one<EPI, BQ_DENSE16, USAF_BF16>(g, (unsigned)blocks, st)
         : dma ? launch_q4_one<EPI, USAF_BF16>(g, (unsigned)blocks, st)
               : launch_nk_one<EPI, BQ_Q4, USAF_BF16>(g, (unsigned)blocks, st);
  else if (dt == USAF_F16)
    rc = dw ? launch_dw_one<EPI, USAF_F16>(g, (unsigned)blocks, st)
         : dense ? launch_nk_one<EPI, BQ_DENSE16, USAF_F16>(g, (unsigned)blocks, st)
         : dma ? launch_q4_one<EPI, USAF_F16>(g, (unsigned)blocks, st)
               : launch_nk_one<EPI, BQ_Q4, USAF_F16>(g, (unsigned)blocks, st);
  else
    return set_error(USAF_ERR_INVALID, "%s: dtype must be fp16 or bf16", what);
  if (rc) return rc;
  return check_launch(what);
}

template <int BMODE, int EPI, int BQ, int DT>
void ws_prepare() {
  static const bool done = raise_lds_limit(reinterpret_cast<const void*>(&moe_gemm_kernel<BMODE, EPI, BQ, DT>), kSmemBytes);
  (void)done;
}

template <int BMODE, int EPI, int BQ, int DT>
int launch_one(const GemmArgs& g, unsigned blocks, hipStream_t st) {
  ws_prepare<BMODE, EPI, BQ, DT>();
  moe_gemm_kernel<BMODE, EPI, BQ, DT><<<blocks, kThreads, kSmemBytes, st>>>(g);
  return USAF_OK;
}

template <int BMODE, int EPI>
int launch_gemm(const GemmArgs& g, int dt, int64_t max_tiles, int64_t a_rows_total, hipStream_t st,
                const char* what) {
  // activation offsets are 32-bit inside the kernel
  if (a_rows_total * g.lda >= ((int64_t)1 << 31))
    return set_error(USAF_ERR_UNSUPPORTED, "%s: activation operand of %lld x %lld elements exceeds 2^31", what,
                     (long long)a_rows_total, (long long)g.lda);
  int64_t blocks = (int64_t)device_cu_count();
  if (blocks > max_tiles) blocks = max_tiles;
  if (blocks < 1) blocks = 1;
  const bool dense = g.w16 != nullptr;
  int rc;
  if (dt == USAF_BF16)
    rc = dense ? launch_one<BMODE, EPI, BQ_DENSE16, USAF_BF16>(g, (unsigned)blocks, st)
               : launch_one<BMODE, EPI, BQ_Q4, USAF_BF16>(g, (unsigned)blocks, st);
  else if (dt == USAF_F16)
    rc = dense ? launch_one<BMODE, EPI, BQ_DENSE16, USAF_F16>(g, (unsigned)blocks, st)
               : launch_one<BMODE, EPI, BQ_Q4, USAF_F16>(g, (unsigned)blocks, st);
  else
    return set_error(USAF_ERR_INVALID, "%s: dtype must be fp16 or bf16", what);
  if (rc) return rc;
  return check_launch(what);
}

int check_common(const char* what, int64_t S, int64_t E, const void* offsets, const void* wq, const void* wsz,
                 const void* w16) {
  if (E <= 0 || E > MAX_E) return set_error(USAF_ERR_INVALID, "%s: need 0 < E <= %d", what, MAX_E);
  if (S < 0) return set_error(USAF_ERR_INVALID, "%s: negative slot count", what);
  if (!offsets || (!w16 && (!wq || !wsz)))
    return set_error(USAF_ERR_INVALID, "%s: null pointer (offsets, and either codes + scale/zero pairs or the dense weight)", what);
  if (w16 && ((uintptr_t)w16 & 15)) return set_error(USAF_ERR_INVALID, "%s: dense weight must be 16-byte aligned", what);
  if (!w16 && ((uintptr_t)wq & 15)) return set_error(USAF_ERR_INVALID, "%s: codes must be 16-byte aligned", what);
  return USAF_OK;
}

template <int DT>
void prepare_dt() {
  nk_prepare<EPI_SWIGLU_FWD, BQ_Q4, DT>();
  nk_prepare<EPI_SWIGLU_FWD, BQ_DENSE16, DT>();
  nk_prepare<EPI_STORE, BQ_Q4, DT>();
  nk_prepare<EPI_STORE, BQ_DENSE16, DT>();
  q4_prepare<EPI_SWIGLU_FWD, DT, false, false>();
  q4_prepare<EPI_STORE, DT, false, false>();
  q4_prepare<EPI_SWIGLU_BWD, DT, true, false>();
  q4_prepare<EPI_STORE, DT, true, false>();
  q4_prepare<EPI_SWIGLU_FWD, DT, false, true>();
  q4_prepare<EPI_STORE, DT, false, true>();
  q4_prepare<EPI_SWIGLU_BWD, DT, true, true>();
  q4_prepare<EPI_STORE, DT, true, true>();
  q4_prepare<EPI_SWIGLU_FWD, DT, false, false, true>();
  q4_prepare<EPI_STORE, DT, false, false, true>();
  ws_prepare<BMODE_KN, EPI_SWIGLU_BWD, BQ_Q4, DT>();
  ws_prepare<BMODE_KN, EPI_SWIGLU_BWD, BQ_DENSE16, DT>();
  ws_prepare<BMODE_KN, EPI_STORE, BQ_Q4, DT>();
  ws_prepare<BMODE_KN, EPI_STORE, BQ_DENSE16, DT>();
}

}  // namespace

// Every kernel instantiation the GEMM entry points launch.
void prepare_gemm_kernels() {
  prepare_dt<USAF_F16>();
  prepare_dt<USAF_BF16>();
}

}  // namespace usaf

using namespace usaf;

// Forward gate_up + SwiGLU (qwen3moe_dml.py:58-60, per routed slot).
extern "C" int usaf_hip_moe_gate_up_fwd(const void* x, int64_t T_rows, int64_t H, const int32_t* token_idx, const int32_t* offsets,
                                        int64_t S, int64_t E, int64_t I, const int8_t* wq, const uint32_t* wsz,
                                        const void* w16, int32_t dtype, void* gu, void* act, void* act_blk,
                                        const int32_t* blk_table, const uint32_t* overlay, int64_t overlay_words,
                                        void* stream) {
  if (int rc = check_common("moe_gate_up_fwd", S, E, offsets, wq, wsz, w16)) return rc;
  if (H % 128 != 0 || H <= 0 || I % 32 != 0 || I <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_fwd: needs H %% 128 == 0 and I %% 32 == 0 (H=%lld, I=%lld)",
                     (long long)H, (long long)I);
  if (S == 0) return clear_error();
  if (!x || !token_idx || !gu || !act) return set_error(USAF_ERR_INVALID, "moe_gate_up_fwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)x; g.lda = H; g.a_rows = token_idx;
  g.wq = (const uint8_t*)wq; g.wsz = wsz; g.w16 = (const uint16_t*)w16; g.w_rows = 2 * I; g.w_cols = H;
  g.N = I; g.K = H; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)act; g.ldo = I; g.out2 = (uint16_t*)gu; g.ldo2 = 2 * I;
  g.ovl = overlay;
  g.ovl_words = overlay_words;
  if (act_blk && !blk_table) return set_error(USAF_ERR_INVALID, "moe_gate_up_fwd: act_blk needs blk_table");
  if (act_blk && ((uintptr_t)act_blk & 15)) return set_error(USAF_ERR_INVALID, "moe_gate_up_fwd: act_blk must be 16-byte aligned");
  // the 4-bit DMA kernel writes the blocked act^T from its epilogue; the other
  // kernels leave it to the blocked transpose of act afterwards
  const bool fused_t = act_blk && q4_dma_ok(g, T_rows);
  if (fused_t) {
    g.out_t = (uint16_t*)act_blk;
    g.blk_table = blk_table;
  }
  const int64_t max_tiles = (S / NK_BM + E) * ((I + 127) / 128);
  if (int rc = launch_gemm_nk<EPI_SWIGLU_FWD>(g, dtype, max_tiles, T_rows, as_stream(stream), "moe_gate_up_fwd")) return rc;
  if (act_blk && !fused_t)
    return usaf_hip_gather_transpose_blocked(act, I, nullptr, offsets, blk_table, S, E, I, act_blk, stream);
  return USAF_OK;
}

// Forward down projection (qwen3moe_dml.py:61): y[m] = act[m] @ W_down[e]^T.
extern "C" int usaf_hip_moe_down_fwd(const void* act, int64_t I, const int32_t* offsets, int64_t S, int64_t E,
                                     int64_t H, const int8_t* wq, const uint32_t* wsz,
                                     const void* w16, int32_t dtype, void* y, const uint32_t* overlay,
                                     int64_t overlay_words, void* stream) {
  if (int rc = check_common("moe_down_fwd", S, E, offsets, wq, wsz, w16)) return rc;
  if (I % 128 != 0 || I <= 0 || H % 64 != 0 || H <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_fwd: needs I %% 128 == 0 and H %% 64 == 0 (I=%lld, H=%lld)",
                     (long long)I, (long long)H);
  if (S == 0) return clear_error();
  if (!act || !y) return set_error(USAF_ERR_INVALID, "moe_down_fwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)act; g.lda = I; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq; g.wsz = wsz; g.w16 = (const uint16_t*)w16; g.w_rows = H; g.w_cols = I;
  g.N = H; g.K = I; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)y; g.ldo = H;
  g.ovl = overlay;
  g.ovl_words = overlay_words;
  const int64_t max_tiles = (S / NK_BM + E) * ((H + NK_BN - 1) / NK_BN);
  return launch_gemm_nk<EPI_STORE>(g, dtype, max_tiles, S, as_stream(stream), "moe_down_fwd");
}

// Forward gate_up + SwiGLU with dense weights held in a slot arena (usaf_amd's
// per-expert cache of dequantized copies): expert e's [2I, H] weight is block
// slot_of[e] of arena [n_slots, 2I, H].
extern "C" int usaf_hip_moe_gate_up_fwd_slots(const void* x, int64_t T_rows, int64_t H, const int32_t* token_idx,
                                              const int32_t* offsets, int64_t S, int64_t E, int64_t I,
                                              const void* arena, const int32_t* slot_of, int64_t n_slots,
                                              int32_t dtype, void* gu, void* act, void* stream) {
  if (int rc = check_common("moe_gate_up_fwd_slots", S, E, offsets, nullptr, nullptr, arena)) return rc;
  if (!slot_of || n_slots <= 0) return set_error(USAF_ERR_INVALID, "moe_gate_up_fwd_slots: needs slot_of and n_slots > 0");
  if (H % 128 != 0 || H <= 0 || I % 32 != 0 || I <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_fwd_slots: needs H %% 128 == 0 and I %% 32 == 0");
  if (S == 0) return clear_error();
  if (!x || !token_idx || !gu || !act) return set_error(USAF_ERR_INVALID, "moe_gate_up_fwd_slots: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)x; g.lda = H; g.a_rows = token_idx;
  g.w16 = (const uint16_t*)arena; g.w_slot = slot_of; g.n_slots = n_slots; g.w_rows = 2 * I; g.w_cols = H;
  g.N = I; g.K = H; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)act; g.ldo = I; g.out2 = (uint16_t*)gu; g.ldo2 = 2 * I;
  g.w_frag = 1;
  g.w_blk_elems = usaf_hip_frag_slot_elems(2 * I, H, I);
  if (!dw_dma_ok(g, T_rows))
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_fwd_slots: the fragment-order arena needs 16-byte aligned "
                                           "activation rows, H %% 128 == 0, E <= %d and blocks below 4 GiB", Q_MAX_E);
  const int64_t max_tiles = (S / NK_BM + E) * ((I + 127) / 128);
  return launch_gemm_nk<EPI_SWIGLU_FWD>(g, dtype, max_tiles, T_rows, as_stream(stream), "moe_gate_up_fwd_slots");
}

// Forward down projection with dense weights in a slot arena [n_slots, H, I].
extern "C" int usaf_hip_moe_down_fwd_slots(const void* act, int64_t I, const int32_t* offsets, int64_t S, int64_t E,
                                           int64_t H, const void* arena, const int32_t* slot_of, int64_t n_slots,
                                           int32_t dtype, void* y, void* stream) {
  if (int rc = check_common("moe_down_fwd_slots", S, E, offsets, nullptr, nullptr, arena)) return rc;
  if (!slot_of || n_slots <= 0) return set_error(USAF_ERR_INVALID, "moe_down_fwd_slots: needs slot_of and n_slots > 0");
  if (I % 128 != 0 || I <= 0 || H % 64 != 0 || H <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_fwd_slots: needs I %% 128 == 0 and H %% 64 == 0");
  if (S == 0) return clear_error();
  if (!act || !y) return set_error(USAF_ERR_INVALID, "moe_down_fwd_slots: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)act; g.lda = I; g.a_rows = nullptr;
  g.w16 = (const uint16_t*)arena; g.w_slot = slot_of; g.n_slots = n_slots; g.w_rows = H; g.w_cols = I;
  g.N = H; g.K = I; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)y; g.ldo = H;
  g.w_frag = 1;
  g.w_blk_elems = usaf_hip_frag_slot_elems(H, I, 0);
  if (!dw_dma_ok(g, S))
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_fwd_slots: the fragment-order arena needs 16-byte aligned "
                                           "activation rows, I %% 128 == 0, E <= %d and blocks below 4 GiB", Q_MAX_E);
  const int64_t max_tiles = (S / NK_BM + E) * ((H + NK_BN - 1) / NK_BN);
  return launch_gemm_nk<EPI_STORE>(g, dtype, max_tiles, S, as_stream(stream), "moe_down_fwd_slots");
}

// Backward through the down projection and SwiGLU: dgu[m] from dcur[m] @ W_down[e].
extern "C" int usaf_hip_moe_down_bwd(const void* dcur, int64_t H, const void* gu, const int32_t* offsets, int64_t S,
                                     int64_t E, int64_t I, const int8_t* wq, const uint32_t* wsz,
                                     const void* w16, int32_t dtype, void* dgu, void* stream) {
  if (int rc = check_common("moe_down_bwd", S, E, offsets, wq, wsz, w16)) return rc;
  if (I % 128 != 0 || I <= 0 || H % BK != 0 || H <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_bwd: needs I %% 128 == 0 and H %% 64 == 0 (I=%lld, H=%lld)",
                     (long long)I, (long long)H);
  if (S == 0) return clear_error();
  if (!dcur || !gu || !dgu) return set_error(USAF_ERR_INVALID, "moe_down_bwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)dcur; g.lda = H; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq; g.wsz = wsz; g.w16 = (const uint16_t*)w16; g.w_rows = H; g.w_cols = I;
  g.N = I; g.K = H; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)dgu; g.ldo = 2 * I; g.aux = (const uint16_t*)gu; g.ld_aux = 2 * I;
  const int64_t max_tiles = (S / BM + E) * (I / BN);
  return launch_gemm<BMODE_KN, EPI_SWIGLU_BWD>(g, dtype, max_tiles, S, as_stream(stream), "moe_down_bwd");
}

// Backward grad-input through gate_up: dx_slots[m] = dgu[m] @ W_gate_up[e].
extern "C" int usaf_hip_moe_gate_up_bwd(const void* dgu, int64_t I, const int32_t* offsets, int64_t S, int64_t E,
                                        int64_t H, const int8_t* wq, const uint32_t* wsz,
                                        const void* w16, int32_t dtype, void* dx_slots, void* stream) {
  if (int rc = check_common("moe_gate_up_bwd", S, E, offsets, wq, wsz, w16)) return rc;
  if (H % 128 != 0 || H <= 0 || (2 * I) % BK != 0 || I <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_bwd: needs H %% 128 == 0 and 2I %% 64 == 0 (H=%lld, I=%lld)",
                     (long long)H, (long long)I);
  if (S == 0) return clear_error();
  if (!dgu || !dx_slots) return set_error(USAF_ERR_INVALID, "moe_gate_up_bwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)dgu; g.lda = 2 * I; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq; g.wsz = wsz; g.w16 = (const uint16_t*)w16; g.w_rows = 2 * I; g.w_cols = H;
  g.N = H; g.K = 2 * I; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)dx_slots; g.ldo = H;
  const int64_t max_tiles = (S / BM + E) * (H / BN);
  return launch_gemm<BMODE_KN, EPI_STORE>(g, dtype, max_tiles, S, as_stream(stream), "moe_gate_up_bwd");
}

// dgu from dcur @ W_down[e] on the transposed copy W_down^T [E, I, H].
extern "C" int usaf_hip_moe_down_bwd_t(const void* dcur, int64_t H, const void* gu, const int32_t* offsets, int64_t S,
                                       int64_t E, int64_t I, const int8_t* wq_t, const uint32_t* wsz_t, int32_t dtype,
                                       void* dgu, const uint32_t* overlay, int64_t overlay_words, void* stream) {
  if (int rc = check_common("moe_down_bwd_t", S, E, offsets, wq_t, wsz_t, nullptr)) return rc;
  if (I % 128 != 0 || I <= 0 || H % 128 != 0 || H <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_bwd_t: needs I %% 128 == 0 and H %% 128 == 0 (I=%lld, H=%lld)",
                     (long long)I, (long long)H);
  if (S == 0) return clear_error();
  if (!dcur || !gu || !dgu) return set_error(USAF_ERR_INVALID, "moe_down_bwd_t: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)dcur; g.lda = H; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq_t; g.wsz = wsz_t; g.w16 = nullptr; g.w_rows = I; g.w_cols = H;
  g.N = I; g.K = H; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)dgu; g.ldo = 2 * I; g.aux = (const uint16_t*)gu; g.ld_aux = 2 * I;
  g.ovl = overlay;
  g.ovl_words = overlay_words;
  const int64_t max_tiles = (S / Q_BM + E) * ((I + Q_BN - 1) / Q_BN);
  return launch_q4t<EPI_SWIGLU_BWD>(g, dtype, max_tiles, S, as_stream(stream), "moe_down_bwd_t");
}

// dx_slots from dgu @ W_gate_up[e] on the transposed copy W_gate_up^T [E, H, 2I].
extern "C" int usaf_hip_moe_gate_up_bwd_t(const void* dgu, int64_t I, const int32_t* offsets, int64_t S, int64_t E,
                                          int64_t H, const int8_t* wq_t, const uint32_t* wsz_t, int32_t dtype,
                                          void* dx_slots, const uint32_t* overlay, int64_t overlay_words,
                                          void* stream) {
  if (int rc = check_common("moe_gate_up_bwd_t", S, E, offsets, wq_t, wsz_t, nullptr)) return rc;
  if (H % 128 != 0 || H <= 0 || I % 64 != 0 || I <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_bwd_t: needs H %% 128 == 0 and I %% 64 == 0 (H=%lld, I=%lld)",
                     (long long)H, (long long)I);
  if (S == 0) return clear_error();
  if (!dgu || !dx_slots) return set_error(USAF_ERR_INVALID, "moe_gate_up_bwd_t: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)dgu; g.lda = 2 * I; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq_t; g.wsz = wsz_t; g.w16 = nullptr; g.w_rows = H; g.w_cols = 2 * I;
  g.N = H; g.K = 2 * I; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)dx_slots; g.ldo = H;
  g.ovl = overlay;
  g.ovl_words = overlay_words;
  const int64_t max_tiles = (S / Q_BM + E) * ((H + Q_BN - 1) / Q_BN);
  return launch_q4t<EPI_STORE>(g, dtype, max_tiles, S, as_stream(stream), "moe_gate_up_bwd_t");
}
