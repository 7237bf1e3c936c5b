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
// Block: 256 threads = 4 waves in a 2x2 grid, tile BM x BN x BK = 128 x 128 x 64,
// each wave 64 x 64 (2 x 2 MFMA 32x32 tiles), two LDS stages.  The grid is
// persistent: block b walks tiles b, b + gridDim.x, ... of the device-side
// tile list (m-tiles of every expert x n-tiles), so no host sync is needed.
#include "common.h"

namespace usaf {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDSW = BK + 8;  // LDS row stride in 16-bit elements (16 B pad: conflict-free 128-bit reads)
constexpr int MAX_E = 1024;

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
  const uint16_t* ws;      // fp16 scales, one per 128 elements
  const uint16_t* wz;      // fp16 zeros
  const uint16_t* w16;     // dense 16-bit weight [E, w_rows, w_cols] (BQ == BQ_DENSE16)
  int64_t w_rows, w_cols;  // per-expert weight matrix
  int64_t N, K;            // output columns, contraction length
  int64_t inter;           // I (SwiGLU epilogues)
  const int32_t* offsets;  // [E+1]
  int E;
  uint16_t* out;  int64_t ldo;   // STORE: C; SWIGLU_FWD: act; SWIGLU_BWD: dgu
  uint16_t* out2; int64_t ldo2;  // SWIGLU_FWD: gu
  const uint16_t* aux; int64_t ld_aux;  // SWIGLU_BWD: saved gu
};

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

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

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

template <int BMODE, int EPI, int BQ, int DT>
__global__ __launch_bounds__(256, 2) void moe_gemm_kernel(const GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDSW];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDSW];
  __shared__ int32_t s_mt[MAX_E + 1];   // m-tile prefix over experts
  __shared__ int32_t s_part[256];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int E = g.E;

  // m-tile prefix: each thread owns a run of experts, then a block scan of the runs
  {
    const int per = (E + 255) / 256;
    const int e0 = tid * per;
    int local = 0;
    for (int i = 0; i < per; ++i) {
      const int e = e0 + i;
      if (e < E) local += (g.offsets[e + 1] - g.offsets[e] + BM - 1) / BM;
    }
    s_part[tid] = local;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int v = (tid >= off) ? s_part[tid - off] : 0;
      __syncthreads();
      s_part[tid] += v;
      __syncthreads();
    }
    int run = s_part[tid] - local;
    for (int i = 0; i < per; ++i) {
      const int e = e0 + i;
      if (e < E) {
        s_mt[e] = run;
        run += (g.offsets[e + 1] - g.offsets[e] + BM - 1) / BM;
      }
    }
    if (tid == 255) s_mt[E] = s_part[255];
    __syncthreads();
  }
  const int64_t n_mt = s_mt[E];
  const int64_t n_nt = (EPI == EPI_SWIGLU_FWD) ? g.N / 64 : g.N / BN;
  const int64_t n_tiles = n_mt * n_nt;
  const int nk = (int)(g.K / BK);
  const int64_t groups_per_row = g.w_cols / 128;

  for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
    const int64_t mt = tile / n_nt, nt = tile % n_nt;
    // expert of m-tile mt: largest e with s_mt[e] <= mt
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_mt[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    const int64_t m_beg = g.offsets[e] + (mt - s_mt[e]) * BM;
    const int64_t m_end = g.offsets[e + 1];
    const int64_t n0 = (EPI == EPI_SWIGLU_FWD) ? nt * 64 : nt * BN;
    const int64_t w_base = (int64_t)e * g.w_rows * g.w_cols;  // element offset of expert e

    // ---- per-thread global load coordinates ----
    // A: chunks c = tid + 256*i (i < 4) of 16 B: row c>>3, 8-element column block c&7
    const uint16_t* a_src[4];
    bool a_ok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int64_t m = m_beg + (c >> 3);
      a_ok[i] = m < m_end;
      const int64_t row = a_ok[i] ? (g.a_rows ? (int64_t)g.a_rows[m] : m) : 0;
      a_src[i] = g.A + row * g.lda + (c & 7) * 8;
    }
    // B (4-bit): one 16-byte code load per thread per k-tile, 32 codes of one group.
    // B (dense 16-bit): four 16-byte loads per thread per k-tile.
    int64_t b_elem = 0;   // element offset (within the whole tensor) of the thread's first B element at k0 = 0
    int64_t b_kstep = 0;  // element offset advance per k-tile
    if constexpr (BQ == BQ_Q4) {
      if constexpr (BMODE == BMODE_NK) {
        const int b = tid >> 1, half = tid & 1;
        const int64_t r = nk_weight_row<EPI>(b, n0, g.inter);
        b_elem = w_base + r * g.w_cols + half * 32;
        b_kstep = BK;
      } else {
        b_elem = w_base + (int64_t)lane * g.w_cols + n0 + wave * 32;
        b_kstep = (int64_t)BK * g.w_cols;
      }
    }
    const uint16_t* d_src[4];
    if constexpr (BQ == BQ_DENSE16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        if constexpr (BMODE == BMODE_NK) {  // tile row c>>3 (weight row), 8-element k block c&7
          const int64_t r = nk_weight_row<EPI>(c >> 3, n0, g.inter);
          d_src[i] = g.w16 + w_base + r * g.w_cols + (c & 7) * 8;
        } else {  // contraction row c>>4, 8-element n block c&15
          d_src[i] = g.w16 + w_base + (int64_t)(c >> 4) * g.w_cols + n0 + (c & 15) * 8;
        }
      }
      b_kstep = (BMODE == BMODE_NK) ? (int64_t)BK : (int64_t)BK * g.w_cols;
    }

    u32x4 ra[4];
    u32x4 rb;
    u32x4 rd[4];
    uint16_t rs = 0, rz = 0;
    auto load_tile = [&](int kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (a_ok[i]) ra[i] = *reinterpret_cast<const u32x4*>(a_src[i] + (int64_t)kt * BK);
        else ra[i] = u32x4{0, 0, 0, 0};
      }
      if constexpr (BQ == BQ_Q4) {
        const int64_t el = b_elem + (int64_t)kt * b_kstep;
        rb = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g.wq + (el >> 1)));
        const int64_t grp = el >> 7;  // groups are 128 consecutive elements of the flat tensor
        rs = g.ws[grp];
        rz = g.wz[grp];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) rd[i] = *reinterpret_cast<const u32x4*>(d_src[i] + (int64_t)kt * b_kstep);
      }
    };
    auto store_tile = [&](int st) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        *reinterpret_cast<u32x4*>(&sA[st][(c >> 3) * LDSW + (c & 7) * 8]) = ra[i];
      }
      if constexpr (BQ == BQ_Q4) {
        uint32_t o[16];
        dequant32<DT>(rb, rs, rz, o);
        if constexpr (BMODE == BMODE_NK) {
          const int b = tid >> 1, half = tid & 1;
          u32x4* dst = reinterpret_cast<u32x4*>(&sB[st][b * LDSW + half * 32]);
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[j] = u32x4{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
        } else {
          // transpose: code j of this thread is column wave*32 + j, contraction index lane
          uint16_t* dst = &sB[st][(wave * 32) * LDSW + lane];
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            dst[(2 * j) * LDSW] = (uint16_t)(o[j] & 0xFFFFu);
            dst[(2 * j + 1) * LDSW] = (uint16_t)(o[j] >> 16);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = tid + 256 * i;
          if constexpr (BMODE == BMODE_NK) {
            *reinterpret_cast<u32x4*>(&sB[st][(c >> 3) * LDSW + (c & 7) * 8]) = rd[i];
          } else {
            uint16_t* dst = &sB[st][((c & 15) * 8) * LDSW + (c >> 4)];
            const uint32_t w4[4] = {rd[i].x, rd[i].y, rd[i].z, rd[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              dst[(2 * j) * LDSW] = (uint16_t)(w4[j] & 0xFFFFu);
              dst[(2 * j + 1) * LDSW] = (uint16_t)(w4[j] >> 16);
            }
          }
        }
      }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        u32x4 fa[2], fb[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          fa[i] = *reinterpret_cast<const u32x4*>(
              &sA[cur][(wm * 64 + i * 32 + (lane & 31)) * LDSW + kk * 16 + (lane >> 5) * 8]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          fb[j] = *reinterpret_cast<const u32x4*>(
              &sB[cur][(wn * 64 + j * 32 + (lane & 31)) * LDSW + kk * 16 + (lane >> 5) * 8]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<DT>(fa[i], fb[j], acc[i][j]);
      }
      if (kt + 1 < nk) store_tile(cur ^ 1);
      __syncthreads();
    }

    // ---- epilogue: acc[i][j][r] is row wm*64 + i*32 + 8*(r/4) + 4*(lane/32) + r%4,
    //      column wn*64 + j*32 + lane%32 of the tile ----
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m_beg + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= m_end) continue;
        if constexpr (EPI == EPI_STORE) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
            store_from_f32<DT>(g.out, m * g.ldo + n, acc[i][j][r]);
          }
        } else if constexpr (EPI == EPI_SWIGLU_FWD) {
          const int64_t n = n0 + wn * 32 + (lane & 31);
          const float gt = round_to<DT>(acc[i][0][r]);
          const float up = round_to<DT>(acc[i][1][r]);
          store_from_f32<DT>(g.out2, m * g.ldo2 + n, gt);
          store_from_f32<DT>(g.out2, m * g.ldo2 + g.inter + n, up);
          const float sg = round_to<DT>(silu_f(gt));
          store_from_f32<DT>(g.out, m * g.ldo + n, sg * up);
        } else {  // EPI_SWIGLU_BWD
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
            const float da = round_to<DT>(acc[i][j][r]);
            const float gt = load_as_f32<DT>(g.aux, m * g.ld_aux + n);
            const float up = load_as_f32<DT>(g.aux, m * g.ld_aux + g.inter + n);
            const float sig = 1.0f / (1.0f + expf(-gt));
            const float sg = round_to<DT>(gt * sig);
            const float du = da * sg;
            const float dsil = round_to<DT>(da * up);
            const float dg = dsil * (sig * (1.0f + gt * (1.0f - sig)));
            store_from_f32<DT>(g.out, m * g.ldo + n, dg);
            store_from_f32<DT>(g.out, m * g.ldo + g.inter + n, du);
          }
        }
      }
    }
  }
}

template <int BMODE, int EPI>
int launch_gemm(const GemmArgs& g, int dt, int64_t max_tiles, hipStream_t st, const char* what) {
  int64_t blocks = (int64_t)device_cu_count() * 2;
  if (blocks > max_tiles) blocks = max_tiles;
  if (blocks < 1) blocks = 1;
  const bool dense = g.w16 != nullptr;
  if (dt == USAF_BF16) {
    if (dense) moe_gemm_kernel<BMODE, EPI, BQ_DENSE16, USAF_BF16><<<(unsigned)blocks, 256, 0, st>>>(g);
    else moe_gemm_kernel<BMODE, EPI, BQ_Q4, USAF_BF16><<<(unsigned)blocks, 256, 0, st>>>(g);
  } else if (dt == USAF_F16) {
    if (dense) moe_gemm_kernel<BMODE, EPI, BQ_DENSE16, USAF_F16><<<(unsigned)blocks, 256, 0, st>>>(g);
    else moe_gemm_kernel<BMODE, EPI, BQ_Q4, USAF_F16><<<(unsigned)blocks, 256, 0, st>>>(g);
  } else {
    return set_error(USAF_ERR_INVALID, "%s: dtype must be fp16 or bf16", what);
  }
  return check_launch(what);
}

int check_common(const char* what, int64_t S, int64_t E, const void* offsets, const void* wq, const void* ws,
                 const void* wz, const void* w16) {
  if (E <= 0 || E > MAX_E) return set_error(USAF_ERR_INVALID, "%s: need 0 < E <= %d", what, MAX_E);
  if (S < 0) return set_error(USAF_ERR_INVALID, "%s: negative slot count", what);
  if (!offsets || (!w16 && (!wq || !ws || !wz)))
    return set_error(USAF_ERR_INVALID, "%s: null pointer (offsets, and either q/s/z or the dense weight)", what);
  if (w16 && ((uintptr_t)w16 & 15)) return set_error(USAF_ERR_INVALID, "%s: dense weight must be 16-byte aligned", what);
  if (!w16 && ((uintptr_t)wq & 15)) return set_error(USAF_ERR_INVALID, "%s: codes must be 16-byte aligned", what);
  return USAF_OK;
}

}  // namespace
}  // namespace usaf

using namespace usaf;

// Forward gate_up + SwiGLU (qwen3moe_dml.py:58-60, per routed slot).
extern "C" int usaf_hip_moe_gate_up_fwd(const void* x, int64_t H, const int32_t* token_idx, const int32_t* offsets,
                                        int64_t S, int64_t E, int64_t I, const int8_t* wq, const uint16_t* ws,
                                        const uint16_t* wz, const void* w16, int32_t dtype, void* gu, void* act, void* stream) {
  if (int rc = check_common("moe_gate_up_fwd", S, E, offsets, wq, ws, wz, w16)) return rc;
  if (H % 128 != 0 || H <= 0 || I % 64 != 0 || I <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_fwd: needs H %% 128 == 0 and I %% 64 == 0 (H=%lld, I=%lld)",
                     (long long)H, (long long)I);
  if (S == 0) return clear_error();
  if (!x || !token_idx || !gu || !act) return set_error(USAF_ERR_INVALID, "moe_gate_up_fwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)x; g.lda = H; g.a_rows = token_idx;
  g.wq = (const uint8_t*)wq; g.ws = ws; g.wz = wz; g.w16 = (const uint16_t*)w16; g.w_rows = 2 * I; g.w_cols = H;
  g.N = I; g.K = H; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)act; g.ldo = I; g.out2 = (uint16_t*)gu; g.ldo2 = 2 * I;
  const int64_t max_tiles = (S / BM + E) * (I / 64);
  return launch_gemm<BMODE_NK, EPI_SWIGLU_FWD>(g, dtype, max_tiles, as_stream(stream), "moe_gate_up_fwd");
}

// Forward down projection (qwen3moe_dml.py:61): y[m] = act[m] @ W_down[e]^T.
extern "C" int usaf_hip_moe_down_fwd(const void* act, int64_t I, const int32_t* offsets, int64_t S, int64_t E,
                                     int64_t H, const int8_t* wq, const uint16_t* ws, const uint16_t* wz,
                                     const void* w16, int32_t dtype, void* y, void* stream) {
  if (int rc = check_common("moe_down_fwd", S, E, offsets, wq, ws, wz, w16)) return rc;
  if (I % 128 != 0 || I <= 0 || H % BN != 0 || H <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_fwd: needs I %% 128 == 0 and H %% 128 == 0 (I=%lld, H=%lld)",
                     (long long)I, (long long)H);
  if (S == 0) return clear_error();
  if (!act || !y) return set_error(USAF_ERR_INVALID, "moe_down_fwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)act; g.lda = I; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq; g.ws = ws; g.wz = wz; g.w16 = (const uint16_t*)w16; g.w_rows = H; g.w_cols = I;
  g.N = H; g.K = I; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)y; g.ldo = H;
  const int64_t max_tiles = (S / BM + E) * (H / BN);
  return launch_gemm<BMODE_NK, EPI_STORE>(g, dtype, max_tiles, as_stream(stream), "moe_down_fwd");
}

// Backward through the down projection and SwiGLU: dgu[m] from dcur[m] @ W_down[e].
extern "C" int usaf_hip_moe_down_bwd(const void* dcur, int64_t H, const void* gu, const int32_t* offsets, int64_t S,
                                     int64_t E, int64_t I, const int8_t* wq, const uint16_t* ws, const uint16_t* wz,
                                     const void* w16, int32_t dtype, void* dgu, void* stream) {
  if (int rc = check_common("moe_down_bwd", S, E, offsets, wq, ws, wz, w16)) return rc;
  if (I % 128 != 0 || I <= 0 || H % BK != 0 || H <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_down_bwd: needs I %% 128 == 0 and H %% 64 == 0 (I=%lld, H=%lld)",
                     (long long)I, (long long)H);
  if (S == 0) return clear_error();
  if (!dcur || !gu || !dgu) return set_error(USAF_ERR_INVALID, "moe_down_bwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)dcur; g.lda = H; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq; g.ws = ws; g.wz = wz; g.w16 = (const uint16_t*)w16; g.w_rows = H; g.w_cols = I;
  g.N = I; g.K = H; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)dgu; g.ldo = 2 * I; g.aux = (const uint16_t*)gu; g.ld_aux = 2 * I;
  const int64_t max_tiles = (S / BM + E) * (I / BN);
  return launch_gemm<BMODE_KN, EPI_SWIGLU_BWD>(g, dtype, max_tiles, as_stream(stream), "moe_down_bwd");
}

// Backward grad-input through gate_up: dx_slots[m] = dgu[m] @ W_gate_up[e].
extern "C" int usaf_hip_moe_gate_up_bwd(const void* dgu, int64_t I, const int32_t* offsets, int64_t S, int64_t E,
                                        int64_t H, const int8_t* wq, const uint16_t* ws, const uint16_t* wz,
                                        const void* w16, int32_t dtype, void* dx_slots, void* stream) {
  if (int rc = check_common("moe_gate_up_bwd", S, E, offsets, wq, ws, wz, w16)) return rc;
  if (H % 128 != 0 || H <= 0 || (2 * I) % BK != 0 || I <= 0)
    return set_error(USAF_ERR_UNSUPPORTED, "moe_gate_up_bwd: needs H %% 128 == 0 and 2I %% 64 == 0 (H=%lld, I=%lld)",
                     (long long)H, (long long)I);
  if (S == 0) return clear_error();
  if (!dgu || !dx_slots) return set_error(USAF_ERR_INVALID, "moe_gate_up_bwd: null pointer");
  GemmArgs g{};
  g.A = (const uint16_t*)dgu; g.lda = 2 * I; g.a_rows = nullptr;
  g.wq = (const uint8_t*)wq; g.ws = ws; g.wz = wz; g.w16 = (const uint16_t*)w16; g.w_rows = 2 * I; g.w_cols = H;
  g.N = H; g.K = 2 * I; g.inter = I; g.offsets = offsets; g.E = (int)E;
  g.out = (uint16_t*)dx_slots; g.ldo = H;
  const int64_t max_tiles = (S / BM + E) * (H / BN);
  return launch_gemm<BMODE_KN, EPI_STORE>(g, dtype, max_tiles, as_stream(stream), "moe_gate_up_bwd");
}
