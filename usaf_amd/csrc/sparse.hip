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
// 64 x 64 tiles through LDS so that both the row reads and the column writes
// are contiguous 128-byte segments.
__global__ __launch_bounds__(256) void gather_transpose_kernel(const uint16_t* __restrict__ in, int64_t ld_in,
                                                               const int32_t* __restrict__ rows, int64_t S, int64_t C,
                                                               uint16_t* __restrict__ out, int64_t ld_out) {
  __shared__ uint16_t tile[64][65];
  const int64_t s0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  for (int r = ty; r < 64; r += 4) {
    const int64_t s = s0 + r, c = c0 + tx;
    uint16_t v = 0;
    if (s < S && c < C) {
      const int64_t row = rows ? (int64_t)rows[s] : s;
      v = in[row * ld_in + c];
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t c = c0 + r, s = s0 + tx;
    if (c < C && s < S) out[c * ld_out + s] = tile[tx][r];
  }
}

// One wavefront per weight row r = e * R + o of the [E, R, Cw] weight.  For
// each active position (o, i) of the row (CSR: row_ptr, col_idx; compact
// index pos_map[p] or p), dot over the expert's slots s of
//   rowT[o, s] * colT[i, s]
// rounded to the gradient's dtype (the reference's dense grad is a 16-bit
// tensor), added to compact[pos] in fp32 (index_add_).
template <int DT>
__global__ __launch_bounds__(256) void sddmm_kernel(const uint16_t* __restrict__ rowT, const uint16_t* __restrict__ colT,
                                                    int64_t ldT, const int32_t* __restrict__ offsets, int64_t R,
                                                    int64_t n_rows, const int64_t* __restrict__ row_ptr,
                                                    const int32_t* __restrict__ col_idx,
                                                    const int64_t* __restrict__ pos_map, float* __restrict__ compact) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t r = wave; r < n_rows; r += n_waves) {
    const int64_t p0 = row_ptr[r], p1 = row_ptr[r + 1];
    if (p0 == p1) continue;
    const int64_t e = r / R, o = r - e * R;
    const int64_t s0 = offsets[e], s1 = offsets[e + 1];
    const uint16_t* rv = rowT + o * ldT;
    for (int64_t p = p0; p < p1; ++p) {
      const int64_t i = col_idx[p];
      const uint16_t* cv = colT + i * ldT;
      float acc = 0.f;
      for (int64_t s = s0 + lane; s < s1; s += 64)
        acc += load_as_f32<DT>(rv, s) * load_as_f32<DT>(cv, s);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
      if (lane == 0) {
        const int64_t pos = pos_map ? pos_map[p] : p;
        compact[pos] += round_to<DT>(acc);
      }
    }
  }
}

// SparseAdam.step for one compact vector (sparse_optim.py:96-130), with the
// rounding of torch's vectorized CPU kernels the reference runs:
//   g = g + wd*p                       mul, add
//   m = fma(1-b1, g, m*b1)             mul_; add_(alpha=) is one fused multiply-add
//   v = v*b2 + ((1-b2)*g)*g            mul_; addcmul_ multiplies then adds
//   p = p + (-lr) * ((m/bias1) / (sqrt(v/bias2) + eps))
__global__ __launch_bounds__(256) void sparse_adam_kernel(float* __restrict__ p, const float* __restrict__ grad,
                                                          float* __restrict__ m, float* __restrict__ v, int64_t n,
                                                          float lr, float b1, float omb1, float b2, float omb2,
                                                          float eps, float wd, float bias1, float bias2) {
#pragma clang fp contract(off)
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
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

int grid_for(int64_t n, int per_cu = 8) {
  int64_t b = (n + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  if (b > cap) b = cap;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace
}  // namespace usaf

using namespace usaf;

extern "C" int usaf_hip_gather_transpose(const void* in, int64_t ld_in, const int32_t* rows, int64_t S, int64_t C,
                                         void* out, int64_t ld_out, void* stream) {
  if (S < 0 || C < 0 || ld_in < C || ld_out < S) return set_error(USAF_ERR_INVALID, "gather_transpose: bad sizes");
  if (S == 0 || C == 0) return clear_error();
  if (!in || !out) return set_error(USAF_ERR_INVALID, "gather_transpose: null pointer");
  const int64_t gx = (S + 63) / 64, gy = (C + 63) / 64;
  if (gx > 0x7fffffff || gy > 65535) return set_error(USAF_ERR_INVALID, "gather_transpose: too large");
  gather_transpose_kernel<<<dim3((unsigned)gx, (unsigned)gy), 256, 0, as_stream(stream)>>>(
      (const uint16_t*)in, ld_in, rows, S, C, (uint16_t*)out, ld_out);
  return check_launch("gather_transpose");
}

extern "C" int usaf_hip_sddmm_masked(const void* rowT, const void* colT, int64_t ldT, const int32_t* offsets,
                                     int64_t E, int64_t R, const int64_t* row_ptr, const int32_t* col_idx,
                                     const int64_t* pos_map, int32_t dtype, float* compact, void* stream) {
  if (E <= 0 || R <= 0 || ldT < 0) return set_error(USAF_ERR_INVALID, "sddmm_masked: bad sizes");
  if (!rowT || !colT || !offsets || !row_ptr || !col_idx || !compact)
    return set_error(USAF_ERR_INVALID, "sddmm_masked: null pointer");
  if (dtype != USAF_F16 && dtype != USAF_BF16) return set_error(USAF_ERR_INVALID, "sddmm_masked: dtype must be 16-bit");
  const int64_t n_rows = E * R;
  int64_t blocks = (n_rows + 3) / 4;
  const int64_t cap = (int64_t)device_cu_count() * 16;
  if (blocks > cap) blocks = cap;
  hipStream_t st = as_stream(stream);
  if (dtype == USAF_BF16)
    sddmm_kernel<USAF_BF16><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)rowT, (const uint16_t*)colT, ldT,
                                                              offsets, R, n_rows, row_ptr, col_idx, pos_map, compact);
  else
    sddmm_kernel<USAF_F16><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)rowT, (const uint16_t*)colT, ldT,
                                                             offsets, R, n_rows, row_ptr, col_idx, pos_map, compact);
  return check_launch("sddmm_masked");
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

extern "C" int usaf_hip_scale_check(const float* in, float* out, int64_t n, float denom, int32_t* finite_flag,
                                    void* stream) {
  if (n < 0) return set_error(USAF_ERR_INVALID, "scale_check: negative n");
  if (n == 0) return clear_error();
  if (!in || !out || !finite_flag) return set_error(USAF_ERR_INVALID, "scale_check: null pointer");
  scale_check_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(in, out, n, denom, finite_flag);
  return check_launch("scale_check");
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
