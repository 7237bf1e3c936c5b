/*
 * usaf_hip.h -- C-ABI of the MI355X (gfx950) quantized-expert hot path.
 *
 * Plain C: device pointers, element counts, a dtype code and the caller's HIP
 * stream (hipStream_t passed as void*, NULL = legacy default stream).  Every
 * function returns a status code (USAF_OK on success); the message for the
 * last failure on the calling thread is returned by usaf_hip_last_error().
 * The library owns no device memory: callers allocate inputs, outputs and
 * workspaces.  Work is enqueued on `stream` and is asynchronous to the host.
 *
 * Tensor formats follow the reference's 4-bit codec
 * (usaf/quantization.py:21-132): a tensor of `numel` elements, flattened in
 * row-major order, is cut into groups of `group_size` elements (the last group
 * zero-padded); each group owns one fp16 scale and one fp16 zero (the group
 * minimum) and ceil(group_size/2) bytes of codes, element 2j in the low nibble
 * of byte j and element 2j+1 in the high nibble.
 */
#ifndef USAF_HIP_H
#define USAF_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define USAF_HIP_ABI_VERSION 1

/* status codes */
#define USAF_OK 0
#define USAF_ERR_INVALID 1     /* bad argument (shape, pointer, dtype)            */
#define USAF_ERR_UNSUPPORTED 2 /* valid request this build does not implement     */
#define USAF_ERR_RUNTIME 3     /* HIP runtime reported an error                    */

/* element type codes */
#define USAF_F32 0
#define USAF_F16 1
#define USAF_BF16 2

/* ABI version this library was built with (USAF_HIP_ABI_VERSION). */
int usaf_hip_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* usaf_hip_last_error(void);

/*
 * 4-bit unpack + dequant.
 * Replaces usaf/quantization.py:88-132 `dequantize_4bit` (and the Vulkan
 * `dequant_pipe`, usaf/vulkan/src/pybind_module.cpp:175-200).
 *   packed  int8  [n_groups, packed_cols]    (flat, row-major)
 *   scale   fp16  [n_groups]
 *   zero    fp16  [n_groups]
 *   out     fp16 or bf16 [numel]
 * Output element i takes nibble i of the flat packed byte array (low nibble
 * first) and the scale/zero of group i / eff_gs, eff_gs = min(group_size,
 * numel), and is computed as fp16(fp16(q * scale) + zero) -- two fp16
 * roundings, as the reference's fp16 tensor arithmetic does.  A bf16 output is
 * the round-to-nearest-even bf16 of that fp16 value.
 * Requires n_groups * eff_gs >= numel and n_groups * eff_gs <= 2 * n_groups * packed_cols.
 */
int usaf_hip_dequant_q4(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                        int64_t n_groups, int64_t packed_cols, int64_t group_size, int64_t numel,
                        void* out, int32_t out_dtype, void* stream);

/*
 * 4-bit group quantization.
 * Replaces usaf/quantization.py:21-85 `quantize_4bit`.
 *   x       fp32 / fp16 / bf16 [numel]  (flattened tensor)
 *   packed  int8 [n_groups, ceil(eff_gs/2)], scale fp16 [n_groups], zero fp16 [n_groups]
 * with eff_gs = min(group_size, numel), n_groups = ceil(numel / eff_gs).  Per group
 * (zero padding included): scale = max((max-min)/15, 1e-12), q = clamp(rint((x-min)/scale), 0, 15)
 * in fp32, then scale and min are rounded to fp16.
 */
int usaf_hip_quantize_q4(const void* x, int32_t x_dtype, int64_t numel, int64_t group_size,
                         int8_t* packed, uint16_t* scale_f16, uint16_t* zero_f16, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* USAF_HIP_H */
