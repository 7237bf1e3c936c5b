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

#define USAF_HIP_ABI_VERSION 2

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
 * One-time host set-up for the current device: caches its CU count, raises the
 * dynamic-LDS limit of every GEMM kernel and queries the occupancy of the
 * sampled-gradient kernels.  Every entry point does the parts it needs on first
 * use (thread-safe); calling this once beforehand keeps those host-side HIP
 * calls out of later work, e.g. out of a stream capture.  No counterpart in the
 * reference (its Vulkan module initialises on import, usaf/vulkan/src/pybind_module.cpp:487-555).
 */
int usaf_hip_init(void);

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
 * Dequantized values at flat positions, without the whole tensor:
 *   out[j] = fp32( fp16(fp16(q_i * scale) + zero) ),  i = idx[j]
 * with q_i, scale, zero as usaf_hip_dequant_q4 takes them for element i; this
 * is the reference's dequantize_4bit(...).reshape(-1)[idx].float(), the
 * master values of newly active positions (train.py:456-465, :589-595).
 * Positions outside [0, numel) give NaN and set *bad_flag = 1 (bad_flag may be NULL).
 */
int usaf_hip_dequant_q4_at(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                           int64_t n_groups, int64_t packed_cols, int64_t group_size, int64_t numel,
                           const int64_t* idx, int64_t n, float* out, int32_t* bad_flag, void* stream);

/*
 * Batched dequant of whole slices into slots of an arena (the per-expert cache
 * of dequantized copies, filled on demand as moe_loader.py:183-224 fills its
 * LRU): job j writes the dequant (as usaf_hip_dequant_q4, out_dtype) of elements
 * [src_slice[j] * slice_elems, +slice_elems) of the flat 4-bit tensor into
 * elements [dst_slice[j] * slice_elems, +slice_elems) of `out`.  Group size 128
 * (64 code bytes per group), slice_elems % 2048 == 0, codes 4-byte and out
 * 16-byte aligned; src_slice / dst_slice int64 [n_jobs] on the device; `out`
 * holds n_dst_slices slices.  Jobs naming a slice outside the tensor
 * (n_groups * 128 / slice_elems slices) or the arena are skipped.
 */
int usaf_hip_dequant_q4_slices(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                               int64_t n_groups, int64_t slice_elems, int64_t n_jobs, const int64_t* src_slice,
                               const int64_t* dst_slice, int64_t n_dst_slices, void* out, int32_t out_dtype,
                               void* stream);

/*
 * The same on-demand fill of the per-expert copy cache (moe_loader.py:183-224),
 * written in the fragment order the *_fwd_slots GEMMs read: job j dequantizes
 * expert src_expert[j] of a [n_experts, w_rows, K] 4-bit tensor (group size 128
 * along K) into slot dst_slot[j] of an arena of n_slots slots, each
 * usaf_hip_frag_slot_elems(w_rows, K, inter) elements of out_dtype (fp16 / bf16).
 * Values are those of usaf_hip_dequant_q4; only the order differs.  inter > 0
 * marks a gate_up block (w_rows == 2 inter, SwiGLU row pairing); inter == 0 a
 * plain block such as down.  K % 128 == 0; codes and out 16-byte aligned;
 * jobs naming an expert or slot out of range are skipped.
 */
int usaf_hip_dequant_q4_slices_frag(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16,
                                    int64_t n_experts, int64_t w_rows, int64_t K, int64_t inter, int64_t n_jobs,
                                    const int64_t* src_expert, const int64_t* dst_slot, int64_t n_slots, void* out,
                                    int32_t out_dtype, void* stream);
/* Elements of one fragment-order slot (rows padded to whole GEMM tiles); -1 for
 * shapes the layout does not take (K % 128 != 0, w_rows != 2 inter). */
int64_t usaf_hip_frag_slot_elems(int64_t w_rows, int64_t K, int64_t inter);

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

/*
 * Scale/zero pairs for the fused GEMMs: scale_zero[g] = scale bits | zero bits << 16
 * (both fp16), one 32-bit word per group, so a GEMM reads a group's parameters with
 * one load.  Derived once per 4-bit tensor from the codec's scale/zero arrays
 * (the fp16 scale/zero of usaf/quantization.py:82-83); no counterpart in the reference.
 */
int usaf_hip_pack_scale_zero(const uint16_t* scale_f16, const uint16_t* zero_f16, int64_t n_groups,
                             uint32_t* scale_zero, void* stream);

/*
 * Transposed copy of a 4-bit [E, rows, cols] tensor (groups of 128 along cols) for
 * the grad-input GEMMs, which contract over rows:
 *   packed_t [E, cols, rows/2] int8: the code of element (r, c) at row c, nibble r
 *            (even r in the low nibble, the codec's order applied to W^T)
 *   sz_t     [E, cols/128, rows/2, 2] uint32: {s(r) | s(r+1) << 16, z(r) | z(r+1) << 16}
 *            with s(r), z(r) the fp16 scale/zero of the group holding (r, c)
 * Bits are copied unchanged, so W^T dequantizes to exactly the transposed
 * values of W.  Needs cols % 128 == 0, rows % 64 == 0, 16-byte aligned code
 * buffers.  A derived layout of this build; no counterpart in the reference.
 */
int usaf_hip_q4_transpose(const int8_t* packed, const uint16_t* scale_f16, const uint16_t* zero_f16, int64_t E,
                          int64_t rows, int64_t cols, int8_t* packed_t, uint32_t* sz_t, void* stream);

/* ---- routing and bucketing ------------------------------------------------ */

/*
 * Router softmax + top-k threshold mask.
 * Replaces usaf/qwen3moe_dml.py:73-83 (dml_qwen3_moe_block_forward's routing).
 *   logits   [T, E] fp32/fp16/bf16 (the router F.linear output)
 *   weights  [T, E] out, weights_dtype: p * (p >= kth_largest(p)) (ties may select
 *            more than top_k experts), divided by max(sum, 1e-9) if norm_topk_prob
 *   probs    [T, E] fp32 out (optional, NULL to skip): p = softmax(logits) in fp32
 * 0 < E <= 1024, 0 < top_k <= E.
 */
int usaf_hip_route_topk(const void* logits, int32_t logits_dtype, int64_t T, int64_t E, int64_t top_k,
                        int32_t norm_topk_prob, void* weights, int32_t weights_dtype, float* probs, void* stream);

/*
 * Backward of usaf_hip_route_topk (autograd of qwen3moe_dml.py:74-83):
 * dlogits [T, E] (logits_dtype) from dweights [T, E] and the forward's probs.
 */
int usaf_hip_route_topk_bwd(const void* dweights, int32_t weights_dtype, const float* probs, int64_t T, int64_t E,
                            int64_t top_k, int32_t norm_topk_prob, void* dlogits, int32_t logits_dtype,
                            void* stream);

/*
 * The router forward of qwen3moe_dml.py:72-83 from one call:
 *   logits [T, E] = dtype(x @ W^T)  (x [T, H], W [E, H], 16-bit, H % 256 == 0),
 * then usaf_hip_route_topk on those logits: weights [T, E] (weights_dtype),
 * probs fp32 [T, E] (may be NULL).
 */
int usaf_hip_router_fwd(const void* x, const void* w, int64_t T, int64_t E, int64_t H, int32_t dtype, int64_t top_k,
                        int32_t norm_topk_prob, void* logits, void* weights, int32_t weights_dtype, float* probs,
                        void* stream);

/*
 * Weight gradient of the router's linear layer (autograd of qwen3moe_dml.py:72,
 * router_logits = F.linear(hs, router.weight)):
 *   dw[e, h] = dtype( sum_t fp32(dlogits[t, e]) * fp32(x[t, h]) )      [E, H]
 * dlogits [T, E] and x [T, H] row-major 16-bit; E and H multiples of 8, 16-byte
 * aligned; workspace fp32 [usaf_hip_router_dw_ws_floats(T, E, H)].
 */
/*
 * Grad-input of the router's F.linear (qwen3moe_dml.py:72):
 *   accumulate == 0: dx = dtype(dlogits @ W)
 *   accumulate != 0: dx = dtype(dtype(dlogits @ W) + dx)
 * dlogits [T, E], W [E, H], dx [T, H] in the dtype, fp32 accumulation.  The
 * accumulating form adds the gradient the experts' branch gave the same hidden
 * states (on entry in dx) with autograd's two roundings: the matmul's, then the
 * accumulation's.  Needs E % 16 == 0, H % 8 == 0, 16-byte aligned dlogits, W, dx.
 */
int usaf_hip_router_dx(const void* dlogits, const void* w, int64_t T, int64_t E, int64_t H, int32_t dtype, void* dx,
                       int32_t accumulate, void* stream);
int64_t usaf_hip_router_dw_ws_floats(int64_t T, int64_t E, int64_t H);
int usaf_hip_router_dw(const void* dlogits, const void* x, int64_t T, int64_t E, int64_t H, int32_t dtype, void* dw,
                       float* workspace, void* stream);

/* int32 workspace entries usaf_hip_bucket_by_expert needs for T tokens, E experts. */
int64_t usaf_hip_bucket_workspace_ints(int64_t T, int64_t E);

/*
 * Bucket routed (token, expert) pairs by expert -- the histogram + prefix sum +
 * stable scatter that replaces benchmarks/kaggle_t4_bench.py:293-306
 * (nonzero -> bincount -> argsort(stable) -> cumsum).
 *   weights    [T, E] routing weights; a pair is routed iff its weight != 0
 *   counts     [E] int32 out; offsets [E+1] int32 out (offsets[E] = S, the pair count)
 *   token_idx  [capacity] int32 out: slot s -> token, tokens ascending within each expert
 *   slot_w     [capacity] fp32 out: fp32 of the routing weight of slot s
 *   pair_slot  [T, E] int32 out: slot of (t, e), -1 if not routed (or beyond capacity)
 * counts are the true per-expert pair counts; offsets are clamped to `capacity`,
 * so pairs beyond it are dropped and every offset indexes the slot buffers.
 * overflow == NULL: callers size capacity >= T*E (nothing is dropped) and read
 * the slot count S = offsets[E].  overflow != NULL (capacity mode, no host read
 * of S needed): the slots [offsets[E], capacity) are filled with token 0 and
 * weight 0, and *overflow is set to 1 (never cleared) when pairs were dropped.
 */
int usaf_hip_bucket_by_expert(const void* weights, int32_t weights_dtype, int64_t T, int64_t E, int32_t* workspace,
                              int32_t* counts, int32_t* offsets, int32_t* token_idx, float* slot_w,
                              int32_t* pair_slot, int64_t capacity, int32_t* overflow, void* stream);

/*
 * usaf_hip_bucket_by_expert without a workspace argument and without any
 * allocation: its kernels use a file-scope device array of
 * usaf_hip_bucket_noalloc_max_ints() int32 (4 MiB, one per GPU, held until the
 * process ends), so ceil(T / 16) * E must not exceed 2^20 (larger calls return
 * USAF_ERR_UNSUPPORTED).  Same arguments (minus workspace), outputs and errors.
 * Calls that overlap on one GPU share the array and race; the array keeps the
 * last call's contents.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).
 */
int64_t usaf_hip_bucket_noalloc_max_ints(void);
int usaf_hip_bucket_by_expert_noalloc(const void* weights, int32_t weights_dtype, int64_t T, int64_t E,
                                      int32_t* counts, int32_t* offsets, int32_t* token_idx, float* slot_w,
                                      int32_t* pair_slot, int64_t capacity, int32_t* overflow, void* stream);

/*
 * Expert-ordered combine.  Replaces usaf/qwen3moe_dml.py:62-64:
 *   out[t] = dtype( sum_{e ascending, routed} fp32(y[slot(t,e)]) * fp32(w[t,e]) )
 * accumulated in fp32 with each product rounded before the add, as the
 * reference's `final = final + cur.float() * w.float()`.  weights == NULL: the
 * unweighted sum (used for the grad-input accumulation over experts).
 *   y_slots [S, H], weights [T, E], out [T, H]; dtype fp16 or bf16; E <= 1024.
 */
int usaf_hip_moe_combine(const void* y_slots, const void* weights, const int32_t* pair_slot, int64_t T, int64_t E,
                         int64_t H, int32_t dtype, void* out, void* stream);

/*
 * Backward of the weighted combine (autograd of qwen3moe_dml.py:62-64):
 *   dcur[s]          = dtype(fp32(dout[t]) * w_s)                 [S, H]
 *   dweights[t, e]   = dtype(sum_h fp32(dout[t,h]) * fp32(y[s,h])) (routed pairs only;
 *                      other entries are left untouched -- callers zero them)
 * Slots s >= offsets[E] (the padding of a capacity-mode bucketing) are skipped.
 */
int usaf_hip_moe_combine_bwd(const void* dout, const void* y_slots, const int32_t* token_idx, const float* slot_w,
                             const int32_t* offsets, int64_t S, int64_t E, int64_t H, int32_t dtype, void* dcur,
                             void* dweights, void* stream);

/* ---- fused 4-bit dequant grouped GEMMs (MFMA) ----------------------------- */
/*
 * Weights are whole [E, rows, cols] tensors in the codec format above
 * (packed int8 [E*rows*cols/128, 64]) with their scale/zero pairs `wsz`
 * (usaf_hip_pack_scale_zero, [E*rows*cols/128]);
 * expert e owns slots offsets[e] .. offsets[e+1]-1.  Activations are fp16 or
 * bf16 (`dtype`); with bf16 the weight operand is the bf16 rounding of the
 * fp16 dequantized value.  Accumulation is fp32 on MFMA.  When `w16` is not
 * NULL the weight is instead that dense [E, rows, cols] tensor of `dtype` (the
 * reference's dense expert weights) and wq/wsz may be NULL.  Weight pointers
 * must be 16-byte aligned.
 */

/* Replaces qwen3moe_dml.py:58-60 per routed slot: gu[s] = x[token_idx[s]] @ W_gate_up[e]^T
 * ([S, 2I], dtype-rounded), act[s] = dtype(dtype(silu(gate)) * up) ([S, I]).
 * x [T, H] (token_idx values < T); W_gate_up [E, 2I, H]; needs H % 128 == 0, I % 64 == 0.
 * act_blk (optional, 16-byte aligned): act also in the blocked slot-major layout
 * of blk_table (usaf_hip_blocked_layout of the same offsets and S), as
 * usaf_hip_gather_transpose_blocked(act, ...) would write it -- the column operand
 * of the down projection's sampled gradient; the 4-bit kernel writes it from its
 * epilogue. */
int usaf_hip_moe_gate_up_fwd(const void* x, int64_t T, int64_t H, const int32_t* token_idx, const int32_t* offsets, int64_t S,
                             int64_t E, int64_t I, const int8_t* wq, const uint32_t* wsz,
                             const void* w16, int32_t dtype, void* gu, void* act, void* act_blk,
                             const int32_t* blk_table, const uint32_t* overlay, int64_t overlay_words, void* stream);

/* Replaces qwen3moe_dml.py:61: y[s] = act[s] @ W_down[e]^T ([S, H]).  W_down [E, H, I];
 * needs I % 128 == 0, H % 128 == 0. */
int usaf_hip_moe_down_fwd(const void* act, int64_t I, const int32_t* offsets, int64_t S, int64_t E, int64_t H,
                          const int8_t* wq, const uint32_t* wsz, const void* w16, int32_t dtype, void* y,
                          const uint32_t* overlay, int64_t overlay_words, void* stream);

/* usaf_hip_moe_gate_up_fwd / usaf_hip_moe_down_fwd with dense weights held in a
 * slot arena (dequantized expert copies of usaf_amd's per-expert cache, the
 * on-demand fp16 copies of moe_loader.py:130-181): expert e's weight is slot
 * slot_of[e] of the arena, in the fragment order of
 * usaf_hip_dequant_q4_slices_frag (gate_up: w_rows 2I, K H, inter I; down:
 * w_rows H, K I, inter 0), in the activation dtype.  slot_of int32 [E] on the
 * device; entries outside [0, n_slots) are clamped (wrong weights, never an
 * access outside the arena).  Needs the contraction dimension % 128 == 0,
 * E <= 255, 16-byte aligned activations and arena. */
int usaf_hip_moe_gate_up_fwd_slots(const void* x, int64_t T, int64_t H, const int32_t* token_idx,
                                   const int32_t* offsets, int64_t S, int64_t E, int64_t I, const void* arena,
                                   const int32_t* slot_of, int64_t n_slots, int32_t dtype, void* gu, void* act,
                                   void* stream);
int usaf_hip_moe_down_fwd_slots(const void* act, int64_t I, const int32_t* offsets, int64_t S, int64_t E, int64_t H,
                                const void* arena, const int32_t* slot_of, int64_t n_slots, int32_t dtype, void* y,
                                void* stream);

/* Autograd of qwen3moe_dml.py:60-61: dact = dcur @ W_down[e] through the SwiGLU
 * (saved gu) -> dgu [S, 2I] (gate half, up half).  Needs I % 128 == 0, H % 64 == 0. */
int usaf_hip_moe_down_bwd(const void* dcur, int64_t H, const void* gu, const int32_t* offsets, int64_t S, int64_t E,
                          int64_t I, const int8_t* wq, const uint32_t* wsz, const void* w16, int32_t dtype,
                          void* dgu, void* stream);

/* Autograd of qwen3moe_dml.py:58 (grad-input): dx_slots[s] = dgu[s] @ W_gate_up[e]
 * ([S, H]); sum per token with usaf_hip_moe_combine(weights=NULL).
 * Needs H % 128 == 0, 2I % 64 == 0. */
int usaf_hip_moe_gate_up_bwd(const void* dgu, int64_t I, const int32_t* offsets, int64_t S, int64_t E, int64_t H,
                             const int8_t* wq, const uint32_t* wsz, const void* w16, int32_t dtype, void* dx_slots,
                             void* stream);

/* The two grad-input GEMMs above on the transposed 4-bit copies (usaf_hip_q4_transpose
 * of W_down [E, H, I] -> [E, I, H], of W_gate_up [E, 2I, H] -> [E, H, 2I]); same
 * results up to fp32 summation order.  Replace the same autograd steps
 * (qwen3moe_dml.py:58-61).  down_bwd_t needs I % 128 == 0 and H % 128 == 0;
 * gate_up_bwd_t needs H % 128 == 0 and I % 64 == 0; both E <= 255. */
int usaf_hip_moe_down_bwd_t(const void* dcur, int64_t H, const void* gu, const int32_t* offsets, int64_t S, int64_t E,
                            int64_t I, const int8_t* wq_t, const uint32_t* wsz_t, int32_t dtype, void* dgu,
                            const uint32_t* overlay, int64_t overlay_words, void* stream);
int usaf_hip_moe_gate_up_bwd_t(const void* dgu, int64_t I, const int32_t* offsets, int64_t S, int64_t E, int64_t H,
                               const int8_t* wq_t, const uint32_t* wsz_t, int32_t dtype, void* dx_slots,
                               const uint32_t* overlay, int64_t overlay_words, void* stream);

/*
 * Overlays on the 4-bit GEMMs: trained values (the optimizer's fp32 masters)
 * that replace the dequantized weight at a fixed set of flat positions, so that
 * the forward and grad-input GEMMs above see the weights the reference builds
 * by scattering the masters into its fp16 expert weights every step
 * (moe_loader.py:218-221 _dequant_cpu, :425-443 sync_resident, train.py:666).
 * `overlay` (NULL: none) of usaf_hip_moe_gate_up_fwd, usaf_hip_moe_down_fwd,
 * usaf_hip_moe_down_bwd_t and usaf_hip_moe_gate_up_bwd_t is that GEMM's entry
 * table of `overlay_words` uint32 words (at least the count below, else
 * USAF_ERR_INVALID): for each (expert e, n-tile nt, wave w in 0..7) unit u = (e * n_nt + nt)
 * * 8 + w and each k-step ks (64 contraction elements; n_nt = ceil(I / 128) for
 * gate_up_fwd, else ceil(N / 256)), 64 uint32 words at ((u * K / 64 + ks) * 64):
 * word 16 j + r is entry r (< 16) of the wave's fragment register j (lane
 * 16 j + r stores it): {byte offset | value << 16}, the offset into the 1 KiB
 * image of register j, which holds lane l's copy (the wave's weight row l % 32,
 * k = 32 (l / 32) + 8 j + [0, 8) of the k-step) at byte 16 l, element k at
 * 2 (k % 8) within it.  Wave w's 32 rows are the n-tile's rows 32 w + [0, 32)
 * (gate_up_fwd: gate rows n = 128 nt + 16 w + [0, 16), then the up rows I + n);
 * unused words hold an offset in [1024, 2048) (a scratch area of the wave's LDS
 * epilogue tile).  The Python layer (usaf_amd/moe.py overlay_entries,
 * Q4Overlay) builds the tables once per set of positions.  A GEMM with an overlay
 * runs the 4-bit LDS-DMA kernel only (NotImplemented otherwise).
 *
 * usaf_hip_overlay_refresh writes new values into one or two such tables: for
 * j < n, word words_a[j] of table_a takes the 16-bit `dtype` (fp16 or bf16)
 * value of fp16(p[index_a[j]]) -- the reference's fp16 weight after the
 * scatter -- in its high half (index_a NULL: p[j]); likewise words_b, index_b,
 * table_b.  Ordering j by word keeps each table's writes together.  Words
 * outside [0, n_words) or indices outside [0, n) set *bad_flag (optional) and
 * are skipped.  Replaces the per-step master scatter of moe_loader.py:425-443
 * (sync_resident) for weights the fused GEMMs read.
 */
int usaf_hip_overlay_refresh(const float* p, int64_t n, const int32_t* words_a, const int32_t* index_a,
                             uint32_t* table_a, int64_t n_words_a, const int32_t* words_b, const int32_t* index_b,
                             uint32_t* table_b, int64_t n_words_b, int32_t dtype, int32_t* bad_flag, void* stream);

/* ---- sparse gradient path and optimizer ----------------------------------- */

/*
 * Per-expert blocked slot-major operands for the sampled gradient: expert e's
 * slots form a contiguous block of C rows of ld_e = round_up(S_e, 16) elements at
 * element offset C * sum_{e' < e} ld_e', padding columns zero:
 *   out_blk[C * P[e] + c * ld_e + j] = in[rows ? rows[s0_e + j] : s0_e + j, c]   (j < S_e)
 * usaf_hip_blocked_elems bounds the element count (C * (S + 15 E)).  Needs C, ld_in
 * % 8 == 0, 16-byte aligned bases, E <= 1024.  A layout of this build: the
 * operands of the dense per-expert weight grads qwen3moe_dml.py:44-47 reads.
 */
int64_t usaf_hip_blocked_elems(int64_t S, int64_t E, int64_t C);
/* The layout table of one bucketing of S slots, int32 [usaf_hip_blocked_table_elems(S, E)]:
 * P[e] (padded slots before expert e), the 64-slot chunk counts before e, then the
 * owning expert of each 64-slot chunk; built once and shared by every blocked
 * operand and sampled gradient of that bucketing. */
int64_t usaf_hip_blocked_table_elems(int64_t S, int64_t E);
int usaf_hip_blocked_layout(const int32_t* offsets, int64_t E, int64_t S, int32_t* table, void* stream);
int usaf_hip_gather_transpose_blocked(const void* in, int64_t ld_in, const int32_t* rows, const int32_t* offsets,
                                      const int32_t* table, int64_t S, int64_t E, int64_t C, void* out_blk,
                                      void* stream);

/*
 * usaf_hip_sddmm_masked on blocked operands (row_blk: R rows per expert block,
 * col_blk: C rows per expert block, both from usaf_hip_gather_transpose_blocked
 * with the same layout table).  Replaces the same reference steps (qwen3moe_dml.py:44-56,
 * moe_loader.py:564-578).  accumulate = 0 writes 0 + sum instead of compact + sum
 * (the first add into a zeroed buffer, without the zeroing pass); every position
 * of the list is written.
 */
int usaf_hip_sddmm_blocked(const void* row_blk, const void* col_blk, const int32_t* table, int64_t E, int64_t R,
                           int64_t C, int64_t n_pos, const int32_t* row_code, const int32_t* col_idx,
                           const int64_t* pos_map, int32_t dtype, float* compact, int32_t accumulate, void* stream);

/* Backward of the weighted combine (as usaf_hip_moe_combine_bwd) that also writes
 * dcur in the blocked slot-major layout of `table` (usaf_hip_blocked_layout of the
 * same offsets and S), the row operand of the down projection's sampled gradient:
 *   dcur [S, H] row-major, dcur_blk [usaf_hip_blocked_elems(S, E, H)],
 *   dweights [T, E] (routed pairs only, as usaf_hip_moe_combine_bwd),
 *   workspace fp32 [usaf_hip_combine_bwd_blocked_ws_floats(S, H)].
 * Needs H % 8 == 0 and 16-byte aligned dout, y_slots, dcur and dcur_blk. */
int64_t usaf_hip_combine_bwd_blocked_ws_floats(int64_t S, int64_t H);
int usaf_hip_moe_combine_bwd_blocked(const void* dout, const void* y_slots, const int32_t* token_idx,
                                     const float* slot_w, const int32_t* offsets, const int32_t* table, int64_t S,
                                     int64_t E, int64_t H, int32_t dtype, void* dcur, void* dcur_blk, void* dweights,
                                     float* workspace, void* stream);

/* out[c, s] = in[rows ? rows[s] : s, c] for 16-bit [.., C] -> [C, S] (slot-major operands).
 * When C, ld_in and ld_out are multiples of 8 and both bases 16-byte aligned, the
 * transposed rows are written as 16-byte vectors and out[c, S .. round_up(S, 8)) is
 * zero-filled. */
int usaf_hip_gather_transpose(const void* in, int64_t ld_in, const int32_t* rows, int64_t S, int64_t C, void* out,
                              int64_t ld_out, void* stream);

/*
 * Sampled weight gradient at the active positions only.  Replaces the dense
 * per-expert F.linear weight grad + SparseGradStore.add gather
 * (usaf/qwen3moe_dml.py:44-56, usaf/moe_loader.py:564-578):
 *   compact[pos(p)] += fp32(dtype( sum_{s in expert e} rowT[o, s] * colT[i, s] ))
 * for each active position p < n_pos of a [E, R, C] weight, given as
 * row_code[p] = e << 21 | o and col_idx[p] = i (int32; out-of-range entries are
 * skipped) and pos_map[p] (int64 compact index of entry p; NULL = identity; each
 * compact index at most once).  rowT [R, ldT] and colT [C, ldT] are slot-major
 * 16-bit operands (dtype), 16-byte aligned, ldT a multiple of 8 and >= offsets[E].
 * E <= 1024, R < 2^21.
 */
int usaf_hip_sddmm_masked(const void* rowT, const void* colT, int64_t ldT, const int32_t* offsets, int64_t E,
                          int64_t R, int64_t C, int64_t n_pos, const int32_t* row_code, const int32_t* col_idx,
                          const int64_t* pos_map, int32_t dtype, float* compact, void* stream);

/*
 * Positions of the k largest magnitudes |x[i]| among n values (fp32, fp16 or
 * bf16; NaN ranks above +inf, as torch.topk ranks it): pos int64 [min(k, n)] in
 * ascending position order, ties at the k-th largest magnitude taken from the
 * lowest positions; vals fp32 [min(k, n)] = |x[pos]| (may be NULL).  The same
 * set as torch.topk(x.abs(), k) whenever the k-th and (k+1)-th magnitudes
 * differ.  Replaces the selections of usaf/moe_loader.py:584-631
 * (TopKImportanceStore.add: per-expert top |grad| candidates; .select: global
 * top-k over the candidates).  n < 2^31; workspace int32
 * [usaf_hip_topk_abs_ws_ints(n)]; nothing is read back to the host.
 */
int64_t usaf_hip_topk_abs_ws_ints(int64_t n);
int usaf_hip_topk_abs(const void* x, int32_t dtype, int64_t n, int64_t k, int64_t* pos, float* vals,
                      int32_t* workspace, void* stream);

/*
 * One SparseAdam step on compact fp32 vectors (usaf/sparse_optim.py:94-130,
 * compact_params=True): p, m, v updated in place from grad; `step` >= 1 is the
 * step count after increment.  Scalars are the reference's Python floats.
 */
int usaf_hip_sparse_adam_step(float* p, const float* grad, float* m, float* v, int64_t n, double lr, double beta1,
                              double beta2, double eps, double weight_decay, int64_t step, void* stream);

/* usaf_hip_sparse_adam_step gated on the device, for training loops that launch
 * the update before the host has read the step's finite flag (train.py:649-672
 * applies SparseAdam only to finite steps): the update is skipped unless
 * finite[0] != 0 and halt[0] == 0 (either pointer may be NULL = open).  The
 * step number is t = step_count[0] + 1, where step_count (int32, device) is the
 * number of steps applied so far; its bias corrections are bias_table[2 (t - 1)]
 * = fp32(1 - beta1^t) and bias_table[2 (t - 1) + 1] = fp32(1 - beta2^t),
 * computed by the caller in double as the reference's Python scalars are.
 * t > table_steps skips the update and sets *bad_flag (optional).
 * usaf_hip_count_step advances step_count by one under the same gate; call it
 * once after all of a step's gated launches. */
int usaf_hip_sparse_adam_step_gated(float* p, const float* grad, float* m, float* v, int64_t n, double lr, double beta1,
                                    double beta2, double eps, double weight_decay, const int32_t* finite,
                                    const int32_t* halt, const int32_t* step_count, const float* bias_table,
                                    int64_t table_steps, int32_t* bad_flag, void* stream);
int usaf_hip_count_step(const int32_t* finite, const int32_t* halt, int32_t* step_count, void* stream);

/* torch.optim.SGD.step with momentum (dampening 0, no Nesterov) for one tensor, the
 * router's optimizer in the reference trainer (train.py:493-498, 667-672):
 * d = grad + wd*p; buf = d on the first step, else buf*momentum + d; p -= lr*buf;
 * rounded to the tensor dtype after each torch op as the single-tensor path does.
 * Optional device gate (either pointer may be NULL): the step is skipped on the
 * device when *finite == 0 or *halt != 0, so a training loop can launch it
 * before it reads the step's finite flag on the host (train.py:649-672 decides
 * on the host).  A gated call cannot be the first step (first_step != 0).
 * Optional loss scale (scale_state, NULL = none): the gradient is first divided
 * by loss_scale * accum read from the device state of usaf_hip_loss_scale_update
 * and rounded to the dtype, as train.py:669-670 `p.grad.data.div_(loss_scale *
 * ACCUM)` does before the router step; the grad buffer itself is left unchanged. */
int usaf_hip_sgd_momentum_step(void* p, const void* grad, void* momentum_buf, int64_t n, int32_t dtype, double lr,
                               double momentum, double weight_decay, int32_t first_step, const int32_t* finite,
                               const int32_t* halt, const int32_t* scale_state, double accum, void* stream);

/* out = in / denom (fp32) and *finite_flag = 0 if any result is inf/NaN (train.py:661-663);
 * the caller sets *finite_flag = 1 beforehand. */
int usaf_hip_scale_check(const float* in, float* out, int64_t n, float denom, int32_t* finite_flag, void* stream);

/*
 * Dynamic loss scale with its state on the device, for training loops that
 * launch step n + 1 before the host reads step n's finite flag.  Replaces the
 * host variables of train.py:31 (LOSS_SCALE_INIT = 4096, SCALE_UP_EVERY = 200),
 * :351-353 (`(loss * loss_scale).backward()`) and :661-677 (denom = loss_scale *
 * ACCUM; on a finite step good_streak += 1 and every SCALE_UP_EVERY-th good step
 * loss_scale = min(2 loss_scale, 65536); on a skipped step n_skipped += 1 and
 * loss_scale = max(loss_scale / 2, 64)).  scale_state is int32[4]: [0] the scale
 * as fp32 bits, [1] good steps (never reset, as good_streak), [2] skipped steps.
 *
 * usaf_hip_loss_scale_apply: out = dtype(x * scale) for fp16/bf16 x (the gradient
 * seed of the scaled loss; out may alias x).
 * usaf_hip_scale_check_state: usaf_hip_scale_check with denom = scale * accum.
 * usaf_hip_loss_scale_update: the schedule above for the step whose finite flag
 * is *finite (NULL = finite); nothing changes when *halt != 0.  Launch it after
 * the step's gated updates, which read the scale it replaces.
 */
int usaf_hip_loss_scale_apply(const void* x, void* out, int64_t n, int32_t dtype, const int32_t* scale_state,
                              void* stream);
int usaf_hip_scale_check_state(const float* in, float* out, int64_t n, const int32_t* scale_state, double accum,
                               int32_t* finite_flag, void* stream);
int usaf_hip_loss_scale_update(int32_t* scale_state, const int32_t* finite, const int32_t* halt,
                               int32_t scale_up_every, double min_scale, double max_scale, void* stream);

/* base.flat[idx[j]] = dtype(vals[j]) (usaf/moe_loader.py:218-221, 411-443); out-of-range
 * indices are skipped and set *bad_flag = 1. */
int usaf_hip_overlay_scatter(void* base, int32_t dtype, int64_t numel, const int64_t* idx, const float* vals,
                             int64_t n, int32_t* bad_flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* USAF_HIP_H */
