/*
 * q4_oracle.c -- TEST INFRASTRUCTURE ONLY (the parity checker, never shipped
 * or measured as the product).  Scalar C restatement of the reference 4-bit
 * codec, usaf/quantization.py:21-132, used by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg.
 *
 * Every function follows the reference's torch-CPU op sequence in IEEE fp32
 * (x86-64 SSE arithmetic, FLT_EVAL_METHOD 0) and models fp16 tensors by
 * round-to-nearest-even conversion after each op, which is what torch's CPU
 * fp16 kernels do (upcast, op, round).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- IEEE binary16 <-> binary32, round to nearest even -------------------- */

float q4o_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do { man <<= 1; e++; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t q4o_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7FFFFFFFu;
  if (absx > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((absx >> 13) & 0x3FFu)); /* NaN */
  if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
  if (absx < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
    if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 (ties at 2^-25 go to even 0) */
    uint32_t e = absx >> 23;
    uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126 - e; /* 14..24 : value = m * 2^(e-150); subnormal unit 2^-24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (absx >> 23) - 127 + 15;
  uint32_t m = absx & 0x7FFFFFu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++; /* carry may roll into the exponent: still correct */
  return (uint16_t)(sign | q);
}

/* fp16 bits -> bf16 bits the way torch converts a Half tensor to BFloat16:
 * widen to fp32 (exact), then round to nearest even; NaN -> 0x7FC0. */
uint16_t q4o_half_to_bf16(uint16_t h) {
  float f = q4o_half_to_float(h);
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* Exact double -> fp16 bits, round to nearest even (finite inputs). */
static uint16_t double_to_half(double d) {
  uint64_t x;
  memcpy(&x, &d, 8);
  const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
  const uint64_t absx = x & 0x7FFFFFFFFFFFFFFFull;
  if (absx == 0) return sign;
  const int e = (int)(absx >> 52) - 1023;                      /* value = m * 2^(e-52) */
  const uint64_t m = (absx & ((1ull << 52) - 1)) | (1ull << 52);
  const int ulp_exp = e >= -14 ? e - 10 : -24;                 /* fp16 unit in the last place */
  const int shift = 52 + ulp_exp - e;
  if (shift >= 64) return sign;                                /* below 2^-35: rounds to zero */
  uint64_t q = m >> shift;
  const uint64_t rem = m & ((1ull << shift) - 1);
  const uint64_t half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (q & 1))) q++;
  if (e >= -14) {
    const uint32_t bits = ((uint32_t)(e + 15) << 10) + (uint32_t)(q - 1024); /* q == 2048 carries */
    return (uint16_t)(sign | (bits >= 0x7C00u ? 0x7C00u : bits));
  }
  return (uint16_t)(sign | (uint16_t)q); /* subnormal (q == 1024 encodes the smallest normal) */
}

/* fp16 multiply / add, each correctly rounded (torch CPU Half arithmetic:
 * upcast, op, round).  The exact product (22 significant bits) and the exact
 * sum (at most 51 bits) of two fp16 values fit a double, so one RNE of the
 * double result is the correctly rounded fp16 result. */
static uint16_t half_mul(uint16_t a, uint16_t b) {
  double fa = q4o_half_to_float(a), fb = q4o_half_to_float(b);
  double r = fa * fb;
  if (isnan(r) || isinf(r)) return q4o_float_to_half((float)r);
  return double_to_half(r);
}

static uint16_t half_add(uint16_t a, uint16_t b) {
  double fa = q4o_half_to_float(a), fb = q4o_half_to_float(b);
  double r = fa + fb;
  if (isnan(r) || isinf(r)) return q4o_float_to_half((float)r);
  return double_to_half(r);
}

/* Exposed for the oracle's own tests. */
uint16_t q4o_half_mul(uint16_t a, uint16_t b) { return half_mul(a, b); }
uint16_t q4o_half_add(uint16_t a, uint16_t b) { return half_add(a, b); }

/* ---- quantize_4bit (quantization.py:21-85) -------------------------------- */

int64_t q4o_num_groups(int64_t numel, int64_t group_size) {
  int64_t egs = group_size < numel ? group_size : numel;
  return (numel + egs - 1) / egs;
}

/* x: fp32 [numel] (the reference flattens and casts to float, :47).
 * packed: int8 [G, (egs+1)/2]; scale, zero: fp16 bits [G]. */
void q4o_quantize(const float* x, int64_t numel, int64_t group_size, int8_t* packed, uint16_t* scale,
                  uint16_t* zero) {
  const int64_t egs = group_size < numel ? group_size : numel; /* :50 */
  const int64_t G = (numel + egs - 1) / egs;                   /* :51 */
  const int64_t pb = (egs + 1) / 2;                            /* :71 */
  for (int64_t g = 0; g < G; ++g) {
    float mn = INFINITY, mx = -INFINITY;
    for (int64_t e = 0; e < egs; ++e) { /* :59-60, zero padding included (:54-55) */
      int64_t i = g * egs + e;
      float v = i < numel ? x[i] : 0.0f;
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    float sc = (mx - mn) / 15.0f;  /* :62 */
    if (sc < 1e-12f) sc = 1e-12f;  /* :63 clamp_min */
    for (int64_t j = 0; j < pb; ++j) {
      uint32_t qq[2] = {0, 0};
      for (int h = 0; h < 2; ++h) {
        int64_t e = 2 * j + h;
        if (e >= egs) continue; /* :75-77 odd tail stays 0 */
        int64_t i = g * egs + e;
        float v = i < numel ? x[i] : 0.0f;
        float r = rintf((v - mn) / sc); /* :66 round half to even */
        if (r < 0.0f) r = 0.0f;         /* :67 */
        if (r > 15.0f) r = 15.0f;
        qq[h] = (uint32_t)r; /* :68 */
      }
      packed[g * pb + j] = (int8_t)(uint8_t)(qq[0] | (qq[1] << 4)); /* :79 */
    }
    scale[g] = q4o_float_to_half(sc); /* :82 */
    zero[g] = q4o_float_to_half(mn);  /* :83 */
  }
}

/* ---- dequantize_4bit (quantization.py:88-132) ----------------------------- */

/* packed: int8 [G, pb] flat; out: fp16 bits [numel].  Element i uses nibble i
 * of the flat bytes (:110-118 interleave, :127 flatten/slice) and group
 * i / egs, egs = min(group_size, numel) (:124).  Returns 0, or -1 if the
 * reference's view would fail. */
int q4o_dequant(const int8_t* packed, const uint16_t* scale, const uint16_t* zero, int64_t G, int64_t pb,
                int64_t group_size, int64_t numel, uint16_t* out) {
  const int64_t egs = group_size < numel ? group_size : numel;
  if (G * egs > 2 * G * pb || numel > G * egs) return -1;
  for (int64_t i = 0; i < numel; ++i) {
    uint8_t byte = (uint8_t)packed[i >> 1];
    uint16_t q = (i & 1) ? (uint16_t)(byte >> 4) : (uint16_t)(byte & 0xF);
    int64_t g = i / egs;
    uint16_t qh = q4o_float_to_half((float)q);      /* :127 .to(float16) */
    uint16_t m = half_mul(qh, scale[g]);             /* :129 q * scale */
    out[i] = half_add(m, zero[g]);                   /* :129 ... + zero */
  }
  return 0;
}

void q4o_dequant_bf16(const int8_t* packed, const uint16_t* scale, const uint16_t* zero, int64_t G, int64_t pb,
                      int64_t group_size, int64_t numel, uint16_t* out) {
  if (q4o_dequant(packed, scale, zero, G, pb, group_size, numel, out) != 0) return;
  for (int64_t i = 0; i < numel; ++i) out[i] = q4o_half_to_bf16(out[i]);
}
