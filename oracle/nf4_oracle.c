/*
 * CPU oracle for NF4 dequantization (test infrastructure only: tests/, smoke() and bench.py's
 * CPU baseline use it as the checker; the product never links it).
 *
 * Restates, element by element and bit for bit:
 *   - the grouped kernel nf4_group_dequant_kernel, solution/qgroup.py:72-91 (scale from the
 *     double-quantized absmax, solution/qgroup.py:80-83; levels :60-63; both halves of a byte,
 *     high nibble first, :86-91), compiled without FMA (:99, enable_fp_fusion=False);
 *   - the per-projection kernel nf4_dequant_pairs_kernel, solution/nf4_dequant.py:38-80, which is
 *     bitsandbytes' dequantize_4bit (solution/test_fuzz.py:860-868 `_nf4_manual`).
 * Built with -ffp-contract=off, so every product and sum is rounded to binary32 on its own.
 * The binary32 -> binary16 conversion is written out below (IEEE 754 round to nearest, ties to
 * even, subnormals kept, overflow to infinity) so the result does not depend on the host
 * compiler's _Float16 support; tests compare it with numpy's float16 cast on every class of
 * input (normal, subnormal, ties, overflow).
 */
#include <stdint.h>
#include <string.h>

static const float NF4_LEVELS[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t a = x & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;            /* NaN (quiet) */
  if (a >= 0x47800000u) return sign | 0x7c00u;           /* >= 2^16 (and inf): infinity */
  if (a >= 0x38800000u) {                                /* fp16 normal range, >= 2^-14 */
    const uint32_t mant = a & 0x7fffffu;
    const uint32_t exp16 = (a >> 23) - 127u + 15u;       /* 1 .. 30 */
    uint32_t h = (exp16 << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;  /* a carry may reach inf */
    return sign | (uint16_t)h;
  }
  if (a <= 0x33000000u) return sign;                     /* <= 2^-25: rounds to (signed) zero */
  {
    /* fp16 subnormal k * 2^-24: k = rne(|f| * 2^24) = rne(mant * 2^(e + 1)), e in [-25, -15] */
    const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    const int e = (int)(a >> 23) - 127;
    const int shift = -(e + 1);                          /* 14 .. 24 */
    uint32_t k = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (k & 1u))) k += 1u;
    return sign | (uint16_t)k;
  }
}

void oracle_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}

/* solution/qgroup.py:72-91, for n_rows blocks of qblock weights. */
void oracle_nf4_group_dequant(const uint8_t* packed, const uint8_t* absmax8, const float* code,
                              const float* absmax2, const float* offset2, uint16_t* out,
                              int64_t n_rows, int32_t qblock, int32_t qblock2) {
  const int64_t half = qblock / 2;
  for (int64_t r = 0; r < n_rows; ++r) {
    const int64_t b2 = r / qblock2;
    const float prod = code[absmax8[r]] * absmax2[b2]; /* rounded to binary32 */
    const float scale = prod + offset2[b2];
    for (int64_t j = 0; j < half; ++j) {
      const uint8_t byte = packed[r * half + j];
      const float first = NF4_LEVELS[byte >> 4] * scale;
      const float second = NF4_LEVELS[byte & 15] * scale;
      out[2 * (r * half + j)] = oracle_f32_to_f16(first);
      out[2 * (r * half + j) + 1] = oracle_f32_to_f16(second);
    }
  }
}

/* solution/nf4_dequant.py:38-80: absmax already in fp32, one per `blocksize` weights. */
void oracle_nf4_dequant(const uint8_t* packed, const float* absmax, uint16_t* out, int64_t n,
                        int32_t blocksize) {
  for (int64_t i = 0; i < n / 2; ++i) {
    const uint8_t byte = packed[i];
    const float scale = absmax[(2 * i) / blocksize];
    out[2 * i] = oracle_f32_to_f16(NF4_LEVELS[byte >> 4] * scale);
    out[2 * i + 1] = oracle_f32_to_f16(NF4_LEVELS[byte & 15] * scale);
  }
}
