/* Second, independent CPU restatement of the bfp16ebs8 encoder/decoder (oracle; test infrastructure only).
 *
 * Follows redline/npu_layouts.py:62-73 (encode) and :90-94 (decode). Where the numpy oracle scales in float64 and
 * calls rint, this one works on the float32 bit pattern with integers only: the element's 24-bit significand is
 * shifted right by (E + 17 - e) places with round-half-to-even on the discarded bits, then signed and clipped to
 * [-128, 127]. The two agree only if both follow the format, which is what the tests check.
 *
 * Also exports the reference's "truncate" variant (npu_layouts.py:74-87) statement-for-statement, for negative
 * tests only. Non-finite inputs (E = 255) are out of the contract; infinities saturate like np.clip does.
 */
#include <stdint.h>
#include <string.h>

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* round-half-to-even of m / 2^s for s >= 1 */
static uint32_t rne_shift(uint32_t m, uint32_t s) {
  if (s >= 32) return 0; /* m < 2^24 <= 2^(s-1): below one half */
  uint32_t q = m >> s;
  uint32_t rem = m & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1u);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return q;
}

void rl_ref_encode_block(const float *x, uint8_t *out) {
  uint32_t u[8], e[8], E = 0;
  for (int i = 0; i < 8; i++) {
    u[i] = f32_bits(x[i]);
    e[i] = (u[i] >> 23) & 0xFFu;
    if (e[i] > E) E = e[i];
  }
  out[0] = (uint8_t)E;
  for (int i = 0; i < 8; i++) {
    int neg = (u[i] >> 31) & 1;
    int32_t q;
    if (e[i] == 255u) {
      q = neg ? -128 : 127; /* +-inf * 2^(133-255) stays inf; clip saturates */
    } else {
      uint32_t m = u[i] & 0x7FFFFFu;
      uint32_t ee = e[i];
      if (ee) m |= 0x800000u; else ee = 1u; /* subnormal: no implicit bit, exponent of 2^-126 */
      /* |x| * 2^(133-E) = m * 2^(ee - 150 + 133 - E) = m / 2^(E + 17 - ee) */
      uint32_t mag = rne_shift(m, E + 17u - ee);
      q = neg ? -(int32_t)mag : (int32_t)mag;
      if (q > 127) q = 127;
      if (q < -128) q = -128;
    }
    out[1 + i] = (uint8_t)(int8_t)q;
  }
}

void rl_ref_to_bfp16(const float *x, int64_t nblocks, uint8_t *out) {
  for (int64_t b = 0; b < nblocks; b++) rl_ref_encode_block(x + 8 * b, out + 9 * b);
}

void rl_ref_from_bfp16(const uint8_t *raw, int64_t nblocks, float *out) {
  for (int64_t b = 0; b < nblocks; b++) {
    const uint8_t *p = raw + 9 * b;
    int E = p[0];
    for (int i = 0; i < 8; i++) {
      int q = (int)(int8_t)p[1 + i];
      /* q * 2^(E-133): build 2^(E-133) exactly (subnormal in float32 when E < 7) */
      float s;
      if (E >= 7) { uint32_t sb = (uint32_t)(E - 6) << 23; memcpy(&s, &sb, 4); }
      else { uint32_t sb = 1u << (E + 16); memcpy(&s, &sb, 4); }
      out[8 * b + i] = (float)q * s;
    }
  }
}

/* npu_layouts.py:74-87 (truncate=True), statement for statement */
void rl_ref_to_bfp16_truncate(const float *x, int64_t nblocks, uint8_t *out) {
  for (int64_t b = 0; b < nblocks; b++) {
    uint32_t bits[8], exp[8], E = 0;
    for (int i = 0; i < 8; i++) {
      bits[i] = f32_bits(x[8 * b + i]);
      exp[i] = (bits[i] >> 23) & 0xFFu;
      if (exp[i] > E) E = exp[i];
    }
    out[9 * b] = (uint8_t)E;
    for (int i = 0; i < 8; i++) {
      int sign = (bits[i] & 0x80000000u) != 0;
      uint32_t mant = bits[i] & 0x7FFFFFu;
      if (exp[i] != 0) mant |= 0x800000u;
      if (sign) mant = ~mant + 1u;
      int32_t val = (int32_t)(int8_t)(uint8_t)(mant >> 17);
      int32_t shift = (int32_t)(E - exp[i]);
      int32_t r = shift >= 32 ? (sign ? -1 : 0) : (val >> (shift < 31 ? shift : 31));
      out[9 * b + 1 + i] = (uint8_t)(int8_t)r;
    }
  }
}
