// Device-side helpers shared by the bfp16 kernels (gfx950 / CDNA4, wave64).
//
// bfp16ebs8: 8 values in 9 bytes [E][q0..q7], value = q * 2^(E-133), E = the block's largest float32 exponent field,
// q = clip(rint(x * 2^(133-E)), -128, 127), round half to even (redline/npu_layouts.py:62-73, :90-94).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two floats -> one word of two bf16 (lo in bits 0..15), each rounded to nearest even: one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlockBytes = 9;

// Cache policy of the GEMV's weight loads: the non-temporal bit (streaming: the lines are not kept). A weight stream
// is read once per launch and, in a model step, was last read a whole step earlier, so caching it gains nothing. A
// plain read of a 64 MB stream measured 10.75 us with the bit against 12.2 us without (5.9 against 5.2 TB/s). Reads of
// activations that the previous kernel has just written keep the default policy: they hit in the Infinity Cache, and
// the bit measured slower there (quantize 13.2 -> 13.8 us, LN 22.8 -> 24.2 us).
constexpr int kLoadStream = 2;

// ---- exact encode: integer arithmetic on the float32 bit pattern -----------------------------------------------

// Largest exponent field of 8 float32 bit patterns.
__device__ __forceinline__ uint32_t block_exp(const uint32_t u[8]) {
  uint32_t E = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) E = max(E, (u[i] >> 23) & 0xFFu);
  return E;
}

// q for one element given the block exponent E: |x| * 2^(133-E) = m / 2^(E + 17 - e') with m the 24-bit significand
// (no implicit bit and e' = 1 for subnormals), rounded half to even, signed, clipped to [-128, 127].
// Infinities saturate (+127 / -128) as np.clip does; NaN is outside the contract.
__device__ __forceinline__ int32_t encode_elem(uint32_t u, uint32_t E) {
  const uint32_t e = (u >> 23) & 0xFFu;
  uint32_t m = u & 0x7FFFFFu;
  const uint32_t ee = e ? e : 1u;
  m |= e ? 0x800000u : 0u;
  const uint32_t s = E + 17u - ee;  // >= 16
  uint32_t mag = 0;
  if (s < 32u) {
    const uint32_t q = m >> s;
    const uint32_t rem = m & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1u);
    mag = q + ((rem > half) | ((rem == half) & (q & 1u)));
  }
  const bool neg = (u >> 31) != 0;
  int32_t v = neg ? -(int32_t)mag : (int32_t)mag;
  if (e == 255u) v = neg ? -128 : 127;
  return min(v, 127);
}

// bf16 bit pattern of q * 2^(E-133), built with integers (exact for every E, including bf16 subnormal results).
// q == 0 gives +0, as from_bfp16 does; a product of 2^128 or more (E = 254 with q = -128, E = 255 with |q| >= 64)
// gives +-inf, as from_bfp16's float32 product does.
__device__ __forceinline__ uint32_t decode_bf16_bits(int32_t q, uint32_t E) {
  if (q == 0) return 0u;
  const uint32_t sign = q < 0 ? 0x8000u : 0u;
  const uint32_t a = (uint32_t)(q < 0 ? -q : q);  // 1..128
  const int p = 31 - __clz(a);                      // leading one, 0..7
  const int be = p + (int)E - 6;                    // biased exponent of the result
  uint32_t bits;
  if (be >= 255)
    bits = 0x7F80u;  // overflow: infinity
  else if (be >= 1)
    bits = ((uint32_t)be << 7) | ((a << (7 - p)) & 0x7Fu);
  else
    bits = a << E;  // subnormal: value / 2^-133
  return sign | bits;
}

// ---- fast decode for the GEMM's B operand ---------------------------------------------------------------------

// 2^(E-133) as float (subnormal for E < 7).
__device__ __forceinline__ float block_scale(uint32_t E) { return __builtin_amdgcn_ldexpf(1.0f, (int)E - 133); }

// Pack the high halves of two float32 (both exactly representable in bf16) into one bf16x2 word: lo | hi << 16.
__device__ __forceinline__ uint32_t pack_hi(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// One 9-byte block held in a 12-byte window w0..w2 that starts `o` bytes before it (o = 0..3) -> 8 bf16 values.
// q bytes are sign-extended to float (one SDWA convert each), scaled by the block exponent, and truncated to bf16
// (exact: |q| < 2^8 fits bf16's significand).
__device__ __forceinline__ bf16x8 decode_window(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t o) {
  const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, o);  // bytes o..o+3: E q0 q1 q2
  const uint32_t hi = __builtin_amdgcn_alignbyte(w2, w1, o);  // bytes o+4..o+7: q3 q4 q5 q6
  const uint32_t q7 = w2 >> (8u * o);                         // byte o+8 in bits 0..7
  const float s = block_scale(lo & 0xFFu);
  const float f0 = (float)(int8_t)(lo >> 8) * s;
  const float f1 = (float)(int8_t)(lo >> 16) * s;
  const float f2 = (float)(int8_t)(lo >> 24) * s;
  const float f3 = (float)(int8_t)(hi) * s;
  const float f4 = (float)(int8_t)(hi >> 8) * s;
  const float f5 = (float)(int8_t)(hi >> 16) * s;
  const float f6 = (float)(int8_t)(hi >> 24) * s;
  const float f7 = (float)(int8_t)(q7) * s;
  u32x4 r;
  r.x = pack_hi(f0, f1);
  r.y = pack_hi(f2, f3);
  r.z = pack_hi(f4, f5);
  r.w = pack_hi(f6, f7);
  return __builtin_bit_cast(bf16x8, r);
}

// Byte address of the 12-byte window holding the 9-byte block at byte offset b9: start rounded down to 4 bytes.
// For a stream whose block count is a multiple of 8 the window never leaves the stream: a window passes the block's
// end only when b9 % 4 == 0, i.e. for blocks 0 mod 4, which are never the last block.
struct Window {
  uint32_t w0, w1, w2;
};
__device__ __forceinline__ Window load_window(const uint8_t* base, int64_t b9) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(base + (b9 & ~(int64_t)3));
  return Window{p[0], p[1], p[2]};
}

// Same block, safe for any stream length: a window that would pass the end of a stream of `nblocks` blocks is
// replaced by byte loads.
__device__ __forceinline__ Window load_window_safe(const uint8_t* base, int64_t blk, int64_t nblocks) {
  const int64_t b9 = blk * 9;
  if ((blk & 3) != 0 || blk + 1 < nblocks) return load_window(base, b9);
  uint32_t w[3] = {0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 9; i++) w[i >> 2] |= (uint32_t)base[b9 + i] << (8 * (i & 3));
  return Window{w[0], w[1], w[2]};
}

// ---- exact quantize of 8 bf16 values (as 4 packed words) to bfp16, returned as bf16 words ----------------------
__device__ __forceinline__ u32x4 quantize_bf16x8(u32x4 v, uint32_t* E_out = nullptr, int32_t* q_out = nullptr) {
  uint32_t u[8];
  u[0] = v.x << 16; u[1] = v.x & 0xFFFF0000u;
  u[2] = v.y << 16; u[3] = v.y & 0xFFFF0000u;
  u[4] = v.z << 16; u[5] = v.z & 0xFFFF0000u;
  u[6] = v.w << 16; u[7] = v.w & 0xFFFF0000u;
  const uint32_t E = block_exp(u);
  uint32_t b[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int32_t q = encode_elem(u[i], E);
    if (q_out) q_out[i] = q;
    b[i] = decode_bf16_bits(q, E);
  }
  if (E_out) *E_out = E;
  u32x4 r;
  r.x = b[0] | (b[1] << 16);
  r.y = b[2] | (b[3] << 16);
  r.z = b[4] | (b[5] << 16);
  r.w = b[6] | (b[7] << 16);
  return r;
}

// Float fast path of the encoder for a block exponent E in 8..237 (kFastEMin..kFastEMax). With s = 2^(133-E) and t = 127 * 2^(E-133):
// fma(min(x, t), s, 1.5 * 2^23) scales exactly (a power of two) and rounds once, half to even, at integer
// granularity, because the 1.5 * 2^23 term is even and |x * s| < 2^22. The result's bits are 0x4B400000 + q, so the
// low byte is q in two's complement; min(x, t) clips q at 127, and q >= -128 holds by the choice of E. Values too small
// to reach 0.5 after scaling round to 0, as the integer encoder gives. (f - 1.5 * 2^23) * 2^(E-133) is the decoded
// value, exactly, and a normal float. Above E = 237 the constant -1.5 * 2^23 * 2^(E-133) of decode_fast overflows
// float32, so such blocks (values of 2^111 and more) take the integer encoder. From E = 8 up every float32 subnormal
// element scales below 0.5 (x < 2^-126, s <= 2^125) and rounds to 0 whether or not the hardware flushes denormals, so
// the fast path's result does not depend on the denormal mode; at E = 7 a subnormal in [2^-127, 2^-126) would scale
// into [0.5, 1), so E <= 7 takes the integer encoder.
constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
constexpr uint32_t kFastEMin = 8u, kFastEMax = 237u;
struct BlockScale {
  float s, t, inv;  // 2^(133-E), 127 * 2^(E-133), 2^(E-133)
};
__device__ __forceinline__ BlockScale block_scales(uint32_t E) {
  return BlockScale{__uint_as_float((260u - E) << 23), __uint_as_float(0x42FE0000u + ((E - 133u) << 23)),
                    __uint_as_float((E - 6u) << 23)};
}
// min(x, t) as one v_med3_f32 against -FLT_MAX: x is finite here, so no NaN quieting is needed (fminf would add a
// canonicalising v_max of each operand)
__device__ __forceinline__ float encode_fast(float x, const BlockScale& k) {
  return __builtin_fmaf(__builtin_amdgcn_fmed3f(x, -3.402823466e38f, k.t), k.s, kMagic);
}
// Decoded value of an encode_fast result: f * 2^(E-133) is exact, and adding -1.5 * 2^23 * 2^(E-133) leaves
// q * 2^(E-133), representable, so the fma does not round (+0 for q = 0)
__device__ __forceinline__ float decode_fast(float f, const BlockScale& k, float off) { return __builtin_fmaf(f, k.inv, off); }
__device__ __forceinline__ uint32_t decode_fast_bits(float f, const BlockScale& k) {
  return __float_as_uint(decode_fast(f, k, -kMagic * k.inv)) >> 16;
}

// Encode 8 float32 bit patterns (finite) to one block: returns E, writes q (the int8 value in the low byte of each
// word: callers store the byte) and the decoded values as bf16, packed two per word (value 2i in the low half of word
// i). The largest exponent field is that of the largest magnitude. For block exponents 8..237 the float fast path
// above is used; other exponents (subnormal blocks, very large ones, and infinities, which saturate) take the integer
// encoder.
__device__ __forceinline__ uint32_t encode_block(const uint32_t u[8], int32_t q[8], u32x4& bw) {
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(__uint_as_float(u[i])));
  const uint32_t E = __float_as_uint(mx) >> 23;
  if (E >= kFastEMin && E <= kFastEMax) {
    const BlockScale k = block_scales(E);
    const float off = -kMagic * k.inv;
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float f = encode_fast(__uint_as_float(u[i]), k);
      q[i] = (int32_t)__float_as_uint(f);
      d[i] = decode_fast(f, k, off);
    }
    bw = u32x4{pack_hi(d[0], d[1]), pack_hi(d[2], d[3]), pack_hi(d[4], d[5]), pack_hi(d[6], d[7])};
  } else {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      q[i] = encode_elem(u[i], E);
      b[i] = decode_bf16_bits(q[i], E);
    }
    bw = u32x4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
  }
  return E;
}

// One element quantized with a given block exponent E (the block's largest exponent field, found by the caller):
// the bf16 bits of its bfp16 value. Same arithmetic as encode_block.
__device__ __forceinline__ uint32_t quantize_with_exp(uint32_t u, uint32_t E) {
  if (E >= kFastEMin && E <= kFastEMax) {
    const BlockScale k = block_scales(E);
    return decode_fast_bits(encode_fast(__uint_as_float(u), k), k);
  }
  return decode_bf16_bits(encode_elem(u, E), E);
}

// Waits until at most N vector-memory loads of this wave are outstanding (s_waitcnt vmcnt(N), gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// ---- XCD-aware workgroup order -----------------------------------------------------------------------------------
// Workgroups are dispatched round robin over the 8 XCDs (pid % 8). Map them so that each XCD works on a contiguous
// range of logical tiles, which then share operands in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int pid, int nwg) {
  constexpr int kXcd = 8;
  const int xcd = pid % kXcd, local = pid / kXcd;
  const int per = (nwg + kXcd - 1) / kXcd;
  const int rem = nwg % kXcd;
  if (rem == 0 || xcd < rem) return xcd * per + local;
  return rem * per + (xcd - rem) * (per - 1) + local;
}

}  // namespace rl
