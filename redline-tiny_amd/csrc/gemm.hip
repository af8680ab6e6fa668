// bfp16-weight GEMM for gfx950: C = epilogue(A @ B), B streamed from HBM in the packed b_layout(64, 128) order that
// redline/pack_weights.py:72-79 writes, decoded to bf16 on chip, bf16 MFMA (16x16x32) with fp32 accumulation.
//
// Replaces the ATB microkernels (kernels/atb3/mm_bfp_mixed.cc:61, mm_bfp_rho.cc:64, kernels/vlm/mm_bfp_c16.cc:62)
// and the SwiGLU-flush GEMM (kernels/atb3/mm_bfp_swiglu.cc:88) behind forward.gemm / NPU.run (redline/forward.py).
//
// Two whole-K kernels, both for bf16 A (bfp16 values), one workgroup per CU (160 KB of LDS), K steps of 64:
//   * gemm8_kernel: 8 waves (two per SIMD), tiles of 32 MF rows x 256 columns. Each K step the waves decode the
//     tile's raw B blocks once into an LDS stage of MFMA operands; A arrives by direct-to-LDS buffer loads.
//   * gemm4w_kernel: 4 waves (one per SIMD), tiles of 64 MF rows x 128 columns, each wave 16 MF rows x all 128
//     columns, so per MFMA it decodes half the B blocks and reads a third fewer operand bytes from LDS.
// A planner picks the kernel and fragment count per shape from a rounds-of-the-CUs cost model, and may run the
// rows past the last full round as a second launch of shorter tiles. Small-M, deep-K shapes may split K across
// workgroups (fp32 partials in a workspace, summed by gemm_reduce_kernel). A non-bf16 A (the NPU's packed
// a_layout stream, packed row blocks, or bf16 to be quantized) is first staged as bf16 in one HBM-bound pass.
// The epilogue (bias, GELU or SwiGLU, gate * v + residual, bf16 rounding, re-quantize) runs from an LDS tile of
// the fp32 accumulators.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kAStage = BM * BK * 2;  // bytes of one A stage
constexpr int kTileBytes = 64 * 128 * 9 / 8;  // one b_layout tile (64 K x 128 N)
// Tiles are walked kGroupM M-tiles at a time within each XCD's contiguous range: the 32 CUs of an XCD then hold a
// block of 4 M-tiles x 8 N-tiles, which fetches fewer A + B bytes through L2 than 8 x 4 (A tiles are the larger ones).
constexpr int kGroupM = 4;

struct GemmDesc {
  const void* A;
  int64_t lda;
  const uint8_t* B;
  uint16_t* C;
  int64_t ldc;
  int32_t M, N, K;
  int32_t act, flags;
  int32_t gate_split;
  const float* bias;
  const float* gate;
  const uint16_t* res;
  int64_t ldr;
  int32_t tiles_m, tiles_n, tile_start;
  int32_t ksplit;  // K pieces: 1 = whole K; > 1 = each piece writes fp32 partials to `part`
  float* part;     // [ksplit][M][N] fp32 partial sums of the pieces, summed by gemm_reduce_kernel
  uint8_t* pk;       // NULL, or the output's bfp16 blocks in pk_order (RL_ORDER_C_ATB or RL_ORDER_A_LAYOUT)
  int32_t pk_order;
  int32_t c_atb;     // C (if not NULL) is flat in the c_layout_atb(., 128, 128) element order instead of row major
  int32_t prow;      // row of the whole output at this descriptor's row 0 (a second launch's rows start past it)
};

template <int G>
struct GemmArgs {
  GemmDesc d[G];
  int32_t n;
};

// 16-byte chunk swizzle of the A tile: chunk c of row r is stored at chunk c ^ swz(r). A wave's ds_read_b128 of one
// chunk column over 16 consecutive rows then spreads over all banks.
__device__ __forceinline__ int a_swz(int r) { return (r >> 1) & 7; }

// silu(x) = x * sigmoid(x) with the hardware exp2 and reciprocal (about 1e-6 relative; the epilogue rounds to bf16)
__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

__device__ __forceinline__ float gelu_tanh_f(float x) {
  // x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3)
  const float u2 = 1.5957691216057308f * (x + 0.044715f * x * x * x);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * u2));
}

// Re-quantize one block of 8 bf16 values (4 packed words) to bfp16, returned as bf16 words: the encoder's float fast
// path (encode_fast / decode_fast: one exact power-of-two scaling and one half-to-even rounding per value) for block
// exponents 8..237, the integer encoder otherwise, so the result equals the integer encoder's and does not depend on
// the denormal mode. -0 comes back as +0, as from_bfp16 gives it.
__device__ __forceinline__ uint32_t block_exp8(u32x4 o) {
  const uint32_t w[4] = {o.x, o.y, o.z, o.w};
  uint32_t E = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) E = max(E, max((w[k] >> 7) & 0xFFu, (w[k] >> 23) & 0xFFu));
  return E;
}
// the fast path of requantize8 for a block whose exponent E is in kFastEMin..kFastEMax
__device__ __forceinline__ u32x4 requantize8_fast(u32x4 o, uint32_t E) {
  const uint32_t w[4] = {o.x, o.y, o.z, o.w};
  const BlockScale sc = block_scales(E);
  const float off = -kMagic * sc.inv;
  uint32_t r[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float lo = decode_fast(encode_fast(__uint_as_float(w[k] << 16), sc), sc, off);
    const float hi = decode_fast(encode_fast(__uint_as_float(w[k] & 0xFFFF0000u), sc), sc, off);
    r[k] = pack_hi(lo, hi);
  }
  return u32x4{r[0], r[1], r[2], r[3]};
}
__device__ __forceinline__ u32x4 requantize8(u32x4 o) {
  const uint32_t w[4] = {o.x, o.y, o.z, o.w};
  const uint32_t E = block_exp8(o);
  if (E < kFastEMin || E > kFastEMax) return quantize_bf16x8(o);
  const BlockScale sc = block_scales(E);
  const float off = -kMagic * sc.inv;
  uint32_t r[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float lo = decode_fast(encode_fast(__uint_as_float(w[k] << 16), sc), sc, off);
    const float hi = decode_fast(encode_fast(__uint_as_float(w[k] & 0xFFFF0000u), sc), sc, off);
    r[k] = pack_hi(lo, hi);
  }
  return u32x4{r[0], r[1], r[2], r[3]};
}

// requantize8_fast that also returns the blocks' q bytes: q0..q3 in qw[0], q4..q7 in qw[1] (the low byte of each
// encode_fast result is q in two's complement)
__device__ __forceinline__ u32x4 requantize8_fast_q(u32x4 o, uint32_t E, uint32_t (&qw)[2]) {
  const uint32_t w[4] = {o.x, o.y, o.z, o.w};
  const BlockScale sc = block_scales(E);
  const float off = -kMagic * sc.inv;
  uint32_t r[4], qp[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float flo = encode_fast(__uint_as_float(w[k] << 16), sc);
    const float fhi = encode_fast(__uint_as_float(w[k] & 0xFFFF0000u), sc);
    r[k] = pack_hi(decode_fast(flo, sc, off), decode_fast(fhi, sc, off));
    qp[k] = __builtin_amdgcn_perm(__float_as_uint(fhi), __float_as_uint(flo), 0x0c0c0400u);
  }
  qw[0] = qp[0] | (qp[1] << 16);
  qw[1] = qp[2] | (qp[3] << 16);
  return u32x4{r[0], r[1], r[2], r[3]};
}
// the integer encoder of requantize8 with the q bytes as in requantize8_fast_q; not inlined: it serves only blocks of
// extreme exponents (E < 8, E > 237), and inline it would take registers from every packed-output epilogue. The
// result comes back by value (registers), not through memory.
struct ReqQ {
  u32x4 r;
  uint32_t q0, q1;
};
__device__ __attribute__((noinline)) ReqQ requantize8_int_qv(u32x4 o) {
  int32_t q[8];
  const u32x4 r = quantize_bf16x8(o, nullptr, q);
  return ReqQ{r, (q[0] & 0xFFu) | ((q[1] & 0xFFu) << 8) | ((q[2] & 0xFFu) << 16) | ((uint32_t)q[3] << 24),
              (q[4] & 0xFFu) | ((q[5] & 0xFFu) << 8) | ((q[6] & 0xFFu) << 16) | ((uint32_t)q[7] << 24)};
}
__device__ __forceinline__ u32x4 requantize8_int_q(u32x4 o, uint32_t (&qw)[2]) {
  const ReqQ t = requantize8_int_qv(o);
  qw[0] = t.q0;
  qw[1] = t.q1;
  return t.r;
}

// Index of the block holding row r, columns c .. c + 7 (c % 8 == 0) of an (rows, nout) output in a packed order:
//   RL_ORDER_C_ATB: c_layout_atb(., 128, 128) (redline/npu_layouts.py:42-47), blocks (rg, cg, col, row, sbr, sbc,
//     br, bc, rib) with rg = r / 512, row = r / 128 % 4, sbr = r / 16 % 8, br = r / 8 % 2, rib = r % 8, cg = c / 1024,
//     col = c / 128 % 8, sbc = c / 16 % 8, bc = c / 8 % 2 (nout % 1024 == 0);
//   RL_ORDER_A_LAYOUT: a_layout(., 128, 64) (npu_layouts.py:18-22), blocks (mt, kt, sbr, bc, bis, rib) with
//     mt = r / 128, kt = c / 64, sbr = r / 16 % 8, bc = c / 8 % 8, bis = r / 8 % 2, rib = r % 8 (nout % 64 == 0).
// In both, rows 4j .. 4j + 3 of one 8-column block are 4 consecutive blocks (rib is the last digit).
__device__ __forceinline__ int64_t out_block(int order, int r, int c, int nout) {
  if (order == RL_ORDER_C_ATB) {
    const int64_t g = (int64_t)(r >> 9) * (nout >> 10) + (c >> 10);
    const int t = ((((((c >> 7) & 7) * 4 + ((r >> 7) & 3)) * 8 + ((r >> 4) & 7)) * 8 + ((c >> 4) & 7)) * 2 +
                   ((r >> 3) & 1)) * 2 + ((c >> 3) & 1);
    return (g * 8192 + t) * 8 + (r & 7);  // 8192 = 8 col x 4 row x 8 sbr x 8 sbc x 2 br x 2 bc
  }
  const int64_t g = (int64_t)(r >> 7) * (nout >> 6) + (c >> 6);
  return ((g * 8 + ((r >> 4) & 7)) * 8 + ((c >> 3) & 7)) * 16 + (r & 15);
}

// The 8 bf16 of output block (row, col .. col + 7): row major, or 8 consecutive elements of the ATB element order
__device__ __forceinline__ uint16_t* c_block(const GemmDesc& d, int row, int col, int nout) {
  if (d.c_atb) return d.C + 8 * out_block(RL_ORDER_C_ATB, d.prow + row, col, nout);
  return d.C + (int64_t)row * d.ldc + col;
}

// Four bfp16 blocks (exponents E[i], q0..q3 in ql[i], q4..q7 in qh[i]) as their 36 consecutive bytes
// [E0 q0..q7][E1 ...][E2 ...][E3 ...], written as 9 dwords (p is 4-byte aligned: a block index that is a multiple
// of 4 times 9 bytes)
__device__ __forceinline__ void store_blocks4(uint8_t* p, const uint32_t (&E)[4], const uint32_t (&ql)[4],
                                              const uint32_t (&qh)[4]) {
  uint32_t* w = reinterpret_cast<uint32_t*>(p);
  w[0] = E[0] | (ql[0] << 8);
  w[1] = (ql[0] >> 24) | (qh[0] << 8);
  w[2] = (qh[0] >> 24) | (E[1] << 8) | (ql[1] << 16);
  w[3] = (ql[1] >> 16) | (qh[1] << 16);
  w[4] = (qh[1] >> 16) | (E[2] << 16) | (ql[2] << 24);
  w[5] = (ql[2] >> 8) | (qh[2] << 24);
  w[6] = (qh[2] >> 8) | (E[3] << 24);
  w[7] = ql[3];
  w[8] = qh[3];
}

// Epilogue tile in LDS for 64 rows x 256 columns of fp32 accumulators, "row-quad" layout: the 4 values of rows
// 4q..4q+3 of column c are 16 contiguous bytes at float index (q * 256 + slot(c)) * 4, so a lane writes one MFMA
// accumulator (4 rows, one column) with one 16-byte store and a reader of 8 consecutive columns of 4 rows issues
// eight 16-byte loads. slot(c) = c ^ ((c >> 4) & 15) permutes columns inside their 16-column group, so that both the
// writers (16 consecutive columns) and the readers (the same column offset of 16 neighbouring 8-column blocks) cover
// all banks.
constexpr int kG8ThreadsDecl = 512;  // threads of the 8-wave kernel
constexpr int kEpFloats = 16 * 256 * 4;
static_assert(kEpFloats * 4 <= 3 * kAStage, "epilogue tile must fit the LDS allocation");
__device__ __forceinline__ int ep_slot(int c) { return c ^ ((c >> 4) & 15); }

// 8 values of one output block: bias, activation, gate / residual, bf16 rounding (RNE) and the optional bfp16
// re-quantize, all in fp32; returns the 8 bf16 as 4 words.
__device__ __forceinline__ u32x4 finish_bf16(const GemmDesc& d, int row, int ocol, int nout, float (&v)[8]) {
  if (d.gate || d.res) {
    f32x4 g4[2] = {f32x4{1.f, 1.f, 1.f, 1.f}, f32x4{1.f, 1.f, 1.f, 1.f}};  // NULL gate = 1
    if (d.gate) __builtin_memcpy(g4, d.gate + (row < d.gate_split ? nout : 0) + ocol, 32);
    u32x4 r = {0u, 0u, 0u, 0u};
    if (d.res) r = *reinterpret_cast<const u32x4*>(d.res + (int64_t)row * d.ldr + ocol);
    const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float gk = g4[k >> 2][k & 3];
      const float rk = __uint_as_float(k & 1 ? rw[k >> 1] & 0xFFFF0000u : rw[k >> 1] << 16);
      v[k] = rk + gk * v[k];
    }
  }
  return u32x4{pack_bf16_rne(v[0], v[1]), pack_bf16_rne(v[2], v[3]), pack_bf16_rne(v[4], v[5]),
               pack_bf16_rne(v[6], v[7])};
}
__device__ __forceinline__ u32x4 finish_block(const GemmDesc& d, int row, int ocol, int nout, float (&v)[8]) {
  u32x4 o = finish_bf16(d, row, ocol, nout, v);
  if (d.flags & RL_EP_QUANTIZE_OUT) o = requantize8(o);
  return o;
}

// finish_block for an output that also goes out packed (d.pk): the bf16 block (re-quantized only with
// RL_EP_QUANTIZE_OUT) and the packed block of the bf16 values, its exponent E and q bytes qw.
__device__ __forceinline__ u32x4 finish_block_pk(const GemmDesc& d, int row, int ocol, int nout, float (&v)[8],
                                                 uint32_t& E, uint32_t (&qw)[2]) {
  const u32x4 o = finish_bf16(d, row, ocol, nout, v);
  E = block_exp8(o);
  // the float fast path when every lane's block allows it (a wave-uniform test), else the integer encoder for all
  // lanes (it gives the fast path's bits wherever that applies)
  u32x4 oq;
  if (__builtin_amdgcn_ballot_w64(E < kFastEMin || E > kFastEMax) == 0)
    oq = requantize8_fast_q(o, E, qw);
  else
    oq = requantize8_int_q(o, qw);
  return (d.flags & RL_EP_QUANTIZE_OUT) ? oq : o;
}

// The 9 bytes of one packed block at p (any alignment)
__device__ __forceinline__ void store_block1(uint8_t* p, uint32_t E, const uint32_t (&qw)[2]) {
  p[0] = (uint8_t)E;
#pragma unroll
  for (int i = 0; i < 8; i++) p[1 + i] = (uint8_t)(qw[i >> 2] >> (8 * (i & 3)));
}

// Gate / residual, bf16 rounding and the optional re-quantize of rows row0..row0+3 of one 8-column block (v[i]:
// row i's values), as finish_block does for one row. All four rows are computed, rows past M on the last valid row's
// operands (the caller does not store them), and the re-quantize takes its float fast path for all four at once when
// every lane's blocks allow it (a wave-uniform test): the rows' dependency chains then interleave, which a wave with
// no other wave on its SIMD needs.
__device__ __forceinline__ void finish_rows4_bf16(const GemmDesc& d, int row0, int ocol, int nout, float (&v)[4][8],
                                                  u32x4 (&o)[4]) {
  if (d.gate || d.res) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = min(row0 + i, d.M - 1);
      // the row's 8 gate values as two 16-byte loads under a wave-uniform test (NULL gate = 1): a per-value test of
      // a per-lane pointer would branch around each load
      f32x4 g4[2] = {f32x4{1.f, 1.f, 1.f, 1.f}, f32x4{1.f, 1.f, 1.f, 1.f}};
      if (d.gate) __builtin_memcpy(g4, d.gate + (row < d.gate_split ? nout : 0) + ocol, 32);
      u32x4 r = {0u, 0u, 0u, 0u};
      if (d.res) r = *reinterpret_cast<const u32x4*>(d.res + (int64_t)row * d.ldr + ocol);
      const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float gk = g4[k >> 2][k & 3];
        const float rk = __uint_as_float(k & 1 ? rw[k >> 1] & 0xFFFF0000u : rw[k >> 1] << 16);
        v[i][k] = rk + gk * v[i][k];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
    o[i] = u32x4{pack_bf16_rne(v[i][0], v[i][1]), pack_bf16_rne(v[i][2], v[i][3]), pack_bf16_rne(v[i][4], v[i][5]),
                 pack_bf16_rne(v[i][6], v[i][7])};
}
__device__ __forceinline__ void finish_rows4(const GemmDesc& d, int row0, int ocol, int nout, float (&v)[4][8],
                                             u32x4 (&o)[4]) {
  finish_rows4_bf16(d, row0, ocol, nout, v, o);
  if (d.flags & RL_EP_QUANTIZE_OUT) {
    uint32_t E[4];
    bool slow = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      E[i] = block_exp8(o[i]);
      slow |= E[i] < kFastEMin || E[i] > kFastEMax;
    }
    if (__builtin_amdgcn_ballot_w64(slow) == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = requantize8_fast(o[i], E[i]);
    } else {
      // the integer encoder for all four blocks (it gives the fast path's bits wherever that applies), so neither
      // side shares the other's per-block branches
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = quantize_bf16x8(o[i]);
    }
  }
}

// Second half of the GEMM epilogue. The LDS tile holds fp32 values (bias, activation and the SwiGLU product already
// applied) of `nquads` row quads x W staged columns in the row-quad layout; staged column c is output column c0 + c.
// Each thread takes blocks of 4 rows x 8 columns, one 16-byte store per row (the 4-wave kernel: finish_rows4).
// kOut: the kernel variant for outputs in the reference's stream orders (d.pk, d.c_atb); without it those fields are
// not read, and the code is that of a row-major bf16 C alone.
template <int W, int NTH, bool kOut>
__device__ __forceinline__ void ep8_finish(const GemmDesc& d, const float* ep, int r0, int c0, int nquads, int nout,
                                          int tid) {
  constexpr int kBlocks = W / 8;
  if constexpr (NTH == kG8ThreadsDecl) {
    // the 8-wave kernel (two waves per SIMD, 256 registers each): one row at a time, which fits its registers; the
    // other wave on the SIMD hides the latencies
    for (int it = tid; it < nquads * kBlocks; it += NTH) {
      const int q = it / kBlocks, cb = it % kBlocks;
      const int col = c0 + 8 * cb;
      if (col >= nout) continue;
      f32x4 a[8];
#pragma unroll
      for (int k = 0; k < 8; k++) a[k] = *reinterpret_cast<const f32x4*>(ep + (q * W + ep_slot(8 * cb + k)) * 4);
      if (kOut && d.pk) {
        // packed output: a row quad is all inside M or all past it (M % 128 == 0); the last M-tile of a launch can
        // reach past M, and its quads there are skipped (their blocks would lie past the end of the packed stream).
        // The four rows' blocks are 36 consecutive bytes.
        if (r0 + 4 * q >= d.M) continue;
        uint32_t E[4], ql[4], qh[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int row = r0 + 4 * q + i;
          float v[8];
#pragma unroll
          for (int k = 0; k < 8; k++) v[k] = a[k][i];
          uint32_t qw[2];
          const u32x4 o = finish_block_pk(d, row, col, nout, v, E[i], qw);
          ql[i] = qw[0];
          qh[i] = qw[1];
          if (d.C) *reinterpret_cast<u32x4*>(c_block(d, row, col, nout)) = o;
        }
        store_blocks4(d.pk + 9 * out_block(d.pk_order, d.prow + r0 + 4 * q, col, nout), E, ql, qh);
        continue;
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = r0 + 4 * q + i;
        if (row >= d.M) break;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = a[k][i];
        const u32x4 o = finish_block(d, row, col, nout, v);
        *reinterpret_cast<u32x4*>(kOut ? c_block(d, row, col, nout) : d.C + (int64_t)row * d.ldc + col) = o;
      }
    }
    return;
  }
  for (int it = tid; it < nquads * kBlocks; it += NTH) {
    const int q = it / kBlocks, cb = it % kBlocks;
    const int col = c0 + 8 * cb;
    const int row0 = r0 + 4 * q;
    if (col >= nout || row0 >= d.M) continue;
    f32x4 a[8];
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = *reinterpret_cast<const f32x4*>(ep + (q * W + ep_slot(8 * cb + k)) * 4);
    if (kOut && d.pk) {
      // packed output, the four rows together (the quad is inside M, checked above, and then all four rows are,
      // M % 128 == 0), as finish_block_pk does per row but with one wave-uniform test for the float fast path of all
      // four blocks, so that their dependency chains interleave (1% faster than row by row); the four rows' blocks
      // are 36 consecutive bytes of the packed order
      float v4[4][8];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int k = 0; k < 8; k++) v4[i][k] = a[k][i];
      u32x4 o4[4];
      finish_rows4_bf16(d, row0, col, nout, v4, o4);
      uint32_t E[4], ql[4], qh[4];
      bool slow = false;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        E[i] = block_exp8(o4[i]);
        slow |= E[i] < kFastEMin || E[i] > kFastEMax;
      }
      const bool quant = (d.flags & RL_EP_QUANTIZE_OUT) != 0;
      if (__builtin_amdgcn_ballot_w64(slow) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t qw[2];
          const u32x4 oq = requantize8_fast_q(o4[i], E[i], qw);
          if (quant) o4[i] = oq;
          ql[i] = qw[0];
          qh[i] = qw[1];
        }
      } else {
        // the integer encoder for all four blocks (it gives the fast path's bits wherever that applies)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t qw[2];
          const u32x4 oq = requantize8_int_q(o4[i], qw);
          if (quant) o4[i] = oq;
          ql[i] = qw[0];
          qh[i] = qw[1];
        }
      }
      if (d.C) {
#pragma unroll
        for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4*>(c_block(d, row0 + i, col, nout)) = o4[i];
      }
      store_blocks4(d.pk + 9 * out_block(d.pk_order, d.prow + row0, col, nout), E, ql, qh);
      continue;
    }
    float v[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int k = 0; k < 8; k++) v[i][k] = a[k][i];
    u32x4 o[4];
    finish_rows4(d, row0, col, nout, v, o);
    if (kOut && !d.C) continue;
    // row major: the other rows at uniform strides of ldc; the ATB element order: the next 8 elements (rib is the
    // last block digit, and row0 % 4 == 0)
    uint16_t* const c = kOut ? c_block(d, row0, col, nout) : d.C + (int64_t)row0 * d.ldc + col;
    const int64_t rs = kOut && d.c_atb ? 8 : d.ldc;
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (row0 + i < d.M) *reinterpret_cast<u32x4*>(c + i * rs) = o[i];
  }
}

// The K-piece variant of ep8_finish: the LDS tile holds raw fp32 sums of `nquads` row quads x 256 computed columns
// (staged column c is column c0 + c); each thread stores blocks of 4 rows x 8 columns to plane `piece` of d.part.
__device__ __forceinline__ void ep8_partial(const GemmDesc& d, const float* ep, int r0, int c0, int nquads, int piece,
                                           int tid) {
  for (int it = tid; it < nquads * 32; it += kG8ThreadsDecl) {
    const int q = it >> 5, cb = it & 31;
    const int col = c0 + 8 * cb;
    if (col >= d.N) continue;
    f32x4 a[8];
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = *reinterpret_cast<const f32x4*>(ep + (q * 256 + ep_slot(8 * cb + k)) * 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * q + i;
      if (row >= d.M) break;
      float* dst = d.part + ((int64_t)piece * d.M + row) * d.N + col;
      *reinterpret_cast<f32x4*>(dst) = f32x4{a[0][i], a[1][i], a[2][i], a[3][i]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{a[4][i], a[5][i], a[6][i], a[7][i]};
    }
  }
}

// Sum of the K pieces' partials of a split GEMM, in piece order, then the epilogue: bias, activation (for SwiGLU
// silu(gate) * proj of the output block's gate and proj columns), gate / residual, bf16 rounding and the optional
// re-quantize, as the whole-K kernel applies them. One thread per output block of 8 columns.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const GemmDesc d) {
  const bool swiglu = d.act == RL_ACT_SWIGLU;
  const int nout = swiglu ? d.N / 2 : d.N;
  const int nb = nout / 8;
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= (int64_t)d.M * nb) return;
  const int row = (int)(b / nb), ocol = 8 * (int)(b % nb);
  const int64_t plane = (int64_t)d.M * d.N;
  const float* p = d.part + (int64_t)row * d.N;
  // computed columns of the block: ocol itself, or the gate columns 128 t + u and proj columns 128 t + 64 + u
  const int c0 = swiglu ? 128 * (ocol >> 6) + (ocol & 63) : ocol;
  float s0[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, s1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < d.ksplit; k++) {
    const float* q = p + k * plane + c0;
    const f32x4 a = *reinterpret_cast<const f32x4*>(q), a2 = *reinterpret_cast<const f32x4*>(q + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) { s0[e] += a[e]; s0[4 + e] += a2[e]; }
    if (swiglu) {
      const f32x4 g = *reinterpret_cast<const f32x4*>(q + 64), g2 = *reinterpret_cast<const f32x4*>(q + 68);
#pragma unroll
      for (int e = 0; e < 4; e++) { s1[e] += g[e]; s1[4 + e] += g2[e]; }
    }
  }
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float x = s0[e] + (d.bias ? d.bias[c0 + e] : 0.f);
    if (swiglu)
      v[e] = silu_f(x) * (s1[e] + (d.bias ? d.bias[c0 + 64 + e] : 0.f));
    else
      v[e] = d.act == RL_ACT_GELU_TANH ? gelu_tanh_f(x) : x;
  }
  if (d.pk) {
    uint32_t E, qw[2];
    const u32x4 o = finish_block_pk(d, row, ocol, nout, v, E, qw);
    store_block1(d.pk + 9 * out_block(d.pk_order, d.prow + row, ocol, nout), E, qw);
    if (d.C) *reinterpret_cast<u32x4*>(c_block(d, row, ocol, nout)) = o;
    return;
  }
  const u32x4 o = finish_block(d, row, ocol, nout, v);
  *reinterpret_cast<u32x4*>(c_block(d, row, ocol, nout)) = o;
}

// ---- 8-wave kernel for bf16 A ---------------------------------------------------------------------------------
// Tiles of 32 MF rows x 256 columns (MF = 8: 256 x 256) and K steps of 64, with 8 waves: one SIMD's MFMA pipe only
// stays full with two waves issuing. Wave (wm, wn) = (w / 4, w % 4) owns rows 16 MF wm .. +16 MF - 1 and the four
// 16-column groups in B slots 4 wn .. 4 wn + 3: MF x 4 MFMA accumulators.
//
// LDS (up to 160 KB): two A stages (tile rows x 64 bf16 with the 16-byte chunk swizzle, filled by direct-to-LDS
// buffer loads) and three B stages. A B stage holds the 2048 decoded blocks of the tile's two b_layout tiles, 16
// bytes each, as MFMA operands: slot s is one 16-column group x 64 K as two 1 KB fragments (K half h at 1024 h; lane
// l's block l at 16 frag_pos(l)). Groups are put in slots at decode time so that each wave's four groups are
// adjacent (for SwiGLU, gate groups
// {g, g+1} and proj groups {g+4, g+5} of one 128-column tile, so silu(gate) * proj pairs share lane and register).
//
// A K step is two phases, one per 32-deep half of K (32 MFMAs per wave). The operands of a phase are read into
// registers during the phase before, so MFMAs never wait on LDS: A fragment mf of the next phase is read right after
// the four MFMAs that consume A fragment mf of this phase (rotating registers); the next phase's B fragments are read
// first. Per step k:
//   phase 0: MFMAs on K half 0 of step k; read K half 1 of step k; load raw B(k+2) blocks r = 0, 1; decode raw
//            B(k+1) blocks r = 2, 3 into B stage (k+1) % 3; wait for A(k+1); barrier (publishes A(k+1), B(k+1)).
//   phase 1: MFMAs on K half 1 of step k; read K half 0 of step k+1; DMA A(k+2) into A stage k % 2 (its last reads
//            were in phase 0, before the barrier); load raw B(k+2) blocks r = 2, 3; decode raw B(k+2) blocks r = 0, 1
//            into B stage (k+2) % 3 (last read in phase 0 of step k-1).
// The loop body has no branches, so the compiler's wait counts are exact; loads past the last step re-read step KT-1
// and land in stages that are never read again.
constexpr int kG8Threads = 512;
constexpr int kBStage = 2 * 1024 * 16;  // decoded blocks of two 64 x 128 tiles, 16 bytes each

// Position of block m (0..63) of a decoded B fragment inside its 1 KB: a 4 x 4 transpose within each group of 16
// blocks, with bit 2 flipped in odd groups.
__device__ __forceinline__ int frag_pos(int m) {
  return (m & ~15) | ((((m & 3) * 4 + ((m >> 2) & 3)) ^ (((m >> 4) & 1) * 4)));
}
static_assert(2 * kAStage + 3 * kBStage <= 160 * 1024, "LDS budget");

// Scheduling pattern for one quarter phase (kM MFMAs, one A fragment per four): the next phase's B fragment reads
// first (quarter 0), then the quarter's buffer loads (at most two: a burst of them stalls instruction issue behind a
// full address queue), then the MFMAs with kValu VALU ops after each and one A fragment read after every four; what
// remains (VALU, the LDS store of a decoded block) goes last.
template <int kM, int kB, int kLoads, int kValu>
__device__ __forceinline__ void quarter_schedule() {
  constexpr int kMfma = 0x008, kValuM = 0x002, kVmem = 0x060, kDsRead = 0x100, kDsWrite = 0x200;
  if (kB) __builtin_amdgcn_sched_group_barrier(kDsRead, kB, 0);
  if (kLoads) __builtin_amdgcn_sched_group_barrier(kVmem, kLoads, 0);
#pragma unroll
  for (int g = 0; g < kM; g++) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    if (kValu) __builtin_amdgcn_sched_group_barrier(kValuM, kValu, 0);
    if (g % 4 == 3) __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(kValuM, 64, 0);
  __builtin_amdgcn_sched_group_barrier(kDsWrite, 1, 0);
}

template <int G, int MF, bool kOut>
__global__ __launch_bounds__(kG8Threads, 1) void gemm8_kernel(const GemmArgs<G> args) {
  constexpr int TM = 32 * MF;                 // tile rows: MF 16-row fragments per wave, two waves down
  constexpr int kAS = TM * BK * 2;            // bytes of one A stage
  constexpr int kDma = (MF + 1) / 2;          // A loads of 8 rows per wave per stage
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kAS + 3 * kBStage];
  uint8_t* const bl = lds + 2 * kAS;

  const int pid = xcd_remap(blockIdx.x, gridDim.x);
  int di = 0;
  if constexpr (G > 1) {
    for (int i = 1; i < args.n; i++)
      if (pid >= args.d[i].tile_start) di = i;
  }
  const GemmDesc& d = args.d[di];
  int local = pid - d.tile_start;
  // K pieces: piece p covers K steps [p KT / ksplit, (p + 1) KT / ksplit) of every tile; tiles of one piece are
  // consecutive in launch order
  int piece = 0;
  if (d.ksplit > 1) {
    piece = local / (d.tiles_m * d.tiles_n);
    local -= piece * d.tiles_m * d.tiles_n;
  }
  const int group = local / (kGroupM * d.tiles_n);
  const int first_m = group * kGroupM;
  const int gm = min(d.tiles_m - first_m, kGroupM);
  const int in_group = local - group * kGroupM * d.tiles_n;
  const int m0 = (first_m + in_group % gm) * TM;
  const int n0 = (in_group / gm) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int KTt = d.K / BK;                    // K steps of the whole product (the b_layout tile stride)
  const int kb = piece * KTt / d.ksplit;        // this piece's first K step
  const int KT = (piece + 1) * KTt / d.ksplit - kb;
  const int N = d.N;
  const bool swiglu = d.act == RL_ACT_SWIGLU;

  // The 16-column groups of the tile in this wave's slots 4 wn + j: groups {g, g+1, g+4, g+5} of 128-column tile
  // wn / 2, g = 2 (wn % 2) (for SwiGLU the gate and proj groups of the same output columns; the other activations
  // use the same assignment)
  int grp[4];
  {
    const int g = 8 * (wn >> 1) + 2 * (wn & 1);
    grp[0] = g; grp[1] = g + 1; grp[2] = g + 4; grp[3] = g + 5;
  }
  const bool active = n0 + 16 * grp[0] < d.N;

  const __amdgpu_buffer_rsrc_t brs =
      __builtin_amdgcn_make_buffer_rsrc((void*)d.B, (short)0, (int)((int64_t)d.K * d.N / 8 * 9), 0x00020000);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      (void*)d.A, (short)0, (int)(((int64_t)d.M - 1) * d.lda * 2 + (int64_t)d.K * 2), 0x00020000);

  // B decode: thread t decodes the 4 consecutive blocks bi = 4 u .. 4 u + 3 (u = t % 256) of tile h = t / 256, a
  // 36-byte dword-aligned run at byte 36 u of the tile, so every byte's position is known at compile time. The run
  // is read as two halves of 5 dwords (blocks 0, 1: dwords 0..4; blocks 2, 3: dwords 4..8), each a 16-byte and a
  // 4-byte load. The blocks share column group c = u / 32 and K half u / 16 % 2 and are operand lanes 4 (u % 16)
  // + j of that fragment. The second tile reads zeros (offset past the stream, outside the range
  // check) when it lies beyond N; its decode is never read.
  const int64_t nt0 = n0 >> 7;
  const int bh = tid >> 8, bu = tid & 255;
  const uint32_t vb =
      nt0 + bh < (N >> 7) ? (uint32_t)(((nt0 + bh) * KTt + kb) * kTileBytes + 36 * bu) : 0x7FFFFFF0u;
  // group G = 8 h + c goes to LDS slot 4 (2 h + c / 2 % 2) + 2 (c / 4) + c % 2. Inside a 1 KB fragment, block m sits
  // at position frag_pos(m) (a 4 x 4 transpose in each 16 blocks, bit 2 flipped in odd 16s), not m: measured on
  // gfx950, this keeps both the operand reads (lane m reads block m) and the decode stores (store J: lane a writes
  // block 4 a + J; a 16-byte-per-lane store is served 8 lanes at a time, which must hit distinct 16-byte slots of
  // a 128-byte line) free of bank conflicts, where the plain order makes the stores 4-way conflicted.
  const int bc = bu >> 5, ba = bu & 15;
  uint32_t st_off[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    st_off[j] = (4 * (2 * bh + ((bc >> 1) & 1)) + 2 * (bc >> 2) + (bc & 1)) * 2048 + ((bu >> 4) & 1) * 1024 +
                16 * frag_pos(4 * ba + j);
  struct RawHalf {
    u32x4 v;
    uint32_t w;
  };
  RawHalf raw_a, raw_b;  // the run's first (blocks 0, 1) and second (blocks 2, 3) half
  // part 0: the half's first 4 dwords, part 1: its fifth
  auto load_part = [&](RawHalf& r, int half, int part, int k) {
    if (part == 0)
      r.v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, vb, k * kTileBytes + 16 * half, 0));
    else
      r.w = __builtin_amdgcn_raw_buffer_load_b32(brs, vb, k * kTileBytes + 16 * half + 16, 0);
  };
  // block j (0..3) of the run from its half: E at byte 9 j, q at bytes 9 j + 1 .. 9 j + 8, byte b of the run in
  // dword b / 4 - 4 half of the half
  auto decode_store = [&]<int J>(const RawHalf& r, uint8_t* stage) {
    const uint32_t d[5] = {r.v.x, r.v.y, r.v.z, r.v.w, r.w};
    constexpr int base = 16 * (J / 2);
    auto sbyte = [&](int b) { return (float)(int8_t)(d[(b - base) >> 2] >> (8 * ((b - base) & 3))); };
    constexpr int e = 9 * J;
    const float sc = block_scale((d[(e - base) >> 2] >> (8 * ((e - base) & 3))) & 0xFFu);
    u32x4 o;
    o.x = pack_hi(sbyte(e + 1) * sc, sbyte(e + 2) * sc);
    o.y = pack_hi(sbyte(e + 3) * sc, sbyte(e + 4) * sc);
    o.z = pack_hi(sbyte(e + 5) * sc, sbyte(e + 6) * sc);
    o.w = pack_hi(sbyte(e + 7) * sc, sbyte(e + 8) * sc);
    *reinterpret_cast<u32x4*>(stage + st_off[J]) = o;
  };
  // A: a stage is TM / 8 loads of 8 rows (64 lanes x 16 bytes); wave w issues loads g = g0 + i (i < kDma), g0 =
  // min(kDma w, TM / 8 - kDma) (a wave past the end repeats its neighbour's loads, which write the same bytes).
  // Load g covers row r = 8 g + lane / 8, 16-byte chunk (lane % 8) ^ swz(r). swz(r + 8) = swz(r) ^ 4, so loads i
  // and i + 2 differ by 16 rows only: two offset registers, recomputed at each use (the empty asm hides their values
  // from the compiler, which would otherwise keep kDma loop-invariant registers). Rows past M lie past the end of
  // the buffer resource and read zeros.
  const int g0 = min(kDma * wave, TM / 8 - kDma);
  const int ar0 = 8 * g0 + (lane >> 3);
  const uint32_t va_e =
      (uint32_t)(((int64_t)(m0 + ar0) * d.lda + (int64_t)kb * BK + ((lane & 7) ^ a_swz(ar0)) * 8) * 2);
  const uint32_t va_o =
      (uint32_t)(((int64_t)(m0 + ar0 + 8) * d.lda + (int64_t)kb * BK + ((lane & 7) ^ a_swz(ar0 + 8)) * 8) * 2);
  const uint32_t va_16 = (uint32_t)(16 * d.lda * 2);
  auto dma_a = [&](int stage, int k, int i) {
    uint32_t v = (i & 1) ? va_o : va_e;
    asm volatile("" : "+v"(v));
    uint8_t* dst = lds + stage * kAS + 8 * (g0 + i) * (BK * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (__attribute__((address_space(3))) void*)dst, 16,
                                             v + (i >> 1) * va_16, k * BK * 2, 0, 0);
  };
  f32x4 acc[MF][4];
#pragma unroll
  for (int mf = 0; mf < MF; mf++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[mf][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int arow = lane & 15;
  const uint32_t aoff0 = 16 * MF * wm * (BK * 2) + arow * (BK * 2) + (((lane >> 4) ^ a_swz(arow)) << 4);
  const uint32_t aoff1 = 16 * MF * wm * (BK * 2) + arow * (BK * 2) + (((4 + (lane >> 4)) ^ a_swz(arow)) << 4);
  const uint32_t boff = 4 * wn * 2048 + 16 * frag_pos(lane);

  bf16x8 fa[MF], fb0[4], fb1[4];
  auto read_a = [&](const uint8_t* p, int mf) { return *reinterpret_cast<const bf16x8*>(p + mf * 16 * (BK * 2)); };
  auto read_b = [&](const uint8_t* p, int j) { return *reinterpret_cast<const bf16x8*>(p + j * 2048); };

  // prologue: B(0) decoded into stage 0 and A(0) landed; B(1) blocks 0, 1 decoded into stage 1, raw B(1) blocks 2, 3
  // and A(1) in flight; K half 0 of step 0 read into registers
  const int k1 = min(1, KT - 1);
#pragma unroll
  for (int i = 0; i < kDma; i++) dma_a(0, 0, i);
  load_part(raw_a, 0, 0, 0); load_part(raw_a, 0, 1, 0);
  load_part(raw_b, 1, 0, 0); load_part(raw_b, 1, 1, 0);
  wait_vm<0>();
  decode_store.template operator()<0>(raw_a, bl); decode_store.template operator()<1>(raw_a, bl);
  decode_store.template operator()<2>(raw_b, bl); decode_store.template operator()<3>(raw_b, bl);
  load_part(raw_a, 0, 0, k1); load_part(raw_a, 0, 1, k1);
  wait_vm<0>();
  decode_store.template operator()<0>(raw_a, bl + kBStage); decode_store.template operator()<1>(raw_a, bl + kBStage);
  // the loads in flight now are those of a phase 1, in its order, so the loop's wait counts hold on entry too
  load_part(raw_b, 1, 0, k1); load_part(raw_b, 1, 1, k1);
#pragma unroll
  for (int i = 0; i < kDma; i++) dma_a(1, k1, i);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; j++) fb0[j] = read_b(bl + boff, j);
#pragma unroll
  for (int mf = 0; mf < MF; mf++) fa[mf] = read_a(lds + aoff0, mf);

  // One phase of step k in four quarters (fragments Q MF / 4 .. (Q + 1) MF / 4 - 1, scheduling fences between them).
  // P = 0: MFMAs on K half 0 with
  // fb0, reads K half 1 of step k into fa / fb1, loads raw B(kl) blocks 0, 1 (quarters 0, 1), decodes raw B(k+1)
  // blocks 2, 3 into stage ds (quarters 0, 2). P = 1: MFMAs on K half 1 with fb1, reads K half 0 of step k+1 into
  // fa / fb0, loads raw B(kl) blocks 2, 3 (quarter 0) and DMAs A(kl) into A stage sa (quarters 1, 2), decodes raw
  // B(k+2) blocks 0, 1 into stage ds (quarters 0, 2).
  auto quarter = [&]<int P, int Q>(bf16x8(&cur)[4], bf16x8(&nxt)[4], const uint8_t* na, const uint8_t* nb,
                                   uint8_t* ds, int kl, int sa) {
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (Q == 0) {
#pragma unroll
      for (int j = 0; j < 4; j++) nxt[j] = read_b(nb, j);
    }
    if constexpr (P == 0) {
      if constexpr (Q < 2) load_part(raw_a, 0, Q, kl);
    } else {
      if constexpr (Q == 0) {
        load_part(raw_b, 1, 0, kl);
        load_part(raw_b, 1, 1, kl);
      } else {
        if constexpr (Q >= 1 && 2 * (Q - 1) < kDma) dma_a(sa, kl, 2 * (Q - 1));
        if constexpr (Q >= 1 && 2 * (Q - 1) + 1 < kDma) dma_a(sa, kl, 2 * (Q - 1) + 1);
      }
    }
    constexpr int lo = Q * MF / 4, hi = (Q + 1) * MF / 4;
#pragma unroll
    for (int mf = lo; mf < hi; mf++) {
#pragma unroll
      for (int j = 0; j < 4; j++) acc[mf][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[mf], cur[j], acc[mf][j], 0, 0, 0);
      fa[mf] = read_a(na, mf);
    }
    if constexpr (Q == 0 || Q == 2) {
      if constexpr (P == 0)
        decode_store.template operator()<2 + Q / 2>(raw_b, ds);
      else
        decode_store.template operator()<Q / 2>(raw_a, ds);
    }
    constexpr int kDq = kDma - 2 * (Q - 1);  // A loads left for quarters Q >= 1
    constexpr int kL = P == 0 ? (Q < 2 ? 1 : 0)
                              : (Q == 0 ? 2 : (Q <= 2 ? (kDq < 0 ? 0 : (kDq > 2 ? 2 : kDq)) : 0));
    quarter_schedule<4 * (hi - lo), Q == 0 ? 4 : 0, kL, (Q == 0 || Q == 2) ? 3 : 0>();
  };
  auto phase = [&]<int P>(bf16x8(&cur)[4], bf16x8(&nxt)[4], const uint8_t* na, const uint8_t* nb, uint8_t* ds, int kl,
                          int sa) {
    quarter.template operator()<P, 0>(cur, nxt, na, nb, ds, kl, sa);
    quarter.template operator()<P, 1>(cur, nxt, na, nb, ds, kl, sa);
    quarter.template operator()<P, 2>(cur, nxt, na, nb, ds, kl, sa);
    quarter.template operator()<P, 3>(cur, nxt, na, nb, ds, kl, sa);
    __builtin_amdgcn_sched_barrier(0);
  };

  int sb0 = 0, sb1 = 1, sb2 = 2;  // B stages of steps k, k+1, k+2
  for (int k = 0; k < KT; k++) {
    const int sa0 = k & 1;
    const int kl = min(k + 2, KT - 1);
    phase.template operator()<0>(fb0, fb1, lds + sa0 * kAS + aoff1, bl + sb0 * kBStage + 1024 + boff,
                                 bl + sb1 * kBStage, kl, sa0);
    wait_vm<2>();  // A(k+1) done; raw B(k+2) blocks 0, 1 may stay in flight
    __syncthreads();
    phase.template operator()<1>(fb1, fb0, lds + (sa0 ^ 1) * kAS + aoff0, bl + sb1 * kBStage + boff,
                                 bl + sb2 * kBStage, kl, sa0);
    const int t = sb0;
    sb0 = sb1; sb1 = sb2; sb2 = t;
  }
  wait_vm<0>();
  __syncthreads();

  // ---- epilogue --------------------------------------------------------------------------------------------
  // Bias and activation (and for SwiGLU the product silu(gate) * proj, whose operands share lane and register) are
  // applied in registers by all waves; the fp32 results are staged in LDS (row-quad layout, 128 KB) and finished
  // 8 columns at a time by all threads. SwiGLU stages the whole tile (256 rows x 128 output columns) at once, the
  // other activations TM / 2 rows x 256 columns per pass.
  float* ep = reinterpret_cast<float*>(lds);
  const int col_in = lane & 15;
  if (d.ksplit > 1) {
    // a K piece: the raw fp32 sums (no bias, activation or SwiGLU product) of TM / 2 rows x 256 columns per pass,
    // staged like the plain epilogue, then stored to the piece's partial plane
#pragma unroll
    for (int P = 0; P < 2; P++) {
      if (active && wm == P) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int c = ep_slot(16 * grp[j] + col_in);
#pragma unroll
          for (int mf = 0; mf < MF; mf++)
            *reinterpret_cast<f32x4*>(ep + ((4 * mf + (lane >> 4)) * 256 + c) * 4) = acc[mf][j];
        }
      }
      __syncthreads();
      ep8_partial(d, ep, m0 + TM / 2 * P, n0, TM / 8, piece, tid);
      __syncthreads();
    }
    return;
  }
  const int nout = swiglu ? N / 2 : N;
  float bj[4];
#pragma unroll
  for (int j = 0; j < 4; j++) bj[j] = (active && d.bias) ? d.bias[n0 + 16 * grp[j] + col_in] : 0.f;
  if (swiglu) {
    if (active) {
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        const int tc = 16 * grp[jj] + col_in;
        const int c = ep_slot(64 * (tc >> 7) + (tc & 63));
#pragma unroll
        for (int mf = 0; mf < MF; mf++) {
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; i++) v[i] = silu_f(acc[mf][jj][i] + bj[jj]) * (acc[mf][jj + 2][i] + bj[jj + 2]);
          *reinterpret_cast<f32x4*>(ep + ((4 * MF * wm + 4 * mf + (lane >> 4)) * 128 + c) * 4) = v;
        }
      }
    }
    __syncthreads();
    ep8_finish<128, kG8ThreadsDecl, kOut>(d, ep, m0, n0 / 2, TM / 4, nout, tid);
  } else {
    const bool gelu = d.act == RL_ACT_GELU_TANH;
#pragma unroll
    for (int P = 0; P < 2; P++) {
      if (active && wm == P) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int c = ep_slot(16 * grp[j] + col_in);
#pragma unroll
          for (int mf = 0; mf < MF; mf++) {
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; i++) {
              v[i] = acc[mf][j][i] + bj[j];
              if (gelu) v[i] = gelu_tanh_f(v[i]);
            }
            *reinterpret_cast<f32x4*>(ep + ((4 * mf + (lane >> 4)) * 256 + c) * 4) = v;
          }
        }
      }
      __syncthreads();
      ep8_finish<256, kG8ThreadsDecl, kOut>(d, ep, m0 + TM / 2 * P, n0, TM / 8, nout, tid);
      __syncthreads();
    }
  }
}

// ---- 4-wave kernel for bf16 A: one wave per SIMD, tiles of 64 MF rows x 128 columns ----------------------------
// With one wave per SIMD a wave may hold 512 registers, so wave w owns rows 16 MF w .. +16 MF - 1 and all eight
// 16-column groups of the tile: MF x 8 MFMA 16x16x32 accumulators. Against the 8-wave kernel (256 x 256 tiles,
// waves of 128 x 64), per MFMA this halves the B decode (one 64 x 128 b_layout tile per K step serves 64 MF rows)
// and cuts the operand reads from LDS by a third (8 A + 8 B fragments feed 64 MFMAs), the two costs that keep the
// matrix pipe from issuing back to back. For SwiGLU the tile's groups 0..3 are the gate columns and 4..7 the proj
// columns of the same 64 output columns, so silu(gate) * proj pairs share lane and register.
//
// LDS: two A stages (64 MF rows x 64 bf16, the 16-byte chunk swizzle, direct-to-LDS loads) and two B stages (the
// step's 1024 decoded blocks as MFMA operands, fragment (group g, K half h) at 1 KB * (2 g + h), lane l's block at
// 16 frag_pos(l)). Per K step k (A and B stage k % 2):
//   phase 0: MFMAs on K half 0; read K half 1 of step k; decode raw B(k+1) (4 blocks per thread) into B stage
//            (k+1) % 2, whose last reads were in phase 0 of step k-1; load raw B(k+2); wait for A(k+1); barrier.
//   phase 1: MFMAs on K half 1; read K half 0 of step k+1; DMA A(k+2) into A stage k % 2 (last read in phase 0).
// The loop body has no branches; loads past the last step re-read step KT-1 into stages never read again.
constexpr int kW4Threads = 256;
constexpr int kW4BStage = 1024 * 16;  // decoded blocks of one 64 x 128 b_layout tile
constexpr int kW4GroupM = 2;           // M-tiles per group in an XCD's tile range (x 16 N-tiles: 32 CUs)

// The K-piece store of the 4-wave kernel: the LDS tile holds raw fp32 sums of `nquads` row quads x 128 computed columns
// (staged column c is column c0 + c); each thread stores blocks of 4 rows x 8 columns to plane `piece` of d.part.
__device__ __forceinline__ void ep4_partial(const GemmDesc& d, const float* ep, int r0, int c0, int nquads, int piece,
                                            int tid) {
  for (int it = tid; it < nquads * 16; it += kW4Threads) {
    const int q = it >> 4, cb = it & 15;
    const int col = c0 + 8 * cb;
    f32x4 a[8];
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = *reinterpret_cast<const f32x4*>(ep + (q * 128 + ep_slot(8 * cb + k)) * 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + 4 * q + i;
      if (row >= d.M) break;
      float* dst = d.part + ((int64_t)piece * d.M + row) * d.N + col;
      *reinterpret_cast<f32x4*>(dst) = f32x4{a[0][i], a[1][i], a[2][i], a[3][i]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{a[4][i], a[5][i], a[6][i], a[7][i]};
    }
  }
}

// kReg: the variant for a SwiGLU GEMM with no bias, gate or residual, whole K, into a row-major bf16 C (the FFN up
// GEMMs). Its MFMAs take B as the first operand and A as the second, which gives the transposed accumulator tile
// with the same sums: lane l then holds row l % 16, columns 4 (l / 16) .. + 3 of each 16 x 16 fragment, so the
// gate and proj values of one output sit in one lane, and an output block of 8 columns in lanes l and l ^ 16. The
// epilogue runs from those registers (no LDS tile, no barrier).
template <int G, int MF, bool kOut, bool kReg = false>
__global__ __launch_bounds__(kW4Threads, 1) void gemm4w_kernel(const GemmArgs<G> args) {
  static_assert(MF >= 4 && MF <= 8, "four decode octets per phase, 8 x 8 accumulators at most");
  static_assert(!kReg || (G == 1 && !kOut), "the register epilogue serves one row-major GEMM");
  constexpr int TM = 64 * MF;       // tile rows: 16 MF per wave, four waves down
  constexpr int kAS = TM * BK * 2;  // bytes of one A stage
  constexpr int kDma = TM / 32;     // A loads of 8 rows per wave per stage
  static_assert(2 * kAS + 2 * kW4BStage <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kAS + 2 * kW4BStage];
  uint8_t* const bl = lds + 2 * kAS;

  const int pid = xcd_remap(blockIdx.x, gridDim.x);
  int di = 0;
  if constexpr (G > 1) {
    for (int i = 1; i < args.n; i++)
      if (pid >= args.d[i].tile_start) di = i;
  }
  const GemmDesc& d = args.d[di];
  int local = pid - d.tile_start;
  // K pieces: piece p covers K steps [p KT / ksplit, (p + 1) KT / ksplit) of every tile; the workgroups of a piece
  // are tiles_m * tiles_n apart
  int piece = 0;
  if (d.ksplit > 1) {
    piece = local / (d.tiles_m * d.tiles_n);
    local -= piece * d.tiles_m * d.tiles_n;
  }
  const int group = local / (kW4GroupM * d.tiles_n);
  const int first_m = group * kW4GroupM;
  const int gm = min(d.tiles_m - first_m, kW4GroupM);
  const int in_group = local - group * kW4GroupM * d.tiles_n;
  const int m0 = (first_m + in_group % gm) * TM;
  const int n0 = (in_group / gm) * 128;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS and row offsets stay scalar
  const int KTt = d.K / BK;                    // K steps of the whole GEMM
  const int kb = piece * KTt / d.ksplit;        // this piece's first K step
  const int KT = (piece + 1) * KTt / d.ksplit - kb;
  const bool swiglu = d.act == RL_ACT_SWIGLU;

  const __amdgpu_buffer_rsrc_t brs =
      __builtin_amdgcn_make_buffer_rsrc((void*)d.B, (short)0, (int)((int64_t)d.K * d.N / 8 * 9), 0x00020000);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      (void*)d.A, (short)0, (int)(((int64_t)d.M - 1) * d.lda * 2 + (int64_t)d.K * 2), 0x00020000);

  // B decode: thread t decodes blocks 4t .. 4t + 3 of the step's b_layout tile, a 36-byte dword-aligned run, read
  // with three loads (bytes 0..15, 16..31, 32..35). The four blocks are lanes 4 (t % 16) + J of fragment t / 16 =
  // 2 g + h (column group g, K half h).
  const uint32_t vb = (uint32_t)(((int64_t)(n0 >> 7) * KTt + kb) * kTileBytes + 36 * tid);
  uint32_t st_off[4];
#pragma unroll
  for (int j = 0; j < 4; j++) st_off[j] = (tid >> 4) * 1024 + 16 * frag_pos(4 * (tid & 15) + j);
  u32x4 raw0, raw1;  // bytes 0..15, 16..31 of the run
  uint32_t raw2;     // bytes 32..35
  auto load_raw = [&](int k, int part) {
    if (part == 0) raw0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, vb, k * kTileBytes, 0));
    if (part == 1)
      raw1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, vb, k * kTileBytes + 16, 0));
    if (part == 2) raw2 = __builtin_amdgcn_raw_buffer_load_b32(brs, vb, k * kTileBytes + 32, 0);
  };
  // block J (0..3) of the run: E at byte 9 J, q at bytes 9 J + 1 .. 9 J + 8 (compile-time byte positions)
  auto decode_store = [&]<int J>(uint8_t* stage) {
    const uint32_t dw[9] = {raw0.x, raw0.y, raw0.z, raw0.w, raw1.x, raw1.y, raw1.z, raw1.w, raw2};
    constexpr int base = 0;
    auto sbyte = [&](int b) { return (float)(int8_t)(dw[(b - base) >> 2] >> (8 * ((b - base) & 3))); };
    constexpr int e = 9 * J;
    const float sc = block_scale((dw[(e - base) >> 2] >> (8 * ((e - base) & 3))) & 0xFFu);
    u32x4 o;
    o.x = pack_hi(sbyte(e + 1) * sc, sbyte(e + 2) * sc);
    o.y = pack_hi(sbyte(e + 3) * sc, sbyte(e + 4) * sc);
    o.z = pack_hi(sbyte(e + 5) * sc, sbyte(e + 6) * sc);
    o.w = pack_hi(sbyte(e + 7) * sc, sbyte(e + 8) * sc);
    *reinterpret_cast<u32x4*>(stage + st_off[J]) = o;
  };
  // A: a stage is TM / 8 loads of 8 rows (64 lanes x 16 bytes); wave w issues loads g = kDma w + i. Load g covers
  // row r = 8 g + lane / 8, 16-byte chunk (lane % 8) ^ swz(r); swz(r + 16) = swz(r), so loads i and i + 2 differ by
  // 16 rows in the same chunk pattern: two base offsets plus a uniform row step, added in the vector offset (the
  // buffer range check covers the vector offset), the K step in the scalar offset. Rows past M lie past the end of
  // the buffer resource and read zeros.
  const int ar0 = 8 * kDma * wave + (lane >> 3);
  const uint32_t va_e = (uint32_t)(((int64_t)(m0 + ar0) * d.lda + ((lane & 7) ^ a_swz(ar0)) * 8 + kb * BK) * 2);
  const uint32_t va_o = (uint32_t)(((int64_t)(m0 + ar0 + 8) * d.lda + ((lane & 7) ^ a_swz(ar0 + 8)) * 8 + kb * BK) * 2);
  const uint32_t row16 = (uint32_t)(16 * d.lda * 2);
  auto dma_a = [&](int stage, int k, int i) {
    uint8_t* dst = lds + stage * kAS + 8 * (kDma * wave + i) * (BK * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (__attribute__((address_space(3))) void*)dst, 16,
                                             ((i & 1) ? va_o : va_e) + (uint32_t)(i >> 1) * row16, k * BK * 2, 0, 0);
  };

  f32x4 acc[MF][8];
#pragma unroll
  for (int mf = 0; mf < MF; mf++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[mf][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int arow = lane & 15;
  const uint32_t aoff0 = 16 * MF * wave * (BK * 2) + arow * (BK * 2) + (((lane >> 4) ^ a_swz(arow)) << 4);
  const uint32_t aoff1 = 16 * MF * wave * (BK * 2) + arow * (BK * 2) + (((4 + (lane >> 4)) ^ a_swz(arow)) << 4);
  const uint32_t boff = 16 * frag_pos(lane);
  bf16x8 fa[MF], fb0[8], fb1[8];
  auto read_a = [&](const uint8_t* p, int mf) { return *reinterpret_cast<const bf16x8*>(p + mf * 16 * (BK * 2)); };
  auto read_b = [&](const uint8_t* p, int j) { return *reinterpret_cast<const bf16x8*>(p + j * 2048); };

  // prologue: A(0) and B(0) in stage 0, A(1) in flight to stage 1, raw B(1) in registers (in flight), raw B(2)
  // issued in phase 0 of step 0
  const int k1 = min(1, KT - 1);
#pragma unroll
  for (int i = 0; i < kDma; i++) dma_a(0, 0, i);
  load_raw(0, 0);
  load_raw(0, 1);
  load_raw(0, 2);
  wait_vm<0>();
  decode_store.template operator()<0>(bl);
  decode_store.template operator()<1>(bl);
  decode_store.template operator()<2>(bl);
  decode_store.template operator()<3>(bl);
  load_raw(k1, 0);
  load_raw(k1, 1);
  load_raw(k1, 2);
#pragma unroll
  for (int i = 0; i < kDma; i++) dma_a(1, k1, i);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 8; j++) fb0[j] = read_b(bl + boff, j);
#pragma unroll
  for (int mf = 0; mf < MF; mf++) fa[mf] = read_a(lds + aoff0, mf);

  // One phase in octets (row fragment mf: its 8 MFMAs, then the next phase's fragment mf read into the same
  // registers), scheduling fences between octets. The next phase's B fragments are read one per octet (the last
  // octet reads what MF < 8 leaves), so LDS reads never come in bursts. P = 0 also decodes raw B(k+1) into stage ds
  // (block J in octet J) and issues the three loads of raw B(kl) in octets 4..6 (MF = 6: 3..5; MF = 4: all in the
  // last octet); P = 1 issues the DMA of A(kl) into A stage sa, two loads per octet.
  auto phase = [&]<int P>(bf16x8(&cur)[8], bf16x8(&nxt)[8], const uint8_t* na, const uint8_t* nb, uint8_t* ds, int kl,
                          int sa) {
    constexpr int kRaw0 = MF >= 7 ? 4 : 3;
#pragma unroll
    for (int mf = 0; mf < MF; mf++) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        if constexpr (kReg)
          acc[mf][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[j], fa[mf], acc[mf][j], 0, 0, 0);
        else
          acc[mf][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[mf], cur[j], acc[mf][j], 0, 0, 0);
        if (j == 1) nxt[mf] = read_b(nb, mf);
        if (mf == MF - 1 && j >= 2 && MF + j - 2 < 8) nxt[MF + j - 2] = read_b(nb, MF + j - 2);
      }
      fa[mf] = read_a(na, mf);
      if constexpr (P == 0) {
        if (mf == 0) decode_store.template operator()<0>(ds);
        if (mf == 1) decode_store.template operator()<1>(ds);
        if (mf == 2) decode_store.template operator()<2>(ds);
        if (mf == 3) decode_store.template operator()<3>(ds);
        if constexpr (MF >= 6) {
          if (mf >= kRaw0 && mf < kRaw0 + 3) load_raw(kl, mf - kRaw0);
        } else if (mf == MF - 1) {  // MF = 4, 5: all three after the last decode
          load_raw(kl, 0);
          load_raw(kl, 1);
          load_raw(kl, 2);
        }
        constexpr int kMfma = 0x008, kValu = 0x002, kDsWrite = 0x200;
        if (mf < 4) {
#pragma unroll
          for (int g = 0; g < 8; g++) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kValu, 3, 0);
          }
          __builtin_amdgcn_sched_group_barrier(kValu, 8, 0);
          __builtin_amdgcn_sched_group_barrier(kDsWrite, 1, 0);
        }
      } else {
        if (2 * mf < kDma) dma_a(sa, kl, 2 * mf);
        if (2 * mf + 1 < kDma) dma_a(sa, kl, 2 * mf + 1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  for (int k = 0; k < KT; k++) {
    const int s0 = k & 1, s1 = s0 ^ 1;
    const int kl = min(k + 2, KT - 1);
    // phase 0: MFMAs on half 0 of step k, read half 1 of step k, decode B(k+1) into stage s1, load raw B(k+2)
    phase.template operator()<0>(fb0, fb1, lds + s0 * kAS + aoff1, bl + s0 * kW4BStage + 1024 + boff,
                                 bl + s1 * kW4BStage, kl, s0);
    wait_vm<3>();  // A(k+1) done; the three raw B(k+2) loads may stay in flight
    __syncthreads();
    // phase 1: MFMAs on half 1, read half 0 of step k+1, DMA A(k+2) into stage s0
    phase.template operator()<1>(fb1, fb0, lds + s1 * kAS + aoff0, bl + s1 * kW4BStage + boff, nullptr, kl, s0);
  }
  wait_vm<0>();
  if constexpr (kReg) {
    // SwiGLU of the gate group g and the proj group g + 4 of one row fragment (16 outputs per lane) at a time, each
    // step of silu_f over all 16 so that independent exp2 / reciprocal latencies overlap (per output the operations
    // and their order are silu_f's), then bf16 rounding. Lane l = 16 k + r holds columns 4 k .. 4 k + 3 of each
    // group; one row swap (permlane16_swap: lanes of odd k trade with lanes of k - 1) per word of a group pair
    // (g0, g1) leaves lanes of even k with the 8-column block of g0 at columns 8 (k / 2) .., odd k with that of g1.
    // Each lane then re-quantizes (RL_EP_QUANTIZE_OUT) and stores whole blocks, as finish_rows4 does: the float
    // fast path when every block of the wave allows it, else the integer encoder for all (the same bits wherever
    // the fast path applies). The four lanes of a row store 64 contiguous bytes per group pair.
    const bool quant = (d.flags & RL_EP_QUANTIZE_OUT) != 0;
    const int k = lane >> 4;
    const int row0 = m0 + 16 * MF * wave + (lane & 15);
    uint16_t* const c0 = d.C + (int64_t)row0 * d.ldc + n0 / 2 + 16 * (k & 1) + 8 * (k >> 1);
#pragma unroll
    for (int mf = 0; mf < MF; mf++) {
      __builtin_amdgcn_sched_barrier(0);  // one row fragment at a time (interleaving them all runs out of registers)
      float x[16], u[16], e[16];
#pragma unroll
      for (int g = 0; g < 4; g++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          x[4 * g + i] = acc[mf][g][i];
          u[4 * g + i] = acc[mf][g + 4][i];
        }
#pragma unroll
      for (int t = 0; t < 16; t++) e[t] = -1.4426950408889634f * x[t];
#pragma unroll
      for (int t = 0; t < 16; t++) e[t] = __builtin_amdgcn_exp2f(e[t]);
#pragma unroll
      for (int t = 0; t < 16; t++) e[t] = 1.0f + e[t];
#pragma unroll
      for (int t = 0; t < 16; t++) e[t] = __builtin_amdgcn_rcpf(e[t]);
#pragma unroll
      for (int t = 0; t < 16; t++) e[t] = (x[t] * e[t]) * u[t];
      uint32_t w[8];  // w[2 g + h]: columns 4 k + 2 h, + 1 of group g
#pragma unroll
      for (int t = 0; t < 8; t++) w[t] = pack_bf16_rne(e[2 * t], e[2 * t + 1]);
      u32x4 o[2];  // block of group 2 p + (k & 1), columns 8 (k >> 1) .. + 7
#pragma unroll
      for (int p = 0; p < 2; p++) {
        const auto r0 = __builtin_amdgcn_permlane16_swap(w[4 * p], w[4 * p + 2], false, false);
        const auto r1 = __builtin_amdgcn_permlane16_swap(w[4 * p + 1], w[4 * p + 3], false, false);
        o[p] = u32x4{(uint32_t)r0[0], (uint32_t)r1[0], (uint32_t)r0[1], (uint32_t)r1[1]};
      }
      if (quant) {
        const uint32_t E0 = block_exp8(o[0]), E1 = block_exp8(o[1]);
        const bool slow = E0 < kFastEMin || E0 > kFastEMax || E1 < kFastEMin || E1 > kFastEMax;
        if (__builtin_amdgcn_ballot_w64(slow) == 0) {
          o[0] = requantize8_fast(o[0], E0);
          o[1] = requantize8_fast(o[1], E1);
        } else {
          o[0] = quantize_bf16x8(o[0]);
          o[1] = quantize_bf16x8(o[1]);
        }
      }
      if (row0 + 16 * mf < d.M) {
        *reinterpret_cast<u32x4*>(c0 + 16 * mf * d.ldc) = o[0];
        *reinterpret_cast<u32x4*>(c0 + 16 * mf * d.ldc + 32) = o[1];
      }
    }
    return;
  }
  __syncthreads();

  // ---- epilogue: bias and activation (SwiGLU: silu(gate) * proj of groups g and g + 4) in registers, fp32 results
  // staged in LDS in the row-quad layout, then finished 8 columns at a time by all threads (ep8_finish)
  float* ep = reinterpret_cast<float*>(lds);
  const int col_in = lane & 15;
  const int nout = swiglu ? d.N / 2 : d.N;
  float bj[8];
#pragma unroll
  for (int j = 0; j < 8; j++) bj[j] = d.bias ? d.bias[n0 + 16 * j + col_in] : 0.f;
  if (swiglu && d.ksplit == 1) {
    // without a bias (the FFN up GEMMs) the two adds per output are left out of this transcendental-bound pass.
    // Two fragments (8 outputs) go through each step of silu_f together, so that with one wave per SIMD the
    // exp2 / reciprocal latencies of independent outputs overlap; per output the operations and their order are
    // silu_f's.
    auto swiglu_pass = [&]<bool kBias>() {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int c = ep_slot(16 * g + col_in);
#pragma unroll
        for (int mf = 0; mf < MF; mf += 2) {
          const int nh = mf + 1 < MF ? 2 : 1;  // MF odd: the last step has one fragment
          float x[8], u[8], e[8];
#pragma unroll
          for (int h = 0; h < 2; h++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              x[4 * h + i] = h < nh ? (kBias ? acc[mf + h][g][i] + bj[g] : acc[mf + h][g][i]) : 0.f;
              u[4 * h + i] = h < nh ? (kBias ? acc[mf + h][g + 4][i] + bj[g + 4] : acc[mf + h][g + 4][i]) : 0.f;
            }
#pragma unroll
          for (int k = 0; k < 8; k++) e[k] = -1.4426950408889634f * x[k];
#pragma unroll
          for (int k = 0; k < 8; k++) e[k] = __builtin_amdgcn_exp2f(e[k]);
#pragma unroll
          for (int k = 0; k < 8; k++) e[k] = 1.0f + e[k];
#pragma unroll
          for (int k = 0; k < 8; k++) e[k] = __builtin_amdgcn_rcpf(e[k]);
#pragma unroll
          for (int k = 0; k < 8; k++) e[k] = (x[k] * e[k]) * u[k];
#pragma unroll
          for (int h = 0; h < 2; h++)
            if (h < nh)
              *reinterpret_cast<f32x4*>(ep + ((4 * MF * wave + 4 * (mf + h) + (lane >> 4)) * 64 + c) * 4) =
                  f32x4{e[4 * h], e[4 * h + 1], e[4 * h + 2], e[4 * h + 3]};
        }
      }
    };
    if (d.bias)
      swiglu_pass.template operator()<true>();
    else
      swiglu_pass.template operator()<false>();
    __syncthreads();
    ep8_finish<64, kW4Threads, kOut>(d, ep, m0, n0 / 2, TM / 4, nout, tid);
  } else {
    // bias and GELU chosen once per tile, so the staging loop has no per-value branches
    auto stage_pass = [&]<bool kBias, bool kGelu>() {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int c = ep_slot(16 * j + col_in);
#pragma unroll
        for (int mf = 0; mf < MF; mf++) {
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            v[i] = kBias ? acc[mf][j][i] + bj[j] : acc[mf][j][i];
            if (kGelu) v[i] = gelu_tanh_f(v[i]);
          }
          *reinterpret_cast<f32x4*>(ep + ((4 * MF * (wave & 1) + 4 * mf + (lane >> 4)) * 128 + c) * 4) = v;
        }
      }
    };
    // a K piece stages its raw fp32 sums (no bias, activation or SwiGLU product) and stores them to its partial plane
    const bool gelu = d.act == RL_ACT_GELU_TANH, part = d.ksplit > 1;
#pragma unroll
    for (int P = 0; P < 2; P++) {
      if ((wave >> 1) == P) {
        if (part)
          stage_pass.template operator()<false, false>();
        else if (gelu)
          stage_pass.template operator()<true, true>();
        else if (d.bias)
          stage_pass.template operator()<true, false>();
        else
          stage_pass.template operator()<false, false>();
      }
      __syncthreads();
      if (part)
        ep4_partial(d, ep, m0 + TM / 2 * P, n0, TM / 8, piece, tid);
      else
        ep8_finish<128, kW4Threads, kOut>(d, ep, m0 + TM / 2 * P, n0, TM / 8, nout, tid);
      __syncthreads();
    }
  }
}

template <int G>
static int fill_desc(GemmDesc& g, const void* A, int64_t lda, const uint8_t* B, uint16_t* C, int64_t ldc, int64_t M,
                     int64_t N, int64_t K, const rl_epilogue* ep, int32_t a_fmt, int tile_start) {
  int s = rl_validate_gemm(a_fmt, lda, ldc, M, N, K, ep);
  if (s) return s;
  if (!A || !B) return fail(RL_ERR_NULL, "A or B is NULL");
  if (!C && !(ep && ep->packed_out)) return fail(RL_ERR_NULL, "C is NULL and there is no packed output");
  if (ep && ep->packed_out && ((uintptr_t)ep->packed_out % 4))
    return fail(RL_ERR_ALIGN, "packed_out must be 4-byte aligned");
  if ((a_fmt == RL_A_BF16 || a_fmt == RL_A_BF16_QUANTIZE) && ((uintptr_t)A % 16))
    return fail(RL_ERR_ALIGN, "bf16 A must be 16-byte aligned");
  if (a_fmt >= RL_A_PACKED_ROWBLOCK && ((uintptr_t)A % 4)) return fail(RL_ERR_ALIGN, "packed A must be 4-byte aligned");
  if ((uintptr_t)B % 4) return fail(RL_ERR_ALIGN, "B must be 4-byte aligned");
  if ((uintptr_t)C % 16) return fail(RL_ERR_ALIGN, "C must be 16-byte aligned");
  if (K * N / 8 * 9 > INT32_MAX || (M - 1) * lda * 2 + K * 2 > INT32_MAX || M * K / 8 * 9 > INT32_MAX)
    return fail(RL_ERR_SHAPE, "an operand is above 2^31 bytes (buffer offsets are 32-bit)");
  if (a_fmt != RL_A_BF16 && M * K * 2 > INT32_MAX)
    return fail(RL_ERR_SHAPE, "the bf16 copy of A staged for this format is above 2^31 bytes");
  if (ep && ep->residual && (((uintptr_t)ep->residual % 16) || ep->ld_residual % 8))
    return fail(RL_ERR_ALIGN, "residual must be 16-byte aligned with ld_residual %% 8 == 0");
  if (ep && ep->bias && ((uintptr_t)ep->bias % 4)) return fail(RL_ERR_ALIGN, "bias must be 4-byte aligned");
  if (ep && ep->gate && ((uintptr_t)ep->gate % 4)) return fail(RL_ERR_ALIGN, "gate must be 4-byte aligned");
  g.A = A; g.lda = lda; g.B = B; g.C = C; g.ldc = ldc;
  g.M = (int32_t)M; g.N = (int32_t)N; g.K = (int32_t)K;
  g.act = ep ? ep->act : RL_ACT_NONE;
  g.flags = ep ? ep->flags : 0;
  g.bias = ep ? ep->bias : nullptr;
  g.gate = ep ? ep->gate : nullptr;
  g.gate_split = ep ? (int32_t)ep->gate_split_row : 0;
  g.res = ep ? ep->residual : nullptr;
  g.ldr = ep ? ep->ld_residual : 0;
  g.tiles_m = (int32_t)((M + BM - 1) / BM);
  g.tiles_n = (int32_t)((N + BN - 1) / BN);
  g.tile_start = tile_start;
  g.ksplit = 1;
  g.part = nullptr;
  g.pk = ep ? ep->packed_out : nullptr;
  g.pk_order = ep ? ep->packed_order : 0;
  g.c_atb = ep && ep->c_order == RL_C_ATB;
  g.prow = 0;
  return RL_OK;
}

// ---- launch planning for the 8-wave kernel ------------------------------------------------------------------------
// Workgroups hold a whole CU (160 KB of LDS), so a launch of T tiles runs in ceil(T / CUs) rounds, each as long as one
// tile: MF fragment rows per wave plus a part that does not shrink with the tile's rows (the B decode, prologue and
// epilogue), about 1.5 fragments' worth. The planner picks the fragment count, and may run the rows past a multiple
// of 256 as a second launch of shorter tiles, so that the last round is not a mostly idle full-height one.
constexpr double kTileFixed = 1.5, kSecondLaunch = 1.0;
constexpr int kMfChoices[] = {8, 7, 6, 4};

static int64_t tiles8(int64_t M, int64_t N, int mf) { return ((M + 32 * mf - 1) / (32 * mf)) * ((N + BN - 1) / BN); }
static double launch_cost(int64_t tiles, int mf, int cus) {
  return (double)((tiles + cus - 1) / cus) * (mf + kTileFixed);
}

struct Plan8 {
  int mf;         // fragments per wave of the (first) launch
  int64_t split;  // rows of the first launch; 0 = a single launch over all rows
  int mf_tail;    // fragments per wave of the second launch
};

static Plan8 plan8(int64_t M, int64_t N, int cus) {
  Plan8 best{8, 0, 8};
  double bc = 1e300;
  for (int mf : kMfChoices) {
    const double c = launch_cost(tiles8(M, N, mf), mf, cus);
    if (c < bc) { bc = c; best = Plan8{mf, 0, mf}; }
  }
  for (int64_t R = 256; R < M; R += 256) {
    const double c0 = launch_cost(tiles8(R, N, 8), 8, cus) + kSecondLaunch;
    for (int mf : kMfChoices) {
      const double c = c0 + launch_cost(tiles8(M - R, N, mf), mf, cus);
      if (c < bc) { bc = c; best = Plan8{8, R, mf}; }
    }
  }
  return best;
}

// ---- whole-K plan over both kernels -----------------------------------------------------------------------------
// A tile of the 4-wave kernel (64 mf rows x 128 columns) costs about mf + kTileFixed4 in the 8-wave kernel's units
// (a 256 x 256 tile of MF = 8 costs 9.5): per round of the CUs it runs ~6% faster than the 8-wave kernel on the same
// FLOPs, because it decodes half the B blocks per MFMA and reads a third fewer operand bytes from LDS (measured on
// the DiT FFN shapes, bit-identical results). Its last M-tile may be partial. The plan is one launch, or a first
// launch over rows [0, split) and a second one, of either kernel, over the rest (GELU: the 8-wave kernel only).
constexpr double kTileFixed4 = 0.9;
constexpr int kMf4Choices[] = {8, 7, 6, 4};

static int64_t tiles4(int64_t M, int64_t N, int mf) { return ((M + 64 * mf - 1) / (64 * mf)) * (N / 128); }
static double launch_cost4(int64_t tiles, int mf, int cus) {
  return (double)((tiles + cus - 1) / cus) * (mf + kTileFixed4);
}

struct PlanG {
  bool w4;        // the first launch runs the 4-wave kernel
  int mf;         // its fragment count
  int64_t split;  // rows of the first launch; 0 = one launch over all rows
  bool tail_w4;   // the second launch runs the 4-wave kernel
  int mf_tail;    // its fragment count
};

// RLBFP_GEMM_KERNEL=4w or 8w restricts the plan to plans whose first launch runs that kernel (for A/B measurements).
static int kernel_restriction() {
  static int v = -1;
  if (v < 0) {
    const char* e = getenv("RLBFP_GEMM_KERNEL");
    v = e && strcmp(e, "4w") == 0 ? 1 : (e && strcmp(e, "8w") == 0 ? 2 : 0);
  }
  return v;
}

static PlanG plan_gemm(int64_t M, int64_t N, int cus, int act, double* cost = nullptr) {
  // the tanh GELU epilogue's transcendentals cost more on one wave per SIMD than they save in the main loop
  // (measured at 4096 x 3072 x 3072: 102 against 97 us), so GELU stays on the 8-wave kernel unless forced
  const int only = kernel_restriction() ? kernel_restriction() : (act == RL_ACT_GELU_TANH ? 2 : 0);
  PlanG best{false, 8, 0, false, 8};
  double bc = 1e300;
  // the cheapest launch over `rows` rows: the 8-wave kernel, or (unless GELU) the 4-wave one
  auto best_tail = [&](int64_t rows, bool& w4_out, int& mf_out) {
    double c = 1e300;
    for (int mf : kMfChoices) {
      const double t = launch_cost(tiles8(rows, N, mf), mf, cus);
      if (t < c) { c = t; w4_out = false; mf_out = mf; }
    }
    if (act != RL_ACT_GELU_TANH) {
      for (int mf : kMf4Choices) {
        const double t = launch_cost4(tiles4(rows, N, mf), mf, cus);
        if (t < c) { c = t; w4_out = true; mf_out = mf; }
      }
    }
    return c;
  };
  if (only != 1) {
    const Plan8 p = plan8(M, N, cus);
    double c = launch_cost(tiles8(p.split ? p.split : M, N, p.mf), p.mf, cus);
    if (p.split) c += kSecondLaunch + launch_cost(tiles8(M - p.split, N, p.mf_tail), p.mf_tail, cus);
    bc = c;
    best = PlanG{false, p.mf, p.split, false, p.mf_tail};
  }
  if (only != 2) {
    for (int mf : kMf4Choices) {
      const double c = launch_cost4(tiles4(M, N, mf), mf, cus);
      if (c < bc) { bc = c; best = PlanG{true, mf, 0, false, 8}; }
      for (int64_t R = 64 * mf; R < M; R += 64 * mf) {
        bool tw = false;
        int mt = 8;
        const double c2 = launch_cost4(tiles4(R, N, mf), mf, cus) + kSecondLaunch + best_tail(M - R, tw, mt);
        if (c2 < bc) { bc = c2; best = PlanG{true, mf, R, tw, mt}; }
      }
    }
  }
  if (cost) *cost = bc;
  return best;
}

// ---- K split (one GEMM whose tiles fill few CUs: small M, deep K) ------------------------------------------------
// Model, in microseconds at the running clock: a tile of MF fragments costs kStepUs (MF + 1) per K step plus kTileUs
// (prologue and epilogue), and a launch of T tiles takes ceil(T / CUs) such rounds. The reduce launch reads the
// ksplit fp32 planes of M x N and writes the output: kReduceUs + bytes / kReduceBw. A split, with every piece in one
// round, is taken when the model puts it under 3/4 of the best whole-K launch.
constexpr double kStepUs = 0.18, kTileUs = 3.0, kReduceUs = 2.0, kReduceBw = 4.0e6;  // kReduceBw: bytes per us
constexpr double kStep4Us = 0.157;
constexpr int kMaxSplit = 16, kMinPieceSteps = 8;
constexpr int64_t kMaxSplitBytes = int64_t(1) << 30;

struct SplitPlan {
  int mf;            // fragments per wave
  int ks;            // K pieces; 1 = no split
  int64_t ws_bytes;  // fp32 partial planes: ks * M * N * 4
  bool w4;           // pieces on the 4-wave kernel (64 MF x 128 tiles) rather than the 8-wave one (32 MF x 256)
};

static SplitPlan plan_split(int64_t M, int64_t N, int64_t K, int cus) {
  SplitPlan best{8, 1, 0, false};
  if (cus <= 0) return best;
  const int64_t KT = K / BK;
  auto tile_us = [](int mf, int64_t steps) { return (double)steps * (mf + 1) * kStepUs + kTileUs; };
  // a 4-wave tile (the same MFMA work per MF) costs (MF + 0.9) kStep4Us per K step: 1.4 us per step at MF = 8 on
  // the FFN up GEMM, against 1.6 for the 8-wave tile
  auto tile4_us = [](int mf, int64_t steps) { return (double)steps * (mf + 0.9) * kStep4Us + kTileUs; };
  double whole = 1e300;
  for (int mf : kMfChoices) {
    const int64_t t = tiles8(M, N, mf);
    const double c = (double)((t + cus - 1) / cus) * tile_us(mf, KT);
    if (c < whole) whole = c;
  }
  double bc = 0.75 * whole;
  for (int w4 = 0; w4 < 2; w4++)
    for (int mf : kMfChoices) {
      const int64_t t = w4 ? tiles4(M, N, mf) : tiles8(M, N, mf);
      for (int ks = 2; ks <= kMaxSplit && t * ks <= cus && KT / ks >= kMinPieceSteps; ks++) {
        const int64_t bytes = (int64_t)ks * M * N * 4;
        if (bytes > kMaxSplitBytes) break;
        const int64_t steps = (KT + ks - 1) / ks;
        const double c =
            (w4 ? tile4_us(mf, steps) : tile_us(mf, steps)) + kReduceUs + (double)(bytes + M * N) / kReduceBw;
        if (c < bc) { bc = c; best = SplitPlan{mf, ks, bytes, w4 != 0}; }
      }
    }
  return best;
}

template <int G>
static void set_tiles8(GemmArgs<G>& args, int mf, int& total) {
  total = 0;
  for (int i = 0; i < args.n; i++) {
    GemmDesc& g = args.d[i];
    g.tiles_m = (int32_t)((g.M + 32 * mf - 1) / (32 * mf));
    g.tiles_n = (int32_t)((g.N + BN - 1) / BN);
    g.tile_start = total;
    total += g.tiles_m * g.tiles_n * g.ksplit;
  }
  for (int i = args.n; i < G; i++) args.d[i] = args.d[args.n - 1];
}

template <int G, bool kOut>
static int launch8_v(const GemmArgs<G>& args, int total_tiles, int mf, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(total_tiles), block(kG8Threads);
  switch (mf) {
    case 8: hipLaunchKernelGGL((gemm8_kernel<G, 8, kOut>), grid, block, 0, st, args); break;
    case 7: hipLaunchKernelGGL((gemm8_kernel<G, 7, kOut>), grid, block, 0, st, args); break;
    case 6: hipLaunchKernelGGL((gemm8_kernel<G, 6, kOut>), grid, block, 0, st, args); break;
    default: hipLaunchKernelGGL((gemm8_kernel<G, 4, kOut>), grid, block, 0, st, args); break;
  }
  return launch_status("rl_bfp16_gemm");
}

// The kernel variant for the descriptors: the stream-order outputs (packed blocks, ATB-ordered C) compile into a
// kernel of their own, so that the row-major kernels keep their register allocation.
template <int G>
static bool wants_out_variant(const GemmArgs<G>& args) {
  for (int i = 0; i < args.n; i++)
    if (args.d[i].pk || args.d[i].c_atb) return true;
  return false;
}
template <int G>
static int launch8(const GemmArgs<G>& args, int total_tiles, int mf, void* stream) {
  return wants_out_variant(args) ? launch8_v<G, true>(args, total_tiles, mf, stream)
                                 : launch8_v<G, false>(args, total_tiles, mf, stream);
}

// Tiles of the 4-wave kernel: 64 mf rows x 128 columns (one b_layout N-tile), times the K pieces.
template <int G>
static void set_tiles4w(GemmArgs<G>& args, int mf, int& total) {
  total = 0;
  for (int i = 0; i < args.n; i++) {
    GemmDesc& g = args.d[i];
    g.tiles_m = (int32_t)((g.M + 64 * mf - 1) / (64 * mf));
    g.tiles_n = (int32_t)(g.N / 128);
    g.tile_start = total;
    total += g.tiles_m * g.tiles_n * g.ksplit;
  }
  for (int i = args.n; i < G; i++) args.d[i] = args.d[args.n - 1];
}

template <int G, bool kOut>
static int launch4w_v(const GemmArgs<G>& args, int total_tiles, int mf, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(total_tiles), block(kW4Threads);
  switch (mf) {
    case 8: hipLaunchKernelGGL((gemm4w_kernel<G, 8, kOut>), grid, block, 0, st, args); break;
    case 7: hipLaunchKernelGGL((gemm4w_kernel<G, 7, kOut>), grid, block, 0, st, args); break;
    case 6: hipLaunchKernelGGL((gemm4w_kernel<G, 6, kOut>), grid, block, 0, st, args); break;
    default: hipLaunchKernelGGL((gemm4w_kernel<G, 4, kOut>), grid, block, 0, st, args); break;
  }
  return launch_status("rl_bfp16_gemm");
}
// The register-epilogue variant (gemm4w_kernel's kReg) serves a SwiGLU GEMM of whole K with no bias, gate or
// residual, into a row-major bf16 C only.
static bool wants_reg_variant(const GemmDesc& g) {
  return g.act == RL_ACT_SWIGLU && g.ksplit == 1 && !g.bias && !g.gate && !g.res && !g.pk && !g.c_atb && g.C;
}
static int launch4w_reg(const GemmArgs<1>& args, int total_tiles, int mf, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(total_tiles), block(kW4Threads);
  switch (mf) {
    case 8: hipLaunchKernelGGL((gemm4w_kernel<1, 8, false, true>), grid, block, 0, st, args); break;
    case 7: hipLaunchKernelGGL((gemm4w_kernel<1, 7, false, true>), grid, block, 0, st, args); break;
    case 6: hipLaunchKernelGGL((gemm4w_kernel<1, 6, false, true>), grid, block, 0, st, args); break;
    default: hipLaunchKernelGGL((gemm4w_kernel<1, 4, false, true>), grid, block, 0, st, args); break;
  }
  return launch_status("rl_bfp16_gemm");
}
template <int G>
static int launch4w(const GemmArgs<G>& args, int total_tiles, int mf, void* stream) {
  if constexpr (G == 1) {
    if (wants_reg_variant(args.d[0])) return launch4w_reg(args, total_tiles, mf, stream);
  }
  return wants_out_variant(args) ? launch4w_v<G, true>(args, total_tiles, mf, stream)
                                 : launch4w_v<G, false>(args, total_tiles, mf, stream);
}

// The descriptor of rows R.. of a GEMM.
static GemmDesc rows_from(const GemmDesc& g, int64_t R) {
  GemmDesc t = g;
  t.A = static_cast<const uint16_t*>(g.A) + R * g.lda;
  t.C = g.C && !g.c_atb ? g.C + R * g.ldc : g.C;  // packed and ATB positions come from prow
  t.prow = (int32_t)(g.prow + R);
  if (g.res) t.res = g.res + R * g.ldr;
  t.M = (int32_t)(g.M - R);
  t.gate_split = (int32_t)(g.gate_split > R ? g.gate_split - R : 0);
  return t;
}

// One whole-K GEMM (a filled descriptor, bf16 A) as the plan's one or two launches.
static int launch_planned(const GemmDesc& g, const PlanG& p, void* stream) {
  GemmArgs<1> args, tail;
  args.d[0] = g;
  args.n = tail.n = 1;
  if (p.split) {
    tail.d[0] = rows_from(g, p.split);
    args.d[0].M = (int32_t)p.split;
  }
  int total = 0, s;
  if (p.w4) {
    set_tiles4w(args, p.mf, total);
    s = launch4w<1>(args, total, p.mf, stream);
  } else {
    set_tiles8(args, p.mf, total);
    s = launch8<1>(args, total, p.mf, stream);
  }
  if (s || !p.split) return s;
  if (p.tail_w4) {
    set_tiles4w(tail, p.mf_tail, total);
    return launch4w<1>(tail, total, p.mf_tail, stream);
  }
  set_tiles8(tail, p.mf_tail, total);
  return launch8<1>(tail, total, p.mf_tail, stream);
}

// Bytes of the bf16 A copy that rl_bfp16_gemm_ws stages at the start of the workspace for a non-bf16 A format,
// rounded up so that the K-split partials after it stay 256-byte aligned.
static int64_t staged_a_bytes(int64_t M, int64_t K) { return (M * K * 2 + 255) / 256 * 256; }

// Writes A of a non-bf16 format as bf16 into a16 (M x K, row stride K): its bfp16 values, after quantizing along K
// for RL_A_BF16_QUANTIZE. One HBM-bound pass (9/8 or 2 bytes read and 2 written per value).
static int stage_a(const void* A, int32_t a_fmt, int64_t lda, int64_t M, int64_t K, uint16_t* a16, void* stream) {
  if (a_fmt == RL_A_BF16_QUANTIZE)
    return rl_bfp16_quantize(A, RL_DTYPE_BF16, M, K, lda, RL_ORDER_ROWBLOCK, nullptr, a16, stream);
  return rl_bfp16_dequantize(static_cast<const uint8_t*>(A),
                             a_fmt == RL_A_PACKED_A_LAYOUT ? RL_ORDER_A_LAYOUT : RL_ORDER_ROWBLOCK, M, K, a16,
                             RL_DTYPE_BF16, stream);
}

// Device memory for a call that was given no workspace: a stream-ordered allocation on the call's stream, released
// by stream_free once the call's launches are queued. A stream under graph capture is refused (RL_ERR_WORKSPACE):
// such callers pass a workspace (rl_bfp16_gemm_ws) or use the fixed scratch (rl_bfp16_gemm_noalloc).
static int stream_alloc(void** p, int64_t bytes, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return fail(RL_ERR_DEVICE, "hipStreamIsCapturing: %s", hipGetErrorString(e));
  if (cs != hipStreamCaptureStatusNone)
    return fail(RL_ERR_WORKSPACE, "a non-bf16 A under stream capture needs a workspace (rl_bfp16_gemm_ws, "
                                  "rl_bfp16_gemm_workspace_size bytes) or rl_bfp16_gemm_noalloc");
  e = hipMallocAsync(p, (size_t)bytes, st);
  if (e != hipSuccess) return fail(RL_ERR_DEVICE, "hipMallocAsync(%lld bytes): %s", (long long)bytes,
                                   hipGetErrorString(e));
  return RL_OK;
}

// Releases a stream_alloc allocation on the same stream; returns the call's status s, or the free's failure.
static int stream_free(void* p, void* stream, int s) {
  const hipError_t e = hipFreeAsync(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess && s == RL_OK) return fail(RL_ERR_DEVICE, "hipFreeAsync: %s", hipGetErrorString(e));
  return s;
}

}  // namespace rl

extern "C" {

int64_t rl_bfp16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  using namespace rl;
  if (rl_validate_gemm(RL_A_BF16, K, N, M, N, K, nullptr)) return -1;
  check_device();  // fills the compute-unit count when a device is present; 256 otherwise
  ok();
  return plan_split(M, N, K, device_cus()).ws_bytes;
}

int64_t rl_bfp16_gemm_workspace_size(int32_t a_fmt, int64_t M, int64_t N, int64_t K) {
  using namespace rl;
  if (rl_validate_gemm(a_fmt, a_fmt == RL_A_BF16 || a_fmt == RL_A_BF16_QUANTIZE ? K : 0, N, M, N, K, nullptr))
    return -1;
  check_device();
  ok();
  const int64_t split = plan_split(M, N, K, device_cus()).ws_bytes;
  return a_fmt == RL_A_BF16 ? split : staged_a_bytes(M, K) + split;
}

int rl_bfp16_gemm_ws(const void* A, int32_t a_fmt, int64_t lda, const uint8_t* B_packed, uint16_t* C, int64_t ldc,
                     int64_t M, int64_t N, int64_t K, const rl_epilogue* ep, void* workspace, int64_t workspace_bytes,
                     void* stream) {
  using namespace rl;
  GemmArgs<1> args;
  int s = fill_desc<1>(args.d[0], A, lda, B_packed, C, ldc, M, N, K, ep, a_fmt, 0);
  if (s) return s;
  if ((uintptr_t)workspace % 16) return fail(RL_ERR_ALIGN, "the workspace must be 16-byte aligned");
  args.n = 1;
  if ((s = check_device())) return s;
  if (a_fmt != RL_A_BF16) {
    // stage A as bf16 (its bfp16 values) at the start of the workspace, then run the bf16 path with the rest of it
    const int64_t sa = staged_a_bytes(M, K);
    if (!workspace) {
      // no workspace: the staged copy alone goes into a stream-ordered allocation and the product runs whole K, so
      // rl_bfp16_gemm gives every A format the bits of the RL_A_BF16 call on the same values
      void* tmp = nullptr;
      if ((s = stream_alloc(&tmp, sa, stream))) return s;
      uint16_t* a16 = static_cast<uint16_t*>(tmp);
      s = stage_a(A, a_fmt, lda, M, K, a16, stream);
      if (!s) s = rl_bfp16_gemm_ws(a16, RL_A_BF16, K, B_packed, C, ldc, M, N, K, ep, nullptr, 0, stream);
      return stream_free(tmp, stream, s);
    }
    // the whole workspace (the staged copy, then any K-split partials) is checked before anything is enqueued
    const bool whole = ep && (ep->flags & RL_EP_WHOLE_K);
    const int64_t need = sa + (whole ? 0 : plan_split(M, N, K, device_cus()).ws_bytes);
    if (workspace_bytes < need)
      return fail(RL_ERR_WORKSPACE, "workspace %lld bytes, this shape and A format need %lld "
                  "(rl_bfp16_gemm_workspace_size)", (long long)workspace_bytes, (long long)need);
    uint16_t* a16 = static_cast<uint16_t*>(workspace);
    if ((s = stage_a(A, a_fmt, lda, M, K, a16, stream))) return s;
    const int64_t rest = workspace_bytes - sa;
    return rl_bfp16_gemm_ws(a16, RL_A_BF16, K, B_packed, C, ldc, M, N, K, ep,
                            rest > 0 ? static_cast<uint8_t*>(workspace) + sa : nullptr, rest, stream);
  }
  int total = 0;
  if (workspace && !(ep && (ep->flags & RL_EP_WHOLE_K))) {
    const SplitPlan sp = plan_split(M, N, K, device_cus());
    if (sp.ks > 1) {
      if (sp.ws_bytes > workspace_bytes)
        return fail(RL_ERR_WORKSPACE, "workspace %lld bytes, this shape needs %lld (rl_bfp16_gemm_workspace_bytes)",
                    (long long)workspace_bytes, (long long)sp.ws_bytes);
      args.d[0].ksplit = sp.ks;
      args.d[0].part = static_cast<float*>(workspace);
      if (sp.w4) {
        set_tiles4w(args, sp.mf, total);
        if ((s = launch4w<1>(args, total, sp.mf, stream))) return s;
      } else {
        set_tiles8(args, sp.mf, total);
        if ((s = launch8<1>(args, total, sp.mf, stream))) return s;
      }
      const int64_t nblocks = M * ((ep && ep->act == RL_ACT_SWIGLU) ? N / 2 : N) / 8;
      hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), args.d[0]);
      return launch_status("rl_bfp16_gemm (reduce)");
    }
  }
  return launch_planned(args.d[0], plan_gemm(M, N, device_cus(), ep ? ep->act : RL_ACT_NONE), stream);
}

int rl_bfp16_gemm(const void* A, int32_t a_fmt, int64_t lda, const uint8_t* B_packed, uint16_t* C, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, const rl_epilogue* ep, void* stream) {
  return rl_bfp16_gemm_ws(A, a_fmt, lda, B_packed, C, ldc, M, N, K, ep, nullptr, 0, stream);
}

}  // extern "C"

// ---- the allocation-free variant: the workspace is a file-scope device array --------------------------------------
// Each GPU that runs this code holds its own copy of `scratch` until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in symbol): the device address of this GPU's copy is
// looked up once per device with hipGetSymbolAddress and kept in scratch_ptr[device].
static __device__ __align__(256) uint8_t scratch[RL_NOALLOC_SCRATCH_BYTES];

namespace rl {
namespace {
constexpr int kScratchDevices = 64;
uint8_t* scratch_ptr[kScratchDevices] = {};
std::mutex scratch_mu;

// This device's address of `scratch` (the current device), looked up on its first use; RL_OK or RL_ERR_DEVICE.
int scratch_for_current_device(uint8_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(RL_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kScratchDevices) return fail(RL_ERR_DEVICE, "device %d: at most %d devices", dev, kScratchDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(RL_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = scratch_ptr[dev];
  return RL_OK;
}
}  // namespace
}  // namespace rl

extern "C" {

int rl_bfp16_gemm_noalloc(const void* A, int32_t a_fmt, int64_t lda, const uint8_t* B_packed, uint16_t* C,
                          int64_t ldc, int64_t M, int64_t N, int64_t K, const rl_epilogue* ep, void* stream) {
  using namespace rl;
  int s = rl_validate_gemm(a_fmt, lda, ldc, M, N, K, ep);
  if (s) return s;
  if ((s = check_device())) return s;
  const int64_t need = rl_bfp16_gemm_workspace_size(a_fmt, M, N, K);
  if (need < 0) return fail(RL_ERR_SHAPE, "M %lld N %lld K %lld: invalid shape for A format %d", (long long)M,
                            (long long)N, (long long)K, a_fmt);
  if (need > RL_NOALLOC_SCRATCH_BYTES)
    return fail(RL_ERR_WORKSPACE,
                "M %lld N %lld K %lld (A format %d) needs %lld bytes of scratch, above the fixed %lld "
                "(RL_NOALLOC_SCRATCH_BYTES); use rl_bfp16_gemm_ws with a workspace of that size",
                (long long)M, (long long)N, (long long)K, a_fmt, (long long)need, (long long)RL_NOALLOC_SCRATCH_BYTES);
  uint8_t* ws = nullptr;
  if ((s = scratch_for_current_device(&ws))) return s;
  return rl_bfp16_gemm_ws(A, a_fmt, lda, B_packed, C, ldc, M, N, K, ep, need > 0 ? ws : nullptr, need, stream);
}

int rl_bfp16_gemm_grouped(const rl_gemm_desc* descs, int32_t n, int32_t a_fmt, void* stream) {
  using namespace rl;
  if (!descs) return fail(RL_ERR_NULL, "descs is NULL");
  if (n < 1 || n > RL_MAX_GROUP) return fail(RL_ERR_ARG, "n %d: need 1..%d", n, RL_MAX_GROUP);
  GemmArgs<RL_MAX_GROUP> args;
  int total = 0;
  for (int i = 0; i < n; i++) {
    const rl_gemm_desc& e = descs[i];
    int s = fill_desc<RL_MAX_GROUP>(args.d[i], e.A, e.lda, e.B_packed, e.C, e.ldc, e.M, e.N, e.K, &e.ep, a_fmt, total);
    if (s) {
      char msg[256];
      snprintf(msg, sizeof msg, "%s", rl_last_error());
      return fail(s, "descriptor %d: %s", i, msg);
    }
    total += args.d[i].tiles_m * args.d[i].tiles_n;
  }
  for (int i = n; i < RL_MAX_GROUP; i++) args.d[i] = args.d[n - 1];
  args.n = n;
  int s = check_device();
  if (s) return s;
  if (a_fmt != RL_A_BF16) {
    // stage every member's A as bf16 in one stream-ordered allocation, then run the group on the bf16 path
    int64_t off[RL_MAX_GROUP], bytes = 0;
    for (int i = 0; i < n; i++) {
      off[i] = bytes;
      bytes += staged_a_bytes(descs[i].M, descs[i].K);
    }
    void* tmp = nullptr;
    if ((s = stream_alloc(&tmp, bytes, stream))) return s;
    rl_gemm_desc staged[RL_MAX_GROUP];
    for (int i = 0; i < n && !s; i++) {
      staged[i] = descs[i];
      staged[i].A = static_cast<uint8_t*>(tmp) + off[i];
      staged[i].lda = descs[i].K;
      s = stage_a(descs[i].A, a_fmt, descs[i].lda, descs[i].M, descs[i].K,
                  static_cast<uint16_t*>(const_cast<void*>(staged[i].A)), stream);
    }
    if (!s) s = rl_bfp16_gemm_grouped(staged, n, RL_A_BF16, stream);
    return stream_free(tmp, stream, s);
  }
  // one 8-wave launch for the whole group, with the fragment count that minimises its rounds; or, when the model
  // puts it lower, each member as its own planned launches (e.g. the SwiGLU up GEMMs of the image and text streams:
  // the 4-wave kernel's 512-row tiles over the 4096 image rows and 256-row tiles over the 256 text rows, where one
  // launch would round both to 256-row tiles of the 8-wave kernel). The 4-wave kernel is not used for the single
  // launch: with members of different weights it measured slower than the 8-wave one (627-646 against 619 us for
  // the two up GEMMs, 299-306 against 280 us for the two QKV GEMMs).
  const int cus = device_cus();
  int best_mf = 8;
  double bc = 1e300;
  for (int mf : kMfChoices) {
    int64_t t = 0;
    for (int i = 0; i < n; i++) t += tiles8(args.d[i].M, args.d[i].N, mf);
    const double c = launch_cost(t, mf, cus);
    if (c < bc) { bc = c; best_mf = mf; }
  }
  PlanG plans[RL_MAX_GROUP];
  double each = kSecondLaunch * (n - 1);
  for (int i = 0; i < n; i++) {
    double c = 0;
    plans[i] = plan_gemm(args.d[i].M, args.d[i].N, cus, args.d[i].act, &c);
    each += c;
  }
  if (each < bc) {
    for (int i = 0; i < n; i++)
      if ((s = launch_planned(args.d[i], plans[i], stream))) return s;
    return RL_OK;
  }
  set_tiles8(args, best_mf, total);
  return launch8<RL_MAX_GROUP>(args, total, best_mf, stream);
}

}  // extern "C"
