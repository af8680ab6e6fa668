// Fused residual add + LayerNorm / RMSNorm + modulate, producing the next GEMM's A operand.
//
// Replaces the fused artifact of kernels/glue/ln_design.py:38-118 (microkernels ln_par / ln_p1 / ln_fin / ln_p2,
// kernels/glue/ln_mod.cc:92-204) that run_ln.ln_run drives (redline/run_ln.py:43-57), and its RMSNorm copies
// (kernels/vlm/rms_mod.cc with a bfp16 branch, rms16_mod.cc with a bf16 branch). The NPU kernel streams each 128-row
// tile twice, statistics first and outputs second. Here one wave owns one row and keeps its D values in registers,
// so x and the branch are read once. The kernel is HBM-bound: per value it reads 2 bytes of x and 2 (bf16) or 9/8
// (packed) bytes of branch, and writes 2 bytes of x', 9/8 bytes of packed A and/or 2 bytes of bf16 A.
//
// Lane l of a row's wave owns the 8-value blocks l, l + 64, l + 128, ... of the row, so every load and store is a
// coalesced 16-byte access and a wave covers 1 KB of the row per instruction. The packed output is assembled in LDS
// in output order and written with 16-byte stores. In rowblock order the workgroup's 4 rows are one contiguous span.
// In A-layout order the workgroup takes 16 rows, one 16-row band (sbr) of the 128-row A tiles, which is a contiguous
// 128-block (1152-byte) span per 64-column K tile.
#include <math.h>

#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int kLnThreads = 256;  // 4 waves
constexpr int kLnMaxNB = 16;     // blocks per lane: D <= 64 lanes * 16 blocks * 8 = 8192

struct LnArgs {
  const uint16_t* x;
  int64_t ldx;
  const void* br;
  int32_t br_fmt;
  int64_t ld_br;
  const uint16_t* params;
  int64_t split_row;
  int32_t norm;
  uint16_t* x_out;
  int64_t ld_xo;
  uint8_t* a_packed;
  int32_t a_order;
  uint16_t* a_deq;
  int64_t ld_a;
  int64_t M;
  int32_t D;
  int32_t rows_wg;  // rows per workgroup: 4, or 16 for the A-layout order
};

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the wave, every lane getting the same value: within rows of 16 by DPP adds (quad swaps, half-row and row
// mirrors), then across the four rows with two lane permutes.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ void unpack8(u32x4 v, float f[8]) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xFFFF0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xFFFF0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xFFFF0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xFFFF0000u);
}


// Template NB = blocks of 8 per lane (D / 512 rounded up); lanes whose block lies past the row end hold zeros and
// skip every access. Up to 8 blocks a row's first-pass loads are all in flight at once (in chunks of up to 6), which
// needs more registers than one block at a time: the register budget per NB is the smallest that compiles without
// spills. For D = 3072 (NB 6) it allows 4 waves per SIMD, so a launch of one wave per row for M = 4352 rows leaves a
// short second round; that costs less than the per-block round trips of the 5-wave form (23.0 -> 22.0 us with a bf16
// branch, 19.9 -> 18.6 us with a packed one, same bits).
template <int NB>
constexpr int ln_waves_per_simd() { return NB <= 2 ? 6 : NB <= 4 ? 5 : NB <= 6 ? 4 : NB <= 8 ? 3 : NB <= 13 ? 4 : 3; }

// BR: the branch's format for NB <= 8 (0 none, 1 bf16, 2 packed); above 8 blocks it is tested at run time (BR = -1)
template <int NB, int BR>
__global__ __launch_bounds__(kLnThreads, ln_waves_per_simd<NB>()) void ln_kernel(LnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t stage[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int D = a.D, nbr = D >> 3;
  const int rpw = a.rows_wg >> 2;
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_wg;
  const bool a_lay = a.a_order == RL_ORDER_A_LAYOUT;

  for (int i = 0; i < rpw; i++) {
    const int lr = wave * rpw + i;  // row within the workgroup
    const int64_t r = r0 + lr;
    if (r >= a.M) break;
    const uint16_t* prm = a.params + (r < a.split_row ? 2 * (int64_t)D : 0);  // [g | sc] row

    // x' = bf16(x + g * branch) of block j from its loaded words, kept as its bf16 bits (two per register: the row
    // stays resident at 4 registers per block); sum for the mean. g * branch is exact in fp32: one rounding in the
    // fma, then RNE to bf16; the mean's sum takes the bf16 pairs with one dot2 against (1, 1).
    u32x4 v[NB];
    float s = 0.f;
    auto first = [&](int j, const u32x4& xw4, const u32x4& gw4, const float (&bf)[8]) {
      const int cb = lane + 64 * j;
      float xf[8], gf[8];
      unpack8(xw4, xf);
      unpack8(gw4, gf);
      uint32_t xw[4];
      const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i2 = 2 * e;
        xw[e] = pack_bf16_rne(fmaf(gf[i2], bf[i2], xf[i2]), fmaf(gf[i2 + 1], bf[i2 + 1], xf[i2 + 1]));
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, xw[e]), one, s, false);
      }
      v[j] = u32x4{xw[0], xw[1], xw[2], xw[3]};
      if (a.x_out) *reinterpret_cast<u32x4*>(a.x_out + r * a.ld_xo + cb * 8) = v[j];
    };
    // a packed branch block from its 12-byte window (block blk starts at byte 9 blk): exact, as from_bfp16
    auto branch_block = [&](int64_t blk, uint32_t w0, uint32_t w1, uint32_t w2, float (&bf)[8]) {
      const uint32_t o = (uint32_t)(blk & 3);  // (9 * blk) % 4
      const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, o);
      const uint32_t hi = __builtin_amdgcn_alignbyte(w2, w1, o);
      const int sh = (int)(lo & 0xFFu) - 133;
      const int32_t q[8] = {(int8_t)(lo >> 8), (int8_t)(lo >> 16), (int8_t)(lo >> 24), (int8_t)hi,
                            (int8_t)(hi >> 8), (int8_t)(hi >> 16), (int8_t)(hi >> 24), (int8_t)(w2 >> (8 * o))};
#pragma unroll
      for (int e = 0; e < 8; e++) bf[e] = __builtin_amdgcn_ldexpf((float)q[e], sh);
    };
    if constexpr (NB <= 8) {
      // chunks of at most 6 blocks (4 for 7 or 8 blocks): every load of a chunk (x, the gate row and the branch;
      // for the packed branch the block's 12-byte window in .x .y .z) is issued before any of them is used, so a
      // row takes one or two memory round trips rather than one per block
      constexpr int kMaxC = NB <= 6 ? 6 : 4, kNC = (NB + kMaxC - 1) / kMaxC, kC = (NB + kNC - 1) / kNC;
#pragma unroll
      for (int j0 = 0; j0 < NB; j0 += kC) {
        u32x4 xr[kC], gr[kC], brw[kC];
#pragma unroll
        for (int c = 0; c < kC; c++) {
          const int cb = lane + 64 * (j0 + c);
          xr[c] = gr[c] = brw[c] = u32x4{0u, 0u, 0u, 0u};
          if (j0 + c < NB && cb < nbr) {
            xr[c] = *reinterpret_cast<const u32x4*>(a.x + r * a.ldx + cb * 8);
            gr[c] = *reinterpret_cast<const u32x4*>(prm + cb * 8);
            if constexpr (BR == 1) {
              brw[c] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.br) + r * a.ld_br + cb * 8);
            } else if constexpr (BR == 2) {
              const Window w = load_window_safe(static_cast<const uint8_t*>(a.br), r * nbr + cb, a.M * nbr);
              brw[c] = u32x4{w.w0, w.w1, w.w2, 0u};
            }
          }
        }
#pragma unroll
        for (int c = 0; c < kC; c++) {
          const int j = j0 + c;
          if (j >= NB) break;
          v[j] = u32x4{0u, 0u, 0u, 0u};
          if (lane + 64 * j < nbr) {
            float bf[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if constexpr (BR == 1) unpack8(brw[c], bf);
            if constexpr (BR == 2) branch_block(r * nbr + lane + 64 * j, brw[c].x, brw[c].y, brw[c].z, bf);
            first(j, xr[c], gr[c], bf);
          }
        }
        // the next chunk's loads stay behind this chunk's math (registers)
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // above 8 blocks: one block at a time, the branch's format tested at run time
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int cb = lane + 64 * j;
        v[j] = u32x4{0u, 0u, 0u, 0u};
        if (cb < nbr) {
          float bf[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          if (a.br && a.br_fmt == RL_BRANCH_BF16) {
            unpack8(*reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.br) + r * a.ld_br + cb * 8), bf);
          } else if (a.br) {
            const Window w = load_window_safe(static_cast<const uint8_t*>(a.br), r * nbr + cb, a.M * nbr);
            branch_block(r * nbr + cb, w.w0, w.w1, w.w2, bf);
          }
          first(j, *reinterpret_cast<const u32x4*>(a.x + r * a.ldx + cb * 8),
                *reinterpret_cast<const u32x4*>(prm + cb * 8), bf);
        }
      }
    }
    // up to 8 blocks, the scale row's loads go out before the two reductions
    constexpr bool kScaleEarly = NB <= 8;
    u32x4 sr[kScaleEarly ? NB : 1];
    if constexpr (kScaleEarly) {
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int cb = lane + 64 * j;
        sr[j] = u32x4{0u, 0u, 0u, 0u};
        if (cb < nbr) sr[j] = *reinterpret_cast<const u32x4*>(prm + D + cb * 8);
      }
    }
    s = wave_sum(s);
    const float mean = a.norm == RL_NORM_LAYER ? s / (float)D : 0.f;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      if (lane + 64 * j < nbr) {
        float xf[8];
        unpack8(v[j], xf);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float d = xf[e] - mean;
          ss = fmaf(d, d, ss);
        }
      }
    }
    ss = wave_sum(ss);
    const float rstd = __builtin_amdgcn_rsqf(ss / (float)D + 1e-6f);

    // y = (x' - mean) * rstd * sc -> bfp16
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int cb = lane + 64 * j;
      if (cb < nbr) {
        float sf[8], xf[8];
        if constexpr (kScaleEarly)
          unpack8(sr[j], sf);
        else
          unpack8(*reinterpret_cast<const u32x4*>(prm + D + cb * 8), sf);
        unpack8(v[j], xf);
        uint32_t u[8];
        int32_t q[8];
        u32x4 bw;
#pragma unroll
        for (int e = 0; e < 8; e++) u[e] = __float_as_uint((xf[e] - mean) * rstd * sf[e]);
        const uint32_t E = encode_block(u, q, bw);
        if (a.a_deq) *reinterpret_cast<u32x4*>(a.a_deq + r * a.ld_a + cb * 8) = bw;
        if (a.a_packed) {
          const int pos = a_lay ? (cb >> 3) * 128 + (cb & 7) * 16 + (lr >> 3) * 8 + (lr & 7) : lr * nbr + cb;
          uint8_t* p = stage + pos * kBlockBytes;
          p[0] = (uint8_t)E;
#pragma unroll
          for (int e = 0; e < 8; e++) p[1 + e] = (uint8_t)(int8_t)q[e];
        }
      }
    }
  }

  if (!a.a_packed) return;
  __syncthreads();
  if (a_lay) {
    // rows r0 .. r0 + 15 = band sbr of A tile mt: for K tile kt, 128 blocks at block ((mt * KT + kt) * 8 + sbr) * 128
    const int KT = D >> 6;
    const int64_t mt = r0 >> 7, sbr = (r0 >> 4) & 7;
    const int chunks = KT * 72;  // 1152 bytes = 72 x 16 per K tile
    for (int c = threadIdx.x; c < chunks; c += kLnThreads) {
      const int kt = c / 72, w = c - kt * 72;
      uint8_t* dst = a.a_packed + (((mt * KT + kt) * 8 + sbr) * 128) * kBlockBytes + 16 * w;
      *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(stage + kt * 1152 + 16 * w);
    }
  } else {
    // rows r0 .. r0 + nrows - 1 are one span; r0 * nbr * 9 is a multiple of 16 (r0 % 4 == 0, nbr % 8 == 0)
    const int64_t nrows = min((int64_t)a.rows_wg, a.M - r0);
    const int bytes = (int)(nrows * nbr * kBlockBytes);
    uint8_t* dst = a.a_packed + r0 * nbr * kBlockBytes;
    const int full = bytes / 16;
    for (int c = threadIdx.x; c < full; c += kLnThreads)
      *reinterpret_cast<u32x4*>(dst + 16 * c) = *reinterpret_cast<const u32x4*>(stage + 16 * c);
    for (int c = full * 16 + threadIdx.x; c < bytes; c += kLnThreads) dst[c] = stage[c];
  }
}

template <int NB, int BR>
static int launch_nb_br(const LnArgs& a, hipStream_t st) {
  const int64_t lds = a.a_packed ? (int64_t)a.rows_wg * (a.D / 8) * kBlockBytes : 0;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&ln_kernel<NB, BR>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(RL_ERR_DEVICE, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  }
  const dim3 grid((unsigned)((a.M + a.rows_wg - 1) / a.rows_wg));
  hipLaunchKernelGGL((ln_kernel<NB, BR>), grid, dim3(kLnThreads), (unsigned)lds, st, a);
  return launch_status("rl_ln_modulate");
}

// the branch's format is a template parameter, so that the first pass is straight-line code whose loads all issue
// before the first use
template <int NB>
static int launch_nb(const LnArgs& a, hipStream_t st) {
  if constexpr (NB > 8) {
    return launch_nb_br<NB, -1>(a, st);
  } else {
    if (!a.br) return launch_nb_br<NB, 0>(a, st);
    if (a.br_fmt == RL_BRANCH_BF16) return launch_nb_br<NB, 1>(a, st);
    return launch_nb_br<NB, 2>(a, st);
  }
}

template <int NB>
static int launch_upto(int nb, const LnArgs& a, hipStream_t st) {
  if constexpr (NB > kLnMaxNB) {
    return fail(RL_ERR_SHAPE, "D %d too large", a.D);
  } else {
    if (nb <= NB) return launch_nb<NB>(a, st);
    return launch_upto<NB + 1>(nb, a, st);
  }
}

}  // namespace rl

extern "C" int rl_ln_modulate(const uint16_t* x, int64_t ldx, const void* branch, int32_t br_fmt, int64_t ld_br,
                              const uint16_t* params, int64_t split_row, int32_t norm, uint16_t* x_out, int64_t ld_xo,
                              uint8_t* a_packed, int32_t a_order, uint16_t* a_deq, int64_t ld_a, int64_t M, int64_t D,
                              void* stream) {
  using namespace rl;
  // the leading dimension of an absent operand is not used
  if (!branch) ld_br = D;
  if (!x_out) ld_xo = D;
  if (!a_deq) ld_a = D;
  int s = rl_validate_ln(ldx, br_fmt, ld_br, norm, ld_xo, a_order, ld_a, split_row, M, D);
  if (s) return s;
  if (!x || !params) return fail(RL_ERR_NULL, "x or params is NULL");
  if (!x_out && !a_packed && !a_deq) return fail(RL_ERR_NULL, "every output is NULL");
  if (((uintptr_t)x | (uintptr_t)params | (uintptr_t)x_out | (uintptr_t)a_deq | (uintptr_t)a_packed) % 16)
    return fail(RL_ERR_ALIGN, "x, params and the outputs must be 16-byte aligned");
  if (branch && (uintptr_t)branch % (br_fmt == RL_BRANCH_BF16 ? 16 : 4))
    return fail(RL_ERR_ALIGN, "branch must be 16-byte (bf16) or 4-byte (packed) aligned");
  if ((s = check_device())) return s;
  LnArgs a;
  a.x = x; a.ldx = ldx;
  a.br = branch; a.br_fmt = br_fmt; a.ld_br = ld_br;
  a.params = params; a.split_row = split_row; a.norm = norm;
  a.x_out = x_out; a.ld_xo = ld_xo;
  a.a_packed = a_packed; a.a_order = a_order;
  a.a_deq = a_deq; a.ld_a = ld_a;
  a.M = M; a.D = (int32_t)D;
  a.rows_wg = (a_packed && a_order == RL_ORDER_A_LAYOUT) ? 16 : 4;
  const int nb = (int)((D / 8 + 63) / 64);
  return launch_upto<1>(nb, a, static_cast<hipStream_t>(stream));
}
