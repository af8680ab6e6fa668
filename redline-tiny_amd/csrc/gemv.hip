// Bandwidth-bound bfp16-weight GEMV for the adaLN modulation projection: y (M x N) = act(x) @ B, 1 <= M <= 8.
//
// Replaces host_glue.modulation = linear(silu(te), W) (redline/host_glue.py:22-28, :43-44), which the reference
// computes in numpy float32 on fp32 weights; here the weights are the packed b_layout(W.T, 64, 128) stream and the
// work is one pass over it (K * N * 9/8 bytes), which is the HBM roofline.
//
// One wave per 16-column group of the b_layout: that group's 64 K x 16 columns are 1152 contiguous bytes in every
// 64 x 128 tile, 128 blocks of 8 K. The wave walks 8 K tiles at a time: lane (c, br) = (l/8, l%8) reads the 144
// contiguous, 16-byte aligned bytes of K tile 8b+c, K rows br*8..+7 (16 blocks, one per column), with nine
// 16-byte loads, and accumulates 16 column sums per row of x. Each block costs eight sign-extending converts, 8 FMAs
// per row of x and one scale FMA per row: sum_k x_k q_k * 2^(E-133). The 64 lanes' partial sums are then reduced
// with a transposing butterfly so that lane 4j holds column j's total.
#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int kVWaves = 4;
constexpr int kVThreads = 64 * kVWaves;

__device__ __forceinline__ float silu_v(float x) { return x / (1.0f + __expf(-x)); }

template <int M, bool SILU>
__global__ __launch_bounds__(kVThreads) void gemv_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                         const uint8_t* __restrict__ B, uint16_t* __restrict__ y,
                                                         int64_t ldy, int32_t N, int32_t K) {
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * kVWaves + (threadIdx.x >> 6);  // 16-column group
  if (g * 16 >= N) return;
  const int KT = K / 64;
  const int nt = g >> 3, sbc = g & 7;
  const int c = lane >> 3, br = lane & 7;
  const uint8_t* base = B + ((int64_t)nt * KT) * 9216 + sbc * 1152 + br * 144;

  float part[M][16];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < 16; j++) part[m][j] = 0.f;

  const int nbatch = (KT + 7) / 8;
  u32x4 w[9];
  auto load = [&](int b) {
    const int kt = 8 * b + c;
    if (kt < KT) {
      const u32x4* p = reinterpret_cast<const u32x4*>(base + (int64_t)kt * 9216);
#pragma unroll
      for (int i = 0; i < 9; i++) w[i] = __builtin_nontemporal_load(p + i);
    }
  };
  load(0);
  for (int b = 0; b < nbatch; b++) {
    const int kt = 8 * b + c;
    u32x4 cur[9];
#pragma unroll
    for (int i = 0; i < 9; i++) cur[i] = w[i];
    if (b + 1 < nbatch) load(b + 1);
    if (kt < KT) {
      // activations of this lane's 8 K rows
      float a[M][8];
#pragma unroll
      for (int m = 0; m < M; m++) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(x + m * ldx + kt * 64 + br * 8);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int r = 0; r < 8; r++) {
          const float v = __uint_as_float(r & 1 ? xw[r >> 1] & 0xFFFF0000u : xw[r >> 1] << 16);
          a[m][r] = SILU ? silu_v(v) : v;
        }
      }
      const uint32_t* wd = reinterpret_cast<const uint32_t*>(cur);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        // block j: byte 9j = E, bytes 9j+1..9j+8 = q
        const int e0 = 9 * j;
        const uint32_t E = (wd[e0 >> 2] >> (8 * (e0 & 3))) & 0xFFu;
        const float s = block_scale(E);
        float q[8];
#pragma unroll
        for (int r = 0; r < 8; r++) {
          const int bi = e0 + 1 + r;
          q[r] = (float)(int8_t)(wd[bi >> 2] >> (8 * (bi & 3)));
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
          float dot = 0.f;
#pragma unroll
          for (int r = 0; r < 8; r++) dot = __builtin_fmaf(a[m][r], q[r], dot);
          part[m][j] = __builtin_fmaf(dot, s, part[m][j]);
        }
      }
    }
  }

  // transposing butterfly: after the steps over lane bits 5..2, lane l holds the sum for column
  // 8*b5 + 4*b4 + 2*b3 + b2 over the lanes that differ in those bits; bits 1..0 are then summed directly.
#pragma unroll
  for (int m = 0; m < M; m++) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = part[m][j];
    int cnt = 16;
#pragma unroll
    for (int s = 32; s >= 4; s >>= 1) {
      const int half = cnt / 2;
      const bool up = (lane & s) != 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if (i < half) {
          const float send = up ? v[i] : v[i + half];
          const float keep = up ? v[i + half] : v[i];
          v[i] = keep + __shfl_xor(send, s);
        }
      }
      cnt = half;
    }
    float t = v[0];
    t += __shfl_xor(t, 2);
    t += __shfl_xor(t, 1);
    if ((lane & 3) == 0) {
      const int col = ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
      const uint32_t u = __float_as_uint(t);
      y[m * ldy + g * 16 + col] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
  }
}

template <int M>
static void launch_m(bool silu, dim3 grid, hipStream_t st, const uint16_t* x, int64_t ldx, const uint8_t* B,
                     uint16_t* y, int64_t ldy, int32_t N, int32_t K) {
  if (silu)
    hipLaunchKernelGGL((gemv_kernel<M, true>), grid, dim3(kVThreads), 0, st, x, ldx, B, y, ldy, N, K);
  else
    hipLaunchKernelGGL((gemv_kernel<M, false>), grid, dim3(kVThreads), 0, st, x, ldx, B, y, ldy, N, K);
}

}  // namespace rl

extern "C" int rl_bfp16_gemv(const uint16_t* x, int64_t ldx, const uint8_t* B_packed, uint16_t* y, int64_t ldy,
                             int64_t M, int64_t N, int64_t K, int32_t act, void* stream) {
  using namespace rl;
  int s = rl_validate_gemv(ldx, ldy, M, N, K, act);
  if (s) return s;
  if (!x || !B_packed || !y) return fail(RL_ERR_NULL, "x, B or y is NULL");
  if (((uintptr_t)x % 16) || (ldx % 8)) return fail(RL_ERR_ALIGN, "x must be 16-byte aligned with ldx %% 8 == 0");
  if ((uintptr_t)B_packed % 16) return fail(RL_ERR_ALIGN, "B must be 16-byte aligned");
  if ((uintptr_t)y % 2) return fail(RL_ERR_ALIGN, "y must be 2-byte aligned");
  if ((s = check_device())) return s;
  const dim3 grid((unsigned)(N / 16 / kVWaves));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool silu = act == RL_GEMV_SILU;
  switch (M) {
    case 1: launch_m<1>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    case 2: launch_m<2>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    case 3: launch_m<3>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    case 4: launch_m<4>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    case 5: launch_m<5>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    case 6: launch_m<6>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    case 7: launch_m<7>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
    default: launch_m<8>(silu, grid, st, x, ldx, B_packed, y, ldy, (int32_t)N, (int32_t)K); break;
  }
  return launch_status("rl_bfp16_gemv");
}
