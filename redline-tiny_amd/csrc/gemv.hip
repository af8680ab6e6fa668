// Bandwidth-bound bfp16-weight GEMV for the adaLN modulation projection: y (M x N) = act(x) @ B, 1 <= M <= 8.
//
// Replaces host_glue.modulation = linear(silu(te), W) (redline/host_glue.py:22-28, :43-44), which the reference
// computes in numpy float32 on fp32 weights; here the weights are the packed b_layout(W.T, 64, 128) stream and the
// work is one pass over it (K * N * 9/8 bytes), which is the HBM roofline.
//
// The packed stream is read once with coalesced 1 KB loads: a workgroup owns one 16-column group, which for every K
// tile is 1152 contiguous bytes. Lanes re-read whole blocks (16 columns x 8 K) from LDS. The activation is quantized
// to bfp16 blocks of 8 along K like the GEMM's A operand, so every block product is two int8 dot4 instructions and
// one exact power-of-two scale. Lane sums are reduced with a transposing butterfly, then the three waves' K parts in LDS.
#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int kVWaves = 3;                    // waves per workgroup; they split K
constexpr int kVThreads = 64 * kVWaves;
constexpr int kVIterBytes = 8 * 1152;         // one wave iteration: 8 K tiles of one 16-column group = 9 x 1 KB

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float silu_v(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// Workgroup = one 16-column group g of the b_layout (N tile g / 8, super-block g % 8), all of K. Wave w of 3 takes
// the iterations it = w, w + 3, ... of 8 K tiles each (2 per wave at K = 3072: 3456 waves, at most 4 per SIMD, all
// resident). An iteration's 8 x 1152 bytes are read with 9 coalesced 1 KB direct-to-LDS
// loads into the wave's own 9 KB of LDS, from which lane l = (run, br) = (l/8, l%8) reads its 16 blocks (K rows
// br*8..+7 of K tile 8 it + run, 16 columns) as 144 aligned bytes at offset 144 l (a 36-dword stride, which covers
// all banks). The next iteration's loads go into the same buffer as soon as the lanes' reads of the current one have
// returned, before its block products: so no iteration is staged through registers, and the math left behind the
// last bytes to arrive is one iteration's block products. act(x) of a pair of iterations is quantized while the
// first one's blocks are in flight. (The previous form, the second iteration loaded into registers at once and staged
// through LDS after the first, measured 1-3% slower with the same bits; two waves of three iterations each 5% slower.)
//
// act(x) of the lane's 8 K rows is quantized to one bfp16 block per row of x (E = largest float32 exponent field,
// q = rint(v * 2^(133-E)) clipped to [-128, 127], as the activation encoder does), so that each weight block
// contributes 2^(Ew + Ex - 266) * (qw . qx) with two 4-way int8 dot products, exactly in int32.
template <int M, bool SILU>
__global__ __launch_bounds__(kVThreads, M == 1 ? 4 : (M <= 3 ? 2 : 1)) void gemv_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ B, uint16_t* __restrict__ y,
    int64_t ldy, int32_t N, int32_t K) {
  __shared__ __attribute__((aligned(16))) uint8_t buf[kVWaves][kVIterBytes];
  __shared__ float red[kVWaves][M][16];
  // the wave index is uniform across the wave: readfirstlane puts it (and the load offsets built from it) in scalar
  // registers, as buffer loads need
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KT = K / 64;
  const int iters = (KT + 7) / 8;
  const int mine = wave < iters ? (iters - wave + kVWaves - 1) / kVWaves : 0;  // this wave's iterations
  const int g = blockIdx.x, nt = g >> 3, sbc = g & 7;
  const int run = lane >> 3, br = lane & 7;

  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)((int64_t)K * N / 8 * 9), 0x00020000);
  // load lane offsets: instruction i, lane l -> chunk ci = 64 i + l of the iteration, K tile ci / 72 of the 8, byte
  // 16 (ci % 72) of that tile's 1152-byte run; the iteration's first K tile enters as the scalar offset. K tiles past
  // the end read zeros (their offsets are beyond the stream or in the next column group) and are skipped below.
  uint32_t voff[9];
#pragma unroll
  for (int i = 0; i < 9; i++) {
    const int ci = 64 * i + lane;
    voff[i] = (uint32_t)(((int64_t)nt * KT + ci / 72) * 9216 + sbc * 1152 + 16 * (ci % 72));
  }
  u32x4 x1[M], x0[M];
  // x rows of iteration idx (M loads, unconditional: past the last K tile they read the clamped tile)
  auto xload = [&](int idx, u32x4 (&dx)[M]) {
    const int kt = min(8 * (wave + kVWaves * idx) + run, KT - 1);
#pragma unroll
    for (int m = 0; m < M; m++) dx[m] = *reinterpret_cast<const u32x4*>(x + m * ldx + kt * 64 + br * 8);
  };
  // iteration 0 goes straight to the wave's LDS buffer (lane l of load i lands at 1024 i + 16 l, the staged order)
  auto dma = [&](int idx) {
    const int it = wave + kVWaves * idx;
#pragma unroll
    for (int i = 0; i < 9; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)&buf[wave][1024 * i], 16,
                                               voff[i], it * 8 * 9216, 0, kLoadStream);
  };

  float part[M][16];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < 16; j++) part[m][j] = 0.f;

  // act(x) of iteration idx's 8 K rows, quantized to one bfp16 block per row of x. Past the last K tile (whose
  // blocks may be the next N tile's) the x block is zero, so those products are exactly 0 and the block loop runs
  // without a branch.
  struct XQ {
    uint32_t q[M][2];
    int e[M];
  };
  auto quant = [&](int idx, const u32x4 (&xv)[M], XQ& o) {
    const int kt = 8 * (wave + kVWaves * idx) + run;
#pragma unroll
    for (int m = 0; m < M; m++) {
      const uint32_t xw[4] = {xv[m].x, xv[m].y, xv[m].z, xv[m].w};
      float v[8];
      uint32_t e = 0;
#pragma unroll
      for (int r = 0; r < 8; r++) {
        const float t = __uint_as_float(r & 1 ? xw[r >> 1] & 0xFFFF0000u : xw[r >> 1] << 16);
        v[r] = SILU ? silu_v(t) : t;
        e = max(e, (__float_as_uint(v[r]) >> 23) & 0xFFu);
      }
      o.e[m] = (int)e;
      int qi[8];
#pragma unroll
      for (int r = 0; r < 8; r++)
        qi[r] = (int)fminf(__builtin_rintf(__builtin_amdgcn_ldexpf(v[r], 133 - (int)e)), 127.0f);
      o.q[m][0] = (qi[0] & 0xFF) | ((qi[1] & 0xFF) << 8) | ((qi[2] & 0xFF) << 16) | ((uint32_t)qi[3] << 24);
      o.q[m][1] = (qi[4] & 0xFF) | ((qi[5] & 0xFF) << 8) | ((qi[6] & 0xFF) << 16) | ((uint32_t)qi[7] << 24);
      if (kt >= KT) o.q[m][0] = o.q[m][1] = 0u;
    }
  };
  // the lane's 144-byte run of the iteration in the wave's buffer
  auto rd = [&](u32x4 (&cur)[9]) {
#pragma unroll
    for (int i = 0; i < 9; i++) cur[i] = *reinterpret_cast<const u32x4*>(&buf[wave][144 * lane + 16 * i]);
  };
  auto body = [&](const XQ& xq, const u32x4 (&cur)[9]) {
    const auto& qx = xq.q;
    const auto& ex = xq.e;
    {
      const uint32_t* wd = reinterpret_cast<const uint32_t*>(cur);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        // block j (column j of the group, K rows br*8..+7): byte 9j = E, bytes 9j+1..9j+8 = q as two words
        const int e0 = 9 * j, b1 = e0 + 1, b5 = e0 + 5;
        const uint32_t E = (wd[e0 >> 2] >> (8 * (e0 & 3))) & 0xFFu;
        const uint32_t lo = (b1 & 3) ? __builtin_amdgcn_alignbyte(wd[(b1 >> 2) + 1], wd[b1 >> 2], b1 & 3) : wd[b1 >> 2];
        const uint32_t hi = (b5 & 3) ? __builtin_amdgcn_alignbyte(wd[(b5 >> 2) + 1], wd[b5 >> 2], b5 & 3) : wd[b5 >> 2];
#pragma unroll
        for (int m = 0; m < M; m++) {
          const int dot = __builtin_amdgcn_sdot4((int)lo, (int)qx[m][0],
                                                 __builtin_amdgcn_sdot4((int)hi, (int)qx[m][1], 0, false), false);
          part[m][j] += __builtin_amdgcn_ldexpf((float)dot, (int)E + ex[m] - 266);
        }
      }
    }
  };

  // Iterations go in pairs: the x rows of both, then the first one's blocks straight into the wave's LDS buffer; the
  // second's go into the same buffer once the lanes' reads of the first have returned, and the first one's block
  // products run while they are in flight. A pair is straight-line code, so each wait counts exactly (with uses under
  // a branch the compiler would sink the loads into it). Loads past this wave's iterations are safe: buffer loads
  // beyond the stream return zeros, x loads use a clamped K tile, and their x blocks are zero.
  for (int g0 = 0; g0 < mine; g0 += 2) {
    // issue order (fenced, and the waits below count on it): the pair's x rows, then the first iteration's blocks
    xload(g0, x0);
    xload(g0 + 1, x1);
    __builtin_amdgcn_sched_barrier(0);
    dma(g0);
    __builtin_amdgcn_sched_barrier(0);
    // the x rows land first: for up to 4 rows of x, act(x) of both iterations is quantized while the blocks are still
    // in flight (more rows would not fit the registers; they are quantized per iteration)
    constexpr bool kEarly = M <= 4;
    XQ xq[2];
    if constexpr (kEarly) {
      wait_vm<9>();
      quant(g0, x0, xq[0]);
      quant(g0 + 1, x1, xq[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm<0>();  // the first iteration has landed
    if constexpr (!kEarly) quant(g0, x0, xq[0]);
    u32x4 cur[9];
    rd(cur);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the reads have returned, the buffer is free
    __builtin_amdgcn_sched_barrier(0);
    dma(g0 + 1);
    __builtin_amdgcn_sched_barrier(0);
    body(xq[0], cur);
    __builtin_amdgcn_sched_barrier(0);  // the first iteration's math before the second one's wait
    // iterations past this wave's last one have every K tile >= KT, so their x blocks are zero and they add 0
    wait_vm<0>();
    if constexpr (!kEarly) quant(g0 + 1, x1, xq[1]);
    rd(cur);
    body(xq[1], cur);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the reads are done before the next pair's loads rewrite the buffer
    __builtin_amdgcn_sched_barrier(0);
  }

  // reduce over the 64 lanes (run: lane bits 5..3, br: bits 2..0) with a transposing butterfly over bits 5..2
  // (16 values -> 1; column 8 b5 + 4 b4 + 2 b3 + b2) and sums over bits 1 and 0; then over the two waves via LDS
  const int col = ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
#pragma unroll
  for (int m = 0; m < M; m++) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = part[m][j];
    // bits 5 and 4: the row-swap permutes exchange (v[i], v[i + hv]) between the halves, so each lane gets its own
    // kept value and its partner's sent one, with no selects and no LDS
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]), false, false);
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 4]), false, false);
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    // bit 3 (partner lane ^ 8: a row rotation by 8) and bit 2 (partner 7 - i within 8, the half-row mirror: the
    // quad sums below still cover all 8 lanes), each lane sending one value and keeping the other
    {
      const bool up = (lane & 8) != 0;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const float send = up ? v[i] : v[i + 2], keep = up ? v[i + 2] : v[i];
        v[i] = keep + dpp_f<0x128>(send);  // row_ror:8
      }
    }
    {
      const bool up = (lane & 4) != 0;
      const float send = up ? v[0] : v[1], keep = up ? v[1] : v[0];
      v[0] = keep + dpp_f<0x141>(send);  // row_half_mirror
    }
    float t = v[0] + dpp_f<0x4E>(v[0]);  // quad_perm [2, 3, 0, 1]
    t += dpp_f<0xB1>(t);                 // quad_perm [1, 0, 3, 2]
    if ((lane & 3) == 0) red[wave][m][col] = t;
  }
  __syncthreads();
  if (threadIdx.x < M * 16) {
    const int m = threadIdx.x >> 4, c = threadIdx.x & 15;
    float t = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kVWaves; w2++) t += red[w2][m][c];
    const uint32_t u = __float_as_uint(t);
    y[m * ldy + g * 16 + c] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
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
  if (K * N / 8 * 9 > INT32_MAX) return fail(RL_ERR_SHAPE, "packed B above 2^31 bytes");
  if ((s = check_device())) return s;
  const dim3 grid((unsigned)(N / 16));
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
