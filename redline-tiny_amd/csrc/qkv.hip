// QKV post: the QKV GEMM's output -> attention Q / K / V (per-head RMSNorm * w, RoPE, bfp16 tiles).
//
// Replaces the QKV-post artifact of kernels/glue/qkv_design.py:40-118 (microkernels q_post / k_post / v_post,
// kernels/glue/qkv_post.cc:134-177) that run_qkv.qkv32_npu drives (redline/run_qkv.py:67-82). One workgroup takes
// one part (q, k or v) of one head of one 64-token tile: 64 x 128 values (16 KB of bf16 in), and writes the 9216-byte
// tile the attention kernel reads. The pass is HBM-bound: 2 bytes read and 9/8 bytes written per value (plus 2 per
// value for each bf16 output requested). Small workgroups (9 KB of LDS) keep many tiles in flight per CU.
//
// Q and K: thread (token r, 8-dim block bc) holds 8 dims of one token; the 16 threads of a token (16 lanes of a wave)
// reduce the sum of squares across their lanes. RoPE pairs (2i, 2i + 1) lie inside a block, so each thread rotates
// its own 4 pairs. V: each thread reads the 8 tokens of one dim that a V block holds (and writes them, as one 16-byte
// store, to the optional V^T output). The tile is assembled in LDS in output order and written with 16-byte stores.
#include <math.h>

#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int kQkvThreads = 256;
constexpr int kHeadDim = 128;
constexpr int kTileTokens = 64;
constexpr int kTileBlocks = kTileTokens * kHeadDim / 8;     // 1024
constexpr int kTile9 = kTileBlocks * kBlockBytes;          // 9216

struct QkvArgs {
  const uint16_t* C;
  int64_t ldc;
  int64_t M;
  int32_t hq, hkv;  // q heads, k / v heads (equal for the DiT; grouped-query attention has hq a multiple of hkv)
  const uint16_t* cos;
  const uint16_t* sin;
  const uint16_t* wq;
  const uint16_t* wk;
  uint8_t* q_tiles;
  uint8_t* kv_tiles;
  uint16_t* q;
  uint16_t* k;
  uint16_t* v;
};

__device__ __forceinline__ void unpack8f(u32x4 v, float f[8]) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xFFFF0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xFFFF0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xFFFF0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xFFFF0000u);
}

// Sum over each row of 16 lanes, every lane of the row getting the same value: quad swaps, then half-row and row
// mirrors, each one v_add_f32 with a DPP operand (no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);  // row_half_mirror: lane i <- 7 - i within each 8
  v += dpp_f<0x140>(v);  // row_mirror: lane i <- 15 - i
  return v;
}

__device__ __forceinline__ void stage_block(uint8_t* stage, int pos, uint32_t E, const int32_t q[8]) {
  uint8_t* p = stage + pos * kBlockBytes;
  p[0] = (uint8_t)E;
#pragma unroll
  for (int e = 0; e < 8; e++) p[1 + e] = (uint8_t)(int8_t)q[e];
}

// TILES / NATIVE: whether any tile / any head-major bf16 output is requested (the other's work is compiled out).
template <bool TILES, bool NATIVE>
__global__ __launch_bounds__(kQkvThreads) void qkv_post_kernel(QkvArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[kTile9];
  const int tid = threadIdx.x;
  // workgroup = (part, head) item j of 64-token tile t; C's columns are [q hq x 128 | k hkv x 128 | v hkv x 128].
  // With hq == hkv the three parts of one (head, tile) are neighbours in launch order (j = 3 h + part); otherwise
  // the q heads come first, then k and v head g side by side.
  const int per_tile = a.hq + 2 * a.hkv;
  const int t = blockIdx.x / per_tile, j = blockIdx.x - t * per_tile;
  int part, h;
  if (a.hq == a.hkv) {
    part = j % 3; h = j / 3;
  } else if (j < a.hq) {
    part = 0; h = j;
  } else {
    part = 1 + ((j - a.hq) & 1); h = (j - a.hq) >> 1;
  }
  const int64_t row0 = (int64_t)t * kTileTokens;
  const int64_t col0 = (part == 0 ? 0 : (int64_t)a.hq * kHeadDim + (part - 1) * (int64_t)a.hkv * kHeadDim) +
                       (int64_t)h * kHeadDim;
  const bool tiles = TILES && (part == 0 ? a.q_tiles != nullptr : a.kv_tiles != nullptr);

  if (part < 2) {
    // Q (part 0) and K (part 1): thread = (token rr + 16 pass, dim block bc)
    const int bc = tid & 15, rr = tid >> 4;
    float wf[8];
    unpack8f(*reinterpret_cast<const u32x4*>((part ? a.wk : a.wq) + bc * 8), wf);
    uint16_t* nat = NATIVE ? (part ? a.k : a.q) : nullptr;
    // every pass's loads (the token's 8 values, its cos and sin) are issued before the first use: the encoder's
    // rarely taken integer path is a branch that later loads are not hoisted over
    u32x4 xr[4];
    uint2 cr4[4], sr4[4];
#pragma unroll
    for (int pass = 0; pass < 4; pass++) {
      const int64_t row = row0 + pass * 16 + rr;
      xr[pass] = *reinterpret_cast<const u32x4*>(a.C + row * a.ldc + col0 + bc * 8);
      cr4[pass] = *reinterpret_cast<const uint2*>(a.cos + row * 64 + bc * 4);
      sr4[pass] = *reinterpret_cast<const uint2*>(a.sin + row * 64 + bc * 4);
    }
#pragma unroll
    for (int pass = 0; pass < 4; pass++) {
      const int r = pass * 16 + rr;
      const int64_t row = row0 + r;
      float xf[8];
      unpack8f(xr[pass], xf);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) ss = fmaf(xf[e], xf[e], ss);
      ss = row16_sum(ss);  // the token's 16 lanes
      const float inv = __builtin_amdgcn_rsqf(ss / (float)kHeadDim + 1e-6f);
      const uint2 cr = cr4[pass], sr = sr4[pass];
      const float c4[4] = {__uint_as_float(cr.x << 16), __uint_as_float(cr.x & 0xFFFF0000u),
                           __uint_as_float(cr.y << 16), __uint_as_float(cr.y & 0xFFFF0000u)};
      const float s4[4] = {__uint_as_float(sr.x << 16), __uint_as_float(sr.x & 0xFFFF0000u),
                           __uint_as_float(sr.y << 16), __uint_as_float(sr.y & 0xFFFF0000u)};
      uint32_t u[8];
      int32_t q[8];
      u32x4 bw;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ev = xf[2 * i] * inv * wf[2 * i], od = xf[2 * i + 1] * inv * wf[2 * i + 1];
        u[2 * i] = __float_as_uint(ev * c4[i] - od * s4[i]);
        u[2 * i + 1] = __float_as_uint(ev * s4[i] + od * c4[i]);
      }
      const uint32_t E = encode_block(u, q, bw);
      if (nat) *reinterpret_cast<u32x4*>(nat + (((int64_t)h * a.M + row) * kHeadDim + bc * 8)) = bw;
      // a_layout(64, 128) for Q and b_layout(K^T, 128, 64) for K order a tile's blocks the same way:
      // 16-token band, 8-dim block, 8-token half, token
      if (tiles) stage_block(stage, (((r >> 4) * 16 + bc) * 2 + ((r >> 3) & 1)) * 8 + (r & 7), E, q);
    }
  } else {
    // V: thread = (dim d, 8-token block kb), reading its 8 tokens of one dim (consecutive lanes read consecutive
    // dims: 128 contiguous bytes of a row per load); b_layout(V, 64, 128): 16-dim band, token block, 8-dim half, dim
    // all four items' loads first, as for Q and K
    uint16_t vr[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int item = tid + kQkvThreads * i, d = item & 127, kb = item >> 7;
#pragma unroll
      for (int e = 0; e < 8; e++) vr[i][e] = a.C[(row0 + kb * 8 + e) * a.ldc + col0 + d];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int item = tid + kQkvThreads * i, d = item & 127, kb = item >> 7;
      uint32_t u[8];
      int32_t q[8];
      u32x4 bw;
#pragma unroll
      for (int e = 0; e < 8; e++) u[e] = (uint32_t)vr[i][e] << 16;
      const uint32_t E = encode_block(u, q, bw);
      if (NATIVE && a.v)  // V^T: the block's 8 tokens are contiguous in row d
        *reinterpret_cast<u32x4*>(a.v + ((int64_t)h * kHeadDim + d) * a.M + row0 + kb * 8) = bw;
      if (tiles) stage_block(stage, (((d >> 4) * 8 + kb) * 2 + ((d >> 3) & 1)) * 8 + (d & 7), E, q);
    }
  }
  if (!tiles) return;
  __syncthreads();
  const int64_t T = a.M / kTileTokens;
  uint8_t* dst = part == 0 ? a.q_tiles + ((int64_t)h * T + t) * kTile9
                           : a.kv_tiles + (((int64_t)h * T + t) * 2 + (part - 1)) * kTile9;
  for (int c = tid; c < kTile9 / 16; c += kQkvThreads)
    *reinterpret_cast<u32x4*>(dst + 16 * c) = *reinterpret_cast<const u32x4*>(&stage[16 * c]);
}

}  // namespace rl

extern "C" int rl_qkv_post_gqa(const uint16_t* C, int64_t ldc, int64_t M, int32_t hq, int32_t hkv,
                               const uint16_t* cos, const uint16_t* sin, const uint16_t* wq, const uint16_t* wk,
                               uint8_t* q_tiles, uint8_t* kv_tiles, uint16_t* q, uint16_t* k, uint16_t* v,
                               void* stream) {
  using namespace rl;
  int s = rl_validate_qkv_post_gqa(ldc, M, hq, hkv);
  if (s) return s;
  if (!C || !cos || !sin || !wq || !wk) return fail(RL_ERR_NULL, "C, cos, sin, wq or wk is NULL");
  if (!q_tiles && !kv_tiles && !q && !k && !v) return fail(RL_ERR_NULL, "every output is NULL");
  if (((uintptr_t)C | (uintptr_t)wq | (uintptr_t)wk | (uintptr_t)q_tiles | (uintptr_t)kv_tiles | (uintptr_t)q |
       (uintptr_t)k) % 16)
    return fail(RL_ERR_ALIGN, "C, wq, wk, the tiles and q / k must be 16-byte aligned");
  if ((uintptr_t)v % 16) return fail(RL_ERR_ALIGN, "v must be 16-byte aligned");
  if (((uintptr_t)cos | (uintptr_t)sin) % 8) return fail(RL_ERR_ALIGN, "cos / sin must be 8-byte aligned");
  if ((s = check_device())) return s;
  QkvArgs a;
  a.C = C; a.ldc = ldc; a.M = M; a.hq = hq; a.hkv = hkv;
  a.cos = cos; a.sin = sin; a.wq = wq; a.wk = wk;
  a.q_tiles = q_tiles; a.kv_tiles = kv_tiles; a.q = q; a.k = k; a.v = v;
  const dim3 grid((unsigned)(M / kTileTokens * (hq + 2 * hkv)));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool tiles = q_tiles || kv_tiles, native = q || k || v;
  if (tiles && native)
    hipLaunchKernelGGL((qkv_post_kernel<true, true>), grid, dim3(kQkvThreads), 0, st, a);
  else if (tiles)
    hipLaunchKernelGGL((qkv_post_kernel<true, false>), grid, dim3(kQkvThreads), 0, st, a);
  else
    hipLaunchKernelGGL((qkv_post_kernel<false, true>), grid, dim3(kQkvThreads), 0, st, a);
  return launch_status("rl_qkv_post");
}

extern "C" int rl_qkv_post(const uint16_t* C, int64_t ldc, int64_t M, int32_t heads, const uint16_t* cos,
                           const uint16_t* sin, const uint16_t* wq, const uint16_t* wk, uint8_t* q_tiles,
                           uint8_t* kv_tiles, uint16_t* q, uint16_t* k, uint16_t* v, void* stream) {
  return rl_qkv_post_gqa(C, ldc, M, heads, heads, cos, sin, wq, wk, q_tiles, kv_tiles, q, k, v, stream);
}
