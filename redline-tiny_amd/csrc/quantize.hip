// bfp16 encode / decode kernels and their C-ABI entry points.
//
// rl_bfp16_quantize replaces npu_layouts.to_bfp16 (redline/npu_layouts.py:62-73) composed with the stream layouts
// (:11-47) and pack_weights.pack_b (redline/pack_weights.py:72-79); rl_bfp16_dequantize replaces from_bfp16 (:90-94)
// composed with the inverse layouts.
//
// The encoder takes one block per thread, walking the OUTPUT stream in order, so that a workgroup's 256 blocks are
// 2304 contiguous bytes: they are assembled in LDS and written with 16-byte stores. Each block's 8 source values are
// one contiguous 16-byte (bf16) or 32-byte (fp32) read (4 blocks per thread, the decoder's form below, measured 1-17%
// slower for the encoder). The decoder takes 4 blocks per thread, 1024 per workgroup. HBM-bound: 2 (or 4) bytes read
// + 9/8 written per value (+ 2 written for the encoder's decoded copy; 9/8 read and 2 or 4 written for the decoder).
#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int kQThreads = 256;

// Source (row, column block) of output block `ob` in the given order. rows x cols is the matrix; for
// RL_ORDER_B_LAYOUT the matrix is the Linear weight W (N rows, K cols) and the stream is b_layout(W.T, 64, 128).
__device__ __forceinline__ void block_source(int32_t order, int64_t ob, int64_t rows, int64_t cols, int64_t& r,
                                             int64_t& cb) {
  const int64_t cblocks = cols / 8;
  switch (order) {
    case RL_ORDER_A_LAYOUT: {  // ((((mt*KT + kt)*8 + sbr)*8 + bc)*2 + bis)*8 + rib
      const int64_t KT = cols / 64;
      const int64_t rib = ob & 7, bis = (ob >> 3) & 1, bc = (ob >> 4) & 7, sbr = (ob >> 7) & 7, t = ob >> 10;
      const int64_t kt = t % KT, mt = t / KT;
      r = mt * 128 + sbr * 16 + bis * 8 + rib;
      cb = kt * 8 + bc;
      break;
    }
    case RL_ORDER_B_LAYOUT: {  // ((((nt*KT + kt)*8 + sbc)*8 + br)*2 + bis)*8 + col ; W row n, K block kt*8 + br
      const int64_t KT = cols / 64;
      const int64_t col = ob & 7, bis = (ob >> 3) & 1, br = (ob >> 4) & 7, sbc = (ob >> 7) & 7, t = ob >> 10;
      const int64_t kt = t % KT, nt = t / KT;
      r = nt * 128 + sbc * 16 + bis * 8 + col;
      cb = kt * 8 + br;
      break;
    }
    case RL_ORDER_C_ATB: {  // (((((((rg*NG + cg)*8 + colg)*4 + rowg)*8 + sbr)*8 + sbc)*2 + br)*2 + bc)*8 + rib
      const int64_t NG = cols / 1024;
      const int64_t rib = ob & 7, bc = (ob >> 3) & 1, br = (ob >> 4) & 1, sbc = (ob >> 5) & 7, sbr = (ob >> 8) & 7;
      const int64_t rowg = (ob >> 11) & 3, colg = (ob >> 13) & 7, t = ob >> 16;
      const int64_t cg = t % NG, rg = t / NG;
      r = rg * 512 + rowg * 128 + sbr * 16 + br * 8 + rib;
      cb = (cg * 1024 + colg * 128 + sbc * 16 + bc * 8) / 8;
      break;
    }
    default:  // RL_ORDER_ROWBLOCK
      r = ob / cblocks;
      cb = ob - r * cblocks;
  }
}

template <int XDT>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(const void* __restrict__ x, int64_t rows, int64_t cols,
                                                             int64_t ld_x, int32_t order, uint8_t* __restrict__ packed,
                                                             uint16_t* __restrict__ deq) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[kQThreads * kBlockBytes];
  const int64_t nblocks = rows * cols / 8;
  const int64_t ob0 = (int64_t)blockIdx.x * kQThreads;
  const int64_t ob = ob0 + threadIdx.x;
  if (ob < nblocks) {
    int64_t r, cb;
    block_source(order, ob, rows, cols, r, cb);
    uint32_t u[8];
    if (XDT == RL_DTYPE_BF16) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + r * ld_x + cb * 8);
      u[0] = v.x << 16; u[1] = v.x & 0xFFFF0000u; u[2] = v.y << 16; u[3] = v.y & 0xFFFF0000u;
      u[4] = v.z << 16; u[5] = v.z & 0xFFFF0000u; u[6] = v.w << 16; u[7] = v.w & 0xFFFF0000u;
    } else {
      const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(x) + r * ld_x + cb * 8);
      const u32x4 a = p[0], b = p[1];
      u[0] = a.x; u[1] = a.y; u[2] = a.z; u[3] = a.w; u[4] = b.x; u[5] = b.y; u[6] = b.z; u[7] = b.w;
    }
    int32_t q[8];
    u32x4 bw;
    const uint32_t E = encode_block(u, q, bw);
    if (packed) {
      uint8_t* s = stage + threadIdx.x * kBlockBytes;
      s[0] = (uint8_t)E;
#pragma unroll
      for (int i = 0; i < 8; i++) s[1 + i] = (uint8_t)(int8_t)q[i];
    }
    if (deq) *reinterpret_cast<u32x4*>(deq + r * cols + cb * 8) = bw;
  }
  if (!packed) return;
  __syncthreads();
  // this workgroup's blocks are bytes [9*ob0, 9*(ob0 + nb)) of the output; 9*ob0 is a multiple of 16 (ob0 % 256 == 0)
  const int64_t nb = min((int64_t)kQThreads, nblocks - ob0);
  const int bytes = (int)(nb * kBlockBytes);
  uint8_t* dst = packed + ob0 * kBlockBytes;
  const int full = bytes / 16;
  for (int i = threadIdx.x; i < full; i += kQThreads)
    *reinterpret_cast<u32x4*>(dst + 16 * i) = *reinterpret_cast<const u32x4*>(stage + 16 * i);
  for (int i = full * 16 + threadIdx.x; i < bytes; i += kQThreads) dst[i] = stage[i];
}

// One decoded block (8 values, bf16 words) stored at row r, column block cb of the output.
template <int ODT>
__device__ __forceinline__ void store_decoded(void* out, int64_t r, int64_t cb, int64_t cols, u32x4 v) {
  if (ODT == RL_DTYPE_BF16) {
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + r * cols + cb * 8) = v;
  } else {
    u32x4* p = reinterpret_cast<u32x4*>(static_cast<float*>(out) + r * cols + cb * 8);
    p[0] = u32x4{v.x << 16, v.x & 0xFFFF0000u, v.y << 16, v.y & 0xFFFF0000u};
    p[1] = u32x4{v.z << 16, v.z & 0xFFFF0000u, v.w << 16, v.w & 0xFFFF0000u};
  }
}

// Each thread decodes 4 blocks, so a wave keeps 2304 bytes of loads in flight (one block per thread kept 576, too
// few to cover HBM latency: 3.7-3.9 TB/s at 4352 x 3072).
//   Tiled orders: thread t takes blocks 4t .. 4t + 3, whose 36 bytes (dword aligned) are one run read with two 16-byte
//   loads and one 4-byte load. They are rows r .. r + 3 of one 8-column block (the within-8 digit rib / col is the
//   last), so store j of a wave writes 8 rows x 128 bytes.
//   Row-block order: thread t takes blocks t, t + 256, t + 512, t + 768 (a 12-byte window each), so each store of a
//   wave writes 1 KB contiguous.
// Values are q * 2^(E - 133) in float32 (decode_window), as from_bfp16 computes them: exact, and +-inf where the
// product overflows (E = 254, q = -128; E = 255, |q| >= 64).
template <int ODT>
__global__ __launch_bounds__(kQThreads) void dequantize_kernel(const uint8_t* __restrict__ packed, int32_t order,
                                                               int64_t rows, int64_t cols, void* __restrict__ out) {
  typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
  const int64_t nblocks = rows * cols / 8;
  const int64_t g0 = (int64_t)blockIdx.x * (4 * kQThreads);
  if (order == RL_ORDER_ROWBLOCK) {
    const int64_t cblocks = cols / 8;
    Window w[4] = {};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int64_t ob = g0 + threadIdx.x + j * kQThreads;
      if (ob < nblocks) w[j] = load_window_safe(packed, ob, nblocks);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int64_t ob = g0 + threadIdx.x + j * kQThreads;
      if (ob >= nblocks) break;
      const int64_t r = ob / cblocks;
      const u32x4 v = __builtin_bit_cast(u32x4, decode_window(w[j].w0, w[j].w1, w[j].w2, (uint32_t)(ob & 3)));
      store_decoded<ODT>(out, r, ob - r * cblocks, cols, v);
    }
    return;
  }
  const int64_t ob0 = g0 + 4 * threadIdx.x;
  if (ob0 >= nblocks) return;  // tiled streams hold a multiple of 1024 blocks: a thread's run is whole
  const uint8_t* src = packed + 9 * ob0;
  const u32x4 a = reinterpret_cast<const u32x4_a4*>(src)[0], b = reinterpret_cast<const u32x4_a4*>(src)[1];
  const uint32_t w[9] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, reinterpret_cast<const uint32_t*>(src)[8]};
  int64_t r, cb;
  block_source(order, ob0, rows, cols, r, cb);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    // block j starts at byte 9 j of the run: dword 2 j, byte offset j
    const u32x4 v = __builtin_bit_cast(u32x4, decode_window(w[2 * j], w[2 * j + 1], w[2 * j + 2], (uint32_t)j));
    store_decoded<ODT>(out, r + j, cb, cols, v);
  }
}

}  // namespace rl

extern "C" {

int rl_bfp16_quantize(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, int64_t ld_x, int32_t order,
                      uint8_t* packed, uint16_t* deq, void* stream) {
  using namespace rl;
  int s = rl_validate_quantize(x_dtype, rows, cols, ld_x, order);
  if (s) return s;
  if (!x) return fail(RL_ERR_NULL, "x is NULL");
  if (!packed && !deq) return fail(RL_ERR_NULL, "both outputs are NULL");
  const int64_t elt = x_dtype == RL_DTYPE_BF16 ? 2 : 4;
  if (((uintptr_t)x % 16) || ((ld_x * elt) % 16)) return fail(RL_ERR_ALIGN, "x must be 16-byte aligned, rows too");
  if (((uintptr_t)packed % 16) || ((uintptr_t)deq % 16)) return fail(RL_ERR_ALIGN, "outputs must be 16-byte aligned");
  if ((s = check_device())) return s;
  const int64_t nblocks = rows * cols / 8;
  const dim3 grid((unsigned)((nblocks + kQThreads - 1) / kQThreads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == RL_DTYPE_BF16)
    hipLaunchKernelGGL(quantize_kernel<RL_DTYPE_BF16>, grid, dim3(kQThreads), 0, st, x, rows, cols, ld_x, order,
                       packed, deq);
  else
    hipLaunchKernelGGL(quantize_kernel<RL_DTYPE_F32>, grid, dim3(kQThreads), 0, st, x, rows, cols, ld_x, order,
                       packed, deq);
  return launch_status("rl_bfp16_quantize");
}

int rl_bfp16_dequantize(const uint8_t* packed, int32_t order, int64_t rows, int64_t cols, void* out,
                        int32_t out_dtype, void* stream) {
  using namespace rl;
  int s = rl_validate_quantize(RL_DTYPE_F32, rows, cols, cols, order);
  if (s) return s;
  if (out_dtype != RL_DTYPE_F32 && out_dtype != RL_DTYPE_BF16) return fail(RL_ERR_ARG, "out_dtype %d", out_dtype);
  if (!packed || !out) return fail(RL_ERR_NULL, "packed / out is NULL");
  if (((uintptr_t)packed % 4) || ((uintptr_t)out % 16)) return fail(RL_ERR_ALIGN, "packed 4-, out 16-byte aligned");
  if ((s = check_device())) return s;
  const int64_t nblocks = rows * cols / 8;
  const dim3 grid((unsigned)((nblocks + 4 * kQThreads - 1) / (4 * kQThreads)));  // 4 blocks per thread
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype == RL_DTYPE_BF16)
    hipLaunchKernelGGL(dequantize_kernel<RL_DTYPE_BF16>, grid, dim3(kQThreads), 0, st, packed, order, rows, cols, out);
  else
    hipLaunchKernelGGL(dequantize_kernel<RL_DTYPE_F32>, grid, dim3(kQThreads), 0, st, packed, order, rows, cols, out);
  return launch_status("rl_bfp16_dequantize");
}

}  // extern "C"
