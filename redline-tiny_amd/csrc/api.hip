// C-ABI plumbing: per-thread error messages, the gfx950 device check, validators that need no GPU, version.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "rlbfp_host.h"

namespace rl {

static thread_local char g_msg[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof g_msg, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_msg[0] = '\0';
  return RL_OK;
}

static constexpr int kMaxDev = 64;
static int g_cus[kMaxDev] = {0};

int check_device() {
  static int state[kMaxDev] = {0};  // 0 unknown, 1 gfx950, 2 other
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(RL_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev >= 0 && dev < kMaxDev && state[dev] == 1) return RL_OK;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return fail(RL_ERR_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  const bool is950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  if (dev >= 0 && dev < kMaxDev) {
    g_cus[dev] = prop.multiProcessorCount;
    state[dev] = is950 ? 1 : 2;
  }
  if (!is950) return fail(RL_ERR_DEVICE, "device %d is %s; this library is built for gfx950 only", dev, prop.gcnArchName);
  return RL_OK;
}

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev || g_cus[dev] <= 0) return 256;
  return g_cus[dev];
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RL_ERR_DEVICE, "%s launch: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace rl

extern "C" {

const char* rl_last_error(void) { return rl::g_msg; }

const char* rl_version(void) { return "rlbfp 0.1.0 gfx950"; }

int rl_device_check(void) {
  int s = rl::check_device();
  return s == RL_OK ? rl::ok() : s;
}

int64_t rl_packed_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0 || cols % 8) return -1;
  return rows * cols / 8 * 9;
}

int rl_validate_quantize(int32_t x_dtype, int64_t rows, int64_t cols, int64_t ld_x, int32_t order) {
  using rl::fail;
  if (x_dtype != RL_DTYPE_F32 && x_dtype != RL_DTYPE_BF16) return fail(RL_ERR_ARG, "x_dtype %d unknown", x_dtype);
  if (rows < 1 || cols < 8 || cols % 8) return fail(RL_ERR_SHAPE, "rows %lld, cols %lld: need rows >= 1, cols %% 8 == 0",
                                                    (long long)rows, (long long)cols);
  if (ld_x < cols) return fail(RL_ERR_SHAPE, "ld_x %lld < cols %lld", (long long)ld_x, (long long)cols);
  if (rows * cols / 8 > (int64_t)1 << 31) return fail(RL_ERR_SHAPE, "more than 2^31 blocks");
  switch (order) {
    case RL_ORDER_ROWBLOCK: break;
    case RL_ORDER_A_LAYOUT:
    case RL_ORDER_B_LAYOUT:
      if (rows % 128 || cols % 64)
        return fail(RL_ERR_SHAPE, "order %d needs rows %% 128 == 0 and cols %% 64 == 0 (got %lld x %lld)", order,
                    (long long)rows, (long long)cols);
      break;
    case RL_ORDER_C_ATB:
      if (rows % 512 || cols % 1024)
        return fail(RL_ERR_SHAPE, "order C_ATB needs rows %% 512 == 0 and cols %% 1024 == 0 (got %lld x %lld)",
                    (long long)rows, (long long)cols);
      break;
    default: return fail(RL_ERR_ARG, "order %d unknown", order);
  }
  return rl::ok();
}

int rl_validate_gemm(int32_t a_fmt, int64_t lda, int64_t ldc, int64_t M, int64_t N, int64_t K, const rl_epilogue* ep) {
  using rl::fail;
  if (M < 1 || N < 128 || K < 64 || N % 128 || K % 64)
    return fail(RL_ERR_SHAPE, "M %lld N %lld K %lld: need M >= 1, N %% 128 == 0, K %% 64 == 0", (long long)M,
                (long long)N, (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return fail(RL_ERR_SHAPE, "dimension above 2^30");
  const int act = ep ? ep->act : RL_ACT_NONE;
  if (act != RL_ACT_NONE && act != RL_ACT_GELU_TANH && act != RL_ACT_SWIGLU)
    return fail(RL_ERR_ARG, "epilogue act %d unknown", act);
  if (ep && (ep->flags & ~(RL_EP_QUANTIZE_OUT | RL_EP_WHOLE_K)))
    return fail(RL_ERR_ARG, "epilogue flags 0x%x unknown", ep->flags);
  const int64_t nout = act == RL_ACT_SWIGLU ? N / 2 : N;
  const int c_order = ep ? ep->c_order : RL_C_ROWMAJOR;
  if (c_order != RL_C_ROWMAJOR && c_order != RL_C_ATB) return fail(RL_ERR_ARG, "c_order %d unknown", c_order);
  if (c_order == RL_C_ATB && (M % 512 || nout % 1024))
    return fail(RL_ERR_SHAPE, "a C in the ATB order needs M %% 512 == 0 and Nout %% 1024 == 0 (M %lld, Nout %lld)",
                (long long)M, (long long)nout);
  if (c_order == RL_C_ROWMAJOR && (ldc < nout || ldc % 8))
    return fail(RL_ERR_ALIGN, "ldc %lld: need >= %lld and a multiple of 8", (long long)ldc, (long long)nout);
  if (ep && ep->packed_out) {
    if (ep->packed_order == RL_ORDER_C_ATB) {
      if (M % 512 || nout % 1024)
        return fail(RL_ERR_SHAPE, "packed C in the ATB order needs M %% 512 == 0 and Nout %% 1024 == 0 (M %lld, "
                    "Nout %lld)", (long long)M, (long long)nout);
    } else if (ep->packed_order == RL_ORDER_A_LAYOUT) {
      if (M % 128 || nout % 64)
        return fail(RL_ERR_SHAPE, "packed C in the A layout needs M %% 128 == 0 and Nout %% 64 == 0 (M %lld, "
                    "Nout %lld)", (long long)M, (long long)nout);
    } else {
      return fail(RL_ERR_ARG, "packed_order %d: RL_ORDER_C_ATB or RL_ORDER_A_LAYOUT", ep->packed_order);
    }
  }
  switch (a_fmt) {
    case RL_A_BF16:
    case RL_A_BF16_QUANTIZE:
      if (lda < K || lda % 8) return fail(RL_ERR_ALIGN, "lda %lld: need >= K and a multiple of 8", (long long)lda);
      break;
    case RL_A_PACKED_ROWBLOCK: break;
    case RL_A_PACKED_A_LAYOUT:
      if (M % 128) return fail(RL_ERR_SHAPE, "A_LAYOUT input needs M %% 128 == 0 (got %lld)", (long long)M);
      break;
    default: return fail(RL_ERR_ARG, "a_fmt %d unknown", a_fmt);
  }
  if (ep && ep->residual && (ep->ld_residual < nout))
    return fail(RL_ERR_SHAPE, "ld_residual %lld < %lld", (long long)ep->ld_residual, (long long)nout);
  if (ep && ep->gate_split_row < 0) return fail(RL_ERR_ARG, "gate_split_row < 0");
  return rl::ok();
}

int rl_validate_gemv(int64_t ldx, int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t act) {
  using rl::fail;
  if (M < 1 || M > 8) return fail(RL_ERR_SHAPE, "GEMV M %lld: need 1..8", (long long)M);
  if (N < 128 || N % 128 || K < 64 || K % 64)
    return fail(RL_ERR_SHAPE, "GEMV N %lld K %lld: need N %% 128 == 0, K %% 64 == 0", (long long)N, (long long)K);
  if (N > (1 << 30) || K > (1 << 30)) return fail(RL_ERR_SHAPE, "dimension above 2^30");
  if (ldx < K || ldy < N) return fail(RL_ERR_SHAPE, "ldx %lld / ldy %lld too small", (long long)ldx, (long long)ldy);
  if (act != RL_ACT_NONE && act != RL_GEMV_SILU) return fail(RL_ERR_ARG, "GEMV act %d unknown", act);
  return rl::ok();
}

int rl_validate_ln(int64_t ldx, int32_t br_fmt, int64_t ld_br, int32_t norm, int64_t ld_xo, int32_t a_order,
                   int64_t ld_a, int64_t split_row, int64_t M, int64_t D) {
  using rl::fail;
  if (M < 1 || M > (1 << 30) || D < 64 || D > 8192 || D % 64)
    return fail(RL_ERR_SHAPE, "M %lld D %lld: need M >= 1, D %% 64 == 0, 64 <= D <= 8192", (long long)M,
                (long long)D);
  if (norm != RL_NORM_LAYER && norm != RL_NORM_RMS) return fail(RL_ERR_ARG, "norm %d unknown", norm);
  if (br_fmt != RL_BRANCH_BF16 && br_fmt != RL_BRANCH_PACKED) return fail(RL_ERR_ARG, "br_fmt %d unknown", br_fmt);
  if (a_order != RL_ORDER_ROWBLOCK && a_order != RL_ORDER_A_LAYOUT)
    return fail(RL_ERR_ARG, "a_order %d: RL_ORDER_ROWBLOCK or RL_ORDER_A_LAYOUT", a_order);
  if (a_order == RL_ORDER_A_LAYOUT && M % 128)
    return fail(RL_ERR_SHAPE, "a_order A_LAYOUT needs M %% 128 == 0 (got %lld)", (long long)M);
  if (split_row < 0) return fail(RL_ERR_ARG, "split_row < 0");
  if (ldx < D || ldx % 8) return fail(RL_ERR_ALIGN, "ldx %lld: need >= D and a multiple of 8", (long long)ldx);
  if (br_fmt == RL_BRANCH_BF16 && (ld_br < D || ld_br % 8))
    return fail(RL_ERR_ALIGN, "ld_br %lld: need >= D and a multiple of 8", (long long)ld_br);
  if (ld_xo < D || ld_xo % 8) return fail(RL_ERR_ALIGN, "ld_xo %lld: need >= D and a multiple of 8", (long long)ld_xo);
  if (ld_a < D || ld_a % 8) return fail(RL_ERR_ALIGN, "ld_a %lld: need >= D and a multiple of 8", (long long)ld_a);
  return rl::ok();
}

int rl_validate_qkv_post_gqa(int64_t ldc, int64_t M, int32_t hq, int32_t hkv) {
  using rl::fail;
  if (hq < 1 || hq > 1024 || hkv < 1 || hkv > 1024)
    return fail(RL_ERR_SHAPE, "heads %d / %d: need 1..1024 each", hq, hkv);
  if (M < 64 || M % 64 || M > (1 << 30))
    return fail(RL_ERR_SHAPE, "M %lld: need a positive multiple of 64", (long long)M);
  if (M / 64 * (hq + 2 * (int64_t)hkv) > ((int64_t)1 << 31) - 1) return fail(RL_ERR_SHAPE, "more than 2^31 tiles");
  if (ldc < 128 * ((int64_t)hq + 2 * hkv) || ldc % 8)
    return fail(RL_ERR_ALIGN, "ldc %lld: need >= 128 * (hq + 2 hkv) and a multiple of 8", (long long)ldc);
  return rl::ok();
}

int rl_validate_qkv_post(int64_t ldc, int64_t M, int32_t heads) { return rl_validate_qkv_post_gqa(ldc, M, heads, heads); }

int rl_validate_attention(int32_t heads, int64_t nq, int64_t nk, int64_t nkv, int64_t ldo, int32_t h0) {
  using rl::fail;
  if (heads < 1 || heads > 1024) return fail(RL_ERR_SHAPE, "heads %d: need 1..1024", heads);
  if (nq < 128 || nq % 128 || nq > (1 << 24))
    return fail(RL_ERR_SHAPE, "nq %lld: need a positive multiple of 128", (long long)nq);
  if (nk < 64 || nk % 64 || nk > (1 << 24))
    return fail(RL_ERR_SHAPE, "nk %lld: need a positive multiple of 64", (long long)nk);
  if (nkv < 1 || nkv > nk) return fail(RL_ERR_SHAPE, "nkv %lld: need 1..nk", (long long)nkv);
  if (h0 < 0) return fail(RL_ERR_ARG, "h0 < 0");
  if (ldo < ((int64_t)h0 + heads) * 128 || ldo % 8)
    return fail(RL_ERR_ALIGN, "ldo %lld: need >= (h0 + heads) * 128 and a multiple of 8", (long long)ldo);
  if ((int64_t)heads * (nq / 128) > ((int64_t)1 << 31) - 1) return fail(RL_ERR_SHAPE, "too many workgroups");
  return rl::ok();
}

}  // extern "C"
