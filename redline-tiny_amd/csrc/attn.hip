// Attention over the QKV post pass's output: O = softmax2(Q K^T) V per head, flash style (one pass over the keys with
// a running max and sum), on bf16 MFMA with fp32 scores and accumulation.
//
// Replaces the attention artifacts (kernels/attn/attn_bfp.cc with attn_design.py) that run_attn.attn_npu and the DiT
// step drive (redline/run_attn.py:67-82, redline/forward.py:247, :369-377). As there, Q carries the score scale
// log2(e)/sqrt(128), so scores are in log2 units and the softmax is 2^(s - max) / sum (attn_bfp.cc:1-12).
//
// Workgroup = 4 or 8 waves x 32 queries of one head; key blocks of 64 are staged in LDS (double buffered) and read by
// all the waves. Per wave and key block, with v_mfma_f32_16x16x32_bf16:
//   S^T (64 keys x 32 queries) = K Q^T: K rows are the A operand, Q^T (kept in registers) the B operand, so each lane
//     holds 16 keys of one query and the softmax statistics of a query live in one lane column;
//   O^T (128 dims x 32 queries) += V^T P^T: P^T comes straight out of the S^T registers as the B operand (its 8 keys
//     per lane are keys 4g..4g+3 and 16+4g..16+4g+3 of a 32-key step), and the V^T A operand is read from LDS with
//     the same key order. V arrives transposed (rl_qkv_post's V^T output), so no transpose is needed anywhere.
// K rows in LDS are 256 bytes with the 16-byte chunks XOR-swizzled by key & 15. V^T rows are 128 bytes in which each
// 32-key step keeps the 4-key groups g and g + 4 side by side (16-byte chunk 4c + g of step c), so that one 16-byte
// read is a whole A operand; those chunks are XOR-swizzled by ((dim >> 1) & 7) ^ (dim & 1). Either way the lanes of
// an operand read (16 per pass) and of a staging store hit distinct banks.
// Built with -fno-honor-nans (Makefile): the running maxes then skip NaN quieting; +-inf keep their meaning. NaN in
// Q, K or V is outside the contract.
#include <math.h>

#include <algorithm>

#include "rlbfp.h"
#include "rlbfp_device.h"
#include "rlbfp_host.h"

namespace rl {

constexpr int kAtQW = 32;                       // queries per wave (two 16-query sets)
constexpr int kAtQMin = 4 * kAtQW;              // queries per task of the 4-wave kernel (the nq granule)
constexpr int kAtKB = 64;                       // keys per staged block
constexpr int kAtHD = 128;                      // head dim
constexpr int kAtK = kAtKB * kAtHD * 2;         // 16 KB: K block, 64 rows x 256 bytes
constexpr int kAtStage = 2 * kAtK;              // K block + V^T block (128 rows x 128 bytes)

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  uint16_t* o;
  int64_t ldo;
  int32_t h0;
  int32_t heads;
  int32_t nq;
  int32_t nk;
  int32_t nkv;
  const int32_t* lim;
  int32_t quantize;
  // work split (see attn_plan): tasks below nfull run whole; the rest in ranges of `per` key blocks, a task cut by a
  // range boundary leaving one partial per range in ws (mp slots per tail task)
  int32_t ntask;
  int32_t nfull;
  int32_t per;
  int32_t mp;
  float* ws;
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}


// Reductions over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the lane groups holding one query's keys), with the
// gfx950 row-swap permutes instead of LDS round trips: permlane16_swap(x, x) yields rows {0,0,2,2} and {1,1,3,3},
// permlane32_swap(x, x) rows {0,1,0,1} and {2,3,2,3}.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max4(float v) {
  v = max_xor16(v);
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum4(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A rebase of the running max happens only when a block's scores exceed it by more than this many log2 units, so
// most blocks skip the rescale of O; P then stays below 2^8 (exact enough in fp32, rounded to bf16 like any P).
constexpr float kAtRebase = 8.0f;


// Swizzle of the 16-byte chunks of V^T row dim (only dim % 16 matters)
__device__ __forceinline__ int vswz(int dim) { return ((dim >> 1) & 7) ^ (dim & 1); }

// A partial result of a key range, for the combine pass: O^T unnormalised [queries][128 dims], then the running max
// m (log2 units; -inf when no key of the range was visible) and the sum l of each query, all fp32.
constexpr int part_floats(int q) { return q * kAtHD + 2 * q; }

// W waves per workgroup (4 or 8), 32 queries each; two 4-wave or one 8-wave workgroup per CU (256 VGPRs per wave,
// 64 KB of LDS per workgroup). The 8 waves of the larger workgroup meet at every key block's barrier, so they
// progress together, and each staged key block serves 256 queries.
template <int W>
__global__ __launch_bounds__(W * 64, 8 / W) void attn_kernel(AttnArgs a) {
  constexpr int kAtThreads = W * 64, kAtQ = W * kAtQW, kAtPart = part_floats(kAtQ);
  constexpr int NI = 16 / W;  // 16-byte staging chunks per thread per K (and per V^T) block
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kAtStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int nqb = a.nq / kAtQ, nblk = a.nk / kAtKB;

  // Work is the flattened (task, key block) space, task = (head, query block) with a head's query blocks adjacent.
  // Workgroups below nfull take one whole task. The others split the tail tasks' key blocks into contiguous ranges
  // of `per` blocks; a task cut by a range boundary leaves one partial per range in the workspace, merged by
  // attn_combine_kernel. Workgroups are dispatched round robin over the 8 XCDs; xcd_remap gives each XCD a contiguous
  // run of tasks (and of ranges), so a head's K and V^T are pulled into fewer of the XCDs' L2 caches.
  const int bid = (int)blockIdx.x < a.nfull ? xcd_remap(blockIdx.x, a.nfull)
                                            : a.nfull + xcd_remap(blockIdx.x - a.nfull, gridDim.x - a.nfull);
  const int ti = bid - a.nfull;  // tail range index (negative for a whole-task workgroup)
  const int f0 = ti < 0 ? bid * nblk : a.nfull * nblk + ti * a.per;
  const int f1 = ti < 0 ? f0 + nblk : min(f0 + a.per, a.ntask * nblk);
  for (int f = f0; f < f1;) {
    const int task = f / nblk, kb0 = f - task * nblk, kb1 = min(nblk, f1 - task * nblk);
    if (f > f0) __syncthreads();  // a second segment reuses the LDS buffers
    f = task * nblk + kb1;
    const int h = task / nqb, qb = task - h * nqb;
    const int q0 = qb * kAtQ + wave * kAtQW;
    const uint16_t* Qh = a.q + (int64_t)h * a.nq * kAtHD;
    const uint16_t* Kh = a.k + (int64_t)h * a.nk * kAtHD;
    const uint16_t* Vh = a.vt + (int64_t)h * kAtHD * a.nk;

    // Q^T as the B operand: set s, 32-dim step st: Q[q0 + 16 s + l16][32 st + 8 lg .. + 7]
    bf16x8 qB[2][4];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int st = 0; st < 4; st++)
        qB[s][st] = *reinterpret_cast<const bf16x8*>(Qh + (int64_t)(q0 + 16 * s + l16) * kAtHD + 32 * st + 8 * lg);
    int lim[2];
#pragma unroll
    for (int s = 0; s < 2; s++) lim[s] = a.lim ? a.lim[q0 + 16 * s + l16] : 0x7FFFFFFF;

    f32x4 O[2][8];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int dg = 0; dg < 8; dg++) O[s][dg] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f};
    // {-m, -m, -m, -m} per set (0 while no key has been visible), the first score product's accumulator input;
    // changed only when the running max is rebased
    f32x4 nb4[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};

    // LDS: K buffers 0, 1, then V^T buffers 0, 1 (16 KB each). K runs one key block ahead of V: iteration j computes
    // S(j + 1) from K buffer (j + 1) % 2 while O accumulates P(j) V(j) from V buffer j % 2, and the softmax of block
    // j + 1 (VALU) can be scheduled between the P(j) V(j) MFMAs.
    uint8_t* const kbuf = lds;
    uint8_t* const vbuf = lds + 2 * kAtK;
    // staging: K chunks c = tid + 256 i -> (key c / 16, 16-byte chunk c % 16); V^T chunks -> (dim c / 8, 8 keys c % 8);
    // buffer loads with one 32-bit lane offset per operand, the chunk and block offsets wave-uniform
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void*)Kh, (short)0, (int)((int64_t)a.nk * kAtHD * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)Vh, (short)0, (int)((int64_t)a.nk * kAtHD * 2), 0x00020000);
    const uint32_t kvo = (uint32_t)((tid >> 4) * kAtHD * 2 + (tid & 15) * 16);  // + i * 4W keys, + block
    const uint32_t vvo = (uint32_t)((tid >> 3) * a.nk * 2 + (tid & 7) * 16);    // + i * 8W dims, + block
    u32x4 rk[NI], rv[NI];
    auto load_k = [&](int kb) {
#pragma unroll
      for (int i = 0; i < NI; i++)
        rk[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              krs, kvo, (kb * kAtKB + 4 * W * i) * kAtHD * 2, 0));
    };
    auto load_v = [&](int kb) {
#pragma unroll
      for (int i = 0; i < NI; i++)
        rv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              vrs, vvo, 8 * W * i * a.nk * 2 + kb * kAtKB * 2, 0));
    };
    auto store_k = [&](int buf) {
      uint8_t* sk = kbuf + buf * kAtK;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const int c = tid + kAtThreads * i, key = c >> 4, ch = c & 15;
        *reinterpret_cast<u32x4*>(sk + key * 256 + ((ch ^ (key & 15)) << 4)) = rk[i];
      }
    };
    // V^T row byte of 4-key group k (keys 4k..4k+3 of the block): step c = k / 8, group w = k % 8 -> 16-byte chunk
    // 4c + w % 4, half w / 4. Chunks are XOR-swizzled by vswz(dim): a permutation of 0..7 over the 8 rows of either
    // parity among 16 consecutive rows (16 lanes of an operand read hit distinct banks), and of opposite parity for
    // rows d, d + 1 (the 16 lanes of an 8-byte staging store, two rows, hit distinct 8-byte slots)
    auto vslot = [](int dim, int k) {
      const int w = k & 7;
      return dim * 128 + ((((k >> 3) * 4 + (w & 3)) ^ vswz(dim)) << 4) + ((w >> 2) << 3);
    };
    auto store_v = [&](int buf) {
      uint8_t* sv = vbuf + buf * kAtK;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const int c = tid + kAtThreads * i, dim = c >> 3, k = 2 * (c & 7);
        *reinterpret_cast<uint2*>(sv + vslot(dim, k)) = uint2{rv[i].x, rv[i].y};
        *reinterpret_cast<uint2*>(sv + vslot(dim, k + 1)) = uint2{rv[i].z, rv[i].w};
      }
    };

    // S^T - m of the segment's key block r: S[s][g] lane = keys 16 g + 4 lg + i (i = 0..3) of query 16 s + l16, minus
    // the query's running max (the accumulators start at -m; 0 while no key has been visible)
    f32x4 S[2][4];
    auto scores = [&](int r) {
      const uint8_t* sk = kbuf + (r & 1) * kAtK;
      // the first product of each tile takes {-m, -m, -m, -m} as its accumulator input straight from one register
      // group per set, so no tile is initialised with moves
#pragma unroll
      for (int g = 0; g < 4; g++) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
          const int key = 16 * g + l16, ch = 4 * st + lg;
          const bf16x8 kA = *reinterpret_cast<const bf16x8*>(sk + key * 256 + ((ch ^ l16) << 4));
#pragma unroll
          for (int s = 0; s < 2; s++) S[s][g] = mfma16(kA, qB[s][st], st == 0 ? nb4[s] : S[s][g]);
        }
      }
    };

    // online softmax (base 2) of key block b (absolute index): P^T -> Pb (bf16), row sums into lsum; alpha[s] is the factor O must take
    // (after its P V products of the previous block) when the running max was rebased, rebased[s] whether any lane of
    // the set did. The four lanes l16, l16 + 16, + 32, + 48 hold a query's 64 keys.
    auto softmax = [&](int b, u32x4 (&Pb)[2][2], float (&alpha)[2], bool (&rebased)[2]) {
      const bool full = (b + 1) * kAtKB <= a.nkv && !a.lim;
#pragma unroll
      for (int s = 0; s < 2; s++) {
        if (!full) {
#pragma unroll
          for (int g = 0; g < 4; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const int key = b * kAtKB + 16 * g + 4 * lg + i;
              if (key >= a.nkv || key > lim[s]) S[s][g][i] = -INFINITY;
            }
        }
        float mx = S[s][0][0];
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
          for (int i = 0; i < 4; i++) mx = fmaxf(mx, S[s][g][i]);
        mx = max4(mx);
        // rebase when the query has no reference yet, or this block exceeds it by more than kAtRebase
        const bool need = mx != -INFINITY && (m[s] == -INFINITY || mx > kAtRebase);
        const float delta = need ? mx : 0.f;
        alpha[s] = 1.f;
        rebased[s] = __any(need);
        if (rebased[s]) {  // wave-uniform branch, rare after the first block
          asm volatile("" ::: "memory");  // a real branch: executing this body on every block costs ~20 VALU per set
          alpha[s] = __builtin_amdgcn_exp2f(-delta);
          m[s] = need ? (m[s] == -INFINITY ? mx : m[s] + mx) : m[s];
          const float nb = m[s] == -INFINITY ? 0.f : -m[s];
          nb4[s] = f32x4{nb, nb, nb, nb};
          lsum[s] *= alpha[s];
#pragma unroll
          for (int g = 0; g < 4; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) S[s][g][i] -= delta;
        }
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
          for (int i = 0; i < 4; i++) S[s][g][i] = __builtin_amdgcn_exp2f(S[s][g][i]);
        // P^T operand for 32-key step c: keys 32c + 4 lg + 0..3 (group 2c), then 32c + 16 + 4 lg + 0..3 (group 2c + 1)
#pragma unroll
        for (int c = 0; c < 2; c++)
          Pb[s][c] = u32x4{pack_bf16_rne(S[s][2 * c][0], S[s][2 * c][1]), pack_bf16_rne(S[s][2 * c][2], S[s][2 * c][3]),
                           pack_bf16_rne(S[s][2 * c + 1][0], S[s][2 * c + 1][1]),
                           pack_bf16_rne(S[s][2 * c + 1][2], S[s][2 * c + 1][3])};
        // the row sum from the same bf16 P the second product uses
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
          for (int w = 0; w < 4; w++) {
            const uint32_t pw = Pb[s][c][w];  // a scalar copy: bit_cast of a vector-element lvalue reads element 0
            lsum[s] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pw), one, lsum[s], false);
          }
      }
    };

    // O^T += V^T P^T of the segment's block r: A = V^T rows 16 dg + l16, keys in the P^T order (4-key groups lg and
    // lg + 4 of step c: one 16-byte chunk)
    auto pv = [&](int r, const u32x4 (&Pb)[2][2]) {
      const uint8_t* sv = vbuf + (r & 1) * kAtK;
#pragma unroll
      for (int dg = 0; dg < 8; dg++) {
        const uint8_t* row = sv + (16 * dg + l16) * 128;
#pragma unroll
        for (int c = 0; c < 2; c++) {
          const bf16x8 vA = *reinterpret_cast<const bf16x8*>(row + (((4 * c + lg) ^ vswz(l16)) << 4));
#pragma unroll
          for (int s = 0; s < 2; s++) O[s][dg] = mfma16(vA, __builtin_bit_cast(bf16x8, Pb[s][c]), O[s][dg]);
        }
      }
    };

    const int nb = kb1 - kb0;  // key blocks kb0 .. kb1 - 1; segment-relative index r = block - kb0
    load_k(kb0);
    load_v(kb0);
    store_k(0);
    store_v(0);
    load_k(kb0 + min(1, nb - 1));
    store_k(1);
    __syncthreads();
    u32x4 Pb[2][2];
    float alpha[2];
    bool rebased[2];
    scores(0);
    softmax(kb0, Pb, alpha, rebased);  // O is still 0: no rescale
    // Every load and store below is unconditional: past the last block they repeat block kb1 - 1 into a buffer that is
    // not read again, which keeps the loop free of branches around memory operations. The loop runs two blocks per
    // trip, so each buffer index is a constant (an immediate LDS offset, no address arithmetic per block).
    auto iter = [&]<int P>(int j) {  // P = j % 2
      load_v(kb0 + j + 1);
      load_k(kb0 + min(j + 2, nb - 1));
      scores(1 - P);
      pv(P, Pb);
      u32x4 Pn[2][2];
      softmax(kb0 + j + 1, Pn, alpha, rebased);
#pragma unroll
      for (int s = 0; s < 2; s++) {
        if (rebased[s]) {  // O has P(j) V(j) now; a rebase at block j + 1 applies to all of it
#pragma unroll
          for (int dg = 0; dg < 8; dg++) O[s][dg] *= alpha[s];
        }
#pragma unroll
        for (int c = 0; c < 2; c++) Pb[s][c] = Pn[s][c];
      }
      store_v(1 - P);  // V buffer (j + 1) % 2 held V(j - 1), read in iteration j - 1
      store_k(P);      // K buffer j % 2 held K(j), read in iteration j - 1
      __syncthreads();
    };
    int j = 0;
    for (; j + 2 < nb; j += 2) {
      iter.template operator()<0>(j);
      iter.template operator()<1>(j + 1);
    }
    if (j + 1 < nb) {
      iter.template operator()<0>(j);
      pv(1, Pb);  // block nb - 1 = j + 1 is odd
    } else {
      pv(0, Pb);  // block nb - 1 = j is even
    }

    if (kb0 > 0 || kb1 < nblk) {
      // a piece of a task: O^T, m and l unnormalised into the workspace slot (tail task, piece)
      const int u = task - a.nfull;
      float* part = a.ws + ((int64_t)u * a.mp + (ti - u * nblk / a.per)) * kAtPart;
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const int ql = wave * kAtQW + 16 * s + l16;
        const float l = sum4(lsum[s]);
#pragma unroll
        for (int dg = 0; dg < 8; dg++) *reinterpret_cast<f32x4*>(part + ql * kAtHD + 16 * dg + 4 * lg) = O[s][dg];
        if (lg == 0) {
          part[kAtQ * kAtHD + ql] = m[s];
          part[kAtQ * kAtHD + kAtQ + ql] = l;
        }
      }
      continue;
    }

    // O = O^T / l: lane holds dims 16 dg + 4 lg + i of query q0 + 16 s + l16
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const float l = sum4(lsum[s]);
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t* orow = a.o + (int64_t)(q0 + 16 * s + l16) * a.ldo + (int64_t)(a.h0 + h) * kAtHD;
#pragma unroll
      for (int dg = 0; dg < 8; dg++) {
        uint32_t u[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; i++) u[i] = __float_as_uint(O[s][dg][i] * inv);
        if (a.quantize) {
          // an 8-dim block is split over lanes lg = 2t, 2t + 1 (4 dims each): exchange the exponent with lane ^ 16
          uint32_t E = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) E = max(E, (u[i] >> 23) & 0xFFu);
          const auto r = __builtin_amdgcn_permlane16_swap(E, E, false, false);
          E = max((uint32_t)r[0], (uint32_t)r[1]);
#pragma unroll
          for (int i = 0; i < 4; i++) b[i] = quantize_with_exp(u[i], E);
          *reinterpret_cast<uint2*>(orow + 16 * dg + 4 * lg) = uint2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
        } else {
          *reinterpret_cast<uint2*>(orow + 16 * dg + 4 * lg) =
              uint2{pack_bf16_rne(__uint_as_float(u[0]), __uint_as_float(u[1])),
                    pack_bf16_rne(__uint_as_float(u[2]), __uint_as_float(u[3]))};
        }
      }
    }
  }  // segments
}

// Merges the partials of one tail task cut into pieces: O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p with
// M = max_p m_p, summed in piece order (the result does not depend on which piece finished last), then the same
// bf16 or bfp16 output as the attention kernel's. Workgroup = (tail task, 16 queries); thread = (query, 8-dim block),
// 16 threads per query row. The pieces' loads are issued four at a time, so a thread waits about twice in all.
struct CombineArgs {
  const float* ws;
  uint16_t* o;
  int64_t ldo;
  int32_t h0;
  int32_t nq;
  int32_t nk;
  int32_t nfull;
  int32_t per;
  int32_t mp;
  int32_t quantize;
  int32_t qt;  // queries per task (128 or 256)
};

constexpr int kCbQ = 16;  // queries per combine workgroup

__global__ __launch_bounds__(256) void attn_combine_kernel(CombineArgs c) {
  const int kAtQ = c.qt, kAtPart = part_floats(kAtQ);
  const int nqb = c.nq / kAtQ, nblk = c.nk / kAtKB;
  const int u = blockIdx.x / (kAtQ / kCbQ), qs = blockIdx.x - u * (kAtQ / kCbQ), task = c.nfull + u;
  const int p0 = u * nblk / c.per, p1 = (u * nblk + nblk - 1) / c.per;
  if (p0 == p1) return;  // the task lay inside one range and was written whole
  const int np = p1 - p0 + 1;
  const int h = task / nqb, qb = task - h * nqb;
  const int ql = qs * kCbQ + (threadIdx.x >> 4), d8 = threadIdx.x & 15;
  const float* base = c.ws + (int64_t)u * c.mp * kAtPart;
  float mx = -INFINITY;
  for (int p = 0; p < np; p += 4) {
    float mm[4];
#pragma unroll
    for (int i = 0; i < 4; i++) mm[i] = p + i < np ? base[(p + i) * kAtPart + kAtQ * kAtHD + ql] : -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) mx = fmaxf(mx, mm[i]);
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, L = 0.f;
  if (mx != -INFINITY) {
    for (int p = 0; p < np; p += 4) {
      float mm[4], ll[4];
      f32x4 a0[4], a1[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float* pp = base + (int64_t)min(p + i, np - 1) * kAtPart;
        mm[i] = p + i < np ? pp[kAtQ * kAtHD + ql] : -INFINITY;
        ll[i] = pp[kAtQ * kAtHD + kAtQ + ql];
        a0[i] = *reinterpret_cast<const f32x4*>(pp + ql * kAtHD + 8 * d8);
        a1[i] = *reinterpret_cast<const f32x4*>(pp + ql * kAtHD + 8 * d8 + 4);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float w = __builtin_amdgcn_exp2f(mm[i] - mx);  // 0 for a piece with no visible key, or none at all
        L = fmaf(w, ll[i], L);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          acc[e] = fmaf(w, a0[i][e], acc[e]);
          acc[4 + e] = fmaf(w, a1[i][e], acc[4 + e]);
        }
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint32_t uu[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; i++) uu[i] = __float_as_uint(acc[i] * inv);
  uint16_t* orow = c.o + (int64_t)(qb * kAtQ + ql) * c.ldo + (int64_t)(c.h0 + h) * kAtHD + 8 * d8;
  if (c.quantize) {
    uint32_t E = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) E = max(E, (uu[i] >> 23) & 0xFFu);
#pragma unroll
    for (int i = 0; i < 8; i++) b[i] = quantize_with_exp(uu[i], E);
    *reinterpret_cast<u32x4*>(orow) =
        u32x4{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
  } else {
    *reinterpret_cast<u32x4*>(orow) =
        u32x4{pack_bf16_rne(__uint_as_float(uu[0]), __uint_as_float(uu[1])),
              pack_bf16_rne(__uint_as_float(uu[2]), __uint_as_float(uu[3])),
              pack_bf16_rne(__uint_as_float(uu[4]), __uint_as_float(uu[5])),
              pack_bf16_rne(__uint_as_float(uu[6]), __uint_as_float(uu[7]))};
  }
}


// The work split. T tasks meet R = CUs x 2 resident workgroups; whole rounds of tasks run as they are, and when the
// remainder is at most 4/5 of a round its tasks' key blocks are spread over R ranges of `per` blocks (at least 4)
// instead of taking a whole round. Returns the workspace floats the split needs (0: no split).
struct AttnPlan {
  int32_t w, ntask, nfull, per, mp, nwg;
  int64_t ws_floats;
};
static AttnPlan attn_plan(int32_t heads, int64_t nq, int64_t nk, int cus) {
  AttnPlan p;
  p.w = nq % (2 * kAtQMin) == 0 ? 8 : 4;  // waves per workgroup
  const int qt = p.w * kAtQW;
  p.ntask = (int32_t)(heads * (nq / qt));
  p.nfull = p.ntask;
  p.per = 0;
  p.mp = 0;
  p.nwg = p.ntask;
  p.ws_floats = 0;
  const int64_t R = (int64_t)cus * (8 / p.w), nblk = nk / kAtKB;  // resident workgroups
  if (R <= 0) return p;
  const int64_t rem = p.ntask % R;
  if (rem == 0 || rem * 5 > R * 4) return p;
  const int64_t tail = rem * nblk;
  const int64_t per = std::max<int64_t>(4, (tail + R - 1) / R);
  if (per >= nblk || (int64_t)p.ntask * nblk > INT32_MAX) return p;
  p.nfull = (int32_t)(p.ntask - rem);
  p.per = (int32_t)per;
  p.mp = (int32_t)((nblk + per - 1) / per + 1);
  p.nwg = (int32_t)(p.nfull + (tail + per - 1) / per);
  p.ws_floats = rem * p.mp * (int64_t)part_floats(qt);
  return p;
}

}  // namespace rl

extern "C" int64_t rl_attention_workspace_bytes(int32_t heads, int64_t nq, int64_t nk) {
  using namespace rl;
  if (rl_validate_attention(heads, nq, nk, nk, (int64_t)heads * kAtHD, 0)) return -1;
  check_device();  // fills the compute-unit count when a device is present; 256 otherwise
  ok();
  return attn_plan(heads, nq, nk, device_cus()).ws_floats * 4;
}

extern "C" int rl_attention_ws(const uint16_t* q, const uint16_t* k, const uint16_t* vt, int32_t heads, int64_t nq,
                               int64_t nk, int64_t nkv, const int32_t* lim, uint16_t* o, int64_t ldo, int32_t h0,
                               int32_t quantize_out, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace rl;
  int s = rl_validate_attention(heads, nq, nk, nkv, ldo, h0);
  if (s) return s;
  if (!q || !k || !vt || !o) return fail(RL_ERR_NULL, "q, k, vt or o is NULL");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)vt | (uintptr_t)o | (uintptr_t)workspace) % 16 || (uintptr_t)lim % 4)
    return fail(RL_ERR_ALIGN, "q, k, vt, o and the workspace must be 16-byte aligned, lim 4-byte aligned");
  if ((s = check_device())) return s;
  AttnPlan plan = attn_plan(heads, nq, nk, device_cus());
  if (!workspace) plan = attn_plan(heads, nq, nk, 0);  // no workspace: every task whole
  if (plan.ws_floats * 4 > workspace_bytes && plan.ws_floats > 0)
    return fail(RL_ERR_WORKSPACE, "workspace %lld bytes, this shape needs %lld (rl_attention_workspace_bytes)",
                (long long)workspace_bytes, (long long)(plan.ws_floats * 4));
  AttnArgs a;
  a.q = q; a.k = k; a.vt = vt; a.o = o; a.ldo = ldo; a.h0 = h0;
  a.heads = heads; a.nq = (int32_t)nq; a.nk = (int32_t)nk; a.nkv = (int32_t)nkv; a.lim = lim;
  a.quantize = quantize_out ? 1 : 0;
  a.ntask = plan.ntask; a.nfull = plan.nfull; a.per = plan.per; a.mp = plan.mp;
  a.ws = static_cast<float*>(workspace);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (plan.w == 8)
    hipLaunchKernelGGL(attn_kernel<8>, dim3((unsigned)plan.nwg), dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL(attn_kernel<4>, dim3((unsigned)plan.nwg), dim3(256), 0, st, a);
  if ((s = launch_status("rl_attention"))) return s;
  if (plan.nfull == plan.ntask) return RL_OK;
  CombineArgs c;
  c.ws = a.ws; c.o = o; c.ldo = ldo; c.h0 = h0; c.nq = a.nq; c.nk = a.nk; c.nfull = plan.nfull; c.per = plan.per;
  c.mp = plan.mp; c.quantize = a.quantize; c.qt = plan.w * kAtQW;
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)((plan.ntask - plan.nfull) * (c.qt / kCbQ))), dim3(256),
                     0, st, c);
  return launch_status("rl_attention (combine)");
}

extern "C" int rl_attention(const uint16_t* q, const uint16_t* k, const uint16_t* vt, int32_t heads, int64_t nq,
                            int64_t nk, int64_t nkv, const int32_t* lim, uint16_t* o, int64_t ldo, int32_t h0,
                            int32_t quantize_out, void* stream) {
  return rl_attention_ws(q, k, vt, heads, nq, nk, nkv, lim, o, ldo, h0, quantize_out, nullptr, 0, stream);
}
