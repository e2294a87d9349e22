// Online Hadamard transform of rotated down_proj inputs.
//
// Rotation-preprocessed checkpoints (SpinQuant-style, onecomp/pre_process)
// store down_proj weights multiplied by a normalised Hadamard matrix, so the
// layer input must be transformed online (vllm_plugins/utils/rotation.py:
// 100-112; onecomp/pre_process/hadamard_utils.py:178-199):
//     n = K * L with L a power of two; x viewed as K rows of length L;
//     u = FWHT_L(row) / sqrt(n) (natural-order Walsh-Hadamard per row);
//     y = H_K @ u, i.e. y = (H_K (x) H_L) x / sqrt(n).
// K is the largest supported block order dividing n with n / K a power of two
// (hadamard_utils.py:79-175 checks the orders in a fixed descending list).
//
// H_K is built here, not stored: the orders the reference ships that this
// build supports are reproduced exactly by three classical constructions
// (checked bit for bit against the reference's matrices by digest):
//   Paley I  (q prime, q = 3 mod 4, K = q + 1): H = I + S with S[0][j>0] = -1,
//            S[i>0][0] = +1, S[i][j] = chi(i - j) on the Jacobsthal block;
//   Paley II (q prime, q = 1 mod 4, K = 2(q + 1)): H = A (x) C + B (x) I with
//            C the symmetric conference matrix [[0, 1], [1, chi(j - i)]],
//            A = [[1, 1], [1, -1]], B = [[1, -1], [-1, -1]];
//   doubling: H_2K = [[1, 1], [1, -1]] (x) H_K;
//   Williamson (K = 4q): H = [[A, B, C, D], [-B, A, -D, C], [-C, D, A, -B],
//            [-D, -C, B, A]] with A..D symmetric q x q circulants,
//            A^2 + B^2 + C^2 + D^2 = 4q I.  The reference's orders 52, 100,
//            156 and 172 are Williamson matrices of this array; a symmetric
//            circulant is fixed by the first (q + 1) / 2 entries of its first
//            row, which kWill lists (the data that selects the reference's
//            matrices among the Williamson quadruples of each order).
// chi is the quadratic character mod q.
//
// One kernel, one workgroup per row: the length-L transforms in fp32 in LDS,
// then the 1/sqrt(n) scaling and the H_K block mix on MFMA (fp32
// accumulation), with the rounding points of the reference
// (rotation.py:100-112 -> hadamard_utils.py:178-199), by `rounding`:
//   OC_HAD_ROUND_FP32 (fp32_had = true: x.float() throughout, one cast back):
//     y = RNE(H_K (U / s)) with U / s kept in fp32: the mix multiplies H_K by
//     u split into two (fp16) or three (bf16) activation-dtype parts,
//     hi + lo (+ lo2), each an exact MFMA operand (fp16 lo is stored times
//     2^11, out of the subnormal range, and its fp32 sums scaled back), so the
//     fp32 sum carries u to 22 (fp16) / 24 (bf16) bits -- one rounding;
//   OC_HAD_ROUND_ONCE (fp32_had = false with the fused transform op, which
//     returns the activation dtype from fp32 sums): u = RNE(RNE(U) / s),
//     y = RNE(H_K u) -- three roundings (two with K = 1);
//   OC_HAD_ROUND_STAGES (fp32_had = false with the reference's pure-PyTorch
//     transform, hadamard_utils.py:26-44, which adds in the activation dtype):
//     every butterfly stage (bit 0 first, as the reference) rounds, then as
//     ROUND_ONCE.  Only the one-workgroup-per-row kernel has stages.
// U is the fp32 length-L transform and s = float32(sqrt(n)), the reference's
// torch.tensor(n).sqrt(); the divisions are IEEE fp32 divisions.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oc_common.h"

namespace {

// Orders in the reference's search order (largest first), with how to build them.
struct HadOrder {
  int K;
  int kind;  // 1 Paley I, 2 Paley II, 3 doubling of the order K/2, 4 Williamson (q = K/4)
  int q;
};
constexpr HadOrder kOrders[] = {{172, 4, 43}, {156, 4, 39}, {140, 1, 139}, {108, 1, 107}, {100, 4, 25},
                                {76, 2, 37},  {68, 1, 67},  {60, 1, 59},   {52, 4, 13},   {44, 1, 43},
                                {40, 3, 0},   {36, 2, 17},  {28, 2, 13},   {20, 1, 19},   {12, 1, 11}};

// Williamson generators: for each q, the first (q + 1) / 2 signs of the first
// rows of A, B, C, D ('+' = 1).
struct WillGen {
  int q;
  const char* half[4];
};
constexpr WillGen kWill[] = {
    {13, {"+-+--++", "+---+++", "++-+--+", "+----+-"}},
    {25, {"+-++++----++-", "+++-+++---+-+", "+-++-+++-++--", "+--++-+-+----"}},
    {39, {"+++--+-+-----+--++--", "++++---+--++----+-+-", "+++--++-+---+-+--+--", "+---++-+-+-----+++-+"}},
    {43, {"+---++--++++-+-+++-++-", "++-++++++----+-+--++-+", "+++-+-++--+-+-++++-+--",
          "++---++++-+--+--++----"}},
};

bool build_williamson(int q, int8_t* H) {
  const WillGen* g = nullptr;
  for (const WillGen& w : kWill)
    if (w.q == q) g = &w;
  if (!g) return false;
  int8_t row[4][64];
  for (int b = 0; b < 4; ++b)
    for (int j = 0; j <= q / 2; ++j) {
      const int8_t v = g->half[b][j] == '+' ? 1 : -1;
      row[b][j] = v;
      row[b][(q - j) % q] = v;  // symmetric circulant: entry j equals entry q - j
    }
  // block (bi, bj) of the array is sign * X with X in {A, B, C, D} (indices 0..3)
  static const int blk[4][4] = {{0, 1, 2, 3}, {1, 0, 3, 2}, {2, 3, 0, 1}, {3, 2, 1, 0}};
  static const int sgn[4][4] = {{1, 1, 1, 1}, {-1, 1, -1, 1}, {-1, 1, 1, -1}, {-1, -1, 1, 1}};
  const int K = 4 * q;
  for (int bi = 0; bi < 4; ++bi)
    for (int bj = 0; bj < 4; ++bj)
      for (int i = 0; i < q; ++i)
        for (int j = 0; j < q; ++j)
          H[(bi * q + i) * K + bj * q + j] = (int8_t)(sgn[bi][bj] * row[blk[bi][bj]][((j - i) % q + q) % q]);
  return true;
}

int quad_char(int a, int q) {
  a %= q;
  if (a < 0) a += q;
  if (a == 0) return 0;
  // Euler's criterion: a^((q-1)/2) mod q is 1 for residues, q-1 otherwise
  long long r = 1, b = a;
  int e = (q - 1) / 2;
  while (e) {
    if (e & 1) r = r * b % q;
    b = b * b % q;
    e >>= 1;
  }
  return r == 1 ? 1 : -1;
}

void build_paley1(int q, int8_t* H) {
  const int K = q + 1;
  for (int i = 0; i < K; ++i)
    for (int j = 0; j < K; ++j) {
      int v;
      if (i == 0) v = j == 0 ? 0 : -1;
      else if (j == 0) v = 1;
      else v = quad_char((i - 1) - (j - 1), q);
      H[i * K + j] = (int8_t)(v + (i == j ? 1 : 0));
    }
}

void build_paley2(int q, int8_t* H) {
  const int n = q + 1, K = 2 * n;
  static const int A[2][2] = {{1, 1}, {1, -1}}, B[2][2] = {{1, -1}, {-1, -1}};
  for (int bi = 0; bi < 2; ++bi)
    for (int bj = 0; bj < 2; ++bj)
      for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
          int c;
          if (i == 0) c = j == 0 ? 0 : 1;
          else if (j == 0) c = 1;
          else c = quad_char((j - 1) - (i - 1), q);
          H[(bi * n + i) * K + bj * n + j] = (int8_t)(A[bi][bj] * c + (i == j ? B[bi][bj] : 0));
        }
}

bool build_order(int K, int8_t* H) {
  for (const HadOrder& o : kOrders) {
    if (o.K != K) continue;
    if (o.kind == 1) {
      build_paley1(o.q, H);
      return true;
    }
    if (o.kind == 2) {
      build_paley2(o.q, H);
      return true;
    }
    if (o.kind == 4) return build_williamson(o.q, H);
    if (o.kind == 3) {
      const int h = K / 2;
      int8_t* S = (int8_t*)malloc((size_t)h * h);
      if (!S || !build_order(h, S)) {
        free(S);
        return false;
      }
      for (int bi = 0; bi < 2; ++bi)
        for (int bj = 0; bj < 2; ++bj)
          for (int i = 0; i < h; ++i)
            for (int j = 0; j < h; ++j)
              H[(bi * h + i) * K + bj * h + j] = (int8_t)((bi && bj ? -1 : 1) * S[i * h + j]);
      free(S);
      return true;
    }
    return false;
  }
  return false;
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// The block order the reference picks for n (hadamard_utils.py:79-175), or 0.
int pick_order(int n) {
  for (const HadOrder& o : kOrders)
    if (n % o.K == 0) return is_pow2(n / o.K) ? o.K : 0;
  return is_pow2(n) ? 1 : 0;
}

constexpr int kHadThreads = 1024;           // one workgroup per row
constexpr size_t kHadMaxLds = 160 * 1024;   // LDS of one CU

typedef float had_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 had_bf2 __attribute__((ext_vector_type(2)));

template <bool BF16>
__device__ __forceinline__ float had_in(uint16_t v) {
  return BF16 ? oc_bf2f(v) : oc_h2f(v);
}
template <bool BF16>
__device__ __forceinline__ uint16_t had_out(float v) {
  return BF16 ? oc_f2bf(v) : oc_f2h(v);
}
// Two fp32 rounded (RNE) to one packed pair of the activation dtype.
template <bool BF16>
__device__ __forceinline__ uint32_t had_pair(float lo, float hi) {
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(had_f2{lo, hi}, had_bf2));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(had_f2{lo, hi}, oc_half2));
}

// u of one transform value U under the rounding mode (see the top of the
// file): ROUND_FP32 gives the fp32 U / s, the others the activation-dtype
// value RNE(RNE(U) / s) as fp32.
template <bool BF16>
__device__ __forceinline__ float had_u(float U, float sq, int mode) {
  return mode == OC_HAD_ROUND_FP32 ? U / sq : had_in<BF16>(had_out<BF16>(had_in<BF16>(had_out<BF16>(U)) / sq));
}
// One value rounded to the activation dtype (a butterfly stage of ROUND_STAGES).
template <bool BF16>
__device__ __forceinline__ float had_rnd(float v) {
  return had_in<BF16>(had_out<BF16>(v));
}
// Part p of u as an exact activation-dtype operand: p = 0 the rounded value,
// p = 1, 2 the rounded remainders (ROUND_FP32 only; otherwise u is part 0).
// fp16's remainder is stored times 2^11 (kept out of the subnormal range,
// which MFMA operands need not honour); the sums of parts p >= 1 are
// multiplied by had_lo_scale.
template <bool BF16>
__device__ __forceinline__ float had_part(float u, int p) {
  const float hi = had_rnd<BF16>(u);
  if (p == 0) return hi;
  if constexpr (BF16) {
    const float lo = had_rnd<BF16>(u - hi);  // u - hi is exact, as is (u - hi) - lo
    return p == 1 ? lo : had_rnd<BF16>((u - hi) - lo);
  } else {
    return had_rnd<BF16>((u - hi) * 2048.f);
  }
}
template <bool BF16>
__device__ __forceinline__ constexpr float had_lo_scale() {
  return BF16 ? 1.f : 1.f / 2048.f;
}
// Operand parts of the H_K mix: 2 (fp16) or 3 (bf16) for ROUND_FP32, else 1.
__host__ __device__ __forceinline__ int had_parts(int mode, bool bf16) {
  return mode == OC_HAD_ROUND_FP32 ? (bf16 ? 3 : 2) : 1;
}

// One radix-2^R pass: butterflies (a, b) -> (a + b, a - b) over bits
// [b0, b0 + R) of the in-segment index, for every segment of the row at once
// (the segment index sits above those bits, so one group never straddles two).
// With b0 >= 6 the 64 lanes of a wave read 64 consecutive words per t: no
// bank conflicts.
template <int R, bool BF16, bool STAGES>
__device__ __forceinline__ void had_pass(float* f, int n, int b0) {
  const int groups = n >> R;
  for (int g = threadIdx.x; g < groups; g += kHadThreads) {
    const int base = ((g >> b0) << (b0 + R)) | (g & ((1 << b0) - 1));
    float v[1 << R];
#pragma unroll
    for (int t = 0; t < (1 << R); ++t) v[t] = f[base + (t << b0)];
#pragma unroll
    for (int s = 0; s < R; ++s)
#pragma unroll
      for (int t = 0; t < (1 << R); ++t)
        if (!(t & (1 << s))) {
          const float p = v[t], q = v[t | (1 << s)];
          v[t] = STAGES ? had_rnd<BF16>(p + q) : p + q;
          v[t | (1 << s)] = STAGES ? had_rnd<BF16>(p - q) : p - q;
        }
#pragma unroll
    for (int t = 0; t < (1 << R); ++t) f[base + (t << b0)] = v[t];
  }
}

// Workgroup barrier for LDS traffic only.  __syncthreads() carries a release
// fence that also waits for every outstanding global load, which would drain
// the next row's prefetch at each barrier; the row's own global stores and the
// prefetched loads need no ordering against other waves.
__device__ __forceinline__ void had_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// v from lane (lane ^ (1 << s)), s = 0, 1, 2, by DPP: quad permutations for
// xor 1 and 2; xor 4 as the half-row mirror (l -> 7 - l) then quad xor 3.
template <int S>
__device__ __forceinline__ float had_lane_xor(float v) {
  const int b = __float_as_int(v);
  if constexpr (S == 0) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));
  if constexpr (S == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));
  const int m = __builtin_amdgcn_mov_dpp(b, 0x141, 0xF, 0xF, false);
  return __int_as_float(__builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, false));
}

// Butterflies over bits 0 .. min(lgL, 6) - 1 of 8 consecutive elements per
// lane (element 8g + t, g = lane mod 64 + multiple of 64): bits 0-2 in
// registers, bits 3-5 across lanes g ^ 1, g ^ 2, g ^ 4.  Every lane whose
// elements are in the row has its partners in the row too (L >= 16 makes n
// a multiple of 8 * (partner span)).
template <bool BF16, bool STAGES>
__device__ __forceinline__ void had_first_bits(float (&v)[8], int lgL, int lane) {
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    if (b < lgL) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (!(t & (1 << b))) {
          const float p = v[t], q = v[t | (1 << b)];
          v[t] = STAGES ? had_rnd<BF16>(p + q) : p + q;
          v[t | (1 << b)] = STAGES ? had_rnd<BF16>(p - q) : p - q;
        }
    }
  }
  // the lane stages: the partner's value plus or minus this lane's (sg v + partner
  // is the exact sum or difference, rounded like a butterfly of the stage)
  if (lgL > 3) {
    const float sg = (lane & 1) ? -1.f : 1.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float r = fmaf(sg, v[t], had_lane_xor<0>(v[t]));
      v[t] = STAGES ? had_rnd<BF16>(r) : r;
    }
  }
  if (lgL > 4) {
    const float sg = (lane & 2) ? -1.f : 1.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float r = fmaf(sg, v[t], had_lane_xor<1>(v[t]));
      v[t] = STAGES ? had_rnd<BF16>(r) : r;
    }
  }
  if (lgL > 5) {
    const float sg = (lane & 4) ? -1.f : 1.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float r = fmaf(sg, v[t], had_lane_xor<2>(v[t]));
      v[t] = STAGES ? had_rnd<BF16>(r) : r;
    }
  }
}

// Four +-1 int8 of H_K (one 32-bit word) as two packed halves of +-1.0.
template <bool BF16>
__device__ __forceinline__ void had_signs(uint32_t w, uint32_t& p01, uint32_t& p23) {
  constexpr uint32_t one2 = BF16 ? 0x3F803F80u : 0x3C003C00u;
  p01 = one2 | ((w & 0x80u) << 8) | ((w & 0x8000u) << 16);
  p23 = one2 | ((w >> 8) & 0x8000u) | (w & 0x80000000u);
}

// Eight row elements 8g .. 8g+7 (zero past n) as fp32.
template <bool BF16>
__device__ __forceinline__ void had_load8(const uint16_t* xr, int n, int g, bool vx, float (&v)[8]) {
  if (vx) {
    const oc_u4 w = *(const oc_u4*)(xr + 8 * g);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      v[2 * t] = had_in<BF16>((uint16_t)(w[t] & 0xFFFF));
      v[2 * t + 1] = had_in<BF16>((uint16_t)(w[t] >> 16));
    }
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = 8 * g + t < n ? had_in<BF16>(xr[8 * g + t]) : 0.f;
  }
}

constexpr int kHadPre = 4;  // prefetched 16-byte words of the next row per thread (n <= 32768)

// y[m] = (H_K (x) H_L) x[m] / sqrt(n); each workgroup takes rows
// blockIdx.x, + gridDim.x, ... and prefetches its next row into registers
// while it transforms the current one.  Per row:
//  1. the row's elements, 8 consecutive per thread; bits 0-5 of the length-L
//     transform in registers and across lanes; fp32 to LDS;
//  2. radix passes over the remaining bits in LDS (fp32);
//  3. K = 1: scale, round, store.  K > 1: per chunk of J columns j, write
//     the NS operand parts of u^T[j][c] (zero for c >= K) to LDS and form
//     y[i][j] = sum_c H[i][c] u[c][j] with 16x16x32 MFMA (A = H_K as exact
//     +-1 halves, staged in LDS once; fp32 accumulate over the parts; one
//     rounding).
// A row is read whole before any of it is stored, so y may alias x.
template <bool BF16, bool STAGES>
__global__ __launch_bounds__(kHadThreads) void k_hadamard(const uint16_t* x, int ld_x, int M, int n, int lgL, int K,
                                                          const int8_t* __restrict__ hadk, int lgJ, float sq,
                                                          int mode, bool vx, bool vy, bool vy4, uint16_t* y,
                                                          int ld_y) {
  extern __shared__ __align__(16) float fbuf[];  // n floats | H_K [KR][US] | u^T parts [NS][J][US]
  const int tid = threadIdx.x;
  const int L = 1 << lgL;
  const int G8 = (n + 7) / 8;
  const int KP = (K + 31) & ~31, US = KP + 8;  // LDS rows of H_K and u^T: KP halves + 8 of padding
  const int J = 1 << lgJ, lgCT = lgJ - 4, RT = (K + 15) / 16, KS = KP / 32;
  uint16_t* hs = (uint16_t*)(fbuf + n);
  uint16_t* ut = hs + RT * 16 * US;
  const int lane = tid & 63, wave = tid >> 6, col = lane & 15, kq = lane >> 4;
  const bool pre = vx && G8 <= kHadPre * kHadThreads;
  const int NS = had_parts(mode, BF16);

  if (K > 1) {
    for (int q = tid; q < RT * 16 * (KP / 8); q += kHadThreads) {
      const int i = q / (KP / 8), c0 = 8 * (q % (KP / 8));
      uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
      if (i < K && c0 < K) had_signs<BF16>(*(const uint32_t*)(hadk + i * K + c0), a0, a1);
      if (i < K && c0 + 4 < K) had_signs<BF16>(*(const uint32_t*)(hadk + i * K + c0 + 4), a2, a3);
      *(oc_u4*)(hs + i * US + c0) = oc_u4{a0, a1, a2, a3};
    }
  }
  oc_u4 nxt[kHadPre];
  if (pre && blockIdx.x < M) {
    const uint16_t* xr = x + (size_t)blockIdx.x * ld_x;
#pragma unroll
    for (int s = 0; s < kHadPre; ++s)
      if (tid + s * kHadThreads < G8) nxt[s] = *(const oc_u4*)(xr + 8 * (tid + s * kHadThreads));
  }

  for (int row = blockIdx.x; row < M; row += gridDim.x) {
    const uint16_t* xr = x + (size_t)row * ld_x;
    uint16_t* yr = y + (size_t)row * ld_y;
#pragma unroll
    for (int s = 0; s < kHadPre; ++s) {
      const int g = tid + s * kHadThreads;
      if (!pre && s > 0) break;
      for (int gg = g; gg < G8; gg += pre ? G8 : kHadThreads) {  // one pass when prefetched
        float v[8];
        if (pre) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            v[2 * t] = had_in<BF16>((uint16_t)(nxt[s][t] & 0xFFFF));
            v[2 * t + 1] = had_in<BF16>((uint16_t)(nxt[s][t] >> 16));
          }
        } else {
          had_load8<BF16>(xr, n, gg, vx, v);
        }
        had_first_bits<BF16, STAGES>(v, lgL, lane);
        float* fp = fbuf + 8 * gg;
        if (8 * gg + 8 <= n) {
          *(oc_f4*)fp = oc_f4{v[0], v[1], v[2], v[3]};
          *(oc_f4*)(fp + 4) = oc_f4{v[4], v[5], v[6], v[7]};
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t)
            if (8 * gg + t < n) fp[t] = v[t];
        }
      }
    }
    had_sync();
    // the next row's loads run under this row's LDS work
    if (pre && row + (int)gridDim.x < M) {
      const uint16_t* xn = x + (size_t)(row + gridDim.x) * ld_x;
#pragma unroll
      for (int s = 0; s < kHadPre; ++s)
        if (tid + s * kHadThreads < G8) nxt[s] = *(const oc_u4*)(xn + 8 * (tid + s * kHadThreads));
    }

    // bits 6 and up in LDS, in passes of at most 4 bits
    int b0 = 6;
    while (b0 < lgL) {
      const int rem = lgL - b0;
      const int r = (rem + (rem + 3) / 4 - 1) / ((rem + 3) / 4);
      switch (r) {
        case 1: had_pass<1, BF16, STAGES>(fbuf, n, b0); break;
        case 2: had_pass<2, BF16, STAGES>(fbuf, n, b0); break;
        case 3: had_pass<3, BF16, STAGES>(fbuf, n, b0); break;
        default: had_pass<4, BF16, STAGES>(fbuf, n, b0); break;
      }
      b0 += r;
      had_sync();
    }

    if (K == 1) {
      for (int g = tid; g < G8; g += kHadThreads) {
        const float* fp = fbuf + 8 * g;
        if (vy) {
          const oc_f4 a = *(const oc_f4*)fp, b = *(const oc_f4*)(fp + 4);
          oc_u4 w;
          w[0] = had_pair<BF16>(had_u<BF16>(a[0], sq, mode), had_u<BF16>(a[1], sq, mode));
          w[1] = had_pair<BF16>(had_u<BF16>(a[2], sq, mode), had_u<BF16>(a[3], sq, mode));
          w[2] = had_pair<BF16>(had_u<BF16>(b[0], sq, mode), had_u<BF16>(b[1], sq, mode));
          w[3] = had_pair<BF16>(had_u<BF16>(b[2], sq, mode), had_u<BF16>(b[3], sq, mode));
          *(oc_u4*)(yr + 8 * g) = w;
        } else {
          for (int t = 0; t < 8; ++t)
            if (8 * g + t < n) yr[8 * g + t] = had_out<BF16>(had_u<BF16>(fp[t], sq, mode));
        }
      }
    } else {
      for (int j0 = 0; j0 < L; j0 += J) {
        for (int q = tid; q < (J << 2) * (KP / 32); q += kHadThreads) {
          const int jj = q & (J - 1), c0 = 8 * (q >> lgJ), j = j0 + jj;
          const float* fc = fbuf + c0 * L + j;
          float v[8];
          if (c0 + 8 <= K && j < L) {
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = had_u<BF16>(fc[t * L], sq, mode);
          } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = (c0 + t < K && j < L) ? had_u<BF16>(fc[t * L], sq, mode) : 0.f;
          }
          for (int p = 0; p < NS; ++p) {
            float w[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) w[t] = had_part<BF16>(v[t], p);
            *(oc_u4*)(ut + (p * J + jj) * US + c0) = oc_u4{had_pair<BF16>(w[0], w[1]), had_pair<BF16>(w[2], w[3]),
                                                           had_pair<BF16>(w[4], w[5]), had_pair<BF16>(w[6], w[7])};
          }
        }
        had_sync();
        // y^T = u^T H^T: A = u^T rows j, B = H_K rows i; lane (col, kq) ends
        // with y[i = 16 it + col][j = 16 ct + 4 kq .. + 3], one 8-byte store.
        for (int p = wave; p < (RT << lgCT); p += kHadThreads / 64) {
          const int it = p >> lgCT, ct = p & ((1 << lgCT) - 1);
          oc_f4 acc = oc_f4{0.f, 0.f, 0.f, 0.f}, accl = acc;
          for (int ks = 0; ks < KS; ++ks) {
            const int c0 = ks * 32 + 8 * kq;
            const oc_u4 bv = *(const oc_u4*)(hs + (it * 16 + col) * US + c0);
            acc = oc_mfma16<BF16>(*(const oc_u4*)(ut + (ct * 16 + col) * US + c0), bv, acc);
            for (int p = 1; p < NS; ++p) {
              const oc_u4 av = *(const oc_u4*)(ut + (p * J + ct * 16 + col) * US + c0);
              accl = oc_mfma16<BF16>(av, bv, accl);
            }
          }
          if (NS > 1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = fmaf(accl[r], had_lo_scale<BF16>(), acc[r]);
          }
          const int i = it * 16 + col, j = j0 + ct * 16 + 4 * kq;
          if (i < K) {
            uint16_t* yo = yr + (size_t)i * L + j;
            if (vy4 && j + 3 < L) {
              *(uint2*)yo = uint2{had_pair<BF16>(acc[0], acc[1]), had_pair<BF16>(acc[2], acc[3])};
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (j + r < L) yo[r] = had_out<BF16>(acc[r]);
            }
          }
        }
        had_sync();
      }
    }
    if (K == 1) had_sync();  // fbuf is rewritten by the next row
  }
}

// Small M: the same transform as products.  Workgroup (row, jt), four waves,
// stages the row in LDS (all loads in flight at once) and computes outputs
// j = 16 jt .. 16 jt + 15 of the length-L transforms of all K blocks:
// U[j][c] = sum_l W[j][l] x[c L + l] with W[j][l] = (-1)^popcount(j & l)
// formed in registers (16x16x32 MFMA, A = W, B = x from LDS, fp32
// accumulate), the waves taking every fourth 32-deep l-step and adding their
// sums in LDS; u (had_u: the rounding mode's value) then forms y[i L + j] =
// sum_c H_K[i][c] u[j][c] (a second MFMA over u's NS operand parts, one
// rounding): the rounding points of k_hadamard, with L / 16 workgroups per
// row instead of one.  Needs L >= 16
// and y not overlapping x (workgroups of a row read all of it while others
// store).
constexpr int kHadMmMaxKT = 11;                     // K <= 176
constexpr int kHadMmUS = kHadMmMaxKT * 16 + 24;     // LDS row of the u tile (halves)
constexpr int kHadMmMaxN = 32768;                   // row staged whole in LDS
// LDS: block c of the row at c (L + 8) halves (the 16-B pad keeps the 16 lanes of a B read, one
// block each, in different banks), the waves' partial sums, the u tile.
size_t had_mm_lds(int n, int K, int NS) {
  return (size_t)(n + 8 * K) * 2 + (size_t)4 * ((K + 15) / 16) * 256 * 4 + (size_t)NS * 16 * kHadMmUS * 2;
}

template <int KT, bool BF16>
__global__ __launch_bounds__(256) void k_hadamard_mm(const uint16_t* __restrict__ x, int ld_x, int n, int L, int K,
                                                      const int8_t* __restrict__ hadk, float sq, int mode,
                                                      uint16_t* __restrict__ y, int ld_y) {
  extern __shared__ __align__(16) uint16_t xsm[];
  const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kq = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ntile = L >> 4;
  const int row = blockIdx.x / ntile, jt = blockIdx.x - row * ntile;
  const uint16_t* xr = x + (size_t)row * ld_x;
  uint16_t* yr = y + (size_t)row * ld_y;
  const int G8 = n >> 3, LP = L + 8, lgL = 31 - __builtin_clz(L);
  float* red = (float*)(xsm + K * LP);                  // [4 waves][KT][4][64]
  uint16_t* ut = (uint16_t*)(red + 4 * KT * 256);       // [NS][16][US]
  const int NS = had_parts(mode, BF16);
  // stage the row: 8 chunks of 16 B per thread in flight per batch
  for (int q0 = 0; q0 < G8; q0 += 256 * 8) {
    oc_u4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int q = q0 + t * 256 + tid;
      if (q < G8) v[t] = *(const oc_u4*)(xr + 8 * q);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int q = q0 + t * 256 + tid;
      if (q < G8) *(oc_u4*)(xsm + ((8 * q) >> lgL) * LP + ((8 * q) & (L - 1))) = v[t];
    }
  }
  __syncthreads();
  constexpr int KP = (16 * KT + 31) & ~31;  // c padded to whole 32-deep MFMA steps
  constexpr int US = KP + 8;
  const uint32_t one = BF16 ? 0x3F80u : 0x3C00u;
  const int j = 16 * jt + col;
  oc_f4 acc[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) acc[t] = oc_f4{0.f, 0.f, 0.f, 0.f};
  for (int l0 = 32 * wave; l0 < L; l0 += 128) {
    const int lb = l0 + 8 * kq;  // this lane's 8 l's
    uint32_t aw[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t s0 = __builtin_popcount(j & (lb + 2 * t)) & 1, s1 = __builtin_popcount(j & (lb + 2 * t + 1)) & 1;
      aw[t] = (one | (s0 << 15)) | ((one | (s1 << 15)) << 16);
    }
    const oc_u4 av = oc_u4{aw[0], aw[1], aw[2], aw[3]};
#pragma unroll
    for (int ct = 0; ct < KT; ++ct) {
      const int c = 16 * ct + col;
      oc_u4 bv = oc_u4{0u, 0u, 0u, 0u};
      if (c < K && lb < L) bv = *(const oc_u4*)(xsm + c * LP + lb);
      acc[ct] = oc_mfma16<BF16>(av, bv, acc[ct]);
    }
  }
#pragma unroll
  for (int ct = 0; ct < KT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wave * KT + ct) * 4 + r) * 64 + lane] = acc[ct][r];
  __syncthreads();
  // the four partial sums; red[(ct * 4 + r) * 64 + lane] = U[j = 16 jt + 4 kq + r][c = 16 ct + col]
  for (int e = tid; e < KT * 256; e += 256) {
    const float u = red[e] + red[KT * 256 + e] + red[2 * KT * 256 + e] + red[3 * KT * 256 + e];
    const int ln = e & 63, r = (e >> 6) & 3, ct = e >> 8;
    const int jj = 4 * (ln >> 4) + r, c = 16 * ct + (ln & 15);
    const float uu = had_u<BF16>(u, sq, mode);
    if (K == 1) {
      if (c == 0) yr[16 * jt + jj] = had_out<BF16>(uu);
    } else {
      for (int p = 0; p < NS; ++p) ut[(p * 16 + jj) * US + c] = had_out<BF16>(had_part<BF16>(uu, p));
    }
  }
  if (K == 1) return;
  if constexpr (KP > 16 * KT) {  // c in [16 KT, KP): zero
    for (int q = tid; q < NS * 16 * (KP - 16 * KT); q += 256)
      ut[(q / (KP - 16 * KT)) * US + 16 * KT + q % (KP - 16 * KT)] = 0;
  }
  __syncthreads();
  // y[i][j] = sum_c u[j][c] H[i][c]: A = u rows j, B = H_K rows i (k = c); wave w takes i-tiles w, w + 4, ...
  for (int it = wave; it < KT; it += 4) {
    const int i = 16 * it + col;
    oc_f4 a2 = oc_f4{0.f, 0.f, 0.f, 0.f}, a2l = a2;
#pragma unroll
    for (int c0 = 0; c0 < KP; c0 += 32) {
      const int cb = c0 + 8 * kq;
      uint32_t p0 = 0, p1 = 0, p2 = 0, p3 = 0;
      if (i < K && cb < K) had_signs<BF16>(*(const uint32_t*)(hadk + i * K + cb), p0, p1);
      if (i < K && cb + 4 < K) had_signs<BF16>(*(const uint32_t*)(hadk + i * K + cb + 4), p2, p3);
      a2 = oc_mfma16<BF16>(*(const oc_u4*)(ut + col * US + cb), oc_u4{p0, p1, p2, p3}, a2);
      for (int p = 1; p < NS; ++p) {
        const oc_u4 uv = *(const oc_u4*)(ut + (p * 16 + col) * US + cb);
        a2l = oc_mfma16<BF16>(uv, oc_u4{p0, p1, p2, p3}, a2l);
      }
    }
    if (NS > 1) {
#pragma unroll
      for (int r = 0; r < 4; ++r) a2[r] = fmaf(a2l[r], had_lo_scale<BF16>(), a2[r]);
    }
    // a2[r] = y[i = 16 it + col][j = 16 jt + 4 kq + r]
    if (i < K) {
      uint16_t* yo = yr + (size_t)i * L + 16 * jt + 4 * kq;
#pragma unroll
      for (int r = 0; r < 4; ++r) yo[r] = had_out<BF16>(a2[r]);
    }
  }
}

// Dynamic LDS of k_hadamard for (n, K) with chunks of J columns.
size_t had_lds_bytes(int n, int K, int J, int NS) {
  size_t b = (size_t)n * 4;
  if (K > 1) b += (size_t)(((K + 15) / 16) * 16 + NS * J) * (((K + 31) & ~31) + 8) * 2;
  return b;
}

// log2 of the widest chunk (a power of two, 16 .. max(L, 16)) that fits the
// LDS; -1 if none does.
int had_chunk_log2(int n, int K, int NS) {
  int lg = 4;
  while ((1 << (lg + 1)) <= n / K) ++lg;
  while (lg >= 4 && had_lds_bytes(n, K, 1 << lg, NS) > kHadMaxLds) --lg;
  return lg >= 4 ? lg : -1;
}

}  // namespace


extern "C" int oc_hadamard_order(int n) { return n > 0 ? pick_order(n) : 0; }

extern "C" int oc_hadamard_block(int K, int8_t* out) {
  OC_REQUIRE(out, OC_ERR_INVALID, "null pointer");
  if (K == 1) {
    out[0] = 1;
    return 0;
  }
  OC_REQUIRE(build_order(K, out), OC_ERR_UNSUPPORTED,
             "no Hadamard block of order %d (the reference lists 12, 20, 28, 36, 40, 44, 52, 60, 68, 76, 100, 108, "
             "140, 156, 172)",
             K);
  return 0;
}

extern "C" int oc_hadamard(const void* x, int M, int n, int ld_x, const int8_t* hadk, int K, int act_dtype,
                           int rounding, void* y, int ld_y, void* stream) {
  OC_REQUIRE(x && y, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(M >= 0 && n > 0 && ld_x >= n && ld_y >= n, OC_ERR_INVALID, "bad shape M=%d n=%d ld_x=%d ld_y=%d", M,
             n, ld_x, ld_y);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d",
             act_dtype);
  OC_REQUIRE(K >= 1 && n % K == 0 && is_pow2(n / K), OC_ERR_SHAPE, "n=%d is not K=%d times a power of two", n, K);
  OC_REQUIRE(K == 1 || hadk, OC_ERR_INVALID, "K=%d needs the K x K block", K);
  OC_REQUIRE(K == 1 || K % 4 == 0, OC_ERR_SHAPE, "Hadamard order K=%d is not a multiple of 4", K);
  OC_REQUIRE(K == 1 || ((uintptr_t)hadk & 3) == 0, OC_ERR_INVALID, "the K x K block must be 4-byte aligned");
  OC_REQUIRE(rounding == OC_HAD_ROUND_FP32 || rounding == OC_HAD_ROUND_ONCE || rounding == OC_HAD_ROUND_STAGES,
             OC_ERR_INVALID, "bad rounding %d", rounding);
  const int mode = rounding;
  const int NS = had_parts(mode, act_dtype == OC_DTYPE_BF16);
  const int lgJ = K > 1 ? had_chunk_log2(n, K, NS) : 4;
  const size_t lds = had_lds_bytes(n, K, lgJ >= 4 ? 1 << lgJ : 16, NS);
  OC_REQUIRE(lds <= kHadMaxLds, OC_ERR_UNSUPPORTED, "n=%d (K=%d) needs %zu bytes of LDS, above the %zu of one CU",
             n, K, lds, kHadMaxLds);
  if (M == 0) return 0;
  int lgL = 0;
  while ((1 << lgL) < n / K) ++lgL;
  const float sq = sqrtf((float)n);  // IEEE-rounded, as torch.tensor(n).sqrt()
  const bool vx = n % 8 == 0 && ld_x % 8 == 0 && ((uintptr_t)x & 15) == 0;
  const bool vy = n % 8 == 0 && ld_y % 8 == 0 && ((uintptr_t)y & 15) == 0;
  const bool vy4 = (n / K) % 4 == 0 && ld_y % 4 == 0 && ((uintptr_t)y & 7) == 0;
  const int Lh = n / K;
  const char *xb = (const char*)x, *yb = (const char*)y;
  const bool overlap = xb < yb + (size_t)M * ld_y * 2 && yb < xb + (size_t)M * ld_x * 2;
  const int mm_max = oc::knob("OC_HAD_MM_M", 16);
  if (mode != OC_HAD_ROUND_STAGES && M <= mm_max && Lh >= 16 && K <= 16 * kHadMmMaxKT && n <= kHadMmMaxN && !overlap && vx &&
      ((uintptr_t)y & 1) == 0) {
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(M * (Lh / 16)));
    const size_t mlds = had_mm_lds(n, K, NS);
    const int KT = (K + 15) / 16;
    const bool bf = act_dtype == OC_DTYPE_BF16;
#define OC_HM(KT_)                                                                                              \
  if (KT == KT_) {                                                                                              \
    if (bf)                                                                                                     \
      hipLaunchKernelGGL((k_hadamard_mm<KT_, true>), grid, dim3(256), mlds, st, (const uint16_t*)x, ld_x, n, Lh, K, \
                         hadk, sq, mode, (uint16_t*)y, ld_y);                                                   \
    else                                                                                                        \
      hipLaunchKernelGGL((k_hadamard_mm<KT_, false>), grid, dim3(256), mlds, st, (const uint16_t*)x, ld_x, n, Lh,   \
                         K, hadk, sq, mode, (uint16_t*)y, ld_y);                                                \
  }
    OC_HM(1) OC_HM(2) OC_HM(3) OC_HM(4) OC_HM(5) OC_HM(6) OC_HM(7) OC_HM(8) OC_HM(9) OC_HM(10) OC_HM(11)
#undef OC_HM
    OC_HIP(hipGetLastError());
    return 0;
  }
  const int per_cu = (int)(kHadMaxLds / lds) < 2 ? 1 : 2;
  const int grid = M < oc_device_cus() * per_cu ? M : oc_device_cus() * per_cu;
  hipStream_t st = (hipStream_t)stream;
#define OC_HK(B_, S_)                                                                                       \
  hipLaunchKernelGGL((k_hadamard<B_, S_>), dim3(grid), dim3(kHadThreads), lds, st, (const uint16_t*)x, ld_x, M, n, \
                     lgL, K, hadk, lgJ, sq, mode, vx, vy, vy4, (uint16_t*)y, ld_y)
  const bool stages = mode == OC_HAD_ROUND_STAGES;
  if (act_dtype == OC_DTYPE_BF16) {
    if (stages) OC_HK(true, true);
    else OC_HK(true, false);
  } else {
    if (stages) OC_HK(false, true);
    else OC_HK(false, false);
  }
#undef OC_HK
  OC_HIP(hipGetLastError());
  return 0;
}
