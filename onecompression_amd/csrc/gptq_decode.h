// Register-level decoders of the lane-chunk layout (see oc_common.h).
//
// Every decoder turns packed codes into MFMA B-operand pair words: the low
// and high 16-bit halves hold (off + q) for k = 2p and k = 2p + 1 of a lane's
// 8-deep k-slice, as fp16 (0x6400 | q == 1024 + q, exact for q < 1024) or
// bf16 (0x4300 | q == 128 + q, exact for q < 128).  8-bit codes under bf16
// are converted exactly through fp32 instead (offset 0).  One pair costs one
// shift and one v_and_or_b32.
#pragma once

#include "oc_common.h"

template <int BITS>
struct Geo {
  static constexpr int U = BITS == 2 ? 2 : (BITS == 3 ? 4 : 1);  // k-blocks per unit
  static constexpr int P = BITS == 3 ? 3 : (BITS == 8 ? 2 : 1);  // 16-B parts per lane per unit
  static constexpr uint32_t MASK = BITS == 2 ? 0x00030003u
                                 : BITS == 3 ? 0x00070007u
                                 : BITS == 4 ? 0x000F000Fu
                                             : 0x00FF00FFu;
};

// 16-bit offset added by the decoder (value of the magic exponent).
template <int BITS, bool BF16>
__device__ __forceinline__ constexpr float dec_offset() {
  return BF16 ? (BITS == 8 ? 0.f : 128.f) : 1024.f;
}

template <bool BF16>
__device__ __forceinline__ uint32_t dec_magic() {
  return BF16 ? 0x43004300u : 0x64006400u;
}

__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t c) { return (v & m) | c; }

// bf16 pair of bytes `b` and `b + 2` of w (exact: integers <= 255 fit bf16).
template <int B>
__device__ __forceinline__ uint32_t bf16_byte_pair(uint32_t w) {
  const uint32_t lo = __builtin_bit_cast(uint32_t, (float)((w >> (8 * B)) & 0xFFu));
  const uint32_t hi = __builtin_bit_cast(uint32_t, (float)((w >> (8 * (B + 2))) & 0xFFu));
  return (hi & 0xFFFF0000u) | (lo >> 16);
}

// Decode k-block `kbl` of a lane's unit payload `w` (4*P words) into the B
// operands of its four MFMA steps.
template <int BITS, bool BF16>
__device__ __forceinline__ void decode_kblock(const uint32_t* w, int kbl, oc_u4 (&b)[4], uint32_t msk,
                                              uint32_t mag) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t W = w[t];
      b[t] = oc_u4{and_or(W, msk, mag), and_or(W >> 4, msk, mag), and_or(W >> 8, msk, mag),
                   and_or(W >> 12, msk, mag)};
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t W0 = w[2 * t], W1 = w[2 * t + 1];
      if constexpr (BF16) {
        b[t] = oc_u4{bf16_byte_pair<0>(W0), bf16_byte_pair<1>(W0), bf16_byte_pair<0>(W1),
                     bf16_byte_pair<1>(W1)};
      } else {
        b[t] = oc_u4{and_or(W0, msk, mag), and_or(W0 >> 8, msk, mag), and_or(W1, msk, mag),
                     and_or(W1 >> 8, msk, mag)};
      }
    }
  } else if constexpr (BITS == 2) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t W = w[2 * kbl + (t >> 1)];
      const int s = 8 * (t & 1);
      b[t] = oc_u4{and_or(W >> s, msk, mag), and_or(W >> (s + 2), msk, mag),
                   and_or(W >> (s + 4), msk, mag), and_or(W >> (s + 6), msk, mag)};
    }
  } else {  // BITS == 3
    const uint32_t w0 = w[3 * kbl], w1 = w[3 * kbl + 1], w2 = w[3 * kbl + 2];
    uint32_t pr[16];
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      pr[j] = and_or(w0 >> (3 * j), msk, mag);
      pr[5 + j] = and_or(w1 >> (3 * j), msk, mag);
      pr[10 + j] = and_or(w2 >> (3 * j), msk, mag);
    }
    // pair 15: bit i of both codes lives in bits 15 / 31 of word i
    pr[15] = and_or(w2 >> 13, 0x00040004u, and_or(w1 >> 14, 0x00020002u,
                                                  and_or(w0 >> 15, 0x00010001u, mag)));
#pragma unroll
    for (int t = 0; t < 4; ++t) b[t] = oc_u4{pr[4 * t], pr[4 * t + 1], pr[4 * t + 2], pr[4 * t + 3]};
  }
}

// Decode only MFMA step t (pairs 4t .. 4t+3) of k-block 0 of w.
template <int BITS, bool BF16>
__device__ __forceinline__ oc_u4 decode_step(const uint32_t* w, int t, uint32_t msk, uint32_t mag) {
  if constexpr (BITS == 4) {
    const uint32_t W = w[t];
    return oc_u4{and_or(W, msk, mag), and_or(W >> 4, msk, mag), and_or(W >> 8, msk, mag),
                 and_or(W >> 12, msk, mag)};
  } else if constexpr (BITS == 8) {
    const uint32_t W0 = w[2 * t], W1 = w[2 * t + 1];
    if constexpr (BF16) {
      return oc_u4{bf16_byte_pair<0>(W0), bf16_byte_pair<1>(W0), bf16_byte_pair<0>(W1), bf16_byte_pair<1>(W1)};
    } else {
      return oc_u4{and_or(W0, msk, mag), and_or(W0 >> 8, msk, mag), and_or(W1, msk, mag),
                   and_or(W1 >> 8, msk, mag)};
    }
  } else if constexpr (BITS == 2) {
    const uint32_t W = w[t >> 1];
    const int s = 8 * (t & 1);
    return oc_u4{and_or(W >> s, msk, mag), and_or(W >> (s + 2), msk, mag), and_or(W >> (s + 4), msk, mag),
                 and_or(W >> (s + 6), msk, mag)};
  } else {  // BITS == 3
    uint32_t pr[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int P = 4 * t + p;
      if (P < 15) {
        pr[p] = and_or(w[P / 5] >> (3 * (P % 5)), msk, mag);
      } else {
        pr[p] = and_or(w[2] >> 13, 0x00040004u, and_or(w[1] >> 14, 0x00020002u, and_or(w[0] >> 15, 0x00010001u, mag)));
      }
    }
    return oc_u4{pr[0], pr[1], pr[2], pr[3]};
  }
}
