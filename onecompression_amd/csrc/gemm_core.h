// Large-M dequant/sign GEMM core shared by the GPTQ and DBF paths.
//
// k_gemm<BITS, CS, BF16>: BITS in {2, 3, 4, 8} reads GPTQ codes in the
// lane-chunk layout and dequantises them exactly; BITS == 1 reads +-1 factors
// in the sign layout (dbf.hip) and applies an optional per-column post scale
// to the fp32 sums.  Everything else (tiling, x staging, pipelining, K-split
// tail) is shared.
#pragma once

#include <stdlib.h>

#include "gptq_decode.h"
#include "oc_common.h"

namespace oc_gemm {

constexpr int kGemmMaxTerms = 4;

struct GemmArgs {
  const uint16_t* x;     // [M, ldx] activations (16-bit), K valid columns
  const uint8_t* w;      // packed codes (lane-chunk layout) or sign words
  const uint32_t* meta;  // GPTQ: [G, N_pad] fp16 scale | restored zero << 16; signs: unused
  const uint16_t* post;  // optional per-column scale applied to the fp32 sums (signs)
  const uint16_t* bias;
  uint16_t* y;
  float* part;  // fp32 partial tiles of the K-split pieces (tiles_main.. onwards)
  int M, K, N, N_pad, NT_total, NU, G, gs, gshift, NKB, MB, NB;
  int ldx;       // row stride of x in elements
  int ldy;       // row stride of y in elements
  int uk_shift;  // signs: log2 of the k-blocks per unit
  int pstride;   // partial tiles per output tile in `part` (the fixup sums pstride)
  int poff;      // this launch's first partial slot inside a tile
  int tiles_main;  // workgroups below this index compute a whole tile
  int S, kper;     // the remaining tiles are split into S pieces of kper k-blocks
  // grouped launches (MoE experts, rows sorted by expert): workgroup L computes row tile
  // L / NB, column block L % NB; gtab[4 i ..] = expert, first row, rows of row tile i
  // (*gcount tiles); expert e's words / scale-zero words / bias start e * the strides in
  const int* gtab;
  const int* gcount;
  size_t gw_stride, gmeta_stride;
  int gbias_stride;
  // signs: columns npost .. N - 1 have no scale and come out as zeros
  int npost;
  // signs, k_gemm<.., MULTI>: nterms terms summed in one accumulation (MDBF).
  // x holds the terms' inputs side by side (k-blocks [tkb[t], tkb[t + 1]) of
  // the concatenated K are term t's); term t reads its own sign words (tw, tNU
  // units per row tile, 2^uk_shift k-blocks per unit for every term) and its
  // per-column scale tpost (null: 1) is folded into its +-1 operand (post unused)
  int nterms;
  int tkb[kGemmMaxTerms + 1];
  const uint8_t* tw[kGemmMaxTerms];
  const uint16_t* tpost[kGemmMaxTerms];
  int tNU[kGemmMaxTerms];
};

// Tile order: consecutive workgroups go to consecutive XCDs; with 8 | MB the
// 8 XCDs take 8 M-blocks of one column block at once (shared weights) and
// the CUs of one XCD share an M-block (x stays in that XCD's L2).
__device__ __forceinline__ void gemm_tile(int t, int MB, int NB, int& mb, int& nb) {
  if ((MB % 8) == 0) {
    const int xcd = t & 7, j = t >> 3;
    mb = (j / NB) * 8 + xcd;
    nb = j % NB;
  } else {
    mb = t / NB;
    nb = t % NB;
  }
}

// Packed words of one k-block per lane and chunk (lane-chunk layout of
// oc_common.h); BITS == 1 is the sign layout (one word per lane and k-block).
template <int BITS>
struct KbWords {
  static constexpr int n = BITS == 1 ? 1 : (BITS == 2 ? 2 : (BITS == 3 ? 3 : (BITS == 4 ? 4 : 8)));
};

typedef float oc_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 oc_bf2 __attribute__((ext_vector_type(2)));

// Two fp32 values rounded (RNE) to one bf16 pair word: v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16_pair_f32(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(oc_f2{lo, hi}, oc_bf2));
}

// ---------------------------------------------------------------------------
// Large M: fused dequant-GEMM with 32x32x16 MFMAs.  One wave per SIMD (4 waves, 256 threads)
// computes a 256 x 256 tile; wave w owns columns [64w, 64w + 64) over all 256
// rows, so every dequantised B fragment feeds 8 MFMAs.  The accumulators
// (8 x 2 tiles of 32 x 32 fp32 = 256 registers per lane) live in AGPRs.
//
// x tiles (256 rows x 128 k, 64 KB) go from HBM straight into LDS with
// buffer_load ... lds (no VGPR staging); 16-B chunk c of row r is stored at
// chunk position c ^ (r % 16) so that the A-fragment reads of 16 consecutive
// rows hit 16 distinct bank groups.  Rows >= M and chunks at k >= K read as
// zero through the buffer's range check.  Two LDS buffers alternate per
// k-block.
//
// B operands: the 32 columns of an MFMA are two 16-column chunks of the
// packed layout.  Lane l needs column l % 32 and the k-slice 8(l/32) of each
// 16-deep step; in chunk terms that is chunk-lane (l % 16) + 16 q with
// q = 2(s % 2) + l/32 for step s, so each lane loads two chunk-lanes per
// n32-tile and decodes exactly as the 16-column kernels do.  Codes decode to
// fp16 (1024 + q); fp16 output uses packed half subtract/multiply, bf16
// output forms s * (1024 + q) - s * (1024 + z) with one fma per value on an
// fp16 operand (v_fma_mix), exact in fp32, then rounds once to bf16.
// ---------------------------------------------------------------------------
constexpr int kGemmBM = 256, kGemmBN = 256;
constexpr size_t kGemmXBuf = (size_t)kGemmBM * 256;  // bytes of one x buffer (128 k of bf16 per row)

// Tile height 64 MT rows (MT = 1, 2, 4; 256 columns always): each wave holds
// NI = 2 MT m32-tiles of its 64 columns and loads XJ = 4 MT KB of each x block.
// (Prefetching x three k-blocks ahead instead of one, into four buffers, was
// measured at 64- and 128-row tiles and M <= 512: no change.)
template <int MT>
struct GemmTile {
  static_assert(MT == 1 || MT == 2 || MT == 4, "tile height 64, 128 or 256");
  static constexpr int BM = 64 * MT, NI = 2 * MT, XJ = 4 * MT;
  static constexpr size_t XBUF = (size_t)BM * 256;  // bytes of one x buffer
  static constexpr size_t LDS = 2 * XBUF;           // two buffers alternate per k-block
};

// Dynamic LDS bytes of a k_gemm launch with tile height 64 mt.
inline size_t gemm_lds_bytes(int mt) {
  return mt == 1 ? GemmTile<1>::LDS : (mt == 2 ? GemmTile<2>::LDS : GemmTile<4>::LDS);
}

typedef __attribute__((address_space(3))) void* oc_lds_ptr;

template <bool BF16>
struct GemmDeq {
  // fp16: pair (1024+z) and pair s; bf16: s and -s * (1024 + z) as fp32
  uint32_t a, b;
};

template <bool BF16>
__device__ __forceinline__ GemmDeq<BF16> gemm_deq(uint32_t md) {
  GemmDeq<BF16> d;
  const uint16_t sh = (uint16_t)(md & 0xFFFFu);
  const float zoff = 1024.f + (float)(md >> 16);
  if constexpr (BF16) {
    const float sf = oc_h2f(sh);
    d.a = __builtin_bit_cast(uint32_t, sf);
    d.b = __builtin_bit_cast(uint32_t, -sf * zoff);  // exact: 11-bit scale times an 11-bit integer
  } else {
    const uint16_t oz = oc_f2h(zoff);
    d.a = (uint32_t)oz | ((uint32_t)oz << 16);
    d.b = (uint32_t)sh | ((uint32_t)sh << 16);
  }
  return d;
}

template <bool BF16>
__device__ __forceinline__ uint32_t gemm_pair(uint32_t pr, GemmDeq<BF16> d) {
  if constexpr (BF16) {
    const oc_half2 h = __builtin_bit_cast(oc_half2, pr);
    const float sf = __builtin_bit_cast(float, d.a), cf = __builtin_bit_cast(float, d.b);
    return bf16_pair_f32(fmaf((float)h[0], sf, cf), fmaf((float)h[1], sf, cf));
  } else {
    const oc_half2 v = (__builtin_bit_cast(oc_half2, pr) - __builtin_bit_cast(oc_half2, d.a)) *
                       __builtin_bit_cast(oc_half2, d.b);
    return __builtin_bit_cast(uint32_t, v);
  }
}

// Built element by element on purpose: filling the vector in a loop has been
// miscompiled here (every element took the value of element 0).
template <bool BF16>
__device__ __forceinline__ oc_u4 gemm_apply(oc_u4 pr, GemmDeq<BF16> d) {
  return oc_u4{gemm_pair<BF16>(pr[0], d), gemm_pair<BF16>(pr[1], d), gemm_pair<BF16>(pr[2], d),
               gemm_pair<BF16>(pr[3], d)};
}

// Scheduling of one 16-MFMA step: the next step's LDS reads go out first (16
// MFMAs before their use), then each MFMA is followed by a share of the next
// step's dequantisation, so the matrix pipe never waits on a burst of VALU.
template <int NI = 8>
__device__ __forceinline__ void gemm_interleave() {
  constexpr int VPM = 24 / NI > 3 ? 24 / NI : 3;  // VALU per MFMA: the step's dequant spread evenly
  __builtin_amdgcn_sched_group_barrier(0x100, NI, 0);  // the next step's NI LDS reads first
#pragma unroll
  for (int i = 0; i < 2 * NI; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);  // VALU
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Vector-memory instructions of one k-block's weight loads in k_gemm: per
// n32-tile and chunk-lane half, b4 one 16-B load, b8 two, b2 one 8-B load, b3
// three 4-B loads, signs one 4-B load; plus (GPTQ) one scale/zero word per
// n32-tile and group segment.
template <int BITS, int CS>
struct GemmLoads {
  static constexpr int per = BITS == 8 ? 2 : (BITS == 3 ? 3 : 1);
  static constexpr int n = 4 * per + (BITS == 1 ? 0 : 2 * (4 / CS));
};

// Term of concatenated k-block kb (uniform; compares, no dynamic indexing of
// the kernel arguments; tkb[t] of absent terms is past every k-block).
__device__ __forceinline__ int gemm_term(const GemmArgs& a, int kb) {
  return (kb >= a.tkb[1]) + (kb >= a.tkb[2]) + (kb >= a.tkb[3]);
}

template <typename T>
__device__ __forceinline__ T gemm_pick(int t, T v0, T v1, T v2, T v3) {
  return t == 0 ? v0 : (t == 1 ? v1 : (t == 2 ? v2 : v3));
}

template <int BITS, int CS, bool BF16, int MT = 4, bool GROUPED = false, bool MULTI = false>
__global__ __launch_bounds__(256, 1) void k_gemm(const GemmArgs a) {
  using TL = GemmTile<MT>;
  constexpr int NI = TL::NI;
  constexpr int NWB = KbWords<BITS>::n;
  constexpr int SPK = 4 / CS;  // meta words per n32-tile per k-block
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, r16 = lane & 15;
  const int L = blockIdx.x;
  // whole tile, or piece `split` of a tile cut along K
  const bool piece = !GROUPED && L >= a.tiles_main;
  const int pidx = L - a.tiles_main;
  const int tile = piece ? a.tiles_main + pidx / a.S : L;
  const int kb0 = piece ? (pidx % a.S) * a.kper : 0;
  const int kb1 = piece ? min(kb0 + a.kper, a.NKB) : a.NKB;
  int mb, nb, m0, mlim;
  const uint8_t* wsrc = a.w;
  const uint32_t* msrc = a.meta;
  const uint16_t* bsrc = a.bias;
  if constexpr (GROUPED) {
    const int i = L / a.NB;
    nb = L - i * a.NB;
    if (i >= __builtin_amdgcn_readfirstlane(*a.gcount)) return;
    const int e = __builtin_amdgcn_readfirstlane(a.gtab[4 * i]);
    m0 = __builtin_amdgcn_readfirstlane(a.gtab[4 * i + 1]);
    mlim = m0 + __builtin_amdgcn_readfirstlane(a.gtab[4 * i + 2]);
    wsrc += (size_t)e * a.gw_stride;
    msrc += (size_t)e * a.gmeta_stride;
    if (bsrc) bsrc += (size_t)e * a.gbias_stride;
    mb = 0;
  } else {
    gemm_tile(tile, a.MB, a.NB, mb, nb);
    m0 = mb * TL::BM;
    mlim = a.M;
  }
  const int n0 = nb * kGemmBN + wave * 64;  // first column of this wave
  int nt[2], cl[2];
#pragma unroll
  for (int T = 0; T < 2; ++T) nt[T] = min(n0 / 16 + 2 * T + ((lane >> 4) & 1), a.NT_total - 1);
#pragma unroll
  for (int q2 = 0; q2 < 2; ++q2) cl[q2] = r16 + 16 * (2 * q2 + h);
  constexpr bool SIGN = BITS == 1;
  // GPTQ: code mask and the fp16 (1024 + q) magic; signs: sign-bit mask and the +1 pair
  const uint32_t msk = oc_opaque(SIGN ? 0x80008000u : Geo<BITS>::MASK);
  const uint32_t mag = oc_opaque(SIGN ? (BF16 ? 0x3F803F80u : 0x3C003C00u) : dec_magic<false>());

  extern __shared__ __align__(16) uint8_t smem[];

  // x tile loader: wave w, instruction j fills LDS bytes [(XJ w + j) KB, +1 KB):
  // row 16 MT w + 4j + lane/16, chunk position lane % 16.
  const int rows_here = min(mlim - m0, TL::BM);
  const int X2 = a.ldx * 2;  // bytes per x row
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.x + (size_t)m0 * a.ldx), 0, rows_here * X2, 0x00020000);
  const int xrow = 16 * MT * wave + (lane >> 4);
  int xcoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xcoff[j] = (r16 ^ ((4 * j + (lane >> 4)) & 15));
  auto load_x = [&](int kb, int buf) {
    const bool tail = (kb + 1) * 128 > a.K;
#pragma unroll
    for (int j = 0; j < TL::XJ; ++j) {
      const int c = xcoff[j & 3];
      int off = (xrow + 4 * j) * X2 + kb * 256 + c * 16;
      if (tail && kb * 128 + 8 * c >= a.K) off = 0x7FFFFFF0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (oc_lds_ptr)(smem + buf * TL::XBUF + (TL::XJ * wave + j) * 1024),
                                               16, off, 0, 0, 0);
    }
  };
  // Packed words and scale/zero words of one k-block: loaded two k-blocks
  // ahead into one of three rotating register sets.  Each set costs exactly
  // GemmLoads<BITS, CS>::n vector-memory instructions (no two of its loads are
  // adjacent in memory, so none are merged), which the vmcnt waits rely on.
  auto load_w = [&](int kb, uint32_t (&wb)[2][2][NWB], uint32_t (&mw)[2][SPK]) {
    using GG = Geo<SIGN ? 4 : BITS>;
    const int u = kb / GG::U, kbl = kb % GG::U;
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      if constexpr (SIGN) {
        // word (rt, unit, lane, kbl) of the sign layout (MULTI: of the k-block's term)
        const uint8_t* ws = wsrc;
        int nu = a.NU, kbl = kb;
        if constexpr (MULTI) {
          const int t = gemm_term(a, kb);
          kbl = kb - gemm_pick(t, a.tkb[0], a.tkb[1], a.tkb[2], a.tkb[3]);
          ws = gemm_pick(t, a.tw[0], a.tw[1], a.tw[2], a.tw[3]);
          nu = gemm_pick(t, a.tNU[0], a.tNU[1], a.tNU[2], a.tNU[3]);
          mw[T][0] = (uint32_t)t;  // selects the term's operand scale (no load)
        }
        const int su = kbl >> a.uk_shift, skb = kbl & ((1 << a.uk_shift) - 1);
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2)
          wb[T][q2][0] = *((const uint32_t*)ws + ((((size_t)nt[T] * nu + su) * 64 + cl[q2]) << a.uk_shift) + skb);
      } else {
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        const uint8_t* base = wsrc + ((size_t)(nt[T] * a.NU + u) * GG::P) * 1024 + cl[q2] * 16;
        uint32_t* o = wb[T][q2];
        if constexpr (BITS == 4 || BITS == 8) {
#pragma unroll
          for (int pt = 0; pt < GG::P; ++pt) {
            const oc_u4 v = *(const oc_u4*)(base + pt * 1024);
            o[4 * pt] = v[0];
            o[4 * pt + 1] = v[1];
            o[4 * pt + 2] = v[2];
            o[4 * pt + 3] = v[3];
          }
        } else if constexpr (BITS == 2) {
          typedef uint32_t u2v __attribute__((ext_vector_type(2)));
          const u2v v = *(const u2v*)(base + 8 * kbl);
          o[0] = v[0];
          o[1] = v[1];
        } else {  // 3 words of k-block kbl inside the 12-word payload (3 parts of 4 words)
#pragma unroll
          for (int q = 0; q < 3; ++q) {
            const int wi = 3 * kbl + q;
            o[q] = *((const uint32_t*)(base + (wi >> 2) * 1024) + (wi & 3));
          }
        }
      }
#pragma unroll
      for (int q = 0; q < SPK; ++q) {
        const int k = kb * 128 + 32 * CS * q;
        const int g = min(a.gshift >= 0 ? (k >> a.gshift) : k / a.gs, a.G - 1);
        mw[T][q] = msrc[(size_t)g * a.N_pad + nt[T] * 16 + r16];
      }
      }
    }
  };
  // A-fragment byte offset of step s inside an x buffer (m-tile i adds 8 KB)
  int xa[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) xa[s] = (lane & 31) * 256 + (((2 * s + h) ^ r16) * 16);

  oc_f16v acc[NI][2];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][T][r] = 0.f;

  // MULTI: operand scale per term and n32-tile of this lane's column
  // (magnitude pair and the mask that flips the signs where it is negative):
  // post[n] (+1 without a post vector) below npost, 0 above.
  uint32_t smag[kGemmMaxTerms][2], sneg[kGemmMaxTerms][2];
  if constexpr (SIGN && MULTI) {
#pragma unroll
    for (int t = 0; t < kGemmMaxTerms; ++t)
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const int n = n0 + 32 * T + (lane & 31);
        const uint16_t* pp = gemm_pick(t, a.tpost[0], a.tpost[1], a.tpost[2], a.tpost[3]);
        const uint32_t p = (t < a.nterms && n < a.npost) ? (pp ? (uint32_t)pp[n] : (mag & 0xFFFFu)) : 0u;
        smag[t][T] = (p & 0x7FFFu) * 0x00010001u;
        sneg[t][T] = (p & 0x8000u) ? 0xFFFFFFFFu : 0u;
      }
  }
  // B operands of step s (both n32-tiles); dq holds the scale terms of the
  // current group and is refreshed when a new group starts.
  auto make_b = [&](const uint32_t (&wb)[2][2][NWB], const uint32_t (&mw)[2][SPK], int s, oc_u4 (&B)[2],
                    GemmDeq<BF16> (&dq)[2]) {
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      if constexpr (SIGN) {
        // pairs 4t .. 4t+3 of the lane's word: bits 15-P / 31-P, set for -1
        const int P = 4 * (s >> 1);
        if constexpr (MULTI) {  // the term's scale: dq = (magnitude pair, sign-flip mask)
          if (s == 0) {
            const int t = (int)mw[T][0];
            dq[T].a = gemm_pick(t, smag[0][T], smag[1][T], smag[2][T], smag[3][T]);
            dq[T].b = gemm_pick(t, sneg[0][T], sneg[1][T], sneg[2][T], sneg[3][T]);
          }
          const uint32_t w = wb[T][s & 1][0] ^ dq[T].b, pm = dq[T].a;
          B[T] = oc_u4{((w << P) & msk) | pm, ((w << (P + 1)) & msk) | pm, ((w << (P + 2)) & msk) | pm,
                       ((w << (P + 3)) & msk) | pm};
        } else {
          const uint32_t w = wb[T][s & 1][0];
          B[T] = oc_u4{((w << P) & msk) | mag, ((w << (P + 1)) & msk) | mag, ((w << (P + 2)) & msk) | mag,
                       ((w << (P + 3)) & msk) | mag};
        }
      } else {
        if (s == 0 || (CS == 1 && (s & 1) == 0)) dq[T] = gemm_deq<BF16>(mw[T][(s >> 1) / CS]);
        B[T] = gemm_apply<BF16>(decode_step<BITS, false>(wb[T][s & 1], s >> 1, msk, mag), dq[T]);
      }
    }
  };
  auto mma = [&](const oc_u4 (&A)[NI], const oc_u4 (&B)[2]) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int T = 0; T < 2; ++T) acc[i][T] = oc_mfma32<BF16>(A[i], B[T], acc[i][T]);
  };
  // One k-block: 8 steps of 16 k.  The A fragments and B operands of step
  // s + 1 are read / dequantised while the 2 NI MFMAs of step s run; B of step 0
  // (B0 on entry) was prepared before the barrier that opened this k-block.
  auto compute = [&](int buf, const uint32_t (&wb)[2][2][NWB], const uint32_t (&mw)[2][SPK], oc_u4 (&B0)[2],
                     GemmDeq<BF16> (&dq)[2]) {
    const uint8_t* xb = smem + buf * TL::XBUF;
    auto read_a = [&](int s, oc_u4 (&A)[NI]) {
#pragma unroll
      for (int i = 0; i < NI; ++i) A[i] = *(const oc_u4*)(xb + xa[s] + i * 8192);
    };
    oc_u4 A0[NI], A1[NI], B1[2];
    read_a(0, A0);
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
      read_a(s + 1, A1);
      make_b(wb, mw, s + 1, B1, dq);
      mma(A0, B0);
      gemm_interleave<NI>();
      if (s + 2 < 8) {
        read_a(s + 2, A0);
        make_b(wb, mw, s + 2, B0, dq);
      }
      mma(A1, B1);
      gemm_interleave<NI>();
    }
  };

  oc_u4 B0[2];
  GemmDeq<BF16> dq[2];
  constexpr int NW = GemmLoads<BITS, CS>::n;
  // One k-block with register roles: wc/mc hold k-block kb, wn/mn k-block
  // kb + 1 (in flight), wf/mf receive k-block kb + 2.  x of kb + 1 goes out
  // first, so vmcnt(NW) at the end waits for it and for wn but not for wf.
  // Loads past the last k-block re-read the last one (clamped index) so that
  // every body issues the same instructions: the compiler's own waits stay
  // exact and never fall back to waiting for everything.
  const int last = kb1 - 1;
  // tail = one of the bodies after the loop: their prefetched weights are never used, so the
  // compiler deletes those loads and vmcnt(NW) would leave NW of the x-tile loads in flight
  // across the barrier (the next body would read stale x); they wait for everything instead.
  auto body = [&](int kb, const uint32_t (&wc)[2][2][NWB], const uint32_t (&mc)[2][SPK],
                  const uint32_t (&wn)[2][2][NWB], const uint32_t (&mn)[2][SPK], uint32_t (&wf)[2][2][NWB],
                  uint32_t (&mf)[2][SPK], const bool tail) {
    const int buf = (kb - kb0) & 1;
    load_x(min(kb + 1, last), buf ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(min(kb + 2, last), wf, mf);
    __builtin_amdgcn_sched_barrier(0);
    compute(buf, wc, mc, B0, dq);
    if (tail)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NW) : "memory");
    make_b(wn, mn, 0, B0, dq);
    // Plain s_barrier: __syncthreads() adds a workgroup release fence, which
    // waits for every outstanding load (vmcnt(0)) including k-block kb + 2.
    // LDS needs no fence: each wave's own x writes are complete (vmcnt above)
    // and its LDS reads of the buffer refilled next were consumed by MFMAs.
    asm volatile("s_barrier" ::: "memory");
  };

  uint32_t w0[2][2][NWB], w1[2][2][NWB], w2[2][2][NWB];
  uint32_t m0w[2][SPK], m1w[2][SPK], m2w[2][SPK];
  load_x(kb0, 0);
  load_w(kb0, w0, m0w);
  load_w(min(kb0 + 1, last), w1, m1w);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  make_b(w0, m0w, 0, B0, dq);
  __syncthreads();
  const int nkb = kb1 - kb0, groups = nkb / 3;
  for (int g = 0; g < groups; ++g) {
    body(kb0 + 3 * g, w0, m0w, w1, m1w, w2, m2w, false);
    body(kb0 + 3 * g + 1, w1, m1w, w2, m2w, w0, m0w, false);
    body(kb0 + 3 * g + 2, w2, m2w, w0, m0w, w1, m1w, false);
  }
  if (nkb % 3 >= 1) body(kb0 + 3 * groups, w0, m0w, w1, m1w, w2, m2w, true);
  if (nkb % 3 == 2) body(kb0 + 3 * groups + 1, w1, m1w, w2, m2w, w0, m0w, true);
  // the last body prefetched into the idle x buffer: let it land before exit
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  float ps[2] = {1.f, 1.f};  // per-column post scale (single-operand signs; 0 past npost)
  if constexpr (SIGN && !MULTI) {
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      const int n = n0 + 32 * T + (lane & 31);
      if (n >= a.npost) ps[T] = 0.f;
      else if (a.post) ps[T] = BF16 ? oc_bf2f(a.post[n]) : oc_h2f(a.post[n]);
    }
  }
  if (piece) {
    // fp32 partial tile in register order [wave][i][T][r][lane]: 256-B stores
    const int slot = (pidx / a.S) * a.pstride + a.poff + pidx % a.S;
    float* pp = a.part + (size_t)slot * (TL::BM * kGemmBN) + wave * (NI * 2 * 16 * 64) + lane;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 16; ++r)  // rows past M are never read by the fixup (skipped below 256-row tiles)
          if (MT == 4 || m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3) < mlim)
            pp[((i * 2 + T) * 16 + r) * 64] = acc[i][T][r] * ps[T];
    return;
  }
  // epilogue: register r of tile (i, T) is row 32i + 8(r/4) + 4h + r%4, column n0 + 32T + lane%32
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    const int n = n0 + 32 * T + (lane & 31);
    if (n >= a.N) continue;
    float b = 0.f;
    if (bsrc) b = BF16 ? oc_bf2f(bsrc[n]) : oc_h2f(bsrc[n]);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < mlim) {
          const float v = fmaf(acc[i][T][r], ps[T], b);
          a.y[(size_t)m * a.ldy + n] = BF16 ? oc_f2bf(v) : oc_f2h(v);
        }
      }
  }
}

// y for the K-split tiles: the pstride fp32 partial tiles summed in slot
// order (deterministic) plus bias.  One thread per element of a BM x 256 tile,
// in the partials' register order [wave][i][T][r][lane].
template <bool BF16, int MT = 4>
__global__ __launch_bounds__(256) void k_gemm_fixup(const GemmArgs a) {
  using TL = GemmTile<MT>;
  constexpr int LNI = MT == 1 ? 1 : (MT == 2 ? 2 : 3);  // log2 NI
  const int t = blockIdx.y;  // split tile
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int lane = e & 63, r = (e >> 6) & 15, T = (e >> 10) & 1, i = (e >> 11) & (TL::NI - 1),
            wave = e >> (11 + LNI);
  int mb, nb;
  gemm_tile(a.tiles_main + t, a.MB, a.NB, mb, nb);
  const int m = mb * TL::BM + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  const int n = nb * kGemmBN + 64 * wave + 32 * T + (lane & 31);
  if (m >= a.M || n >= a.N) return;
  const float* pp = a.part + (size_t)t * a.pstride * (TL::BM * kGemmBN) + e;
  float v = 0.f;
  for (int s = 0; s < a.pstride; ++s) v += pp[(size_t)s * (TL::BM * kGemmBN)];
  if (a.bias) v += BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
  a.y[(size_t)m * a.ldy + n] = BF16 ? oc_f2bf(v) : oc_f2h(v);
}


// Large-M tiling: whole 64 MT x 256 tiles, except that a last round of tiles
// that would leave more than half of the CUs idle is cut along K into S
// pieces (at least 4 k-blocks each) whose fp32 partials k_gemm_fixup sums.
struct GemmPlan {
  int MB, NB, NKB, tiles_main, split_tiles, S, kper;
  size_t part_bytes;
};

inline int device_cus() { return oc_device_cus(); }

// Tile height (64 MT rows, 256 columns) for M rows: the tallest that still
// leaves at least half as many tiles as CUs (measured: fewer, taller tiles
// lose to more, shorter ones until the grid covers the GPU).
inline int gemm_tile_height(int M, int N_pad) {
  const int NB = (N_pad + kGemmBN - 1) / kGemmBN, C = device_cus();
  for (int mt = 4; mt > 1; mt /= 2)
    if (((M + 64 * mt - 1) / (64 * mt)) * NB * 2 >= C) return mt;
  return 1;
}

// M rows, N_pad columns (multiple of 16), K_pad = 128 * k-blocks; split_env
// forces the piece count (1 = never split, 0 = automatic).
inline GemmPlan plan_gemm(int M, int N_pad, int K_pad, int split_env, int MT = 4) {
  GemmPlan p;
  const int BM = 64 * MT;
  p.MB = (M + BM - 1) / BM;
  p.NB = (N_pad + kGemmBN - 1) / kGemmBN;
  p.NKB = K_pad / 128;
  const int T = p.MB * p.NB, C = device_cus();
  const int rem = T % C;
  p.tiles_main = T;
  p.split_tiles = 0;
  p.S = 1;
  p.kper = p.NKB;
  int S = rem > 0 && 2 * rem <= C ? C / rem : 1;
  if (split_env > 0) S = split_env;
  if (S > 8) S = 8;
  while (S > 1 && p.NKB / S < 4) --S;
  if (rem > 0 && S > 1) {
    p.kper = (p.NKB + S - 1) / S;
    p.S = (p.NKB + p.kper - 1) / p.kper;
    p.split_tiles = rem;
    p.tiles_main = T - rem;
  }
  p.part_bytes = (size_t)p.split_tiles * p.S * BM * kGemmBN * 4;
  return p;
}


}  // namespace oc_gemm
