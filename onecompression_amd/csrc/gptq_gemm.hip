// GPTQ dequant-GEMM hot path: y[M, N] = x[M, K] @ dequant(W)^T.
//
// Small M (<= 64): "skinny" kernel.  Bandwidth-bound: the packed weights are
// streamed once with 16-byte lane loads (1 KiB per wave instruction), decoded
// in registers into (off + q) fp16/bf16 pairs and fed as the B operand of
// v_mfma_f32_16x16x32_{f16,bf16}; x rows are the A operand.  The zero point
// and scale are applied once per group and column instead of per weight:
//     y[m, n] += s[g, n] * (sum_k x[m,k] (off + q[k,n]) - (off + z[g,n]) * sum_k x[m,k])
// where the group sums of x come from one extra MFMA against a ones operand.
// Work split: a workgroup (4 waves) owns NT n-tiles of 16 columns and one of
// S k-splits; its waves take the k-units round-robin, partials are reduced in
// LDS, and with S > 1 the fp32 partials of the S splits are summed in split
// order (deterministic) by k_splitk_reduce, a second launch on the same
// stream.  (An in-kernel last-arrival reduction needs agent-scope fences,
// which on gfx950 write back and invalidate the whole per-XCD L2: measured
// ~50 us per call.)
//
// Large M: k_gemm below (x tiles staged in LDS, weights dequantised in registers).
#include <stdlib.h>

#include "gptq_decode.h"
#include "oc_common.h"

namespace {

struct SkinnyArgs {
  const uint16_t* x;
  const uint8_t* w;
  const uint32_t* meta;
  const uint16_t* bias;
  uint16_t* y;
  float* partial;      // [S, M, N_pad] fp32 when S > 1
  int M, K, N, N_pad, NT_total, NU, G, gs, S, ups;
};

template <int BITS, int MB, int NT, bool BF16>
__global__ __launch_bounds__(256) void k_skinny(const SkinnyArgs a) {
  using GG = Geo<BITS>;
  constexpr int U = GG::U, P = GG::P;
  constexpr float OFF = dec_offset<BITS, BF16>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ntg = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const int col = lane & 15, kq = lane >> 4;
  const uint32_t msk = oc_opaque(GG::MASK), mag = oc_opaque(dec_magic<BF16>());
  const uint32_t one16 = BF16 ? 0x3F803F80u : 0x3C003C00u;
  const oc_u4 ones = oc_u4{one16, one16, one16, one16};

  int nt[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) nt[j] = min(ntg * NT + j, a.NT_total - 1);

  oc_f4 yacc[NT][MB];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) yacc[j][mb] = oc_f4{0.f, 0.f, 0.f, 0.f};

  const int u0 = s * a.ups, u1 = min(u0 + a.ups, a.NU);
  const int cs = a.gs >= 128 && (a.gs % 128) == 0 ? 4 : ((a.gs % 64) == 0 ? 2 : 1);

  for (int u = u0 + wave; u < u1; u += 4) {
    uint32_t wv[NT][4 * P];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const uint8_t* base = a.w + ((size_t)(nt[j] * a.NU + u) * P) * 1024 + lane * 16;
#pragma unroll
      for (int pt = 0; pt < P; ++pt) {
        const oc_u4 v = __builtin_nontemporal_load((const oc_u4*)(base + pt * 1024));
        wv[j][4 * pt + 0] = v[0];
        wv[j][4 * pt + 1] = v[1];
        wv[j][4 * pt + 2] = v[2];
        wv[j][4 * pt + 3] = v[3];
      }
    }
#pragma unroll
    for (int kbl = 0; kbl < U; ++kbl) {
      const int kb = u * U + kbl;
      oc_u4 bq[NT][4];
#pragma unroll
      for (int j = 0; j < NT; ++j) decode_kblock<BITS, BF16>(wv[j], kbl, bq[j], msk, mag);
      oc_f4 acc[NT][MB], xs[MB];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int k0 = kb * 128 + 32 * t + 8 * kq;
        oc_u4 av[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int m = mb * 16 + col;
          av[mb] = (m < a.M && k0 < a.K) ? *(const oc_u4*)(a.x + (size_t)m * a.K + k0)
                                         : oc_u4{0u, 0u, 0u, 0u};
        }
        const bool first = (t % cs) == 0;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          xs[mb] = oc_mfma16<BF16>(av[mb], ones, first ? oc_f4{0.f, 0.f, 0.f, 0.f} : xs[mb]);
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[j][mb] = oc_mfma16<BF16>(av[mb], bq[j][t], first ? oc_f4{0.f, 0.f, 0.f, 0.f} : acc[j][mb]);
        }
        if (((t + 1) % cs) == 0) {
          const int g = min((kb * 128 + 32 * t) / a.gs, a.G - 1);
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            const uint32_t md = a.meta[(size_t)g * a.N_pad + nt[j] * 16 + col];
            const float sc = oc_h2f((uint16_t)(md & 0xFFFFu));
            const float oz = OFF + (float)(md >> 16);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                yacc[j][mb][i] = fmaf(sc, fmaf(-oz, xs[mb][i], acc[j][mb][i]), yacc[j][mb][i]);
          }
        }
      }
    }
  }

  // ---- reduce the 4 waves in LDS ----
  extern __shared__ float red[];  // [4][NT][MB][4][64]
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave * NT + j) * MB + mb) * 4 + i) * 64 + lane] = yacc[j][mb][i];
  __syncthreads();
  constexpr int NE = NT * MB * 4 * 64;  // elements per wave slice
  const bool last_split = a.S == 1;
  float* part = a.partial + (size_t)s * a.M * a.N_pad;
  for (int e = threadIdx.x; e < NE; e += 256) {
    const float v = red[e] + red[NE + e] + red[2 * NE + e] + red[3 * NE + e];
    const int ln = e & 63, i = (e >> 6) & 3, mb = (e >> 8) % MB, j = (e >> 8) / MB;
    const int m = mb * 16 + 4 * (ln >> 4) + i;
    const int n = (ntg * NT + j) * 16 + (ln & 15);
    if (m >= a.M || ntg * NT + j >= a.NT_total) continue;
    if (last_split) {
      if (n < a.N) {
        float o = v;
        if (a.bias) o += BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
        a.y[(size_t)m * a.N + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
      }
    } else {
      part[(size_t)m * a.N_pad + n] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// M <= 16: latency-hiding GEMV.  Same math as k_skinny with one 16-row MFMA
// block.  Each wave streams its own k-units of the workgroup's columns and
// keeps the next D units in flight in registers: packed weights, scale/zero
// words and the x rows of that k-range.  x is bounced through a wave-private
// LDS slot to form the A operand (no workgroup barrier on the way in), A rows
// >= M read row M-1 (their output rows are never stored), and the group sums
// of x come from one MFMA against a ones operand.  W waves per workgroup
// split the k-range and are reduced in LDS at the end.
// ---------------------------------------------------------------------------
struct GemvArgs {
  const uint16_t* x;
  const uint8_t* w;
  const uint32_t* meta;
  const uint16_t* bias;
  uint16_t* y;
  float* partial;
  int M, K, N, N_pad, NT_total, NU, G, gs, gshift, S, ups;
};

template <int BITS, int NT, int CS, int D, int W, int XCH, bool BF16>
__global__ __launch_bounds__(64 * W) void k_gemv(const GemvArgs a) {
  using GG = Geo<BITS>;
  constexpr int U = GG::U, P = GG::P;
  constexpr int SPK = 4 / CS;        // correction segments per k-block
  constexpr int MPU = U * SPK;       // scale/zero words per unit and n-tile
  constexpr int XW = U * 128 + 8;    // halfs per staged x row (padded)
  constexpr float OFF = dec_offset<BITS, BF16>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ntg = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const int col = lane & 15, kq = lane >> 4;
  const uint32_t msk = oc_opaque(GG::MASK), mag = oc_opaque(dec_magic<BF16>());
  const uint32_t one16 = BF16 ? 0x3F803F80u : 0x3C003C00u;
  const oc_u4 ones = oc_u4{one16, one16, one16, one16};

  int nt[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) nt[j] = min(ntg * NT + j, a.NT_total - 1);

  const int u0 = s * a.ups, u1 = min(u0 + a.ups, a.NU);
  const int n_my = u0 + wave < u1 ? (u1 - u0 - wave + W - 1) / W : 0;

  // x chunk c of a unit (16 B = 8 k): row c / (16U), k offset 8 * (c % (16U))
  auto xchunk_ok = [&](int c) { return c < a.M * 16 * U; };

  uint32_t buf[D][NT][4 * P];
  uint32_t mbuf[D][NT][MPU];
  oc_u4 xbuf[D][XCH];
  auto load_unit = [&](int unit, uint32_t (&wb)[NT][4 * P], uint32_t (&mb)[NT][MPU], oc_u4 (&xb)[XCH]) {
#pragma unroll
    for (int q = 0; q < XCH; ++q) {
      const int c = lane + 64 * q;
      const int m = c / (16 * U), k = unit * U * 128 + 8 * (c % (16 * U));
      xb[q] = (xchunk_ok(c) && k < a.K) ? *(const oc_u4*)(a.x + (size_t)m * a.K + k) : oc_u4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const uint8_t* base = a.w + ((size_t)(nt[j] * a.NU + unit) * P) * 1024 + lane * 16;
#pragma unroll
      for (int pt = 0; pt < P; ++pt) {
        const oc_u4 v = __builtin_nontemporal_load((const oc_u4*)(base + pt * 1024));
        wb[j][4 * pt + 0] = v[0];
        wb[j][4 * pt + 1] = v[1];
        wb[j][4 * pt + 2] = v[2];
        wb[j][4 * pt + 3] = v[3];
      }
#pragma unroll
      for (int ci = 0; ci < MPU; ++ci) {
        const int kseg = (unit * U + ci / SPK) * 128 + 32 * ((ci % SPK) * CS);
        const int g = min(a.gshift >= 0 ? (kseg >> a.gshift) : kseg / a.gs, a.G - 1);
        mb[j][ci] = a.meta[(size_t)g * a.N_pad + nt[j] * 16 + col];
      }
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < n_my) load_unit(u0 + wave + W * d, buf[d], mbuf[d], xbuf[d]);

  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* xslot = (uint16_t*)smem + (size_t)wave * a.M * XW;  // this wave's x rows
  const uint16_t* arow = xslot + min(col, a.M - 1) * XW + 8 * kq;

  oc_f4 yacc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) yacc[j] = oc_f4{0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < n_my; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = i0 + d;
      if (i >= n_my) break;
      const int u = u0 + wave + W * i;
      // Bounce this unit's x rows through the wave's LDS slot.  Lanes read
      // what other lanes of the same wave wrote: the compiler barriers make
      // that exchange explicit (a wave's DS operations execute in order).
      oc_wave_lds_barrier();
#pragma unroll
      for (int q = 0; q < XCH; ++q) {
        const int c = lane + 64 * q;
        if (xchunk_ok(c)) *(oc_u4*)(xslot + (c / (16 * U)) * XW + 8 * (c % (16 * U))) = xbuf[d][q];
      }
      oc_wave_lds_barrier();
#pragma unroll
      for (int kbl = 0; kbl < U; ++kbl) {
        oc_u4 av[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) av[t] = *(const oc_u4*)(arow + kbl * 128 + 32 * t);
        oc_u4 bq[NT][4];
#pragma unroll
        for (int j = 0; j < NT; ++j) decode_kblock<BITS, BF16>(buf[d][j], kbl, bq[j], msk, mag);
        oc_f4 acc[NT], xs;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bool first = (t % CS) == 0;
          xs = oc_mfma16<BF16>(av[t], ones, first ? oc_f4{0.f, 0.f, 0.f, 0.f} : xs);
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[j] = oc_mfma16<BF16>(av[t], bq[j][t], first ? oc_f4{0.f, 0.f, 0.f, 0.f} : acc[j]);
          if ((t % CS) == CS - 1) {
            const int ci = kbl * SPK + t / CS;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
              const uint32_t md = mbuf[d][j][ci];
              const float sc = oc_h2f((uint16_t)(md & 0xFFFFu));
              const float oz = OFF + (float)(md >> 16);
#pragma unroll
              for (int r = 0; r < 4; ++r) yacc[j][r] = fmaf(sc, fmaf(-oz, xs[r], acc[j][r]), yacc[j][r]);
            }
          }
        }
      }
      if (i + D < n_my) load_unit(u + W * D, buf[d], mbuf[d], xbuf[d]);
    }
  }

  // ---- reduce the W waves ----
  __syncthreads();  // x slots no longer needed: reuse LDS
  float* red = (float*)smem;  // [W][NT][4][64]
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wave * NT + j) * 4 + r) * 64 + lane] = yacc[j][r];
  __syncthreads();
  constexpr int NE = NT * 4 * 64;
  float* part = a.partial + (size_t)s * a.M * a.N_pad;
  for (int e = threadIdx.x; e < NE; e += 64 * W) {
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) v += red[ww * NE + e];
    const int ln = e & 63, r = (e >> 6) & 3, j = e >> 8;
    const int m = 4 * (ln >> 4) + r;
    const int n = (ntg * NT + j) * 16 + (ln & 15);
    if (m >= a.M || ntg * NT + j >= a.NT_total) continue;
    if (a.S == 1) {
      if (n < a.N) {
        float o = v;
        if (a.bias) o += BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
        a.y[(size_t)m * a.N + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
      }
    } else {
      part[(size_t)m * a.N_pad + n] = v;
    }
  }
}

// y[m, n] = sum over splits (in split order) of partial[s, m, n] (+ bias).
template <bool BF16>
__global__ void k_splitk_reduce(const float* __restrict__ partial, int S, int M, int N, int N_pad,
                                const uint16_t* __restrict__ bias, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  float o = 0.f;
  for (int s = 0; s < S; ++s) o += partial[((size_t)s * M + m) * N_pad + n];
  if (bias) o += BF16 ? oc_bf2f(bias[n]) : oc_h2f(bias[n]);
  y[(size_t)m * N + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
}

struct GemmArgs {
  const uint16_t* x;
  const uint8_t* w;
  const uint32_t* meta;
  const uint16_t* bias;
  uint16_t* y;
  float* part;  // fp32 partial tiles of the K-split pieces (tiles_main.. onwards)
  int M, K, N, N_pad, NT_total, NU, G, gs, gshift, NKB, MB, NB;
  int tiles_main;  // workgroups below this index compute a whole tile
  int S, kper;     // the remaining tiles are split into S pieces of kper k-blocks
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

// Packed words of one k-block per lane and chunk (lane-chunk layout of oc_common.h).
template <int BITS>
struct KbWords {
  static constexpr int n = BITS == 2 ? 2 : (BITS == 3 ? 3 : (BITS == 4 ? 4 : 8));
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
__device__ __forceinline__ void gemm_interleave() {
  __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // the next step's 8 LDS reads first
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Vector-memory instructions of one k-block's weight loads in k_gemm: per
// n32-tile and chunk-lane half, b4 one 16-B load, b8 two, b2 one 8-B load, b3
// three 4-B loads; plus one scale/zero word per n32-tile and group segment.
template <int BITS, int CS>
struct GemmLoads {
  static constexpr int per = BITS == 8 ? 2 : (BITS == 3 ? 3 : 1);
  static constexpr int n = 4 * per + 2 * (4 / CS);
};

template <int BITS, int CS, bool BF16>
__global__ __launch_bounds__(256, 1) void k_gemm(const GemmArgs a) {
  constexpr int NWB = KbWords<BITS>::n;
  constexpr int SPK = 4 / CS;  // meta words per n32-tile per k-block
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, r16 = lane & 15;
  const int L = blockIdx.x;
  // whole tile, or piece `split` of a tile cut along K
  const bool piece = L >= a.tiles_main;
  const int pidx = L - a.tiles_main;
  const int tile = piece ? a.tiles_main + pidx / a.S : L;
  const int kb0 = piece ? (pidx % a.S) * a.kper : 0;
  const int kb1 = piece ? min(kb0 + a.kper, a.NKB) : a.NKB;
  int mb, nb;
  gemm_tile(tile, a.MB, a.NB, mb, nb);
  const int m0 = mb * kGemmBM;
  const int n0 = nb * kGemmBN + wave * 64;  // first column of this wave
  int nt[2], cl[2];
#pragma unroll
  for (int T = 0; T < 2; ++T) nt[T] = min(n0 / 16 + 2 * T + ((lane >> 4) & 1), a.NT_total - 1);
#pragma unroll
  for (int q2 = 0; q2 < 2; ++q2) cl[q2] = r16 + 16 * (2 * q2 + h);
  const uint32_t msk = oc_opaque(Geo<BITS>::MASK), mag = oc_opaque(dec_magic<false>());

  extern __shared__ __align__(16) uint8_t smem[];

  // x tile loader: wave w, instruction j fills LDS bytes [(16w + j) KB, +1 KB):
  // row 64w + 4j + lane/16, chunk position lane % 16.
  const int rows_here = min(a.M - m0, kGemmBM);
  const int K2 = a.K * 2;
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.x + (size_t)m0 * a.K), 0, rows_here * K2, 0x00020000);
  const int xrow = 64 * wave + (lane >> 4);
  int xcoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xcoff[j] = (r16 ^ ((4 * j + (lane >> 4)) & 15));
  auto load_x = [&](int kb, int buf) {
    const bool tail = (kb + 1) * 128 > a.K;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int c = xcoff[j & 3];
      int off = (xrow + 4 * j) * K2 + kb * 256 + c * 16;
      if (tail && kb * 128 + 8 * c >= a.K) off = 0x7FFFFFF0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (oc_lds_ptr)(smem + buf * kGemmXBuf + (16 * wave + j) * 1024), 16,
                                               off, 0, 0, 0);
    }
  };
  // Packed words and scale/zero words of one k-block: loaded two k-blocks
  // ahead into one of three rotating register sets.  Each set costs exactly
  // GemmLoads<BITS, CS>::n vector-memory instructions (no two of its loads are
  // adjacent in memory, so none are merged), which the vmcnt waits rely on.
  uint32_t w0[2][2][NWB], w1[2][2][NWB], w2[2][2][NWB];
  uint32_t m0w[2][SPK], m1w[2][SPK], m2w[2][SPK];
  auto load_w = [&](int kb, uint32_t (&wb)[2][2][NWB], uint32_t (&mw)[2][SPK]) {
    using GG = Geo<BITS>;
    const int u = kb / GG::U, kbl = kb % GG::U;
#pragma unroll
    for (int T = 0; T < 2; ++T) {
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        const uint8_t* base = a.w + ((size_t)(nt[T] * a.NU + u) * GG::P) * 1024 + cl[q2] * 16;
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
        mw[T][q] = a.meta[(size_t)g * a.N_pad + nt[T] * 16 + r16];
      }
    }
  };
  // A-fragment byte offset of step s inside an x buffer (m-tile i adds 8 KB)
  int xa[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) xa[s] = (lane & 31) * 256 + (((2 * s + h) ^ r16) * 16);

  oc_f16v acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][T][r] = 0.f;

  // B operands of step s (both n32-tiles); dq holds the scale terms of the
  // current group and is refreshed when a new group starts.
  auto make_b = [&](const uint32_t (&wb)[2][2][NWB], const uint32_t (&mw)[2][SPK], int s, oc_u4 (&B)[2],
                    GemmDeq<BF16> (&dq)[2]) {
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      if (s == 0 || (CS == 1 && (s & 1) == 0)) dq[T] = gemm_deq<BF16>(mw[T][(s >> 1) / CS]);
      B[T] = gemm_apply<BF16>(decode_step<BITS, false>(wb[T][s & 1], s >> 1, msk, mag), dq[T]);
    }
  };
  auto mma = [&](const oc_u4 (&A)[8], const oc_u4 (&B)[2]) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int T = 0; T < 2; ++T) acc[i][T] = oc_mfma32<BF16>(A[i], B[T], acc[i][T]);
  };
  // One k-block: 8 steps of 16 k.  The A fragments and B operands of step
  // s + 1 are read / dequantised while the 16 MFMAs of step s run; B of step 0
  // (B0 on entry) was prepared before the barrier that opened this k-block.
  auto compute = [&](int buf, const uint32_t (&wb)[2][2][NWB], const uint32_t (&mw)[2][SPK], oc_u4 (&B0)[2],
                     GemmDeq<BF16> (&dq)[2]) {
    const uint8_t* xb = smem + buf * kGemmXBuf;
    auto read_a = [&](int s, oc_u4 (&A)[8]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) A[i] = *(const oc_u4*)(xb + xa[s] + i * 8192);
    };
    oc_u4 A0[8], A1[8], B1[2];
    read_a(0, A0);
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
      read_a(s + 1, A1);
      make_b(wb, mw, s + 1, B1, dq);
      mma(A0, B0);
      gemm_interleave();
      if (s + 2 < 8) {
        read_a(s + 2, A0);
        make_b(wb, mw, s + 2, B0, dq);
      }
      mma(A1, B1);
      gemm_interleave();
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
  auto body = [&](int kb, const uint32_t (&wc)[2][2][NWB], const uint32_t (&mc)[2][SPK],
                  const uint32_t (&wn)[2][2][NWB], const uint32_t (&mn)[2][SPK], uint32_t (&wf)[2][2][NWB],
                  uint32_t (&mf)[2][SPK]) {
    const int buf = (kb - kb0) & 1;
    load_x(min(kb + 1, last), buf ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(min(kb + 2, last), wf, mf);
    __builtin_amdgcn_sched_barrier(0);
    compute(buf, wc, mc, B0, dq);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NW) : "memory");
    make_b(wn, mn, 0, B0, dq);
    // Plain s_barrier: __syncthreads() adds a workgroup release fence, which
    // waits for every outstanding load (vmcnt(0)) including k-block kb + 2.
    // LDS needs no fence: each wave's own x writes are complete (vmcnt above)
    // and its LDS reads of the buffer refilled next were consumed by MFMAs.
    asm volatile("s_barrier" ::: "memory");
  };

  load_x(kb0, 0);
  load_w(kb0, w0, m0w);
  load_w(min(kb0 + 1, last), w1, m1w);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  make_b(w0, m0w, 0, B0, dq);
  __syncthreads();
  const int nkb = kb1 - kb0, groups = nkb / 3;
  for (int g = 0; g < groups; ++g) {
    body(kb0 + 3 * g, w0, m0w, w1, m1w, w2, m2w);
    body(kb0 + 3 * g + 1, w1, m1w, w2, m2w, w0, m0w);
    body(kb0 + 3 * g + 2, w2, m2w, w0, m0w, w1, m1w);
  }
  if (nkb % 3 >= 1) body(kb0 + 3 * groups, w0, m0w, w1, m1w, w2, m2w);
  if (nkb % 3 == 2) body(kb0 + 3 * groups + 1, w1, m1w, w2, m2w, w0, m0w);
  // the last body prefetched into the idle x buffer: let it land before exit
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if (piece) {
    // fp32 partial tile in register order [wave][i][T][r][lane]: 256-B stores
    float* pp = a.part + (size_t)pidx * (kGemmBM * kGemmBN) + wave * (8 * 2 * 16 * 64) + lane;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int r = 0; r < 16; ++r) pp[((i * 2 + T) * 16 + r) * 64] = acc[i][T][r];
    return;
  }
  // epilogue: register r of tile (i, T) is row 32i + 8(r/4) + 4h + r%4, column n0 + 32T + lane%32
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    const int n = n0 + 32 * T + (lane & 31);
    if (n >= a.N) continue;
    float b = 0.f;
    if (a.bias) b = BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < a.M) a.y[(size_t)m * a.N + n] = BF16 ? oc_f2bf(acc[i][T][r] + b) : oc_f2h(acc[i][T][r] + b);
      }
  }
}

// y for the K-split tiles: the S fp32 partial tiles summed in split order
// (deterministic) plus bias.  One thread per element of a 256 x 256 tile, in
// the partials' register order.
template <bool BF16>
__global__ __launch_bounds__(256) void k_gemm_fixup(const GemmArgs a) {
  const int t = blockIdx.y;  // split tile
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int lane = e & 63, r = (e >> 6) & 15, T = (e >> 10) & 1, i = (e >> 11) & 7, wave = e >> 14;
  int mb, nb;
  gemm_tile(a.tiles_main + t, a.MB, a.NB, mb, nb);
  const int m = mb * kGemmBM + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  const int n = nb * kGemmBN + 64 * wave + 32 * T + (lane & 31);
  if (m >= a.M || n >= a.N) return;
  const float* pp = a.part + (size_t)t * a.S * (kGemmBM * kGemmBN) + e;
  float v = 0.f;
  for (int s = 0; s < a.S; ++s) v += pp[(size_t)s * (kGemmBM * kGemmBN)];
  if (a.bias) v += BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
  a.y[(size_t)m * a.N + n] = BF16 ? oc_f2bf(v) : oc_f2h(v);
}

// x_perm[m, p] = x[m, perm[p]] (act-order activations, 16-bit elements).
__global__ void k_gather(const uint16_t* __restrict__ x, const int32_t* __restrict__ perm, int M, int K,
                         uint16_t* __restrict__ xp) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (p < K) xp[(size_t)m * K + p] = x[(size_t)m * K + perm[p]];
}

// ---------------------------------------------------------------------------
// launch planning
// ---------------------------------------------------------------------------
struct SkinnyPlan {
  int nt, mb, S, ups, ngroups;
};

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

SkinnyPlan plan_skinny(const oc::Layout& L, int M) {
  SkinnyPlan p;
  p.mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.nt = env_int("OC_SKINNY_NT", L.NT >= 512 ? 4 : 2);
  if (p.nt != 2 && p.nt != 4) p.nt = 2;
  p.ngroups = (L.NT + p.nt - 1) / p.nt;
  // enough workgroups to cover 256 CUs about twice, but at least one unit per wave
  int S = env_int("OC_SKINNY_S", 0);
  if (S <= 0) {
    S = 1;
    while (p.ngroups * S < 512 && L.NU / (S * 2) >= 4) S *= 2;
  }
  S = S < 1 ? 1 : (S > L.NU ? L.NU : S);
  p.ups = (L.NU + S - 1) / S;
  p.S = (L.NU + p.ups - 1) / p.ups;
  return p;
}

template <int BITS, bool BF16>
int launch_skinny(const SkinnyPlan& p, const SkinnyArgs& a, hipStream_t st) {
  const dim3 grid(p.ngroups * p.S), block(256);
  const size_t lds = (size_t)4 * p.nt * p.mb * 4 * 64 * sizeof(float);
#define OC_SK(NT_, MB_)                                                              \
  if (p.nt == NT_ && p.mb == MB_) {                                                  \
    hipLaunchKernelGGL((k_skinny<BITS, MB_, NT_, BF16>), grid, block, lds, st, a);   \
    OC_HIP(hipGetLastError());                                                       \
    return 0;                                                                        \
  }
  OC_SK(2, 1) OC_SK(2, 2) OC_SK(2, 4) OC_SK(4, 1) OC_SK(4, 2) OC_SK(4, 4)
#undef OC_SK
  return oc::set_error(OC_ERR_UNSUPPORTED, "no skinny kernel for nt=%d mb=%d", p.nt, p.mb);
}

template <bool BF16>
int dispatch_skinny_bits(int bits, const SkinnyPlan& p, const SkinnyArgs& a, hipStream_t st) {
  switch (bits) {
    case 2: return launch_skinny<2, BF16>(p, a, st);
    case 3: return launch_skinny<3, BF16>(p, a, st);
    case 4: return launch_skinny<4, BF16>(p, a, st);
    case 8: return launch_skinny<8, BF16>(p, a, st);
  }
  return oc::set_error(OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
}

struct GemvPlan {
  int nt, w, cs, S, ups, ngroups, xch, deep;
  size_t lds;
};

constexpr int kGemvMaxM = 16;
constexpr size_t kGemvLds = 96 * 1024;

int log2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

GemvPlan plan_gemv(const oc::Layout& L, int M, int gs) {
  GemvPlan p;
  p.cs = (gs % 128) == 0 ? 4 : 1;
  // x chunks of 16 B per lane per unit: M rows x 16U chunks over 64 lanes
  const int xc = (M * 16 * L.U + 63) / 64;
  p.xch = xc <= 1 ? 1 : (xc <= 4 ? 4 : (xc <= 8 ? 8 : 16));
  // Two n-tiles per workgroup when there are enough column groups left to
  // fill the GPU: fewer, longer waves (measured better on 3-bit gate/up).
  const int nt_env = env_int("OC_GEMV_NT", 0);
  p.nt = (p.xch == 1 && (nt_env == 2 || (nt_env == 0 && (L.NT + 1) / 2 >= 384))) ? 2 : 1;
  p.ngroups = (L.NT + p.nt - 1) / p.nt;
  // One workgroup streams the whole K of its columns; few column groups get
  // more waves per workgroup.  Each wave owns an x slot of M x (128U + 8) halfs.
  int w = env_int("OC_GEMV_W", 0);
  if (w != 4 && w != 8 && w != 16) w = (p.ngroups >= 512 || p.nt == 2) ? 8 : 16;
  if (p.cs == 1 && w == 16) w = 8;
  if (p.xch > 1 && w == 16) w = 8;
  const size_t slot = (size_t)M * (L.U * 128 + 8) * 2;
  while (w > 4 && slot * w > kGemvLds) w /= 2;
  p.w = w;
  p.deep = env_int("OC_GEMV_DEEP", 0);
  int S = env_int("OC_GEMV_S", 1);
  S = S < 1 ? 1 : (S > L.NU ? L.NU : S);
  p.ups = (L.NU + S - 1) / S;
  p.S = (L.NU + p.ups - 1) / p.ups;
  const size_t xb = slot * w;
  const size_t rb = (size_t)p.w * p.nt * 4 * 64 * 4;
  p.lds = ((xb > rb ? xb : rb) + 15) / 16 * 16;
  return p;
}

template <int BITS, bool BF16>
int launch_gemv(const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  constexpr int DB = (BITS == 3 || BITS == 8) ? 2 : 4;
  const dim3 grid(p.ngroups * p.S);
#define OC_GV(NT_, CS_, W_, XC_)                                                                    \
  if (p.nt == NT_ && p.cs == CS_ && p.w == W_ && p.xch == XC_) {                                    \
    constexpr int D_ = (XC_ >= 8 || (CS_ == 1 && BITS == 3)) ? 1 : (DB / NT_ > 0 ? DB / NT_ : 1);                            \
    hipLaunchKernelGGL((k_gemv<BITS, NT_, CS_, D_, W_, XC_, BF16>), grid, dim3(64 * W_), p.lds, st, \
                       a);                                                                          \
    OC_HIP(hipGetLastError());                                                                      \
    return 0;                                                                                       \
  }
#define OC_GVD(NT_, W_)                                                                               \
  if (p.deep && p.nt == NT_ && p.cs == 4 && p.w == W_ && p.xch == 1) {                               \
    constexpr int D_ = 2 * (DB / NT_ > 0 ? DB / NT_ : 1);                                            \
    hipLaunchKernelGGL((k_gemv<BITS, NT_, 4, D_, W_, 1, BF16>), grid, dim3(64 * W_), p.lds, st, a);  \
    OC_HIP(hipGetLastError());                                                                       \
    return 0;                                                                                        \
  }
  OC_GVD(2, 8) OC_GVD(2, 4) OC_GVD(1, 4)
#undef OC_GVD
  OC_GV(1, 4, 16, 1) OC_GV(2, 4, 16, 1)
  OC_GV(1, 4, 8, 1) OC_GV(1, 1, 8, 1) OC_GV(2, 4, 8, 1) OC_GV(2, 1, 8, 1)
  OC_GV(1, 4, 4, 1) OC_GV(1, 1, 4, 1) OC_GV(2, 4, 4, 1) OC_GV(2, 1, 4, 1)
  OC_GV(1, 4, 8, 4) OC_GV(1, 1, 8, 4) OC_GV(1, 4, 4, 4) OC_GV(1, 1, 4, 4)
  OC_GV(1, 4, 8, 8) OC_GV(1, 1, 8, 8) OC_GV(1, 4, 4, 8) OC_GV(1, 1, 4, 8)
  OC_GV(1, 4, 4, 16) OC_GV(1, 1, 4, 16)
#undef OC_GV
  return oc::set_error(OC_ERR_UNSUPPORTED, "no gemv kernel for nt=%d cs=%d w=%d xch=%d", p.nt, p.cs,
                       p.w, p.xch);
}

template <bool BF16>
int dispatch_gemv_bits(int bits, const GemvPlan& p, const GemvArgs& a, hipStream_t st) {
  switch (bits) {
    case 2: return launch_gemv<2, BF16>(p, a, st);
    case 3: return launch_gemv<3, BF16>(p, a, st);
    case 4: return launch_gemv<4, BF16>(p, a, st);
    case 8: return launch_gemv<8, BF16>(p, a, st);
  }
  return oc::set_error(OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
}

int launch_reduce(bool bf16, const float* partial, int S, int M, int N, int N_pad, const void* bias,
                  void* y, hipStream_t st) {
  const dim3 grid((N + 255) / 256, M);
  if (bf16)
    hipLaunchKernelGGL(k_splitk_reduce<true>, grid, dim3(256), 0, st, partial, S, M, N, N_pad,
                       (const uint16_t*)bias, (uint16_t*)y);
  else
    hipLaunchKernelGGL(k_splitk_reduce<false>, grid, dim3(256), 0, st, partial, S, M, N, N_pad,
                       (const uint16_t*)bias, (uint16_t*)y);
  OC_HIP(hipGetLastError());
  return 0;
}

constexpr int kSkinnyMaxM = 64;

// Large-M tiling: whole 256 x 256 tiles, except that a last round of tiles
// that would leave more than half of the CUs idle is cut along K into S
// pieces (at least 4 k-blocks each) whose fp32 partials k_gemm_fixup sums.
struct GemmPlan {
  int MB, NB, NKB, tiles_main, split_tiles, S, kper;
  size_t part_bytes;
};

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cus[dev] = c;
  }
  return cus[dev];
}

GemmPlan plan_gemm(const oc::Layout& L, int M) {
  GemmPlan p;
  p.MB = (M + kGemmBM - 1) / kGemmBM;
  p.NB = (L.N_pad + kGemmBN - 1) / kGemmBN;
  p.NKB = L.K_pad / 128;
  const int T = p.MB * p.NB, C = device_cus();
  const int rem = T % C;
  p.tiles_main = T;
  p.split_tiles = 0;
  p.S = 1;
  p.kper = p.NKB;
  int S = rem > 0 && 2 * rem <= C ? C / rem : 1;
  const int env = env_int("OC_GEMM_SPLIT", 0);
  if (env > 0) S = env;
  if (S > 8) S = 8;
  while (S > 1 && p.NKB / S < 4) --S;
  if (rem > 0 && S > 1) {
    p.kper = (p.NKB + S - 1) / S;
    p.S = (p.NKB + p.kper - 1) / p.kper;
    p.split_tiles = rem;
    p.tiles_main = T - rem;
  }
  p.part_bytes = (size_t)p.split_tiles * p.S * kGemmBM * kGemmBN * 4;
  return p;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

extern "C" size_t oc_gptq_workspace_bytes(int M, int K, int N, int bits, int group_size, int has_perm) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (bits != 2 && bits != 3 && bits != 4 && bits != 8) return 0;
  const oc::Layout L = oc::make_layout(bits, K, N);
  size_t ws = 0;
  if (has_perm) ws += align256((size_t)M * K * 2);
  if (M <= kGemvMaxM) {
    const GemvPlan p = plan_gemv(L, M, oc::eff_group(group_size, K));
    if (p.S > 1) ws += align256((size_t)p.S * M * L.N_pad * 4);
    return ws;
  }
  if (M >= env_int("OC_GEMM_MIN_M", 128)) return ws + align256(plan_gemm(L, M).part_bytes);
  const int Mc = M < kSkinnyMaxM ? M : kSkinnyMaxM;
  const SkinnyPlan p = plan_skinny(L, Mc);
  if (p.S > 1) ws += align256((size_t)p.S * Mc * L.N_pad * 4);
  return ws;
}

extern "C" int oc_gptq_gemm(const void* x, int M, int K, int N, const void* packed, const uint32_t* meta,
                            const int32_t* perm, int bits, int group_size, int act_dtype, const void* bias,
                            void* y, void* workspace, size_t ws_bytes, void* stream) {
  OC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
  OC_REQUIRE(M >= 0 && K > 0 && N > 0, OC_ERR_INVALID, "bad shape M=%d K=%d N=%d", M, K, N);
  OC_REQUIRE(K % 32 == 0, OC_ERR_SHAPE, "K=%d must be a multiple of 32", K);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d", act_dtype);
  OC_REQUIRE(x && packed && meta && y, OC_ERR_INVALID, "null pointer");
  if (M == 0) return 0;
  const int gs = oc::eff_group(group_size, K);
  OC_REQUIRE(gs % 32 == 0, OC_ERR_UNSUPPORTED, "group_size=%d must be a multiple of 32 (or -1)", group_size);
  const int G = (K + gs - 1) / gs;
  hipStream_t st = (hipStream_t)stream;
  const oc::Layout L = oc::make_layout(bits, K, N);
  const size_t need = oc_gptq_workspace_bytes(M, K, N, bits, group_size, perm != nullptr);
  OC_REQUIRE(ws_bytes >= need && (need == 0 || workspace), OC_ERR_WORKSPACE,
             "workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  uint8_t* ws = (uint8_t*)workspace;
  const uint16_t* xa = (const uint16_t*)x;
  if (perm) {
    uint16_t* xp = (uint16_t*)ws;
    hipLaunchKernelGGL(k_gather, dim3((K + 255) / 256, M), dim3(256), 0, st, xa, perm, M, K, xp);
    OC_HIP(hipGetLastError());
    xa = xp;
    ws += align256((size_t)M * K * 2);
  }
  const bool bf16 = act_dtype == OC_DTYPE_BF16;
  if (M <= kGemvMaxM) {
    const GemvPlan p = plan_gemv(L, M, gs);
    GemvArgs a;
    a.x = xa;
    a.w = (const uint8_t*)packed;
    a.meta = meta;
    a.bias = (const uint16_t*)bias;
    a.y = (uint16_t*)y;
    a.partial = (float*)ws;
    a.M = M;
    a.K = K;
    a.N = N;
    a.N_pad = L.N_pad;
    a.NT_total = L.NT;
    a.NU = L.NU;
    a.G = G;
    a.gs = gs;
    a.gshift = log2_exact(gs);
    a.S = p.S;
    a.ups = p.ups;
    const int rc = bf16 ? dispatch_gemv_bits<true>(bits, p, a, st) : dispatch_gemv_bits<false>(bits, p, a, st);
    if (rc || p.S == 1) return rc;
    return launch_reduce(bf16, a.partial, p.S, M, N, L.N_pad, bias, y, st);
  }
  if (M >= env_int("OC_GEMM_MIN_M", 128)) {
    GemmArgs g;
    g.x = xa;
    g.w = (const uint8_t*)packed;
    g.meta = meta;
    g.bias = (const uint16_t*)bias;
    g.y = (uint16_t*)y;
    g.M = M;
    g.K = K;
    g.N = N;
    g.N_pad = L.N_pad;
    g.NT_total = L.NT;
    g.NU = L.NU;
    g.G = G;
    g.gs = gs;
    g.gshift = log2_exact(gs);
    g.NKB = L.K_pad / 128;
    const bool cs4 = (gs % 128) == 0;
    const GemmPlan gp = plan_gemm(L, M);
    g.MB = gp.MB;
    g.NB = gp.NB;
    g.tiles_main = gp.tiles_main;
    g.S = gp.S;
    g.kper = gp.kper;
    g.part = (float*)ws;
    const dim3 grid(gp.tiles_main + gp.split_tiles * gp.S);
    const size_t lds = 2 * kGemmXBuf;
    switch (bits) {
#define OC_GM(B_)                                                                                 \
  case B_:                                                                                        \
    if (bf16) {                                                                                   \
      if (cs4) hipLaunchKernelGGL((k_gemm<B_, 4, true>), grid, dim3(256), lds, st, g);            \
      else hipLaunchKernelGGL((k_gemm<B_, 1, true>), grid, dim3(256), lds, st, g);                \
    } else {                                                                                      \
      if (cs4) hipLaunchKernelGGL((k_gemm<B_, 4, false>), grid, dim3(256), lds, st, g);           \
      else hipLaunchKernelGGL((k_gemm<B_, 1, false>), grid, dim3(256), lds, st, g);               \
    }                                                                                             \
    break;
      OC_GM(2) OC_GM(3) OC_GM(4) OC_GM(8)
#undef OC_GM
    }
    OC_HIP(hipGetLastError());
    if (gp.split_tiles > 0) {
      const dim3 fgrid(kGemmBM * kGemmBN / 256, gp.split_tiles);
      if (bf16) hipLaunchKernelGGL(k_gemm_fixup<true>, fgrid, dim3(256), 0, st, g);
      else hipLaunchKernelGGL(k_gemm_fixup<false>, fgrid, dim3(256), 0, st, g);
      OC_HIP(hipGetLastError());
    }
    return 0;
  }
  // Rows are processed in chunks of at most 64 by the skinny kernel.
  for (int m0 = 0; m0 < M; m0 += kSkinnyMaxM) {
    const int Mc = M - m0 < kSkinnyMaxM ? M - m0 : kSkinnyMaxM;
    const SkinnyPlan p = plan_skinny(L, Mc);
    SkinnyArgs a;
    a.x = xa + (size_t)m0 * K;
    a.w = (const uint8_t*)packed;
    a.meta = meta;
    a.bias = (const uint16_t*)bias;
    a.y = (uint16_t*)y + (size_t)m0 * N;
    a.partial = (float*)ws;
    a.M = Mc;
    a.K = K;
    a.N = N;
    a.N_pad = L.N_pad;
    a.NT_total = L.NT;
    a.NU = L.NU;
    a.G = G;
    a.gs = gs;
    a.S = p.S;
    a.ups = p.ups;
    int rc = bf16 ? dispatch_skinny_bits<true>(bits, p, a, st) : dispatch_skinny_bits<false>(bits, p, a, st);
    if (!rc && p.S > 1) rc = launch_reduce(bf16, a.partial, p.S, Mc, N, L.N_pad, bias, a.y, st);
    if (rc) return rc;
  }
  return 0;
}
