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

#include "gemm_core.h"
#include "gptq_decode.h"
#include "oc_common.h"

namespace {

using namespace oc_gemm;

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

// Tile height of the GEMM for M rows (64 MT rows, 256 columns): see
// gemm_tile_height; only 256-row tiles for groups that are not multiples of 128.
int gemm_mt(int M, int N_pad, int gs) {
  const int e = env_int("OC_GEMM_MT", 0);
  if ((gs % 128) != 0) return 4;
  if (e == 1 || e == 2 || e == 4) return e;
  return gemm_tile_height(M, N_pad);
}

// The tiled GEMM from M = 33 (17 when there are 64 or more column tiles; 128
// for groups that are not multiples of 128, which only have 256-row tiles);
// the skinny kernel below that.  OC_GEMM_MIN_M overrides the threshold.
bool use_gemm(int M, int N_pad, int gs) {
  const int e = env_int("OC_GEMM_MIN_M", 0);
  if (e > 0) return M >= e;
  if ((gs % 128) != 0) return M >= 128;
  return M > 32 || (M > kGemvMaxM && (N_pad + 255) / 256 >= 64);
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
  if (use_gemm(M, L.N_pad, oc::eff_group(group_size, K))) {
    const int mt = gemm_mt(M, L.N_pad, oc::eff_group(group_size, K));
    return ws + align256(plan_gemm(M, L.N_pad, L.K_pad, env_int("OC_GEMM_SPLIT", 0), mt).part_bytes);
  }
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
  if (use_gemm(M, L.N_pad, gs)) {
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
    const int mt = gemm_mt(M, L.N_pad, gs);
    const GemmPlan gp = plan_gemm(M, L.N_pad, L.K_pad, env_int("OC_GEMM_SPLIT", 0), mt);
    g.post = nullptr;
    g.ldx = K;
    g.ldy = N;
    g.uk_shift = 0;
    g.pstride = gp.S;
    g.poff = 0;
    g.MB = gp.MB;
    g.NB = gp.NB;
    g.tiles_main = gp.tiles_main;
    g.S = gp.S;
    g.kper = gp.kper;
    g.part = (float*)ws;
    const dim3 grid(gp.tiles_main + gp.split_tiles * gp.S);
    const size_t lds = 2 * (size_t)(64 * mt) * 256;
    switch (bits) {
#define OC_GM(B_)                                                                                   \
  case B_:                                                                                          \
    if (!cs4) {                                                                                     \
      if (bf16) hipLaunchKernelGGL((k_gemm<B_, 1, true, 4>), grid, dim3(256), lds, st, g);          \
      else hipLaunchKernelGGL((k_gemm<B_, 1, false, 4>), grid, dim3(256), lds, st, g);              \
    } else if (mt == 1) {                                                                           \
      if (bf16) hipLaunchKernelGGL((k_gemm<B_, 4, true, 1>), grid, dim3(256), lds, st, g);          \
      else hipLaunchKernelGGL((k_gemm<B_, 4, false, 1>), grid, dim3(256), lds, st, g);              \
    } else if (mt == 2) {                                                                           \
      if (bf16) hipLaunchKernelGGL((k_gemm<B_, 4, true, 2>), grid, dim3(256), lds, st, g);          \
      else hipLaunchKernelGGL((k_gemm<B_, 4, false, 2>), grid, dim3(256), lds, st, g);              \
    } else {                                                                                        \
      if (bf16) hipLaunchKernelGGL((k_gemm<B_, 4, true, 4>), grid, dim3(256), lds, st, g);          \
      else hipLaunchKernelGGL((k_gemm<B_, 4, false, 4>), grid, dim3(256), lds, st, g);              \
    }                                                                                               \
    break;
      OC_GM(2) OC_GM(3) OC_GM(4) OC_GM(8)
#undef OC_GM
    }
    OC_HIP(hipGetLastError());
    if (gp.split_tiles > 0) {
      const dim3 fgrid(64 * mt * kGemmBN / 256, gp.split_tiles);
#define OC_FX(MT_)                                                                      \
  if (mt == MT_) {                                                                      \
    if (bf16) hipLaunchKernelGGL((k_gemm_fixup<true, MT_>), fgrid, dim3(256), 0, st, g); \
    else hipLaunchKernelGGL((k_gemm_fixup<false, MT_>), fgrid, dim3(256), 0, st, g);     \
  }
      OC_FX(1) OC_FX(2) OC_FX(4)
#undef OC_FX
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
