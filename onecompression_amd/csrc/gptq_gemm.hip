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
#include <stdio.h>
#include <stdlib.h>

#include <mutex>

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
  int ldy;  // row stride of y
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
        a.y[(size_t)m * a.ldy + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
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
  int ldy;   // row stride of y (N, or the fused width for a part of a fused layer)
  int bits;  // the part's bit width (grouped launches pick the decoder by it)
  int out_f32;  // 1: write the fp32 sums (no bias) to partial[m * N_pad + n] instead of y
};

// The accumulation of one workgroup of a GEMV: each wave streams units
// u0 + wave, u0 + wave + W, ... (< u1) of the n-tiles nt[] and sums its share
// of x @ W^T into yacc (lane l: column l % 16 of n-tile j, rows 4 (l / 16) + r).
// rows <= a.M x rows are live; xrow(q, m) is the start of row m, which this
// lane's x chunk q (of XCH) belongs to.  The wave's LDS x slot holds a.M rows.
template <int BITS, int NT, int CS, int D, int W, int XCH, bool BF16, class XRow>
__device__ __forceinline__ void gemv_accum(const GemvArgs& a, const int (&nt)[NT], const int u0, const int u1,
                                           const int rows, XRow xrow, oc_f4 (&yacc)[NT]) {
  using GG = Geo<BITS>;
  constexpr int U = GG::U, P = GG::P;
  constexpr int SPK = 4 / CS;        // correction segments per k-block
  constexpr int MPU = U * SPK;       // scale/zero words per unit and n-tile
  constexpr int XW = U * 128 + 8;    // halfs per staged x row (padded)
  constexpr float OFF = dec_offset<BITS, BF16>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kq = lane >> 4;
  const uint32_t msk = oc_opaque(GG::MASK), mag = oc_opaque(dec_magic<BF16>());
  const uint32_t one16 = BF16 ? 0x3F803F80u : 0x3C003C00u;
  const oc_u4 ones = oc_u4{one16, one16, one16, one16};

  const int n_my = u0 + wave < u1 ? (u1 - u0 - wave + W - 1) / W : 0;

  // x chunk c of a unit (16 B = 8 k): row c / (16U), k offset 8 * (c % (16U))
  auto xchunk_ok = [&](int c) { return c < rows * 16 * U; };

  uint32_t buf[D][NT][4 * P];
  uint32_t mbuf[D][NT][MPU];
  oc_u4 xbuf[D][XCH];
  auto load_unit = [&](int unit, uint32_t (&wb)[NT][4 * P], uint32_t (&mb)[NT][MPU], oc_u4 (&xb)[XCH]) {
#pragma unroll
    for (int q = 0; q < XCH; ++q) {
      const int c = lane + 64 * q;
      const int m = c / (16 * U), k = unit * U * 128 + 8 * (c % (16 * U));
      xb[q] = (xchunk_ok(c) && k < a.K) ? *(const oc_u4*)(xrow(q, m) + k) : oc_u4{0u, 0u, 0u, 0u};
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
  const uint16_t* arow = xslot + min(col, rows - 1) * XW + 8 * kq;

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
}

// One workgroup's share of a GEMV launch: block = column group * S + split.
template <int BITS, int NT, int CS, int D, int W, int XCH, bool BF16>
__device__ __forceinline__ void gemv_tile(const GemvArgs& a, const int block) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ntg = block / a.S, s = block % a.S;
  int nt[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) nt[j] = min(ntg * NT + j, a.NT_total - 1);
  const int u0 = s * a.ups, u1 = min(u0 + a.ups, a.NU);
  oc_f4 yacc[NT];
  gemv_accum<BITS, NT, CS, D, W, XCH, BF16>(a, nt, u0, u1, a.M,
                                            [&](int, int m) { return a.x + (size_t)m * a.K; }, yacc);

  // ---- reduce the W waves ----
  extern __shared__ __align__(16) uint8_t smem[];
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
    if (a.S == 1 && !a.out_f32) {
      if (n < a.N) {
        float o = v;
        if (a.bias) o += BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
        a.y[(size_t)m * a.ldy + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
      }
    } else {
      part[(size_t)m * a.N_pad + n] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// MoE experts at decode sizes.  Pair p = t * topk + j (token t, top-k slot j)
// runs expert ids[p].  The pairs that share an expert are served RM at a
// time: the pairs of expert e, in pair order, are cut into runs of RM, and the
// workgroups of the first pair of each run read e's weights once for all the
// run's rows (the rows of the MFMA A operand); the other pairs' workgroups
// exit.  With RM = 1 every pair is its own run.  RM > 1 needs pairs <= 64
// (one id per lane of a wave).  RM = kMoeSorted: k_moe_sort has put the pairs
// in expert order and cut them into runs of at most 16; workgroup group r
// serves run r of that table (any number of pairs).
// ---------------------------------------------------------------------------
constexpr int kMoeSorted = 0;
constexpr int kMoeMaxE = 2048;  // experts the sort handles (its LDS tables)

__host__ __device__ constexpr int moe_cap(int RM) { return RM == kMoeSorted ? 16 : RM; }

struct MoeArgs {
  GemvArgs base;        // the layer's shape; M = rows per run (x slot rows); w / meta = expert 0
  const int32_t* ids;   // [pairs]
  const int* runs;      // sorted runs: [runs][4] = expert, first index into sorted, rows, 0
  const int* sorted;    // sorted runs: pair indices in expert order
  const int* nruns;     // sorted runs: number of runs
  const uint16_t* bias; // gate|up bias [E, 2I], or null
  uint16_t* out;        // gate|up launch: h [pairs, I]
  float* part;          // down launch: fp32 sums per pair [pairs, N_pad]
  int pairs, topk, E;
  int xdiv;             // gate|up: x row of pair p = p / xdiv (topk: token rows; 1: rows gathered per pair)
  int ntiles;           // workgroups per pair: I / 16 (gate|up) or NT(H) (down)
  int I;                // intermediate size
  int act;
  float alpha, limit;
  size_t w_stride, meta_stride;  // bytes / words between experts
};

struct MoeRun {
  int e;          // expert of the workgroup's pair
  int rows;       // rows this workgroup serves (0: none)
  uint64_t mask;  // pairs of the run and of later runs of e (bit q = pair q), 1 < RM <= 64 only
  int start;      // sorted runs: the run's first index into sorted
};

template <int RM>
__device__ __forceinline__ MoeRun moe_run(const MoeArgs& g, const int p) {
  MoeRun r;
  r.rows = 0;
  r.mask = 0;
  r.start = 0;
  if constexpr (RM == kMoeSorted) {  // p is a run index
    r.e = -1;
    if (p >= __builtin_amdgcn_readfirstlane(*g.nruns)) return r;
    r.e = __builtin_amdgcn_readfirstlane(g.runs[4 * p]);
    r.start = __builtin_amdgcn_readfirstlane(g.runs[4 * p + 1]);
    r.rows = __builtin_amdgcn_readfirstlane(g.runs[4 * p + 2]);
    return r;
  }
  r.e = __builtin_amdgcn_readfirstlane(g.ids[p]);
  if (r.e < 0 || r.e >= g.E) return r;
  if constexpr (RM == 1) {
    r.rows = 1;
  } else {
    const int lane = threadIdx.x & 63;
    const int id = lane < g.pairs ? g.ids[lane] : -1;
    const uint64_t same = __ballot(id == r.e);
    const uint64_t below = same & ((1ull << p) - 1ull);
    if (__popcll(below) % RM) return r;  // a run of an earlier pair covers p
    r.mask = same & ~below;
    r.rows = min(RM, __popcll(r.mask));
  }
  return r;
}

// pair of row m (< rows) of a run
template <int RM>
__device__ __forceinline__ int moe_pair(const MoeArgs& g, const MoeRun& r, const int p, int m) {
  if constexpr (RM == kMoeSorted) {
    return g.sorted[r.start + m];
  } else if constexpr (RM == 1) {
    return p;
  } else {
    uint64_t b = r.mask;
    for (; m > 0; --m) b &= b - 1ull;
    return (int)__builtin_ctzll(b);
  }
}

// per-lane x row offsets (elements) of the lane's XCH chunks: row m = chunk / (16 U)
template <int BITS, int XCH, int RM>
__device__ __forceinline__ void moe_xrows(const MoeArgs& g, const MoeRun& r, const int p, const int div, const int K,
                                          const int rows, int (&xo)[XCH]) {
  constexpr int U = Geo<BITS>::U;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < XCH; ++q) {
    const int m = (lane + 64 * q) / (16 * U);
    xo[q] = m < rows ? (moe_pair<RM>(g, r, p, m) / div) * K : 0;
  }
}

__device__ __forceinline__ float oc_round_act(float v, bool bf16) {
  return bf16 ? oc_bf2f(oc_f2bf(v)) : oc_h2f(oc_f2h(v));
}

// act: 0 = SiLU(gate) * up, 1 = GELU(tanh)(gate) * up, 2 = gpt-oss combine (alpha, limit),
// each step rounded to the activation dtype as the reference's torch ops round
template <bool BF16>
__device__ __forceinline__ float moe_act(float g, float u, int act, float alpha, float limit) {
  if (act == 2) {
    const float gc = oc_round_act(fminf(g, limit), BF16);
    const float uc = oc_round_act(fminf(fmaxf(u, -limit), limit), BF16);
    const float sg = oc_round_act(1.f / (1.f + expf(-oc_round_act(gc * alpha, BF16))), BF16);
    const float glu = oc_round_act(gc * sg, BF16);
    return oc_round_act(oc_round_act(uc + 1.f, BF16) * glu, BF16);
  }
  float a;
  if (act == 0) {
    a = g / (1.f + expf(-g));
  } else {
    const float c = 0.7978845608028654f;  // sqrt(2 / pi)
    a = 0.5f * g * (1.f + tanhf(c * (g + 0.044715f * g * g * g)));
  }
  return oc_round_act(oc_round_act(a, BF16) * u, BF16);
}

// gate|up of the merged layer (H -> 2I: gate columns, then up columns) and the
// activation: workgroup (p, j) computes gate tile j and up tile j (n-tiles j and
// I/16 + j) for its run's rows and writes h[pair, 16 j .. 16 j + 15].
template <int BITS, int CS, int D, int W, int XCH, int RM, bool BF16>
__global__ __launch_bounds__(64 * W) void k_moe_gate_up(const MoeArgs g) {
  const int p = blockIdx.x / g.ntiles, j = blockIdx.x % g.ntiles;
  const MoeRun r = moe_run<RM>(g, p);
  if (r.rows == 0) return;
  GemvArgs a = g.base;
  a.w = g.base.w + (size_t)r.e * g.w_stride;
  a.meta = g.base.meta + (size_t)r.e * g.meta_stride;
  int xo[XCH];
  moe_xrows<BITS, XCH, RM>(g, r, p, g.xdiv, a.K, r.rows, xo);
  const int nt[2] = {j, g.ntiles + j};
  oc_f4 yacc[2];
  gemv_accum<BITS, 2, CS, D, W, XCH, BF16>(a, nt, 0, a.NU, r.rows, [&](int q, int) { return a.x + xo[q]; },
                                           yacc);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  extern __shared__ __align__(16) uint8_t smem[];
  __syncthreads();  // x slots no longer needed: reuse LDS
  float* red = (float*)smem;  // [W][2][4][64]
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) red[((wave * 2 + t) * 4 + rr) * 64 + lane] = yacc[t][rr];
  __syncthreads();
  for (int el = threadIdx.x; el < 256; el += 64 * W) {
    const int ln = el & 63, m = 4 * (ln >> 4) + (el >> 6);
    if (m >= r.rows) continue;
    float gv = 0.f, uv = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) {
      gv += red[(ww * 2) * 256 + el];
      uv += red[(ww * 2 + 1) * 256 + el];
    }
    const int i = 16 * j + (ln & 15);
    if (g.bias) {
      const uint16_t* b = g.bias + (size_t)r.e * 2 * g.I;
      gv += BF16 ? oc_bf2f(b[i]) : oc_h2f(b[i]);
      uv += BF16 ? oc_bf2f(b[g.I + i]) : oc_h2f(b[g.I + i]);
    }
    const float h = moe_act<BF16>(oc_round_act(gv, BF16), oc_round_act(uv, BF16), g.act, g.alpha, g.limit);
    g.out[(size_t)moe_pair<RM>(g, r, p, m) * g.I + i] = BF16 ? oc_f2bf(h) : oc_f2h(h);
  }
}

// down (I -> H) per run: the fp32 sums of the run's rows go to part[pair].
template <int BITS, int CS, int D, int W, int XCH, int RM, bool BF16>
__global__ __launch_bounds__(64 * W) void k_moe_down(const MoeArgs g) {
  const int p = blockIdx.x / g.ntiles, j = blockIdx.x % g.ntiles;
  const int lane = threadIdx.x & 63;
  const MoeRun r = moe_run<RM>(g, p);
  if (r.rows == 0) return;
  GemvArgs a = g.base;
  a.w = g.base.w + (size_t)r.e * g.w_stride;
  a.meta = g.base.meta + (size_t)r.e * g.meta_stride;
  int xo[XCH];
  moe_xrows<BITS, XCH, RM>(g, r, p, 1, a.K, r.rows, xo);
  const int nt[1] = {j};
  oc_f4 yacc[1];
  gemv_accum<BITS, 1, CS, D, W, XCH, BF16>(a, nt, 0, a.NU, r.rows, [&](int q, int) { return a.x + xo[q]; },
                                           yacc);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  extern __shared__ __align__(16) uint8_t smem[];
  __syncthreads();
  float* red = (float*)smem;  // [W][4][64]
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) red[(wave * 4 + rr) * 64 + lane] = yacc[0][rr];
  __syncthreads();
  for (int el = threadIdx.x; el < 256; el += 64 * W) {
    const int ln = el & 63, m = 4 * (ln >> 4) + (el >> 6);
    if (m >= r.rows) continue;
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) v += red[ww * 256 + el];
    g.part[(size_t)moe_pair<RM>(g, r, p, m) * a.N_pad + 16 * j + (ln & 15)] = v;
  }
}

// The pairs of each expert in expert order (atomic order within an expert: the
// rows of an MFMA do not mix, so the outputs do not depend on it), cut into
// runs of at most rs: runs[r] = {expert, first index into sorted, rows, 0};
// counts = {runs, valid pairs}; pos[p] = the index of pair p in sorted (when
// pos is not null).  One workgroup; E <= kMoeMaxE.
__global__ __launch_bounds__(1024) void k_moe_sort(const int32_t* __restrict__ ids, int pairs, int E, int rs,
                                                   int* __restrict__ sorted, int* __restrict__ pos,
                                                   int* __restrict__ runs, int* __restrict__ counts) {
  __shared__ int cnt[kMoeMaxE], off[kMoeMaxE], roff[kMoeMaxE];
  __shared__ int part[2][1024];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < pairs; p += 1024) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scans of the pair counts and run counts: per-thread chunks of experts, then a
  // scan over the 1024 chunk sums
  const int per = (E + 1023) / 1024, e0 = min(E, tid * per), e1 = min(E, e0 + per);
  int s1 = 0, s2 = 0;
  for (int e = e0; e < e1; ++e) {
    s1 += cnt[e];
    s2 += (cnt[e] + rs - 1) / rs;
  }
  part[0][tid] = s1;
  part[1][tid] = s2;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int a1 = tid >= o ? part[0][tid - o] : 0, a2 = tid >= o ? part[1][tid - o] : 0;
    __syncthreads();
    part[0][tid] += a1;
    part[1][tid] += a2;
    __syncthreads();
  }
  int b1 = part[0][tid] - s1, b2 = part[1][tid] - s2;
  for (int e = e0; e < e1; ++e) {
    off[e] = b1;
    roff[e] = b2;
    b1 += cnt[e];
    b2 += (cnt[e] + rs - 1) / rs;
  }
  if (tid == 1023) {
    counts[0] = part[1][1023];
    counts[1] = part[0][1023];
  }
  __syncthreads();
  for (int e = tid; e < E; e += 1024) {
    const int c = cnt[e];
    for (int i = 0; rs * i < c; ++i) {
      int* run = runs + 4 * (roff[e] + i);
      run[0] = e;
      run[1] = off[e] + rs * i;
      run[2] = min(rs, c - rs * i);
      run[3] = 0;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;  // now the fill cursor of each expert
  __syncthreads();
  for (int p = tid; p < pairs; p += 1024) {
    const int e = ids[p];
    if (e >= 0 && e < E) {
      const int i = off[e] + atomicAdd(&cnt[e], 1);
      sorted[i] = p;
      if (pos) pos[p] = i;
    }
  }
}

// Prefill path (rows sorted by expert, large-M GEMM per run of rows): x rows in sorted order.
__global__ __launch_bounds__(256) void k_moe_gather_x(const uint16_t* __restrict__ x, int H, int topk,
                                                      const int* __restrict__ sorted,
                                                      const int* __restrict__ counts, uint16_t* __restrict__ xs) {
  const int i = blockIdx.x;
  if (i >= counts[1]) return;
  const uint16_t* src = x + (size_t)(sorted[i] / topk) * H;
  for (int c = threadIdx.x; c < H / 8; c += 256)
    *(oc_u4*)(xs + (size_t)i * H + 8 * c) = *(const oc_u4*)(src + 8 * c);
}

// Act-order experts (weights stored in each expert's sorted-k order): dst[p, k] =
// src[(p / div) K + perm[e K + k]] with e = ids[p], zero for pairs without an expert.
__global__ __launch_bounds__(256) void k_moe_gather_perm(const uint16_t* __restrict__ src, int div, int K,
                                                         const int32_t* __restrict__ perm,
                                                         const int32_t* __restrict__ ids, int E,
                                                         uint16_t* __restrict__ dst) {
  const int p = blockIdx.y, k = blockIdx.x * 256 + threadIdx.x;
  if (k >= K) return;
  const int e = ids[p];
  uint16_t v = 0;
  if (e >= 0 && e < E) v = src[(size_t)(p / div) * K + perm[(size_t)e * K + k]];
  dst[(size_t)p * K + k] = v;
}

// Prefill path: h = act(gate, up) for the sorted rows (gate|up rounded, bias included).
template <bool BF16>
__global__ void k_moe_act_sorted(const uint16_t* __restrict__ h13, int I, const int* __restrict__ counts, int act,
                                 float alpha, float limit, uint16_t* __restrict__ h) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  const int i = blockIdx.y;
  if (j >= I || i >= counts[1]) return;
  const uint16_t* r = h13 + (size_t)i * 2 * I;
  const float g = BF16 ? oc_bf2f(r[j]) : oc_h2f(r[j]);
  const float u = BF16 ? oc_bf2f(r[I + j]) : oc_h2f(r[I + j]);
  const float v = moe_act<BF16>(g, u, act, alpha, limit);
  h[(size_t)i * I + j] = BF16 ? oc_f2bf(v) : oc_f2h(v);
}

// Prefill path: y[t] = sum over t's valid slots, in slot order, of w[p] * ys[pos[p]] (the
// down outputs, rounded with their bias); zero for a token with no valid slot.
template <bool BF16>
__global__ void k_moe_combine_sorted(const uint16_t* __restrict__ ys, int H, int topk, int M,
                                     const int32_t* __restrict__ ids, int E, const float* __restrict__ w,
                                     const int* __restrict__ pos, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (n >= H || t >= M) return;
  float acc = 0.f;
  for (int s = 0; s < topk; ++s) {
    const int p = t * topk + s, e = ids[p];
    if (e < 0 || e >= E) continue;
    const uint16_t v = ys[(size_t)pos[p] * H + n];
    acc = fmaf(w[p], BF16 ? oc_bf2f(v) : oc_h2f(v), acc);
  }
  y[(size_t)t * H + n] = BF16 ? oc_f2bf(acc) : oc_f2h(acc);
}

// y[t] = sum over t's valid slots, in slot order, of w[p] * (part[p] + b2_e); zero for a token
// with no valid slot.  The ids, then the sums, weights and biases of 8 slots at a time are
// loaded before any is used (two dependent round trips per 8 slots, not two per slot).
template <bool BF16>
__global__ void k_moe_combine(const float* __restrict__ part, int H, int H_pad, int topk, int M,
                              const int32_t* __restrict__ ids, int E, const float* __restrict__ w,
                              const uint16_t* __restrict__ b2, uint16_t* __restrict__ y) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int t = blockIdx.y;
  if (n >= H || t >= M) return;
  float acc = 0.f;
  for (int j0 = 0; j0 < topk; j0 += 8) {
    int e[8], pp[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      pp[jj] = t * topk + min(j0 + jj, topk - 1);
      e[jj] = ids[pp[jj]];
    }
    float v[8], wt[8], bv[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const bool ok = j0 + jj < topk && e[jj] >= 0 && e[jj] < E;
      e[jj] = ok ? e[jj] : -1;
      v[jj] = part[(size_t)pp[jj] * H_pad + n];
      wt[jj] = w[pp[jj]];
      const uint16_t bb = b2 ? b2[(size_t)(ok ? e[jj] : 0) * H + n] : (uint16_t)0;
      bv[jj] = BF16 ? oc_bf2f(bb) : oc_h2f(bb);
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      if (e[jj] >= 0) acc = fmaf(wt[jj], v[jj] + bv[jj], acc);
  }
  y[(size_t)t * H + n] = BF16 ? oc_f2bf(acc) : oc_f2h(acc);
}

template <int BITS, int NT, int CS, int D, int W, int XCH, bool BF16>
__global__ __launch_bounds__(64 * W) void k_gemv(const GemvArgs a) {
  gemv_tile<BITS, NT, CS, D, W, XCH, BF16>(a, blockIdx.x);
}

// Units in flight per wave for BITS and NT n-tiles per workgroup.
template <int BITS, int NT, int XCH>
struct GemvDepth {
  static constexpr int DB = (BITS == 3 || BITS == 8) ? 2 : 4;
  static constexpr int D = XCH >= 8 ? 1 : (DB / NT > 0 ? DB / NT : 1);
};

// Several layers that read the same activations (the parts of a fused
// module, which may differ in bit width) in one launch: workgroup b belongs
// to part p for block_start[p] <= b < block_start[p + 1] and runs that part's
// decoder (a uniform branch on its bit width) over part_nt[p] n-tiles (2 for a
// part whose n-tiles are at most half the bytes of the widest part's, so the
// workgroups carry about the same bytes; NTMAX = 2 enables it).
constexpr int kMaxParts = 4;
struct GemvGroupArgs {
  GemvArgs part[kMaxParts];
  int block_start[kMaxParts + 1];
  int part_nt[kMaxParts];
  int n_parts;
};

template <int NT, int W, int XCH, bool BF16>
__device__ __forceinline__ void gemv_group_part(const GemvArgs& a, const int b) {
  switch (a.bits) {
    case 2: gemv_tile<2, NT, 4, GemvDepth<2, NT, XCH>::D, W, XCH, BF16>(a, b); break;
    case 3: gemv_tile<3, NT, 4, GemvDepth<3, NT, XCH>::D, W, XCH, BF16>(a, b); break;
    case 4: gemv_tile<4, NT, 4, GemvDepth<4, NT, XCH>::D, W, XCH, BF16>(a, b); break;
    default: gemv_tile<8, NT, 4, GemvDepth<8, NT, XCH>::D, W, XCH, BF16>(a, b); break;
  }
}

template <int NTMAX, int W, int XCH, bool BF16>
__global__ __launch_bounds__(64 * W) void k_gemv_group(const GemvGroupArgs g) {
  int p = 0;
#pragma unroll
  for (int q = 1; q < kMaxParts; ++q)
    if (q < g.n_parts && (int)blockIdx.x >= g.block_start[q]) p = q;
  const GemvArgs& a = g.part[p];
  const int b = blockIdx.x - g.block_start[p];
  if constexpr (NTMAX == 2) {
    if (g.part_nt[p] == 2) {
      gemv_group_part<2, W, XCH, BF16>(a, b);
      return;
    }
  }
  gemv_group_part<1, W, XCH, BF16>(a, b);
}

// ---------------------------------------------------------------------------
// Wide layers at small M (thousands of n-tiles, e.g. a fused gate|up): one
// wave per n-tile streams the whole K of its 16 columns through a ring of D
// units, so memory and the decode overlap for the wave's whole life and no
// cross-wave reduction is needed.  The workgroup (4 waves, 4 consecutive
// n-tiles) stages all M x K of x in LDS once, together with the sums of x over
// each k-block that the zero-point correction needs (so no MFMA is spent on
// them).  Every wave runs the same number of units (NU, a multiple of D), so
// the loads are unconditional and the compiler's vmcnt waits are exact:
// prologue (D units), steady state (consume a slot, refill it D units ahead),
// drain (the last D units).  Groups are a power of two >= 128 (one
// scale/zero word per k-block).  MR = the output rows 4 kq + r (r < MR) a
// lane accumulates (MR = 1 for M = 1).
// ---------------------------------------------------------------------------
struct StreamArgs {
  const uint16_t* x;
  const uint8_t* w;
  const uint32_t* meta;
  const uint16_t* bias;
  uint16_t* y;
  int M, K, K_pad, N, N_pad, NT_total, NU, G, gs, gkb_shift, ldy;
  int tpw;  // k_gemv_stream_bal: n-tiles per workgroup
  // k_gemm_stream: split blockIdx.y takes units [y NU / S, (y + 1) NU / S) and, with S > 1,
  // writes fp32 partial[((y M + m) N_pad + n)] for k_splitk_reduce
  int S;
  float* partial;
};

template <int BITS, int D, int MR, int KS, bool BF16>
__global__ __launch_bounds__(256, 4) void k_gemv_stream(const StreamArgs a) {
  using GG = Geo<BITS>;
  constexpr int U = GG::U, P = GG::P;
  constexpr float OFF = dec_offset<BITS, BF16>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kq = lane >> 4;
  const uint32_t msk = oc_opaque(GG::MASK), mag = oc_opaque(dec_magic<BF16>());
  // KS waves share an n-tile, each taking NU / KS consecutive units
  const int nt = blockIdx.x * (4 / KS) + wave / KS, ks = wave % KS;
  const int nu = a.NU / KS, ub = ks * nu;
  const int M = a.M;

  // LDS: x rows [M][K_pad + 8] (zero past K), then group sums [G][16] fp32
  extern __shared__ __align__(16) uint16_t xl[];
  const int XL = a.K_pad + 8;  // halfs per LDS row
  float* xsum = (float*)(xl + (size_t)M * XL);
  const int cpr = a.K_pad / 8;
  for (int c = threadIdx.x; c < M * cpr; c += 256) {
    const int m = c / cpr, k = 8 * (c % cpr);
    oc_u4 v = oc_u4{0u, 0u, 0u, 0u};
    if (k < a.K) v = *(const oc_u4*)(a.x + (size_t)m * a.K + k);
    *(oc_u4*)(xl + m * XL + k) = v;
  }
  const bool has_bias = a.bias != nullptr;
  const uint16_t braw = __builtin_amdgcn_raw_buffer_load_b16(
      oc_rsrc(a.bias, (uint32_t)a.N * 2), has_bias && nt * 16 + col < a.N ? (uint32_t)(nt * 16 + col) * 2 : kOcOob,
      0, 0);
  __syncthreads();
  // sum of x over each k-block of 128 for rows < M (fp32): 16 lanes per sum,
  // 8 values each, then a 16-lane butterfly.  Entries of rows >= M stay
  // unset: they only reach accumulators of rows that are never stored.
  const int nkb = a.K_pad / 128;
  for (int c = threadIdx.x; c < M * nkb * 16; c += 256) {
    const int e = c >> 4, kb = e % nkb, m = e / nkb;
    const oc_u4 v = *(const oc_u4*)(xl + m * XL + kb * 128 + 8 * (c & 15));
    float sum = 0.f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const uint32_t pr = v[h];
      sum += (BF16 ? oc_bf2f((uint16_t)(pr & 0xFFFFu)) : oc_h2f((uint16_t)(pr & 0xFFFFu))) +
             (BF16 ? oc_bf2f((uint16_t)(pr >> 16)) : oc_h2f((uint16_t)(pr >> 16)));
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 16);
    if ((c & 15) == 0) xsum[kb * 16 + m] = sum;
  }
  __syncthreads();
  if (KS == 1 && nt >= a.NT_total) return;  // a whole wave past the last n-tile (no barrier follows)

  const int ntc = min(nt, a.NT_total - 1);  // KS > 1: waves past the last n-tile recompute it, unused
  const __amdgpu_buffer_rsrc_t wr = oc_rsrc(a.w + (size_t)ntc * a.NU * P * 1024, (uint32_t)a.NU * P * 1024);
  const __amdgpu_buffer_rsrc_t mr = oc_rsrc(a.meta, (uint32_t)a.G * a.N_pad * 4);
  const uint16_t* arow = xl + min(col, M - 1) * XL + 8 * kq;
  const float* srow = xsum + 4 * kq;
  const uint32_t mcol = (uint32_t)(ntc * 16 + col) * 4;
  uint32_t wb[D][4 * P];
  uint32_t mb[D][U];
  auto load = [&](int u, uint32_t (&w)[4 * P], uint32_t (&m)[U]) {
#pragma unroll
    for (int pt = 0; pt < P; ++pt) {
      const oc_u4 v = oc_bload16_nt(wr, (uint32_t)(u * P + pt) * 1024 + lane * 16);
      w[4 * pt] = v[0];
      w[4 * pt + 1] = v[1];
      w[4 * pt + 2] = v[2];
      w[4 * pt + 3] = v[3];
    }
#pragma unroll
    for (int kbl = 0; kbl < U; ++kbl) {
      const int g = (u * U + kbl) >> a.gkb_shift;
      m[kbl] = __builtin_amdgcn_raw_buffer_load_b32(mr, mcol + (uint32_t)(g * a.N_pad) * 4, 0, 0);
    }
  };
  oc_f4 yacc = oc_f4{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](int u, const uint32_t (&w)[4 * P], const uint32_t (&m)[U]) {
#pragma unroll
    for (int kbl = 0; kbl < U; ++kbl) {
      const int kb = u * U + kbl;
      oc_u4 av[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) av[t] = *(const oc_u4*)(arow + kb * 128 + 32 * t);
      oc_u4 bq[4];
      decode_kblock<BITS, BF16>(w, kbl, bq, msk, mag);
      oc_f4 acc = oc_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = oc_mfma16<BF16>(av[t], bq[t], acc);
      const uint32_t md = m[kbl];
      const float sc = oc_h2f((uint16_t)(md & 0xFFFFu));
      const float oz = OFF + (float)(md >> 16);
      const float* sg = srow + kb * 16;
      if constexpr (MR == 1) {
        yacc[0] = fmaf(sc, fmaf(-oz, sg[0], acc[0]), yacc[0]);
      } else {
        const oc_f4 xs = *(const oc_f4*)sg;
#pragma unroll
        for (int r = 0; r < MR; ++r) yacc[r] = fmaf(sc, fmaf(-oz, xs[r], acc[r]), yacc[r]);
      }
    }
  };
  // prologue, steady state, drain (NU / KS is a multiple of D and at least D)
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(ub + d, wb[d], mb[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int i0 = 0; i0 < nu - D; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(ub + i0 + d, wb[d], mb[d]);
      load(ub + i0 + D + d, wb[d], mb[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) consume(ub + nu - D + d, wb[d], mb[d]);
  if constexpr (KS > 1) {
    // the KS partial sums of an n-tile meet in LDS (reusing the x rows)
    __syncthreads();
    float* red = (float*)xl;  // [4 waves][MR][64]
#pragma unroll
    for (int r = 0; r < MR; ++r) red[(wave * MR + r) * 64 + lane] = yacc[r];
    __syncthreads();
    if (ks != 0 || nt >= a.NT_total) return;
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int q = 1; q < KS; ++q) yacc[r] += red[((wave + q) * MR + r) * 64 + lane];
  }

  const int n = nt * 16 + col;
  if (n < a.N) {
    const float b = has_bias ? (BF16 ? oc_bf2f(braw) : oc_h2f(braw)) : 0.f;
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const int m = 4 * kq + r;
      if (m < M) a.y[(size_t)m * a.ldy + n] = BF16 ? oc_f2bf(yacc[r] + b) : oc_f2h(yacc[r] + b);
    }
  }
}

// Wide layers whose n-tile count is not a multiple of 4 x CUs, where
// k_gemv_stream would leave some CUs with twice the n-tiles of others (1792
// n-tiles on 256 CUs: 192 CUs run 8 waves, 64 run 4): each workgroup of 8
// waves owns T consecutive n-tiles (one workgroup per CU for T = ceil(n-tiles
// / CUs)) and splits their T x NU units evenly over its waves, so a wave's
// range may start or end inside an n-tile.  A range is at most NU units long
// (T <= 8), so a wave touches at most two n-tiles and keeps one partial sum for
// each; the partials of an n-tile meet in LDS and are added in wave order.  A
// wave's unit count is rounded up to a multiple of D with loads of its last
// unit again (no consume), so every load stays unconditional.
// ---------------------------------------------------------------------------
constexpr int kStreamBalWaves = 8;

template <int BITS, int D, int MR, bool BF16>
__global__ __launch_bounds__(64 * kStreamBalWaves) void k_gemv_stream_bal(const StreamArgs a) {
  using GG = Geo<BITS>;
  constexpr int U = GG::U, P = GG::P, WV = kStreamBalWaves;
  constexpr float OFF = dec_offset<BITS, BF16>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kq = lane >> 4;
  const uint32_t msk = oc_opaque(GG::MASK), mag = oc_opaque(dec_magic<BF16>());
  const int M = a.M, NU = a.NU, T = a.tpw;
  const int t0 = blockIdx.x * T;  // first n-tile of the workgroup
  const int total = T * NU;       // units of the workgroup's n-tiles
  const int ws = wave * total / WV, we = (wave + 1) * total / WV;
  const int npad = ((total + WV - 1) / WV + D - 1) / D * D;  // units per wave, incl. repeats

  // LDS: x rows [M][K_pad + 8] (zero past K), group sums [G][16] fp32, then
  // the partial sums [8 waves][2][MR][64] fp32
  extern __shared__ __align__(16) uint16_t xl[];
  const int XL = a.K_pad + 8;
  float* xsum = (float*)(xl + (size_t)M * XL);
  const int nkb = a.K_pad / 128;
  float* red = xsum + nkb * 16;
  // the workgroup's n-tiles are contiguous in the packed weights
  const int tiles = min(T, a.NT_total - t0);
  const __amdgpu_buffer_rsrc_t wr = oc_rsrc(a.w + (size_t)t0 * NU * P * 1024, (uint32_t)tiles * NU * P * 1024);
  const __amdgpu_buffer_rsrc_t mr = oc_rsrc(a.meta, (uint32_t)a.G * a.N_pad * 4);
  const uint16_t* arow = xl + min(col, M - 1) * XL + 8 * kq;
  const float* srow = xsum + 4 * kq;
  const int first = ws / NU;  // the wave's first n-tile (workgroup-local)
  uint32_t wb[D][4 * P];
  uint32_t mb[D][U];
  auto load = [&](int f, uint32_t (&w)[4 * P], uint32_t (&m)[U]) {
    f = min(f, we - 1);
    const int tl = f / NU, uk = f - tl * NU;
#pragma unroll
    for (int pt = 0; pt < P; ++pt) {
      const oc_u4 v = oc_bload16_nt(wr, (uint32_t)(f * P + pt) * 1024 + lane * 16);
      w[4 * pt] = v[0];
      w[4 * pt + 1] = v[1];
      w[4 * pt + 2] = v[2];
      w[4 * pt + 3] = v[3];
    }
    const uint32_t mcol = (uint32_t)(min(t0 + tl, a.NT_total - 1) * 16 + col) * 4;
#pragma unroll
    for (int kbl = 0; kbl < U; ++kbl) {
      const int g = (uk * U + kbl) >> a.gkb_shift;
      m[kbl] = __builtin_amdgcn_raw_buffer_load_b32(mr, mcol + (uint32_t)(g * a.N_pad) * 4, 0, 0);
    }
  };
  const int cpr = a.K_pad / 8;
  for (int c = threadIdx.x; c < M * cpr; c += 64 * WV) {
    const int m = c / cpr, k = 8 * (c % cpr);
    oc_u4 v = oc_u4{0u, 0u, 0u, 0u};
    if (k < a.K) v = *(const oc_u4*)(a.x + (size_t)m * a.K + k);
    *(oc_u4*)(xl + m * XL + k) = v;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < M * nkb * 16; c += 64 * WV) {
    const int e = c >> 4, kb = e % nkb, m = e / nkb;
    const oc_u4 v = *(const oc_u4*)(xl + m * XL + kb * 128 + 8 * (c & 15));
    float sum = 0.f;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const uint32_t pr = v[h];
      sum += (BF16 ? oc_bf2f((uint16_t)(pr & 0xFFFFu)) : oc_h2f((uint16_t)(pr & 0xFFFFu))) +
             (BF16 ? oc_bf2f((uint16_t)(pr >> 16)) : oc_h2f((uint16_t)(pr >> 16)));
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 16);
    if ((c & 15) == 0) xsum[kb * 16 + m] = sum;
  }
  __syncthreads();

  oc_f4 yacc = oc_f4{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](int f, const uint32_t (&w)[4 * P], const uint32_t (&m)[U]) {
    if (f >= we) return;  // a repeat load past the wave's range
    const int tl = f / NU, uk = f - tl * NU;
#pragma unroll
    for (int kbl = 0; kbl < U; ++kbl) {
      const int kb = uk * U + kbl;
      oc_u4 av[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) av[t] = *(const oc_u4*)(arow + kb * 128 + 32 * t);
      oc_u4 bq[4];
      decode_kblock<BITS, BF16>(w, kbl, bq, msk, mag);
      oc_f4 acc = oc_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = oc_mfma16<BF16>(av[t], bq[t], acc);
      const uint32_t md = m[kbl];
      const float sc = oc_h2f((uint16_t)(md & 0xFFFFu));
      const float oz = OFF + (float)(md >> 16);
      const float* sg = srow + kb * 16;
      if constexpr (MR == 1) {
        yacc[0] = fmaf(sc, fmaf(-oz, sg[0], acc[0]), yacc[0]);
      } else {
        const oc_f4 xs = *(const oc_f4*)sg;
#pragma unroll
        for (int r = 0; r < MR; ++r) yacc[r] = fmaf(sc, fmaf(-oz, xs[r], acc[r]), yacc[r]);
      }
    }
    if (uk == NU - 1 || f == we - 1) {  // the wave leaves this n-tile: park its partial sum
      const int slot = tl - first;
#pragma unroll
      for (int r = 0; r < MR; ++r) red[((wave * 2 + slot) * MR + r) * 64 + lane] = yacc[r];
      yacc = oc_f4{0.f, 0.f, 0.f, 0.f};
    }
  };
  if (we > ws) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      load(ws + d, wb[d], mb[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int i0 = 0; i0 < npad - D; i0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        consume(ws + i0 + d, wb[d], mb[d]);
        load(ws + i0 + D + d, wb[d], mb[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) consume(ws + npad - D + d, wb[d], mb[d]);
  }
  __syncthreads();
  // wave w < tiles finishes n-tile t0 + w: the partials of every wave whose
  // range meets the n-tile's units [w NU, (w + 1) NU), in wave order
  if (wave >= tiles) return;
  oc_f4 y = oc_f4{0.f, 0.f, 0.f, 0.f};
  for (int v = 0; v < WV; ++v) {
    const int vs = v * total / WV, ve = (v + 1) * total / WV;
    if (vs >= ve || vs >= (wave + 1) * NU || ve <= wave * NU) continue;
    const int slot = wave - vs / NU;
#pragma unroll
    for (int r = 0; r < MR; ++r) y[r] += red[((v * 2 + slot) * MR + r) * 64 + lane];
  }
  const int n = (t0 + wave) * 16 + col;
  if (n < a.N) {
    float b = 0.f;
    if (a.bias != nullptr) b = BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const int m = 4 * kq + r;
      if (m < M) a.y[(size_t)m * a.ldy + n] = BF16 ? oc_f2bf(y[r] + b) : oc_f2h(y[r] + b);
    }
  }
}

// ---------------------------------------------------------------------------
// Mid M (up to 128 rows): one wave per n-tile streams its split of K, with x
// staged one k-block (128 k) at a time in a two-buffer LDS ring shared by the
// workgroup's 4 waves, one barrier per k-block.  Each decoded B operand feeds
// MB = ceil(M / 16) MFMAs (the 16-row blocks of x).  The staging loads of
// k-block kb + 2 are issued while kb is computed.
// MB <= 2: codes decode to (off + q) and the zero point and scale are applied
// to the sums, y += s (sum x (off + q) - (off + z) sum x), with the rows' sums
// over each k-block formed from the staged registers (16-lane butterfly).
// MB >= 4: that correction would cost more than the weights it saves, so the
// B operand is the dequantised weight RNE(s (q - z)) itself (the large-M
// GEMM's arithmetic, bit for bit) and no sums are formed.
// The k-block barrier waits for LDS traffic only: __syncthreads() also waits
// for every outstanding global load, i.e. for the x and weight prefetches,
// which would expose a memory round trip per k-block.
// ---------------------------------------------------------------------------
template <int BITS, int MB, bool BF16, int NTW = 1>
__global__ __launch_bounds__(256, 2) void k_gemm_stream(const StreamArgs a) {
  static_assert(NTW == 1 || MB > 2, "two n-tiles per wave on the dequantised-B path only");
  using GG = Geo<BITS>;
  constexpr int U = GG::U, P = GG::P;
  constexpr int D = 2;        // units in flight per wave
  constexpr int XLD = 136;    // halfs per staged row (128 + 8 pad)
  constexpr int ROWS = 16 * MB;
  constexpr bool SUMS = MB <= 2;  // zero-point correction on the sums (else dequantised B)
  constexpr float OFF = dec_offset<BITS, BF16>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kq = lane >> 4;
  const uint32_t msk = oc_opaque(GG::MASK), mag = oc_opaque(dec_magic<SUMS && BF16>());
  // the wave's NTW n-tiles (NTW = 2: every A fragment read from LDS feeds two MFMAs, and
  // a workgroup's x staging serves 32 NTW columns per wave)
  const int nt0 = (blockIdx.x * 4 + wave) * NTW;
  int ntc[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) ntc[j] = min(nt0 + j, a.NT_total - 1);  // past the last n-tile: computed, unused
  // rows of this workgroup: blockIdx.z's block of 16 MB rows (one block unless the rows are split
  // across workgroups as well)
  const int m0 = blockIdx.z * 16 * MB;
  const int M = min(a.M - m0, 16 * MB);
  // this split's units (a multiple of D: the planner keeps NU / S even)
  const int split = blockIdx.y;
  const int nu = a.NU / a.S, ub = split * nu;

  extern __shared__ __align__(16) uint16_t xl[];   // [2][ROWS][XLD]
  float* xsum = (float*)(xl + 2 * ROWS * XLD);     // [2][ROWS] (SUMS only)

  // staging of k-block kb: thread t owns chunks c = t + 256 j (row c / 16, 8 k at 8 (c % 16))
  const __amdgpu_buffer_rsrc_t xr = oc_rsrc(a.x + (size_t)m0 * a.K, (uint32_t)M * a.K * 2);
  oc_u4 xs_reg[MB];
  auto stage_load = [&](int kb) {
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int c = threadIdx.x + 256 * j, row = c >> 4, k = kb * 128 + 8 * (c & 15);
      // (& not &&: a short-circuit here can become branches around duplicated loads)
      xs_reg[j] = oc_bload16(xr, ((row < M) & (k < a.K)) ? (uint32_t)(row * a.K + k) * 2 : kOcOob);
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int c = threadIdx.x + 256 * j, row = c >> 4;
      *(oc_u4*)(xl + (buf * ROWS + row) * XLD + 8 * (c & 15)) = xs_reg[j];
      if constexpr (SUMS) {
        float sum = 0.f;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t pr = xs_reg[j][h];
          sum += (BF16 ? oc_bf2f((uint16_t)(pr & 0xFFFFu)) : oc_h2f((uint16_t)(pr & 0xFFFFu))) +
                 (BF16 ? oc_bf2f((uint16_t)(pr >> 16)) : oc_h2f((uint16_t)(pr >> 16)));
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 16);
        if ((c & 15) == 0) xsum[buf * ROWS + row] = sum;
      }
    }
  };

  const bool has_bias = a.bias != nullptr && a.S == 1;
  uint16_t braw[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int n = (nt0 + j) * 16 + col;
    braw[j] = __builtin_amdgcn_raw_buffer_load_b16(oc_rsrc(a.bias, (uint32_t)a.N * 2),
                                                   has_bias && n < a.N ? (uint32_t)n * 2 : kOcOob, 0, 0);
  }
  __amdgpu_buffer_rsrc_t wr[NTW];
  uint32_t mcol[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    wr[j] = oc_rsrc(a.w + (size_t)ntc[j] * a.NU * P * 1024, (uint32_t)a.NU * P * 1024);
    mcol[j] = (uint32_t)(ntc[j] * 16 + col) * 4;
  }
  const __amdgpu_buffer_rsrc_t mr = oc_rsrc(a.meta, (uint32_t)a.G * a.N_pad * 4);
  uint32_t wb[D][NTW][4 * P];
  uint32_t mb[D][NTW][U];
  auto load = [&](int u, uint32_t (&w)[NTW][4 * P], uint32_t (&m)[NTW][U]) {
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int pt = 0; pt < P; ++pt) {
        const oc_u4 v = oc_bload16_nt(wr[j], (uint32_t)(u * P + pt) * 1024 + lane * 16);
        w[j][4 * pt] = v[0];
        w[j][4 * pt + 1] = v[1];
        w[j][4 * pt + 2] = v[2];
        w[j][4 * pt + 3] = v[3];
      }
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int kbl = 0; kbl < U; ++kbl) {
        const int g = (u * U + kbl) >> a.gkb_shift;
        m[j][kbl] = __builtin_amdgcn_raw_buffer_load_b32(mr, mcol[j] + (uint32_t)(g * a.N_pad) * 4, 0, 0);
      }
  };
  oc_f4 yacc[MB][NTW];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j) yacc[i][j] = oc_f4{0.f, 0.f, 0.f, 0.f};
  const int kb_end = (ub + nu) * U;  // one past this split's last k-block
  // k-block kb: x from buffer (kb - first) & 1; afterwards the staged
  // registers of kb + 1 go to the other buffer, kb + 2 is loaded, one barrier.
  auto consume = [&](int u, const uint32_t (&w)[NTW][4 * P], const uint32_t (&m)[NTW][U]) {
#pragma unroll
    for (int kbl = 0; kbl < U; ++kbl) {
      const int kb = u * U + kbl, buf = (kb - ub * U) & 1;
      oc_u4 bq[NTW][4];
#pragma unroll
      for (int j = 0; j < NTW; ++j) decode_kblock<BITS, SUMS && BF16>(w[j], kbl, bq[j], msk, mag);
      if constexpr (SUMS) {
        const uint32_t md = m[0][kbl];
        const float sc = oc_h2f((uint16_t)(md & 0xFFFFu));
        const float oz = OFF + (float)(md >> 16);
        oc_u4 av[MB][4];  // the k-block's A fragments first: one LDS latency, not one per MFMA
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t) av[i][t] = *(const oc_u4*)(xl + (buf * ROWS + 16 * i + col) * XLD + 8 * kq + 32 * t);
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          oc_f4 acc = oc_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < 4; ++t) acc = oc_mfma16<BF16>(av[i][t], bq[0][t], acc);
          const oc_f4 xsv = *(const oc_f4*)(xsum + buf * ROWS + 16 * i + 4 * kq);
#pragma unroll
          for (int r = 0; r < 4; ++r) yacc[i][0][r] = fmaf(sc, fmaf(-oz, xsv[r], acc[r]), yacc[i][0][r]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const oc_gemm::GemmDeq<BF16> dq = oc_gemm::gemm_deq<BF16>(m[j][kbl]);
#pragma unroll
          for (int t = 0; t < 4; ++t) bq[j][t] = oc_gemm::gemm_apply<BF16>(bq[j][t], dq);
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          oc_u4 av[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) av[t] = *(const oc_u4*)(xl + (buf * ROWS + 16 * i + col) * XLD + 8 * kq + 32 * t);
#pragma unroll
          for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t) yacc[i][j] = oc_mfma16<BF16>(av[t], bq[j][t], yacc[i][j]);
        }
      }
      stage_store(buf ^ 1);                  // k-block kb + 1 (its buffer was last read at kb - 1)
      stage_load(min(kb + 2, kb_end - 1));   // past the end: reload the last k-block, unused
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);     // one k-block's decode at a time (register pressure)
    }
  };
  // prologue: x of this split's k-blocks 0 (to LDS) and 1 (in registers), D weight units
  stage_load(ub * U);
  stage_store(0);
  stage_load(min(ub * U + 1, kb_end - 1));
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(ub + d, wb[d], mb[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  for (int i0 = 0; i0 < nu - D; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(ub + i0 + d, wb[d], mb[d]);
      load(ub + i0 + D + d, wb[d], mb[d]);
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) consume(ub + nu - D + d, wb[d], mb[d]);

#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int n = (nt0 + j) * 16 + col;
    if (nt0 + j >= a.NT_total || n >= a.N) continue;
    if (a.S > 1) {
      float* pp = a.partial + ((size_t)split * a.M + m0) * a.N_pad + n;
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * i + 4 * kq + r;
          if (m < M) pp[(size_t)m * a.N_pad] = yacc[i][j][r];
        }
      continue;
    }
    const float b = has_bias ? (BF16 ? oc_bf2f(braw[j]) : oc_h2f(braw[j])) : 0.f;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * i + 4 * kq + r;
        if (m < M) a.y[(size_t)(m0 + m) * a.ldy + n] = BF16 ? oc_f2bf(yacc[i][j][r] + b) : oc_f2h(yacc[i][j][r] + b);
      }
  }
}

// y[m, n] = sum over splits (in split order) of partial[s, m, n] (+ bias).
template <bool BF16>
__global__ void k_splitk_reduce(const float* __restrict__ partial, int S, int M, int N, int N_pad,
                                const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int ldy) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N) return;
  float o = 0.f;
  for (int s = 0; s < S; ++s) o += partial[((size_t)s * M + m) * N_pad + n];
  if (bias) o += BF16 ? oc_bf2f(bias[n]) : oc_h2f(bias[n]);
  y[(size_t)m * ldy + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
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


SkinnyPlan plan_skinny(const oc::Layout& L, int M) {
  SkinnyPlan p;
  p.mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.nt = oc::knob("OC_SKINNY_NT", L.NT >= 512 ? 4 : 2);
  if (p.nt != 2 && p.nt != 4) p.nt = 2;
  p.ngroups = (L.NT + p.nt - 1) / p.nt;
  // enough workgroups to cover 256 CUs about twice, but at least one unit per wave
  int S = oc::knob("OC_SKINNY_S", 0);
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
constexpr int kStreamMaxM = 128;  // rows of k_gemm_stream (8 MFMA row blocks)
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
  const int nt_env = oc::knob("OC_GEMV_NT", 0);
  p.nt = (p.xch == 1 && (nt_env == 2 || (nt_env == 0 && (L.NT + 1) / 2 >= 384))) ? 2 : 1;
  p.ngroups = (L.NT + p.nt - 1) / p.nt;
  // One workgroup streams the whole K of its columns; few column groups get
  // more waves per workgroup.  Each wave owns an x slot of M x (128U + 8) halfs.
  // A CU holds one 16-wave workgroup of this kernel (its registers), so more
  // column groups than CUs take 8 waves: one round of workgroups, not two.
  int w = oc::knob("OC_GEMV_W", 0);
  if (w != 4 && w != 8 && w != 16) w = (p.ngroups > oc_device_cus() || p.nt == 2) ? 8 : 16;
  if (p.cs == 1 && w == 16) w = 8;
  if (p.xch > 1 && w == 16) w = 8;
  if (p.xch == 16) w = 4;  // the 16-chunk x ring is built for 4 waves only
  const size_t slot = (size_t)M * (L.U * 128 + 8) * 2;
  while (w > 4 && slot * w > kGemvLds) w /= 2;
  p.w = w;
  p.deep = oc::knob("OC_GEMV_DEEP", 0);
  int S = oc::knob("OC_GEMV_S", 1);
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
                  void* y, int ldy, hipStream_t st) {
  const dim3 grid((N + 255) / 256, M);
  if (bf16)
    hipLaunchKernelGGL(k_splitk_reduce<true>, grid, dim3(256), 0, st, partial, S, M, N, N_pad,
                       (const uint16_t*)bias, (uint16_t*)y, ldy);
  else
    hipLaunchKernelGGL(k_splitk_reduce<false>, grid, dim3(256), 0, st, partial, S, M, N, N_pad,
                       (const uint16_t*)bias, (uint16_t*)y, ldy);
  OC_HIP(hipGetLastError());
  return 0;
}

constexpr int kSkinnyMaxM = 64;
constexpr size_t kStreamLds = 80 * 1024;  // two workgroups per CU (160 KB of LDS)

// Waves per n-tile of k_gemv_stream (OC_GEMV_STREAM_KS = 1 or 2; default 1,
// measured faster than two half-K waves on the configs' wide layers).
int stream_ksplit(const oc::Layout& L) {
  const int e = oc::knob("OC_GEMV_STREAM_KS", 0);
  const int ks = (e == 1 || e == 2) ? e : 1;
  return (L.NU % ks) == 0 ? ks : 1;
}

size_t stream_lds(const oc::Layout& L, int M) {
  return (size_t)M * (L.K_pad + 8) * 2 + (size_t)(L.K_pad / 128) * 16 * 4;
}

// k_gemm_stream serves groups that are powers of two >= 128 with an even
// number of units: wide layers (at least 1024 n-tiles) at 12 < M <= 32 (and
// M <= 12 when x does not fit k_gemv_stream's LDS), long-K layers (>= 64
// k-blocks) at 16 < M <= 32, every layer at 32 < M <= 64, and short-K layers
// (<= 32 k-blocks) at 64 < M <= 128; the tiled GEMM (or the skinny kernel)
// takes the rest (measured per configuration-1/2 shape and M).  OC_GEMM_STREAM=0
// turns it off, =1 forces it where it applies (up to M = 128).
bool use_gemm_stream(const oc::Layout& L, int M, int gs) {
  const int e = oc::knob("OC_GEMM_STREAM", -1);
  if (e == 0 || M > kStreamMaxM || gs < 128 || log2_exact(gs) < 0 || (L.NU % 2) != 0) return false;
  if (e == 1) return true;
  const int nkb = L.K_pad / 128;
  if (M > 64) return nkb <= 32;
  if (M > 32) return true;
  if (M > 16 && nkb >= 64) return true;
  // measured: k_gemv is faster for 4 < M <= 12, the streaming GEMM from 13 rows
  return L.NT >= 1024 && (M > 12 || (size_t)M * (L.K_pad + 8) * 2 + (size_t)(L.K_pad / 128) * 64 > 80 * 1024);
}

// K splits of k_gemm_stream (workgroups of 4 NTW n-tiles, times the row blocks):
// enough workgroups for one per CU (two per CU on layers of >= 64 k-blocks or
// with the rows split), at most 8 splits, at
// least 4 k-blocks per split, none when the column workgroups cover 3/4 of the
// CUs, and an even number of units per split.
// OC_GEMM_STREAM_S forces the count.
int gemm_stream_split(const oc::Layout& L, int ntw, int mz) {
  const int e = oc::knob("OC_GEMM_STREAM_S", 0);
  const int wgs = (L.NT + 4 * ntw - 1) / (4 * ntw) * mz, nkb = L.K_pad / 128;
  const int target = oc_device_cus() * ((nkb >= 64 || mz > 1) ? 2 : 1);
  int S = e > 0 ? e : (target + wgs - 1) / wgs;
  if (e <= 0) {
    if (S > 8) S = 8;
    if (S > nkb / 4) S = nkb / 4;
    // column workgroups alone cover 3/4 of the CUs: no split, no fp32 partials and no reduce
    // (config-1 gate|up, 224 workgroups of two n-tiles per wave: M = 64 37.7 -> 29.8 us,
    // M = 128 52.1 -> 46.2)
    if (4 * wgs >= 3 * oc_device_cus()) S = 1;
  }
  if (S > L.NU / 2) S = L.NU / 2;
  while (S > 1 && (L.NU % (2 * S)) != 0) --S;
  return S < 1 ? 1 : S;
}

int gemm_stream_rows(int M) { return M <= 16 ? 1 : (M <= 32 ? 2 : (M <= 64 ? 4 : 8)); }

// n-tiles per wave of k_gemm_stream: 2 on the dequantised-B path (more than
// 32 rows) of wide layers (>= 512 n-tiles: config-1 gate at M = 128 41.5 ->
// 37.7 us, config-2 gate 42.8 -> 38.4); narrow layers keep 1 (half the
// workgroups would need more K splits: config-1 o_proj at M = 128 19.6 ->
// 21.6 us).  OC_GEMM_STREAM_NTW forces 1 or 2 on that path.
int gemm_stream_ntw(const oc::Layout& L, int M) {
  if (gemm_stream_rows(M) <= 2) return 1;
  const int e = oc::knob("OC_GEMM_STREAM_NTW", 0);
  if (e == 1 || e == 2) return e;
  return L.NT >= 512 ? 2 : 1;
}

// Row blocks of k_gemm_stream across workgroups (grid.z): above 64 rows two (64-row halves:
// twice the workgroups, each with half the MFMA chain and LDS traffic per k-block, two per CU to
// hide each other's step latency; the weights are read twice, from L2).  Measured (graph of 32
// calls, µs): config 1 q/o M = 128 19.4 -> 17.2, k|v 13.2 -> 11.1, gate 38.2 -> 29.3; config 2
// gate 39.9 -> 32.8.  OC_GEMM_STREAM_MZ = 1 or 2 forces the count there.
int gemm_stream_mz(const oc::Layout& L, int M) {
  if (M <= 32) return 1;
  const int e = oc::knob("OC_GEMM_STREAM_MZ", 0);
  if (e == 1 || e == 2) return e;
  if (M <= 64) return 1;
  // not where the column workgroups alone cover 3/4 of the CUs: there the second half only
  // doubles the weight reads (config-1 merged gate|up M = 128: 49.1 -> 52.1 us, 55 -> 72 MB)
  const int ntw = gemm_stream_ntw(L, 64), wgs = (L.NT + 4 * ntw - 1) / (4 * ntw);
  return 4 * wgs >= 3 * oc_device_cus() ? 1 : 2;
}

struct GemmStreamPlan {
  int mz, mb, ntw, S;  // row blocks across workgroups, row blocks of 16 per workgroup, n-tiles per wave, K splits
};

GemmStreamPlan plan_gemm_stream(const oc::Layout& L, int M) {
  GemmStreamPlan p;
  p.mz = gemm_stream_mz(L, M);
  const int mr = (M + p.mz - 1) / p.mz;
  p.mb = gemm_stream_rows(mr);
  p.ntw = gemm_stream_ntw(L, mr);
  p.S = gemm_stream_split(L, p.ntw, p.mz);
  return p;
}

template <bool BF16>
int dispatch_gemm_stream(int bits, int M, const oc::Layout& L, const StreamArgs& a, hipStream_t st) {
  const GemmStreamPlan sp = plan_gemm_stream(L, M);
  const int mz = sp.mz, mbt = sp.mb, ntw = sp.ntw;
  const dim3 grid((L.NT + 4 * ntw - 1) / (4 * ntw), a.S, mz), block(256);
  const size_t lds = (size_t)2 * 16 * mbt * 136 * 2 + (mbt <= 2 ? (size_t)2 * 16 * mbt * 4 : 0);
#define OC_GS(B_, MB_, NTW_)                                                                \
  if (bits == B_ && mbt == MB_ && ntw == NTW_) {                                            \
    hipLaunchKernelGGL((k_gemm_stream<B_, MB_, BF16, NTW_>), grid, block, lds, st, a);      \
    OC_HIP(hipGetLastError());                                                              \
    return 0;                                                                               \
  }
#define OC_GSB(B_) OC_GS(B_, 1, 1) OC_GS(B_, 2, 1) OC_GS(B_, 4, 1) OC_GS(B_, 8, 1) OC_GS(B_, 4, 2) OC_GS(B_, 8, 2)
  OC_GSB(2) OC_GSB(3) OC_GSB(4) OC_GSB(8)
#undef OC_GSB
#undef OC_GS
  return oc::set_error(OC_ERR_UNSUPPORTED, "no streaming gemm for bits=%d M=%d", bits, M);
}

// Units in flight per wave of k_gemv_stream for this layer, or 0 when the
// layer takes another path: the streaming kernel serves wide layers (at least
// 1024 n-tiles) at M <= 4 (measured slower than k_gemv at M = 8) whose x (and
// its k-block sums) fits in 80 KB of LDS and whose groups are powers of two
// >= 128.  OC_GEMV_STREAM=0 turns it off, =1 forces it (up to M = 8) where it
// applies; OC_GEMV_STREAM_D picks the depth (2 or 4).
int stream_depth(const oc::Layout& L, int M, int gs) {
  const int e = oc::knob("OC_GEMV_STREAM", -1);
  if (e == 0 || M > (e == 1 ? 8 : 4) || gs < 128 || log2_exact(gs) < 0) return 0;
  if (stream_lds(L, M) > kStreamLds) return 0;
  if (e != 1 && L.NT < 1024) return 0;
  const int de = oc::knob("OC_GEMV_STREAM_D", 0);
  const int ks = stream_ksplit(L);
  const int nu = L.NU / ks;
  int d = (de == 2 || de == 4) ? de : ((nu % 4) == 0 ? 4 : 2);
  if (de == 0 && (L.bits == 2 || L.bits == 3)) d = 2;  // measured best
  while (d > 1 && (nu % d) != 0) d /= 2;
  return d >= 2 && nu >= d ? d : 0;
}

// n-tiles per workgroup of k_gemv_stream_bal for this layer, or 0 for
// k_gemv_stream: the balanced kernel takes layers at M >= 3 whose n-tiles
// would not give every CU the same number of 4-wave workgroups, at T =
// ceil(n-tiles / CUs) <= 8 (measured: at M = 1 k_gemv_stream is faster on the
// configs' wide layers even where its CUs are unevenly loaded).
// OC_GEMV_STREAM_BAL=0 turns it off, =1 forces it where T <= 8.
int stream_bal_tiles(const oc::Layout& L, int bits, int M, int ks) {
  const int e = oc::knob("OC_GEMV_STREAM_BAL", -1);
  if (e == 0 || ks != 1 || (e != 1 && M < 3)) return 0;
  const int cus = oc_device_cus();
  const int t = (L.NT + cus - 1) / cus;
  const size_t tile_bytes = (size_t)L.NU * (bits == 3 ? 3 : (bits == 8 ? 2 : 1)) * 1024;
  if (t > kStreamBalWaves || (size_t)t * tile_bytes >= ((size_t)1 << 32)) return 0;
  if (e != 1 && L.NT % (4 * cus) == 0) return 0;
  return t;
}

template <bool BF16>
int dispatch_stream(int bits, int d, int M, const oc::Layout& L, StreamArgs a, hipStream_t st) {
  const int ks = stream_ksplit(L);
  a.tpw = stream_bal_tiles(L, bits, M, ks);
  if (a.tpw > 0) {
    const dim3 grid((L.NT + a.tpw - 1) / a.tpw), block(64 * kStreamBalWaves);
    const int mr = M >= 3 ? 4 : M;
    const size_t lds = stream_lds(L, M) + (size_t)kStreamBalWaves * 2 * mr * 64 * 4;
#define OC_SB(B_, D_, MR_)                                                          \
  if (bits == B_ && d == D_ && mr == MR_) {                                         \
    hipLaunchKernelGGL((k_gemv_stream_bal<B_, D_, MR_, BF16>), grid, block, lds, st, a); \
    OC_HIP(hipGetLastError());                                                      \
    return 0;                                                                       \
  }
#define OC_SBB(B_) OC_SB(B_, 2, 1) OC_SB(B_, 2, 2) OC_SB(B_, 2, 4)
#define OC_SBB4(B_) OC_SBB(B_) OC_SB(B_, 4, 1) OC_SB(B_, 4, 2) OC_SB(B_, 4, 4)
    OC_SBB4(2) OC_SBB4(3) OC_SBB4(4) OC_SBB4(8)
#undef OC_SBB4
#undef OC_SBB
#undef OC_SB
    return oc::set_error(OC_ERR_UNSUPPORTED, "no balanced streaming gemv for bits=%d d=%d", bits, d);
  }
  const dim3 grid((L.NT * ks + 3) / 4), block(256);
  size_t lds = stream_lds(L, M);
  const int mr = M >= 3 ? 4 : M;
  if (ks > 1 && lds < (size_t)4 * mr * 64 * 4) lds = (size_t)4 * mr * 64 * 4;
#define OC_ST(B_, D_, MR_)                                                                         \
  if (bits == B_ && d == D_ && mr == MR_) {                                                        \
    if (ks == 2) hipLaunchKernelGGL((k_gemv_stream<B_, D_, MR_, 2, BF16>), grid, block, lds, st, a); \
    else hipLaunchKernelGGL((k_gemv_stream<B_, D_, MR_, 1, BF16>), grid, block, lds, st, a);         \
    OC_HIP(hipGetLastError());                                                                     \
    return 0;                                                                                      \
  }
#define OC_STB(B_) OC_ST(B_, 2, 1) OC_ST(B_, 2, 2) OC_ST(B_, 2, 4)
#define OC_STB4(B_) OC_STB(B_) OC_ST(B_, 4, 1) OC_ST(B_, 4, 2) OC_ST(B_, 4, 4)
  OC_STB4(2) OC_STB4(3) OC_STB4(4) OC_STB4(8)
#undef OC_STB4
#undef OC_STB
#undef OC_ST
  return oc::set_error(OC_ERR_UNSUPPORTED, "no streaming gemv for bits=%d d=%d", bits, d);
}

// Tile height of the GEMM for M rows (64 MT rows, 256 columns): see
// gemm_tile_height; only 256-row tiles for groups that are not multiples of 128.
int gemm_mt(int M, int N_pad, int gs) {
  const int e = oc::knob("OC_GEMM_MT", 0);
  if ((gs % 128) != 0) return 4;
  if (e == 1 || e == 2 || e == 4) return e;
  return gemm_tile_height(M, N_pad);
}

// The tiled GEMM from M = 33 (17 when there are 64 or more column tiles; 128
// for groups that are not multiples of 128, which only have 256-row tiles);
// the skinny kernel below that.  OC_GEMM_MIN_M overrides the threshold.
bool use_gemm(int M, int N_pad, int gs) {
  const int e = oc::knob("OC_GEMM_MIN_M", 0);
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
  const int gs = oc::eff_group(group_size, K);
  if (M <= kGemvMaxM && stream_depth(L, M, gs) > 0) return ws;
  if (use_gemm_stream(L, M, gs)) {
    const int S = plan_gemm_stream(L, M).S;
    return S > 1 ? ws + align256((size_t)S * M * L.N_pad * 4) : ws;
  }
  if (M <= kGemvMaxM) {
    const GemvPlan p = plan_gemv(L, M, oc::eff_group(group_size, K));
    if (p.S > 1) ws += align256((size_t)p.S * M * L.N_pad * 4);
    return ws;
  }
  if (use_gemm(M, L.N_pad, oc::eff_group(group_size, K))) {
    const int mt = gemm_mt(M, L.N_pad, oc::eff_group(group_size, K));
    return ws + align256(plan_gemm(M, L.N_pad, L.K_pad, oc::knob("OC_GEMM_SPLIT", 0), mt).part_bytes);
  }
  const int Mc = M < kSkinnyMaxM ? M : kSkinnyMaxM;
  const SkinnyPlan p = plan_skinny(L, Mc);
  if (p.S > 1) ws += align256((size_t)p.S * Mc * L.N_pad * 4);
  return ws;
}

extern "C" int oc_gptq_describe_plan(int M, int K, int N, int bits, int group_size, int has_perm, char* buf,
                                     int len) {
  OC_REQUIRE(buf && len > 0, OC_ERR_INVALID, "null buffer");
  OC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
  OC_REQUIRE(M > 0 && K > 0 && N > 0 && K % 32 == 0, OC_ERR_INVALID, "bad shape M=%d K=%d N=%d", M, K, N);
  const oc::Layout L = oc::make_layout(bits, K, N);
  const int gs = oc::eff_group(group_size, K);
  const char* g = has_perm ? "k_gather + " : "";
  const int sd = M <= kGemvMaxM ? stream_depth(L, M, gs) : 0;
  if (sd == 0 && use_gemm_stream(L, M, gs)) {
    const GemmStreamPlan sp = plan_gemm_stream(L, M);
    const int S = sp.S;
    snprintf(buf, len, "%sk_gemm_stream mz=%d mb=%d ntw=%d S=%d%s", g, sp.mz, sp.mb, sp.ntw, S,
             S > 1 ? " + k_splitk_reduce" : "");
  } else if (M <= kGemvMaxM && sd > 0) {
    const int t = stream_bal_tiles(L, bits, M, stream_ksplit(L));
    if (t > 0) snprintf(buf, len, "%sk_gemv_stream_bal d=%d tiles_per_wg=%d", g, sd, t);
    else snprintf(buf, len, "%sk_gemv_stream d=%d ks=%d", g, sd, stream_ksplit(L));
  } else if (M <= kGemvMaxM) {
    const GemvPlan p = plan_gemv(L, M, gs);
    snprintf(buf, len, "%sk_gemv nt=%d w=%d S=%d%s", g, p.nt, p.w, p.S, p.S > 1 ? " + k_splitk_reduce" : "");
  } else if (use_gemm(M, L.N_pad, gs)) {
    const int mt = gemm_mt(M, L.N_pad, gs);
    const GemmPlan gp = plan_gemm(M, L.N_pad, L.K_pad, oc::knob("OC_GEMM_SPLIT", 0), mt);
    snprintf(buf, len, "%sk_gemm mt=%d cs=%d tiles=%d split_tiles=%d S=%d kper=%d%s", g, mt, (gs % 128) ? 1 : 4,
             gp.tiles_main, gp.split_tiles, gp.S, gp.kper, gp.split_tiles ? " + k_gemm_fixup" : "");
  } else {
    const SkinnyPlan p = plan_skinny(L, M < kSkinnyMaxM ? M : kSkinnyMaxM);
    snprintf(buf, len, "%sk_skinny chunks=%d S=%d%s", g, (M + kSkinnyMaxM - 1) / kSkinnyMaxM, p.S,
             p.S > 1 ? " + k_splitk_reduce" : "");
  }
  return 0;
}

namespace {

// y[M, N] (row stride ldy) = x @ dequant(W)^T (+ bias): the body of oc_gptq_gemm.
int gptq_gemm_impl(const void* x, int M, int K, int N, const void* packed, const uint32_t* meta,
                   const int32_t* perm, int bits, int group_size, int act_dtype, const void* bias, void* y,
                   int ldy, void* workspace, size_t ws_bytes, hipStream_t st) {
  OC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
  OC_REQUIRE(M >= 0 && K > 0 && N > 0, OC_ERR_INVALID, "bad shape M=%d K=%d N=%d", M, K, N);
  OC_REQUIRE(K % 32 == 0, OC_ERR_SHAPE, "K=%d must be a multiple of 32", K);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d", act_dtype);
  OC_REQUIRE(x && packed && meta && y, OC_ERR_INVALID, "null pointer");
  if (M == 0) return 0;
  const int gs = oc::eff_group(group_size, K);
  OC_REQUIRE(gs % 32 == 0, OC_ERR_UNSUPPORTED, "group_size=%d must be a multiple of 32 (or -1)", group_size);
  const int G = (K + gs - 1) / gs;
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
  const int sd = M <= kGemvMaxM ? stream_depth(L, M, gs) : 0;
  if (sd == 0 && use_gemm_stream(L, M, gs)) {
    StreamArgs a = {};
    a.x = xa;
    a.w = (const uint8_t*)packed;
    a.meta = meta;
    a.bias = (const uint16_t*)bias;
    a.y = (uint16_t*)y;
    a.M = M;
    a.K = K;
    a.K_pad = L.K_pad;
    a.N = N;
    a.N_pad = L.N_pad;
    a.NT_total = L.NT;
    a.NU = L.NU;
    a.G = G;
    a.gs = gs;
    a.gkb_shift = log2_exact(gs) - 7;
    a.ldy = ldy;
    a.S = plan_gemm_stream(L, M).S;
    a.partial = (float*)ws;
    const int rc = bf16 ? dispatch_gemm_stream<true>(bits, M, L, a, st) : dispatch_gemm_stream<false>(bits, M, L, a, st);
    if (rc || a.S == 1) return rc;
    return launch_reduce(bf16, a.partial, a.S, M, N, L.N_pad, bias, y, ldy, st);
  }
  if (M <= kGemvMaxM) {
    if (sd > 0) {
      StreamArgs a = {};
      a.x = xa;
      a.w = (const uint8_t*)packed;
      a.meta = meta;
      a.bias = (const uint16_t*)bias;
      a.y = (uint16_t*)y;
      a.M = M;
      a.K = K;
      a.K_pad = L.K_pad;
      a.N = N;
      a.N_pad = L.N_pad;
      a.NT_total = L.NT;
      a.NU = L.NU;
      a.G = G;
      a.gs = gs;
      a.gkb_shift = log2_exact(gs) - 7;
      a.ldy = ldy;
      return bf16 ? dispatch_stream<true>(bits, sd, M, L, a, st) : dispatch_stream<false>(bits, sd, M, L, a, st);
    }
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
    a.ldy = ldy;
    a.bits = bits;
    a.out_f32 = 0;
    const int rc = bf16 ? dispatch_gemv_bits<true>(bits, p, a, st) : dispatch_gemv_bits<false>(bits, p, a, st);
    if (rc || p.S == 1) return rc;
    return launch_reduce(bf16, a.partial, p.S, M, N, L.N_pad, bias, y, ldy, st);
  }
  if (use_gemm(M, L.N_pad, gs)) {
    GemmArgs g = {};
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
    const GemmPlan gp = plan_gemm(M, L.N_pad, L.K_pad, oc::knob("OC_GEMM_SPLIT", 0), mt);
    g.post = nullptr;
    g.ldx = K;
    g.ldy = ldy;
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
    const size_t lds = oc_gemm::gemm_lds_bytes(mt);
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
    a.y = (uint16_t*)y + (size_t)m0 * ldy;
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
    a.ldy = ldy;
    int rc = bf16 ? dispatch_skinny_bits<true>(bits, p, a, st) : dispatch_skinny_bits<false>(bits, p, a, st);
    if (!rc && p.S > 1) rc = launch_reduce(bf16, a.partial, p.S, Mc, N, L.N_pad, bias, a.y, ldy, st);
    if (rc) return rc;
  }
  return 0;
}

}  // namespace

extern "C" int oc_gptq_gemm(const void* x, int M, int K, int N, const void* packed, const uint32_t* meta,
                            const int32_t* perm, int bits, int group_size, int act_dtype, const void* bias,
                            void* y, void* workspace, size_t ws_bytes, void* stream) {
  return gptq_gemm_impl(x, M, K, N, packed, meta, perm, bits, group_size, act_dtype, bias, y, N, workspace,
                        ws_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of oc_gptq_gemm: the work buffer is this file's
// device array `scratch` (kNoAllocScratch bytes per GPU, held until the
// process ends).  Host code never passes the array's name to a kernel: its
// device address is looked up once per device with hipGetSymbolAddress and
// kept in g_scratch_ptr.  Every call on a GPU shares that GPU's array, so
// calls that overlap on one GPU race.  No kernel of oc_gptq_gemm needs its
// work buffer cleared (every byte read is written earlier in the same call).
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratch = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratch];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

int scratch_for_current_device(void** out) {
  int dev = 0;
  OC_HIP(hipGetDevice(&dev));
  OC_REQUIRE(dev >= 0 && dev < kMaxDevices, OC_ERR_INVALID, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    OC_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    OC_REQUIRE(p != nullptr, OC_ERR_HIP, "hipGetSymbolAddress returned a null address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" size_t oc_gptq_noalloc_scratch_bytes(void) { return kNoAllocScratch; }

extern "C" int oc_gptq_gemm_noalloc(const void* x, int M, int K, int N, const void* packed, const uint32_t* meta,
                                    const int32_t* perm, int bits, int group_size, int act_dtype, const void* bias,
                                    void* y, void* stream) {
  OC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
  OC_REQUIRE(M >= 0 && K > 0 && N > 0, OC_ERR_INVALID, "bad shape M=%d K=%d N=%d", M, K, N);
  if (M == 0) return 0;
  const size_t need = oc_gptq_workspace_bytes(M, K, N, bits, group_size, perm != nullptr);
  OC_REQUIRE(need <= kNoAllocScratch, OC_ERR_WORKSPACE,
             "this call needs %zu bytes of work buffer; the allocation-free entry point holds at most %zu "
             "(use oc_gptq_gemm with a caller workspace)", need, kNoAllocScratch);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_for_current_device(&ws)) return rc;
  }
  return gptq_gemm_impl(x, M, K, N, packed, meta, perm, bits, group_size, act_dtype, bias, y, N, ws,
                        need > 0 ? kNoAllocScratch : 0, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Fused modules: several GPTQ parts (each with its own bits, group size,
// scales/zeros and act-order permutation) that read the same activations and
// write side by side into one output.  At M <= 16, when every part has groups
// of a multiple of 128, one k_gemv_group launch runs all parts; otherwise the
// parts run one after the other through oc_gptq_gemm's paths.
// ---------------------------------------------------------------------------
namespace {

struct GroupPlan {
  bool fused;
  int w, xch, ntmax;
  int nt[kMaxParts];  // n-tiles per workgroup of each part
  size_t lds;
  size_t perm_off[kMaxParts];  // workspace offset of a part's permuted x
  size_t bytes;
};

GroupPlan plan_group(const oc_gptq_part* parts, int n_parts, int M, int K) {
  GroupPlan g = {};
  g.fused = M <= kGemvMaxM && n_parts <= kMaxParts;
  g.w = 16;
  g.xch = 1;
  size_t slot = 0, off = 0;
  for (int i = 0; i < n_parts; ++i) {
    const oc_gptq_part& P = parts[i];
    const int gs = oc::eff_group(P.group_size, K);
    const oc::Layout L = oc::make_layout(P.bits, K, P.N);
    if ((gs % 128) != 0) g.fused = false;
    if (g.fused) {
      const GemvPlan p = plan_gemv(L, M, gs);
      if (p.S != 1) g.fused = false;
      g.w = p.w < g.w ? p.w : g.w;
      g.xch = p.xch > g.xch ? p.xch : g.xch;
      const size_t sl = (size_t)M * (L.U * 128 + 8) * 2;
      slot = sl > slot ? sl : slot;
    }
    g.perm_off[i < kMaxParts ? i : 0] = off;
    if (P.perm) off += align256((size_t)M * K * 2);
  }
  if (g.fused) {
    // parts whose n-tiles carry at most half the bytes of the widest part's take two n-tiles
    // per workgroup (one x chunk per lane only); then 8 waves per workgroup when some part
    // takes two n-tiles or there are more workgroups than CUs (one 16-wave workgroup per CU)
    // (q 4-bit | k, v 8-bit at M = 1: 8.3 us with one n-tile and 16 waves, 7.1 with one n-tile
    // and 8 waves, 6.7 with two and 8)
    int bmax = 0;
    for (int i = 0; i < n_parts; ++i) bmax = parts[i].bits > bmax ? parts[i].bits : bmax;
    g.ntmax = 1;
    int blocks = 0;
    for (int i = 0; i < n_parts; ++i) {
      const int NT = oc::make_layout(parts[i].bits, K, parts[i].N).NT;
      const int nt = (g.xch == 1 && 2 * parts[i].bits <= bmax && NT >= 2 && oc::knob("OC_GROUP_NT", 2) == 2) ? 2 : 1;
      g.nt[i] = nt;
      g.ntmax = nt > g.ntmax ? nt : g.ntmax;
      blocks += (NT + nt - 1) / nt;
    }
    if ((blocks > oc_device_cus() || g.ntmax == 2) && g.w > 8 && oc::knob("OC_GEMV_W", 0) == 0) g.w = 8;
    if (g.xch > 1 && g.w > 8) g.w = 8;
    while (g.w > 4 && slot * g.w > kGemvLds) g.w /= 2;
    const size_t xb = slot * g.w, rb = (size_t)g.w * g.ntmax * 4 * 64 * 4;
    g.lds = ((xb > rb ? xb : rb) + 15) / 16 * 16;
    g.bytes = off;
  } else {  // parts one after the other: they reuse one workspace
    size_t mx = 0;
    for (int i = 0; i < n_parts; ++i) {
      const size_t b = oc_gptq_workspace_bytes(M, K, parts[i].N, parts[i].bits, parts[i].group_size,
                                               parts[i].perm != nullptr);
      mx = b > mx ? b : mx;
    }
    g.bytes = mx;
  }
  return g;
}

template <bool BF16>
int launch_group(const GroupPlan& gp, const GemvGroupArgs& ga, int blocks, hipStream_t st) {
#define OC_GG(NT_, W_, XC_)                                                                             \
  if (gp.ntmax == NT_ && gp.w == W_ && gp.xch == XC_) {                                                 \
    hipLaunchKernelGGL((k_gemv_group<NT_, W_, XC_, BF16>), dim3(blocks), dim3(64 * W_), gp.lds, st, ga); \
    OC_HIP(hipGetLastError());                                                                          \
    return 0;                                                                                           \
  }
  OC_GG(1, 16, 1) OC_GG(1, 8, 1) OC_GG(1, 8, 4) OC_GG(1, 8, 8) OC_GG(1, 8, 16)
  OC_GG(1, 4, 1) OC_GG(1, 4, 4) OC_GG(1, 4, 8) OC_GG(1, 4, 16)
  OC_GG(2, 16, 1) OC_GG(2, 8, 1) OC_GG(2, 4, 1)
#undef OC_GG
  return oc::set_error(OC_ERR_UNSUPPORTED, "no grouped gemv kernel for w=%d xch=%d", gp.w, gp.xch);
}

int check_part(const oc_gptq_part& P, int i, int K) {
  OC_REQUIRE(P.packed && P.meta, OC_ERR_INVALID, "part %d: null pointer", i);
  OC_REQUIRE(P.bits == 2 || P.bits == 3 || P.bits == 4 || P.bits == 8, OC_ERR_UNSUPPORTED,
             "part %d: unsupported bits=%d", i, P.bits);
  OC_REQUIRE(P.N > 0, OC_ERR_INVALID, "part %d: N=%d", i, P.N);
  const int gs = oc::eff_group(P.group_size, K);
  OC_REQUIRE(gs % 32 == 0, OC_ERR_UNSUPPORTED, "part %d: group_size=%d must be a multiple of 32 (or -1)", i,
             P.group_size);
  return 0;
}

}  // namespace

extern "C" size_t oc_gptq_grouped_workspace_bytes(const oc_gptq_part* parts, int n_parts, int M, int K) {
  if (!parts || n_parts < 1 || M <= 0 || K <= 0) return 0;
  for (int i = 0; i < n_parts; ++i)
    if (check_part(parts[i], i, K)) return 0;
  return plan_group(parts, n_parts, M, K).bytes;
}

extern "C" int oc_gptq_gemm_grouped(const void* x, int M, int K, const oc_gptq_part* parts, int n_parts,
                                    int act_dtype, void* y, int ldy, void* workspace, size_t ws_bytes,
                                    void* stream) {
  OC_REQUIRE(x && y && parts, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(n_parts >= 1, OC_ERR_INVALID, "n_parts=%d", n_parts);
  OC_REQUIRE(M >= 0 && K > 0, OC_ERR_INVALID, "bad shape M=%d K=%d", M, K);
  OC_REQUIRE(K % 32 == 0, OC_ERR_SHAPE, "K=%d must be a multiple of 32", K);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d",
             act_dtype);
  int n_total = 0;
  for (int i = 0; i < n_parts; ++i) {
    const int rc = check_part(parts[i], i, K);
    if (rc) return rc;
    n_total += parts[i].N;
  }
  OC_REQUIRE(ldy >= n_total, OC_ERR_SHAPE, "ldy=%d < total width %d", ldy, n_total);
  if (M == 0) return 0;
  const GroupPlan gp = plan_group(parts, n_parts, M, K);
  OC_REQUIRE(ws_bytes >= gp.bytes && (gp.bytes == 0 || workspace), OC_ERR_WORKSPACE,
             "workspace of %zu bytes is smaller than the %zu required", ws_bytes, gp.bytes);
  hipStream_t st = (hipStream_t)stream;
  const bool bf16 = act_dtype == OC_DTYPE_BF16;
  uint16_t* yo = (uint16_t*)y;
  if (!gp.fused) {
    for (int i = 0, off = 0; i < n_parts; off += parts[i].N, ++i) {
      const oc_gptq_part& P = parts[i];
      const int rc = gptq_gemm_impl(x, M, K, P.N, P.packed, P.meta, P.perm, P.bits, P.group_size, act_dtype,
                                    P.bias, yo + off, ldy, workspace, ws_bytes, st);
      if (rc) return rc;
    }
    return 0;
  }
  GemvGroupArgs ga = {};
  int blocks = 0;
  for (int i = 0, off = 0; i < n_parts; off += parts[i].N, ++i) {
    const oc_gptq_part& P = parts[i];
    const int gs = oc::eff_group(P.group_size, K);
    const oc::Layout L = oc::make_layout(P.bits, K, P.N);
    const uint16_t* xa = (const uint16_t*)x;
    if (P.perm) {
      uint16_t* xp = (uint16_t*)((uint8_t*)workspace + gp.perm_off[i]);
      hipLaunchKernelGGL(k_gather, dim3((K + 255) / 256, M), dim3(256), 0, st, xa, P.perm, M, K, xp);
      OC_HIP(hipGetLastError());
      xa = xp;
    }
    GemvArgs& a = ga.part[i];
    a.x = xa;
    a.w = (const uint8_t*)P.packed;
    a.meta = P.meta;
    a.bias = (const uint16_t*)P.bias;
    a.y = yo + off;
    a.partial = nullptr;
    a.M = M;
    a.K = K;
    a.N = P.N;
    a.N_pad = L.N_pad;
    a.NT_total = L.NT;
    a.NU = L.NU;
    a.G = (K + gs - 1) / gs;
    a.gs = gs;
    a.gshift = log2_exact(gs);
    a.S = 1;
    a.ups = L.NU;
    a.ldy = ldy;
    a.bits = P.bits;
    a.out_f32 = 0;
    ga.block_start[i] = blocks;
    ga.part_nt[i] = gp.nt[i];
    blocks += (L.NT + gp.nt[i] - 1) / gp.nt[i];
  }
  for (int i = n_parts; i <= kMaxParts; ++i) ga.block_start[i] = blocks;
  ga.n_parts = n_parts;
  return bf16 ? launch_group<true>(gp, ga, blocks, st) : launch_group<false>(gp, ga, blocks, st);
}

// ---------------------------------------------------------------------------
// MoE experts with GPTQ weights (OneComp's unfused experts,
// onecomp/utils/unfuse_moe.py:61-114): for every token t and slot j of its
// top-k, pair p = t * topk + j runs expert e = ids[p]:
//   h[p]    = act(x[t] @ Wg_e^T (+ bg_e), x[t] @ Wu_e^T (+ bu_e))   (k_moe_gate_up)
//   part[p] = h[p] @ W2_e^T                                         (k_moe_down, fp32)
//   y[t]    = sum_j w[t, j] * (part[t * topk + j] + b2_e)           (k_moe_combine)
// Three launches, no host synchronisation; pairs with an id outside [0, E)
// contribute nothing.
// ---------------------------------------------------------------------------
namespace {

template <int BITS, int RM>
struct MoeXch {  // x chunks per lane for RM rows of a unit
  static constexpr int xc = (moe_cap(RM) * 16 * Geo<BITS>::U + 63) / 64;
  static constexpr int X = xc <= 1 ? 1 : (xc <= 4 ? 4 : (xc <= 8 ? 8 : 16));
};

template <int BITS, int NT, int CS, int XCH>
struct MoeD {  // units in flight per wave
  static constexpr int DB = (BITS == 3 || BITS == 8) ? 2 : 4;
  static constexpr int D = (XCH >= 8 || (CS == 1 && BITS == 3)) ? 1 : (DB / NT > 0 ? DB / NT : 1);
};

struct MoePlan {
  size_t h_off, part_off, sorted_off, runs_off, nruns_off, xp_off, hp_off, bytes;
  size_t g_sorted, g_pos, g_runs, g_counts, g_xs, g_h13, g_h, g_ys;
  int rm, w1, w2;
  size_t lds1, lds2;
};

MoePlan plan_moe(int M, int H, int I, int E, int topk, int bits, int gs2, bool act_order = false) {
  MoePlan p;
  const size_t pairs = (size_t)M * topk;
  const int h_pad = (H + 15) / 16 * 16;
  p.h_off = 0;
  p.part_off = align256(pairs * I * 2);
  p.sorted_off = p.part_off + align256(pairs * h_pad * 4);
  p.runs_off = p.sorted_off + align256(pairs * 4);
  p.nruns_off = p.runs_off + align256(pairs * 16);
  p.bytes = p.nruns_off + 256;
  // act-order: x gathered per pair in each expert's k order, and h likewise for down
  p.xp_off = p.hp_off = 0;
  if (act_order) {
    p.xp_off = p.bytes;
    p.hp_off = p.xp_off + align256(pairs * H * 2);
    p.bytes = p.hp_off + align256(pairs * I * 2);
  }
  // prefill path (its buffers reuse the workspace from 0): sorted, pos, runs, counts, then
  // x, gate|up, h and the down outputs in sorted row order
  p.g_sorted = 0;
  p.g_pos = align256(pairs * 4);
  p.g_runs = p.g_pos + align256(pairs * 4);
  p.g_counts = p.g_runs + align256(pairs * 16);
  p.g_xs = p.g_counts + 256;
  p.g_h13 = p.g_xs + align256(pairs * H * 2);
  p.g_h = p.g_h13 + align256(pairs * 2 * I * 2);
  p.g_ys = p.g_h + align256(pairs * I * 2);
  const size_t gbytes = p.g_ys + align256(pairs * H * 2);
  if (pairs >= 32 && gbytes > p.bytes) p.bytes = gbytes;
  // rows per run: one for a single token (its slots name distinct experts); else 4, or 16
  // when the pairs spread over the experts give more than 4 per expert on average; beyond
  // 64 pairs, sorted runs of up to 16 (OC_MOE_RM=1: one row per pair)
  const int rm_env = oc::knob("OC_MOE_RM", 0);
  int rm = rm_env;
  if (rm != 1 && rm != 4 && rm != 16) {
    const size_t busy = pairs < (size_t)E ? pairs : (size_t)E;
    rm = M == 1 ? 1 : ((pairs + busy - 1) / busy <= 4 ? 4 : 16);
  }
  if (pairs > 64) rm = (rm_env == 1 || E > kMoeMaxE) ? 1 : kMoeSorted;
  p.rm = rm;
  const int U = bits == 2 ? 2 : (bits == 3 ? 4 : 1);
  const size_t slot = (size_t)moe_cap(rm) * (128 * U + 8) * 2;
  p.w1 = 4;  // gate|up
  const int nu2 = (I + 128 * U - 1) / (128 * U);
  // down: 8 waves for long k-ranges (runs of 1 or 4 rows, groups of 128 or more)
  int w2 = oc::knob("OC_MOE_W2", 0);
  if (w2 != 4 && w2 != 8) w2 = nu2 >= 24 ? 8 : 4;
  if (rm == 16 || rm == kMoeSorted || gs2 % 128 != 0) w2 = 4;
  p.w2 = w2;
  auto lds = [&](int w, int nt) {
    const size_t xb = slot * w, rb = (size_t)w * nt * 256 * 4;
    return ((xb > rb ? xb : rb) + 15) / 16 * 16;
  };
  p.lds1 = lds(p.w1, 2);
  p.lds2 = lds(p.w2, 1);
  return p;
}

template <bool BF16, bool UP>
int launch_moe(const MoeArgs& g, int bits, int cs, int w, int rm, size_t lds, int grid, hipStream_t st) {
#define OC_MK(B_, CS_, W_, RM_)                                                                            \
  if (bits == B_ && cs == CS_ && w == W_ && rm == RM_) {                                                   \
    constexpr int X_ = MoeXch<B_, RM_>::X;                                                                 \
    constexpr int D_ = MoeD<B_, UP ? 2 : 1, CS_, X_>::D;                                                   \
    if constexpr (UP)                                                                                      \
      hipLaunchKernelGGL((k_moe_gate_up<B_, CS_, D_, W_, X_, RM_, BF16>), dim3(grid), dim3(64 * W_), lds,  \
                         st, g);                                                                           \
    else                                                                                                   \
      hipLaunchKernelGGL((k_moe_down<B_, CS_, D_, W_, X_, RM_, BF16>), dim3(grid), dim3(64 * W_), lds, st, \
                         g);                                                                               \
    OC_HIP(hipGetLastError());                                                                             \
    return 0;                                                                                              \
  }
#define OC_MKR(B_, CS_, W_) \
  OC_MK(B_, CS_, W_, 1) OC_MK(B_, CS_, W_, 4) OC_MK(B_, CS_, W_, 16) OC_MK(B_, CS_, W_, kMoeSorted)
#define OC_MKB(B_) OC_MKR(B_, 4, 4) OC_MKR(B_, 1, 4)
  OC_MKB(2) OC_MKB(3) OC_MKB(4) OC_MKB(8)
  if constexpr (!UP) {  // longer k-ranges of down: 8 waves
#define OC_MKW(B_) OC_MK(B_, 4, 8, 1) OC_MK(B_, 4, 8, 4)
    OC_MKW(2) OC_MKW(3) OC_MKW(4) OC_MKW(8)
#undef OC_MKW
  }
#undef OC_MKB
#undef OC_MKR
#undef OC_MK
  return oc::set_error(OC_ERR_UNSUPPORTED, "no MoE kernel for bits=%d cs=%d w=%d rows=%d", bits, cs, w, rm);
}

template <bool BF16>
int launch_grouped_gemm(const GemmArgs& g, int bits, bool cs4, int mt, int grid, hipStream_t st) {
  const size_t lds = oc_gemm::gemm_lds_bytes(mt);
#define OC_GG2(B_)                                                                                           \
  if (bits == B_) {                                                                                          \
    if (!cs4) hipLaunchKernelGGL((k_gemm<B_, 1, BF16, 4, true>), dim3(grid), dim3(256), lds, st, g);        \
    else if (mt == 1) hipLaunchKernelGGL((k_gemm<B_, 4, BF16, 1, true>), dim3(grid), dim3(256), lds, st, g); \
    else if (mt == 2) hipLaunchKernelGGL((k_gemm<B_, 4, BF16, 2, true>), dim3(grid), dim3(256), lds, st, g); \
    else hipLaunchKernelGGL((k_gemm<B_, 4, BF16, 4, true>), dim3(grid), dim3(256), lds, st, g);             \
    OC_HIP(hipGetLastError());                                                                               \
    return 0;                                                                                                \
  }
  OC_GG2(2) OC_GG2(3) OC_GG2(4) OC_GG2(8)
#undef OC_GG2
  return oc::set_error(OC_ERR_UNSUPPORTED, "no grouped GEMM for bits=%d", bits);
}

// Prefill: the pairs sorted by expert (runs of 64 MT rows), x gathered into that order, the
// large-M GEMM per run for gate|up (rounded with its bias, as the reference's linears round)
// and for down, the activation between them, and the top-k sum through each pair's position.
int moe_prefill(const void* x, int M, int H, int I, int E, int topk, const int32_t* ids, const float* weights,
                const void* w13, size_t w13_stride, const uint32_t* meta13, size_t meta13_stride, const void* b13,
                const void* w2, size_t w2_stride, const uint32_t* meta2, size_t meta2_stride, const void* b2,
                int bits, int gs13, int gs2, int act, float alpha, float limit, bool bf16, void* y, uint8_t* ws,
                const MoePlan& mp, hipStream_t st) {
  const int pairs = M * topk;
  const int busy = E < pairs ? E : pairs;
  const int avg = pairs / busy;
  const bool cs4a = gs13 % 128 == 0, cs4b = gs2 % 128 == 0;
  int mt = avg >= 256 ? 4 : (avg >= 128 ? 2 : 1);
  const int mt_env = oc::knob("OC_MOE_GEMM_MT", 0);
  if (mt_env == 1 || mt_env == 2 || mt_env == 4) mt = mt_env;
  if (!cs4a || !cs4b) mt = 4;  // the GEMM for groups below 128 is built for 256-row tiles
  const int BM = 64 * mt;
  int* sorted = (int*)(ws + mp.g_sorted);
  int* pos = (int*)(ws + mp.g_pos);
  int* runs = (int*)(ws + mp.g_runs);
  int* counts = (int*)(ws + mp.g_counts);
  uint16_t* xs = (uint16_t*)(ws + mp.g_xs);
  uint16_t* h13 = (uint16_t*)(ws + mp.g_h13);
  uint16_t* h = (uint16_t*)(ws + mp.g_h);
  uint16_t* ys = (uint16_t*)(ws + mp.g_ys);
  hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(1024), 0, st, ids, pairs, E, BM, sorted, pos, runs, counts);
  hipLaunchKernelGGL(k_moe_gather_x, dim3(pairs), dim3(256), 0, st, (const uint16_t*)x, H, topk, sorted, counts, xs);
  OC_HIP(hipGetLastError());
  const int bound = (pairs + BM - 1) / BM + busy;
  const int tiles = bound < pairs ? bound : pairs;
  auto fill = [&](GemmArgs& g, const oc::Layout& L, int K, int N, int gs) {
    g = GemmArgs{};
    g.M = pairs;
    g.K = K;
    g.N = N;
    g.N_pad = L.N_pad;
    g.NT_total = L.NT;
    g.NU = L.NU;
    g.G = (K + gs - 1) / gs;
    g.gs = gs;
    g.gshift = log2_exact(gs);
    g.NKB = L.K_pad / 128;
    g.NB = (L.N_pad + kGemmBN - 1) / kGemmBN;
    g.ldx = K;
    g.ldy = N;
    g.pstride = 1;
    g.S = 1;
    g.kper = g.NKB;
    g.tiles_main = 0x7FFFFFFF;
    g.gtab = runs;
    g.gcount = counts;
  };
  GemmArgs g = {};
  const oc::Layout L13 = oc::make_layout(bits, H, 2 * I), L2 = oc::make_layout(bits, I, H);
  fill(g, L13, H, 2 * I, gs13);
  g.x = xs;
  g.w = (const uint8_t*)w13;
  g.meta = meta13;
  g.bias = (const uint16_t*)b13;
  g.y = h13;
  g.gw_stride = w13_stride;
  g.gmeta_stride = meta13_stride;
  g.gbias_stride = 2 * I;
  int rc = bf16 ? launch_grouped_gemm<true>(g, bits, cs4a, mt, tiles * g.NB, st)
                : launch_grouped_gemm<false>(g, bits, cs4a, mt, tiles * g.NB, st);
  if (rc) return rc;
  const dim3 ga((I + 255) / 256, pairs);
  if (bf16) hipLaunchKernelGGL(k_moe_act_sorted<true>, ga, dim3(256), 0, st, h13, I, counts, act, alpha, limit, h);
  else hipLaunchKernelGGL(k_moe_act_sorted<false>, ga, dim3(256), 0, st, h13, I, counts, act, alpha, limit, h);
  OC_HIP(hipGetLastError());
  fill(g, L2, I, H, gs2);
  g.x = h;
  g.w = (const uint8_t*)w2;
  g.meta = meta2;
  g.bias = (const uint16_t*)b2;
  g.y = ys;
  g.gw_stride = w2_stride;
  g.gmeta_stride = meta2_stride;
  g.gbias_stride = H;
  rc = bf16 ? launch_grouped_gemm<true>(g, bits, cs4b, mt, tiles * g.NB, st)
            : launch_grouped_gemm<false>(g, bits, cs4b, mt, tiles * g.NB, st);
  if (rc) return rc;
  const dim3 gc((H + 255) / 256, M);
  if (bf16)
    hipLaunchKernelGGL(k_moe_combine_sorted<true>, gc, dim3(256), 0, st, ys, H, topk, M, ids, E, weights, pos,
                       (uint16_t*)y);
  else
    hipLaunchKernelGGL(k_moe_combine_sorted<false>, gc, dim3(256), 0, st, ys, H, topk, M, ids, E, weights, pos,
                       (uint16_t*)y);
  OC_HIP(hipGetLastError());
  return 0;
}

}  // namespace

extern "C" size_t oc_moe_workspace_bytes(int M, int H, int I, int topk, int act_order) {
  if (M <= 0 || H <= 0 || I <= 0 || topk <= 0) return 0;
  return plan_moe(M, H, I, 1, topk, 4, 128, act_order != 0).bytes;
}

extern "C" int oc_moe_gptq_forward(const void* x, int M, int H, int I, int E, int topk, const int32_t* ids,
                                   const float* weights, const void* w13, size_t w13_stride, const uint32_t* meta13,
                                   size_t meta13_stride, const void* b13, const void* w2, size_t w2_stride,
                                   const uint32_t* meta2, size_t meta2_stride, const void* b2,
                                   const int32_t* perm13, const int32_t* perm2, int bits, int group_size, int act,
                                   float alpha, float limit, int act_dtype, void* y, void* workspace,
                                   size_t ws_bytes, void* stream) {
  OC_REQUIRE(x && ids && weights && w13 && meta13 && w2 && meta2 && y, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, OC_ERR_UNSUPPORTED, "unsupported bits=%d", bits);
  OC_REQUIRE(M >= 0 && H > 0 && I > 0 && E > 0 && topk > 0 && topk <= 64, OC_ERR_INVALID,
             "bad shape M=%d H=%d I=%d E=%d topk=%d", M, H, I, E, topk);
  OC_REQUIRE(H % 32 == 0 && I % 32 == 0, OC_ERR_SHAPE, "H=%d and I=%d must be multiples of 32", H, I);
  OC_REQUIRE(act >= 0 && act <= 2, OC_ERR_UNSUPPORTED, "unknown activation %d", act);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d",
             act_dtype);
  if (M == 0) return 0;
  OC_REQUIRE((size_t)M * topk * (I / 16) < (1u << 31) && (size_t)M * topk * ((H + 15) / 16) < (1u << 31),
             OC_ERR_SHAPE, "M=%d x topk=%d is too large for one launch", M, topk);
  const int gs13 = oc::eff_group(group_size, H), gs2 = oc::eff_group(group_size, I);
  OC_REQUIRE(gs13 % 32 == 0 && gs2 % 32 == 0, OC_ERR_UNSUPPORTED, "group_size=%d", group_size);
  const bool act_order = perm13 != nullptr || perm2 != nullptr;
  const MoePlan mp = plan_moe(M, H, I, E, topk, bits, gs2, act_order);
  OC_REQUIRE(ws_bytes >= mp.bytes && workspace, OC_ERR_WORKSPACE,
             "workspace of %zu bytes is smaller than the %zu required", ws_bytes, mp.bytes);
  const oc::Layout L13 = oc::make_layout(bits, H, 2 * I), L2 = oc::make_layout(bits, I, H);
  OC_REQUIRE(w13_stride >= oc::layout_bytes(L13) && w2_stride >= oc::layout_bytes(L2), OC_ERR_INVALID,
             "expert strides smaller than one expert's packed weights");
  const int G13 = (H + gs13 - 1) / gs13, G2 = (I + gs2 - 1) / gs2;
  OC_REQUIRE(meta13_stride >= (size_t)G13 * L13.N_pad && meta2_stride >= (size_t)G2 * L2.N_pad, OC_ERR_INVALID,
             "expert scale/zero strides too small");
  hipStream_t st = (hipStream_t)stream;
  const bool bf16 = act_dtype == OC_DTYPE_BF16;
  uint8_t* ws = (uint8_t*)workspace;
  const int pairs = M * topk;
  auto fill = [&](GemvArgs& a, const oc::Layout& L, int K, int N, int gs, int G) {
    a = GemvArgs{};
    a.M = moe_cap(mp.rm);
    a.K = K;
    a.N = N;
    a.N_pad = L.N_pad;
    a.NT_total = L.NT;
    a.NU = L.NU;
    a.G = G;
    a.gs = gs;
    a.gshift = log2_exact(gs);
    a.S = 1;
    a.ups = L.NU;
    a.bits = bits;
  };
  // The grouped large-M GEMM per run of rows (prefill sizes) serves at least 32 rows per busy
  // expert on average (measured against the sorted-run GEMV path, us: Qwen3-30B-A3B experts
  // M = 512 325 -> 157, M = 2048 1053 -> 430; Mixtral-8x7B M = 128 527 -> 309, M = 512 1782 ->
  // 660); fewer rows take the sorted-run path.  OC_MOE_GEMM = 1 forces it from 32 pairs, = 0
  // turns it off.
  {
    const int gm = oc::knob("OC_MOE_GEMM", -1);
    const int busy = E < pairs ? E : pairs;
    const bool on = gm == 1 || (gm < 0 && busy > 0 && pairs / busy >= 32);
    if (E <= kMoeMaxE && pairs >= 32 && on && !act_order)
      return moe_prefill(x, M, H, I, E, topk, ids, weights, w13, w13_stride, meta13, meta13_stride, b13, w2,
                         w2_stride, meta2, meta2_stride, b2, bits, gs13, gs2, act, alpha, limit, bf16, y, ws, mp, st);
  }
  MoeArgs g = {};
  g.ids = ids;
  g.pairs = pairs;
  // workgroup groups per launch: one per pair, or one per sorted run (at most this many)
  int groups = pairs;
  if (mp.rm == kMoeSorted) {
    int* sorted = (int*)(ws + mp.sorted_off);
    int* runs = (int*)(ws + mp.runs_off);
    int* nruns = (int*)(ws + mp.nruns_off);
    hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(1024), 0, st, ids, pairs, E, 16, sorted, (int*)nullptr, runs,
                       nruns);
    OC_HIP(hipGetLastError());
    g.sorted = sorted;
    g.runs = runs;
    g.nruns = nruns;
    const int bound = (pairs + 15) / 16 + (E < pairs ? E : pairs);
    groups = bound < pairs ? bound : pairs;
  }
  g.topk = topk;
  g.E = E;
  g.I = I;
  g.act = act;
  g.alpha = alpha;
  g.limit = limit;
  uint16_t* h = (uint16_t*)(ws + mp.h_off);
  // 1. gate | up and the activation (act-order: x gathered per pair in the expert's k order)
  fill(g.base, L13, H, 2 * I, gs13, G13);
  g.base.x = (const uint16_t*)x;
  g.xdiv = topk;
  if (perm13) {
    uint16_t* xp = (uint16_t*)(ws + mp.xp_off);
    hipLaunchKernelGGL(k_moe_gather_perm, dim3((H + 255) / 256, pairs), dim3(256), 0, st, (const uint16_t*)x, topk,
                       H, perm13, ids, E, xp);
    OC_HIP(hipGetLastError());
    g.base.x = xp;
    g.xdiv = 1;
  }
  g.base.w = (const uint8_t*)w13;
  g.base.meta = meta13;
  g.bias = (const uint16_t*)b13;
  g.out = h;
  g.part = nullptr;
  g.ntiles = I / 16;
  g.w_stride = w13_stride;
  g.meta_stride = meta13_stride;
  const int cs13 = (gs13 % 128) == 0 ? 4 : 1, cs2 = (gs2 % 128) == 0 ? 4 : 1;
  int rc = bf16 ? launch_moe<true, true>(g, bits, cs13, mp.w1, mp.rm, mp.lds1, groups * g.ntiles, st)
                : launch_moe<false, true>(g, bits, cs13, mp.w1, mp.rm, mp.lds1, groups * g.ntiles, st);
  if (rc) return rc;
  // 2. down per run, fp32 sums per pair (act-order: h gathered in the expert's k order)
  fill(g.base, L2, I, H, gs2, G2);
  g.base.x = h;
  if (perm2) {
    uint16_t* hp = (uint16_t*)(ws + mp.hp_off);
    hipLaunchKernelGGL(k_moe_gather_perm, dim3((I + 255) / 256, pairs), dim3(256), 0, st, (const uint16_t*)h, 1, I,
                       perm2, ids, E, hp);
    OC_HIP(hipGetLastError());
    g.base.x = hp;
  }
  g.base.w = (const uint8_t*)w2;
  g.base.meta = meta2;
  g.bias = nullptr;
  g.out = nullptr;
  g.ntiles = L2.NT;
  g.w_stride = w2_stride;
  g.meta_stride = meta2_stride;
  float* part = (float*)(ws + mp.part_off);
  g.part = part;
  rc = bf16 ? launch_moe<true, false>(g, bits, cs2, mp.w2, mp.rm, mp.lds2, groups * g.ntiles, st)
            : launch_moe<false, false>(g, bits, cs2, mp.w2, mp.rm, mp.lds2, groups * g.ntiles, st);
  if (rc) return rc;
  // 3. weighted sum over the top-k (+ down bias)
  const dim3 grid((H + 255) / 256, M);
  if (bf16)
    hipLaunchKernelGGL(k_moe_combine<true>, grid, dim3(256), 0, st, part, H, L2.N_pad, topk, M, ids, E, weights,
                       (const uint16_t*)b2, (uint16_t*)y);
  else
    hipLaunchKernelGGL(k_moe_combine<false>, grid, dim3(256), 0, st, part, H, L2.N_pad, topk, M, ids, E, weights,
                       (const uint16_t*)b2, (uint16_t*)y);
  OC_HIP(hipGetLastError());
  return 0;
}
