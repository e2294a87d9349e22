// DBF / MDBF sign-factor matmuls.
//
// A DBF layer (vllm_plugins/dbf/vllm_plugin.py:275-294) is
//     y = s4 * (S1 @ (s2 * (S2 @ (s0 * x))))
// with S2 (r x K) and S1 (N x r) +-1 matrices stored as uint8 bits, MSB first,
// flat row-major (onecomp/quantizer/dbf/dbf_layer.py:32-52).  An MDBF path
// (onecomp/quantizer/mdbf/mdbf_layer.py:307-344) has the same shape with
// per-rank envelopes.  Both reduce to one primitive, run twice:
//     out[m, n] = sum_terms post_t[n] * sum_k S_t[n, k] * (pre_t[k] * in_t[m, k])
//
// Sign layout ("lane-chunk" layout for signs): the signs of 16 output rows and
// 128 consecutive k form one word per lane of a wave: lane l owns row l % 16
// and the k-slices 8*(l/16) + [0, 8) of the four 32-deep MFMA steps.  Pair
// P = 4t + p (k = 32t + 8*(l/16) + 2p, +1) sits at bits 15-P (low) and 31-P
// (high), stored as 1 for -1, so ((w << P) & 0x80008000) | one_pair is the
// fp16/bf16 pair (+-1, +-1): one shift and one v_and_or_b32 per pair.  A unit
// is UK consecutive k-blocks; a lane's UK words are contiguous (16-byte loads
// for UK = 4).  Byte offset of (row-tile rt, unit u, lane l) =
//     ((rt * NU + u) * 64 + l) * 4 * UK.
#include <stdlib.h>

#include "gemm_core.h"
#include "oc_common.h"

namespace {

struct SignLayout {
  int R, Kd, UK, NU, RT, K_pad;
};

SignLayout make_sign_layout(int R, int Kd) {
  SignLayout L;
  L.R = R;
  L.Kd = Kd;
  const int kb = (Kd + 127) / 128;
  // the widest unit (16-byte lane loads) whose padding wastes at most ~4 %
  L.UK = 1;
  for (int uk : {4, 2}) {
    const int padded = (kb + uk - 1) / uk * uk;
    if ((padded - kb) * 100 <= 4 * kb) {
      L.UK = uk;
      break;
    }
  }
  L.NU = (kb + L.UK - 1) / L.UK;
  L.K_pad = L.NU * L.UK * 128;
  L.RT = (R + 15) / 16;
  return L;
}

size_t sign_layout_bytes(const SignLayout& L) { return (size_t)L.RT * L.NU * 64 * 4 * L.UK; }

__device__ __forceinline__ uint32_t ckpt_bit(const uint8_t* __restrict__ bp, size_t e) {
  return (bp[e >> 3] >> (7 - (e & 7))) & 1u;
}

__global__ void k_sign_repack(const uint8_t* __restrict__ bp, SignLayout L, uint32_t* __restrict__ out,
                              size_t n_words) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_words) return;
  const int w = (int)(idx % L.UK);
  size_t rest = idx / L.UK;
  const int lane = (int)(rest & 63);
  rest >>= 6;
  const int u = (int)(rest % L.NU);
  const int rt = (int)(rest / L.NU);
  const int row = rt * 16 + (lane & 15), kq = lane >> 4;
  const int kb = u * L.UK + w;
  uint32_t word = 0;
  for (int P = 0; P < 16; ++P) {
    const int t = P >> 2, p = P & 3;
    const int k0 = kb * 128 + 32 * t + 8 * kq + 2 * p;
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int k = k0 + hi;
      uint32_t neg = 0;
      if (row < L.R && k < L.Kd) neg = 1u - ckpt_bit(bp, (size_t)row * L.Kd + k);
      word |= neg << (hi ? 31 - P : 15 - P);
    }
  }
  out[idx] = word;
}

__global__ void k_sign_unpack(const uint8_t* __restrict__ bp, size_t numel, int8_t* __restrict__ out) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < numel) out[e] = ckpt_bit(bp, e) ? (int8_t)1 : (int8_t)-1;
}

// ---------------------------------------------------------------------------
// sign GEMV (M <= 16 rows per launch chunk)
// ---------------------------------------------------------------------------
constexpr int kMaxTerms = 4;

struct TermArgs {
  const uint32_t* sg;
  const uint16_t* in;
  const uint16_t* pre;
  const uint16_t* post;
  int ld_in, Kd, NU, UK;
};

struct SignArgs {
  TermArgs t[kMaxTerms];
  int unit_start[kMaxTerms + 1];  // prefix sums of NU over terms
  int n_terms;
  uint16_t* out;
  const uint16_t* bias;
  int ld_out, M, R, RT, fill_to;
};

template <bool BF16>
__device__ __forceinline__ uint32_t mul2(uint32_t a, uint32_t b) {
  if constexpr (BF16) {
    const float lo = oc_bf2f((uint16_t)(a & 0xFFFFu)) * oc_bf2f((uint16_t)(b & 0xFFFFu));
    const float hi = oc_bf2f((uint16_t)(a >> 16)) * oc_bf2f((uint16_t)(b >> 16));
    return (uint32_t)oc_f2bf(lo) | ((uint32_t)oc_f2bf(hi) << 16);
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(oc_half2, a) * __builtin_bit_cast(oc_half2, b));
  }
}

// One workgroup per 16-row output tile; W waves take the (term, unit) list
// round-robin, each keeping D units of sign words and pre-scaled x rows in
// flight.  All terms of a launch share the same UK.
template <int UK, int XCH, int D, int W, bool BF16>
__global__ __launch_bounds__(64 * W) void k_sign_gemv(const SignArgs a) {
  constexpr int XW = UK * 128 + 8;      // halfs per staged x row
  // XCH: 16-byte x chunks per lane per unit (M * UK / 4 rounded up)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rt = blockIdx.x;
  const int col = lane & 15, kq = lane >> 4;
  const int n = rt * 16 + col;
  const uint32_t one2 = oc_opaque(BF16 ? 0x3F803F80u : 0x3C003C00u);
  const uint32_t smask = oc_opaque(0x80008000u);

  extern __shared__ __align__(16) uint8_t smem[];
  if (rt * 16 >= a.R) {  // padding tiles: zero-fill up to fill_to
    for (int e = threadIdx.x; e < a.M * 16; e += 64 * W) {
      const int m = e >> 4, c = rt * 16 + (e & 15);
      if (c < a.fill_to) a.out[(size_t)m * a.ld_out + c] = 0;
    }
    return;
  }
  const int total = a.unit_start[a.n_terms];
  const int n_my = wave < total ? (total - wave + W - 1) / W : 0;

  // unit i of this wave -> (term, unit index inside the term)
  auto locate = [&](int i, int& term, int& u) {
    const int g = wave + W * i;
    term = 0;
#pragma unroll
    for (int q = 1; q < kMaxTerms; ++q)
      if (q < a.n_terms && g >= a.unit_start[q]) term = q;
    u = g - a.unit_start[term];
  };

  uint32_t sbuf[D][UK];
  oc_u4 xbuf[D][XCH], pbuf[D][XCH];
  int tbuf[D], ubuf[D];
  const uint32_t one1 = BF16 ? 0x3F803F80u : 0x3C003C00u;
  auto load_unit = [&](int i, uint32_t (&sb)[UK], oc_u4 (&xb)[XCH], oc_u4 (&pb)[XCH], int& tt, int& uu) {
    locate(i, tt, uu);
    const TermArgs& T = a.t[tt];
    const uint32_t* p = T.sg + (((size_t)rt * T.NU + uu) * 64 + lane) * UK;
    if constexpr (UK == 4) {
      const oc_u4 v = __builtin_nontemporal_load((const oc_u4*)p);
      sb[0] = v[0]; sb[1] = v[1]; sb[2] = v[2]; sb[3] = v[3];
    } else {
#pragma unroll
      for (int q = 0; q < UK; ++q) sb[q] = __builtin_nontemporal_load(p + q);
    }
    // x rows of this unit and their pre scales (applied when staged):
    // chunk c -> row c / (16 UK), k 8 * (c % (16 UK))
#pragma unroll
    for (int q = 0; q < XCH; ++q) {
      const int c = lane + 64 * q;
      const int m = c / (16 * UK), k = uu * UK * 128 + 8 * (c % (16 * UK));
      const bool ok = m < a.M && k < T.Kd;
      xb[q] = ok ? *(const oc_u4*)(T.in + (size_t)m * T.ld_in + k) : oc_u4{0u, 0u, 0u, 0u};
      pb[q] = (ok && T.pre) ? *(const oc_u4*)(T.pre + k) : oc_u4{one1, one1, one1, one1};
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < n_my) load_unit(d, sbuf[d], xbuf[d], pbuf[d], tbuf[d], ubuf[d]);

  uint16_t* xslot = (uint16_t*)smem + (size_t)wave * a.M * XW;
  const uint16_t* arow = xslot + min(col, a.M - 1) * XW + 8 * kq;
  oc_f4 accT[kMaxTerms];
#pragma unroll
  for (int q = 0; q < kMaxTerms; ++q) accT[q] = oc_f4{0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < n_my; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = i0 + d;
      if (i >= n_my) break;
      oc_wave_lds_barrier();
      const bool has_pre = a.t[tbuf[d]].pre != nullptr;
#pragma unroll
      for (int q = 0; q < XCH; ++q) {
        const int c = lane + 64 * q;
        oc_u4 v = xbuf[d][q];
        if (has_pre) {
#pragma unroll
          for (int h = 0; h < 4; ++h) v[h] = mul2<BF16>(v[h], pbuf[d][q][h]);
        }
        if (c < a.M * 16 * UK) *(oc_u4*)(xslot + (c / (16 * UK)) * XW + 8 * (c % (16 * UK))) = v;
      }
      oc_wave_lds_barrier();
      oc_f4 acc = oc_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kbl = 0; kbl < UK; ++kbl) {
        const uint32_t w = sbuf[d][kbl];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const oc_u4 av = *(const oc_u4*)(arow + kbl * 128 + 32 * t);
          const int P = 4 * t;
          const oc_u4 bv = oc_u4{((w << P) & smask) | one2, ((w << (P + 1)) & smask) | one2,
                                 ((w << (P + 2)) & smask) | one2, ((w << (P + 3)) & smask) | one2};
          acc = oc_mfma16<BF16>(av, bv, acc);
        }
      }
      const int tt = tbuf[d];
#pragma unroll
      for (int q = 0; q < kMaxTerms; ++q)
        if (q == tt) accT[q] += acc;
      if (i + D < n_my) load_unit(i + D, sbuf[d], xbuf[d], pbuf[d], tbuf[d], ubuf[d]);
    }
  }

  // post scales, then reduce the W waves
  oc_f4 y = oc_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < kMaxTerms; ++q) {
    if (q >= a.n_terms) break;
    float ps = 1.f;
    if (a.t[q].post && n < a.R) ps = BF16 ? oc_bf2f(a.t[q].post[n]) : oc_h2f(a.t[q].post[n]);
    y += ps * accT[q];
  }
  __syncthreads();
  float* red = (float*)smem;  // [W][4][64]
#pragma unroll
  for (int r = 0; r < 4; ++r) red[(wave * 4 + r) * 64 + lane] = y[r];
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 64 * W) {
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) v += red[ww * 256 + e];
    const int ln = e & 63, r = e >> 6;
    const int m = 4 * (ln >> 4) + r, c = rt * 16 + (ln & 15);
    if (m >= a.M || c >= a.fill_to) continue;
    if (c < a.R) {
      if (a.bias) v += BF16 ? oc_bf2f(a.bias[c]) : oc_h2f(a.bias[c]);
      a.out[(size_t)m * a.ld_out + c] = BF16 ? oc_f2bf(v) : oc_f2h(v);
    } else {
      a.out[(size_t)m * a.ld_out + c] = 0;
    }
  }
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

constexpr size_t kSignLds = 96 * 1024;

template <int UK, int XCH, bool BF16>
int launch_sign_x(const SignArgs& a, int rt_grid, int w, hipStream_t st) {
  constexpr int D = XCH >= 8 ? 1 : (XCH >= 4 ? 2 : (UK == 1 ? 8 : 4));
  const size_t slot = (size_t)a.M * (UK * 128 + 8) * 2;
  if (XCH > UK && w > 8) w = 8;  // keeps the wider x ring within 256 VGPRs
  while (w > 4 && slot * w > kSignLds) w /= 2;
  const size_t xb = slot * w;
  const size_t rb = (size_t)w * 4 * 64 * 4;
  const size_t lds = ((xb > rb ? xb : rb) + 15) / 16 * 16;
  if (w == 4)
    hipLaunchKernelGGL((k_sign_gemv<UK, XCH, D, 4, BF16>), dim3(rt_grid), dim3(256), lds, st, a);
  else if (XCH > UK || w == 8)
    hipLaunchKernelGGL((k_sign_gemv<UK, XCH, D, 8, BF16>), dim3(rt_grid), dim3(512), lds, st, a);
  else
    hipLaunchKernelGGL((k_sign_gemv<UK, UK, D, 16, BF16>), dim3(rt_grid), dim3(1024), lds, st, a);
  OC_HIP(hipGetLastError());
  return 0;
}

template <int UK, bool BF16>
int launch_sign(const SignArgs& a, int rt_grid, int w, hipStream_t st) {
  const int xc = (a.M * UK + 3) / 4;  // chunks per lane
  if (xc <= UK) return launch_sign_x<UK, UK, BF16>(a, rt_grid, w, st);
  return launch_sign_x<UK, 4 * UK, BF16>(a, rt_grid, w, st);
}

}  // namespace

extern "C" int oc_dbf_layout(int R, int Kd, size_t* packed_bytes, int* k_pad, int* unit_k) {
  OC_REQUIRE(R > 0 && Kd > 0, OC_ERR_INVALID, "R=%d and Kd=%d must be positive", R, Kd);
  const SignLayout L = make_sign_layout(R, Kd);
  if (packed_bytes) *packed_bytes = sign_layout_bytes(L);
  if (k_pad) *k_pad = L.K_pad;
  if (unit_k) *unit_k = L.UK;
  return 0;
}

extern "C" int oc_dbf_unpack_signs(const uint8_t* bp, int R, int Kd, int8_t* out, void* stream) {
  OC_REQUIRE(bp && out, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(R > 0 && Kd > 0, OC_ERR_INVALID, "R=%d and Kd=%d must be positive", R, Kd);
  const size_t numel = (size_t)R * Kd;
  hipLaunchKernelGGL(k_sign_unpack, dim3((unsigned)((numel + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     bp, numel, out);
  OC_HIP(hipGetLastError());
  return 0;
}

extern "C" int oc_dbf_prepare(const uint8_t* bp, int R, int Kd, void* packed, void* stream) {
  OC_REQUIRE(bp && packed, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(R > 0 && Kd > 0, OC_ERR_INVALID, "R=%d and Kd=%d must be positive", R, Kd);
  const SignLayout L = make_sign_layout(R, Kd);
  const size_t n_words = sign_layout_bytes(L) / 4;
  hipLaunchKernelGGL(k_sign_repack, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     bp, L, (uint32_t*)packed, n_words);
  OC_HIP(hipGetLastError());
  return 0;
}

namespace {

// ---------------------------------------------------------------------------
// M >= kSignGemmMinM: the shared large-M GEMM core with the sign decoder.
// A term with a pre scale first writes RNE(in * pre) (the reference's
// `x * scaling0.to(x.dtype)`) to the workspace; the MFMA B operand is then the
// exact +-1 pair.  One term: one k_gemm launch (+ fixup for a split tail).
// Several terms: one launch per term, every tile written as an fp32 partial
// (post-scaled) into its slot, then one fixup sums the slots and adds bias.
// ---------------------------------------------------------------------------
int sign_gemm_min_m() { return env_int("OC_SIGN_GEMM_MIN_M", 128); }

int round8(int v) { return (v + 7) / 8 * 8; }

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

template <bool BF16>
__global__ void k_prescale(const uint16_t* __restrict__ in, int ld_in, const uint16_t* __restrict__ pre, int Kd,
                           int ldx, uint16_t* __restrict__ xs) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (k >= ldx) return;
  uint16_t v = 0;
  if (k < Kd) {
    const uint16_t a = in[(size_t)m * ld_in + k], b = pre[k];
    v = BF16 ? oc_f2bf(oc_bf2f(a) * oc_bf2f(b)) : oc_f2h(oc_h2f(a) * oc_h2f(b));
  }
  xs[(size_t)m * ldx + k] = v;
}

__global__ void k_zero_cols(uint16_t* __restrict__ out, int ld_out, int c0, int c1) {
  const int c = c0 + threadIdx.x;
  if (c < c1) out[(size_t)blockIdx.x * ld_out + c] = 0;
}

struct SignGemmPlan {
  oc_gemm::GemmPlan gp;  // tiling of one term
  size_t xs_off[kMaxTerms], part_off, bytes;
};

SignGemmPlan plan_sign_gemm(const oc_sign_term* terms, int n_terms, int M, int R) {
  SignGemmPlan p;
  const SignLayout L = make_sign_layout(R, terms[0].Kd);
  // several terms are summed through partial slots: no K split inside a term
  p.gp = oc_gemm::plan_gemm(M, L.RT * 16, L.K_pad, n_terms > 1 ? 1 : env_int("OC_GEMM_SPLIT", 0));
  size_t off = 0;
  for (int i = 0; i < n_terms; ++i) {
    p.xs_off[i] = off;
    if (terms[i].pre) off += align256((size_t)M * round8(terms[i].Kd) * 2);
  }
  p.part_off = off;
  if (n_terms > 1)
    off += (size_t)p.gp.MB * p.gp.NB * n_terms * oc_gemm::kGemmBM * oc_gemm::kGemmBN * 4;
  else
    off += align256(p.gp.part_bytes);
  p.bytes = off;
  return p;
}

template <bool BF16>
void launch_sign_gemm_term(const oc_gemm::GemmArgs& g, int grid, hipStream_t st) {
  hipLaunchKernelGGL((oc_gemm::k_gemm<1, 4, BF16>), dim3(grid), dim3(256), 2 * oc_gemm::kGemmXBuf, st, g);
}

int sign_gemm_large(const oc_sign_term* terms, int n_terms, int M, int R, bool bf16, const void* bias,
                    void* out, int ld_out, int fill_to, void* workspace, size_t ws_bytes, hipStream_t st) {
  const SignGemmPlan p = plan_sign_gemm(terms, n_terms, M, R);
  OC_REQUIRE(ws_bytes >= p.bytes && (p.bytes == 0 || workspace), OC_ERR_WORKSPACE,
             "workspace of %zu bytes is smaller than the %zu required", ws_bytes, p.bytes);
  uint8_t* ws = (uint8_t*)workspace;
  for (int i = 0; i < n_terms; ++i) {
    const oc_sign_term& T = terms[i];
    const SignLayout L = make_sign_layout(R, T.Kd);
    oc_gemm::GemmArgs g = {};
    g.w = (const uint8_t*)T.packed;
    g.post = (const uint16_t*)T.post;
    g.y = (uint16_t*)out;
    g.part = (float*)(ws + p.part_off);
    g.M = M;
    g.K = T.Kd;
    g.N = R;
    g.N_pad = L.RT * 16;
    g.NT_total = L.RT;
    g.NU = L.NU;
    g.G = 1;
    g.gs = L.K_pad;
    g.gshift = -1;
    g.NKB = L.K_pad / 128;
    g.MB = p.gp.MB;
    g.NB = p.gp.NB;
    g.ldy = ld_out;
    g.uk_shift = L.UK == 4 ? 2 : (L.UK == 2 ? 1 : 0);
    if (T.pre) {
      const int ldx = round8(T.Kd);
      uint16_t* xs = (uint16_t*)(ws + p.xs_off[i]);
      const dim3 pg((ldx + 255) / 256, M);
      if (bf16)
        hipLaunchKernelGGL(k_prescale<true>, pg, dim3(256), 0, st, (const uint16_t*)T.in, T.ld_in,
                           (const uint16_t*)T.pre, T.Kd, ldx, xs);
      else
        hipLaunchKernelGGL(k_prescale<false>, pg, dim3(256), 0, st, (const uint16_t*)T.in, T.ld_in,
                           (const uint16_t*)T.pre, T.Kd, ldx, xs);
      OC_HIP(hipGetLastError());
      g.x = xs;
      g.ldx = ldx;
    } else {
      g.x = (const uint16_t*)T.in;
      g.ldx = T.ld_in;
    }
    if (n_terms == 1) {
      g.bias = (const uint16_t*)bias;
      g.tiles_main = p.gp.tiles_main;
      g.S = p.gp.S;
      g.kper = p.gp.kper;
      g.pstride = p.gp.S;
      g.poff = 0;
    } else {  // every tile is one partial slot of this term
      g.bias = nullptr;
      g.tiles_main = 0;
      g.S = 1;
      g.kper = g.NKB;
      g.pstride = n_terms;
      g.poff = i;
    }
    const int grid = n_terms == 1 ? p.gp.tiles_main + p.gp.split_tiles * p.gp.S : p.gp.MB * p.gp.NB;
    if (bf16) launch_sign_gemm_term<true>(g, grid, st);
    else launch_sign_gemm_term<false>(g, grid, st);
    OC_HIP(hipGetLastError());
    if (i == n_terms - 1) {
      const int fix_tiles = n_terms == 1 ? p.gp.split_tiles : p.gp.MB * p.gp.NB;
      if (fix_tiles > 0) {
        g.bias = (const uint16_t*)bias;
        g.tiles_main = n_terms == 1 ? p.gp.tiles_main : 0;
        g.pstride = n_terms == 1 ? p.gp.S : n_terms;
        const dim3 fg(oc_gemm::kGemmBM * oc_gemm::kGemmBN / 256, fix_tiles);
        if (bf16) hipLaunchKernelGGL(oc_gemm::k_gemm_fixup<true>, fg, dim3(256), 0, st, g);
        else hipLaunchKernelGGL(oc_gemm::k_gemm_fixup<false>, fg, dim3(256), 0, st, g);
        OC_HIP(hipGetLastError());
      }
    }
  }
  if (fill_to > R) {
    hipLaunchKernelGGL(k_zero_cols, dim3(M), dim3(64), 0, st, (uint16_t*)out, ld_out, R, fill_to);
    OC_HIP(hipGetLastError());
  }
  return 0;
}

}  // namespace

extern "C" size_t oc_sign_workspace_bytes(const oc_sign_term* terms, int n_terms, int M, int R) {
  if (!terms || n_terms < 1 || n_terms > kMaxTerms || M < sign_gemm_min_m() || R <= 0) return 0;
  for (int i = 0; i < n_terms; ++i)
    if (terms[i].Kd <= 0) return 0;
  return plan_sign_gemm(terms, n_terms, M, R).bytes;
}

extern "C" int oc_sign_gemm(const oc_sign_term* terms, int n_terms, int M, int R, int act_dtype,
                            const void* bias, void* out, int ld_out, int fill_to, void* workspace,
                            size_t ws_bytes, void* stream) {
  OC_REQUIRE(terms && out, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(n_terms >= 1 && n_terms <= kMaxTerms, OC_ERR_UNSUPPORTED, "n_terms=%d must be 1..%d", n_terms,
             kMaxTerms);
  OC_REQUIRE(M >= 0 && R > 0, OC_ERR_INVALID, "bad M=%d R=%d", M, R);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d",
             act_dtype);
  if (fill_to < R) fill_to = R;
  OC_REQUIRE(ld_out >= fill_to, OC_ERR_SHAPE, "ld_out=%d < fill_to=%d", ld_out, fill_to);
  if (M == 0) return 0;
  SignArgs a;
  int uk = 0, start = 0;
  for (int i = 0; i < n_terms; ++i) {
    const oc_sign_term& T = terms[i];
    OC_REQUIRE(T.packed && T.in, OC_ERR_INVALID, "term %d: null pointer", i);
    OC_REQUIRE(T.Kd > 0 && T.ld_in >= T.Kd && T.ld_in % 8 == 0, OC_ERR_SHAPE,
               "term %d: Kd=%d / ld_in=%d (ld_in must be >= Kd and a multiple of 8)", i, T.Kd, T.ld_in);
    const SignLayout L = make_sign_layout(R, T.Kd);
    OC_REQUIRE(uk == 0 || uk == L.UK, OC_ERR_UNSUPPORTED, "terms of one call need the same unit size");
    uk = L.UK;
    a.t[i].sg = (const uint32_t*)T.packed;
    a.t[i].in = (const uint16_t*)T.in;
    a.t[i].pre = (const uint16_t*)T.pre;
    a.t[i].post = (const uint16_t*)T.post;
    a.t[i].ld_in = T.ld_in;
    a.t[i].Kd = T.Kd;
    a.t[i].NU = L.NU;
    a.t[i].UK = L.UK;
    a.unit_start[i] = start;
    start += L.NU;
  }
  for (int i = n_terms; i <= kMaxTerms; ++i) a.unit_start[i] = start;
  if (M >= sign_gemm_min_m())
    return sign_gemm_large(terms, n_terms, M, R, act_dtype == OC_DTYPE_BF16, bias, out, ld_out, fill_to,
                           workspace, ws_bytes, (hipStream_t)stream);
  a.n_terms = n_terms;
  a.bias = (const uint16_t*)bias;
  a.R = R;
  a.RT = (R + 15) / 16;
  a.fill_to = fill_to;
  a.ld_out = ld_out;
  const int rt_grid = (fill_to + 15) / 16;
  int w = env_int("OC_SIGN_W", 0);
  if (w != 4 && w != 8 && w != 16) w = a.RT >= 512 ? 8 : 16;
  hipStream_t st = (hipStream_t)stream;
  const bool bf16 = act_dtype == OC_DTYPE_BF16;
  for (int m0 = 0; m0 < M; m0 += 16) {
    SignArgs c = a;
    c.M = M - m0 < 16 ? M - m0 : 16;
    c.out = (uint16_t*)out + (size_t)m0 * ld_out;
    for (int i = 0; i < n_terms; ++i) c.t[i].in = a.t[i].in + (size_t)m0 * a.t[i].ld_in;
    int rc;
    if (uk == 4)
      rc = bf16 ? launch_sign<4, true>(c, rt_grid, w, st) : launch_sign<4, false>(c, rt_grid, w, st);
    else if (uk == 2)
      rc = bf16 ? launch_sign<2, true>(c, rt_grid, w, st) : launch_sign<2, false>(c, rt_grid, w, st);
    else
      rc = bf16 ? launch_sign<1, true>(c, rt_grid, w, st) : launch_sign<1, false>(c, rt_grid, w, st);
    if (rc) return rc;
  }
  return 0;
}
