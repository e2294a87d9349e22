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
// sign GEMV (M <= 16)
// ---------------------------------------------------------------------------
constexpr int kMaxTerms = 4;
constexpr int kSignGemvMaxM = 16;

struct TermArgs {
  const uint32_t* sg;
  const uint16_t* in;
  const uint16_t* pre;
  const uint16_t* post;
  int ld_in, Kd, NU, UK;
};

struct SignArgs {
  TermArgs t[kMaxTerms];
  int n_terms;
  // outs[0]; a batch of independent problems (term p into outs[p], no bias) runs p = blockIdx.y
  uint16_t* outs[kMaxTerms];
  const uint16_t* bias;
  int ld_out, M, R, RT, fill_to, W;
  int batch;  // problems (grid.y; 1 unless batched)
};

// element t of a per-term argument array (t uniform; a compare chain, not a
// dynamic index into the kernel arguments)
template <class V>
__device__ __forceinline__ V term_pick(int t, const V (&v)[kMaxTerms]) {
  return t == 0 ? v[0] : (t == 1 ? v[1] : (t == 2 ? v[2] : v[3]));
}

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

// One workgroup per 16-row output tile; its W waves split each term's units
// (u = wave, wave + W, ...) and keep D units in flight: the sign words, the
// M x 128 UK slice of the input rows (XCH 16-byte chunks per lane) and, with
// PRE, the lane's pre-scale chunk.  Every load is unconditional (invalid
// chunks read a valid address and are zeroed after arrival), so the loads of
// the next D - 1 units stay in flight while one unit is consumed.  The input
// slice is multiplied by the pre scale (RNE to the activation dtype, as the
// reference's `x * scaling0.to(x.dtype)`), bounced through a wave-private LDS
// slot to form the A operand, and multiplied by the +-1 pairs decoded from
// the sign words.  Terms are processed one after another (the pipeline
// drains between them); each term's fp32 sums are multiplied by its per-row
// post scale, then the W waves are reduced in LDS.
//
// Input contract: in[m, k] for Kd <= k < round8(Kd) is finite, and zero
// unless the term has a (zero-padded) pre scale.
template <int UK, int XCH, bool PRE, bool MULTI, bool BF16>
__global__ __launch_bounds__(MULTI ? 512 : 1024) void k_sign_gemv(const SignArgs a) {
  constexpr int XW = UK * 128 + 8;  // halfs per staged x row
  constexpr int CPR = 16 * UK;      // 16-byte chunks per row and unit
  constexpr int VPU = UK + 4 * XCH + (PRE ? 4 : 0);
  constexpr int D = VPU <= 8 ? 8 : (VPU <= 16 ? 4 : (VPU <= 32 ? 2 : 1));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = a.W;
  const int rt = blockIdx.x;
  const int col = lane & 15, kq = lane >> 4;
  const int n = rt * 16 + col;
  const uint32_t one2 = oc_opaque(BF16 ? 0x3F803F80u : 0x3C003C00u);
  const uint32_t smask = oc_opaque(0x80008000u);
  const int M = a.M;
  // problem of a batched launch (single-term kernels only; 0 otherwise) and its output
  const int pb = MULTI ? 0 : blockIdx.y;
  // field by field with constant indices (a dynamic index into the argument structs would copy
  // them to scratch)
  TermArgs T0;
#define OC_TF(f) (pb == 0 ? a.t[0].f : (pb == 1 ? a.t[1].f : (pb == 2 ? a.t[2].f : a.t[3].f)))
  T0.sg = OC_TF(sg);
  T0.in = OC_TF(in);
  T0.pre = OC_TF(pre);
  T0.post = OC_TF(post);
  T0.ld_in = OC_TF(ld_in);
  T0.Kd = OC_TF(Kd);
  T0.NU = OC_TF(NU);
  T0.UK = OC_TF(UK);
#undef OC_TF
  uint16_t* const out = term_pick(pb, a.outs);

  extern __shared__ __align__(16) uint8_t smem[];
  if (rt * 16 >= a.R) {  // padding tiles: zero-fill up to fill_to
    for (int e = threadIdx.x; e < M * 16; e += 64 * W) {
      const int m = e >> 4, c = rt * 16 + (e & 15);
      if (c < a.fill_to) out[(size_t)m * a.ld_out + c] = 0;
    }
    return;
  }
  uint16_t* xslot = (uint16_t*)smem + (size_t)wave * M * XW;
  const uint16_t* arow = xslot + min(col, M - 1) * XW + 8 * kq;
  // chunk q of this lane: row xm[q], k offset (inside the unit) xk (the same
  // for every q because 64 is a multiple of CPR)
  const int xk = 8 * (lane % CPR);
  int xm[XCH];
#pragma unroll
  for (int q = 0; q < XCH; ++q) xm[q] = (lane + 64 * q) / CPR;

  // Post scales of every term and the bias of this thread's output column are
  // loaded up front (buffer loads: an absent vector reads zero at an offset
  // past the descriptor) and converted where they are used, so that their
  // latency hides behind the sign loads.
  uint16_t praw[kMaxTerms];
#pragma unroll
  for (int q = 0; q < (MULTI ? kMaxTerms : 1); ++q) {
    const uint16_t* post_q = q == 0 ? T0.post : (q < a.n_terms ? a.t[q].post : nullptr);
    const bool ok = q < a.n_terms && post_q != nullptr && n < a.R;
    praw[q] = __builtin_amdgcn_raw_buffer_load_b16(oc_rsrc(post_q, (uint32_t)a.R * 2),
                                                   ok ? (uint32_t)n * 2 : kOcOob, 0, 0);
  }
  const int ecol = rt * 16 + (threadIdx.x & 15);
  const uint16_t braw = __builtin_amdgcn_raw_buffer_load_b16(
      oc_rsrc(a.bias, (uint32_t)a.R * 2), (a.bias && ecol < a.R) ? (uint32_t)ecol * 2 : kOcOob, 0, 0);

  oc_f4 y = oc_f4{0.f, 0.f, 0.f, 0.f};
  // MULTI: several terms one after another (the pipeline drains between
  // them); a single term is compiled without the loop (exact load waits).
  for (int t = 0; t < (MULTI ? a.n_terms : 1); ++t) {
    const TermArgs T = (MULTI && t > 0) ? a.t[t] : T0;
    const int n_my = wave < T.NU ? (T.NU - wave + W - 1) / W : 0;
    uint32_t sbuf[D][UK];
    oc_u4 xbuf[D][XCH];
    oc_u4 pbuf[D][1];
    // Buffer loads: input chunks at k >= Kd or rows >= M read zero (offset
    // past the end of the descriptor, no memory access).
    const __amdgpu_buffer_rsrc_t sr =
        oc_rsrc(T.sg + (size_t)rt * T.NU * 64 * UK, (uint32_t)T.NU * 64 * UK * 4);
    const __amdgpu_buffer_rsrc_t xr = oc_rsrc(T.in, (uint32_t)M * T.ld_in * 2);
    const __amdgpu_buffer_rsrc_t pr = oc_rsrc(T.pre, (uint32_t)((T.Kd + 7) / 8 * 8) * 2);
    auto load_unit = [&](int i, uint32_t (&sb)[UK], oc_u4 (&xb)[XCH], oc_u4 (&pb)[1]) {
      const int u = wave + W * i;
      const uint32_t so = (uint32_t)(u * 64 + lane) * UK * 4;
      if constexpr (UK == 4) {
        const oc_u4 v = oc_bload16_nt(sr, so);
        sb[0] = v[0]; sb[1] = v[1]; sb[2] = v[2]; sb[3] = v[3];
      } else if constexpr (UK == 2) {
        typedef uint32_t u2v __attribute__((ext_vector_type(2)));
        const u2v v = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(sr, so, 0, 2));
        sb[0] = v[0]; sb[1] = v[1];
      } else {
        sb[0] = __builtin_amdgcn_raw_buffer_load_b32(sr, so, 0, 2);
      }
      const int k = u * UK * 128 + xk;
      const bool kok = k < T.Kd;
#pragma unroll
      for (int q = 0; q < XCH; ++q)
        xb[q] = oc_bload16(xr, kok && xm[q] < M ? (uint32_t)(xm[q] * T.ld_in + k) * 2 : kOcOob);
      if constexpr (PRE) pb[0] = oc_bload16(pr, kok ? (uint32_t)k * 2 : kOcOob);
    };
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < n_my) load_unit(d, sbuf[d], xbuf[d], pbuf[d]);

    oc_f4 acc = oc_f4{0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < n_my; i0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int i = i0 + d;
        if (i >= n_my) break;
        // Lanes read what other lanes of the same wave wrote: the compiler
        // barriers order the exchange (a wave's DS operations run in order).
        oc_wave_lds_barrier();
#pragma unroll
        for (int q = 0; q < XCH; ++q) {
          oc_u4 v = xbuf[d][q];
          if constexpr (PRE) {
#pragma unroll
            for (int h = 0; h < 4; ++h) v[h] = mul2<BF16>(v[h], pbuf[d][0][h]);
          }
          if (xm[q] < M) *(oc_u4*)(xslot + xm[q] * XW + xk) = v;
        }
        oc_wave_lds_barrier();
#pragma unroll
        for (int kbl = 0; kbl < UK; ++kbl) {
          const uint32_t w = sbuf[d][kbl];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const oc_u4 av = *(const oc_u4*)(arow + kbl * 128 + 32 * s);
            const int P = 4 * s;
            const oc_u4 bv = oc_u4{((w << P) & smask) | one2, ((w << (P + 1)) & smask) | one2,
                                   ((w << (P + 2)) & smask) | one2, ((w << (P + 3)) & smask) | one2};
            acc = oc_mfma16<BF16>(av, bv, acc);
          }
        }
        if (i + D < n_my) load_unit(i + D, sbuf[d], xbuf[d], pbuf[d]);
      }
    }
    uint16_t pr16 = praw[0];
#pragma unroll
    for (int q = 1; q < (MULTI ? kMaxTerms : 1); ++q)
      if (q == t) pr16 = praw[q];
    const float ps = (T.post && n < a.R) ? (BF16 ? oc_bf2f(pr16) : oc_h2f(pr16)) : 1.f;
    y += ps * acc;
  }

  // reduce the W waves
  __syncthreads();  // x slots no longer needed: reuse LDS
  float* red = (float*)smem;  // [W][4][64]
#pragma unroll
  for (int r = 0; r < 4; ++r) red[(wave * 4 + r) * 64 + lane] = y[r];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int e = threadIdx.x;
    const float bval = BF16 ? oc_bf2f(braw) : oc_h2f(braw);
    float v = 0.f;
    for (int ww = 0; ww < W; ++ww) v += red[ww * 256 + e];
    const int ln = e & 63, r = e >> 6;
    const int m = 4 * (ln >> 4) + r, c = rt * 16 + (ln & 15);
    if (m < M && c < a.fill_to)
      out[(size_t)m * a.ld_out + c] = c < a.R ? (BF16 ? oc_f2bf(v + bval) : oc_f2h(v + bval)) : (uint16_t)0;
  }
}


constexpr size_t kSignLds = 64 * 1024;

// Waves per workgroup (4, 8 or 16): enough waves in total to cover the GPU
// (the rank-side stage has few row tiles), no more than the units allow, and
// an LDS x slot per wave.
int sign_waves(int RT, int NU, int M, int UK, bool multi) {
  const int e = oc::knob("OC_SIGN_W", 0);
  int w = (e == 4 || e == 8 || e == 16) ? e : (RT >= 768 ? 4 : (RT >= 384 ? 8 : 16));
  while (w > 4 && w > NU) w /= 2;
  // several terms: at most 8 waves (the kernel's 512-thread bound leaves it 256 registers, where
  // 1024 threads' 128 made it spill)
  if (multi && w > 8) w = 8;
  const size_t slot = (size_t)M * (UK * 128 + 8) * 2;
  while (w > 4 && slot * w > kSignLds) w /= 2;
  return w;
}

template <int UK, int XCH, bool BF16>
int launch_sign_x(const SignArgs& a, bool pre, int rt_grid, hipStream_t st) {
  const size_t slot = (size_t)a.M * (UK * 128 + 8) * 2;
  const size_t xb = slot * a.W;
  const size_t rb = (size_t)a.W * 4 * 64 * 4;
  const size_t lds = ((xb > rb ? xb : rb) + 15) / 16 * 16;
  const dim3 g(rt_grid, a.batch > 1 ? a.batch : 1), b(64 * a.W);
  if (a.n_terms > 1) {
    if (pre) hipLaunchKernelGGL((k_sign_gemv<UK, XCH, true, true, BF16>), g, b, lds, st, a);
    else hipLaunchKernelGGL((k_sign_gemv<UK, XCH, false, true, BF16>), g, b, lds, st, a);
  } else {
    if (pre) hipLaunchKernelGGL((k_sign_gemv<UK, XCH, true, false, BF16>), g, b, lds, st, a);
    else hipLaunchKernelGGL((k_sign_gemv<UK, XCH, false, false, BF16>), g, b, lds, st, a);
  }
  OC_HIP(hipGetLastError());
  return 0;
}

// XCH = 16-byte input chunks per lane and unit: M * 16 UK chunks over 64 lanes.
template <int UK, bool BF16>
int launch_sign(const SignArgs& a, bool pre, int rt_grid, hipStream_t st) {
  const int xc = (a.M * UK + 3) / 4;
  if (xc <= 1) return launch_sign_x<UK, 1, BF16>(a, pre, rt_grid, st);
  if (xc <= 2) return launch_sign_x<UK, 2, BF16>(a, pre, rt_grid, st);
  if (xc <= 4) return launch_sign_x<UK, 4, BF16>(a, pre, rt_grid, st);
  if constexpr (UK >= 2) {
    if (xc <= 8) return launch_sign_x<UK, 8, BF16>(a, pre, rt_grid, st);
  }
  if constexpr (UK == 4) {
    if (xc <= 16) return launch_sign_x<UK, 16, BF16>(a, pre, rt_grid, st);
  }
  return oc::set_error(OC_ERR_UNSUPPORTED, "no sign GEMV for M=%d UK=%d", a.M, UK);
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
// M > 16: the shared GEMM core with the sign decoder, 64 MT x 256 tiles.
// A term with a pre scale first writes RNE(in * pre) (the reference's
// `x * scaling0.to(x.dtype)`) to the workspace; the MFMA B operand is then the
// exact +-1 pair.  One term: one k_gemm launch (+ fixup for a split tail).
// Several terms: one launch per term, every tile written as an fp32 partial
// (post-scaled) into its slot, then one fixup sums the slots and adds bias.
// ---------------------------------------------------------------------------
int sign_gemm_min_m() { return oc::knob("OC_SIGN_GEMM_MIN_M", kSignGemvMaxM + 1); }

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

// Several terms' inputs side by side: xs[m, off[t] + k] = RNE(in_t[m, k] * pre_t[k]) (in_t[m, k]
// without a pre scale) for k < Kd_t, 0 for Kd_t <= k < off[t + 1] - off[t].
struct PrescaleTerms {
  const uint16_t* in[4];
  const uint16_t* pre[4];
  int ld_in[4], Kd[4], off[5];
  int n_terms, ldx;
};

template <bool BF16>
__global__ void k_prescale_terms(const PrescaleTerms p, uint16_t* __restrict__ xs) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (c >= p.ldx) return;
  const int t = (c >= p.off[1]) + (c >= p.off[2]) + (c >= p.off[3]);
  const int k = c - (t == 0 ? p.off[0] : (t == 1 ? p.off[1] : (t == 2 ? p.off[2] : p.off[3])));
  const uint16_t* in = t == 0 ? p.in[0] : (t == 1 ? p.in[1] : (t == 2 ? p.in[2] : p.in[3]));
  const uint16_t* pre = t == 0 ? p.pre[0] : (t == 1 ? p.pre[1] : (t == 2 ? p.pre[2] : p.pre[3]));
  const int ld = t == 0 ? p.ld_in[0] : (t == 1 ? p.ld_in[1] : (t == 2 ? p.ld_in[2] : p.ld_in[3]));
  const int kd = t == 0 ? p.Kd[0] : (t == 1 ? p.Kd[1] : (t == 2 ? p.Kd[2] : p.Kd[3]));
  uint16_t v = 0;
  if (k < kd) {
    v = in[(size_t)m * ld + k];
    if (pre) v = BF16 ? oc_f2bf(oc_bf2f(v) * oc_bf2f(pre[k])) : oc_f2h(oc_h2f(v) * oc_h2f(pre[k]));
  }
  xs[(size_t)m * p.ldx + c] = v;
}

__global__ void k_zero_cols(uint16_t* __restrict__ out, int ld_out, int c0, int c1) {
  const int c = c0 + threadIdx.x;
  if (c < c1) out[(size_t)blockIdx.x * ld_out + c] = 0;
}

// ---------------------------------------------------------------------------
// 13 <= M <= 64: one wave per 16-row output tile streams its share of a term's
// k-blocks; the workgroup's 4 waves (4 consecutive tiles) share x, staged in a
// two-buffer LDS ring (KPS = 2 k-blocks per buffer and barrier up to 32 rows,
// 1 at 64) with the pre scale applied on the way (RNE(in * pre), the
// reference's rounding), so no separate scaling launch and no 64-row padding.
// Each +-1 B operand decoded from a sign word feeds MB = ceil(M / 16) MFMAs.
// Latency: a wave's step is a few hundred cycles and there are few waves per
// SIMD, so the loads run far ahead in registers: the sign words 12 k-blocks
// (whole units of UK words, one 4/8/16-byte load per lane), the x and
// pre-scale chunks XL = 4 k-blocks (2 at 64 rows; a register ring: the LDS
// store of a k-block waits only for a load issued XL k-blocks earlier).  The
// loop is unrolled over a period of 12 k-blocks so that every ring index is a
// constant; a split's last partial period runs guarded.  The barrier waits
// for LDS traffic only (no wait for the prefetches).
// blockIdx.y = term * S + split: rows too few to fill the GPU split each
// term's units S ways, and several terms (MDBF's paths) run side by side;
// with T S > 1 each (term, split) writes its post-scaled fp32 sums to
// partial[term S + split][m][n] and k_sign_reduce adds them in that order.
// ---------------------------------------------------------------------------
constexpr int kSignStreamMaxM = 64;
// from 13 rows (one 16-row block) the streaming kernel beats the GEMV at config 3 (M = 16: DBF
// down 21.1 -> 19.5 us, MDBF down 41.6 -> 33.3); at M = 8 the GEMV is faster (16.8 vs 19.1)
constexpr int kSignStreamMinM = 13;

struct SignStreamArgs {
  // per term (T of them): sign layout, input [M, ld_in], pre scale [round8(Kd)] zero-padded (all
  // terms or none), post scale [R] or null (scale 1), Kd and units
  const uint32_t* sg[kMaxTerms];
  const uint16_t* in[kMaxTerms];
  const uint16_t* pre[kMaxTerms];
  const uint16_t* post[kMaxTerms];
  int ld_in[kMaxTerms], Kd[kMaxTerms], NU[kMaxTerms];
  const uint16_t* bias;   // [R] or null (one output, T S == 1 only)
  // summed (separate = 0): every term into outs[0]; separate = 1: term t into outs[t] (a batch of
  // independent problems, no bias)
  uint16_t* outs[kMaxTerms];
  float* partial;         // [T S, M, N_pad] when the outputs take more than one partial
  int ld_out, M, R, RT, S, T, fill_to, N_pad, separate;
  int mz;  // row blocks across workgroups (grid.z; host only)
};


template <int MB, int UK, int KPS, bool PRE, bool BF16>
__global__ __launch_bounds__(256, 2) void k_sign_stream(const SignStreamArgs a) {
  constexpr int XLD = KPS * 128 + 8, ROWS = 16 * MB;
  constexpr int XL = MB == 4 ? 2 : 4;  // x k-blocks in flight (2 at 64 rows: registers)
  constexpr int DU = 12 / UK;     // sign units in flight
  constexpr int PER = DU * UK;    // unroll period (k-blocks)
  constexpr int CPP = PER / KPS;  // steps per period
  static_assert(PER % XL == 0 && PER % KPS == 0 && CPP % 2 == 0 && XL % KPS == 0,
                "ring indices must repeat every period");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kq = lane >> 4;
  const int rt = blockIdx.x * 4 + wave;
  const int rtc = min(rt, a.RT - 1);  // waves past the last tile compute the last one, unused
  // blockIdx.y = term t * S + split: each term's units are cut into S splits
  const int t = blockIdx.y / a.S, split = blockIdx.y - t * a.S;
  const uint32_t* sg = term_pick(t, a.sg);
  const uint16_t* in = term_pick(t, a.in);
  const uint16_t* pre = term_pick(t, a.pre);
  const uint16_t* post = term_pick(t, a.post);
  const int ld_in = term_pick(t, a.ld_in), Kd = term_pick(t, a.Kd), NU = term_pick(t, a.NU);
  const int ups = (NU + a.S - 1) / a.S;
  const int u0 = split * ups, u1 = min(u0 + ups, NU);
  const int kb0 = u0 * UK, kb1 = u1 * UK;
  // rows of this workgroup: blockIdx.z's block of 16 MB rows (one block unless the rows are split
  // across workgroups as well)
  const int m0 = blockIdx.z * 16 * MB;
  const int M = min(a.M - m0, 16 * MB);
  const uint32_t one2 = oc_opaque(BF16 ? 0x3F803F80u : 0x3C003C00u);
  const uint32_t smask = oc_opaque(0x80008000u);

  extern __shared__ __align__(16) uint16_t xl[];  // [2][ROWS][XLD]: KPS k-blocks per buffer
  // x of k-block kb: thread t owns chunks c = t + 256 j (row c / 16, 8 k at
  // 8 (c % 16)); chunks at k >= Kd, rows >= M and k-blocks past the split read
  // zero (offsets past the descriptors, no memory access)
  const __amdgpu_buffer_rsrc_t xr = oc_rsrc(in + (size_t)m0 * ld_in, (uint32_t)M * ld_in * 2);
  const __amdgpu_buffer_rsrc_t pr = oc_rsrc(pre, (uint32_t)((Kd + 7) / 8 * 8) * 2);
  const int ck = 8 * (threadIdx.x & 15);
  oc_u4 xq[XL][MB], pq[XL];  // slot j % XL: x (and pre) of k-block j of the period
  auto x_load = [&](int kb, oc_u4 (&xs)[MB], oc_u4& ps) {
    const int k = kb * 128 + ck;
    const bool kok = (k < Kd) & (kb < kb1);
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int row = (threadIdx.x + 256 * j) >> 4;
      xs[j] = oc_bload16(xr, (kok & (row < M)) ? (uint32_t)(row * ld_in + k) * 2 : kOcOob);
    }
    if constexpr (PRE) ps = oc_bload16(pr, kok ? (uint32_t)k * 2 : kOcOob);
  };
  // k-block kk of a step's KPS into LDS buffer buf
  auto x_store = [&](int buf, int kk, const oc_u4 (&xs)[MB], const oc_u4& ps) {
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int row = (threadIdx.x + 256 * j) >> 4;
      oc_u4 v = xs[j];
      if constexpr (PRE) {
#pragma unroll
        for (int h = 0; h < 4; ++h) v[h] = mul2<BF16>(v[h], ps[h]);
      }
      *(oc_u4*)(xl + (buf * ROWS + row) * XLD + kk * 128 + ck) = v;
    }
  };
  // sign words of unit u for this lane: words (rt, u, lane, 0 .. UK-1) of the layout
  const __amdgpu_buffer_rsrc_t sr = oc_rsrc(sg + (size_t)rtc * NU * 64 * UK, (uint32_t)NU * 64 * UK * 4);
  uint32_t sw[DU][UK];
  auto s_load = [&](int u, uint32_t (&sb)[UK]) {
    const uint32_t so = u < u1 ? (uint32_t)(u * 64 + lane) * UK * 4 : kOcOob;  // past the split: zero
    if constexpr (UK == 4) {
      const oc_u4 v = oc_bload16_nt(sr, so);
      sb[0] = v[0]; sb[1] = v[1]; sb[2] = v[2]; sb[3] = v[3];
    } else if constexpr (UK == 2) {
      typedef uint32_t u2v __attribute__((ext_vector_type(2)));
      const u2v v = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(sr, so, 0, 2));
      sb[0] = v[0]; sb[1] = v[1];
    } else {
      sb[0] = __builtin_amdgcn_raw_buffer_load_b32(sr, so, 0, 2);
    }
  };

  oc_f4 yacc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) yacc[i] = oc_f4{0.f, 0.f, 0.f, 0.f};
  // step c of a period (a constant after unrolling) consumes k-blocks kb .. kb + KPS - 1 (the
  // period's KPS c ..) from LDS buffer c & 1
  auto step = [&](int kb, int c) {
    // all of the step's A fragments first (one LDS latency per step, not one per MFMA)
    oc_u4 av[KPS][4][MB];
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < MB; ++i)
          av[kk][s][i] = *(const oc_u4*)(xl + ((c & 1) * ROWS + 16 * i + col) * XLD + kk * 128 + 32 * s + 8 * kq);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk) {
      const int d = KPS * c + kk;
      const uint32_t w = sw[d / UK][d % UK];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int P = 4 * s;
        const oc_u4 bv = oc_u4{((w << P) & smask) | one2, ((w << (P + 1)) & smask) | one2,
                               ((w << (P + 2)) & smask) | one2, ((w << (P + 3)) & smask) | one2};
#pragma unroll
        for (int i = 0; i < MB; ++i) yacc[i] = oc_mfma16<BF16>(av[kk][s][i], bv, yacc[i]);
      }
    }
    // x of the next step's k-blocks into the other buffer (last read by the
    // previous step), then their ring slots take the k-blocks XL later
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk) {
      const int nx = (KPS * (c + 1) + kk) % XL;
      x_store((c + 1) & 1, kk, xq[nx], pq[nx]);
      x_load(kb + KPS + kk + XL, xq[nx], pq[nx]);
    }
#pragma unroll
    for (int kk = 0; kk < KPS; ++kk) {
      const int d = KPS * c + kk;
      if (d % UK == UK - 1) s_load((kb + kk) / UK + DU, sw[d / UK]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // prologue: x of the first KPS k-blocks to LDS (through ring slots 0 .. KPS-1),
  // then slot j % XL takes k-block KPS + j; sign units u0 .. u0 + DU - 1
#pragma unroll
  for (int kk = 0; kk < KPS; ++kk) {
    x_load(kb0 + kk, xq[kk], pq[kk]);
    x_store(0, kk, xq[kk], pq[kk]);
  }
#pragma unroll
  for (int j = KPS; j < KPS + XL; ++j) x_load(kb0 + j, xq[j % XL], pq[j % XL]);
#pragma unroll
  for (int d = 0; d < DU; ++d) s_load(u0 + d, sw[d]);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  int base = kb0;
  for (; base + PER <= kb1; base += PER) {
#pragma unroll
    for (int c = 0; c < CPP; ++c) step(base + KPS * c, c);
  }
#pragma unroll
  for (int c = 0; c < CPP; ++c)
    if (base + KPS * c < kb1) step(base + KPS * c, c);

  const int n = rt * 16 + col;
  if (rt >= a.RT || n >= a.fill_to) return;
  float ps = 0.f;  // columns R .. fill_to: zeros
  if (n < a.R) ps = post ? (BF16 ? oc_bf2f(post[n]) : oc_h2f(post[n])) : 1.f;
  uint16_t* const out = a.separate ? term_pick(t, a.outs) : a.outs[0];
  if ((a.separate ? a.S : a.S * a.T) > 1) {
    float* pp = a.partial + ((size_t)blockIdx.y * a.M + m0) * a.N_pad + n;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * i + 4 * kq + r;
        if (m < M) pp[(size_t)m * a.N_pad] = yacc[i][r] * ps;
      }
    return;
  }
  const float b = (a.bias && n < a.R) ? (BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n])) : 0.f;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * i + 4 * kq + r;
      if (m < M) out[(size_t)(m0 + m) * a.ld_out + n] = BF16 ? oc_f2bf(fmaf(yacc[i][r], ps, b)) : oc_f2h(fmaf(yacc[i][r], ps, b));
    }
}

// outs[z][m, n] = sum over s < S (in order) of partial[z S + s, m, n] (+ bias[n] for n < R), n < ncols;
// z = blockIdx.z (one output, z = 0; a batch of independent problems, one z per problem).
struct SignReduceArgs {
  const float* partial;
  const uint16_t* bias;
  uint16_t* outs[kMaxTerms];
  int S, M, ncols, N_pad, R, ld_out;
};

template <bool BF16>
__global__ void k_sign_reduce(const SignReduceArgs a) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y, z = blockIdx.z;
  if (n >= a.ncols) return;
  const float* part = a.partial + (size_t)z * a.S * a.M * a.N_pad;
  float o = 0.f;
  for (int s = 0; s < a.S; ++s) o += part[((size_t)s * a.M + m) * a.N_pad + n];
  if (a.bias && n < a.R) o += BF16 ? oc_bf2f(a.bias[n]) : oc_h2f(a.bias[n]);
  term_pick(z, a.outs)[(size_t)m * a.ld_out + n] = BF16 ? oc_f2bf(o) : oc_f2h(o);
}

struct SignStreamPlan {
  bool use;
  int mb, S, T;   // row blocks of 16 per workgroup, K splits per term, terms
  int mz;         // row blocks across workgroups (grid.z)
  bool separate;  // terms into their own outputs (a batch of problems)
  size_t bytes;   // fp32 partials when an output takes more than one (+ k_sign_reduce)
};

// The streaming sign kernel serves 13 <= M <= 64 (OC_SIGN_STREAM = 0 turns it
// off, 1 forces it for any M <= 64), one term or up to four; K splits of each
// term on unit boundaries: enough workgroups (all terms') for one per CU, at
// most 8, at least 4 k-blocks each, none when the column workgroups alone cover
// 3/4 of the CUs (OC_SIGN_STREAM_S forces S).
SignStreamPlan plan_sign_stream(const oc_sign_term* terms, int n_terms, int M, int R, bool has_bias,
                                int fill_to, bool separate = false) {
  SignStreamPlan p = {};
  const int e = oc::knob("OC_SIGN_STREAM", -1);
  const SignLayout L = make_sign_layout(R, terms[0].Kd);
  p.use = n_terms >= 1 && n_terms <= kMaxTerms && e != 0 && M <= kSignStreamMaxM &&
          (e == 1 || M >= kSignStreamMinM) && !(has_bias && fill_to > R) && fill_to <= L.RT * 16;
  // several terms (MDBF): one unit size, and pre scales on all of them or none
  int nu_min = L.NU;
  for (int i = 1; i < n_terms && p.use; ++i) {
    const SignLayout Li = make_sign_layout(R, terms[i].Kd);
    p.use = Li.UK == L.UK && (terms[i].pre != nullptr) == (terms[0].pre != nullptr);
    if (Li.NU < nu_min) nu_min = Li.NU;
  }
  if (!p.use) return p;
  const int nkb = nu_min * L.UK, es = oc::knob("OC_SIGN_STREAM_S", 0);
  auto splits = [&](int wgs) {  // wgs: workgroups per split
    int S = es > 0 ? es : (oc_device_cus() + wgs - 1) / wgs;
    if (es <= 0) {
      if (S > 8) S = 8;
      if (S > nkb / 4) S = nkb / 4;
      // column workgroups that already cover 3/4 of the CUs: no split (one
      // term: no reduce launch; up_proj's output stage at M = 32: 23.8 -> 21.5 us)
      if (4 * wgs >= 3 * oc_device_cus()) S = 1;
    }
    return S;
  };
  const int wgs1 = (L.RT + 3) / 4 * n_terms;
  // Rows split across workgroups as well (two row blocks, grid.z) where one term would run
  // unsplit: twice the workgroups, each with half the step's MFMA chain, two per CU to hide
  // each other's step latency; the signs are read twice, from L2 (up_proj's output stage at
  // M = 32 / 48 / 64: 22.9 -> 21.3, 30.9 -> 27.6, 32.4 -> 29.5 us).  Where K splits already give
  // the parallelism (rank stages, down_proj, MDBF) it measured slower.  OC_SIGN_STREAM_MZ = 1 or 2
  // forces the count.
  const int ez = oc::knob("OC_SIGN_STREAM_MZ", 0);
  p.mz = M <= 16 ? 1 : (ez == 1 || ez == 2) ? ez : (n_terms == 1 && !separate && splits(wgs1) == 1 ? 2 : 1);
  const int mr = (M + p.mz - 1) / p.mz;
  p.mb = mr <= 16 ? 1 : (mr <= 32 ? 2 : 4);
  const int wgs = wgs1 * p.mz;
  int S = splits(wgs);
  if (S > nu_min) S = nu_min;
  if (S < 1) S = 1;
  p.S = S;
  p.T = n_terms;
  p.separate = separate;
  const bool parts = separate ? S > 1 : S * n_terms > 1;
  p.bytes = parts ? align256((size_t)S * n_terms * M * L.RT * 16 * 4) : 0;
  return p;
}

// k-blocks per step (per barrier and LDS round trip): 2 up to 32 rows, 1 at 64
// (the A fragments of two k-blocks of four row blocks would take 128 VGPRs)
constexpr int sign_stream_kps(int mb) { return mb <= 2 ? 2 : 1; }

template <int UK, bool BF16>
int launch_sign_stream_uk(const SignStreamArgs& a, int mb, bool pre, hipStream_t st) {
  const dim3 grid((a.RT + 3) / 4, a.S * a.T, a.mz), block(256);
  const size_t lds = (size_t)2 * 16 * mb * (sign_stream_kps(mb) * 128 + 8) * 2;
#define OC_SS(MB_)                                                                                         \
  if (mb == MB_) {                                                                                         \
    constexpr int KPS_ = sign_stream_kps(MB_);                                                             \
    if (pre) hipLaunchKernelGGL((k_sign_stream<MB_, UK, KPS_, true, BF16>), grid, block, lds, st, a);     \
    else hipLaunchKernelGGL((k_sign_stream<MB_, UK, KPS_, false, BF16>), grid, block, lds, st, a);        \
    OC_HIP(hipGetLastError());                                                                             \
    return 0;                                                                                              \
  }
  OC_SS(1) OC_SS(2) OC_SS(4)
#undef OC_SS
  return oc::set_error(OC_ERR_UNSUPPORTED, "no streaming sign kernel for %d row blocks", mb);
}

template <bool BF16>
int launch_sign_stream(const SignStreamArgs& a, int uk, int mb, bool pre, hipStream_t st) {
  if (uk == 4) return launch_sign_stream_uk<4, BF16>(a, mb, pre, st);
  if (uk == 2) return launch_sign_stream_uk<2, BF16>(a, mb, pre, st);
  return launch_sign_stream_uk<1, BF16>(a, mb, pre, st);
}

// outs: the one output (outs[0]), or one per term with p.separate
int sign_stream(const oc_sign_term* terms, int M, int R, bool bf16, const void* bias, void* const* outs,
                int ld_out, int fill_to, const SignStreamPlan& p, void* workspace, size_t ws_bytes, hipStream_t st) {
  OC_REQUIRE(ws_bytes >= p.bytes && (p.bytes == 0 || workspace), OC_ERR_WORKSPACE,
             "workspace of %zu bytes is smaller than the %zu required", ws_bytes, p.bytes);
  const SignLayout L = make_sign_layout(R, terms[0].Kd);
  const int parts = p.separate ? p.S : p.S * p.T;  // partials per output
  SignStreamArgs a = {};
  for (int i = 0; i < p.T; ++i) {
    const oc_sign_term& T = terms[i];
    a.sg[i] = (const uint32_t*)T.packed;
    a.in[i] = (const uint16_t*)T.in;
    a.pre[i] = (const uint16_t*)T.pre;
    a.post[i] = (const uint16_t*)T.post;
    a.ld_in[i] = T.ld_in;
    a.Kd[i] = T.Kd;
    a.NU[i] = make_sign_layout(R, T.Kd).NU;
    a.outs[i] = (uint16_t*)outs[p.separate ? i : 0];
  }
  a.bias = parts == 1 ? (const uint16_t*)bias : nullptr;
  a.partial = (float*)workspace;
  a.ld_out = ld_out;
  a.M = M;
  a.R = R;
  a.RT = L.RT;
  a.S = p.S;
  a.T = p.T;
  a.fill_to = fill_to;
  a.N_pad = L.RT * 16;
  a.separate = p.separate ? 1 : 0;
  a.mz = p.mz;
  const bool pre = terms[0].pre != nullptr;
  const int rc = bf16 ? launch_sign_stream<true>(a, L.UK, p.mb, pre, st)
                : launch_sign_stream<false>(a, L.UK, p.mb, pre, st);
  if (rc || parts == 1) return rc;
  // each output's fp32 partials, added in (term, split) order
  SignReduceArgs r = {};
  r.partial = a.partial;
  r.bias = (const uint16_t*)bias;
  for (int i = 0; i < kMaxTerms; ++i) r.outs[i] = a.outs[p.separate && i < p.T ? i : 0];
  r.S = parts;
  r.M = M;
  r.ncols = fill_to;
  r.N_pad = a.N_pad;
  r.R = R;
  r.ld_out = ld_out;
  const dim3 g((fill_to + 255) / 256, M, p.separate ? p.T : 1);
  if (bf16) hipLaunchKernelGGL(k_sign_reduce<true>, g, dim3(256), 0, st, r);
  else hipLaunchKernelGGL(k_sign_reduce<false>, g, dim3(256), 0, st, r);
  OC_HIP(hipGetLastError());
  return 0;
}

struct SignGemmPlan {
  oc_gemm::GemmPlan gp;  // tiling (MDBF: over the terms' concatenated k-blocks)
  int mt;                // tile height 64 mt
  int nkb[kMaxTerms];    // k-blocks of each term
  size_t xs_bytes, part_off, bytes;
};

// One term: its input (RNE(in * pre) staged when it has a pre scale), K-split
// pieces and their fixup.  Several terms (MDBF) run as one GEMM over their
// concatenated k-blocks (inputs staged side by side, each term's post scale
// folded into its +-1 operand), so a term adds K, not another output pass.
SignGemmPlan plan_sign_gemm(const oc_sign_term* terms, int n_terms, int M, int R) {
  SignGemmPlan p;
  const SignLayout L0 = make_sign_layout(R, terms[0].Kd);
  const int e = oc::knob("OC_GEMM_MT", 0);
  p.mt = (e == 1 || e == 2 || e == 4) ? e : oc_gemm::gemm_tile_height(M, L0.RT * 16);
  int nkb = 0;
  for (int i = 0; i < n_terms; ++i) {
    p.nkb[i] = make_sign_layout(R, terms[i].Kd).K_pad / 128;
    nkb += p.nkb[i];
  }
  p.gp = oc_gemm::plan_gemm(M, L0.RT * 16, nkb * 128, oc::knob("OC_GEMM_SPLIT", 0), p.mt);
  if (n_terms > 1) p.xs_bytes = align256((size_t)M * nkb * 128 * 2);
  else p.xs_bytes = terms[0].pre ? align256((size_t)M * round8(terms[0].Kd) * 2) : 0;
  p.part_off = p.xs_bytes;
  p.bytes = p.xs_bytes + align256(p.gp.part_bytes);
  return p;
}

template <bool BF16, bool MULTI>
void launch_sign_gemm(const oc_gemm::GemmArgs& g, int mt, int grid, hipStream_t st) {
  const size_t lds = oc_gemm::gemm_lds_bytes(mt);
  if (mt == 1) hipLaunchKernelGGL((oc_gemm::k_gemm<1, 4, BF16, 1, false, MULTI>), dim3(grid), dim3(256), lds, st, g);
  else if (mt == 2) hipLaunchKernelGGL((oc_gemm::k_gemm<1, 4, BF16, 2, false, MULTI>), dim3(grid), dim3(256), lds, st, g);
  else hipLaunchKernelGGL((oc_gemm::k_gemm<1, 4, BF16, 4, false, MULTI>), dim3(grid), dim3(256), lds, st, g);
}

template <bool BF16>
void launch_sign_fixup(const oc_gemm::GemmArgs& g, int mt, int tiles, hipStream_t st) {
  const dim3 fg(64 * mt * oc_gemm::kGemmBN / 256, tiles);
  if (mt == 1) hipLaunchKernelGGL((oc_gemm::k_gemm_fixup<BF16, 1>), fg, dim3(256), 0, st, g);
  else if (mt == 2) hipLaunchKernelGGL((oc_gemm::k_gemm_fixup<BF16, 2>), fg, dim3(256), 0, st, g);
  else hipLaunchKernelGGL((oc_gemm::k_gemm_fixup<BF16, 4>), fg, dim3(256), 0, st, g);
}

int sign_gemm_large(const oc_sign_term* terms, int n_terms, int M, int R, bool bf16, const void* bias,
                    void* out, int ld_out, int fill_to, void* workspace, size_t ws_bytes, hipStream_t st) {
  const SignGemmPlan p = plan_sign_gemm(terms, n_terms, M, R);
  OC_REQUIRE(ws_bytes >= p.bytes && (p.bytes == 0 || workspace), OC_ERR_WORKSPACE,
             "workspace of %zu bytes is smaller than the %zu required", ws_bytes, p.bytes);
  uint8_t* ws = (uint8_t*)workspace;
  const SignLayout L0 = make_sign_layout(R, terms[0].Kd);
  // Columns R .. fill_to of the output (the next stage's zero padding) come
  // out of the GEMM as zeros when there is no bias: their scale is 0 (finite
  // inputs, 0 times a finite sum).
  const bool fold_fill = fill_to > R && bias == nullptr && fill_to <= L0.RT * 16;
  oc_gemm::GemmArgs g = {};
  g.y = (uint16_t*)out;
  g.part = (float*)(ws + p.part_off);
  g.bias = (const uint16_t*)bias;
  g.M = M;
  g.N = fold_fill ? fill_to : R;
  g.npost = R;
  g.N_pad = L0.RT * 16;
  g.NT_total = L0.RT;
  g.NU = L0.NU;
  g.G = 1;
  g.gshift = -1;
  g.uk_shift = L0.UK == 4 ? 2 : (L0.UK == 2 ? 1 : 0);
  g.MB = p.gp.MB;
  g.NB = p.gp.NB;
  g.NKB = p.gp.NKB;
  g.gs = g.NKB * 128;
  g.ldy = ld_out;
  g.tiles_main = p.gp.tiles_main;
  g.S = p.gp.S;
  g.kper = p.gp.kper;
  g.pstride = p.gp.S;
  g.poff = 0;
  if (n_terms == 1) {
    const oc_sign_term& T = terms[0];
    g.w = (const uint8_t*)T.packed;
    g.post = (const uint16_t*)T.post;
    g.K = T.Kd;
    if (T.pre) {
      const int ldx = round8(T.Kd);
      uint16_t* xs = (uint16_t*)ws;
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
  } else {
    // the terms' inputs side by side, k-block aligned (zeros past each Kd)
    PrescaleTerms pt = {};
    int off = 0;
    for (int i = 0; i < n_terms; ++i) {
      pt.in[i] = (const uint16_t*)terms[i].in;
      pt.pre[i] = (const uint16_t*)terms[i].pre;
      pt.ld_in[i] = terms[i].ld_in;
      pt.Kd[i] = terms[i].Kd;
      pt.off[i] = off;
      g.tkb[i] = off / 128;
      g.tw[i] = (const uint8_t*)terms[i].packed;
      g.tpost[i] = (const uint16_t*)terms[i].post;
      g.tNU[i] = make_sign_layout(R, terms[i].Kd).NU;
      off += p.nkb[i] * 128;
    }
    for (int i = n_terms; i <= kMaxTerms; ++i) {
      pt.off[i] = off;
      g.tkb[i] = off / 128;
    }
    pt.n_terms = n_terms;
    pt.ldx = off;
    uint16_t* xs = (uint16_t*)ws;
    const dim3 pg((off + 255) / 256, M);
    if (bf16) hipLaunchKernelGGL(k_prescale_terms<true>, pg, dim3(256), 0, st, pt, xs);
    else hipLaunchKernelGGL(k_prescale_terms<false>, pg, dim3(256), 0, st, pt, xs);
    OC_HIP(hipGetLastError());
    g.x = xs;
    g.ldx = off;
    g.K = off;
    g.w = g.tw[0];
    g.nterms = n_terms;
  }
  const int grid = p.gp.tiles_main + p.gp.split_tiles * p.gp.S;
  if (n_terms == 1) {
    if (bf16) launch_sign_gemm<true, false>(g, p.mt, grid, st);
    else launch_sign_gemm<false, false>(g, p.mt, grid, st);
  } else {
    if (bf16) launch_sign_gemm<true, true>(g, p.mt, grid, st);
    else launch_sign_gemm<false, true>(g, p.mt, grid, st);
  }
  OC_HIP(hipGetLastError());
  if (p.gp.split_tiles > 0) {
    if (bf16) launch_sign_fixup<true>(g, p.mt, p.gp.split_tiles, st);
    else launch_sign_fixup<false>(g, p.mt, p.gp.split_tiles, st);
    OC_HIP(hipGetLastError());
  }
  if (fill_to > R && !fold_fill) {
    hipLaunchKernelGGL(k_zero_cols, dim3(M), dim3(64), 0, st, (uint16_t*)out, ld_out, R, fill_to);
    OC_HIP(hipGetLastError());
  }
  return 0;
}

}  // namespace

extern "C" size_t oc_sign_workspace_bytes(const oc_sign_term* terms, int n_terms, int M, int R) {
  if (!terms || n_terms < 1 || n_terms > kMaxTerms || R <= 0) return 0;
  for (int i = 0; i < n_terms; ++i)
    if (terms[i].Kd <= 0) return 0;
  // the stream plan's split count does not depend on bias / fill_to, but a call with both takes
  // the GEMM path: enough for either
  const SignStreamPlan sp = plan_sign_stream(terms, n_terms, M, R, false, R);
  const size_t gemm = M >= sign_gemm_min_m() ? plan_sign_gemm(terms, n_terms, M, R).bytes : 0;
  if (sp.use) return sp.bytes > gemm ? sp.bytes : gemm;
  return gemm;
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
  int uk = 0;
  bool pre = terms[0].pre != nullptr;
  for (int i = 0; i < n_terms; ++i) {
    const oc_sign_term& T = terms[i];
    OC_REQUIRE(T.packed && T.in, OC_ERR_INVALID, "term %d: null pointer", i);
    OC_REQUIRE(T.Kd > 0 && T.ld_in >= T.Kd && T.ld_in % 8 == 0, OC_ERR_SHAPE,
               "term %d: Kd=%d / ld_in=%d (ld_in must be >= Kd and a multiple of 8)", i, T.Kd, T.ld_in);
    const SignLayout L = make_sign_layout(R, T.Kd);
    OC_REQUIRE(uk == 0 || uk == L.UK, OC_ERR_UNSUPPORTED, "terms of one call need the same unit size");
    OC_REQUIRE((T.pre != nullptr) == pre, OC_ERR_UNSUPPORTED,
               "terms of one call must all have a pre scale or none");
    uk = L.UK;
    a.t[i].sg = (const uint32_t*)T.packed;
    a.t[i].in = (const uint16_t*)T.in;
    a.t[i].pre = (const uint16_t*)T.pre;
    a.t[i].post = (const uint16_t*)T.post;
    a.t[i].ld_in = T.ld_in;
    a.t[i].Kd = T.Kd;
    a.t[i].NU = L.NU;
    a.t[i].UK = L.UK;
  }
  {
    const SignStreamPlan sp = plan_sign_stream(terms, n_terms, M, R, bias != nullptr, fill_to);
    if (sp.use)
      return sign_stream(terms, M, R, act_dtype == OC_DTYPE_BF16, bias, &out, ld_out, fill_to, sp, workspace,
                         ws_bytes, (hipStream_t)stream);
  }
  if (M >= sign_gemm_min_m())
    return sign_gemm_large(terms, n_terms, M, R, act_dtype == OC_DTYPE_BF16, bias, out, ld_out, fill_to,
                           workspace, ws_bytes, (hipStream_t)stream);
  a.n_terms = n_terms;
  a.batch = 1;
  a.bias = (const uint16_t*)bias;
  a.R = R;
  a.RT = (R + 15) / 16;
  a.fill_to = fill_to;
  a.ld_out = ld_out;
  int nu_min = a.t[0].NU;
  for (int i = 1; i < n_terms; ++i) nu_min = a.t[i].NU < nu_min ? a.t[i].NU : nu_min;
  const int rt_grid = (fill_to + 15) / 16;
  hipStream_t st = (hipStream_t)stream;
  const bool bf16 = act_dtype == OC_DTYPE_BF16;
  // Rows in chunks of 16 (only reached below the GEMM threshold, i.e. when
  // OC_SIGN_GEMM_MIN_M raises it).
  for (int m0 = 0; m0 < M; m0 += kSignGemvMaxM) {
    SignArgs c = a;
    c.M = M - m0 < kSignGemvMaxM ? M - m0 : kSignGemvMaxM;
    c.W = sign_waves(a.RT, nu_min, c.M, uk, n_terms > 1);
    c.outs[0] = (uint16_t*)out + (size_t)m0 * ld_out;
    for (int i = 0; i < n_terms; ++i) c.t[i].in = a.t[i].in + (size_t)m0 * a.t[i].ld_in;
    int rc;
    if (uk == 4)
      rc = bf16 ? launch_sign<4, true>(c, pre, rt_grid, st) : launch_sign<4, false>(c, pre, rt_grid, st);
    else if (uk == 2)
      rc = bf16 ? launch_sign<2, true>(c, pre, rt_grid, st) : launch_sign<2, false>(c, pre, rt_grid, st);
    else
      rc = bf16 ? launch_sign<1, true>(c, pre, rt_grid, st) : launch_sign<1, false>(c, pre, rt_grid, st);
    if (rc) return rc;
  }
  return 0;
}

extern "C" size_t oc_sign_batch_workspace_bytes(const oc_sign_term* terms, int n_problems, int M, int R) {
  if (!terms || n_problems < 1 || n_problems > kMaxTerms || R <= 0) return 0;
  for (int i = 0; i < n_problems; ++i)
    if (terms[i].Kd <= 0) return 0;
  const SignStreamPlan sp = plan_sign_stream(terms, n_problems, M, R, false, R, true);
  if (sp.use) return sp.bytes;
  size_t w = 0;  // the GEMV path needs none; otherwise one problem at a time
  for (int i = 0; i < n_problems; ++i) {
    const size_t b = oc_sign_workspace_bytes(&terms[i], 1, M, R);
    w = b > w ? b : w;
  }
  return w;
}

extern "C" int oc_sign_gemm_batch(const oc_sign_term* terms, int n_problems, int M, int R, int act_dtype,
                                  void* const* outs, int ld_out, int fill_to, void* workspace, size_t ws_bytes,
                                  void* stream) {
  OC_REQUIRE(terms && outs, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(n_problems >= 1 && n_problems <= kMaxTerms, OC_ERR_UNSUPPORTED, "n_problems=%d must be 1..%d",
             n_problems, kMaxTerms);
  OC_REQUIRE(M >= 0 && R > 0, OC_ERR_INVALID, "bad M=%d R=%d", M, R);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d",
             act_dtype);
  if (fill_to < R) fill_to = R;
  OC_REQUIRE(ld_out >= fill_to, OC_ERR_SHAPE, "ld_out=%d < fill_to=%d", ld_out, fill_to);
  bool one_launch = n_problems > 1;
  int uk = 0;
  for (int i = 0; i < n_problems; ++i) {
    const oc_sign_term& T = terms[i];
    OC_REQUIRE(outs[i] && T.packed && T.in, OC_ERR_INVALID, "problem %d: null pointer", i);
    OC_REQUIRE(T.Kd > 0 && T.ld_in >= T.Kd && T.ld_in % 8 == 0, OC_ERR_SHAPE,
               "problem %d: Kd=%d / ld_in=%d (ld_in must be >= Kd and a multiple of 8)", i, T.Kd, T.ld_in);
    const SignLayout L = make_sign_layout(R, T.Kd);
    one_launch = one_launch && (uk == 0 || uk == L.UK) && ((T.pre != nullptr) == (terms[0].pre != nullptr));
    uk = L.UK;
  }
  if (M == 0) return 0;
  const bool bf16 = act_dtype == OC_DTYPE_BF16;
  hipStream_t st = (hipStream_t)stream;
  if (one_launch) {
    const SignStreamPlan sp = plan_sign_stream(terms, n_problems, M, R, false, fill_to, true);
    if (sp.use) return sign_stream(terms, M, R, bf16, nullptr, outs, ld_out, fill_to, sp, workspace, ws_bytes, st);
    if (M <= kSignGemvMaxM && M < sign_gemm_min_m()) {
      // the single-term GEMV, blockIdx.y = problem
      SignArgs a = {};
      int nu_min = 1 << 30;
      for (int i = 0; i < n_problems; ++i) {
        const oc_sign_term& T = terms[i];
        const SignLayout L = make_sign_layout(R, T.Kd);
        a.t[i].sg = (const uint32_t*)T.packed;
        a.t[i].in = (const uint16_t*)T.in;
        a.t[i].pre = (const uint16_t*)T.pre;
        a.t[i].post = (const uint16_t*)T.post;
        a.t[i].ld_in = T.ld_in;
        a.t[i].Kd = T.Kd;
        a.t[i].NU = L.NU;
        a.t[i].UK = L.UK;
        a.outs[i] = (uint16_t*)outs[i];
        nu_min = L.NU < nu_min ? L.NU : nu_min;
      }
      a.n_terms = 1;
      a.batch = n_problems;
      a.R = R;
      a.RT = (R + 15) / 16;
      a.fill_to = fill_to;
      a.ld_out = ld_out;
      a.M = M;
      a.W = sign_waves(a.RT, nu_min, M, uk, false);
      const int rt_grid = (fill_to + 15) / 16;
      const bool pre = terms[0].pre != nullptr;
      if (uk == 4) return bf16 ? launch_sign<4, true>(a, pre, rt_grid, st) : launch_sign<4, false>(a, pre, rt_grid, st);
      if (uk == 2) return bf16 ? launch_sign<2, true>(a, pre, rt_grid, st) : launch_sign<2, false>(a, pre, rt_grid, st);
      return bf16 ? launch_sign<1, true>(a, pre, rt_grid, st) : launch_sign<1, false>(a, pre, rt_grid, st);
    }
  }
  // one problem at a time (the workspace is reused: the launches are ordered on the stream)
  for (int i = 0; i < n_problems; ++i) {
    const int rc = oc_sign_gemm(&terms[i], 1, M, R, act_dtype, nullptr, outs[i], ld_out, fill_to, workspace,
                                ws_bytes, stream);
    if (rc) return rc;
  }
  return 0;
}
