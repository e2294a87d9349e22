// GPTQ parity tools and the load-time repack into the lane-chunk layout.
//
// Checkpoint bit layout (AutoGPTQ, as written by OneComp,
// onecomp/quantizer/gptq/gptq_layer.py:36-184): codes are packed along K into
// int32 rows of qweight [K*b/32, N]; for b in {2,4,8} code k sits at bits
// b*(k % (32/b)) of row k / (32/b); for b = 3 the 32 codes of a 96-bit block
// (3 rows) form one little-endian bit stream, so codes 10 and 21 straddle two
// words.  qzeros uses the same rule along N.
#include <algorithm>
#include <vector>

#include "oc_common.h"

namespace {

using oc::Layout;

// Code of (k, n) from a [rows, ld] int32 matrix packed along its rows.
__device__ __forceinline__ uint32_t packed_field(const int32_t* __restrict__ m, int ld, int bits,
                                                 int k, int n) {
  if (bits == 3) {
    const int blk = k >> 5, j = k & 31, bit = 3 * j;
    const int row = 3 * blk + (bit >> 5), off = bit & 31;
    const uint32_t w0 = (uint32_t)m[(size_t)row * ld + n];
    if (off <= 29) return (w0 >> off) & 7u;
    const uint32_t w1 = (uint32_t)m[(size_t)(row + 1) * ld + n];
    const int first = 32 - off;
    return ((w0 >> off) & ((1u << first) - 1u)) | ((w1 & ((1u << (3 - first)) - 1u)) << first);
  }
  const int pf = 32 / bits;
  const uint32_t w = (uint32_t)m[(size_t)(k / pf) * ld + n];
  return (w >> (bits * (k % pf))) & ((1u << bits) - 1u);
}

// Zero field of (g, n): qzeros [G, N*b/32] packed along N -- the same stream
// rule applied to the column index inside row g.
__device__ __forceinline__ uint32_t zero_field(const int32_t* __restrict__ qz, int N, int bits, int g,
                                               int n, int fmt) {
  const int ld = N * bits / 32;
  const int32_t* row = qz + (size_t)g * ld;
  uint32_t z;
  if (bits == 3) {
    const int blk = n >> 5, j = n & 31, bit = 3 * j;
    const int wi = 3 * blk + (bit >> 5), off = bit & 31;
    const uint32_t w0 = (uint32_t)row[wi];
    if (off <= 29) {
      z = (w0 >> off) & 7u;
    } else {
      const uint32_t w1 = (uint32_t)row[wi + 1];
      const int first = 32 - off;
      z = ((w0 >> off) & ((1u << first) - 1u)) | ((w1 & ((1u << (3 - first)) - 1u)) << first);
    }
  } else {
    const int pf = 32 / bits;
    z = ((uint32_t)row[n / pf] >> (bits * (n % pf))) & ((1u << bits) - 1u);
  }
  if (fmt == OC_ZERO_V1) z = (z + 1u) & ((1u << bits) - 1u);
  return z;
}

__global__ void k_unpack_codes(const int32_t* __restrict__ qw, int K, int N, int bits,
                               int32_t* __restrict__ codes) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int k0 = blockIdx.y * 32;
  if (n >= N) return;
  for (int k = k0; k < min(k0 + 32, K); ++k)
    codes[(size_t)n * K + k] = (int32_t)packed_field(qw, N, bits, k, n);
}

__global__ void k_unpack_zeros(const int32_t* __restrict__ qz, int G, int N, int bits, int fmt,
                               int32_t* __restrict__ out) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int g = blockIdx.y;
  if (n >= N) return;
  out[(size_t)g * N + n] = (int32_t)zero_field(qz, N, bits, g, n, fmt);
}

template <bool BF16>
__global__ void k_dequant(const int32_t* __restrict__ qw, const int32_t* __restrict__ qz,
                          const uint16_t* __restrict__ scales, const int32_t* __restrict__ g_idx,
                          int K, int N, int G, int bits, int gs, int fmt, uint16_t* __restrict__ w) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int k0 = blockIdx.y * 32;
  if (n >= N) return;
  for (int k = k0; k < min(k0 + 32, K); ++k) {
    int g = g_idx ? g_idx[k] : k / gs;
    g = min(max(g, 0), G - 1);
    const uint32_t q = packed_field(qw, N, bits, k, n);
    const uint32_t z = zero_field(qz, N, bits, g, n, fmt);
    // fp16 scale times a small integer is exact in fp32: one rounding below.
    const float v = oc_h2f(scales[(size_t)g * N + n]) * (float)((int)q - (int)z);
    w[(size_t)n * K + k] = BF16 ? oc_f2bf(v) : oc_f2h(v);
  }
}

// Inverse of the decoders of the lane-chunk layout (see oc_common.h and
// gptq_decode.h): for word W of a lane's unit payload, which local k each
// bit field holds.  Returns the packed word.
__device__ __forceinline__ uint32_t code_at(const int32_t* __restrict__ qw, const int32_t* __restrict__ perm,
                                            const Layout& L, int u, int k_local, int n) {
  const int ps = 128 * L.U * u + k_local;
  if (ps >= L.K || n >= L.N) return 0u;
  const int k = perm ? perm[ps] : ps;
  return packed_field(qw, L.N, L.bits, k, n);
}

__global__ void k_repack(const int32_t* __restrict__ qw, const int32_t* __restrict__ perm, Layout L,
                         uint32_t* __restrict__ out, size_t n_words) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_words) return;
  const int w = (int)(idx & 3);
  const int lane = (int)((idx >> 2) & 63);
  size_t rest = idx >> 8;
  const int pt = (int)(rest % L.P);
  rest /= L.P;
  const int u = (int)(rest % L.NU);
  const int nt = (int)(rest / L.NU);
  const int Wi = 4 * pt + w;
  const int kq = lane >> 4;
  const int n = 16 * nt + (lane & 15);
  uint32_t word = 0;
  switch (L.bits) {
    case 4: {
      const int t = Wi;
      for (int f = 0; f < 8; ++f) {
        const int p = f & 3, hi = f >> 2;
        word |= code_at(qw, perm, L, u, 32 * t + 8 * kq + 2 * p + hi, n) << (4 * f);
      }
      break;
    }
    case 8: {
      const int t = Wi >> 1, h = Wi & 1;
      for (int f = 0; f < 4; ++f) {
        const int b = f & 1, hi = f >> 1, p = 2 * h + b;
        word |= code_at(qw, perm, L, u, 32 * t + 8 * kq + 2 * p + hi, n) << (8 * f);
      }
      break;
    }
    case 2: {
      const int kbl = Wi >> 1, h = Wi & 1;
      for (int f = 0; f < 16; ++f) {
        const int hi = f >> 3, pp = f & 7, t = 2 * h + (pp >> 2), p = pp & 3;
        word |= code_at(qw, perm, L, u, 128 * kbl + 32 * t + 8 * kq + 2 * p + hi, n) << (2 * f);
      }
      break;
    }
    case 3: {
      const int kbl = Wi / 3, wi = Wi % 3;
      for (int j = 0; j < 5; ++j) {
        const int P = 5 * wi + j, t = P >> 2, p = P & 3;
        const int kl = 128 * kbl + 32 * t + 8 * kq + 2 * p;
        word |= code_at(qw, perm, L, u, kl, n) << (3 * j);
        word |= code_at(qw, perm, L, u, kl + 1, n) << (16 + 3 * j);
      }
      // pair 15 (t = 3, p = 3): bit wi of each code in the spare bits 15 / 31
      const int kl = 128 * kbl + 32 * 3 + 8 * kq + 6;
      word |= ((code_at(qw, perm, L, u, kl, n) >> wi) & 1u) << 15;
      word |= ((code_at(qw, perm, L, u, kl + 1, n) >> wi) & 1u) << 31;
      break;
    }
  }
  out[idx] = word;
}

__global__ void k_meta(const int32_t* __restrict__ qz, const uint16_t* __restrict__ scales, int G,
                       int N, int N_pad, int bits, int fmt, uint32_t* __restrict__ meta) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int g = blockIdx.y;
  if (n >= N_pad) return;
  uint32_t s = 0, z = 0;
  if (n < N) {
    s = scales[(size_t)g * N + n];
    z = zero_field(qz, N, bits, g, n, fmt);
  }
  meta[(size_t)g * N_pad + n] = s | (z << 16);
}

int check_bits(int bits) {
  OC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, OC_ERR_UNSUPPORTED,
             "unsupported bits=%d (expected 2, 3, 4 or 8)", bits);
  return 0;
}

int check_ckpt_shape(int K, int N, int bits) {
  OC_REQUIRE(K > 0 && N > 0, OC_ERR_INVALID, "K=%d and N=%d must be positive", K, N);
  OC_REQUIRE(K % 32 == 0, OC_ERR_SHAPE, "K=%d must be a multiple of 32 (AutoGPTQ packing)", K);
  OC_REQUIRE((N * bits) % 32 == 0, OC_ERR_SHAPE,
             "N=%d * bits=%d must be a multiple of 32 (qzeros packing)", N, bits);
  return 0;
}

}  // namespace

extern "C" int oc_gptq_unpack_codes(const int32_t* qweight, int K, int N, int bits, int32_t* codes,
                                    void* stream) {
  if (int e = check_bits(bits)) return e;
  if (int e = check_ckpt_shape(K, N, bits)) return e;
  OC_REQUIRE(qweight && codes, OC_ERR_INVALID, "null pointer");
  dim3 grid((N + 255) / 256, (K + 31) / 32);
  hipLaunchKernelGGL(k_unpack_codes, grid, dim3(256), 0, (hipStream_t)stream, qweight, K, N, bits, codes);
  OC_HIP(hipGetLastError());
  return 0;
}

extern "C" int oc_gptq_unpack_zeros(const int32_t* qzeros, int G, int N, int bits, int zero_format,
                                    int32_t* zeros, void* stream) {
  if (int e = check_bits(bits)) return e;
  OC_REQUIRE(G > 0 && N > 0 && (N * bits) % 32 == 0, OC_ERR_SHAPE, "bad G=%d N=%d", G, N);
  OC_REQUIRE(qzeros && zeros, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(zero_format >= 0 && zero_format <= 2, OC_ERR_INVALID, "bad zero_format %d", zero_format);
  dim3 grid((N + 255) / 256, G);
  hipLaunchKernelGGL(k_unpack_zeros, grid, dim3(256), 0, (hipStream_t)stream, qzeros, G, N, bits,
                     zero_format, zeros);
  OC_HIP(hipGetLastError());
  return 0;
}

extern "C" int oc_gptq_dequant(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                               const int32_t* g_idx, int K, int N, int G, int bits, int group_size,
                               int zero_format, int out_dtype, void* w, void* stream) {
  if (int e = check_bits(bits)) return e;
  if (int e = check_ckpt_shape(K, N, bits)) return e;
  OC_REQUIRE(qweight && qzeros && scales && w, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(G > 0, OC_ERR_INVALID, "G=%d must be positive", G);
  OC_REQUIRE(out_dtype == OC_DTYPE_F16 || out_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED,
             "bad out_dtype %d", out_dtype);
  const int gs = oc::eff_group(group_size, K);
  dim3 grid((N + 255) / 256, (K + 31) / 32);
  if (out_dtype == OC_DTYPE_BF16)
    hipLaunchKernelGGL(k_dequant<true>, grid, dim3(256), 0, (hipStream_t)stream, qweight, qzeros,
                       scales, g_idx, K, N, G, bits, gs, zero_format, (uint16_t*)w);
  else
    hipLaunchKernelGGL(k_dequant<false>, grid, dim3(256), 0, (hipStream_t)stream, qweight, qzeros,
                       scales, g_idx, K, N, G, bits, gs, zero_format, (uint16_t*)w);
  OC_HIP(hipGetLastError());
  return 0;
}

extern "C" int oc_gptq_layout(int K, int N, int bits, size_t* packed_bytes, int* k_pad, int* n_pad) {
  if (int e = check_bits(bits)) return e;
  OC_REQUIRE(K > 0 && N > 0, OC_ERR_INVALID, "K=%d and N=%d must be positive", K, N);
  const Layout L = oc::make_layout(bits, K, N);
  if (packed_bytes) *packed_bytes = oc::layout_bytes(L);
  if (k_pad) *k_pad = L.K_pad;
  if (n_pad) *n_pad = L.N_pad;
  return 0;
}

extern "C" int oc_gptq_prepare(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                               const int32_t* g_idx, int K, int N, int G, int bits, int group_size,
                               int zero_format, void* packed, uint32_t* meta, int32_t* perm,
                               int* perm_identity, void* stream) {
  if (int e = check_bits(bits)) return e;
  if (int e = check_ckpt_shape(K, N, bits)) return e;
  OC_REQUIRE(qweight && qzeros && scales && packed && meta, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(zero_format == OC_ZERO_V1 || zero_format == OC_ZERO_V2, OC_ERR_INVALID,
             "zero_format must be OC_ZERO_V1 or OC_ZERO_V2");
  const int gs = oc::eff_group(group_size, K);
  OC_REQUIRE(gs % 32 == 0 || group_size <= 0, OC_ERR_UNSUPPORTED,
             "group_size=%d must be a multiple of 32 (or -1)", group_size);
  OC_REQUIRE(G == (K + gs - 1) / gs, OC_ERR_SHAPE, "G=%d does not match K=%d / group_size=%d", G, K, gs);
  hipStream_t st = (hipStream_t)stream;
  const Layout L = oc::make_layout(bits, K, N);

  const int32_t* use_perm = nullptr;
  if (perm_identity) *perm_identity = 1;
  if (g_idx) {
    OC_REQUIRE(perm, OC_ERR_INVALID, "perm must be given with g_idx");
    // Act-order: stable argsort of g_idx so that every group becomes a
    // contiguous run of gs positions.  Runs once per layer at load time.
    std::vector<int32_t> h_g(K), h_perm(K);
    OC_HIP(hipMemcpyAsync(h_g.data(), g_idx, sizeof(int32_t) * K, hipMemcpyDeviceToHost, st));
    OC_HIP(hipStreamSynchronize(st));
    for (int k = 0; k < K; ++k) h_perm[k] = k;
    std::stable_sort(h_perm.begin(), h_perm.end(), [&](int a, int b) { return h_g[a] < h_g[b]; });
    bool identity = true;
    for (int p = 0; p < K; ++p) {
      const int g = h_g[h_perm[p]];
      OC_REQUIRE(g == p / gs, OC_ERR_GIDX,
                 "g_idx does not form %d contiguous groups of %d after sorting (position %d has "
                 "group %d)", G, gs, p, g);
      identity = identity && h_perm[p] == p;
    }
    OC_HIP(hipMemcpyAsync(perm, h_perm.data(), sizeof(int32_t) * K, hipMemcpyHostToDevice, st));
    OC_HIP(hipStreamSynchronize(st));
    if (perm_identity) *perm_identity = identity ? 1 : 0;
    if (!identity) use_perm = perm;
  }
  const size_t n_words = oc::layout_bytes(L) / 4;
  hipLaunchKernelGGL(k_repack, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0, st, qweight,
                     use_perm, L, (uint32_t*)packed, n_words);
  OC_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_meta, dim3((L.N_pad + 255) / 256, G), dim3(256), 0, st, qzeros, scales, G, N,
                     L.N_pad, bits, zero_format, meta);
  OC_HIP(hipGetLastError());
  return 0;
}
