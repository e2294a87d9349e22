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
//   doubling: H_2K = [[1, 1], [1, -1]] (x) H_K.
// chi is the quadratic character mod q.  Orders 52, 100, 156 and 172 (Paley
// over GF(25) / GF(49) and other constructions) are not built.
//
// The kernel computes in fp32 and rounds once to the activation dtype.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oc_common.h"

namespace {

// Orders in the reference's search order (largest first), with how to build them.
struct HadOrder {
  int K;
  int kind;  // 1 Paley I, 2 Paley II, 3 doubling of the order K/2
  int q;
};
constexpr HadOrder kOrders[] = {{172, 0, 0}, {156, 0, 0}, {140, 1, 139}, {108, 1, 107}, {100, 0, 0},
                                {76, 2, 37},  {68, 1, 67},  {60, 1, 59},   {52, 0, 0},    {44, 1, 43},
                                {40, 3, 0},   {36, 2, 17},  {28, 2, 13},   {20, 1, 19},   {12, 1, 11}};

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

constexpr int kHadMaxN = 32768;  // fp32 row in LDS: 128 KiB

// One workgroup per row: FWHT of the K segments in LDS, then the K x K mix.
// x and y may alias (in-place): each row is read completely into LDS before
// any of it is written, and rows belong to distinct workgroups.
template <bool BF16>
__global__ __launch_bounds__(1024) void k_hadamard(const uint16_t* x, int ld_x, int n, int K,
                                                        const int8_t* __restrict__ hadk, float scale, uint16_t* y,
                                                        int ld_y) {
  extern __shared__ __align__(16) float u[];  // n floats, then K*K int8 of H_K
  int8_t* hk = (int8_t*)(u + n);
  const int row = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  const uint16_t* xr = x + (size_t)row * ld_x;
  for (int i = tid; i < n; i += nt) u[i] = BF16 ? oc_bf2f(xr[i]) : oc_h2f(xr[i]);
  if (K > 1)  // K = 1 passes no block (hadk may be NULL)
    for (int i = tid; i < K * K; i += nt) hk[i] = hadk[i];
  __syncthreads();
  const int L = n / K;
  for (int h = 1; h < L; h <<= 1) {
    // n/2 butterflies: pair (i, i + h) with i in the lower half of its 2h block
    for (int b = tid; b < n / 2; b += nt) {
      const int i = (b / h) * 2 * h + (b % h);
      const float p = u[i], q = u[i + h];
      u[i] = p + q;
      u[i + h] = p - q;
    }
    __syncthreads();
  }
  uint16_t* yr = y + (size_t)row * ld_y;
  if (K == 1) {
    for (int i = tid; i < n; i += nt) yr[i] = BF16 ? oc_f2bf(u[i] * scale) : oc_f2h(u[i] * scale);
    return;
  }
  for (int o = tid; o < n; o += nt) {
    const int i = o / L, j = o - i * L;
    const int8_t* hrow = hk + i * K;
    float acc = 0.f;
    for (int c = 0; c < K; ++c) acc += (float)hrow[c] * u[c * L + j];
    acc *= scale;
    yr[o] = BF16 ? oc_f2bf(acc) : oc_f2h(acc);
  }
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
             "Hadamard block of order %d is not built (supported: 12, 20, 28, 36, 40, 44, 60, 68, 76, 108, 140)",
             K);
  return 0;
}

extern "C" int oc_hadamard(const void* x, int M, int n, int ld_x, const int8_t* hadk, int K, int act_dtype,
                           void* y, int ld_y, void* stream) {
  OC_REQUIRE(x && y, OC_ERR_INVALID, "null pointer");
  OC_REQUIRE(M >= 0 && n > 0 && ld_x >= n && ld_y >= n, OC_ERR_INVALID, "bad shape M=%d n=%d ld_x=%d ld_y=%d", M,
             n, ld_x, ld_y);
  OC_REQUIRE(act_dtype == OC_DTYPE_F16 || act_dtype == OC_DTYPE_BF16, OC_ERR_UNSUPPORTED, "bad act_dtype %d",
             act_dtype);
  OC_REQUIRE(K >= 1 && n % K == 0 && is_pow2(n / K), OC_ERR_SHAPE, "n=%d is not K=%d times a power of two", n, K);
  OC_REQUIRE(K == 1 || hadk, OC_ERR_INVALID, "K=%d needs the K x K block", K);
  OC_REQUIRE(n <= kHadMaxN, OC_ERR_UNSUPPORTED, "n=%d above the %d supported", n, kHadMaxN);
  if (M == 0) return 0;
  const size_t lds = (size_t)n * 4 + (size_t)K * K;
  const float scale = 1.0f / sqrtf((float)n);
  hipStream_t st = (hipStream_t)stream;
  if (act_dtype == OC_DTYPE_BF16)
    hipLaunchKernelGGL(k_hadamard<true>, dim3(M), dim3(1024), lds, st, (const uint16_t*)x, ld_x, n, K, hadk,
                       scale, (uint16_t*)y, ld_y);
  else
    hipLaunchKernelGGL(k_hadamard<false>, dim3(M), dim3(1024), lds, st, (const uint16_t*)x, ld_x, n, K, hadk,
                       scale, (uint16_t*)y, ld_y);
  OC_HIP(hipGetLastError());
  return 0;
}
