// Shared device/host helpers for the onecomp-amd HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/onecomp_amd.h"

// ---------------------------------------------------------------------------
// error reporting (thread-local message, negative return codes)
// ---------------------------------------------------------------------------
namespace oc {

int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
// Plan knob `name` (an OC_* name) if a test pinned it with oc_set_plan_override, else dflt.
int knob(const char* name, int dflt);

#define OC_REQUIRE(cond, code, ...)                 \
  do {                                              \
    if (!(cond)) return ::oc::set_error((code), __VA_ARGS__); \
  } while (0)

#define OC_HIP(call)                                       \
  do {                                                     \
    hipError_t _e = (call);                                \
    if (_e != hipSuccess) return ::oc::check_hip(_e, #call); \
  } while (0)

// ---------------------------------------------------------------------------
// packed-weight layout ("lane-chunk" layout)
//
// The weights of 16 output columns (an n-tile) and 128 consecutive k (a
// k-block) are one MFMA-ready chunk: lane l of a wave owns column l % 16 and
// the k-slices 8*(l/16) + [0, 8) of the four 32-deep MFMA steps of the block,
// i.e. exactly the B operand of v_mfma_f32_16x16x32_{f16,bf16}.  Chunks are
// grouped in units of U k-blocks whose per-lane payload is P x 16 bytes, so
// every wave-wide load is one contiguous 1 KiB line of 16-byte lane vectors:
//
//   bits  U  P   per-lane payload per unit
//   2     2  1   4 words: 16 codes each, 2 words per k-block
//   3     4  3   12 words: 3 per k-block (32 codes, 2 spare-bit codes)
//   4     1  1   4 words: one per MFMA step
//   8     1  2   8 words: two per MFMA step
//
// Byte offset of (n-tile nt, unit u, part pt, lane l) =
//   ((nt * NU + u) * P + pt) * 1024 + l * 16,  NU = K_pad / (128 * U).
// Inside each word, codes are placed so that ((w >> shift) & mask) yields an
// fp16/bf16 pair (k = 2p, 2p + 1) in natural k order -- see decode_* below and
// the repack kernel, which is their exact inverse.
// ---------------------------------------------------------------------------
struct Layout {
  int bits, U, P;
  int K, N, K_pad, N_pad, NU, NT;
};

inline __host__ __device__ Layout make_layout(int bits, int K, int N) {
  Layout L;
  L.bits = bits;
  L.U = bits == 2 ? 2 : (bits == 3 ? 4 : 1);
  L.P = bits == 3 ? 3 : (bits == 8 ? 2 : 1);
  L.K = K;
  L.N = N;
  int ku = 128 * L.U;
  L.K_pad = (K + ku - 1) / ku * ku;
  L.N_pad = (N + 15) / 16 * 16;
  L.NU = L.K_pad / ku;
  L.NT = L.N_pad / 16;
  return L;
}

inline __host__ __device__ size_t layout_bytes(const Layout& L) {
  return (size_t)L.NT * L.NU * L.P * 1024;
}

// Effective group size (gs = -1 means a single group spanning K).
inline __host__ __device__ int eff_group(int group_size, int K) {
  return group_size <= 0 ? K : group_size;
}

}  // namespace oc

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
typedef _Float16 oc_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 oc_bf168 __attribute__((ext_vector_type(8)));
typedef _Float16 oc_half2 __attribute__((ext_vector_type(2)));
typedef float oc_f4 __attribute__((ext_vector_type(4)));
typedef float oc_f16v __attribute__((ext_vector_type(16)));
typedef uint32_t oc_u4 __attribute__((ext_vector_type(4)));

// Keep a constant in a VGPR so the compiler can fuse (a & m) | c into one
// v_and_or_b32 (gfx9 VOP3 encodings take no literal operand).
__device__ __forceinline__ uint32_t oc_opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Compiler-level memory barrier for data exchanged between lanes of one wave
// through LDS.  Without it the exchange is a data race in the per-thread
// memory model and loads may be forwarded from earlier reads of the same
// address.  Emits no instruction.
__device__ __forceinline__ void oc_wave_lds_barrier() { asm volatile("" ::: "memory"); }

// Raw buffer resource over [base, base + bytes).  A load at an offset past
// `bytes` returns zero without touching memory; kOcOob is such an offset for
// every buffer this library reads (all are below 2 GiB per descriptor).
constexpr uint32_t kOcOob = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t oc_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, bytes, 0x00020000);
}
// 16-byte buffer loads: plain, and streaming (nt: read once, not kept in L2)
__device__ __forceinline__ oc_u4 oc_bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(oc_u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ oc_u4 oc_bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(oc_u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}

// Compute units of the current device (cached per device; 256 if unknown).
inline int oc_device_cus() {
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

template <bool BF16>
__device__ __forceinline__ oc_f4 oc_mfma16(oc_u4 a, oc_u4 b, oc_f4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(oc_bf168, a),
                                                   __builtin_bit_cast(oc_bf168, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(oc_half8, a),
                                                  __builtin_bit_cast(oc_half8, b), c, 0, 0, 0);
  }
}

// 32x32x16 MFMA: lane l holds A row l%32 / B column l%32, k = 8(l/32) .. +7;
// D register r of lane l is row 8(r/4) + 4(l/32) + r%4, column l%32.
template <bool BF16>
__device__ __forceinline__ oc_f16v oc_mfma32(oc_u4 a, oc_u4 b, oc_f16v c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(oc_bf168, a),
                                                   __builtin_bit_cast(oc_bf168, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(oc_half8, a),
                                                  __builtin_bit_cast(oc_half8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ float oc_h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float oc_bf2f(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t oc_f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint16_t oc_f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
