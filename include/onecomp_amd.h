/*
 * onecomp-amd: C ABI of the MI355X (gfx950) quantized-linear hot path.
 *
 * Drop-in boundary for OneComp's quantized-linear inference path:
 *   - Mixed-GPTQ  LinearMethod.apply()  (vllm_plugins/gptq/vllm_plugin.py:332-353 dispatches it
 *     to vLLM's GPTQ/Marlin kernels; this library replaces those kernels), and
 *   - DBF / MDBF  sign-factor matmuls   (vllm_plugins/dbf/vllm_plugin.py:275-328,
 *     onecomp/quantizer/mdbf/mdbf_layer.py:307-344, :412-420).
 *
 * Conventions
 *   - Every function returns 0 on success or a negative OC_ERR_* code; the message of the last
 *     failure on the calling thread is returned by oc_last_error().
 *   - All pointers are device pointers unless stated otherwise.  `stream` is a hipStream_t
 *     (NULL = the default stream).  No entry point allocates device memory; work buffers are
 *     passed in by the caller.  Launches are asynchronous unless a comment says otherwise.
 *   - Activations, scales and outputs are 16-bit floats: OC_DTYPE_F16 (IEEE half) or
 *     OC_DTYPE_BF16.  GPTQ scales are always fp16 (the checkpoint dtype).
 *   - Layouts follow the OneComp checkpoint (AutoGPTQ layout): qweight [K*b/32, N] int32,
 *     qzeros [G, N*b/32] int32, scales [G, N] fp16, g_idx [K] int32; DBF signs are uint8,
 *     MSB first, flat row-major, padding bits = 1.
 */
#ifndef ONECOMP_AMD_H
#define ONECOMP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OC_ABI_VERSION 7

enum {
  OC_OK = 0,
  OC_ERR_INVALID = -1,     /* bad argument (null pointer, negative size, ...) */
  OC_ERR_UNSUPPORTED = -2, /* unsupported bit width / group size / dtype */
  OC_ERR_SHAPE = -3,       /* shape violates a layout requirement */
  OC_ERR_HIP = -4,         /* a HIP runtime call failed */
  OC_ERR_WORKSPACE = -5,   /* workspace or counter buffer too small */
  OC_ERR_GIDX = -6         /* g_idx does not describe equal-size contiguous groups after sorting */
};

enum { OC_DTYPE_F16 = 0, OC_DTYPE_BF16 = 1 };

/* Rounding points of oc_hadamard, as the reference's apply_online_hadamard
 * (vllm_plugins/utils/rotation.py:100-112 -> hadamard_utils.py:178-199) rounds:
 * FP32   fp32_had=True: fp32 throughout, one rounding to the activation dtype;
 * ONCE   fp32_had=False with the fused transform op (the fast_hadamard_transform
 *        package): transform rounded once, then the 1/sqrt(n) division, then the
 *        H_K product (three roundings; two when K = 1);
 * STAGES fp32_had=False with the reference's pure-PyTorch transform (its default
 *        install, hadamard_utils.py:26-44): every butterfly stage rounded, then as ONCE. */
enum { OC_HAD_ROUND_FP32 = 0, OC_HAD_ROUND_ONCE = 1, OC_HAD_ROUND_STAGES = 2 };

/* Zero-point storage of qzeros (gptq_layer.py:543-557; checkpoint.py:217-221). */
enum {
  OC_ZERO_RAW = 0, /* return the stored fields untouched (parity tool only) */
  OC_ZERO_V1 = 1,  /* checkpoint_format != "gptq_v2": z = (stored + 1) & (2^b - 1) */
  OC_ZERO_V2 = 2   /* checkpoint_format == "gptq_v2": z = stored */
};

int oc_abi_version(void);
const char* oc_last_error(void);

/* Plan pinning for tests and tuning (no counterpart in the reference).  Every launch plan
 * (kernel family, waves, tile height, K split) is a fixed function of the shape and the device;
 * oc_set_plan_override pins one knob by its OC_* name (OC_ERR_INVALID for an unknown name) until
 * oc_clear_plan_overrides.  Not for concurrent use with launches.  Workspace sizes may change
 * with an override: oc_plan_generation() changes on every set/clear so callers that cache
 * workspace sizes know to recompute them.  Host only. */
int oc_set_plan_override(const char* name, int value);
void oc_clear_plan_overrides(void);
int oc_plan_generation(void);

/* ---------------------------------------------------------------- GPTQ parity tools -------- */

/* codes[N, K] = unpacked qweight (int32 in [0, 2^b-1]).
 * Replaces unpack_int_weights, onecomp/quantizer/gptq/gptq_layer.py:142-157 (_unpack_rows :86-126). */
int oc_gptq_unpack_codes(const int32_t* qweight, int K, int N, int bits, int32_t* codes,
                         void* stream);

/* zeros[G, N] = unpacked qzeros, restored per zero_format (OC_ZERO_*).
 * Replaces unpack_zeros gptq_layer.py:173-184 and the restore at gptq_layer.py:550-557. */
int oc_gptq_unpack_zeros(const int32_t* qzeros, int G, int N, int bits, int zero_format,
                         int32_t* zeros, void* stream);

/* W[N, K] = RNE_dtype(fp32(scales[g_idx[k], n]) * (q[n, k] - z[g_idx[k], n])), bit-exact.
 * g_idx may be NULL (then g = k / group_size, or 0 when group_size <= 0).
 * Replaces the dequantisation of GPTQLinear.forward gptq_layer.py:536-569 and
 * iter_gptq_layers + dequantize_layer onecomp/cpu/export/checkpoint.py:186-259. */
int oc_gptq_dequant(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                    const int32_t* g_idx, int K, int N, int G, int bits, int group_size,
                    int zero_format, int out_dtype, void* w, void* stream);

/* ---------------------------------------------------------------- GPTQ load-time repack ----- */

/* Sizes of the internal layout for a K x N layer at `bits`: packed weight bytes, padded K
 * (multiple of 128, 256 or 512 depending on bits) and padded N (multiple of 16).  Host only. */
int oc_gptq_layout(int K, int N, int bits, size_t* packed_bytes, int* k_pad, int* n_pad);

/* Repack a checkpoint layer into the kernel layout.
 *   packed : layout bytes from oc_gptq_layout
 *   meta   : uint32 [G, n_pad]; low half = fp16 scale bits, high half = restored zero
 *   perm   : int32 [K]; receives the stable argsort of g_idx (act-order).  May be NULL when
 *            g_idx is NULL.  *perm_identity (host pointer, may be NULL) is set to 1 when the sort
 *            is the identity, in which case the caller can pass perm = NULL to oc_gptq_gemm.
 * With g_idx != NULL this call synchronizes `stream` to validate that the sorted g_idx forms G
 * contiguous groups of group_size (OC_ERR_GIDX otherwise).
 * Replaces vLLM GPTQLinearMethod.process_weights_after_loading (g_idx argsort + gptq_shuffle),
 * reached via vllm_plugins/gptq/vllm_plugin.py:348-353. */
int oc_gptq_prepare(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                    const int32_t* g_idx, int K, int N, int G, int bits, int group_size,
                    int zero_format, void* packed, uint32_t* meta, int32_t* perm,
                    int* perm_identity, void* stream);

/* ---------------------------------------------------------------- GPTQ hot path ------------ */

/* Workspace bytes oc_gptq_gemm needs for this call (host only). */
size_t oc_gptq_workspace_bytes(int M, int K, int N, int bits, int group_size, int has_perm);

/* Text description of the launches oc_gptq_gemm makes for this call (kernel names and plan
 * parameters, e.g. "k_gemm mt=4 cs=4 tiles=1024 split_tiles=64 S=4 kper=10 + k_gemm_fixup"),
 * written to buf (len bytes, host memory).  Host only; for tests and reports (no counterpart in
 * the reference). */
int oc_gptq_describe_plan(int M, int K, int N, int bits, int group_size, int has_perm, char* buf,
                          int len);

/* y[M, N] = x[M, K] @ dequant(W)^T (+ bias), fp32 accumulation, y in act_dtype.
 * x row stride is K.  perm: int32 [K] from oc_gptq_prepare or NULL.  bias: [N] act_dtype or NULL.
 * workspace: at least oc_gptq_workspace_bytes() bytes of device memory (may be NULL when that is
 * 0); its contents need no initialisation and are dead after the call's kernels finish.
 * Launches 1-3 kernels on `stream`; no host synchronisation, no allocation, no memset, so the
 * call can be captured in a HIP graph.
 * Replaces vLLM GPTQLinearMethod.apply -> ops.gptq_gemm (selected at vllm_plugin.py:348-353)
 * and GPTQMarlinLinearMethod.apply (vllm_plugin.py:332-346). */
int oc_gptq_gemm(const void* x, int M, int K, int N, const void* packed, const uint32_t* meta,
                 const int32_t* perm, int bits, int group_size, int act_dtype, const void* bias,
                 void* y, void* workspace, size_t ws_bytes, void* stream);

/* Allocation-free variant of oc_gptq_gemm (no counterpart in the reference): for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).  Same arguments, plans and results as oc_gptq_gemm, minus the workspace: the
 * work buffer is the library's own per-GPU scratch array of oc_gptq_noalloc_scratch_bytes()
 * (64 MiB) bytes, held until the process ends.  Calls that would need more (act-order x
 * gathers of M * K * 2 bytes, split-K partial tiles) fail with OC_ERR_WORKSPACE.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race.  The current device must be the one `stream` belongs to.  No allocation, no memset, no
 * host synchronisation. */
int oc_gptq_gemm_noalloc(const void* x, int M, int K, int N, const void* packed, const uint32_t* meta,
                         const int32_t* perm, int bits, int group_size, int act_dtype, const void* bias,
                         void* y, void* stream);

/* Bytes of the per-GPU scratch array oc_gptq_gemm_noalloc uses (host only). */
size_t oc_gptq_noalloc_scratch_bytes(void);

/* One part of a fused GPTQ module (e.g. q, k and v of qkv_proj): its repacked weights
 * (oc_gptq_prepare), act-order permutation or NULL, bias [N] or NULL, width, bits, group size. */
typedef struct {
  const void* packed;
  const uint32_t* meta;
  const int32_t* perm;
  const void* bias;
  int N;
  int bits;
  int group_size;
} oc_gptq_part;

/* Workspace bytes oc_gptq_gemm_grouped needs for these parts at M rows (host only). */
size_t oc_gptq_grouped_workspace_bytes(const oc_gptq_part* parts, int n_parts, int M, int K);

/* y[:, off_p : off_p + N_p] = x[M, K] @ dequant(W_p)^T (+ bias_p) for every part p, where off_p is
 * the sum of the widths of the parts before p; y has row stride ldy >= sum N_p.  The parts may
 * differ in bits, group size and act-order: at M <= 16 with groups that are multiples of 128 they
 * run as one launch, otherwise one after the other (same results either way).  Workspace,
 * threading and capture rules as oc_gptq_gemm.
 * The reference rejects fused modules whose shards differ in their quantization settings
 * (vllm_plugins/gptq/vllm_plugin.py:310-317 via utils/module.py:153-177); this entry point serves
 * them, e.g. Mixed-GPTQ qkv_proj with q at 4 bits and k, v at 8 bits as one apply(). */
int oc_gptq_gemm_grouped(const void* x, int M, int K, const oc_gptq_part* parts, int n_parts,
                         int act_dtype, void* y, int ldy, void* workspace, size_t ws_bytes,
                         void* stream);

/* ---------------------------------------------------------------- MoE experts -------------- */

/* Workspace bytes oc_moe_gptq_forward needs (host only); act_order != 0 when perm13 or perm2 is
 * passed. */
size_t oc_moe_workspace_bytes(int M, int H, int I, int topk, int act_order);

/* Mixture-of-experts block with GPTQ experts (all experts share bits and group size).  For token
 * t < M and slot j < topk, pair p = t * topk + j runs expert e = ids[p]
 * (int32; ids outside [0, E) contribute nothing):
 *   gate|up = x[t] @ W13_e^T (+ b13_e),  h = act(gate, up),  y[t] += weights[p] * (h @ W2_e^T + b2_e)
 * act: 0 = SiLU(gate) * up, 1 = GELU-tanh(gate) * up, 2 = the gpt-oss combine
 * (up.clamp(-limit, limit) + 1) * g * sigmoid(alpha * g) with g = gate.clamp(max=limit); each
 * step is rounded to act_dtype as the reference's torch ops round.  weights are fp32 [M * topk].
 * w13: E experts' oc_gptq_prepare output for the merged gate|up layer (H -> 2I, gate columns
 * first), w13_stride bytes apart; meta13 their scale/zero words, meta13_stride words apart; b13
 * [E, 2I] or NULL.  w2 / meta2 / b2 likewise for down (I -> H).  x [M, H], y [M, H] in act_dtype.
 * Act-order experts: perm13 [E, H] / perm2 [E, I] int32 are each expert's oc_gptq_prepare
 * permutation of gate|up (gate and up share one g_idx) / down, or NULL for experts in checkpoint
 * order; x and h are then gathered per pair in that order (one more launch each), and the
 * grouped-GEMM prefill path is not used.
 * Three launches on `stream` (gate|up with the activation, down, the top-k sum), no host
 * synchronisation, no allocation.  Pairs that share an expert share one read of its weights,
 * up to 16 at a time; beyond 64 pairs a fourth launch first sorts the pairs by expert
 * (E <= 2048; above that every pair reads its expert).  With at least 32 pairs per expert on
 * average (prefill) the experts run on the grouped large-M GEMM instead: sort, gather, gate|up,
 * activation, down, top-k sum (six launches).
 * Replaces _UnfusedExperts.forward, onecomp/utils/unfuse_moe.py:61-114 (with the gpt-oss combine
 * of :380-387) over GPTQ experts, and the WNA16 fused-experts dispatch of
 * vllm_plugins/gptq/vllm_plugin.py:240-283. */
int oc_moe_gptq_forward(const void* x, int M, int H, int I, int E, int topk, const int32_t* ids,
                        const float* weights, const void* w13, size_t w13_stride, const uint32_t* meta13,
                        size_t meta13_stride, const void* b13, const void* w2, size_t w2_stride,
                        const uint32_t* meta2, size_t meta2_stride, const void* b2, const int32_t* perm13,
                        const int32_t* perm2, int bits, int group_size, int act, float alpha, float limit,
                        int act_dtype, void* y, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------- DBF / MDBF ---------------- */

/* Sizes of the internal sign layout of an R x Kd +-1 factor (host only): packed bytes, padded
 * reduction length and the k-blocks per lane load (1, 2 or 4). */
int oc_dbf_layout(int R, int Kd, size_t* packed_bytes, int* k_pad, int* unit_k);

/* out[R, Kd] int8 = +-1 signs of a checkpoint factor (uint8, MSB first, flat row-major, 1 -> +1).
 * Replaces unpack_sign_bits vllm_plugins/dbf/modules/naive.py:9-42 and unpack_binary_factor
 * onecomp/quantizer/dbf/dbf_layer.py:71-86 / mdbf_layer.py:86-103 (parity tool). */
int oc_dbf_unpack_signs(const uint8_t* bp, int R, int Kd, int8_t* out, void* stream);

/* Repack a checkpoint sign factor (R x Kd) into the kernel layout (oc_dbf_layout bytes).
 * Replaces the per-call unpack of DBFLinearMethod._apply_naive (vllm_plugin.py:275-294) and the
 * GemLite packing of process_weights_after_loading (vllm_plugin.py:232-273). */
int oc_dbf_prepare(const uint8_t* bp, int R, int Kd, void* packed, void* stream);

/* One term of a sign matmul: post[n] * sum_k S[n, k] * (pre[k] * in[m, k]).
 * packed: oc_dbf_prepare output for S (R x Kd); in: [M, ld_in] activations (ld_in >= Kd, a
 * multiple of 8, 16-byte aligned rows, entries Kd..ld_in-1 zero); pre (16-byte aligned, Kd entries
 * zero-padded to a multiple of 8) and post [R] may be NULL (= ones). */
typedef struct {
  const void* packed;
  const void* in;
  const void* pre;
  const void* post;
  int Kd;
  int ld_in;
} oc_sign_term;

/* Device workspace bytes oc_sign_gemm needs for these terms at M rows (host only).  0 at M <= 12
 * (the GEMV path needs none); at 13 <= M <= 64 the streaming kernel's fp32 partials (one per term
 * and K split, when there is more than one), or what the GEMM path needs if larger; above 64 rows
 * the pre-scaled inputs RNE(in * pre) of the terms that have a pre scale plus the fp32 partial
 * tiles of the K-split pieces (all terms are summed in one accumulation). */
size_t oc_sign_workspace_bytes(const oc_sign_term* terms, int n_terms, int M, int R);

/* out[m, n] = sum over terms of the term above (+ bias[n]) for n < R, rounded once to act_dtype;
 * columns R <= n < fill_to are written as 0.  n_terms <= 4; all terms need the same unit size.
 * A DBF stage is one term (vllm_plugin.py:275-294: stage 1 pre=scaling0, post=scaling2; stage 2
 * post=scaling4), the P paths of MDBF stage 2 are P terms summed in one call
 * (mdbf_layer.py:338-344, :412-420).  workspace: oc_sign_workspace_bytes() bytes of device memory
 * (NULL when that is 0); no allocation, no memset, no host synchronisation.
 * Replaces DBFLinearMethod._apply_naive/_apply_gemlite. */
int oc_sign_gemm(const oc_sign_term* terms, int n_terms, int M, int R, int act_dtype,
                 const void* bias, void* out, int ld_out, int fill_to, void* workspace,
                 size_t ws_bytes, void* stream);

/* Device workspace bytes oc_sign_gemm_batch needs for these problems at M rows (host only). */
size_t oc_sign_batch_workspace_bytes(const oc_sign_term* problems, int n_problems, int M, int R);

/* n_problems <= 4 independent single-term problems with the same M, R, ld_out and fill_to:
 * outs[p][m, n] = problems[p] above (no bias), rounded to act_dtype, zero for R <= n < fill_to.
 * MDBF's per-path rank stages (MultipathMDBFLinear.forward, mdbf_layer.py:412-420: each path's
 * u = Q_V * (B @ (B_amp * x)) on the same x) in one launch where they share a unit size and all
 * or none have a pre scale: the sign GEMV at M <= 12 (blockIdx.y = problem), the streaming sign
 * kernel at 13 <= M <= 64 (+ one reduce launch when K is split); otherwise one oc_sign_gemm per
 * problem.  Each output equals oc_sign_gemm on that problem alone, bit for bit.  workspace:
 * oc_sign_batch_workspace_bytes() bytes (NULL when 0); no allocation, no host synchronisation. */
int oc_sign_gemm_batch(const oc_sign_term* problems, int n_problems, int M, int R, int act_dtype,
                       void* const* outs, int ld_out, int fill_to, void* workspace, size_t ws_bytes,
                       void* stream);

/* ---------------------------------------------------------------- online Hadamard ---------- */

/* Block order K the reference picks for dimension n (host only): the largest listed order dividing
 * n with n / K a power of two, 1 for a power of two, 0 when the reference would assert.
 * Replaces get_hadK's search, onecomp/pre_process/hadamard_utils.py:79-175. */
int oc_hadamard_order(int n);

/* Fill out[K * K] (int8 +-1, row-major) with the order-K block (host only).  K = 1, or one of
 * 12, 20, 28, 36, 40, 44, 60, 68, 76, 108, 140 (built by construction; 52, 100, 156, 172 return
 * OC_ERR_UNSUPPORTED).  Replaces get_had<K>, hadamard_utils.py:211-120444. */
int oc_hadamard_block(int K, int8_t* out);

/* y[m, :] = (H_K (x) H_L) x[m, :] / sqrt(n) with n = K * L, L a power of two, n <= 32768;
 * hadk: device int8 [K * K] from oc_hadamard_block (NULL when K = 1).  rounding: OC_HAD_ROUND_*
 * (above); sqrt(n) is the float32 value, the division an fp32 division.  y may alias x when
 * ld_y == ld_x.  One kernel on `stream`.
 * Replaces matmul_hadU_cuda (hadamard_utils.py:178-199) as applied to the down_proj input by
 * apply_online_hadamard / RotatedLinearMethod (vllm_plugins/utils/rotation.py:100-112, 146-228). */
int oc_hadamard(const void* x, int M, int n, int ld_x, const int8_t* hadk, int K, int act_dtype, int rounding,
                void* y, int ld_y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ONECOMP_AMD_H */
