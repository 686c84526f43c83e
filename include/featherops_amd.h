/*
 * featherops_amd -- C ABI of the MI355X (gfx950) FeatherOps hot path.
 *
 * libfeatherops_amd.so exports these symbols with C linkage. Every pointer is
 * device memory owned by the caller; no entry point allocates, synchronises
 * or keeps state between calls. All work is enqueued asynchronously on
 * `stream`.
 *
 * Tensor layouts:
 *   A            (M, K)        fp16, row-major, 16-byte aligned
 *   b_prepacked  (K/16, N, 16) fp8 bytes (e5m2 or e4m3fn), 16-byte aligned:
 *                element (k, n) of the (K, N) weight is at [k/16][n][k%16]
 *   C            (M, N)        fp16 or bf16, row-major, 16-byte aligned
 *   bias         (N,)          same type as C
 *   scale        one fp32 on the device (read by the kernel, no host sync)
 */
#ifndef FEATHEROPS_AMD_H
#define FEATHEROPS_AMD_H

#include <hip/hip_runtime_api.h>
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes of the int-returning entry points. */
#define FEATHER_OK 0
#define FEATHER_ERR_INVALID 1      /* argument out of the supported domain */
#define FEATHER_ERR_UNSUPPORTED 2  /* no kernel for this configuration */
#define FEATHER_ERR_LAUNCH 3       /* hipGetLastError() reported a launch failure */
#define FEATHER_ERR_SCRATCH 4      /* the call needs more scratch than FEATHER_NOALLOC_SCRATCH_BYTES */

/* Size of the static per-GPU scratch array of feather_launch_scaled_mm_noalloc (16 MiB). */
#define FEATHER_NOALLOC_SCRATCH_BYTES (16u << 20)

/* Data type codes. */
#define FEATHER_DTYPE_F16 0
#define FEATHER_DTYPE_BF16 1
#define FEATHER_DTYPE_F32 2
#define FEATHER_B_E4M3FN 0
#define FEATHER_B_E5M2 1

/*
 * C = out( out(A @ dec(b_prepacked) * scale) + bias ), fp32 accumulation.
 * Replaces `extern "C" bool launch_scaled_mm(...)` of the reference,
 * kernel/hip/hip_kernel.cu:564-632 (same argument order and meaning; `a` is
 * the fp16 A pointer the reference types as `const half*`).
 *   has_scale / has_bias: 0 or 1; scale / bias are only read when set.
 *   (block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n): one of the
 *   configurations the reference lists (hip_kernel.py:60-89) or one of the
 *   gfx950 additions (2,4,4,8,4), (4,2,4,4,8), (4,2,4,4,4), (2,4,4,8,3), (2,4,4,4,6). The tuple keeps the reference's
 *   divisibility meaning (BlockM = 16*wm*rm, BlockN = 16*wn*rn, ChunkK = 16*u)
 *   for callers that pad to it; the kernels themselves accept any M.
 *   b_dtype: FEATHER_B_E4M3FN or FEATHER_B_E5M2. output_dtype: 0 fp16, 1 bf16.
 * Returns false (and launches nothing) for a configuration outside that list,
 * N or K not a multiple of 16, or sizes beyond int32; like the reference it
 * does not call hipGetLastError itself.
 */
bool launch_scaled_mm(const void* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                      uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias, int block_warps_m,
                      int block_warps_n, int unroll_k, int repeat_m, int repeat_n, int b_dtype, int output_dtype,
                      hipStream_t stream);

/*
 * launch_scaled_mm with a caller workspace. For shapes too small to fill the
 * GPU with output tiles (M <= 64, or fewer than 256 tiles of 128 x 128) the
 * kernels then also split K across workgroups, which keeps every CU loading
 * (the reference ABI has no workspace, so launch_scaled_mm runs those shapes
 * without the cross-workgroup split). workspace_bytes must
 * be at least feather_scaled_mm_workspace_size(...) (0 means none needed; a
 * smaller workspace falls back to the unsplit kernel). Its first 64 KB hold
 * arrival counters: they must be zero before the first use and every call
 * leaves them zero; the rest is scratch for fp32 partial sums. One workspace
 * (zero-filled once, sized for the largest call) therefore serves calls of
 * any shapes in sequence on one stream; calls that run concurrently need
 * distinct workspaces. No counterpart in the reference; the torch op binding
 * uses it.
 */
bool feather_launch_scaled_mm_ws(const void* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                                 uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias,
                                 int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n,
                                 int b_dtype, int output_dtype, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/*
 * feather_launch_scaled_mm_ws with the activation dtype as an argument:
 * a_dtype FEATHER_DTYPE_F16 (same as feather_launch_scaled_mm_ws) or
 * FEATHER_DTYPE_BF16 -- bf16 activations are rounded to fp16 inside the
 * kernel with round-to-nearest-even, the values of the x.to(float16) that
 * comfy_feather/ops.py:88 runs before the GEMM, so the separate cast pass
 * over A disappears. bf16 activations are served for e5m2 weights by the
 * small-M kernel (M <= 64 routed to it); any other combination returns false
 * and launches nothing (the caller converts A and calls again). On every
 * other kernel converting each A fragment as it is read costs more than one
 * cast pass: each fragment is read by several waves (measured, M=512 N=3072
 * K=12288 on the split-K tiles: 102 us vs 60 us cast first). Same workspace contract. No counterpart in the
 * reference.
 */
bool feather_launch_scaled_mm_ex(const void* a, int a_dtype, const uint8_t* b_prepacked, const float* scale,
                                 const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale,
                                 int has_bias, int block_warps_m, int block_warps_n, int unroll_k, int repeat_m,
                                 int repeat_n, int b_dtype, int output_dtype, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/*
 * feather_launch_scaled_mm_ex without a workspace argument and without any
 * allocation. No counterpart in the reference: it is for callers that cannot
 * allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc. The K-split scratch (arrival
 * counters and fp32 partials) is a static device array of
 * FEATHER_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; the
 * first call on a device looks up its address (hipGetSymbolAddress) and
 * clears its counters with a fill kernel on `stream`, so that first call on
 * each device must be made eagerly, outside stream capture (the symbol lookup
 * may be refused during capture, and the fill would be recorded into the
 * caller's graph); later calls may be captured. Results equal
 * feather_launch_scaled_mm_ex with a caller workspace of the size
 * feather_scaled_mm_workspace_size reports. Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller. Returns FEATHER_OK,
 * FEATHER_ERR_UNSUPPORTED (no kernel for this configuration / activation
 * dtype, nothing launched), FEATHER_ERR_SCRATCH (the call's K split needs more
 * than the array holds, nothing launched), FEATHER_ERR_INVALID or
 * FEATHER_ERR_LAUNCH.
 */
int feather_launch_scaled_mm_noalloc(const void* a, int a_dtype, const uint8_t* b_prepacked, const float* scale,
                                     const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale,
                                     int has_bias, int block_warps_m, int block_warps_n, int unroll_k, int repeat_m,
                                     int repeat_n, int b_dtype, int output_dtype, hipStream_t stream);

/*
 * feather_launch_scaled_mm_ws with the unmerged-LoRA term fused into the
 * epilogue: C = rnd(acc * scale + T . U^T) (+ bias in the output type), where
 * T is (M, rank) and U is (N, rank), both row-major, 16-byte aligned, in
 * lora_dtype (FEATHER_DTYPE_F16 or FEATHER_DTYPE_BF16), rank % 32 == 0 (pad
 * with zero columns), and the LoRA strengths already folded into T. Replaces
 * the separate y += F.linear(F.linear(x, A), B) * s of the reference's
 * comfy_feather/lora.py:4-35 for the part after F.linear(x, A): the caller
 * computes T = F.linear(x, A) * s. Served by the LDS-DMA tiles (K % 64 == 0,
 * a routed tile of at least 128 x 128) with fp16 activations and e5m2
 * weights, with M * rank and N * rank below 2^30; returns false and
 * launches nothing otherwise (the caller then adds the term itself). Needs no
 * workspace.
 */
bool feather_launch_scaled_mm_lora(const void* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                                   uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias,
                                   const uint16_t* lora_t, const uint16_t* lora_u, int64_t rank, int lora_dtype,
                                   int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n,
                                   int b_dtype, int output_dtype, hipStream_t stream);

/*
 * LoRA down-projection T = x . D^T: x (M, K) and D (R, K) row-major in the
 * same dtype (x_dtype FEATHER_DTYPE_F16 or _BF16), T (M, R) in that dtype,
 * fp32 accumulation rounded to nearest-even -- the F.linear(x, lora_A) that
 * starts the reference's side path (comfy_feather/lora.py:27), for every
 * patch at once when the down matrices are stacked along the rank (the T
 * argument of feather_launch_scaled_mm_lora). K % 8 == 0, K < 2^24 and
 * R % 32 == 0 (else FEATHER_ERR_UNSUPPORTED, nothing launched), 16-byte
 * aligned buffers. For small M the kernel also splits K across workgroups
 * through `workspace` (same contract as feather_launch_scaled_mm_ws: first
 * 64 KB arrival counters, zero before the first call and left zero by every
 * call; a workspace smaller than feather_lora_down_workspace_size, or NULL,
 * runs unsplit with the same result). Returns a status code.
 */
int feather_lora_down(const void* x, int x_dtype, const void* d, void* t, int64_t M, int64_t K, int64_t R,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes feather_lora_down can use for this call (0 = none). */
size_t feather_lora_down_workspace_size(int64_t M, int64_t K, int64_t R);

/*
 * A configuration tuple for this shape on the current device, without timing
 * anything: the output tile whose waves of workgroups times tile cost is
 * smallest (256x256, 256x192, 128x384, 128x256, 256x128 or 128x128; the small-M
 * kernel's tuple for M <= 64). Writes 5 ints (block_warps_m, block_warps_n,
 * unroll_k, repeat_m, repeat_n) to cfg. The tuple ignores the reference's
 * block-divisibility rule (for the any-M entry). No counterpart in the
 * reference; the autotuner (kernel/hip/utils.py:192-223) times configs instead.
 */
int feather_scaled_mm_pick_config(int64_t M, int64_t N, int64_t K, int* cfg);

/* Workspace bytes feather_launch_scaled_mm_ws / _ex can use for this call (0 = none). */
size_t feather_scaled_mm_workspace_size(int64_t M, int64_t N, int64_t K, int block_warps_m, int block_warps_n,
                                        int unroll_k, int repeat_m, int repeat_n);

/*
 * Which gfx950 kernel launch_scaled_mm would run for this shape and
 * configuration (0 = unsupported configuration). Several reference
 * configurations map onto one kernel; the autotuner
 * (kernel/hip/utils.py:192-223 in the reference) times each kernel once.
 * No counterpart in the reference.
 */
int feather_scaled_mm_kernel_id(int64_t M, int64_t N, int64_t K, int block_warps_m, int block_warps_n, int unroll_k,
                                int repeat_m, int repeat_n);

/*
 * Quantize an (N, K) weight to fp8 e5m2 with a per-tensor scale and write it
 * prepacked as (K/16, N, 16). Replaces the torch arithmetic of
 * comfy_feather/quant.py:52-74 followed by prepack_transpose (quant.py:11-13):
 *   native = 0: load path, make_feather_quantized_weight (quant.py:116-136):
 *               fp32 arithmetic on w * ckpt_scale (ckpt_scale may be NULL = 1)
 *   native = 1: patch path, quantize_feather_weight (quant.py:139-146):
 *               arithmetic in w's dtype, fp16 reciprocal clamp (quant.py:56-58)
 * w_dtype: FEATHER_DTYPE_F16 / _BF16 / _F32. K % 16 == 0, w 16-byte aligned.
 * scale_out receives the fp32 scale. workspace: >= 1024 bytes of device
 * memory, overwritten (per-workgroup partial maxima of |w|; no clearing
 * needed). Returns a status code.
 */
int feather_quantize_prepack_e5m2(const void* w, int w_dtype, int64_t N, int64_t K, const float* ckpt_scale,
                                  int native, uint8_t* out, float* scale_out, uint32_t* workspace, hipStream_t stream);

/*
 * Same as feather_quantize_prepack_e5m2, with the workspace contract of
 * feather_launch_scaled_mm_ws: workspace_bytes >= feather_quantize_workspace_size(),
 * the first 64 KB zero before the first call and left zero by every call (one
 * zero-filled workspace serves this and the K-split GEMMs on one stream), the
 * rest scratch. With it, fp16 / bf16 weights take one pass: one workgroup per
 * compute unit keeps its share of the weight in registers and LDS (up to 96 MB
 * of bf16 on an MI355X; the rest of a larger share is read twice) while the
 * workgroups agree on the amax through counters in the zero region (3 bytes of
 * HBM traffic per element instead of 5 for weights that fit); fp32 weights
 * take the two passes. Same results either way. Calls that
 * share a workspace must not overlap (one stream). No counterpart in the
 * reference: it replaces the same quant.py code as feather_quantize_prepack_e5m2.
 */
int feather_quantize_prepack_e5m2_ws(const void* w, int w_dtype, int64_t N, int64_t K, const float* ckpt_scale,
                                     int native, uint8_t* out, float* scale_out, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes feather_quantize_prepack_e5m2_ws needs (64 KB + 4 KB). No counterpart in the reference. */
size_t feather_quantize_workspace_size(void);

/*
 * Same output with a caller-given scale (no amax, no clamp): q = e5m2(w *
 * T(1/scale)) in w's dtype T. Replaces quant.py:59-74 when `scale` is passed
 * to quantize_fp8e5m2_scaled. No workspace.
 */
int feather_quantize_prepack_e5m2_scaled(const void* w, int w_dtype, int64_t N, int64_t K, const float* scale,
                                         uint8_t* out, hipStream_t stream);

/* (N, K) bytes -> (K/16, N, 16). Replaces quant.py:11-13 (prepack_transpose). */
int feather_prepack_transpose(const uint8_t* w_nk, uint8_t* out, int64_t N, int64_t K, hipStream_t stream);

/* (K/16, N, 16) -> (N, K) bytes. Replaces quant.py:17-19 (unprepack_transpose). */
int feather_unprepack_transpose(const uint8_t* packed, uint8_t* out_nk, int64_t N, int64_t K, hipStream_t stream);

/* (K, N) bytes -> (K/16, N, 16). Replaces kernel/hip/hip_kernel.py:170-171
 * (prepack_b_for_scaled_mm). */
int feather_prepack_b(const uint8_t* b_kn, uint8_t* out, int64_t K, int64_t N, hipStream_t stream);

/* bf16 -> fp16, round toward zero (saturating). Replaces kernel/convert.py:6-34
 * (bf16_to_fp16); n may be any count, buffers 16-byte aligned. */
int feather_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream);

/* bf16 -> fp16, round to nearest even, overflow to +-inf: the values of
 * torch's x.to(float16), which comfy_feather/ops.py:88 applies to bf16
 * activations before the GEMM. The any-M Python entry uses it where the GEMM
 * kernel has no bf16-activation variant. n any count, buffers 16-byte aligned.
 * No counterpart in the reference (it uses the torch cast). */
int feather_bf16_to_fp16_rne(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream);

/* (K/16, N, 16) e5m2 -> (N, K) of out_dtype as out_dtype(float32(q) * scale).
 * Replaces quant.py:99-102 (FeatherFP8E5M2PackedLayout.dequantize). */
int feather_dequantize_e5m2(const uint8_t* packed, const float* scale, void* out, int out_dtype, int64_t N, int64_t K,
                            hipStream_t stream);

/* Text for a status code. */
const char* feather_status_string(int status);

/* ABI revision of this header (bumped on any signature change). */
int feather_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FEATHEROPS_AMD_H */
