/*
 * tokenrush_hip.h -- C ABI of libtrhip.so, the gfx950 (MI355X) verify path of token-rush.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream (hipStream_t passed as
 * void*), launches on that stream, never allocates, never synchronizes, and returns 0 or an
 * error code. That makes every call recordable by hipGraph stream capture.
 *
 * Error codes: 0 ok; 1 problem shape not supported; 2 no kernel configuration; 3 bad argument;
 * 4 launch failed. 1 and 2 mean what the reference's Marlin launcher means by them
 * (tokenrush/csrc/marlin_bf16.cu:627-669, surfaced by marlin_bf16.cpp:41-43).
 *
 * Tensor conventions (row-major, contiguous):
 *   x        bf16 [M, K]                 activations (M <= 32)
 *   qweight  uint8 [N, K/2]              engine packing: element 2j in the low nibble of byte j
 *                                        (tokenrush/quant.py:9-10)
 *   packed   uint8 [N/16, K/128, 1088]   strip layout made by tr_pack_int4 (codes + scale/min)
 *   scale,mn [N, K/128]                  bf16 (scale_dtype 0, the engine format) or fp16 (1)
 */
#ifndef TOKENRUSH_HIP_H
#define TOKENRUSH_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- int4 verify GEMM */

/* y = x . (q*s + m)^T for M <= 32 rows, packed weights from tr_pack_int4. Exactly one of
 * `out` (bf16 [M, N]) and `partials` (fp32 [n_slots, M, N], every slot written, sum over slots
 * = product; n_slots must equal tr_partial_slots or be a valid explicit split) is non-null.
 * When out is used and tr_gemm_workspace_bytes(N, K, M) > 0, `workspace` must hold that many
 * bytes: 64 KiB of int32 counters at offset 0, zero-filled before first use (every call leaves
 * them at zero again; no call writes anything else there), then fp32 partials. One buffer
 * sized for the largest call serves every shape; calls that overlap on one device must not
 * share a workspace. N % 16 == 0, K % 128 == 0,
 * group == 128.
 * Replaces: marlin_bf16_cuda (tokenrush/csrc/marlin_bf16.cu:630-670) behind the torch binding
 * `mul(A, B, C, s, m, workspace, red, ...)` (tokenrush/csrc/marlin_bf16.cpp:14-44): C bf16 ->
 * out, C fp32 [slots, m, n] -> partials, workspace/red -> workspace. */
int tr_int4_gemm(const void* x, const void* packed, void* out, void* partials, void* workspace,
                 size_t workspace_bytes, int M, int N, int K, int group, int scale_dtype, int n_slots,
                 void* stream);

/* tr_int4_gemm with an explicit tiling: n_slots K slots (also in out mode; 0 = default) and R
 * 16-row strips per workgroup (R <= 0 = default). The workspace must then fit that S (sizing as
 * tr_gemm_workspace_bytes does, with S slots). The role of Marlin's thread_k/thread_n/sms
 * overrides (tokenrush/csrc/marlin_bf16.cpp:14-16). */
int tr_int4_gemm_ex(const void* x, const void* packed, void* out, void* partials, void* workspace,
                    size_t workspace_bytes, int M, int N, int K, int group, int scale_dtype, int n_slots,
                    int R, void* stream);

/* The default tiling of an N x K weight for M rows: S K-slots, W waves and R strips per
 * workgroup. Depends on M only through M > 16. Host only, no GPU call. */
int tr_gemm_plan(int N, int K, int M, int* S, int* W, int* R);

/* fp32 slots a partial-mode call writes for an N x K weight at M rows (-1: unsupported shape).
 * Replaces: partial_slots (tokenrush/csrc/marlin_bf16.cu:611-625, marlin_bf16.cpp:46-48). */
int tr_partial_slots(int N, int K, int M);

/* Bytes of workspace an out-mode call needs (0: none). Host only.
 * Replaces: the lock + fp32 reduce buffer sizing of marlin.workspaces (tokenrush/marlin.py:121-135). */
size_t tr_gemm_workspace_bytes(int N, int K, int M);

/* Engine packing + scale/min -> strip layout uint8 [N/16, K/128, 1088], and back.
 * Replaces: marlin.pack / marlin.unpack (tokenrush/marlin.py:73-118), torch-op layout
 * conversions in the reference. */
int tr_pack_int4(const void* qweight, const void* scale, const void* mn, void* packed, int N, int K,
                 void* stream);
int tr_unpack_int4(const void* packed, void* qweight, void* scale, void* mn, int N, int K, void* stream);

/* Dense weight [N, K] in the scale dtype: round(round(q*s) + m), two roundings.
 * Replaces: dequantize_int4 (tokenrush/quant.py:47-53). */
int tr_dequant_int4(const void* qweight, const void* scale, const void* mn, void* out, int N, int K,
                    int group, int scale_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOKENRUSH_HIP_H */
