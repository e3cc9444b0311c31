/*
 * tokenrush_hip.h -- C ABI of libtrhip.so, the gfx950 (MI355X) verify path of token-rush.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream (hipStream_t passed as
 * void*), launches on that stream, never allocates, never synchronizes, and returns 0 or an
 * error code. That makes every call recordable by hipGraph stream capture.
 *
 * Error codes: 0 ok; 1 problem shape not supported; 2 no kernel configuration; 3 bad argument;
 * 4 launch failed; 5 the call needs more than a no-allocation entry point's fixed scratch. 1 and 2 mean what the reference's Marlin launcher means by them
 * (tokenrush/csrc/marlin_bf16.cu:627-669, surfaced by marlin_bf16.cpp:41-43).
 *
 * Tensor conventions (row-major, contiguous):
 *   x        bf16 [M, K]                 activations (M <= 32)
 *   qweight  uint8 [N, K/2]              engine packing: element 2j in the low nibble of byte j
 *                                        (tokenrush/quant.py:9-10)
 *   packed   uint8 [N/16, Gp/4, 4352]    quad layout made by tr_pack_int4: Gp = K/128 rounded up to
 *                                        a multiple of 4 (zero padding); per 16-row strip and four
 *                                        groups, 4 x 1024 bytes of codes then 16 rows x 4 groups of
 *                                        (scale | min << 16) -- tr_packed_bytes(N, K) bytes
 *   scale,mn [N, K/128]                  bf16 (scale_dtype 0, the engine format) or fp16 (1)
 */
#ifndef TOKENRUSH_HIP_H
#define TOKENRUSH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- int4 verify GEMM */

/* y = x . (q*s + m)^T for M <= 32 rows, packed weights from tr_pack_int4. Exactly one of
 * `out` (bf16 [M, N]) and `partials` (fp32 [n_slots, M, N], every slot written, sum over slots
 * = product; n_slots must equal tr_partial_slots or be a valid explicit split) is non-null.
 * When out is used and tr_gemm_workspace_bytes(N, K, M) > 0, `workspace` must hold that many
 * bytes: 512 KiB of int32 counters (one per 128-byte line) at offset 0, zero-filled before first use (every call leaves
 * them at zero again; no call writes anything else there), then fp32 partials. One buffer
 * sized for the largest call serves every shape; calls that overlap on one device must not
 * share a workspace. N % 16 == 0, K % 128 == 0, tr_packed_bytes(N, K) > 0,
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

/* tr_int4_gemm in out mode (bf16 [M, N]) with no workspace argument and no allocation: the
 * K-slot partials and arrival counters live in a fixed 16 MiB device array of the library (one
 * copy per GPU, held until the process ends), found with hipGetSymbolAddress on the first call
 * on each device (which also clears its counters with a fill kernel on `stream`). Calls whose
 * workspace need (tr_gemm_workspace_bytes(N, K, M)) exceeds 16 MiB return 5 (TR_ERR_SCRATCH).
 * Every call on one GPU shares that array and leaves its counters at zero; calls that overlap on
 * one GPU (different streams) race. Same results, bit for bit, as tr_int4_gemm.
 * No counterpart in the reference: for callers that cannot allocate (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc). */
int tr_int4_gemm_noalloc(const void* x, const void* packed, void* out, int M, int N, int K, int group, int scale_dtype,
                         void* stream);

/* Fused gate/up + activation: packed is a [gate (N/2 rows); up (N/2 rows)] weight packed by
 * tr_pack_int4_pairs; out bf16 [M, N/2] = silu(bf16(x . gate^T)) * bf16(x . up^T), bit for bit what
 * tr_int4_gemm followed by tr_silu_mul produce. N % 32 == 0; workspace as for tr_int4_gemm.
 * Replaces: silu_mul(gate_up(n)) (tokenrush/model.py:156-160, tokenrush/fused.py:67-87) in one launch, or
 * two when the plan takes more than one K slot (M > 16 at K = 5120): the K slots' partials into the
 * workspace, then their in-order sum and the activation. */
int tr_int4_gemm_silu(const void* x, const void* packed, void* out, void* workspace, size_t workspace_bytes, int M,
                      int N, int K, int group, int scale_dtype, void* stream);

/* The default tiling of an N x K weight for M rows: S K-slots, W waves and R strips per
 * workgroup. Depends on M only through M > 16. Host only, no GPU call. */
int tr_gemm_plan(int N, int K, int M, int* S, int* W, int* R);

/* fp32 slots a partial-mode call writes for an N x K weight at M rows (-1: unsupported shape).
 * Replaces: partial_slots (tokenrush/csrc/marlin_bf16.cu:611-625, marlin_bf16.cpp:46-48). */
int tr_partial_slots(int N, int K, int M);

/* Bytes of workspace an out-mode call needs (0: none). Host only.
 * Replaces: the lock + fp32 reduce buffer sizing of marlin.workspaces (tokenrush/marlin.py:121-135). */
size_t tr_gemm_workspace_bytes(int N, int K, int M);

/* Bytes of the quad layout of an N x K weight (0: unsupported shape -- N % 16, K % 128, or a
 * packed size of 2 GiB or more). Host only. */
size_t tr_packed_bytes(int N, int K);

/* Engine packing + scale/min -> quad layout (tr_packed_bytes(N, K) bytes), and back (padding
 * groups dropped).
 * Replaces: marlin.pack / marlin.unpack (tokenrush/marlin.py:73-118), torch-op layout
 * conversions in the reference. */
int tr_pack_int4(const void* qweight, const void* scale, const void* mn, void* packed, int N, int K,
                 void* stream);
int tr_unpack_int4(const void* packed, void* qweight, void* scale, void* mn, int N, int K, void* stream);

/* The same for a [gate; up] weight (N % 32 == 0) in the pair layout: packed strip s holds gate rows
 * 8s..8s+7 then up rows 8s..8s+7 (engine rows 8s.., N/2 + 8s..). tr_int4_gemm on such a weight
 * writes output column 16 s + i for engine row 8 s + i (i < 8) or N/2 + 8 s + i - 8.
 * No counterpart in the reference (its gate/up output is a plain [gate | up] row, model.py:156). */
int tr_pack_int4_pairs(const void* qweight, const void* scale, const void* mn, void* packed, int N, int K,
                       void* stream);
int tr_unpack_int4_pairs(const void* packed, void* qweight, void* scale, void* mn, int N, int K, void* stream);

/* Dense weight [N, K] in the scale dtype: round(round(q*s) + m), two roundings.
 * Replaces: dequantize_int4 (tokenrush/quant.py:47-53). */
int tr_dequant_int4(const void* qweight, const void* scale, const void* mn, void* out, int N, int K,
                    int group, int scale_dtype, void* stream);

/* ---------------------------------------------------------------- verify accept / commit
 *
 * logits bf16 [M, V] (1 <= M <= 32, 64 <= V <= 262144); tokens int64. `ws` is the accept
 * workspace (tr_accept_workspace_bytes(M, V) bytes, zero-filled before first use; every call
 * leaves its counters at zero again; calls that overlap on one device must not share it).
 * Outputs (device int64): pred [M] (target token per row; may be null), n_accepted [1], tok [1]
 * (correction or bonus token), pos [1] (device position, advanced in place by n + 1), slot [1]
 * (recurrent-state slot to keep), tokens [M] (accepted drafts then tok, -1 beyond), commit [M]
 * (chains: positions pos..pos+n; trees: node indices root..best; -1 beyond).
 * Each call is one launch (residual: three) with no host synchronization. */

size_t tr_accept_workspace_bytes(int M, int V);

/* Per-row argmax, first index on ties. Replaces: logits.argmax(-1) (tokenrush/sample.py:37-38). */
int tr_argmax_rows(const void* logits, int M, int V, void* ws, size_t ws_bytes, int64_t* pred, void* stream);

/* Greedy verify: pred = argmax, n = leading matches of pred[:M-1] with spec_toks[1:M],
 * tok = pred[n], pos += n + 1, slot = n.
 * Replaces: Engine._verify_step's accept with temperature 0 (tokenrush/model.py:302-312). */
int tr_accept_greedy(const void* logits, int M, int V, const int64_t* spec_toks, void* ws, size_t ws_bytes,
                     int64_t* pred, int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot,
                     int64_t* tokens, int64_t* commit, void* stream);

/* sample(): top-64 per row (value desc, index asc), temperature / top_p / top_k masked softmax,
 * inverse-CDF pick with u [M]; greedy when *temperature == 0. Parameters are device scalars.
 * Replaces: sample(logits, params, u) (tokenrush/sample.py:30-51). */
int tr_sample(const void* logits, int M, int V, const float* temperature, const float* top_p,
              const int64_t* top_k, const float* u, void* ws, size_t ws_bytes, int64_t* out, void* stream);

/* Sampled verify: pred = sample(...), then the leading-match commit of tr_accept_greedy.
 * Replaces: Engine._verify_step (tokenrush/model.py:302-312) with SamplingParams. */
int tr_accept_sample(const void* logits, int M, int V, const int64_t* spec_toks, const float* temperature,
                     const float* top_p, const int64_t* top_k, const float* u, void* ws, size_t ws_bytes,
                     int64_t* pred, int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot,
                     int64_t* tokens, int64_t* commit, void* stream);

/* Speculative sampling with residual resample (Leviathan et al. 2023): q fp32 [M-1, V] draft
 * probabilities, u fp32 [M]. Draft i accepted when u[i] q[i, d_i] < p[i, d_i] (p = softmax of
 * row i in a fixed arithmetic: per-1024-chunk exponentials, blocked sums, p = e fl(1 / Z)); at
 * the first rejection j (or j = M-1) tok is drawn with u[M-1] from max(p_j - q_j, 0)
 * (p_{M-1} when all pass). No counterpart in the reference (its sampled verify is
 * tr_accept_sample's rule, tokenrush/model.py:302-308; progress.md:649-656). */
int tr_accept_residual(const void* logits, int M, int V, const float* q, const int64_t* spec_toks,
                       const float* u, void* ws, size_t ws_bytes, int64_t* n_accepted, int64_t* tok,
                       int64_t* pos, int64_t* slot, int64_t* tokens, int64_t* commit, void* stream);

/* lm_head GEMM with the greedy accept fused into its epilogue (one launch): x [M, K] bf16 hidden
 * rows, packed [V, K] weight (quad layout; the plan must use one K slot: K <= 6144 for M <= 16,
 * K <= 3072 above -- otherwise TR_ERR_CONFIG), logits bf16 [M, V] written only when non-null. Each workgroup keeps
 * the per-row (value, first index) maximum of its bf16 outputs; the last workgroup reduces them
 * into pred [M] and, when spec_toks is non-null, finishes exactly as tr_accept_greedy does.
 * workspace: tr_lm_head_workspace_bytes(V, K, M) bytes, zero-filled before first use (every call
 * leaves its counter at zero); calls that overlap on one device must not share it.
 * Replaces: lm_head(n) then sample() with temperature 0 (tokenrush/model.py:260, 299-312,
 * sample.py:37-38), without writing or re-reading the [M, V] logits. */
size_t tr_lm_head_workspace_bytes(int V, int K, int M);
int tr_lm_head_greedy(const void* x, const void* packed, void* logits, void* workspace, size_t workspace_bytes,
                      int M, int V, int K, int group, int scale_dtype, const int64_t* spec_toks, int64_t* pred,
                      int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot, int64_t* tokens,
                      int64_t* commit, void* stream);

/* Draft-tree verify: node 0 is the root (parent -1), parent[i] < i; node i accepted when
 * node_toks[i] == argmax(row parent[i]) and its parent is accepted; the deepest accepted node
 * (lowest index among equals) ends the path. slot = that node, commit = path node indices.
 * Replaces: the host tree simulation of bench/tree_accept.py:91-100. */
int tr_accept_tree(const void* logits, int M, int V, const int64_t* node_toks, const int32_t* parent, void* ws,
                   size_t ws_bytes, int64_t* pred, int64_t* n_accepted, int64_t* tok, int64_t* pos,
                   int64_t* slot, int64_t* tokens, int64_t* commit, void* stream);

/* Tree commit of a cache laid out [planes][max_len][row_bytes]: row (pos - n - 1) + commit[t]
 * moves to row (pos - n - 1) + t for t = 1..n, reading n and pos after the accept. For the
 * reference's KV cache and its scales (tokenrush/state.py:19-29), whose chain commit is only
 * the position advance (model.py:376-382). A commit that would reach rows outside the cache or
 * move more than max_n (<= 32) rows moves nothing and sets *status to 1 (status: device int32,
 * may be null; never cleared by the call). */
int tr_commit_rows(void* data, int planes, long plane_stride_bytes, int row_bytes, const int64_t* pos,
                   const int64_t* n_accepted, const int64_t* commit, int max_n, int32_t* status, void* stream);

/* ---------------------------------------------------------------- row kernels around the GEMMs */

/* Split-K partial consumer: x [T, N] bf16, h per h_mode (0 none, 1 bf16 [T, N], 2 fp32 partials
 * [n_slots, T, N] summed in slot order then rounded to bf16), weight [N] bf16 ->
 * xo = bf16(x + h) (not written when h_mode is 0) and y = rmsnorm(xo) * (1 + weight), or
 * bf16(weight * bf16(rmsnorm(xo))) when plain. N % 8 == 0, N <= 8192, n_slots <= 8; one
 * workgroup per row; x, h, weight, xo, y 16-byte aligned.
 * Replaces: add_rmsnorm (tokenrush/fused.py:23-60). */
int tr_add_rmsnorm(const void* x, const void* h, int h_mode, int n_slots, const void* weight, void* xo, void* y,
                   int T, int N, float eps, int plain, void* stream);

/* gate_up [T, 2F] bf16 (rows ld >= 2F elements apart; 0 = 2F) -> y [T, F] bf16 = silu(gate) * up.
 * F % 8 == 0, ld % 8 == 0, pointers 16-byte aligned.
 * Replaces: silu_mul (tokenrush/fused.py:67-87). */
int tr_silu_mul(const void* gate_up, long ld, void* y, int T, int F, void* stream);

/* Embedding gather: out [T, H] bf16 = table[ids[t]] for int64 ids [T] (device) over a bf16 table
 * [V, H]. H % 8 == 0, pointers 16-byte aligned. An id outside [0, V) gives a zero row and sets
 * *status = 1 when status is not null.
 * Replaces: x = self.w.embed[tokens] (tokenrush/model.py:215), inside the verify step's graph. */
int tr_embed_rows(const void* table, const int64_t* ids, void* out, int T, int H, long V, int* status, void* stream);

/* ---------------------------------------------------------------- GDN (gated delta rule) step */

/* Bytes of the workspace tr_gdn_step / tr_gdn_tree_step need for M tokens (up to 32), H key heads and HV value heads (0 if
 * unsupported; HV <= 256). Zero-filled once by the caller; every call leaves its counters at zero,
 * which sit at a fixed offset, so one buffer sized for the largest call serves calls of every shape. */
size_t tr_gdn_workspace_bytes(int M, int H, int HV);

/* One M-token (1..8) GDN step of one layer: causal conv (kernel 4) over the ring with silu, b/a gates
 * from x . ba_w, L2-normalised q and k, the gated delta rule with the state after token t written to
 * rec slot t, and the gated RMSNorm -> y.
 *   qkvz [M, ld] bf16 (q | k | v | z, ld >= 2 H K + 2 HV V), x [M, hidden] bf16, ba_w [2 HV, hidden]
 *   bf16, ring [2 H K + HV V, R] bf16 (columns (pos + t) % R updated), conv_w [2 H K + HV V, 4] bf16,
 *   A and dt_bias [HV] fp32, rec fp32 slots slot_stride floats apart, each [HV, K, V]; the committed
 *   state is slot *slot (device int64); pos: device int64 position of token 0; norm_w [V] bf16;
 *   y [M, HV V] bf16. K == V == 128, HV % H == 0, R >= M + 3, hidden % 32 == 0. Two launches: the
 *   conv + gates of all heads, then the recurrence per (value head, 16-column block): HV x 8 workgroups.
 * Replaces: gdn_step_fused (tokenrush/fused.py:119-236: _gdn_step_fused_kernel + _gated_norm_kernel),
 * the fused path of gdn_forward (tokenrush/model.py:76-80). */
int tr_gdn_step(const void* qkvz, int ld, const void* x, const void* ba_w, void* ring, const void* conv_w,
                const float* A, const float* dt_bias, float* rec, long slot_stride, const int64_t* slot,
                const void* norm_w, const int64_t* pos, void* y, void* workspace, size_t workspace_bytes, int M,
                int H, int HV, int K, int V, int hidden, int R, float eps, void* stream);

/* Draft-tree GDN step of one layer, M (1..32) nodes with parent[t] < t (node 0 the root, the
 * committed token; a parent outside 0..t-1 reads as the root). Node t continues from its parent's
 * state (the root from slot *slot) and writes its own to rec slot t; its conv window is its three
 * nearest ancestors' inputs, with the ring's committed positions where the root path is shorter.
 * The ring is only read: the nodes' conv inputs go to node_in [M, 2 H K + HV V] bf16 for
 * tr_gdn_tree_commit. Every node's y equals a chain step over its root path. Other arguments as
 * tr_gdn_step (R >= 3); the workspace is tr_gdn_workspace_bytes(M, H, HV).
 * No counterpart in the reference (its trees were simulated on the host, bench/tree_accept.py:91-100);
 * the per-node arithmetic is gdn_step_fused's (tokenrush/fused.py:119-236). */
int tr_gdn_tree_step(const void* qkvz, int ld, const void* x, const void* ba_w, const void* ring, const void* conv_w,
                     const float* A, const float* dt_bias, float* rec, long slot_stride, const int64_t* slot,
                     const void* norm_w, const int64_t* pos, const int32_t* parent, void* node_in, void* y,
                     void* workspace, size_t workspace_bytes, int M, int H, int HV, int K, int V, int hidden, int R,
                     float eps, void* stream);

/* Tree commit of the conv rings of `layers` GDN layers (ring [C, R] bf16 every ring_stride
 * elements, node_in [M, C] bf16 every node_stride elements): ring column (base + d) % R <-
 * node_in[commit[d]] for d = 0..n in order, base = *pos - n - 1 (pos, n_accepted and commit as
 * tr_accept_tree leaves them), so each ring ends as a chain step over the accepted path leaves it.
 * A path outside 0..M-1 or of M or more drafts commits nothing and sets *status (optional) to 1.
 * No counterpart in the reference (chain commits are the position advance, model.py:376-382). */
int tr_gdn_tree_commit(void* ring, long ring_stride, const void* node_in, long node_stride, int layers, int C, int R,
                       int M, const int64_t* pos, const int64_t* n_accepted, const int64_t* commit, int32_t* status,
                       void* stream);

/* ---------------------------------------------------------------- attention over an FP8 KV cache */

/* Bytes of the split-partials workspace of tr_attn_decode / tr_attn_decode_tree (M up to 32; 0 if
 * unsupported). */
size_t tr_attn_workspace_bytes(int M, int HQ, int nsplit);

/* Prep of M (1..8) new tokens of one attention layer: q and k RMSNorm with (1 + w) gain, partial
 * rope on the first rotary_dim dims (a power of two) at positions *pos + t, q_out [M, HQ, D] bf16,
 * and cache rows *pos + t of k_cache / v_cache ([HKV, maxlen, D] float8_e4m3fn) with their scales
 * k_scale / v_scale ([HKV, maxlen] fp32, amax / 448). qkv [M, ld] bf16 = [HQ (q | gate) 2D | HKV D |
 * HKV D]; cos / sin [max_pos, rotary_dim] bf16. D == 256.
 * Replaces: attn_prep (tokenrush/fused.py:247-325). */
int tr_attn_prep(const void* qkv, int ld, const void* q_norm_w, const void* k_norm_w, const void* cos,
                 const void* sin, int rotary_dim, const int64_t* pos, void* k_cache, void* v_cache, float* k_scale,
                 float* v_scale, int maxlen, void* q_out, int M, int HQ, int HKV, int D, float eps, void* stream);

/* Flash-decoding of M (1..8) query tokens over cache rows 0..*pos + M - 1 (query t sees rows
 * <= *pos + t): nsplit key-range splits (two launches: split, then combine + sigmoid output gate
 * from qkv) -> out [M, HQ D] bf16. D == 256.
 * Replaces: attn_decode_fused (tokenrush/fused.py:355-470: _attn_split_kernel + _attn_reduce_kernel). */
int tr_attn_decode(const void* q, const void* qkv, int ld, const void* k_cache, const void* v_cache,
                   const float* k_scale, const float* v_scale, int maxlen, const int64_t* pos, void* out,
                   void* workspace, size_t workspace_bytes, int M, int HQ, int HKV, int D, int nsplit, void* stream);

/* Draft-tree prep, M (1..32) nodes with parent[t] < t: as tr_attn_prep, but node t is roped at
 * position *pos + depth(t) (where its root path puts it once committed) while its key and value go
 * to cache row *pos + t (tr_commit_rows later moves the accepted path's rows into place).
 * No counterpart in the reference; the per-node arithmetic is attn_prep's (tokenrush/fused.py:247-325). */
int tr_attn_prep_tree(const void* qkv, int ld, const void* q_norm_w, const void* k_norm_w, const void* cos,
                      const void* sin, int rotary_dim, const int64_t* pos, const int32_t* parent, void* k_cache,
                      void* v_cache, float* k_scale, float* v_scale, int maxlen, void* q_out, int M, int HQ, int HKV,
                      int D, float eps, void* stream);

/* Draft-tree flash-decoding, M (1..32) nodes: node t sees the committed rows < *pos and the new
 * rows *pos + i of its ancestors and itself (the ancestor mask). Otherwise as tr_attn_decode; the
 * query rows of a kv head run in groups of 64, one more grid dimension.
 * No counterpart in the reference; the per-node arithmetic is attn_decode_fused's (tokenrush/fused.py:355-470). */
int tr_attn_decode_tree(const void* q, const void* qkv, int ld, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale, int maxlen, const int64_t* pos,
                        const int32_t* parent, void* out, void* workspace, size_t workspace_bytes, int M, int HQ,
                        int HKV, int D, int nsplit, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOKENRUSH_HIP_H */
